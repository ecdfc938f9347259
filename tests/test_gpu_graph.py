"""Library calls captured in a HIP graph (the launch-bound sizes a caller
replays): every replay gives the eager call's bytes, with eager work and
synchronisations between replays.  No call on these routes records a memset."""
import numpy as np
import pytest
import torch

import gen

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("m,k,n", [(1024, 1024, 1024), (130, 64, 3008), (1088, 1024, 1024)])
def test_replays_match_eager(uor, dev, m, k, n):
    """slice::gemm (ring and 128-wide tiles) and a view call with beta != 0
    on another output, captured together; each replay is compared with the
    eager results, the outputs reset eagerly between replays."""
    a = torch.from_numpy(gen.i8_full(m * k, 1)).to(dev)
    b = torch.from_numpy(gen.i8_full(k * n, 2)).to(dev)
    c = torch.zeros(m * n, dtype=torch.int32, device=dev)
    c0 = torch.from_numpy(gen.i32_pm2_20(m * n, 5)).to(dev)
    d = c0.clone()
    sc = torch.empty(max(1, uor.suggested_scratch_i8(m, k, n)), dtype=torch.uint8, device=dev)

    def calls(stream):
        assert uor.slice_gemm_i8(m, k, n, a, b, c, scratch=sc, stream=stream) == 0
        st, _ = uor.gemm_i8(a, (m, k), (k, 1), b, (k, n), (n, 1), d, (m, n), (n, 1), alpha=3, beta=-1,
                            stream=stream)
        assert st == 0

    calls(torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    want_c, want_d = c.clone(), d.clone()
    S = a.view(m, k).double() @ b.view(k, n).double()
    assert torch.equal(want_c.view(m, n).double(), S)
    assert torch.equal(want_d.view(m, n).double(), 3 * S - c0.view(m, n).double())

    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        c.zero_()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        calls(torch.cuda.current_stream().cuda_stream)
    for r in range(3):
        c.fill_(7)
        d.copy_(c0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(c, want_c), r
        assert torch.equal(d, want_d), r
        # eager work between replays
        x = (a[:4096].float() * 2).sum().item()
        assert np.isfinite(x)
    del graph
