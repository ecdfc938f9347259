"""Benchmark of the exact-accumulation GEMM hot path on one MI355X.

`python bench.py [--gpus 1] [--steps K] [--warmup W]` prints ONE JSON line.

Headline workload: slice::gemm_ex i8 x i8 -> i32 at
m = n = k = 8192 with lda = ldb = ldc = 8256, alpha = 3, beta = -1, C
pre-filled uniform in [-2^20, 2^20]; inputs resident in HBM before the timed
region.  A step is one call of the library's C ABI (one fused MFMA launch).
`value` is exact-i8 TOPS (2*m*n*k integer ops per step).  The secondary
figure is the 4-bit LUT decode GEMM in GB/s of algorithmic
bytes, rotating weight buffers larger than the 256 MB Infinity Cache.

`roofline` covers the dominant kernel: algorithmic ops per launch divided by
its average launch time, measured with HIP events on the stream the kernel is
launched on, against MI355X's dense int8 MFMA peak of 5.0 POP/s (reported in
the contract's "TFLOP/s" unit, counting integer ops).  `traffic` is the HBM
bytes per launch measured by rocprofv3 PMC counters and committed under
profiles/ (null when no measurement is committed).

`cpu_baseline` times the reference's packed CPU route restated in C++
(oracle/fastroute.cpp, kind "port") on a bounded row slab of the same
workload on this host's cores, scaled to the full problem (rows are
independent).
"""
from __future__ import annotations

import argparse
import itertools
import json
import os
import pathlib
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "uor-matmul_amd"))
sys.path.insert(0, str(ROOT / "tests"))

METRIC = "exact i8 GEMM TOPS @8192³ (% MFMA peak); LUT-GEMM decode GB/s (% HBM peak)"
PEAK_INT8_TOPS = 5000.0  # dense int8 MFMA, MI355X (5.0 POP/s)
PEAK_HBM_GBS = 8000.0    # HBM3E
PEAK_TROP_TERMS = 256 * 64 * 2.4e9  # packed-i16 VALU (+, max) terms/s


def log(msg):
    print(msg, file=sys.stderr, flush=True)


SETTLE_S = 0.3  # untimed running before each timed region, so clocks reach steady state
# Host copies of the secondary configs' inputs and of the GPU's outputs, kept
# for the CPU-baseline leg, which checks every CPU result against them.
CPU_INPUTS = {}


def settle(torch, step, seconds=None):
    """Run `step` untimed for at least `seconds` of wall time (MI355X raises
    its shader clock over the first ~0.2 s of sustained load; a timed region
    that starts cold measures the ramp, not the kernel).  --settle sets the
    default (0 under a profiler, where every dispatch is recorded)."""
    if seconds is None:
        seconds = SETTLE_S
    t0 = time.perf_counter()
    n = 0
    while time.perf_counter() - t0 < seconds:
        for _ in range(4):
            step()
        torch.cuda.synchronize()
        n += 4
    return n


def i8_kernel_name():
    """The 256x256 kernel the headline runs (UOR_GFX950_DL_VARIANT, read by
    the library at load time; s4 unless set)."""
    v = os.environ.get("UOR_GFX950_DL_VARIANT", "s4")
    return {"w8": "gemm_i8_dl_kernel<256,256,2,4,FUSED,FAST,i32>",
            "w8pf": "gemm_i8_dl_kernel<256,256,2,4,FUSED,FAST,i32,prefetch>",
            "w4": "gemm_i8_dl_kernel<256,256,2,2,FUSED,FAST,i32>"}.get(v, "gemm_i8_s4_kernel<FAST,i32>")


def load_traffic(name):
    p = ROOT / "profiles" / f"{name}.traffic.json"
    if p.exists():
        try:
            return json.loads(p.read_text())
        except Exception:
            return None
    return None


def bench_i8(args, torch, uor, gen):
    N, LD = 8192, 8256
    dev = torch.device("cuda:0")
    log("[bench] generating inputs 8192x8256 (A, B i8; C i32)")
    a = gen.i8_full(N * LD, 3)
    b = gen.i8_full(N * LD, 4)
    c0 = gen.i32_pm2_20(N * LD, 5)
    ga = torch.from_numpy(a).to(dev)
    gb = torch.from_numpy(b).to(dev)
    gc = torch.from_numpy(c0).to(dev)
    stream = torch.cuda.current_stream()

    def step():
        st = uor.slice_gemm_ex_i8(N, N, N, 3, ga, LD, gb, LD, -1, gc, LD, stream=stream.cuda_stream)
        if st != 0:
            raise RuntimeError(f"gemm_ex status {st}")

    log(f"[bench] warmup {args.warmup}")
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    settled = settle(torch, step)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    log(f"[bench] timing {args.steps} steps")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(args.steps):
        step()
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = start.elapsed_time(end) / args.steps

    # Parity after timing: W+S+K applications of C := 3AB - C leave C0 (even)
    # or 3AB - C0 (odd).  An even count would compare C0 with C0 whatever the
    # product was, so one more untimed call makes it odd; then every cell is
    # compared with 3AB - C0 in float64 (exact below 2^53).
    log("[bench] verifying output")
    if (args.warmup + settled + args.steps) % 2 == 0:
        step()
        torch.cuda.synchronize()
    A = ga.view(N, LD)[:, :N].to(torch.float64)
    B = gb.view(N, LD)[:, :N].to(torch.float64)
    C0 = torch.from_numpy(c0).to(dev).view(N, LD)[:, :N].to(torch.float64)
    want = 3 * (A @ B) - C0
    parity = bool(torch.equal(gc.view(N, LD)[:, :N].to(torch.float64), want))
    del A, B, C0, want

    ops = 2.0 * N * N * N
    tops = ops / (ms * 1e-3) / 1e12
    result = {
        "metric": METRIC,
        "value": round(tops, 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "i8",
        "data": "synthetic",
        "config": {
            "workload": "slice::gemm_ex i8 x i8 -> i32, m=n=k=8192, lda=ldb=ldc=8256, "
                        "alpha=3, beta=-1, C0 uniform [-2^20, 2^20] (BASELINE configs[1])",
            "m": N, "n": N, "k": N, "ld": LD, "alpha": 3, "beta": -1, "out": "i32",
            "settle": f">= {SETTLE_S} s untimed ({settled} steps) after the warmup steps",
        },
        "parity": parity,
        "wall_s": round(wall, 4),
        "roofline": {
            "bound": "mfma",
            "kernel": i8_kernel_name(),
            "achieved": round(tops, 2),
            "peak": PEAK_INT8_TOPS,
            "unit": "TFLOP/s",
            "frac": round(tops / PEAK_INT8_TOPS, 4),
            "traffic": None,
            "algorithmic_bytes": 2 * N * N + 2 * 4 * N * N,
        },
    }
    t = load_traffic("gemm_i8_8192")
    if t and t.get("kernel") == result["roofline"]["kernel"]:
        result["roofline"]["traffic"] = t.get("bytes_per_launch")
    return result, (a, b, c0)


def bench_deep(args, torch, uor):
    """configs[1] deep case: m = n = 128, k = 2^24, A = B = all -128 (2 GiB
    each), i64 output (every cell 2^38) with the suggested scratch offer (the
    split-K route).  HBM-bound: 2 * 128 * 2^24 bytes per call."""
    m = n = 128
    k = 1 << 24
    dev = torch.device("cuda:0")
    a = torch.full((m * k,), -128, dtype=torch.int8, device=dev)
    b = torch.full((k * n,), -128, dtype=torch.int8, device=dev)
    c = torch.zeros(m * n, dtype=torch.int64, device=dev)
    sc = torch.empty(uor.suggested_scratch_i8(m, k, n), dtype=torch.uint8, device=dev)
    if "cpu" in args.parts:
        CPU_INPUTS["deep"] = True  # the CPU leg builds its own k-sample (A = B = -128)
    stream = torch.cuda.current_stream()
    route = {}

    def step():
        st, r = uor.gemm_i8(a, (m, k), (k, 1), b, (k, n), (n, 1), c, (m, n), (n, 1), out="i64",
                            scratch=sc, stream=stream.cuda_stream)
        if st != 0:
            raise RuntimeError(f"deep status {st}")
        route.update(r)

    for _ in range(2):
        step()
    torch.cuda.synchronize()
    settle(torch, step)
    steps = max(3, min(args.steps, 20))
    s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s0.record(stream)
    for _ in range(steps):
        step()
    s1.record(stream)
    torch.cuda.synchronize()
    ms = s0.elapsed_time(s1) / steps
    parity = bool((c == (1 << 38)).all().item())
    nbytes = 2 * m * k + 8 * m * n
    gbs = nbytes / (ms * 1e-3) / 1e9
    out = {"m": m, "n": n, "k": k, "out": "i64", "ms_per_call": round(ms, 4),
           "GB_s": round(gbs, 1), "frac_hbm": round(gbs / PEAK_HBM_GBS, 4),
           "TOPS": round(2.0 * m * n * k / (ms * 1e-3) / 1e12, 1), "route": route.get("kind"),
           "split_k": route.get("split_k"), "parity": parity}
    del a, b, c, sc
    torch.cuda.empty_cache()
    return out


def lut_kernel_name(route):
    """The LUT kernel a route record names (uor_gfx950_gemm_lut4's choices)."""
    if route.get("kind") == "lut4_dot4":
        return "lut4_dot4_pf_kernel"
    if route.get("split_k") == 16 and route.get("tile_n") == 8:
        return "lut4_tile8_kernel"
    return {1: "lut4_lds_kernel", 4: "lut4_mfma16_kernel", 8: "lut4_tile_kernel", 16: "lut4_tile_kernel"}.get(
        route.get("split_k"), "lut4_mfma_kernel")


def bench_lut4(args, torch, uor, gen, ms_list=(1, 8, 32)):
    """the 4-bit LUT decode GEMM, m in {1, 8, 32}, k = 8192,
    n = 28672, one codebook per 128 coded rows.  Three distinct code buffers
    (3 x 117 MB, beyond the 256 MB Infinity Cache) rotate across steps so the
    codes stream from HBM.  GB/s counts algorithmic bytes:
    n*k/2 + m*k + 4*m*n + books."""
    k, n, group = 8192, 28672, 128
    dev = torch.device("cuda:0")
    codes = [torch.from_numpy(gen.i8_full(n * k // 2, 7 + 100 * r).view("uint8")).to(dev)
             for r in range(3)]
    books = torch.from_numpy(gen.i8_full((n // group) * 16, 8)).to(dev)
    out = []
    stream = torch.cuda.current_stream()
    for m in ms_list:
        a = torch.from_numpy(gen.i8_full(m * k, 6)).to(dev)
        c = torch.zeros(m * n, dtype=torch.int32, device=dev)
        route = {}

        def step(i):
            st, r = uor.gemm_lut4(a, m, k, (k, 1), codes[i % 3], n, books, group, c, (n, 1),
                                  stream=stream.cuda_stream)
            if st != 0:
                raise RuntimeError(f"lut4 status {st}")
            route.update(r)

        for i in range(args.warmup):
            step(i)
        torch.cuda.synchronize()
        # Settle on the rotating buffers too: one buffer alone (117 MB) stays
        # in the 256 MB Infinity Cache.
        calls = itertools.count()
        settle(torch, lambda: step(next(calls)))
        steps = max(args.steps, 30)
        s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s0.record(stream)
        for i in range(steps):
            step(i)
        s1.record(stream)
        torch.cuda.synchronize()
        ms = s0.elapsed_time(s1) / steps
        nbytes = n * k // 2 + m * k + 4 * m * n + (n // group) * 16
        gbs = nbytes / (ms * 1e-3) / 1e9
        if "cpu" in args.parts:
            step(0)
            torch.cuda.synchronize()
            lut = CPU_INPUTS.setdefault("lut", {"k": k, "n": n, "group": group,
                                               "codes": codes[0].cpu().numpy(),
                                               "books": books.cpu().numpy(), "runs": {}})
            lut["runs"][m] = (a.cpu().numpy(), c.cpu().numpy())
        out.append({"m": m, "k": k, "n": n, "group": group, "ms_per_call": round(ms, 5),
                    "GB_s": round(gbs, 1), "frac_hbm": round(gbs / PEAK_HBM_GBS, 4),
                    "TOPS": round(2.0 * m * n * k / (ms * 1e-3) / 1e12, 2),
                    "algorithmic_bytes": nbytes,
                    "kernel": lut_kernel_name(route)})
    return out


def bench_lut_prefill(args, torch, uor, gen, m=2048):
    """LUT prefill: the config 3 weights (k = 8192,
    n = 28672, 224 codebooks) at m = 2048 rows with the suggested offer: W^T
    decoded once per call, then the dense int8 route.  Checked against the
    table-lookup route (no offer) on the same call."""
    k, n, group = 8192, 28672, 128
    dev = torch.device("cuda:0")
    codes = torch.from_numpy(gen.i8_full(n * k // 2, 7).view("uint8")).to(dev)
    books = torch.from_numpy(gen.i8_full((n // group) * 16, 8)).to(dev)
    a = torch.from_numpy(gen.i8_full(m * k, 6)).to(dev)
    c = torch.zeros(m * n, dtype=torch.int32, device=dev)
    sc = torch.empty(uor.suggested_scratch_lut4(m, k, n), dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream()
    route = {}

    def step(scr=sc, cc=c):
        st, r = uor.gemm_lut4(a, m, k, (k, 1), codes, n, books, group, cc, (n, 1), scratch=scr,
                              stream=stream.cuda_stream)
        if st != 0:
            raise RuntimeError(f"lut4 status {st}")
        route.update(r)

    step()
    torch.cuda.synchronize()
    settle(torch, step)
    steps = max(1, min(args.steps, 20))
    s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s0.record(stream)
    for _ in range(steps):
        step()
    s1.record(stream)
    torch.cuda.synchronize()
    ms = s0.elapsed_time(s1) / steps
    kind = route.get("kind")
    ref = torch.zeros_like(c)
    step(None, ref)
    torch.cuda.synchronize()
    tops = 2.0 * m * n * k / (ms * 1e-3) / 1e12
    return {"m": m, "k": k, "n": n, "group": group, "route": kind, "ms_per_call": round(ms, 4),
            "TOPS": round(tops, 1), "frac_int8_mfma_peak": round(tops / PEAK_INT8_TOPS, 4),
            "parity_vs_lut_route": bool(torch.equal(c, ref))}


def bench_coded(args, torch, uor, gen):
    """Coded operands beyond the 4-bit grid: Ternary<4, u8> weights (2-bit
    digits, four per byte) at the config 3 shape (k = 8192, n = 28672, W
    n x k as gemm_tabulated declares it), at m = 1 and m = 2048, with the
    suggested offer: W decoded once per call into the scratch, then the dense
    int8 route.  Parity: the decode-free per-cell route on 16 output rows of
    the same call (the direct route over all rows would take seconds)."""
    import numpy as np
    k, n = 8192, 28672
    dev = torch.device("cuda:0")
    codes = torch.from_numpy(gen.i8_full(n * k // 4, 21).view("uint8")).to(dev)
    cd = uor.codec("ternary", code_bits=8, block=4)
    stream = torch.cuda.current_stream()
    runs = []
    for m in (1, 2048):
        a = torch.from_numpy(gen.i8_full(m * k, 22)).to(dev)
        c = torch.zeros(m * n, dtype=torch.int32, device=dev)
        sc = torch.empty(uor.suggested_scratch_coded(m, k, n), dtype=torch.uint8, device=dev)
        route = {}

        def step():
            st, r = uor.gemm_coded(a, (m, k), (k, 1), cd, codes, n, k, True, c, (m, n), (n, 1),
                                   scratch=sc, stream=stream.cuda_stream)
            if st != 0:
                raise RuntimeError(f"coded status {st}")
            route.update(r)

        step()
        torch.cuda.synchronize()
        settle(torch, step)
        steps = max(1, min(args.steps, 20))
        s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s0.record(stream)
        for _ in range(steps):
            step()
        s1.record(stream)
        torch.cuda.synchronize()
        ms = s0.elapsed_time(s1) / steps
        rows = min(m, 16)
        ref = torch.zeros(rows * n, dtype=torch.int32, device=dev)
        st, _ = uor.gemm_coded(a, (rows, k), (k, 1), cd, codes, n, k, True, ref, (rows, n),
                               (n, 1), stream=stream.cuda_stream)
        torch.cuda.synchronize()
        tops = 2.0 * m * n * k / (ms * 1e-3) / 1e12
        runs.append({"m": m, "k": k, "n": n, "codec": "Ternary<4, u8>", "route": route.get("kind"),
                     "ms_per_call": round(ms, 4), "TOPS": round(tops, 2),
                     "code_bytes": n * k // 4,
                     "parity_vs_direct_rows": rows if st == 0 and torch.equal(c[:rows * n], ref)
                     else False})
    return runs


def bench_collapse(args, torch, uor, gen):
    """The collapse traversal at the headline's size: m = n = k = 8192, A's
    rows drawn from 512 distinct rows (a batch of repeated inputs), alpha = 3,
    beta = 0, i32 out, with the suggested offer; the plain route beside it on
    the same operands, and the bytes compared."""
    import numpy as np
    N, D = 8192, 512
    dev = torch.device("cuda:0")
    base = torch.from_numpy(gen.i8_full(D * N, 31)).to(dev).view(D, N)
    pick = torch.from_numpy((gen.draws(N, 32) % np.uint64(D)).astype(np.int64)).to(dev)
    pick[:D] = torch.arange(D, device=dev)
    a = base[pick].contiguous().view(-1)
    b = torch.from_numpy(gen.i8_full(N * N, 33)).to(dev)
    c = torch.zeros(N * N, dtype=torch.int32, device=dev)
    ref = torch.zeros(N * N, dtype=torch.int32, device=dev)
    sc = torch.empty(uor.suggested_scratch_collapse(N, N, N), dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream()
    route = {}

    def collapsed():
        st, r = uor.gemm_collapsed_i8(a, (N, N), (N, 1), b, (N, N), (N, 1), c, (N, N), (N, 1),
                                      alpha=3, scratch=sc, stream=stream.cuda_stream)
        if st != 0:
            raise RuntimeError(f"collapsed status {st}")
        route.update(r)

    def plain():
        st, _ = uor.gemm_i8(a, (N, N), (N, 1), b, (N, N), (N, 1), ref, (N, N), (N, 1), alpha=3,
                            stream=stream.cuda_stream)
        if st != 0:
            raise RuntimeError(f"plain status {st}")

    def timed(step):
        step()
        torch.cuda.synchronize()
        settle(torch, step)
        steps = max(1, min(args.steps, 20))
        t0 = time.perf_counter()
        for _ in range(steps):
            step()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / steps * 1e3

    # Wall clock per call: the collapse route synchronises on its distinct
    # count, so stream events would not bracket it any better.
    ms_c = timed(collapsed)
    ms_p = timed(plain)
    return {"m": N, "k": N, "n": N, "distinct_rows": route.get("moduli"), "route": route.get("kind"),
            "ms_per_call": round(ms_c, 4), "plain_ms_per_call": round(ms_p, 4),
            "speedup": round(ms_p / ms_c, 2), "bytes_equal_plain": bool(torch.equal(c, ref))}


def bench_trop(args, torch, uor, gen):
    """Trop<i8> max-plus GEMM at m = n = k = 4096, 5% of entries
    at the semiring zero, output Trop<i32>.  One term is one (+, max) pair;
    the packed-i16 VALU ceiling is 256 CUs x 64 lanes x 2.4 GHz = 39.3e12
    terms/s (v_pk_add_u16 and v_pk_max_i16 each cover two terms)."""
    import numpy as np
    N = 4096
    dev = torch.device("cuda:0")
    rec = np.dtype([("value", "i1"), ("finite", "u1")])

    def recs(salt):
        v = gen.i8_full(N * N, salt)
        f = (gen.draws(N * N, 100 + salt) % np.uint64(20)) != 0
        r = np.zeros(N * N, rec)
        r["value"] = np.where(f, v, 0)
        r["finite"] = f
        return torch.from_numpy(r.view(np.uint8)).to(dev)

    a, b = recs(11), recs(12)
    c = torch.zeros(N * N * 8, dtype=torch.uint8, device=dev)
    c_sel = torch.zeros(N * N * 8, dtype=torch.uint8, device=dev)
    w = torch.zeros(N * N, dtype=torch.int64, device=dev)
    stream = torch.cuda.current_stream()

    def plain():
        st, _ = uor.gemm_trop_i8(a, (N, N), (N, 1), b, (N, N), (N, 1), c, (N, N), (N, 1),
                                 stream=stream.cuda_stream)
        if st != 0:
            raise RuntimeError(f"trop status {st}")

    def selected():
        st, _ = uor.gemm_trop_i8_selected(a, (N, N), (N, 1), b, (N, N), (N, 1), c_sel, (N, N),
                                          (N, 1), w, (N, 1), stream=stream.cuda_stream)
        if st != 0:
            raise RuntimeError(f"trop selected status {st}")

    def timed(step):
        for _ in range(max(1, args.warmup)):
            step()
        torch.cuda.synchronize()
        settle(torch, step)
        steps = max(10, min(args.steps, 50))
        s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s0.record(stream)
        for _ in range(steps):
            step()
        s1.record(stream)
        torch.cuda.synchronize()
        return s0.elapsed_time(s1) / steps

    terms = float(N) ** 3
    ms = timed(plain)
    if "cpu" in args.parts:
        CPU_INPUTS["trop"] = {"N": N, "a": a.cpu().numpy(), "b": b.cpu().numpy(),
                              "c": c.cpu().numpy()}
    rate = terms / (ms * 1e-3)
    ms_sel = timed(selected)
    rate_sel = terms / (ms_sel * 1e-3)
    # The witness route's C must be the plain route's bytes, and each witness
    # must attain its cell's value (a gather over all cells).
    rec_i32 = c_sel.view(N * N, 8)
    vals = rec_i32[:, :4].contiguous().view(torch.int32).view(N, N)
    fin = rec_i32[:, 4].view(N, N) != 0
    av = a.view(N, N, 2)
    bv = b.view(N, N, 2)
    W = w.view(N, N)
    rows = torch.arange(N, device=dev)[:, None].expand(N, N)
    cols = torch.arange(N, device=dev)[None, :].expand(N, N)
    ta = av[rows, W]
    tb = bv[W, cols]
    term = ta[..., 0].view(torch.int8).int() + tb[..., 0].view(torch.int8).int()
    attain = bool(((term == vals) & (ta[..., 1] != 0) & (tb[..., 1] != 0) | ~fin).all())
    return {"m": N, "n": N, "k": N, "out": "Trop<i32>", "ms_per_call": round(ms, 5),
            "terms_per_s": round(rate / 1e12, 3), "unit": "Tterm/s",
            "peak": PEAK_TROP_TERMS / 1e12, "frac_valu": round(rate / PEAK_TROP_TERMS, 4),
            "kernel": "trop_i8_kernel<true, false>", "bound": "valu",
            "selected": {"ms_per_call": round(ms_sel, 5), "terms_per_s": round(rate_sel / 1e12, 3),
                         "frac_valu": round(rate_sel / PEAK_TROP_TERMS, 4),
                         "kernel": "trop_i8_kernel<true, true>", "witness": "u64, least index",
                         "values_equal_plain": bool(torch.equal(c_sel, c)),
                         "witness_attains_value": attain}}


def bench_float(args, torch, uor, gen):
    """exact f32 GEMM at m = n = k = 4096 (random sign x [1, 2) x
    2^e, e in [-40, 40], 1% zeros, 1% cancelling pairs) with the suggested
    scratch offer (the CRT route), checked bit for bit against the direct
    route; and the f64 variant at 2048^3 with e in [-300, 300]."""
    dev = torch.device("cuda:0")
    out = []
    for is64, N in ((False, 4096), (True, 2048)):
        a = gen.float_config4(N, N, is64, 9)
        b = gen.float_config4(N, N, is64, 10)
        a, b = gen.cancel_pairs(a, b, 99)
        ga = torch.from_numpy(a.reshape(-1).copy()).to(dev)
        gb = torch.from_numpy(b.reshape(-1).copy()).to(dev)
        del a, b
        c = torch.zeros(N * N, dtype=torch.float64 if is64 else torch.float32, device=dev)
        size = uor.suggested_scratch_float(is64, N, N, N)
        sc = torch.empty(size, dtype=torch.uint8, device=dev) if size else None
        stream = torch.cuda.current_stream()
        route = {}

        def step(scr):
            st, r = uor.gemm_float(ga, (N, N), (N, 1), gb, (N, N), (N, 1), c, (N, N), (N, 1),
                                   scratch=scr, stream=stream.cuda_stream)
            if st != 0:
                raise RuntimeError(f"gemm_float status {st}")
            route.update(r)

        step(sc)
        torch.cuda.synchronize()
        settle(torch, lambda: step(sc))
        plan = None
        if sc is not None:
            off = (-sc.data_ptr()) % 256
            plan = sc[off:off + 12].cpu().view(torch.int32).tolist()
        steps = max(1, min(args.steps, 20)) if not is64 else max(3, min(args.steps, 5))
        s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s0.record(stream)
        for _ in range(steps):
            step(sc)
        s1.record(stream)
        torch.cuda.synchronize()
        ms = s0.elapsed_time(s1) / steps
        fast = c.clone()
        if "cpu" in args.parts:
            CPU_INPUTS.setdefault("float", []).append(
                {"is64": is64, "N": N, "a": ga.cpu().numpy(), "b": gb.cpu().numpy(),
                 "c": fast[:64 * N].cpu().numpy()})
        kind = route.get("kind")
        parity = None
        if sc is not None:
            step(None)
            torch.cuda.synchronize()
            parity = bool(torch.equal(fast.view(torch.int64 if is64 else torch.int32),
                                      c.view(torch.int64 if is64 else torch.int32)))
        run = {"format": "f64" if is64 else "f32", "m": N, "n": N, "k": N,
               "exponents": "[-300, 300]" if is64 else "[-40, 40]", "route": kind,
               "ms_per_call": round(ms, 4),
               "exact_TFLOP_s": round(2.0 * N ** 3 / (ms * 1e-3) / 1e12, 2),
               "parity_vs_direct_route": parity}
        if plan and plan[0] == 0 and not plan[1]:
            run["cells"] = "every line wider than the residue route's 160 bits: per-cell direct loop"
        if plan and plan[0] and not plan[1]:
            nmod = plan[0]
            kp = (N + 63) // 64 * 64
            run["moduli"] = nmod
            run["bound_bits"] = plan[2]
            run["int8_TOPS_issued"] = round(2.0 * N * N * kp * nmod / (ms * 1e-3) / 1e12, 1)
            run["frac_int8_mfma_peak"] = round(run["int8_TOPS_issued"] / PEAK_INT8_TOPS, 4)
        out.append(run)
        del ga, gb, c, sc, fast
        torch.cuda.empty_cache()
    return out


def bench_int(args, torch, uor):
    """The i16/i32/i64 element families (uor_gfx950_gemm_int): full-range
    random operands, alpha = 1, beta = 0, outputs wide enough to be exact (i64
    for i16 elements, i128 for i32 and i64).  Timed on the residue route with
    the suggested offer; 64 rows checked bit for bit against the per-cell
    route (no offer) on the same operands."""
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(21)
    out = []
    for eb, N, outt in ((2, 4096, "i64"), (4, 4096, "i128"), (8, 2048, "i128")):
        dt = {2: torch.int16, 4: torch.int32, 8: torch.int64}[eb]
        info = torch.iinfo(dt)
        a = torch.randint(info.min, info.max, (N * N,), dtype=dt, device=dev, generator=g)
        b = torch.randint(info.min, info.max, (N * N,), dtype=dt, device=dev, generator=g)
        rec = 2 if outt == "i128" else 1
        c = torch.zeros(N * N * rec, dtype=torch.int64, device=dev)
        size = uor.suggested_scratch_int(eb, N, N, N)
        sc = torch.empty(size, dtype=torch.uint8, device=dev)
        stream = torch.cuda.current_stream()
        route = {}

        def step():
            st, r = uor.gemm_int(a, (N, N), (N, 1), b, (N, N), (N, 1), c, (N, N), (N, 1), out=outt,
                                 scratch=sc, stream=stream.cuda_stream)
            if st != 0:
                raise RuntimeError(f"gemm_int status {st}")
            route.update(r)

        step()
        torch.cuda.synchronize()
        settle(torch, step)
        steps = max(1, min(args.steps, 10))
        s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s0.record(stream)
        for _ in range(steps):
            step()
        s1.record(stream)
        torch.cuda.synchronize()
        ms = s0.elapsed_time(s1) / steps
        R = 64
        slab = torch.zeros(R * N * rec, dtype=torch.int64, device=dev)
        st, _ = uor.gemm_int(a, (R, N), (N, 1), b, (N, N), (N, 1), slab, (R, N), (N, 1), out=outt)
        torch.cuda.synchronize()
        parity = st == 0 and bool(torch.equal(slab, c[:R * N * rec]))
        rec_ = {"elements": f"i{8 * eb}", "m": N, "n": N, "k": N, "out": outt,
                "route": route.get("kind"), "ms_per_call": round(ms, 4),
                "exact_TOPS": round(2.0 * N ** 3 / (ms * 1e-3) / 1e12, 2)}
        if route.get("kind") == "int_limb":
            # L = eb limbs per element: L^2 int8 products per exact product.
            issued = 2.0 * N ** 3 * eb * eb / (ms * 1e-3) / 1e12
            rec_.update({"limbs": eb, "plane_gemms": route.get("split_k")})
        else:
            off = (-sc.data_ptr()) % 256
            plan = sc[off:off + 12].cpu().view(torch.int32).tolist()
            nmod = plan[0]
            kp = (N + 63) // 64 * 64
            issued = 2.0 * N * N * kp * nmod / (ms * 1e-3) / 1e12
            rec_.update({"moduli": nmod, "bound_bits": plan[2]})
        rec_.update({"int8_TOPS_issued": round(issued, 1),
                     "frac_int8_mfma_peak": round(issued / PEAK_INT8_TOPS, 4),
                     "parity_vs_direct_route_64_rows": parity})
        out.append(rec_)
        del a, b, c, sc, slab
        torch.cuda.empty_cache()
    return out


def measured_peaks(torch):
    """Calibration probes (uor-matmul_amd/probe/peaks.hip, libuor_probe.so):
    the best HBM read rate of a plain grid-stride streaming kernel over three
    rotating 128 MiB buffers (384 MiB, beyond the 256 MB Infinity Cache), and
    the int8 MFMA rate of a 32x32x32 loop, one workgroup of four waves per
    CU, on random and on constant operands, with the shader clock the loop
    ran at (s_memtime ticks over s_memrealtime ticks times the wall-clock
    rate).  These are what the kernels can reach on this box; the roofline
    fractions are also reported against them."""
    import ctypes
    path = ROOT / "uor-matmul_amd" / "libuor_probe.so"
    if not path.exists():
        return None
    P = ctypes.CDLL(str(path))
    P.uor_probe_read.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_int, ctypes.c_int,
                                 ctypes.c_void_p, ctypes.c_void_p]
    P.uor_probe_mfma.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                 ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                 ctypes.POINTER(ctypes.c_int)]
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    nbytes = 128 << 20
    bufs = [torch.full((nbytes,), r + 1, dtype=torch.uint8, device=dev) for r in range(3)]
    sink = torch.zeros(16, dtype=torch.int32, device=dev)
    reads = []
    for bpc in (2, 4):
        for variant in range(4):
            def step(i):
                st = P.uor_probe_read(bufs[i % 3].data_ptr(), nbytes, bpc * cus, variant,
                                      sink.data_ptr(), stream.cuda_stream)
                if st != 0:
                    raise RuntimeError(f"probe read status {st}")
            for i in range(6):
                step(i)
            torch.cuda.synchronize()
            s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s0.record(stream)
            for i in range(60):
                step(i)
            s1.record(stream)
            torch.cuda.synchronize()
            us = s0.elapsed_time(s1) / 60 * 1e3
            reads.append({"blocks_per_cu": bpc, "unroll": 8 if variant & 2 else 4,
                          "nontemporal": bool(variant & 1), "us": round(us, 3),
                          "GB_s": round(nbytes / (us * 1e-6) / 1e9, 1)})
    best = max(reads, key=lambda r: r["GB_s"])
    del bufs
    out = {"hbm_read_GB_s": best["GB_s"], "hbm_read_best": best,
           "hbm_read_runs": reads}
    iters = 3000
    blocks = cus
    ops_n = blocks * 256 * 16 * 4
    clk = torch.zeros(2 * blocks, dtype=torch.int64, device=dev)
    for name, ops in (("random", torch.randint(-2 ** 31, 2 ** 31 - 1, (ops_n,), dtype=torch.int32,
                                               device=dev)),
                      ("constant", torch.full((ops_n,), 0x01010101, dtype=torch.int32, device=dev))):
        wall = ctypes.c_int(0)

        def run():
            st = P.uor_probe_mfma(ops.data_ptr(), blocks, iters, 4, clk.data_ptr(), sink.data_ptr(),
                                  stream.cuda_stream, ctypes.byref(wall))
            if st != 0:
                raise RuntimeError(f"probe mfma status {st}")
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < 0.3:  # the same settling as the kernels get
            run()
            torch.cuda.synchronize()
        s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s0.record(stream)
        for _ in range(5):
            run()
        s1.record(stream)
        torch.cuda.synchronize()
        ms = s0.elapsed_time(s1) / 5
        ops_done = blocks * 4 * iters * 32 * 65536.0
        c = clk.view(blocks, 2).cpu().double()
        mhz = float((c[:, 0] / c[:, 1]).mean() * wall.value / 1e3) if wall.value else None
        out[f"mfma_i8_{name}_TOPS"] = round(ops_done / (ms * 1e-3) / 1e12, 1)
        out[f"mfma_i8_{name}_clock_MHz"] = round(mhz, 1) if mhz else None
    return out


def bench_config1(args, torch, uor, gen):
    """slice::gemm i8 x i8 -> i32 at m = k = n = 1024, row-major,
    the reference's own xorshift operands (salts 1, 2), the suggested scratch
    offer; launch-bound at this size.  Checked in float64 (exact here)."""
    n = 1024
    dev = torch.device("cuda:0")
    a = gen.i8_full(n * n, 1)
    b = gen.i8_full(n * n, 2)
    ga, gb = torch.from_numpy(a).to(dev), torch.from_numpy(b).to(dev)
    gc = torch.zeros(n * n, dtype=torch.int32, device=dev)
    sc = torch.empty(uor.suggested_scratch_i8(n, n, n), dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream()

    def step():
        st = uor.slice_gemm_i8(n, n, n, ga, gb, gc, scratch=sc, stream=stream.cuda_stream)
        if st != 0:
            raise RuntimeError(f"slice::gemm status {st}")

    for _ in range(max(1, args.warmup)):
        step()
    torch.cuda.synchronize()
    settle(torch, step)
    steps = max(50, args.steps)
    s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s0.record(stream)
    for _ in range(steps):
        step()
    s1.record(stream)
    torch.cuda.synchronize()
    ms = s0.elapsed_time(s1) / steps
    A = ga.view(n, n).to(torch.float64)
    B = gb.view(n, n).to(torch.float64)
    want = A @ B
    parity = bool(torch.equal(gc.view(n, n).to(torch.float64), want))

    # The same calls captured in a HIP graph (50 per graph, replayed): the
    # device's time per call without the host's per-call cost (Python, ctypes
    # and the launch), which bounds the eager loop above at this size.
    per_graph = 50
    gc.zero_()
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        uor.slice_gemm_i8(n, n, n, ga, gb, gc, scratch=sc, stream=side.cuda_stream)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        cs = torch.cuda.current_stream().cuda_stream
        for _ in range(per_graph):
            if uor.slice_gemm_i8(n, n, n, ga, gb, gc, scratch=sc, stream=cs) != 0:
                raise RuntimeError("slice::gemm status under capture")
    graph.replay()
    torch.cuda.synchronize()
    replays = max(4, steps // per_graph)
    g0, g1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    g0.record(stream)
    for _ in range(replays):
        graph.replay()
    g1.record(stream)
    torch.cuda.synchronize()
    ms_graph = g0.elapsed_time(g1) / (replays * per_graph)
    gc.zero_()
    graph.replay()
    torch.cuda.synchronize()
    parity = parity and bool(torch.equal(gc.view(n, n).to(torch.float64), want))
    del graph
    return {"config": "BASELINE configs[0]: slice::gemm i8 -> i32, 1024^3, xorshift operands, "
                      "suggested offer", "m": n, "k": n, "n": n, "ms_per_call": round(ms, 5),
            "TOPS": round(2.0 * n ** 3 / (ms * 1e-3) / 1e12, 1),
            "ms_per_call_graph": round(ms_graph, 5),
            "TOPS_graph": round(2.0 * n ** 3 / (ms_graph * 1e-3) / 1e12, 1), "parity": parity}


def cpu_threads():
    """The worker count for the CPU leg: every core this process may run on,
    at most 16 (one GPU's share of the GPU box's cores)."""
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = os.cpu_count() or 1
    return max(1, min(usable, 16)), usable


def cpu_host():
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    threads, usable = cpu_threads()
    return {"cpu_model": model, "logical_cpus": os.cpu_count(), "usable_cpus": usable,
            "threads_used": threads}


def median_time(fn, runs=5):
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return sorted(times)[len(times) // 2]


def cpu_baseline_i8(host, oracle):
    """The reference's packed route restated (oracle/fastroute.cpp) on the
    same 8192^3 problem: a row slab sized to about 12 s of CPU work (the whole
    problem when it takes less) on all usable cores, median of three runs each
    from the same C; then 256 rows on one core.  Rows 0..8 of both are checked
    against the oracle."""
    import numpy as np
    a, b, c0 = host
    N, LD = 8192, 8256
    threads, _ = cpu_threads()
    c = c0.copy()
    t0 = time.perf_counter()
    oracle.fast_gemm_i8_i32(N, N, N, 3, a, LD, b, LD, -1, c, LD, row0=0, rows=128, threads=threads)
    dt = time.perf_counter() - t0
    rows = int(min(N, max(128, 12.0 / max(dt, 1e-3) * 128)) // 128 * 128)

    def run():
        c[:] = c0
        oracle.fast_gemm_i8_i32(N, N, N, 3, a, LD, b, LD, -1, c, LD, row0=0, rows=rows,
                                threads=threads)

    dt = median_time(run, runs=5)
    rows1 = 256
    c1 = c0.copy()
    t0 = time.perf_counter()
    oracle.fast_gemm_i8_i32(N, N, N, 3, a, LD, b, LD, -1, c1, LD, row0=0, rows=rows1, threads=1)
    dt1 = time.perf_counter() - t0
    want = c0[:8 * LD].copy()
    st = oracle.gemm_int(a[:8 * LD], (8, N), (LD, 1), b, (N, N), (LD, 1), want, (8, N), (LD, 1),
                         alpha=3, beta=-1)
    ok = st == "ok" and bool(np.array_equal(c[:8 * LD], want)) and \
        bool(np.array_equal(c1[:8 * LD], want))
    vnni = bool(oracle.fast().fr_has_vnni())
    return {
        "value": round(2.0 * rows * N * N / dt / 1e12, 4),
        "unit": "TOPS",
        "cores": threads,
        "kind": "port",
        "sample": f"rows 0..{rows} of the 8192^3 gemm_ex (alpha=3, beta=-1), median {dt:.2f} s "
                  f"of 5 runs on {threads} threads, {'AVX-512 VNNI dpbusd' if vnni else 'AVX2'} "
                  "8x16 tile; rows are independent so TOPS scale to the full problem",
        "one_core": {"value": round(2.0 * rows1 * N * N / dt1 / 1e12, 4), "unit": "TOPS",
                     "sample": f"rows 0..{rows1}, {dt1:.2f} s (B packed once)"},
        "rows_0_8_equal_oracle": ok,
        "host": cpu_host(),
    }


def cpu_baselines_secondary(oracle):
    """CPU restatements for the secondary configs, each checked byte for byte
    against the GPU's output on the same inputs:
      LUT decode: tabulation and decode-then-dense, one call per
        codebook group (224 calls), all groups on all cores, the first 28
        groups on one core (extrapolated x 8);
      max-plus: the AVX2_TROP_I16 tile, all 4096 rows on all
        cores, 256 rows on one core (extrapolated);
      deep case (configs[1] 2b): the chunked route on a k-sample, extrapolated,
        every output checked against the closed form;
      exact float: the oracle's per-product exact register on a
        64-row slab on all cores (extrapolated to the full problem), 8 rows on
        one core."""
    import numpy as np
    from concurrent.futures import ThreadPoolExecutor
    threads, _ = cpu_threads()
    out = {"host": cpu_host()}
    lut = CPU_INPUTS.get("lut")
    if lut:
        k, n, group = lut["k"], lut["n"], lut["group"]
        runs = []
        for m, (a, want) in sorted(lut["runs"].items()):
            nbytes = n * k // 2 + m * k + 4 * m * n + (n // group) * 16
            rec = {"m": m}
            for mode in ("tabulate", "decode_dense"):
                c = np.full(m * n, -7, np.int32)
                ms = 1e3 * median_time(lambda: oracle.fast_lut4(m, k, n, a, lut["codes"],
                                                                lut["books"], group, c,
                                                                threads=threads, mode=mode))
                ok = bool(np.array_equal(c, want))
                c1 = np.full(m * n, -7, np.int32)
                ms1 = 1e3 * median_time(lambda: oracle.fast_lut4(m, k, n, a, lut["codes"],
                                                                 lut["books"], group, c1,
                                                                 groups=28, threads=1,
                                                                 mode=mode), runs=3) * 8
                rec[mode] = {"ms_per_call": round(ms, 3), "GB_s": round(nbytes / ms / 1e6, 2),
                             "one_core_ms_extrapolated": round(ms1, 2),
                             "bytes_equal_gpu": ok}
            best = min(("tabulate", "decode_dense"), key=lambda md: rec[md]["ms_per_call"])
            rec["best"] = best
            runs.append(rec)
        out["lut"] = {"unit": "GB/s of algorithmic bytes", "cores": threads, "kind": "port",
                      "runs": runs}
    trop = CPU_INPUTS.get("trop")
    if trop:
        N = trop["N"]
        c = np.full(N * N * 8, 0xEE, np.uint8)
        dt = median_time(lambda: oracle.fast_trop_i8(N, N, N, trop["a"], trop["b"], c,
                                                    threads=threads), runs=5)
        g, w = c.reshape(-1, 8), trop["c"].reshape(-1, 8)
        ok = bool(np.array_equal(g[:, :5], w[:, :5]))
        c1 = np.full(N * N * 8, 0xEE, np.uint8)
        rows1 = 256
        dt1 = median_time(lambda: oracle.fast_trop_i8(N, N, N, trop["a"], trop["b"], c1, rows=rows1,
                                                     threads=1), runs=1)
        out["trop"] = {"value": round(float(N) ** 3 / dt / 1e12, 4), "unit": "Tterm/s",
                       "cores": threads, "kind": "port", "ms_per_call": round(dt * 1e3, 1),
                       "sample": "the whole 4096^3 product", "bytes_equal_gpu": ok,
                       "one_core": {"value": round(rows1 * float(N) ** 2 / dt1 / 1e12, 4),
                                    "sample": f"rows 0..{rows1}, B packing included"}}
    # Deep case (configs[1] 2b): m = n = 128, A = B = -128, the chunked route
    # on a k-sample of 2^21 of the 2^24 (k-chunks are independent sums),
    # extrapolated x 8; every output must be ksample * 2^14.
    if CPU_INPUTS.get("deep"):
        M, KS, KFULL = 128, 1 << 21, 1 << 24
        a = np.full(M * KS, -128, np.int8)
        c = np.zeros(M * M, np.int64)

        def deep(th, kk):
            c[:] = 7
            oracle.fast_gemm_i8_i64_chunked(M, kk, M, a, kk, a, M, c, M, threads=th)

        dt = median_time(lambda: deep(threads, KS), runs=5)
        ok = bool((c == KS * 16384).all())
        dt1 = median_time(lambda: deep(1, KS // 4), runs=1)
        ok = ok and bool((c == (KS // 4) * 16384).all())
        full_s = dt * KFULL / KS
        out["deep"] = {"value": round(2.0 * M * M * KFULL / full_s / 1e12, 4), "unit": "TOPS",
                       "GB_s": round(2.0 * M * KFULL / full_s / 1e9, 2), "cores": threads,
                       "kind": "port",
                       "sample": f"k = 2^21 of 2^24 (A = B = -128) in {dt * 1e3:.1f} ms, median of 5, "
                                 "extrapolated x 8 (k-chunks are independent sums)",
                       "outputs_equal_closed_form": ok,
                       "one_core": {"value": round(2.0 * M * M * (KS // 4) / dt1 / 1e12, 4),
                                    "sample": f"k = 2^19 in {dt1 * 1e3:.1f} ms"}}
        del a
    for fl in CPU_INPUTS.get("float", []):
        N, is64 = fl["N"], fl["is64"]
        ft = np.float64 if is64 else np.float32
        a, b = fl["a"], fl["b"]
        rows = 64

        def slab(r0, r1, c):
            return oracle.gemm_float(a[r0 * N:r1 * N], (r1 - r0, N), (N, 1), b, (N, N), (N, 1),
                                     c[r0 * N:r1 * N], (r1 - r0, N), (N, 1))

        c = np.full(rows * N, np.nan, ft)
        cuts = [rows * t // threads for t in range(threads + 1)]
        sts = []

        def run_slab():
            c[:] = np.nan
            with ThreadPoolExecutor(threads) as pool:
                sts[:] = list(pool.map(lambda t: slab(cuts[t], cuts[t + 1], c), range(threads)))

        dt = median_time(run_slab, runs=3)
        ok = all(st == "ok" for st in sts) and bool(np.array_equal(
            c.view(np.uint64 if is64 else np.uint32), fl["c"].view(np.uint64 if is64 else np.uint32)))
        rows1 = 8
        c1 = np.full(rows * N, np.nan, ft)
        t0 = time.perf_counter()
        slab(0, rows1, c1)
        dt1 = time.perf_counter() - t0
        full_s = dt * N / rows
        out.setdefault("float", []).append({
            "format": "f64" if is64 else "f32", "m": N, "n": N, "k": N,
            "value": round(2.0 * N ** 3 / full_s / 1e9, 3), "unit": "exact GFLOP/s",
            "cores": threads, "kind": "port",
            "sample": f"rows 0..{rows} in {dt:.2f} s (median of 3), extrapolated x{N // rows} "
                      "(rows are independent)",
            "full_problem_s_extrapolated": round(full_s, 1),
            "ns_per_product_per_core": round(dt * threads / (rows * N * N) * 1e9, 2),
            "bytes_equal_gpu": ok,
            "one_core": {"value": round(2.0 * rows1 * N * N / dt1 / 1e9, 3),
                         "sample": f"rows 0..{rows1} in {dt1:.2f} s"}})
    return out


PARTS = ["i8", "config1", "deep", "lut", "prefill", "coded", "collapse", "trop", "float", "int",
         "peaks", "cpu"]


def main():
    global SETTLE_S
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-lut", action="store_true", help="skip the secondary LUT decode figure")
    ap.add_argument("--no-trop", action="store_true", help="skip the secondary max-plus figure")
    ap.add_argument("--no-float", action="store_true", help="skip the secondary exact-float figure")
    ap.add_argument("--no-int", action="store_true", help="skip the i16/i32/i64 element figure")
    ap.add_argument("--only", default=None,
                    help="comma-separated parts to run (" + ",".join(PARTS) + "), e.g. for a "
                         "profiler run of one kernel family; the line then holds only those")
    ap.add_argument("--settle", type=float, default=SETTLE_S,
                    help="seconds of untimed running before each timed region (0 under a profiler)")
    ap.add_argument("--lut-m", default="1,8,32", help="LUT decode row counts")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run one plain 1 GiB device-to-device copy and exit (the known-size "
                         "reference that scales rocprofv3 FETCH_SIZE/WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(sharding is design-only); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    SETTLE_S = max(0.0, args.settle)
    if args.only:
        parts = set(x.strip() for x in args.only.split(",") if x.strip())
        unknown = parts - set(PARTS)
        if unknown:
            ap.error(f"unknown parts {sorted(unknown)}")
    else:
        parts = set(PARTS)
        if args.no_lut:
            parts -= {"lut", "prefill", "coded", "collapse"}
        if args.no_trop:
            parts.discard("trop")
        if args.no_float:
            parts.discard("float")
        if args.no_int:
            parts.discard("int")
        if args.no_cpu_baseline:
            parts.discard("cpu")
    args.parts = parts
    import torch
    if args.copy_calibration:
        n = 1 << 30
        src = torch.ones(n, dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": n}), flush=True)
        return
    import uor_gfx950 as uor
    import gen
    uor.lib()
    result, host = {"metric": METRIC, "parts": sorted(parts)}, None
    if "i8" in parts:
        result, host = bench_i8(args, torch, uor, gen)
    if "config1" in parts:
        log("[bench] config 1 (1024^3 slice::gemm)")
        result["config1"] = bench_config1(args, torch, uor, gen)
    if "deep" in parts:
        log("[bench] deep reduction")
        result["deep"] = {
            "metric": "deep exact i8 GEMM GB/s (% HBM peak)",
            "config": "BASELINE configs[1] deep case: m=n=128, k=2^24, A=B=-128, i64 out",
            "run": bench_deep(args, torch, uor),
        }
    if "lut" in parts:
        log("[bench] lut4 decode")
        ms_list = tuple(int(x) for x in args.lut_m.split(",") if x)
        result["secondary"] = {
            "metric": "LUT-GEMM decode GB/s (% HBM peak)",
            "unit": "GB/s",
            "peak": PEAK_HBM_GBS,
            "config": "BASELINE configs[2]: 4-bit codes, k=8192, n=28672, group=128, "
                      "3 rotating code buffers (>256 MB MALL)",
            "runs": bench_lut4(args, torch, uor, gen, ms_list),
        }
    if "prefill" in parts:
        log("[bench] lut4 prefill")
        result.setdefault("secondary", {})["prefill"] = bench_lut_prefill(args, torch, uor, gen)
    if "coded" in parts:
        log("[bench] coded operands")
        result.setdefault("secondary", {})["ternary"] = bench_coded(args, torch, uor, gen)
    if "collapse" in parts:
        log("[bench] collapse")
        result["collapse"] = bench_collapse(args, torch, uor, gen)
    if "trop" in parts:
        log("[bench] trop max-plus")
        result["tropical"] = {
            "metric": "Trop<i8> max-plus terms/s (% packed-i16 VALU peak)",
            "config": "BASELINE configs[4]: m=n=k=4096, 5% -inf entries, Trop<i32> output",
            "run": bench_trop(args, torch, uor, gen),
        }
    if "float" in parts:
        log("[bench] exact float")
        result["float"] = {
            "metric": "exact float GEMM TFLOP/s (2mnk per second, rounded once)",
            "config": "BASELINE configs[3]",
            "runs": bench_float(args, torch, uor, gen),
        }
    if "int" in parts:
        log("[bench] i16/i32/i64 elements")
        result["integer"] = {
            "metric": "exact integer GEMM TOPS (2mnk per second), i16/i32/i64 elements",
            "config": "the Kernelized i16/i32/i64 families, full-range operands",
            "runs": bench_int(args, torch, uor),
        }
    if "peaks" in parts:
        log("[bench] measured peaks")
        peaks = measured_peaks(torch)
        if peaks:
            result["measured_peaks"] = peaks
            if "roofline" in result and peaks.get("mfma_i8_random_TOPS"):
                rf = result["roofline"]
                rf["measured_peak"] = peaks["mfma_i8_random_TOPS"]
                rf["frac_measured_peak"] = round(rf["achieved"] / peaks["mfma_i8_random_TOPS"], 4)
            for r in result.get("secondary", {}).get("runs", []):
                r["frac_measured_read_peak"] = round(r["GB_s"] / peaks["hbm_read_GB_s"], 4)
    if "cpu" in parts and host is not None:
        from oracle import oracle
        log("[bench] cpu baseline")
        result["cpu_baseline"] = cpu_baseline_i8(host, oracle)
    if "cpu" in parts and CPU_INPUTS:
        from oracle import oracle
        log("[bench] cpu baselines, secondary configs")
        result["cpu_baselines_secondary"] = cpu_baselines_secondary(oracle)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
