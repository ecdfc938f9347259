"""The input generator: `draws` is the reference's fill sequence
(crates/uor-matmul-validate/tests/massive.rs:42-53) at every lane split."""
import numpy as np
import pytest

import gen


@pytest.mark.parametrize("n,lanes", [(1, 16), (7, 3), (1000, 64), (5000, 1 << 16),
                                     (100003, 97), (65537, 1 << 16)])
def test_jump_ahead_draws_are_the_sequential_sequence(n, lanes):
    for salt in (1, 2, 0x5151):
        assert np.array_equal(gen.draws(n, salt, lanes), gen.xorshift_draws(n, salt))


def test_first_draws_by_hand():
    """The first draws of fill(.., salt 1), stepped here with Python ints."""
    s = 0x243F6A8885A308D3 ^ 1
    want = []
    for _ in range(4):
        s ^= (s << 13) & ((1 << 64) - 1)
        s ^= s >> 7
        s ^= (s << 17) & ((1 << 64) - 1)
        want.append(s >> 33)
    assert gen.draws(4, 1).tolist() == want
    assert gen.i8_full(4, 1).tolist() == [((v & 0xFF) ^ 0x80) - 0x80 for v in want]
