"""Deterministic synthetic inputs shared by tests and bench.py.

`fill` is the reference corpus generator: xorshift64 (13, 7, 17) seeded with
0x243F6A8885A308D3 ^ salt, one draw per element, value (s >> 33)
(crates/uor-matmul-validate/tests/massive.rs:42-53), vectorised over
independent lanes for large sizes (each lane is its own xorshift stream
seeded from the salt and the lane index) so multi-GiB fills take seconds.
"""
from __future__ import annotations

import numpy as np

SEED = 0x243F6A8885A308D3
M64 = (1 << 64) - 1


def xorshift_draws(n: int, salt: int) -> np.ndarray:
    """The reference's exact sequence of (s >> 33) draws (uint64), n of them."""
    s = (SEED ^ salt) & M64
    out = np.empty(n, dtype=np.uint64)
    for i in range(n):
        s ^= (s << 13) & M64
        s ^= s >> 7
        s ^= (s << 17) & M64
        out[i] = s >> 33
    return out


def lanes_draws(n: int, salt: int, lanes: int = 1 << 16) -> np.ndarray:
    """n draws from `lanes` independent xorshift streams (round robin)."""
    lanes = max(1, min(lanes, n))
    idx = np.arange(lanes, dtype=np.uint64)
    s = (np.uint64(SEED) ^ np.uint64(salt)) ^ (idx * np.uint64(0x9E3779B97F4A7C15))
    s[s == 0] = np.uint64(1)
    rounds = (n + lanes - 1) // lanes
    out = np.empty(rounds * lanes, dtype=np.uint64)
    sh13, sh7, sh17, sh33 = np.uint64(13), np.uint64(7), np.uint64(17), np.uint64(33)
    for r in range(rounds):
        s ^= s << sh13
        s ^= s >> sh7
        s ^= s << sh17
        out[r * lanes:(r + 1) * lanes] = s >> sh33
    return out[:n]


def i8_full(n: int, salt: int, exact_sequence: bool = False) -> np.ndarray:
    """Uniform over all 256 i8 values: (s >> 33) as u8 as i8."""
    d = xorshift_draws(n, salt) if exact_sequence else lanes_draws(n, salt)
    return (d & np.uint64(0xFF)).astype(np.uint8).view(np.int8)


def i32_pm2_20(n: int, salt: int) -> np.ndarray:
    """Uniform i32 in [-2^20, 2^20]: (s >> 33) mod (2^21 + 1) - 2^20."""
    d = lanes_draws(n, salt)
    return ((d % np.uint64((1 << 21) + 1)).astype(np.int64) - (1 << 20)).astype(np.int32)
