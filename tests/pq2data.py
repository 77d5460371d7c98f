"""PQ2_0 product test data, including the data of the reference's own unit
tests for this path, regenerated with their generators and call order:

- ``avx2_case()``: src/kernels.rs:857-907 (avx2_row_dot_matches_scalar):
  xorshift64 (13, 7, 17) seeded 0x123456789abcdef0, ne0 5120, 8 rows, block
  scales 0.5 + k/1000 through the test's own truncating f32->f16, random code
  bytes, x in [-2, 2] in steps of 1/500;
- ``matmul_case()``: src/kernels.rs:910-946 (pq2_matmul_n_matches_per_token_matvec):
  xorshift32 (13, 17, 5) seeded 0x12345678, ne0 256, 12 rows, 3 tokens,
  scales f32_to_half(k/250 + 0.01).
"""
from __future__ import annotations

import numpy as np

M64 = (1 << 64) - 1
M32 = (1 << 32) - 1


def _xorshift64(seed: int):
    s = seed
    while True:
        s ^= (s << 13) & M64
        s ^= s >> 7
        s ^= (s << 17) & M64
        yield s


def _xorshift32(seed: int):
    s = seed
    while True:
        s ^= (s << 13) & M32
        s ^= s >> 17
        s ^= (s << 5) & M32
        yield s


def _trunc_f16(v: np.float32) -> int:
    """The avx2 test's converter (finite positive values, mantissa truncated)."""
    b = int(np.float32(v).view(np.uint32))
    sign = (b >> 16) & 0x8000
    exp = ((b >> 23) & 0xFF) - 127 + 15
    mant = (b & 0x7FFFFF) >> 13
    return (sign | ((exp << 10) | mant)) & 0xFFFF


def avx2_case():
    """(payload uint8 [8*1360], x f32 [5120], ne0, n_rows)."""
    ne0, n_rows = 5120, 8
    rb = (ne0 + 127) // 128 * 34
    raw = np.zeros(rb * n_rows, np.uint8)
    nxt = _xorshift64(0x1234_5678_9ABC_DEF0)
    for r in range(n_rows):
        for b in range(ne0 // 128):
            base = r * rb + b * 34
            sc = np.float32(0.5) + np.float32((next(nxt) >> 8) % 1000) / np.float32(1000.0)
            h = _trunc_f16(sc)
            raw[base] = h & 0xFF
            raw[base + 1] = h >> 8
            for k in range(32):
                raw[base + 2 + k] = next(nxt) % 256
    x = np.array([(np.float32(next(nxt) % 2001) - np.float32(1000.0)) / np.float32(500.0)
                  for _ in range(ne0)], np.float32)
    return raw, x, ne0, n_rows


def matmul_case(f32_to_half):
    """(payload uint8 [12*68], x f32 [3, 256], ne0, n_rows, n_tok)."""
    ne0, n_rows, n_tok = 256, 12, 3
    rb = (ne0 + 127) // 128 * 34
    nxt = _xorshift32(0x1234_5678)
    payload = np.zeros(n_rows * rb, np.uint8)
    for r in range(n_rows):
        for blk in range(ne0 // 128):
            base = r * rb + blk * 34
            v = np.float32(next(nxt) % 500) / np.float32(250.0) + np.float32(0.01)
            h = int(f32_to_half(np.array([v], np.float32))[0])
            payload[base] = h & 0xFF
            payload[base + 1] = h >> 8
            for k in range(32):
                payload[base + 2 + k] = next(nxt) % 256
    x = np.array([(np.float32(next(nxt) % 2001) - np.float32(1000.0)) / np.float32(500.0)
                  for _ in range(n_tok * ne0)], np.float32).reshape(n_tok, ne0)
    return payload, x, ne0, n_rows, n_tok


def decoded(payload: np.ndarray, ne0: int, n_rows: int, base_row: int = 0) -> np.ndarray:
    """Weights [n_rows, ne0] as float64 (numpy, independent of the oracle):
    (code - 1) * f16 scale, codes LSB first."""
    rb = (ne0 + 127) // 128 * 34
    nblk = rb // 34
    rows = payload[base_row * rb:(base_row + n_rows) * rb].reshape(n_rows, nblk, 34)
    scales = rows[:, :, :2].copy().view(np.float16).astype(np.float64).reshape(n_rows, nblk)
    qs = rows[:, :, 2:]
    codes = np.stack([(qs >> (2 * k)) & 3 for k in range(4)], axis=-1).reshape(n_rows, nblk, 128)
    w = (codes.astype(np.float64) - 1.0) * scales[:, :, None]
    return w.reshape(n_rows, nblk * 128)[:, :ne0]
