"""Synthetic inputs of the five benchmark configurations.

Host generator: SplitMix64 (the generator of the reference's sampler,
src/sampler.rs:15-21) in counter form -- output i is mix(seed + (i+1)*gamma),
identical to i+1 sequential next_u64() calls -- feeding Box-Muller in f64,
rounded to f32.  The same bytes go to the CPU oracle and to the GPU.

PQ2_0 tables: per weight a code in {0,1,2} with probabilities {0.3,0.4,0.3}
(values -1, 0, +1), per 128-weight block an f16 scale |N(0, 0.02)| converted
with the reference's f32_to_half (src/gguf.rs:914-944, restated vectorised
below).  Block layout as src/kernels.rs:204-229.
"""
from __future__ import annotations

import numpy as np

GAMMA = np.uint64(0x9E3779B97F4A7C15)
M1 = np.uint64(0xBF58476D1CE4E5B9)
M2 = np.uint64(0x94D049BB133111EB)
QK = 128
BLOCK_BYTES = 34


def splitmix64(seed: int, start: int, n: int) -> np.ndarray:
    """Outputs start..start+n-1 of SplitMix64(seed) as uint64."""
    idx = np.arange(start + 1, start + n + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + idx * GAMMA
        z = (z ^ (z >> np.uint64(30))) * M1
        z = (z ^ (z >> np.uint64(27))) * M2
    return z ^ (z >> np.uint64(31))


class Rng:
    """Counter-based SplitMix64 stream with f64 uniform / normal draws."""

    def __init__(self, seed: int):
        self.seed = seed
        self.pos = 0

    def u64(self, n: int) -> np.ndarray:
        out = splitmix64(self.seed, self.pos, n)
        self.pos += n
        return out

    def uniform(self, n: int) -> np.ndarray:
        """f64 in [0, 1), as Rng::next_f64 (src/sampler.rs:24-26)."""
        return (self.u64(n) >> np.uint64(11)).astype(np.float64) / float(1 << 53)

    def normal(self, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
        """float32 N(mean, std) by Box-Muller in f64."""
        m = (n + 1) // 2
        u = self.uniform(2 * m)
        r = np.sqrt(-2.0 * np.log1p(-u[0::2]))
        th = 2.0 * np.pi * u[1::2]
        z = np.empty(2 * m, dtype=np.float64)
        z[0::2] = r * np.cos(th)
        z[1::2] = r * np.sin(th)
        return (mean + std * z[:n]).astype(np.float32)


def f32_to_half(v: np.ndarray) -> np.ndarray:
    """Vectorised restatement of gguf::f32_to_half (src/gguf.rs:914-944)."""
    b = np.ascontiguousarray(v, dtype=np.float32).view(np.uint32).astype(np.int64)
    sign = (b >> 16) & 0x8000
    exp = (b >> 23) & 0xFF
    man = b & 0x7FFFFF
    e = exp - 127 + 15
    out = np.zeros(b.shape, dtype=np.int64)
    # normal range
    half = (e << 10) | (man >> 13)
    rem = man & 0x1FFF
    rnd = (rem > 0x1000) | ((rem == 0x1000) & ((half & 1) == 1))
    normal = (half + rnd) & 0xFFFF
    # subnormal range (-10 <= e <= 0); shift is clipped to stay defined
    sh = np.clip(1 - e, 0, 31)
    m = (man | 0x800000) >> sh
    hs = m >> 13
    rs = m & 0x1FFF
    rnds = (rs > 0x1000) | ((rs == 0x1000) & ((hs & 1) == 1))
    sub = hs + rnds
    out = np.where(e > 0, normal, out)
    out = np.where((e <= 0) & (e >= -10), sub, out)
    out = np.where(e >= 0x1F, 0x7C00, out)
    nanm = np.where(man != 0, 0x200, 0)
    out = np.where(exp == 0xFF, 0x7C00 | nanm, out)
    return (sign | out).astype(np.uint16)


def pack_pq2_rows(codes: np.ndarray, scales_f16: np.ndarray) -> np.ndarray:
    """codes uint8 [rows, ne0] in 0..3, scales uint16 [rows, ceil(ne0/128)]
    -> packed uint8 [rows, row_bytes]."""
    rows, ne0 = codes.shape
    nblk = (ne0 + QK - 1) // QK
    padded = np.zeros((rows, nblk * QK), dtype=np.uint8)
    padded[:, :ne0] = codes
    q = padded.reshape(rows, nblk, QK // 4, 4).astype(np.uint8)
    packed = (q[..., 0] | (q[..., 1] << 2) | (q[..., 2] << 4) | (q[..., 3] << 6)).astype(np.uint8)
    out = np.empty((rows, nblk, BLOCK_BYTES), dtype=np.uint8)
    sc = np.ascontiguousarray(scales_f16, dtype="<u2").reshape(rows, nblk)
    out[..., 0] = (sc & 0xFF).astype(np.uint8)
    out[..., 1] = (sc >> 8).astype(np.uint8)
    out[..., 2:] = packed
    return out.reshape(rows, nblk * BLOCK_BYTES)


def pq2_table(rng: Rng, rows: int, ne0: int, scale_std: float = 0.02,
              probs=(0.3, 0.4, 0.3)) -> np.ndarray:
    """Packed PQ2_0 table [rows, row_bytes] with the config's distributions."""
    nblk = (ne0 + QK - 1) // QK
    u = rng.uniform(rows * ne0).reshape(rows, ne0)
    c0, c1 = probs[0], probs[0] + probs[1]
    codes = np.where(u < c0, 0, np.where(u < c1, 1, 2)).astype(np.uint8)
    scales = np.abs(rng.normal(rows * nblk, 0.0, scale_std))
    return pack_pq2_rows(codes, f32_to_half(scales).reshape(rows, nblk))


def positions(n_tok: int) -> np.ndarray:
    """Text positions: p_t = p_h = p_w = p_e = token index, int32 [n_tok, 4]."""
    p = np.arange(n_tok, dtype=np.int32)
    return np.repeat(p[:, None], 4, axis=1).copy()


# ---------------------------------------------------------------------------
# device-side generation for benchmark-sized buffers (torch RNG; the values
# only need the configured distributions, parity is not checked on them)
# ---------------------------------------------------------------------------

def torch_pq2_table(rows: int, ne0: int, device, generator=None, chunk_rows: int = 16384):
    """Packed PQ2_0 table built on the device, same distributions."""
    import torch
    nblk = (ne0 + QK - 1) // QK
    rb = nblk * BLOCK_BYTES
    table = torch.empty((rows, rb), dtype=torch.uint8, device=device)
    for r0 in range(0, rows, chunk_rows):
        r1 = min(rows, r0 + chunk_rows)
        n = r1 - r0
        u = torch.rand((n, nblk, QK), device=device, generator=generator)
        codes = (u >= 0.3).to(torch.int32) + (u >= 0.7).to(torch.int32)
        q = codes.view(n, nblk, QK // 4, 4)
        packed = (q[..., 0] | (q[..., 1] << 2) | (q[..., 2] << 4) | (q[..., 3] << 6))
        sc = (torch.randn((n, nblk), device=device, generator=generator) * 0.02).abs()
        sc16 = sc.to(torch.float16).view(torch.int16).to(torch.int32) & 0xFFFF
        blk = table[r0:r1].view(n, nblk, BLOCK_BYTES)
        blk[..., 0] = (sc16 & 0xFF).to(torch.uint8)
        blk[..., 1] = (sc16 >> 8).to(torch.uint8)
        blk[..., 2:] = packed.to(torch.uint8)
    return table
