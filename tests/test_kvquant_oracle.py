"""Pins the oracle's restatement of the planar-quantized KV cache
(src/kvquant.rs PlanarQuant; the quantized branches of src/forward.rs
:99-140, 296-349) before the HIP kernels are checked against it.

  * the reference's own unit tests (src/kvquant.rs:578-851), restated with
    their xorshift generator, seeds and bounds;
  * independent restatements: the Lloyd-Max centroids from scipy's exact erf
    (the reference uses a 1.5e-7 approximation), the Givens table from a
    Python splitmix64 and math.cos/sin, quantize as float32 numpy steps
    (sequential norm, rotation, first-minimum nearest centroid);
  * attention over the quantized caches equal to plain attention over the
    dequantized caches (rotation is orthogonal and linear, so the scores and
    the inverse-rotated P.V agree up to rounding): a wrong rotation
    direction, a dropped norm or a misplaced index fails by orders of
    magnitude.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from conftest import rel_err

HD = 256


def xorshift(seed: int):
    """rng() of src/kvquant.rs:581-589: values in [-1, 1)."""
    s = (seed | 1) & (2**64 - 1)

    def nxt():
        nonlocal s
        s ^= (s << 13) & (2**64 - 1)
        s ^= s >> 7
        s ^= (s << 17) & (2**64 - 1)
        return np.float32(np.float32((s >> 40)) / np.float32(1 << 24)) * np.float32(2.0) - np.float32(1.0)
    return nxt


def vec(nxt, n=HD):
    return np.array([nxt() for _ in range(n)], np.float32)


# --- src/kvquant.rs:592-612 centroids_are_sorted_symmetric_and_sized --------
@pytest.mark.parametrize("bits", [3, 4])
def test_centroids_sorted_symmetric_sized(oracle, bits):
    c = oracle.planar_codebook(HD, bits)
    assert c.size == 1 << bits
    assert np.all(np.diff(c) > 0)
    assert np.all(np.abs(c + c[::-1]) < 1e-6)
    assert c[-1] < 4.0 / 16.0


# --- :614-628 lloyd_max_beats_uniform ---------------------------------------
def test_lloyd_max_distortion_order(oracle):
    sigma2 = 1.0 / HD
    d3, d4 = oracle.planar_distortion(HD, 3), oracle.planar_distortion(HD, 4)
    assert d3 < sigma2 and d4 < d3


# --- :630-642 givens_is_orthogonal (rotation then its inverse) ----------------
def test_givens_orthogonal(oracle):
    x = vec(xorshift(7))
    rot = oracle.planar_rotate(x)
    c, s = oracle.planar_givens(HD)
    a, b = rot[0::2], rot[1::2]
    back = np.empty_like(rot)
    back[0::2] = c * a + s * b
    back[1::2] = -s * a + c * b
    assert np.max(np.abs(back - x)) < 1e-5


# --- :644-666 quantize_roundtrip_error_is_small ------------------------------
def test_quantize_roundtrip_error_small(oracle):
    nxt = xorshift(11)
    worst = 0.0
    for _ in range(64):
        x = vec(nxt)
        pk, n = oracle.planar_quantize(x, 4)
        y = oracle.planar_dequantize(pk, n, HD, 4)
        worst = max(worst, float(np.linalg.norm(x - y) / max(np.linalg.norm(x), 1e-9)))
    assert worst < 0.12


# --- :714-731 dot_rotated_matches_dequantized_dot ----------------------------
def test_dot_rotated_matches_dequantized(oracle):
    nxt = xorshift(23)
    k, q = vec(nxt), vec(nxt)
    pk, n = oracle.planar_quantize(k, 4)
    khat = oracle.planar_dequantize(pk, n, HD, 4)
    a = oracle.planar_dot_rotated(oracle.planar_rotate(q), pk, n, HD, 4)
    b = float(np.dot(q.astype(np.float64), khat.astype(np.float64)))
    assert abs(a - b) < 1e-4


# --- :750-793 bit packing round trips; groups of 3 bits -----------------------
@pytest.mark.parametrize("bits", range(1, 9))
def test_packing_roundtrip_every_width(oracle, bits):
    nxt = xorshift(17 + bits)
    idx = np.array([int(abs(float(nxt())) * 1000.0) % (1 << bits) for _ in range(HD)], np.uint8)
    pk = oracle.planar_pack(idx, bits)
    assert pk.size == (HD * bits + 7) // 8 == oracle.planar_packed_len(HD, bits)
    assert np.array_equal(oracle.planar_unpack(pk, HD, bits), idx)


def test_groups3_layout(oracle):
    """3 bits: coordinate k of group g at bits 3k of the little-endian
    24-bit value of bytes 3g..3g+2 (the reference's grouped layout)."""
    nxt = xorshift(23)
    idx = np.array([int(abs(float(nxt())) * 800.0) % 8 for _ in range(HD)], np.uint8)
    pk = oracle.planar_pack(idx, 3).astype(np.uint32)
    for g in range(HD // 8):
        v = pk[3 * g] | (pk[3 * g + 1] << 8) | (pk[3 * g + 2] << 16)
        for k in range(8):
            assert (v >> (3 * k)) & 7 == idx[8 * g + k]


@pytest.mark.parametrize("bits", [1, 2, 4])
def test_plane_layouts_equal_bitstream(oracle, bits):
    """1-, 2- and 4-bit planes (src/kvquant.rs:218-291): byte b holds
    coordinates b*(8/bits) + k at bits k*bits."""
    rng = np.random.default_rng(bits)
    idx = rng.integers(0, 1 << bits, HD).astype(np.uint8)
    per = 8 // bits
    planes = np.zeros(HD // per, np.uint32)
    for i in range(HD):
        planes[i // per] |= int(idx[i]) << (bits * (i % per))
    assert np.array_equal(oracle.planar_pack(idx, bits), planes.astype(np.uint8))


# --- independent restatements -------------------------------------------------
def _lloyd_max(bits, erf_f):
    """Lloyd-Max for N(0, 1/HD) in float64 numpy (vectorised): the steps of
    solve_lloyd_max (src/kvquant.rs:58-99) with a given erf."""
    n = 1 << bits
    sigma = 1.0 / math.sqrt(HD)
    c = np.array([-3.5 * sigma + 7.0 * sigma * (i + 0.5) / n for i in range(n)])
    cdf = lambda x: 0.5 * (1 + erf_f(x / (sigma * math.sqrt(2))))
    pdf = lambda x: np.exp(-x * x / (2 * sigma * sigma)) / (sigma * math.sqrt(2 * math.pi))
    for _ in range(300):
        e = np.concatenate([[-12 * sigma], (c[:-1] + c[1:]) / 2, [12 * sigma]])
        mass = cdf(e[1:]) - cdf(e[:-1])
        m1 = sigma * sigma * (pdf(e[:-1]) - pdf(e[1:]))
        nx = np.where(mass > 1e-15, m1 / np.where(mass > 1e-15, mass, 1), c)
        shift = np.max(np.abs(nx - c))
        c = nx
        if shift < 1e-12:
            break
    return c, sigma


def _as_erf(x):
    """Abramowitz & Stegun 7.1.26 (src/kvquant.rs:34-44)."""
    x = np.asarray(x, np.float64)
    sign = np.where(x < 0, -1.0, 1.0)
    x = np.abs(x)
    t = 1.0 / (1.0 + 0.3275911 * x)
    y = 1.0 - (((((1.061405429 * t - 1.453152027) * t) + 1.421413741) * t - 0.284496736) * t
               + 0.254829592) * t * np.exp(-x * x)
    return sign * y


@pytest.mark.parametrize("bits", [1, 2, 3, 4, 8])
def test_codebook_against_numpy_lloyd_max(oracle, bits):
    """The centroids against the same iteration in vectorised numpy (other
    operation order: agreement to f32 rounding shows the C loop has the
    reference's edges, moments, stopping rule and iteration cap)."""
    c, sigma = _lloyd_max(bits, _as_erf)
    got = oracle.planar_codebook(HD, bits).astype(np.float64)
    assert np.max(np.abs(got - c)) <= 1e-6 * sigma


@pytest.mark.parametrize("bits", [1, 2])
def test_codebook_converged_against_exact_erf(oracle, bits):
    """Where the iteration converges (1 and 2 bits) the approximate erf
    changes nothing visible: the centroids of the exact Lloyd-Max solution
    (scipy's erf) to f32 rounding."""
    from scipy.special import erf
    c, sigma = _lloyd_max(bits, erf)
    got = oracle.planar_codebook(HD, bits).astype(np.float64)
    assert np.max(np.abs(got - c)) <= 1e-6 * sigma


def test_givens_table_from_splitmix(oracle):
    st = 42
    M = 2**64 - 1
    cs, ss = [], []
    for _ in range(HD // 2):
        st = (st + 0x9E3779B97F4A7C15) & M
        z = st
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M
        z ^= z >> 31
        t = ((z >> 11) / float(1 << 53)) * (2 * math.pi)
        cs.append(math.cos(t))
        ss.append(math.sin(t))
    c, s = oracle.planar_givens(HD)
    assert np.array_equal(c, np.array(cs, np.float32))
    assert np.array_equal(s, np.array(ss, np.float32))


@pytest.mark.parametrize("bits", [2, 3, 4, 8])
def test_quantize_indices_restated(oracle, bits):
    """Norm as a sequential float32 sum, unit vector, rotation in float32,
    first nearest centroid: the same indices and norm bit for bit."""
    rng = np.random.default_rng(100 + bits)
    cb = oracle.planar_codebook(HD, bits)
    c, s = oracle.planar_givens(HD)
    for trial in range(8):
        x = (rng.standard_normal(HD) * (10.0 ** (trial - 4))).astype(np.float32)
        ss = np.add.accumulate(x * x, dtype=np.float32)[-1]
        n = np.sqrt(ss, dtype=np.float32)
        inv = np.float32(1.0) / n if n > np.float32(1e-12) else np.float32(0.0)
        u = x * inv
        a, b = u[0::2], u[1::2]
        rot = np.empty_like(u)
        rot[0::2] = c * a - s * b
        rot[1::2] = s * a + c * b
        idx = np.argmin(np.abs(rot[:, None] - cb[None, :]), axis=1).astype(np.uint8)
        pk, norm = oracle.planar_quantize(x, bits)
        assert norm == float(n)
        assert np.array_equal(oracle.planar_unpack(pk, HD, bits), idx)


def test_zero_vector_quantizes_to_zero_norm(oracle):
    pk, n = oracle.planar_quantize(np.zeros(HD, np.float32), 4)
    assert n == 0.0
    assert np.array_equal(oracle.planar_dequantize(pk, n, HD, 4), np.zeros(HD, np.float32))


@pytest.mark.parametrize("bits,quantize_v,n_q,pos0", [
    (4, True, 1, 40), (3, True, 2, 17), (2, False, 1, 9), (8, True, 3, 5), (1, True, 1, 30),
])
def test_attention_planar_equals_dequantized_attention(oracle, synth, bits, quantize_v, n_q, pos0):
    n_head, n_kv = 6, 2
    r = synth.Rng(1000 + bits)
    n = pos0 + n_q
    k = r.normal(n * n_kv * HD).reshape(n, n_kv * HD)
    v = r.normal(n * n_kv * HD).reshape(n, n_kv * HD)
    q = r.normal(n_q * n_head * HD).reshape(n_q, n_head, HD)
    kq, kn, vq, vn, vf = oracle.kv_store_planar(k, v, n_kv, HD, bits, n, 0, quantize_v)
    got = oracle.attention_planar(q, pos0, kq, kn, vq, vn, vf, n_kv, bits, quantize_v)
    kd = np.stack([oracle.planar_dequantize(kq[j, h], kn[j, h], HD, bits)
                   for j in range(n) for h in range(n_kv)]).reshape(n, n_kv * HD)
    vd = np.stack([oracle.planar_dequantize(vq[j, h], vn[j, h], HD, bits)
                   for j in range(n) for h in range(n_kv)]).reshape(n, n_kv * HD) \
        if quantize_v else v
    ref = oracle.attention(q, pos0, kd, vd, n_kv)
    assert rel_err(got, ref) <= 2e-5
