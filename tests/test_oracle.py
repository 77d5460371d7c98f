"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the checker.

Every check comes from outside the oracle's own formulas:
  * the reference's unit tests, restated with their literal inputs/answers
    (src/kernels.rs:761-853, src/gguf.rs:950-1033, src/rope.rs:96-114);
  * exhaustive or closed-form facts (all 65536 f16 patterns against numpy's
    IEEE conversion, 2-element softmax = logistic, unit-norm L2 rows,
    rotation by a double-precision brute force with a hand-derived band table);
  * invariants chosen so a dropped term, a wrong sign or a swapped operand
    fails (shift invariance, pair-norm preservation, untouched tail dims).
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from conftest import rel_err
from gdndata import gdn_case


# --- src/kernels.rs:761-772 rms_norm_matches_reference ----------------------
def test_rms_norm_matches_reference(oracle):
    x = np.array([1.0, 2.0, 3.0, 4.0], np.float32)
    w = np.array([0.5, 1.0, 1.5, 2.0], np.float32)
    y = oracle.rms_norm(x, w, 1e-6)
    s = np.float32(1.0) / np.sqrt(np.float32(7.5) + np.float32(1e-6))
    expect = x * w * s
    assert np.all(np.abs(y - expect) < 1e-6)


# --- src/kernels.rs:774-787 pq2_decode_known_row ----------------------------
def test_pq2_decode_known_row(oracle):
    raw = np.zeros(34, np.uint8)
    raw[0], raw[1] = 0x00, 0x40  # scale 2.0
    raw[2] = 0b11                # j=0 code 3 -> +4
    raw[3] = 0b10_01             # j=4 code 1 -> 0, j=5 code 2 -> +2
    v = oracle.decode_pq2_0_row(raw, 128)
    assert v[0] == 4.0
    assert v[1] == -2.0
    assert v[4] == 0.0
    assert v[5] == 2.0


# --- src/kernels.rs:789-812 rms_norm_rows_matches_single_row_math ----------
def test_rms_norm_rows_matches_single_row_math(oracle):
    x = np.array([1.0, 2.0, 3.0, 4.0, 0.5, -0.5, 2.0, -3.0], np.float32)
    w = np.array([0.5, 1.0, 1.5, 2.0], np.float32)
    eps = np.float32(1e-6)
    y = oracle.rms_norm_rows(x, w, 4, eps)
    for row in range(2):
        src = x[row * 4:(row + 1) * 4]
        ss = np.float32(0)
        for v in src:
            ss = np.float32(ss + v * v)
        scale = np.float32(1.0) / np.sqrt(ss / np.float32(4) + eps)
        want = src * scale * w
        assert np.all(np.abs(y[row * 4:(row + 1) * 4] - want) < 1e-6)
    with pytest.raises(ValueError):
        oracle.rms_norm_rows(x, w, 3, eps)       # non-divisible
    with pytest.raises(ValueError):
        oracle.rms_norm_rows(x, w[:2], 4, eps)   # bad weight len


# --- src/kernels.rs:814-828 l2_norm_rows_produce_unit_rows -----------------
def test_l2_norm_rows_produce_unit_rows(oracle):
    x = np.array([3.0, 4.0, 0.0, 0.0, 1.0, 1.0, 1.0, 1.0], np.float32)
    y = oracle.l2_norm_rows(x, 4, 1e-12)
    assert abs(y[0] - 0.6) < 1e-6
    assert abs(y[1] - 0.8) < 1e-6
    assert abs(float(np.sum(y[4:8] ** 2)) - 1.0) < 1e-6
    z = oracle.l2_norm_rows(np.zeros(4, np.float32), 4, 1e-6)
    assert np.array_equal(z, np.zeros(4, np.float32))
    with pytest.raises(ValueError):
        oracle.l2_norm_rows(x, 3, 1e-12)


# --- src/kernels.rs:830-838 activations_hit_expected_points ----------------
def test_activations_hit_expected_points(oracle):
    assert oracle.silu(0.0) == 0.0
    assert abs(oracle.silu(1000.0) - 1000.0) < 1e-3
    assert abs(oracle.sigmoid(0.0) - 0.5) < 1e-7
    assert oracle.sigmoid(-1000.0) == 0.0
    assert abs(oracle.softplus(0.0) - math.log(2.0)) < 1e-7
    assert oracle.softplus(100.0) == 100.0


# --- src/kernels.rs:840-853 softmax_rows_are_normalized_and_mask_safe ------
def test_softmax_rows_are_normalized_and_mask_safe(oracle):
    x = np.array([1.0, 2.0, 3.0, -np.inf, 0.0, 0.0, 0.0, 0.0], np.float32)
    y = oracle.softmax_rows(x, 4)
    assert abs(float(y[0:4].sum()) - 1.0) < 1e-6
    assert y[3] == 0.0
    assert abs(float(y[4:8].sum()) - 1.0) < 1e-6
    assert np.all(np.abs(y[4:8] - 0.25) < 1e-6)
    with pytest.raises(ValueError):
        oracle.softmax_rows(x, 3)


# --- src/gguf.rs:950-963 half_conversions -----------------------------------
def test_half_conversions(oracle):
    h = oracle.half_to_f32
    assert h([0x3C00])[0] == 1.0
    assert h([0xC000])[0] == -2.0
    assert h([0x0000])[0] == 0.0
    assert h([0x3800])[0] == 0.5
    assert h([0x0001])[0] == np.float32(5.9604645e-8)
    assert abs(float(h([0x03FF])[0]) - 6.097555e-5) < 1e-10
    assert h([0x7C00]).view(np.uint32)[0] == np.float32(np.inf).view(np.uint32)
    assert np.isnan(h([0x7E00])[0])


def test_half_to_f32_exhaustive(oracle):
    """All 65536 patterns against numpy's IEEE widening (which also keeps
    NaN payloads unquieted), bit for bit."""
    pats = np.arange(65536, dtype=np.uint16)
    ours = oracle.half_to_f32(pats).view(np.uint32)
    ref = pats.view(np.float16).astype(np.float32).view(np.uint32)
    assert np.array_equal(ours, ref)


# --- src/gguf.rs:965-984 f32_to_half_roundtrips_and_rounds -----------------
def test_f32_to_half_roundtrips_and_rounds(oracle):
    f = lambda v: int(oracle.f32_to_half(np.array([v], np.float32))[0])
    assert f(1.0) == 0x3C00
    assert f(-2.0) == 0xC000
    assert f(0.5) == 0x3800
    assert f(0.0) == 0x0000
    assert f(np.inf) == 0x7C00
    assert f(-np.inf) == 0xFC00
    s = 0x12345678
    mask = (1 << 64) - 1
    vals = []
    for _ in range(2000):
        s ^= (s << 13) & mask
        s ^= s >> 7
        s ^= (s << 17) & mask
        vals.append(np.float32(np.float32((s >> 40)) / np.float32(1 << 24) * np.float32(20.0)
                               - np.float32(10.0)))
    v = np.array(vals, np.float32)
    back = oracle.half_to_f32(oracle.f32_to_half(v))
    tol = np.maximum(np.abs(v), 1e-3) * 1e-3
    assert np.all(np.abs(back - v) <= tol)


def test_f32_to_half_matches_ieee_in_normal_range(oracle):
    """In the f16 normal range the reference rounds to nearest-even, which is
    exactly numpy's float16 cast."""
    rng = np.random.default_rng(7)
    v = (rng.standard_normal(200000) * 50).astype(np.float32)
    v = v[(np.abs(v) >= 6.2e-5) & (np.abs(v) < 65000)]
    assert np.array_equal(oracle.f32_to_half(v), v.astype(np.float16).view(np.uint16))


def test_synth_f32_to_half_matches_oracle(oracle, synth):
    """The vectorised generator's conversion equals the restated reference,
    including its subnormal truncation, overflow and NaN cases."""
    rng = np.random.default_rng(3)
    v = np.concatenate([
        (rng.standard_normal(100000) * 0.02).astype(np.float32),
        (rng.standard_normal(50000) * 1e-6).astype(np.float32),
        (rng.standard_normal(20000) * 7e4).astype(np.float32),
        np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 65504.0, 65520.0, 6.1e-5, 5.96e-8,
                  2.98e-8, 1e-9], np.float32),
    ])
    assert np.array_equal(synth.f32_to_half(v), oracle.f32_to_half(v))


# --- src/gguf.rs:986-1033 pq2_0_decode_matches_reference -------------------
def test_pq2_0_decode_matches_reference(oracle):
    data = bytearray()
    data += (0x3800).to_bytes(2, "little") + bytes(32)
    qs = bytearray(32)
    qs[0] = 0b11
    qs[1] = 0b10_01
    data += (0x4000).to_bytes(2, "little") + bytes(qs)
    v = oracle.decode_pq2_0_row(np.frombuffer(bytes(data), np.uint8), 256)
    assert v[0] == -0.5
    assert v[128] == 4.0
    assert v[129] == -2.0
    assert v[132] == 0.0
    assert v[133] == 2.0


def test_pq2_partial_block_and_row_bytes(oracle, synth):
    """ne0 not a multiple of 128: ceil(ne0/128) blocks, last one truncated."""
    assert oracle.pq2_row_bytes(5120) == 1360
    assert oracle.pq2_row_bytes(130) == 68
    assert oracle.pq2_row_bytes(0) == 0
    codes = np.array([[3, 0, 1, 2] * 50], np.uint8)[:, :200]
    scales = synth.f32_to_half(np.array([0.5, 0.25], np.float32)).reshape(1, 2)
    raw = synth.pack_pq2_rows(codes, scales)[0]
    v = oracle.decode_pq2_0_row(raw, 200)
    expect = (codes[0].astype(np.float32) - 1) * np.where(np.arange(200) < 128, 0.5, 0.25)
    assert np.array_equal(v, expect.astype(np.float32))


def test_pq2_sign_of_zero_and_nonfinite_scales(oracle):
    """code 1 times a negative scale is -0.0; x86 gives the quieted NaN for a
    NaN scale and the default NaN 0xFFC00000 for 0 * inf."""
    raw = np.zeros(34 * 3, np.uint8)
    for b, h in enumerate((0xB800, 0x7D01, 0x7C00)):  # -0.5, sNaN, +inf
        raw[34 * b], raw[34 * b + 1] = h & 0xFF, h >> 8
        raw[34 * b + 2] = 0b10_01_00_11  # codes 3, 0, 1, 2
    v = oracle.decode_pq2_0_row(raw, 384).view(np.uint32)
    assert v[2] == 0x80000000                       # 0 * -0.5 = -0.0
    assert v[128] == 0x7FC00000 | (0x101 << 13)     # quieted payload of 0x7D01
    assert v[256 + 2] == 0xFFC00000                 # 0 * inf
    assert v[256 + 0] == 0x7F800000                 # 2 * inf


# --- src/rope.rs:96-114 and IMROPE facts -----------------------------------
SECTIONS = (11, 11, 10, 0)


def test_rope_pos0_is_identity(oracle):
    h = np.random.default_rng(0).standard_normal(256).astype(np.float32)
    out = oracle.rope_imrope(h, 0, 0, 0, 0, 64, SECTIONS, 1e7)
    assert np.array_equal(out, h)


def test_rope_preserves_pair_norm_and_tail(oracle):
    h = np.random.default_rng(1).standard_normal(256).astype(np.float32)
    out = oracle.rope_imrope(h, 37, 37, 37, 37, 64, SECTIONS, 1e7)
    n0 = h[:32] ** 2 + h[32:64] ** 2
    n1 = out[:32] ** 2 + out[32:64] ** 2
    assert np.all(np.abs(n0 - n1) < 1e-5 * np.maximum(1, n0))
    assert np.array_equal(out[64:], h[64:])


def _rope_double(h, pos4, n_dims, bands, base, chain=False):
    """Rotation in double with theta_j = p_band(j) * base^(-2j/n_dims), or
    (chain=True) with the f32 product chain p*s*...*s of the reference."""
    h = h.astype(np.float64)
    out = h.copy()
    half = n_dims // 2
    scale = np.float32(np.power(np.float32(base), np.float32(-2.0) / np.float32(n_dims)))
    for j in range(half):
        if chain:
            th = np.float32(pos4[bands[j]])
            for _ in range(j):
                th = np.float32(th * scale)
            th = float(th)
        else:
            th = pos4[bands[j]] * base ** (-2.0 * j / n_dims)
        c, s = math.cos(th), math.sin(th)
        out[j] = h[j] * c - h[j + half] * s
        out[j + half] = h[j] * s + h[j + half] * c
    return out


def test_rope_matches_double_brute_force_qwen35(oracle):
    """sections [11,11,10,0], 32 pairs: sector j < 33 always, so band = j % 3
    except j % 3 == 2 with j >= 30 -> e (hand-derived from src/rope.rs:41-49)."""
    bands = [(j % 3 if not (j % 3 == 2 and j >= 30) else 3) for j in range(32)]
    assert bands[30] == 0 and bands[31] == 1 and bands[29] == 2
    h = np.random.default_rng(2).standard_normal(256).astype(np.float32)
    for pos in [(5, 5, 5, 5), (17, 17, 17, 17), (3, 5, 7, 0), (2047, 11, 900, 3)]:
        out = oracle.rope_imrope(h, *pos, 64, SECTIONS, 1e7)
        # closed-form angles: the f32 chain drifts ~1e-4 rad by position 2047
        ref = _rope_double(h, pos, 64, bands, 1e7)
        assert rel_err(out[:64], ref[:64]) < 3e-5, pos
        # chained angles: only the f32 rounding of cos/sin and the rotation remain
        ref = _rope_double(h, pos, 64, bands, 1e7, chain=True)
        assert rel_err(out[:64], ref[:64]) < 1e-6, pos


def test_rope_band_table_small_sections(oracle):
    """sections [1,1,1,1]: sector = j % 4 -> bands t, h, w, e repeating."""
    bands = [0, 1, 2, 3] * 4
    h = np.random.default_rng(3).standard_normal(32).astype(np.float32)
    pos = (3, 50, 700, 9000)
    out = oracle.rope_imrope(h, *pos, 32, (1, 1, 1, 1), 1e4)
    assert rel_err(out, _rope_double(h, pos, 32, bands, 1e4)) < 3e-5
    assert rel_err(out, _rope_double(h, pos, 32, bands, 1e4, chain=True)) < 1e-6
    # a wrong band (e.g. t and h swapped) is far off
    swapped = [1, 0, 2, 3] * 4
    assert rel_err(out, _rope_double(h, pos, 32, swapped, 1e4, chain=True)) > 1e-2


def test_rope_theta_chain_is_sequential_products(oracle):
    """theta_j is the rounded chain p*s*s*...: checked through the angle of a
    unit pair (x0=1, x1=0 -> (cos, sin)) at a position where the chain and
    the closed form differ in f32."""
    n_dims = 64
    s = np.float32(np.power(np.float32(1e7), np.float32(-2.0) / np.float32(n_dims)))
    h = np.zeros(256, np.float32)
    h[31] = 1.0  # pair j = 31
    out = oracle.rope_imrope(h, 2047, 2047, 2047, 2047, n_dims, SECTIONS, 1e7)
    th = np.float32(2047)
    for _ in range(31):
        th = np.float32(th * s)
    assert out[31] == np.float32(math.cos(float(th))) or abs(out[31] - math.cos(float(th))) < 1e-7
    assert abs(out[63] - math.sin(float(th))) < 1e-7


# --- softmax facts -------------------------------------------------------------
def test_softmax_two_elements_is_logistic(oracle):
    a, b = 0.3, -1.7
    y = oracle.softmax_rows(np.array([a, b], np.float32), 2)
    assert abs(y[0] - 1 / (1 + math.exp(b - a))) < 1e-7
    assert abs(y[1] - 1 / (1 + math.exp(a - b))) < 1e-7


def test_softmax_shift_invariance_and_temperature(oracle):
    x = np.random.default_rng(4).standard_normal(4096).astype(np.float32) * 3
    y = oracle.softmax_rows(x, 1024)
    y2 = oracle.softmax_rows(x + np.float32(8.0), 1024)
    assert rel_err(y, y2) < 1e-5
    assert np.array_equal(oracle.softmax_rows(x, 1024, 1.0), y)  # temp 1 is a no-op
    t = oracle.softmax_rows(x, 1024, np.float32(1.0) / np.float32(0.7))
    assert np.array_equal(t, oracle.softmax_rows(x * (np.float32(1) / np.float32(0.7)), 1024))
    assert np.all(np.abs(t.reshape(4, 1024).sum(1) - 1) < 1e-5)


def _ulps(a, b):
    """Distance in f32 ulps of same-sign finite values."""
    ia = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    ib = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    return np.abs(ia - ib)


def test_softmax_sampler_norm_is_the_f64_formula(oracle):
    """src/sampler.rs:108-126: y = logits * inv_t (f32), max, e = exp(y - max)
    (f32, the C library's expf here as Rust's f32::exp), sum += e as f64,
    inv_sum = 1.0 / sum, p = (e as f64 * inv_sum) as f32.  Restated with
    numpy's f64 arithmetic: bit for bit, so a dropped f64 step, an f32
    reciprocal or a wrong sum shows."""
    import ctypes
    import ctypes.util
    libm = ctypes.CDLL(ctypes.util.find_library("m"))
    libm.expf.restype = ctypes.c_float
    libm.expf.argtypes = [ctypes.c_float]
    r = np.random.default_rng(12)
    for row_len, inv_t in ((37, 1.0), (1000, 1.0 / 0.7), (4096, 2.5)):
        x = (r.standard_normal(3 * row_len) * 3).astype(np.float32)
        inv_t = np.float32(inv_t)
        got = oracle.softmax_rows(x, row_len, inv_t, sampler_norm=True)
        for k in range(3):
            y = x[k * row_len:(k + 1) * row_len] * inv_t
            m = y.max()
            e = np.array([libm.expf(float(v)) for v in (y - m)], np.float32)
            total = 0.0
            for v in e:  # the reference's sequential f64 sum
                total += float(v)
            want = (e.astype(np.float64) * (1.0 / total)).astype(np.float32)
            assert np.array_equal(got[k * row_len:(k + 1) * row_len], want)
            # the f32 reciprocal of kernels::softmax_rows differs somewhere
            plain = (e * (np.float32(1.0) / np.float32(total))).astype(np.float32)
            assert not np.array_equal(plain, want) or row_len < 100
        # the plain normalisation of the same exponentials is within 2 ulps
        plain = oracle.softmax_rows(x, row_len, inv_t)
        assert _ulps(plain, got).max() <= 2
        assert abs(got.reshape(3, -1).astype(np.float64).sum(1) - 1).max() < 1e-6


def test_softmax_all_masked_row_is_nan(oracle):
    """An all -inf row gives NaN (exp(-inf - -inf)), as the reference does."""
    y = oracle.softmax_rows(np.full(8, -np.inf, np.float32), 8)
    assert np.all(np.isnan(y))


# --- gate prep ---------------------------------------------------------------
def test_gdn_gate_prep_closed_forms(oracle):
    alpha = np.array([[0.0, 25.0, -3.0]], np.float32)
    dt = np.array([0.0, 0.0, 1.0], np.float32)
    a = np.array([-1.0, -2.0, -0.5], np.float32)
    beta_raw = np.array([[0.0, -1000.0, 2.0]], np.float32)
    gate, beta = oracle.gdn_gate_prep(alpha, dt, a, beta_raw)
    assert abs(gate[0, 0] + math.log(2.0)) < 1e-7         # softplus(0) * -1
    assert gate[0, 1] == np.float32(-50.0)                # identity branch above 20
    assert abs(gate[0, 2] - (-0.5 * math.log1p(math.exp(-2.0)))) < 1e-7
    assert beta[0, 0] == 0.5 and beta[0, 1] == 0.0
    assert abs(beta[0, 2] - 1 / (1 + math.exp(-2.0))) < 1e-7


def test_silu_l2_part_unit_heads(oracle):
    conv = np.random.default_rng(5).standard_normal((3, 512)).astype(np.float32)
    out = oracle.silu_l2_part(conv, 256, 128, 1e-6)
    heads = out[:, :256].reshape(3, 2, 128)
    assert np.all(np.abs((heads.astype(np.float64) ** 2).sum(-1) - 1) < 1e-5)
    silu = conv / (1 + np.exp(-conv.astype(np.float64)))
    assert rel_err(out[:, 256:], silu[:, 256:]) < 1e-6
    with pytest.raises(ValueError):
        oracle.silu_l2_part(conv, 200, 128, 1e-6)


# --- src/forward.rs:524 (SiLU over the conv output), :539-540 (l2_norm_rows on
#     the q/k heads): the fused oracle equals the composition of the pinned
#     pieces bit for bit, and a float64 restatement within 2e-6.  A dropped
#     SiLU (heads of the raw conv) passes the unit-norm check above but fails
#     both of these.
@pytest.mark.parametrize("n_tok,conv_dim,l2_dim,hd", [(3, 512, 256, 128), (17, 1280, 1024, 128),
                                                      (5, 96, 64, 32)])
def test_silu_l2_part_is_silu_then_pinned_l2(oracle, n_tok, conv_dim, l2_dim, hd):
    rng = np.random.default_rng(11 + conv_dim)
    conv = (rng.standard_normal((n_tok, conv_dim)) * 2).astype(np.float32)
    conv[0, :hd] = 0.0                      # a zero head: the eps floor branch
    eps = 1e-6
    out = oracle.silu_l2_part(conv, l2_dim, hd, eps)
    act = oracle.unary(0, conv)
    want = act.copy()
    want[:, :l2_dim] = oracle.l2_norm_rows(np.ascontiguousarray(act[:, :l2_dim]), hd,
                                           eps).reshape(n_tok, l2_dim)
    assert np.array_equal(out.view(np.uint32), want.view(np.uint32))
    # float64: silu, then each head divided by max(its f64 norm, eps)
    xd = conv.astype(np.float64)
    sd = xd / (1 + np.exp(-xd))
    heads = sd[:, :l2_dim].reshape(n_tok, l2_dim // hd, hd)
    norm = np.maximum(np.sqrt((heads ** 2).sum(-1, keepdims=True)), eps)
    ref = sd.copy()
    ref[:, :l2_dim] = (heads / norm).reshape(n_tok, l2_dim)
    assert np.max(np.abs(out - ref)) <= 2e-6
    assert np.all(out[0, :hd] == 0.0)
    # a dropped SiLU is caught: raw-conv heads differ well beyond the bound
    raw = oracle.l2_norm_rows(np.ascontiguousarray(conv[:, :l2_dim]), hd, eps)
    assert np.max(np.abs(raw.reshape(n_tok, l2_dim) - out[:, :l2_dim])) > 1e-2


def test_unary_modes_closed_form(oracle):
    x = np.linspace(-30, 30, 1001).astype(np.float32)
    b = np.linspace(2, -2, 1001).astype(np.float32)
    xd = x.astype(np.float64)
    sig = 1 / (1 + np.exp(-xd))
    sp = np.where(xd > 20, xd, np.log1p(np.exp(xd)))
    assert rel_err(oracle.unary(0, x), xd * sig) < 1e-6
    assert rel_err(oracle.unary(1, x), sig) < 1e-6
    assert rel_err(oracle.unary(2, x), sp) < 1e-6
    assert rel_err(oracle.unary(3, x, b), b * xd * sig) < 1e-6
    assert rel_err(oracle.unary(4, x, b), b * sig) < 1e-6


def test_embed_gather_range_error(oracle, synth):
    table = synth.pq2_table(synth.Rng(9), 4, 256)
    out = oracle.embed_gather(table, 256, 4, np.array([3, 0, 3], np.uint32))
    assert np.array_equal(out[0], out[2])
    with pytest.raises(IndexError):
        oracle.embed_gather(table, 256, 4, np.array([1, 4], np.uint32))


def test_embed_gather_rms_is_rms_of_rows(oracle, synth):
    table = synth.pq2_table(synth.Rng(10), 8, 5120)
    w = synth.Rng(11).normal(5120, 1.0, 0.1)
    ids = np.array([7, 1, 1], np.uint32)
    emb, nrm = oracle.embed_gather(table, 5120, 8, ids, w, 1e-6)
    for k in range(3):
        assert np.array_equal(nrm[k], oracle.rms_norm(emb[k], w, 1e-6))
    xd = emb.astype(np.float64)
    ref = xd / np.sqrt((xd ** 2).mean(1, keepdims=True) + 1e-6) * w
    # the reference sums 5120 squares sequentially in f32: ~1e-5 from exact
    assert rel_err(nrm, ref) < 3e-5


# ---------------------------------------------------------------------------
# PQ2_0 row dot / products (src/kernels.rs:233-423, 633-653)
# ---------------------------------------------------------------------------

def test_pq2_row_dot_one_hot_is_the_decoded_weight(oracle, synth):
    """Closed form: x = e_j gives the row's decoded weight j exactly (one
    non-zero product in one block, every other block adds scale * 0)."""
    import pq2data
    ne0, n_rows = 384, 5
    table = synth.pq2_table(synth.Rng(41), n_rows, ne0).reshape(-1)
    w = pq2data.decoded(table, ne0, n_rows).astype(np.float32)
    for j in (0, 1, 127, 128, 200, 383):
        x = np.zeros(ne0, np.float32)
        x[j] = 1.0
        y = oracle.pq2_matmul_n(table, ne0, n_rows, x)
        assert np.array_equal(y, w[:, j]), j
        # a power-of-two multiple scales exactly
        x[j] = 0.25
        assert np.array_equal(oracle.pq2_matmul_n(table, ne0, n_rows, x), w[:, j] * 0.25)


def test_pq2_row_dot_matches_float64_dot(oracle, synth):
    """The f32 block sums agree with an exact-enough float64 dot of the
    numpy-decoded rows (a dropped block, a wrong code order or a scale
    applied to the wrong block fails by orders of magnitude)."""
    import pq2data
    ne0, n_rows, n_tok = 1280, 40, 3
    table = synth.pq2_table(synth.Rng(42), n_rows, ne0).reshape(-1)
    x = synth.Rng(43).normal(n_tok * ne0).reshape(n_tok, ne0)
    y = oracle.pq2_matmul_n(table, ne0, n_rows, x)
    ref = x.astype(np.float64) @ pq2data.decoded(table, ne0, n_rows).T
    assert np.max(np.abs(y - ref)) / np.max(np.abs(ref)) < 1e-6
    # partial last block (ne0 not a multiple of 128)
    ne0 = 300
    table = synth.pq2_table(synth.Rng(44), 7, ne0).reshape(-1)
    x = synth.Rng(45).normal(ne0)
    y = oracle.pq2_matmul_n(table, ne0, 7, x)
    ref = pq2data.decoded(table, ne0, 7) @ x.astype(np.float64)
    assert np.max(np.abs(y - ref)) / np.max(np.abs(ref)) < 1e-6


def test_pq2_row_dot_reference_avx2_case(oracle):
    """src/kernels.rs:857-907 restated: the reference checks its AVX2 dot
    against row_dot_scalar to 1e-4 relative; the oracle (row_dot_scalar)
    must meet the same bound against the float64 dot of the same rows."""
    import pq2data
    raw, x, ne0, n_rows = pq2data.avx2_case()
    ref = pq2data.decoded(raw, ne0, n_rows) @ x.astype(np.float64)
    rb = oracle.pq2_row_bytes(ne0)
    for r in range(n_rows):
        s = oracle.pq2_row_dot(raw[r * rb:(r + 1) * rb], ne0, x)
        assert abs(s - ref[r]) / max(abs(s), 1e-6) < 1e-4, r
    y = oracle.pq2_matmul_n(raw, ne0, n_rows, x)
    assert np.array_equal(y, np.array([oracle.pq2_row_dot(raw[r * rb:(r + 1) * rb], ne0, x)
                                       for r in range(n_rows)], np.float32))


def test_pq2_matmul_n_reference_case(oracle, synth):
    """src/kernels.rs:910-946 restated: pq2_matmul_n equals the per-token
    matvec exactly; base_row selects the rows of the range."""
    import pq2data
    payload, x, ne0, n_rows, n_tok = pq2data.matmul_case(synth.f32_to_half)
    y = oracle.pq2_matmul_n(payload, ne0, n_rows, x)
    for t in range(n_tok):
        assert np.array_equal(y[t], oracle.pq2_matmul_n(payload, ne0, n_rows, x[t]))
    ref = x.astype(np.float64) @ pq2data.decoded(payload, ne0, n_rows).T
    assert np.max(np.abs(y - ref)) / np.max(np.abs(ref)) < 1e-6
    tail = oracle.pq2_matmul_n(payload, ne0, 5, x, base_row=7)
    assert np.array_equal(tail, y[:, 7:12])


# ---------------------------------------------------------------------------
# causal conv1d + SiLU (src/forward.rs:508-533)
# ---------------------------------------------------------------------------

def test_conv1d_unit_taps_and_state(oracle, synth):
    """Closed form: with tap j set to 1 and the others 0, out[t][c] is
    silu of the input j - (k-1) steps back (the state for negative times),
    and the final state holds the last k-1 inputs."""
    ch, k, n_tok = 12, 4, 6
    r = synth.Rng(61)
    x = r.normal(n_tok * ch).reshape(n_tok, ch)
    st0 = r.normal(ch * (k - 1)).reshape(ch, k - 1)
    seq = np.concatenate([st0.T, x], axis=0)  # position p -> row p + k - 1
    for j in range(k):
        w = np.zeros((ch, k), np.float32)
        w[:, j] = 1.0
        out, st = oracle.conv1d_silu(x, st0, w)
        want = seq[j:j + n_tok]
        silu = np.array([oracle.silu(float(v)) for v in want.ravel()], np.float32).reshape(want.shape)
        assert np.array_equal(out, silu), j
        assert np.array_equal(st, seq[-(k - 1):].T)


def test_conv1d_batched_equals_token_steps(oracle, synth):
    """The reference runs one token at a time with the state threaded
    through; a batch of tokens must give the same outputs and state."""
    ch, k, n_tok = 40, 4, 9
    r = synth.Rng(62)
    x = r.normal(n_tok * ch).reshape(n_tok, ch)
    st0 = r.normal(ch * (k - 1)).reshape(ch, k - 1)
    w = r.normal(ch * k).reshape(ch, k)
    out, st = oracle.conv1d_silu(x, st0, w)
    s = st0
    for t in range(n_tok):
        o1, s = oracle.conv1d_silu(x[t:t + 1], s, w)
        assert np.array_equal(o1[0], out[t]), t
    assert np.array_equal(s, st)
    # and the pre-activation is the float64 convolution to f32 rounding
    seq = np.concatenate([st0.T, x], axis=0).astype(np.float64)
    acc = sum(seq[j:j + n_tok] * w[:, j].astype(np.float64) for j in range(k))
    silu64 = acc / (1 + np.exp(-acc))
    assert np.max(np.abs(out - silu64)) / np.max(np.abs(silu64)) < 1e-6


# ---------------------------------------------------------------------------
# gated delta-net recurrence (src/gdn.rs:17-77)
# ---------------------------------------------------------------------------

def test_gdn_step_closed_forms(oracle, synth):
    """beta = 0: the state only decays, attn = expf(gate) M q / sqrt(s);
    a zero state, gate 0, beta 1 and k = e_i writes v into column i, so
    attn[j] = v[j] q[i] / sqrt(s)."""
    h_k, h_v, s = 2, 4, 16
    q, k, v, gate, beta, st = gdn_case(synth, 1, h_k, h_v, s, 80)
    zero = np.zeros_like(beta)
    attn, st1 = oracle.gdn_step(q, k, v, gate, zero, st)
    for h in range(h_v):
        m = (st[h] * np.float32(np.exp(np.float32(gate[0, h])))).astype(np.float64)
        want = m @ q[0, h % h_k].astype(np.float64) / np.sqrt(s)
        assert np.allclose(attn[0, h], want, rtol=1e-5, atol=1e-6)
    assert np.allclose(st1, st * np.exp(gate[0])[:, None, None].astype(np.float32), rtol=1e-6)
    i = 5
    k1 = np.zeros_like(k)
    k1[0, :, i] = 1.0
    attn, st1 = oracle.gdn_step(q, k1, v, np.zeros_like(gate), np.ones_like(beta),
                                np.zeros_like(st))
    for h in range(h_v):
        assert np.array_equal(st1[h][:, i], v[0, h])
        assert np.allclose(attn[0, h], v[0, h] * q[0, h % h_k, i] / np.float32(np.sqrt(s)),
                           rtol=1e-6)


def test_gdn_step_matches_float64_recurrence(oracle, synth):
    """Several tokens: the f32 restatement tracks a float64 evaluation of the
    same recurrence (a wrong head mapping, a missing decay or a transposed
    update fails by orders of magnitude)."""
    n_tok, h_k, h_v, s = 6, 2, 4, 32
    q, k, v, gate, beta, st = gdn_case(synth, n_tok, h_k, h_v, s, 81)
    attn, st_new = oracle.gdn_step(q, k, v, gate, beta, st)
    m = st.astype(np.float64)
    for t in range(n_tok):
        for h in range(h_v):
            kk, qq = k[t, h % h_k].astype(np.float64), q[t, h % h_k].astype(np.float64)
            m[h] *= np.exp(np.float64(gate[t, h]))
            delta = (v[t, h] - m[h] @ kk) * beta[t, h]
            m[h] += np.outer(delta, kk)
            want = m[h] @ qq / np.sqrt(s)
            assert np.max(np.abs(attn[t, h] - want)) <= 1e-5 * max(1.0, np.max(np.abs(want)))
    assert np.max(np.abs(st_new - m)) <= 1e-5 * np.max(np.abs(m))


# ---- attention over a KV cache (src/forward.rs:273-375) ---------------------

def _attn_case(synth, n_q, pos0, n_head, n_kv, hd, seed, cap=None):
    r = synth.Rng(seed)
    cap = pos0 + n_q if cap is None else cap
    q = r.normal(n_q * n_head * hd).reshape(n_q, n_head, hd)
    kc = r.normal(cap * n_kv * hd).reshape(cap, n_kv * hd)
    vc = r.normal(cap * n_kv * hd).reshape(cap, n_kv * hd)
    return q, kc, vc


def _attn_f64(q, pos0, kc, vc, n_kv):
    """float64 softmax(q k^T / sqrt(hd)) v per query, causal, GQA head
    hq -> hq // (n_head / n_kv)."""
    n_q, n_head, hd = q.shape
    rep = n_head // n_kv
    out = np.zeros((n_q, n_head, hd))
    for i in range(n_q):
        n = pos0 + i + 1
        for h in range(n_head):
            g = h // rep
            k = kc[:n, g * hd:(g + 1) * hd].astype(np.float64)
            v = vc[:n, g * hd:(g + 1) * hd].astype(np.float64)
            s = k @ q[i, h].astype(np.float64) / np.sqrt(hd)
            p = np.exp(s - s.max())
            out[i, h] = (p / p.sum()) @ v
    return out


def test_attention_closed_forms(oracle, synth):
    """One cache position: the output is v_0 exactly (p = 1).  Identical
    keys: uniform probabilities, the output is the mean of the v rows."""
    q, kc, vc = _attn_case(synth, 1, 0, 4, 2, 16, 100)
    out = oracle.attention(q, 0, kc, vc, 2)
    for h in range(4):
        assert np.array_equal(out[0, h], vc[0, (h // 2) * 16:(h // 2 + 1) * 16])
    q, kc, vc = _attn_case(synth, 1, 9, 4, 2, 16, 101)
    kc[:] = kc[0]
    out = oracle.attention(q, 9, kc, vc, 2)
    for h in range(4):
        want = vc[:10, (h // 2) * 16:(h // 2 + 1) * 16].astype(np.float64).mean(0)
        assert np.allclose(out[0, h], want, rtol=0, atol=1e-6)


def test_attention_matches_float64(oracle, synth):
    """Several causal queries over a GQA cache (6 q heads on 2 kv heads: the
    mappings h // 3 and h % 2 differ) against a float64 evaluation."""
    n_q, pos0, n_head, n_kv, hd = 5, 7, 6, 2, 32
    q, kc, vc = _attn_case(synth, n_q, pos0, n_head, n_kv, hd, 102)
    q *= 2.0
    out = oracle.attention(q, pos0, kc, vc, n_kv)
    want = _attn_f64(q, pos0, kc, vc, n_kv)
    assert rel_err(out, want) <= 1e-6


def test_attention_is_causal(oracle, synth):
    """Query i reads positions 0 .. pos0 + i only: rewriting later rows of
    the cache leaves it unchanged."""
    q, kc, vc = _attn_case(synth, 3, 4, 4, 1, 8, 103, cap=12)
    out = oracle.attention(q, 4, kc, vc, 1)
    kc2, vc2 = kc.copy(), vc.copy()
    kc2[5:], vc2[5:] = 1e3, -1e3
    out2 = oracle.attention(q, 4, kc2, vc2, 1)
    assert np.array_equal(out[0], out2[0])
    assert not np.array_equal(out[1], out2[1])


def test_kv_store_and_f16_cache(oracle, synth):
    """append_f16 stores gguf::f32_to_half (= IEEE round to nearest even for
    normal-range values, as numpy's float16); attention over an f16 cache is
    attention over the f32 cache of the widened values, bit for bit."""
    n_q, pos0, n_head, n_kv, hd = 2, 3, 4, 2, 16
    q, kc, vc = _attn_case(synth, n_q, pos0, n_head, n_kv, hd, 104)
    k16 = np.zeros(kc.shape, np.uint16)
    v16 = np.zeros(vc.shape, np.uint16)
    k16, v16 = oracle.kv_store(kc, vc, k16, v16, 0)
    assert np.array_equal(k16, kc.astype(np.float16).view(np.uint16))
    kf = np.zeros_like(kc)
    kf, vf = oracle.kv_store(kc[2:4], vc[2:4], kf, np.zeros_like(vc), 2)
    assert np.array_equal(kf[2:4], kc[2:4]) and not kf[:2].any() and not kf[4:].any()
    wide_k = k16.view(np.float16).astype(np.float32)
    wide_v = v16.view(np.float16).astype(np.float32)
    assert np.array_equal(oracle.attention(q, pos0, k16, v16, n_kv),
                          oracle.attention(q, pos0, wide_k, wide_v, n_kv))


def test_attention_skips_zero_probabilities(oracle, synth):
    """src/forward.rs:363-366 skips p_j == 0: a position whose score is
    ~1e4 below the maximum contributes nothing, not 0 * inf."""
    q, kc, vc = _attn_case(synth, 1, 1, 1, 1, 4, 105)
    q[0, 0] = [100.0, 0.0, 0.0, 0.0]
    kc[0] = [-100.0, 0.0, 0.0, 0.0]
    kc[1] = [100.0, 0.0, 0.0, 0.0]
    vc[0] = np.inf
    out = oracle.attention(q, 1, kc, vc, 1)
    assert np.array_equal(out[0, 0], vc[1])


# --- composite functions: built from the pinned pieces above ------------------
# or_qk_norm_rope restates the attention pre-block of full_attention_layer
# (src/forward.rs:237-270, gate at :379): per token, split each q head's
# [q(hd) | gate(hd)], rms_norm_rows on the q heads and on the k heads with the
# shared hd-long weights, rope_imrope per head at that token's (t, h, w, e),
# sigmoid of the gate.  The composition below calls only the separately
# pinned oracle.rms_norm_rows / rope_imrope / sigmoid, in the reference's
# order, and must agree bit for bit; a float64 brute force bounds it too.
def _qk_case(n_tok, n_q, n_k, hd, stride, seed, mixed):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((n_tok, n_q, stride)).astype(np.float32)
    k = rng.standard_normal((n_tok, n_k, hd)).astype(np.float32)
    wq = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    wk = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    if mixed:
        pos = rng.integers(0, 5000, (n_tok, 4)).astype(np.int32)
    else:
        pos = np.repeat(np.arange(n_tok, dtype=np.int32)[:, None], 4, 1)
    return q, k, wq, wk, pos


def _qk_composed(oracle, q, k, wq, wk, pos, hd, n_dims, sections, base, eps, want_gate):
    n_tok, n_q, _ = q.shape
    n_k = 0 if k is None else k.shape[1]
    q_out = np.empty((n_tok, n_q, hd), np.float32)
    k_out = np.empty((n_tok, n_k, hd), np.float32) if n_k else None
    gate = np.empty((n_tok, n_q, hd), np.float32) if want_gate else None
    for t in range(n_tok):
        qs = np.ascontiguousarray(q[t, :, :hd]).reshape(-1)          # forward.rs:237-241
        qn = oracle.rms_norm_rows(qs, wq, hd, eps).reshape(n_q, hd)  # forward.rs:242-243
        for h in range(n_q):                                          # forward.rs:247-258
            q_out[t, h] = oracle.rope_imrope(qn[h], *map(int, pos[t]), n_dims, sections, base)
        if n_k:
            kn = oracle.rms_norm_rows(k[t].reshape(-1), wk, hd, eps).reshape(n_k, hd)
            for h in range(n_k):                                      # forward.rs:259-270
                k_out[t, h] = oracle.rope_imrope(kn[h], *map(int, pos[t]), n_dims, sections,
                                                 base)
        if want_gate:                                                 # forward.rs:379
            for h in range(n_q):
                gate[t, h] = [oracle.sigmoid(float(v)) for v in q[t, h, hd:2 * hd]]
    return q_out, k_out, gate


QK_CASES = [
    # n_tok, n_q, n_k, hd, stride, gate, mixed positions, n_dims, sections
    (5, 3, 2, 256, 256, False, False, 64, SECTIONS),
    (4, 3, 1, 256, 512, True, True, 64, SECTIONS),
    (3, 2, 0, 256, 512, True, True, 64, SECTIONS),
    (6, 2, 2, 32, 64, True, True, 16, (1, 2, 3, 2)),
]


@pytest.mark.parametrize("case", QK_CASES)
def test_qk_norm_rope_is_composition_of_pinned_pieces(oracle, case):
    n_tok, n_q, n_k, hd, stride, gate, mixed, n_dims, sec = case
    q, k, wq, wk, pos = _qk_case(n_tok, n_q, max(n_k, 1), hd, stride, 11 + n_tok, mixed)
    k = k[:, :n_k] if n_k else None
    got = oracle.qk_norm_rope(q, k, wq, wk if n_k else None, pos, n_q, n_k, hd, n_dims, sec,
                              1e7, 1e-6, q_head_stride=stride, want_gate=gate)
    ref = _qk_composed(oracle, q, k, wq, wk, pos, hd, n_dims, sec, 1e7, np.float32(1e-6), gate)
    assert np.array_equal(got[0].view(np.uint32), ref[0].view(np.uint32))
    if n_k:
        assert np.array_equal(got[1].view(np.uint32), ref[1].view(np.uint32))
    else:
        assert got[1] is None
    if gate:
        assert np.array_equal(got[2].view(np.uint32), ref[2].view(np.uint32))


def _sector_bands(n_dims, sections):
    """Band of pair j from src/rope.rs:37-49, derived by hand: sector =
    j % sum(sections); t for sector % 3 == 0 below 3*s0, h for % 3 == 1 below
    3*s1, w for % 3 == 2 below 3*s2, e otherwise."""
    tot = sum(sections)
    out = []
    for j in range(n_dims // 2):
        sec = j % tot
        if sec % 3 == 0 and sec < 3 * sections[0]:
            out.append(0)
        elif sec % 3 == 1 and sec < 3 * sections[1]:
            out.append(1)
        elif sec % 3 == 2 and sec < 3 * sections[2]:
            out.append(2)
        else:
            out.append(3)
    return out


def test_qk_norm_rope_matches_float64_brute_force(oracle):
    """Independent of every oracle piece: RMSNorm and the rotation in float64
    with the reference's f32 theta chain, the gate as a float64 logistic; a
    swapped q/gate half, a dropped weight or an unrotated k head fails."""
    n_tok, n_q, n_k, hd, stride = 4, 3, 2, 256, 512
    q, k, wq, wk, pos = _qk_case(n_tok, n_q, n_k, hd, stride, 99, True)
    qo, ko, g = oracle.qk_norm_rope(q, k, wq, wk, pos, n_q, n_k, hd, 64, SECTIONS, 1e7, 1e-6,
                                    q_head_stride=stride, want_gate=True)
    bands = _sector_bands(64, SECTIONS)
    assert bands == [(j % 3 if not (j % 3 == 2 and j >= 30) else 3) for j in range(32)]

    def ref_head(x, w, p):
        x = x.astype(np.float64)
        y = x / np.sqrt(np.mean(x * x) + 1e-6) * w.astype(np.float64)
        r = _rope_double(y.astype(np.float32), p, 64, bands, 1e7, chain=True)
        return np.concatenate([r[:64], y[64:]])

    for t in range(n_tok):
        p = tuple(int(v) for v in pos[t])
        for h in range(n_q):
            assert rel_err(qo[t, h], ref_head(q[t, h, :hd], wq, p)) < 2e-6, (t, h)
            gref = 1.0 / (1.0 + np.exp(-q[t, h, hd:].astype(np.float64)))
            assert np.max(np.abs(g[t, h] - gref)) < 2e-7, (t, h)
        for h in range(n_k):
            assert rel_err(ko[t, h], ref_head(k[t, h], wk, p)) < 2e-6, (t, h)


def test_add_rms_norm_rows_is_add_then_pinned_norm(oracle):
    """or_add_rms_norm_rows restates src/forward.rs:708-713 (cur += attn_out,
    then rms_norm(cur, post_w)) per row: the sum must be numpy's f32 add bit
    for bit and the norm the pinned oracle.rms_norm_rows of that sum."""
    rng = np.random.default_rng(21)
    for rows, n in [(1, 5120), (7, 256), (3, 130)]:
        x = rng.standard_normal((rows, n)).astype(np.float32)
        r = (3 * rng.standard_normal((rows, n))).astype(np.float32)
        w = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
        s, out = oracle.add_rms_norm_rows(x, r, w, n, 1e-6)
        s_ref = x + r
        assert np.array_equal(s.view(np.uint32), s_ref.view(np.uint32))
        ref = oracle.rms_norm_rows(s_ref, w, n, 1e-6)
        assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))
        s64 = s_ref.astype(np.float64)
        ref64 = s64 / np.sqrt(np.mean(s64 * s64, axis=1, keepdims=True) + 1e-6) * w
        assert rel_err(out, ref64) < 2e-6
    with pytest.raises(oracle.OracleShapeError):
        oracle.add_rms_norm_rows(np.zeros(10, np.float32), np.zeros(10, np.float32),
                                 np.ones(4, np.float32), 4, 1e-6)
