"""GPU parity: every C-ABI entry point against the CPU oracle on the same
seeded inputs, at the benchmark configurations' full sizes and at the edge
cases the reference's tests cover.

Bars (from the benchmark definition): the PQ2_0 gather is bit-exact; float
kernels reach max|gpu-ref|/max(|ref|,|gpu|) <= 1e-5, softmax <= 2e-5.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from conftest import bits_equal, rel_err

pytestmark = pytest.mark.gpu

TOL = 1e-5
TOL_SOFTMAX = 2e-5
SECTIONS = (11, 11, 10, 0)


def _t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _h(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def _say(*a):
    print(*a, flush=True)


# ---------------------------------------------------------------------------
# RMSNorm family
# ---------------------------------------------------------------------------

def test_rms_norm_known_answer(bh, dev):
    """src/kernels.rs:761-772 on the device."""
    x = _t(np.array([1, 2, 3, 4], np.float32), dev)
    w = _t(np.array([0.5, 1, 1.5, 2], np.float32), dev)
    y = _h(bh.rms_norm_rows(x, w, 1e-6))
    s = np.float32(1) / np.sqrt(np.float32(7.5) + np.float32(1e-6))
    assert np.all(np.abs(y - np.array([1, 2, 3, 4], np.float32) * np.array([.5, 1, 1.5, 2]) * s)
                  < 1e-6)


@pytest.mark.parametrize("rows,row_len", [
    (512, 5120),        # config 1 (block-per-row, 256 lanes x 5 float4)
    (2050, 5120),       # wave-per-row range, ragged last block of four rows
    (2048 * 24, 256),   # per-head q norm (one wave per row)
    (4096, 128),        # ssm_norm heads (half-wave rows)
    (33, 4),            # tiny rows, 64 rows per wave
    (7, 10240),         # 512-lane groups
    (5, 40000),         # beyond the register scheme: looped kernel
    (9, 7),             # odd length: looped kernel
    (3, 2052),          # 64-lane group with a ragged last float4 column
])
def test_rms_norm_rows(bh, oracle, synth, dev, rows, row_len):
    _say("rms_norm_rows", rows, row_len)
    r = synth.Rng(rows * 7 + row_len)
    x = r.normal(rows * row_len)
    w = r.normal(row_len, 1.0, 0.1)
    ref = oracle.rms_norm_rows(x, w, row_len, 1e-6)
    got = _h(bh.rms_norm_rows(_t(x, dev), _t(w, dev), 1e-6))
    err = rel_err(got, ref)
    _say("  rel", err)
    assert err <= TOL


def test_rms_norm_unaligned_and_inplace(bh, oracle, synth, dev):
    r = synth.Rng(3)
    x = r.normal(1 + 64 * 256)
    w = r.normal(256, 1.0, 0.1)
    xt = _t(x, dev)
    view = xt[1:]                       # 4-byte aligned only: looped kernel
    got = _h(bh.rms_norm_rows(view, _t(w, dev), 1e-6))
    assert rel_err(got, oracle.rms_norm_rows(x[1:], w, 256, 1e-6)) <= TOL
    xt2 = _t(x[:64 * 256], dev)         # in place (rms_norm_inplace)
    bh.rms_norm_rows(xt2, _t(w, dev), 1e-6, out=xt2)
    assert rel_err(_h(xt2), oracle.rms_norm_rows(x[:64 * 256], w, 256, 1e-6)) <= TOL


def test_rms_norm_single_vector(bh, oracle, synth, dev):
    r = synth.Rng(4)
    x = r.normal(5120)
    w = r.normal(5120, 1.0, 0.1)
    out = _t(np.zeros(5120, np.float32), dev)
    xt, wt = _t(x, dev), _t(w, dev)
    bh.check(bh.lib().bh_rms_norm(xt.data_ptr(), wt.data_ptr(), 5120, 1e-6, out.data_ptr(), None))
    assert rel_err(_h(out), oracle.rms_norm(x, w, 1e-6)) <= TOL


@pytest.mark.parametrize("rows,row_len", [(2048, 5120), (3071, 5120), (3, 36)])
def test_add_rms_norm_rows(bh, oracle, synth, dev, rows, row_len):
    _say("add_rms_norm_rows", rows, row_len)
    r = synth.Rng(11)
    x = r.normal(rows * row_len)
    a = r.normal(rows * row_len)
    w = r.normal(row_len, 1.0, 0.1)
    s_ref, y_ref = oracle.add_rms_norm_rows(x, a, w, row_len, 1e-6)
    xt = _t(x, dev)
    s, y = bh.add_rms_norm_rows(xt, _t(a, dev), _t(w, dev), 1e-6, sum_out=xt)  # cur += in place
    assert bits_equal(_h(s), s_ref)
    assert rel_err(_h(y), y_ref) <= TOL


# ---------------------------------------------------------------------------
# L2 / activations / gate prep
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("rows,row_len", [(4096 * 48, 128), (16, 128), (5, 6), (4, 2048)])
def test_l2_norm_rows(bh, oracle, synth, dev, rows, row_len):
    _say("l2_norm_rows", rows, row_len)
    x = synth.Rng(rows + row_len).normal(rows * row_len)
    x[:row_len] = 0.0  # a zero row stays zero (eps floor)
    ref = oracle.l2_norm_rows(x, row_len, 1e-6)
    got = _h(bh.l2_norm_rows(_t(x, dev), row_len, 1e-6))
    assert np.all(got[:row_len] == 0)
    err = rel_err(got, ref)
    _say("  rel", err, "bit-identical:", bits_equal(got, ref))
    assert err <= TOL


def test_l2_known_rows(bh, dev):
    """src/kernels.rs:814-828 on the device."""
    x = _t(np.array([3, 4, 0, 0, 1, 1, 1, 1], np.float32), dev)
    y = _h(bh.l2_norm_rows(x, 4, 1e-12))
    assert abs(y[0] - 0.6) < 1e-6 and abs(y[1] - 0.8) < 1e-6
    assert abs(float((y[4:] ** 2).sum()) - 1) < 1e-6


def test_silu_l2_norm_rows(bh, oracle, synth, dev):
    x = synth.Rng(21).normal(4096 * 6144).reshape(4096, 6144)
    ref = oracle.silu_l2_part(x, 6144, 128, 1e-6)
    got = _h(bh.l2_norm_rows(_t(x, dev), 128, 1e-6, silu_first=True))
    assert rel_err(got, ref) <= TOL


SPECIAL = np.array([0.0, -0.0, 1.0, -1.0, 20.0, 20.000002, 19.999998, 1000.0, -1000.0, 88.0,
                    -88.0, 1e-30, -1e-30, np.inf, -np.inf, np.nan, 3.4e38, -3.4e38], np.float32)


@pytest.mark.parametrize("mode", [0, 1, 2, 3, 4])
@pytest.mark.parametrize("n", [17408, 6151, 3])
def test_unary_modes(bh, oracle, synth, dev, mode, n):
    r = synth.Rng(100 + mode)
    a = r.normal(n, 0.0, 4.0)
    a[: min(n, SPECIAL.size)] = SPECIAL[: min(n, SPECIAL.size)]
    b = r.normal(n)
    ref = oracle.unary(mode, a, b)
    got = _h(bh.unary(mode, _t(a, dev), _t(b, dev)))
    err = rel_err(got, ref)
    _say("unary", mode, n, "rel", err)
    assert err <= TOL


def test_unary_special_points_exact(bh, dev):
    """src/kernels.rs:830-838 on the device."""
    x = _t(np.array([0.0, 1000.0, -1000.0, 100.0], np.float32), dev)
    silu = _h(bh.unary(bh.BH_SILU, x))
    sig = _h(bh.unary(bh.BH_SIGMOID, x))
    sp = _h(bh.unary(bh.BH_SOFTPLUS, x))
    assert silu[0] == 0.0 and abs(silu[1] - 1000) < 1e-3
    assert abs(sig[0] - 0.5) < 1e-7 and sig[2] == 0.0
    assert abs(sp[0] - np.log(2)) < 1e-7 and sp[3] == 100.0


def test_unary_unaligned_inplace(bh, oracle, synth, dev):
    a = synth.Rng(5).normal(1001)
    t = _t(a, dev)
    v = t[1:]
    bh.unary(bh.BH_SOFTPLUS, v, out=v)
    assert rel_err(_h(v), oracle.unary(2, a[1:])) <= TOL


def _gdn_inputs(synth, n_tok, conv_dim, inner, n_head, seed):
    r = synth.Rng(seed)
    conv = r.normal(n_tok * conv_dim).reshape(n_tok, conv_dim)
    dt = r.normal(n_tok * n_head).reshape(n_tok, n_head)
    bias = r.normal(n_head, 0.0, 0.5)
    A = (-np.exp(r.uniform(n_head) * 2.0)).astype(np.float32)
    beta = r.normal(n_tok * n_head).reshape(n_tok, n_head)
    z = r.normal(n_tok * inner).reshape(n_tok, inner)
    y = r.normal(n_tok * inner).reshape(n_tok, inner)
    return conv, dt, bias, A, beta, z, y


@pytest.mark.parametrize("gate_mode", [4, 3])
@pytest.mark.parametrize("shape", [
    (4096, 6144, 6144, 6144, 48),    # config 3: whole conv row L2-normed, 48 gates
    (64, 10240, 4096, 6144, 48),     # model layout: q,k (4096 ch) L2, v (6144) silu only
    (3, 100, 60, 10, 5),             # odd widths: looped kernel
])
def test_gdn_prep_fused(bh, oracle, synth, dev, gate_mode, shape):
    import torch
    n_tok, conv_dim, l2_dim, inner, n_head = shape
    _say("gdn_prep_fused", shape, "mode", gate_mode)
    head_dim = 128 if conv_dim % 128 == 0 else 20
    conv, dt, bias, A, beta, z, y = _gdn_inputs(synth, n_tok, conv_dim, inner, n_head, 2)
    d = {k: _t(v, dev) for k, v in dict(conv=conv, dt=dt, bias=bias, A=A, beta=beta, z=z,
                                        y=y).items()}
    conv_out = torch.empty_like(d["conv"])
    gated = torch.empty_like(d["z"])
    gate = torch.empty_like(d["dt"])
    beta_o = torch.empty_like(d["beta"])
    args = bh.make_gdn_args(conv=d["conv"], conv_out=conv_out, z=d["z"], y=d["y"],
                            gated_out=gated, alpha_raw=d["dt"], dt_bias=d["bias"],
                            ssm_a=d["A"], beta_raw=d["beta"], gate_out=gate, beta_out=beta_o,
                            n_tok=n_tok, conv_dim=conv_dim, l2_dim=l2_dim, head_dim=head_dim,
                            inner_dim=inner, n_v_head=n_head, gate_mode=gate_mode, eps=1e-6)
    bh.gdn_prep_fused(args)
    ref_conv = oracle.silu_l2_part(conv, l2_dim, head_dim, 1e-6)
    ref_gated = oracle.unary(gate_mode, z, y)
    ref_gate, ref_beta = oracle.gdn_gate_prep(dt, bias, A, beta)
    errs = [rel_err(_h(conv_out), ref_conv), rel_err(_h(gated), ref_gated),
            rel_err(_h(gate), ref_gate), rel_err(_h(beta_o), ref_beta)]
    _say("  rel conv/gated/gate/beta", errs)
    assert max(errs) <= TOL


def test_gdn_gate_prep_standalone(bh, oracle, synth, dev):
    _, dt, bias, A, beta, _, _ = _gdn_inputs(synth, 4096, 4, 4, 48, 9)
    dt[0, :4] = [25.0, 20.0, -30.0, 0.0]  # identity branch, threshold, tiny
    g, b = bh.gdn_gate_prep(_t(dt, dev), _t(bias, dev), _t(A, dev), _t(beta, dev))
    rg, rb = oracle.gdn_gate_prep(dt, bias, A, beta)
    assert rel_err(_h(g), rg) <= TOL and rel_err(_h(b), rb) <= TOL


# ---------------------------------------------------------------------------
# Softmax
# ---------------------------------------------------------------------------

def test_softmax_vocab_temperature(bh, oracle, synth, dev):
    """config 4a: [64, 248320] ~N(0,3) with 1% +10 spikes, temperature 0.7
    (split-row path)."""
    r = synth.Rng(3)
    n = 64 * 248320
    x = r.normal(n, 0.0, 3.0)
    spikes = r.uniform(n) < 0.01
    x[spikes] += np.float32(10.0)
    inv_t = float(np.float32(1.0) / np.float32(0.7))
    ref = oracle.softmax_rows(x, 248320, inv_t)
    got = _h(bh.softmax_rows(_t(x, dev), 248320, inv_t))
    err = rel_err(got, ref)
    sums = got.reshape(64, -1).astype(np.float64).sum(1)
    _say("softmax vocab rel", err, "row sums", sums.min(), sums.max())
    assert err <= TOL_SOFTMAX
    assert np.all(np.abs(sums - 1) < 1e-4)


def test_softmax_attention_causal(bh, oracle, synth, dev):
    """config 4b: scores [24, 2048, 2048] ~N(0,2), -inf above the diagonal."""
    r = synth.Rng(4)
    x = r.normal(24 * 2048 * 2048, 0.0, 2.0).reshape(24, 2048, 2048)
    mask = np.triu(np.ones((2048, 2048), bool), 1)
    x[:, mask] = -np.inf
    ref = oracle.softmax_rows(x, 2048)
    got = _h(bh.softmax_rows(_t(x, dev), 2048))
    err = rel_err(got, ref)
    _say("softmax causal rel", err)
    assert err <= TOL_SOFTMAX
    assert np.all(got.reshape(24, 2048, 2048)[:, mask] == 0)


@pytest.mark.parametrize("rows,row_len", [(2, 4), (1000, 7), (3, 40000), (5000, 96),
                                          (7, 16384), (2, 1), (2, 1000000), (3, 300004),
                                          (1, 4194304)])
def test_softmax_shapes(bh, oracle, synth, dev, rows, row_len):
    x = synth.Rng(rows * row_len).normal(rows * row_len, 0.0, 2.0)
    ref = oracle.softmax_rows(x, row_len)
    got = _h(bh.softmax_rows(_t(x, dev), row_len))
    assert rel_err(got, ref) <= TOL_SOFTMAX


@pytest.mark.parametrize("rows,row_len", [(64, 248320), (96, 1000), (5, 1001)])
def test_softmax_sampler_norm(bh, oracle, synth, dev, rows, row_len):
    """bh_softmax_rows_ex(BH_SOFTMAX_SAMPLER_NORM): the sampler's f64
    normalisation (src/sampler.rs:118-126) on the split path (vocabulary
    rows), the register path and the looped path (odd row length); within
    2 ulps of the plain normalisation of the same exponentials."""
    x = synth.Rng(rows + row_len).normal(rows * row_len, 0.0, 3.0)
    inv_t = np.float32(1.0) / np.float32(0.7)
    ref = oracle.softmax_rows(x, row_len, inv_t, sampler_norm=True)
    xt = _t(x, dev)
    got = _h(bh.softmax_rows(xt, row_len, inv_t, sampler_norm=True))
    _say("softmax sampler norm", rows, row_len, "rel", rel_err(got, ref))
    assert rel_err(got, ref) <= TOL_SOFTMAX
    plain = _h(bh.softmax_rows(xt, row_len, inv_t))
    d = np.abs(got.view(np.int32).astype(np.int64) - plain.view(np.int32).astype(np.int64))
    assert d.max() <= 2
    lib = bh.lib()
    assert lib.bh_softmax_rows_ex(xt.data_ptr(), xt.numel(), row_len, 1.0, 2,
                                  xt.data_ptr(), None) == bh.BH_ERR_ARG


def test_softmax_mask_safe_and_nan_rows(bh, dev):
    """src/kernels.rs:840-853, plus an all -inf row (NaN, as the reference)."""
    x = np.array([1, 2, 3, -np.inf, 0, 0, 0, 0, -np.inf, -np.inf, -np.inf, -np.inf], np.float32)
    y = _h(bh.softmax_rows(_t(x, dev), 4))
    assert abs(y[:4].sum() - 1) < 1e-6 and y[3] == 0.0
    assert np.all(np.abs(y[4:8] - 0.25) < 1e-6)
    assert np.all(np.isnan(y[8:]))
    # the same on the split path (long rows)
    big = np.full(2 * 20000, -np.inf, np.float32)
    big[:20000] = 0.0
    yb = _h(bh.softmax_rows(_t(big, dev), 20000))
    assert np.allclose(yb[:20000], 1 / 20000) and np.all(np.isnan(yb[20000:]))


def test_softmax_nan_and_inf_entries(bh, oracle, synth, dev):
    """NaN anywhere in a row makes the whole row NaN (it reaches the f64 sum),
    +inf too (inf - inf); a row whose only finite part is one chunk still
    normalises.  Checked on the register path and on the split path."""
    for row_len in (2048, 40000):
        x = synth.Rng(row_len).normal(4 * row_len)
        x[0:row_len] = np.nan                      # all-NaN row
        x[row_len + 17] = np.nan                   # one NaN
        x[2 * row_len + 3] = np.inf                # one +inf
        x[3 * row_len: 3 * row_len + row_len // 2] = -np.inf   # half masked
        got = _h(bh.softmax_rows(_t(x, dev), row_len))
        ref = oracle.softmax_rows(x, row_len)
        assert rel_err(got, ref) <= TOL_SOFTMAX


def test_softmax_wide_nan_inf_rows(bh, oracle, synth, dev):
    """Vocabulary-wide rows (split path, 61 chunk states per row): an all-NaN
    row, one NaN in the last chunk, one +inf in a middle chunk, a row whose
    first three quarters are masked (-inf), and a row masked but for one
    value."""
    row_len = 248320
    x = synth.Rng(77).normal(6 * row_len, 0.0, 3.0)
    x[0:row_len] = np.nan
    x[row_len + 240000] = np.nan
    x[2 * row_len + 100000] = np.inf
    x[3 * row_len: 3 * row_len + 3 * 65536] = -np.inf
    x[4 * row_len: 5 * row_len] = -np.inf
    x[4 * row_len + 70000] = 1.5
    got = _h(bh.softmax_rows(_t(x, dev), row_len, 1.25))
    ref = oracle.softmax_rows(x, row_len, 1.25)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert rel_err(got, ref) <= TOL_SOFTMAX
    assert got[4 * row_len + 70000] == 1.0 and np.count_nonzero(got[4 * row_len: 5 * row_len]) == 1


def test_softmax_split_repeated_mixed_shapes(bh, oracle, synth, dev):
    """The wide-row path keeps per-chunk partial states in the library's
    scratch, reused by every call: repeated calls with changing shapes (whose
    partials overlap earlier calls' stale ones) must all give the oracle's
    result."""
    cases = [(64, 248320), (3, 40000), (200, 20480), (3, 40000), (64, 248320), (1, 16384)]
    for i, (rows, row_len) in enumerate(cases):
        x = synth.Rng(500 + i).normal(rows * row_len, 0.0, 3.0)
        got = _h(bh.softmax_rows(_t(x, dev), row_len, 1.25))
        err = rel_err(got, oracle.softmax_rows(x, row_len, 1.25))
        _say("split repeat", rows, row_len, err)
        assert err <= TOL_SOFTMAX


def test_softmax_inplace(bh, oracle, synth, dev):
    x = synth.Rng(8).normal(49152)
    for row_len in (2048, 49152):
        t = _t(x, dev)
        bh.softmax_rows(t, row_len, out=t)
        assert rel_err(_h(t), oracle.softmax_rows(x, row_len)) <= TOL_SOFTMAX


# ---------------------------------------------------------------------------
# IMROPE and the attention pre-block
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("head_dim,n_dims,sections,pos,n_head", [(*c, 24)[:5] for c in [
    (256, 64, SECTIONS, (37, 37, 37, 37)),
    (256, 64, SECTIONS, (3, 5, 7, 0)),
    (128, 32, (2, 3, 1, 2), (100, 2000, 7, 9)),
    (256, 256, SECTIONS, (2047, 2047, 2047, 2047)),
    (128, 64, SECTIONS, (911, 12, 40, 7)),         # n_dims 64 on 32-lane rows
    (100, 20, (1, 1, 1, 1), (3, 50, 700, 9000)),   # looped kernel
    (256, 256, SECTIONS, (1500, 3, 800, 2), 1),     # one-wave block, 128-pair table
    (256, 64, SECTIONS, (5, 6, 7, 8), 3),           # partial wave
    (64, 64, (4, 2, 2, 0), (900, 901, 902, 0), 61),  # several blocks per token
]])
def test_rope_imrope_heads(bh, oracle, synth, dev, head_dim, n_dims, sections, pos, n_head):
    h = synth.Rng(head_dim + n_dims).normal(n_head * head_dim).reshape(1, n_head, head_dim)
    ref = np.stack([oracle.rope_imrope(h[0, i], *pos, n_dims, sections, 1e7)
                    for i in range(n_head)])[None]
    t = _t(h, dev)
    bh.rope_imrope(t, _t(np.array([pos], np.int32), dev), n_dims, sections, 1e7)
    err = rel_err(_h(t), ref)
    _say("rope", head_dim, n_dims, pos, "rel", err)
    assert err <= TOL


def test_host_rope_mirror(bh, oracle, synth):
    h = synth.Rng(77).normal(256)
    sec = (ctypes.c_int32 * 4)(*SECTIONS)
    got = h.copy()
    bh.check(bh.lib().bh_host_rope_imrope(got.ctypes.data, 256, 37, 37, 37, 37, 64, sec, 1e7))
    assert rel_err(got, oracle.rope_imrope(h, 37, 37, 37, 37, 64, SECTIONS, 1e7)) <= TOL
    # pos 0 is the identity on the device too
    z = h.copy()
    bh.check(bh.lib().bh_host_rope_imrope(z.ctypes.data, 256, 0, 0, 0, 0, 64, sec, 1e7))
    assert np.array_equal(z, h)


def _qk_case(synth, n_tok, n_q, n_k, hd, seed, stride=None):
    r = synth.Rng(seed)
    stride = stride or hd
    q = r.normal(n_tok * n_q * stride).reshape(n_tok, n_q, stride)
    k = r.normal(n_tok * n_k * hd).reshape(n_tok, n_k, hd)
    wq = r.normal(hd, 1.0, 0.1)
    wk = r.normal(hd, 1.0, 0.1)
    return q, k, wq, wk, synth.positions(n_tok)


def test_qk_norm_rope_config2(bh, oracle, synth, dev):
    """config 2: q [2048,24,256], k [2048,4,256], rotary 64, sections
    [11,11,10,0], theta 1e7, positions 0..2047."""
    import torch
    q, k, wq, wk, pos = _qk_case(synth, 2048, 24, 4, 256, 1)
    rq, rk, _ = oracle.qk_norm_rope(q, k, wq, wk, pos, 24, 4, 256, 64, SECTIONS, 1e7, 1e-6)
    d = [_t(a, dev) for a in (q, k, wq, wk, pos)]
    qo, ko = torch.empty_like(d[0]), torch.empty_like(d[1])
    bh.qk_norm_rope(bh.make_qk_args(d[0], qo, d[1], ko, d[2], d[3], d[4], 2048, 24, 4))
    eq, ek = rel_err(_h(qo), rq), rel_err(_h(ko), rk)
    _say("qk_norm_rope config2 rel q/k", eq, ek)
    assert eq <= TOL and ek <= TOL
    # in place gives the same bits
    bh.qk_norm_rope(bh.make_qk_args(d[0], d[0], d[1], d[1], d[2], d[3], d[4], 2048, 24, 4))
    assert bits_equal(_h(d[0]), _h(qo)) and bits_equal(_h(d[1]), _h(ko))


def test_qk_norm_rope_fused_gate_split(bh, oracle, synth, dev):
    """attn_q rows [q | gate] per head (src/forward.rs:237-241): split, norm,
    rope and sigmoid(gate) in one pass."""
    import torch
    q, k, wq, wk, pos = _qk_case(synth, 64, 24, 4, 256, 2, stride=512)
    pos = pos + 1000
    rq, rk, rg = oracle.qk_norm_rope(q, k, wq, wk, pos, 24, 4, 256, 64, SECTIONS, 1e7, 1e-6,
                                     q_head_stride=512, want_gate=True)
    d = [_t(a, dev) for a in (q, k, wq, wk, pos)]
    qo = torch.empty((64, 24, 256), dtype=torch.float32, device=dev)
    go = torch.empty_like(qo)
    ko = torch.empty_like(d[1])
    bh.qk_norm_rope(bh.make_qk_args(d[0], qo, d[1], ko, d[2], d[3], d[4], 64, 24, 4,
                                    q_head_stride=512, gate_out=go))
    assert rel_err(_h(qo), rq) <= TOL and rel_err(_h(ko), rk) <= TOL
    assert rel_err(_h(go), rg) <= TOL


@pytest.mark.parametrize("hd,n_dims,n_q,n_k", [(128, 32, 16, 0), (64, 16, 3, 5), (96, 24, 4, 2),
                                               (128, 64, 8, 2), (64, 64, 5, 3), (256, 128, 6, 1),
                                               (32, 8, 40, 9)])
def test_qk_norm_rope_other_shapes(bh, oracle, synth, dev, hd, n_dims, n_q, n_k):
    import torch
    q, k, wq, wk, pos = _qk_case(synth, 37, n_q, n_k, hd, 3)
    pos[:, 1] += 5
    pos[:, 3] *= 3
    rq, rk, _ = oracle.qk_norm_rope(q, k if n_k else None, wq, wk, pos, n_q, n_k, hd, n_dims,
                                    (2, 2, 1, 1), 1e4, 1e-6)
    d = [_t(a, dev) for a in (q, k, wq, wk, pos)]
    qo, ko = torch.empty_like(d[0]), torch.empty_like(d[1])
    bh.qk_norm_rope(bh.make_qk_args(d[0], qo, d[1] if n_k else None, ko if n_k else None, d[2],
                                    d[3], d[4], 37, n_q, n_k, head_dim=hd, n_dims=n_dims,
                                    sections=(2, 2, 1, 1), freq_base=1e4))
    assert rel_err(_h(qo), rq) <= TOL
    if n_k:
        assert rel_err(_h(ko), rk) <= TOL


# ---------------------------------------------------------------------------
# PQ2_0 gather
# ---------------------------------------------------------------------------

def test_pq2_gather_config5_bit_exact(bh, oracle, synth, dev):
    """config 5: table 248320 x 5120 (built on the device), 8192 uniform ids;
    every gathered row bit-exact, and the fused RMSNorm too: the kernel adds
    the squares in the reference's sequential order (a tree-ordered sum
    drifts ~1e-5 on these quantised rows, beyond the 1e-5 bar)."""
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    table = synth.torch_pq2_table(248320, 5120, dev, generator=g)
    ids = synth.Rng(5).u64(8192) % np.uint64(248320)
    ids = ids.astype(np.uint32)
    w = synth.Rng(6).normal(5120, 1.0, 0.1)
    idt, wt = _t(ids, dev), _t(w, dev)
    emb, nrm = bh.pq2_embed_gather(table, 5120, 248320, idt, w=wt, eps=1e-6)
    emb_only = bh.pq2_embed_gather(table, 5120, 248320, idt)
    host_rows = _h(table[idt.long()])
    ref_e, ref_n = oracle.embed_gather(host_rows, 5120, 8192, np.arange(8192, dtype=np.uint32),
                                       w, 1e-6)
    ge, gn = _h(emb), _h(nrm)
    assert bits_equal(ge, ref_e)
    assert bits_equal(_h(emb_only), ref_e)
    err = rel_err(gn, ref_n)
    _say("gather+rms rel", err, "bit-identical:", bits_equal(gn, ref_n))
    assert err <= TOL
    assert bits_equal(gn, ref_n)


@pytest.mark.parametrize("n_ids", [2048, 2050, 4095, 1000, 17])
def test_pq2_gather_rms_block_shapes(bh, oracle, synth, dev, n_ids):
    """The fused gather + RMSNorm picks 16, 8 or 4 rows per block by batch
    size (2048 and 4095 ids: 8-row blocks, 1000 and 17: 4-row blocks on a
    256-CU device; 2050: a ragged last block): both outputs bit-exact."""
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(n_ids)
    table = synth.torch_pq2_table(4096, 5120, dev, generator=g)
    ids = (synth.Rng(n_ids).u64(n_ids) % np.uint64(4096)).astype(np.uint32)
    w = synth.Rng(n_ids + 1).normal(5120, 1.0, 0.1)
    idt = _t(ids, dev)
    emb, nrm = bh.pq2_embed_gather(table, 5120, 4096, idt, w=_t(w, dev), eps=1e-6)
    host_rows = _h(table[idt.long()])
    ref_e, ref_n = oracle.embed_gather(host_rows, 5120, n_ids, np.arange(n_ids, dtype=np.uint32),
                                       w, 1e-6)
    _say("gather+rms block shapes", n_ids)
    assert bits_equal(_h(emb), ref_e)
    assert bits_equal(_h(nrm), ref_n)


def test_pq2_gather_every_f16_scale(bh, oracle, synth, dev):
    """All 65536 f16 scale patterns x all 4 codes (NaN payloads, infinities,
    subnormals, -0.0 from code 1), bit-exact against the x86 reference."""
    rows, ne0 = 128, 512 * 128
    scales = np.arange(65536, dtype=np.uint16).reshape(rows, 512)
    codes = np.tile(np.array([0, 1, 2, 3], np.uint8), rows * ne0 // 4).reshape(rows, ne0)
    table = synth.pack_pq2_rows(codes, scales)
    ids = np.arange(rows, dtype=np.uint32)[::-1].copy()
    got = _h(bh.pq2_embed_gather(_t(table, dev), ne0, rows, _t(ids, dev)))
    ref = oracle.embed_gather(table, ne0, rows, ids)
    assert bits_equal(got, ref)


# Batches of at least 16 rows per CU (4096 on MI355X) take the two-launch
# path (closed-form row scales + flat writers), shorter ones the one-launch
# kernel; LONG tiles a test's ids up to that size so both paths see its rows.
LONG = 4096


def _tiled(ids, tile):
    return np.tile(ids, -(-LONG // ids.size)) if tile else ids


@pytest.mark.parametrize("tile", [False, True])
def test_pq2_gather_rms_every_f16_scale(bh, oracle, synth, dev, tile):
    """The fused norm over rows holding every f16 scale pattern and every
    code (code 3 included): the closed-form sum of squares must equal the
    reference's sequential f32 sum, so every row with finite scales is
    bit-exact in both outputs; rows with an infinite or NaN scale are NaN at
    the same positions."""
    rows, ne0 = 64, 8 * 128
    scales = np.arange(65536, dtype=np.uint16)[::8][:rows * 8].reshape(rows, 8).copy()
    scales[5] = 0x3c00          # scale 1.0: squares 1 and 4, sums of small integers
    scales[6] = 0x0001          # smallest subnormal scale
    scales[7] = 0x7bff          # largest finite scale
    rng = synth.Rng(17)
    codes = (rng.u64(rows * ne0) % np.uint64(4)).astype(np.uint8).reshape(rows, ne0)
    codes[9] = 3
    table = synth.pack_pq2_rows(codes, scales)
    ids = _tiled(np.arange(rows, dtype=np.uint32)[::-1].copy(), tile)
    w = synth.Rng(18).normal(ne0, 1.0, 0.1)
    e, n = bh.pq2_embed_gather(_t(table, dev), ne0, rows, _t(ids, dev), w=_t(w, dev), eps=1e-6)
    ref_e, ref_n = oracle.embed_gather(table, ne0, rows, ids, w, 1e-6)
    ge, gn = _h(e), _h(n)
    assert bits_equal(ge, ref_e)
    finite = np.all((scales[ids] & 0x7c00) != 0x7c00, axis=1)
    assert finite.sum() >= ids.size * (rows - 8) // rows
    assert bits_equal(gn[finite], ref_n[finite])
    assert np.array_equal(np.isnan(gn), np.isnan(ref_n))


@pytest.mark.parametrize("tile", [False, True])
@pytest.mark.parametrize("case", ["few_scales", "big_then_tiny", "ties", "unit_scale"])
def test_pq2_gather_rms_closed_form_edge_rows(bh, oracle, synth, dev, case, tile):
    """Rows whose sequential sum of squares is easy to get wrong: one scale
    repeated over many blocks (long runs across powers of two), a large scale
    followed by tiny ones (the sum stops moving), power-of-two scales (sums
    that land on rounding ties), and scale 1.0 (exact integer sums).  Both
    outputs bit-exact against the reference's sequential loop."""
    rows, ne0 = 96, 40 * 128
    rng = np.random.default_rng({"few_scales": 1, "big_then_tiny": 2, "ties": 3, "unit_scale": 4}[case])
    codes = rng.choice(np.array([0, 1, 2], np.uint8), size=(rows, ne0), p=[0.3, 0.4, 0.3])
    if case == "few_scales":
        pool = rng.integers(0x0400, 0x7400, size=(rows, 3)).astype(np.uint16)
        scales = np.take_along_axis(pool, rng.integers(0, 3, size=(rows, 40)), 1)
    elif case == "big_then_tiny":
        scales = rng.integers(1, 0x1000, size=(rows, 40)).astype(np.uint16)
        scales[:, 0] = rng.integers(0x7000, 0x7400, size=rows)
    elif case == "ties":
        # scale 2^k: squares are powers of two, so sums land on ties often
        scales = (rng.integers(5, 25, size=(rows, 40)) << 10).astype(np.uint16)
    else:
        scales = np.full((rows, 40), 0x3c00, np.uint16)
    table = synth.pack_pq2_rows(codes, scales)
    ids = _tiled(rng.permutation(rows).astype(np.uint32), tile)
    w = synth.Rng(19).normal(ne0, 1.0, 0.1)
    e, n = bh.pq2_embed_gather(_t(table, dev), ne0, rows, _t(ids, dev), w=_t(w, dev), eps=1e-6)
    ref_e, ref_n = oracle.embed_gather(table, ne0, rows, ids, w, 1e-6)
    assert bits_equal(_h(e), ref_e)
    assert bits_equal(_h(n), ref_n)


@pytest.mark.parametrize("ne0", [128, 200, 256, 5120, 130])
def test_pq2_gather_shapes(bh, oracle, synth, dev, ne0):
    table = synth.pq2_table(synth.Rng(ne0), 50, ne0)
    ids = (synth.Rng(1).u64(300) % np.uint64(50)).astype(np.uint32)
    w = synth.Rng(2).normal(ne0, 1.0, 0.1)
    emb, nrm = bh.pq2_embed_gather(_t(table, dev), ne0, 50, _t(ids, dev), w=_t(w, dev))
    ref_e, ref_n = oracle.embed_gather(table, ne0, 50, ids, w, 1e-6)
    assert bits_equal(_h(emb), ref_e)
    assert bits_equal(_h(nrm), ref_n)   # sequential sum of squares on every path


@pytest.mark.parametrize("ne0", [1000, 1024, 5120])
def test_pq2_gather_rms_long_batch_shapes(bh, oracle, synth, dev, ne0):
    """Long batches (two-launch path) with a partial last 128-block
    (ne0=1000: 104 valid weights in block 7), an 8-block row and the model
    row; random codes 0..3, so code-3 blocks take the weight-by-weight sum
    next to closed-form blocks in the same row."""
    rows = 300
    rng = np.random.default_rng(ne0)
    nblk = -(-ne0 // 128)
    codes = rng.choice(np.array([0, 1, 2, 3], np.uint8), size=(rows, ne0), p=[0.3, 0.4, 0.28, 0.02])
    scales = rng.integers(0x0400, 0x5000, size=(rows, nblk)).astype(np.uint16)
    table = synth.pack_pq2_rows(codes, scales)
    ids = rng.integers(0, rows, size=LONG + 5).astype(np.uint32)
    w = synth.Rng(20).normal(ne0, 1.0, 0.1)
    e, n = bh.pq2_embed_gather(_t(table, dev), ne0, rows, _t(ids, dev), w=_t(w, dev), eps=1e-6)
    ref_e, ref_n = oracle.embed_gather(table, ne0, rows, ids, w, 1e-6)
    assert bits_equal(_h(e), ref_e)
    assert bits_equal(_h(n), ref_n)


@pytest.mark.parametrize("tile", [False, True])
def test_pq2_gather_rms_bad_ids_and_ragged_tail(bh, oracle, synth, dev, tile):
    """Bad ids inside a 16-row block give zero rows in both outputs; the other
    rows of the block stay bit-exact; T not a multiple of 16."""
    import torch
    table = synth.pq2_table(synth.Rng(12), 40, 5120)
    ids = (synth.Rng(13).u64(37) % np.uint64(40)).astype(np.uint32)
    ids[[3, 20, 36]] = [40, 1000, 4294967295]
    ids = _tiled(ids, tile)
    w = synth.Rng(14).normal(5120, 1.0, 0.1)
    bad = torch.full((1,), -1, dtype=torch.int32, device=dev)
    emb, nrm = bh.pq2_embed_gather(_t(table, dev), 5120, 40, _t(ids, dev), w=_t(w, dev),
                                   bad_id=bad)
    e, n = _h(emb), _h(nrm)
    good = ids < 40
    assert np.all(e[~good] == 0) and np.all(n[~good] == 0)
    ref_e, ref_n = oracle.embed_gather(table, 5120, 40, ids[good], w, 1e-6)
    assert bits_equal(e[good], ref_e) and bits_equal(n[good], ref_n)
    assert int(_h(bad)[0]) & 0xFFFFFFFF in (40, 1000, 4294967295)


def test_pq2_gather_bad_ids(bh, synth, dev):
    import torch
    table = synth.pq2_table(synth.Rng(1), 10, 5120)
    ids = np.array([3, 10, 2, 4000000000], np.uint32)
    bad = torch.full((1,), -1, dtype=torch.int32, device=dev)
    out = bh.pq2_embed_gather(_t(table, dev), 5120, 10, _t(ids, dev), bad_id=bad)
    o = _h(out)
    assert np.all(o[1] == 0) and np.all(o[3] == 0) and np.any(o[0] != 0)
    assert int(_h(bad)[0]) & 0xFFFFFFFF in (10, 4000000000)


def test_host_mirrors(bh, oracle, synth):
    lib = bh.lib()
    table = synth.pq2_table(synth.Rng(3), 20, 5120)
    toks = np.array([19, 0, 7, 7], np.uint32)
    out = np.empty((4, 5120), np.float32)
    bh.check(lib.bh_host_batch_embed(table.ctypes.data, table.size, 5120, 20, toks.ctypes.data,
                                     4, out.ctypes.data))
    assert bits_equal(out, oracle.embed_gather(table, 5120, 20, toks))
    row = np.empty(5120, np.float32)
    bh.check(lib.bh_host_decode_pq2_0_row(table[7].ctypes.data, 1360, 5120, row.ctypes.data))
    assert bits_equal(row, oracle.decode_pq2_0_row(table[7], 5120))
    x = synth.Rng(4).normal(8 * 256)
    w = synth.Rng(5).normal(256, 1.0, 0.1)
    y = np.empty_like(x)
    bh.check(lib.bh_host_rms_norm_rows(x.ctypes.data, x.size, w.ctypes.data, 256, 256, 1e-6,
                                       y.ctypes.data))
    assert rel_err(y, oracle.rms_norm_rows(x, w, 256, 1e-6)) <= TOL
    bh.check(lib.bh_host_l2_norm_rows(x.ctypes.data, x.size, 128, 1e-6, y.ctypes.data))
    assert rel_err(y, oracle.l2_norm_rows(x, 128, 1e-6)) <= TOL
    bh.check(lib.bh_host_softmax_rows(x.ctypes.data, x.size, 256, y.ctypes.data))
    assert rel_err(y, oracle.softmax_rows(x, 256)) <= TOL_SOFTMAX
    m = x.copy()
    bh.check(lib.bh_host_map_inplace(m.ctypes.data, m.size, bh.BH_SOFTPLUS))
    assert rel_err(m, oracle.unary(2, x)) <= TOL
    v = x[:5120].copy() if x.size >= 5120 else synth.Rng(6).normal(5120)
    wv = synth.Rng(7).normal(v.size, 1.0, 0.1)
    yv = np.empty_like(v)
    bh.check(lib.bh_host_rms_norm(v.ctypes.data, v.size, wv.ctypes.data, 1e-6, yv.ctypes.data))
    assert rel_err(yv, oracle.rms_norm(v, wv, 1e-6)) <= TOL


def test_side_stream(bh, oracle, synth, dev):
    """Work enqueued on a non-default stream lands there."""
    import torch
    s = torch.cuda.Stream()
    x = synth.Rng(9).normal(4096 * 256)
    w = synth.Rng(10).normal(256, 1.0, 0.1)
    xt, wt = _t(x, dev), _t(w, dev)
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        y = bh.rms_norm_rows(xt, wt, 1e-6, stream=s)
    s.synchronize()
    assert rel_err(y.cpu().numpy(), oracle.rms_norm_rows(x, w, 256, 1e-6)) <= TOL
