"""GPU parity of the KV append (bh_kv_store) and of grouped-query attention
over the cache (bh_attention) against the oracle's restatement of
src/forward.rs:273-375 (the reference's one-token loop, run per query).

Bars: the f32 store bit for bit, the f16 store = gguf::f32_to_half bit for
bit (specials and the subnormal range included); attention outputs
max|gpu-ref| / max(|ref|, |gpu|) <= 1e-5 (scores and P.V summed in another
order; the generic path keeps the reference's sequence except the f64 sum's
order).
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import rel_err

pytestmark = pytest.mark.gpu

TOL = 1e-5
MODEL = (24, 4, 256)  # n_head, n_kv, hd of the model (24 q / 4 kv heads x 256)


def _say(*a):
    print(*a, flush=True)


def _t(a, dev):
    import torch
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16).copy()).to(dev)
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev)


def _h(t):
    import torch
    torch.cuda.synchronize()
    a = t.cpu().numpy()
    return a.view(np.uint16) if a.dtype == np.int16 else a


def _case(synth, n_q, pos0, n_head, n_kv, hd, seed, qscale=2.0):
    r = synth.Rng(seed)
    n = pos0 + n_q
    q = r.normal(n_q * n_head * hd).reshape(n_q, n_head, hd) * np.float32(qscale)
    kc = r.normal(n * n_kv * hd).reshape(n, n_kv * hd)
    vc = r.normal(n * n_kv * hd).reshape(n, n_kv * hd)
    return q.astype(np.float32), kc, vc


def _run(bh, dev, q, pos0, kc, vc, n_kv):
    return _h(bh.attention(_t(q, dev), pos0, _t(kc, dev), _t(vc, dev), n_kv))


@pytest.mark.parametrize("n_q,pos0,f16", [
    (1, 0, False), (1, 6, False), (1, 63, False), (1, 64, False), (1, 999, False),
    (1, 4095, False), (1, 4095, True), (1, 130, True),
    (1, 9000, False), (1, 20000, True),   # one query, chunks of several tiles (ragged last chunk)
    (3, 100, False),     # a few tokens at once (speculative verification)
    (3, 63, False),      # query 0 sees no position of the last chunk (merged as empty)
    (5, 4093, False),    # several queries over several merge groups
    (17, 0, False),      # a causal batch from the first position
    (64, 2000, True),
])
def test_attention_model_heads(bh, oracle, synth, dev, n_q, pos0, f16):
    n_head, n_kv, hd = MODEL
    _say("attention", n_q, pos0, "f16" if f16 else "f32")
    q, kc, vc = _case(synth, n_q, pos0, n_head, n_kv, hd, 300 + n_q + pos0)
    if f16:
        kc = kc.astype(np.float16).view(np.uint16)
        vc = vc.astype(np.float16).view(np.uint16)
    ref = oracle.attention(q, pos0, kc, vc, n_kv)
    got = _run(bh, dev, q, pos0, kc, vc, n_kv)
    err = rel_err(got, ref)
    _say("  rel", err)
    assert err <= TOL


@pytest.mark.parametrize("n_head,n_kv,hd,n_q,pos0", [
    (8, 2, 256, 2, 50),    # grouping 4
    (8, 8, 256, 1, 300),   # grouping 1
    (16, 2, 256, 1, 70),   # grouping 8
    (6, 2, 64, 3, 40),     # other head size: generic path
    (5, 1, 80, 2, 9),      # grouping 5, hd 80: generic path
    (12, 4, 256, 1, 33),   # grouping 3
    (8, 2, 256, 1, 40000), # one query, long context: 3-tile chunks
])
def test_attention_other_shapes(bh, oracle, synth, dev, n_head, n_kv, hd, n_q, pos0):
    _say("attention shape", n_head, n_kv, hd, n_q, pos0)
    q, kc, vc = _case(synth, n_q, pos0, n_head, n_kv, hd, 400 + hd + pos0)
    ref = oracle.attention(q, pos0, kc, vc, n_kv)
    assert rel_err(_run(bh, dev, q, pos0, kc, vc, n_kv), ref) <= TOL


def test_attention_unaligned_q_uses_generic(bh, oracle, synth, dev):
    import torch
    n_head, n_kv, hd = MODEL
    q, kc, vc = _case(synth, 1, 20, n_head, n_kv, hd, 500)
    buf = torch.zeros(q.size + 1, dtype=torch.float32, device=dev)
    buf[1:] = _t(q.reshape(-1), dev)
    got = _h(bh.attention(buf[1:].view(q.shape), 20, _t(kc, dev), _t(vc, dev), n_kv))
    assert rel_err(got, oracle.attention(q, 20, kc, vc, n_kv)) <= TOL


def test_attention_generic_skips_zero_probabilities(bh, oracle, synth, dev):
    """The generic path keeps src/forward.rs:363-366: a position whose
    probability is exactly 0 is skipped, so an inf in its v row does not
    reach the output."""
    q, kc, vc = _case(synth, 1, 1, 1, 1, 4, 501)
    q[0, 0] = [100.0, 0.0, 0.0, 0.0]
    kc[0] = [-100.0, 0.0, 0.0, 0.0]
    kc[1] = [100.0, 0.0, 0.0, 0.0]
    vc[0] = np.inf
    ref = oracle.attention(q, 1, kc, vc, 1)
    got = _run(bh, dev, q, 1, kc, vc, 1)
    assert np.array_equal(got, ref)


def test_kv_store_bits(bh, oracle, synth, dev):
    """f32 rows copied exactly; f16 rows = gguf::f32_to_half, including NaN,
    inf, overflow, ties and the subnormal range, at an offset position."""
    import torch
    r = synth.Rng(502)
    n_tok, elems, cap, pos0 = 3, 1024, 8, 4
    k = r.normal(n_tok * elems).reshape(n_tok, elems) * np.float32(3.0)
    v = r.normal(n_tok * elems).reshape(n_tok, elems)
    special = np.array([np.nan, np.inf, -np.inf, 65504.0, 65520.0, 1e6, -0.0, 1e-8, 6e-8,
                        3e-8, 2.98e-8, 5.96e-8, 1e-5, -6.1e-5, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11,
                        0.1, 1e-40], dtype=np.float32)
    k[0, :special.size] = special
    v[1, :special.size] = special[::-1]
    for f16 in (False, True):
        dt = np.uint16 if f16 else np.float32
        kc0 = np.zeros((cap, elems), dt)
        vc0 = np.zeros((cap, elems), dt)
        want_k, want_v = oracle.kv_store(k, v, kc0, vc0, pos0)
        dk, dv = _t(kc0, dev), _t(vc0, dev)
        bh.kv_store(_t(k, dev), _t(v, dev), dk, dv, pos0)
        gk, gv = _h(dk), _h(dv)
        assert np.array_equal(gk.view(np.uint32 if not f16 else np.uint16),
                              want_k.view(np.uint32 if not f16 else np.uint16))
        assert np.array_equal(gv.view(np.uint32 if not f16 else np.uint16),
                              want_v.view(np.uint32 if not f16 else np.uint16))


def test_store_then_attend_token_loop(bh, oracle, synth, dev):
    """The reference's decode loop: per token, append k/v at pos then attend
    with n_q = 1; the same caches and outputs as one 6-token batch call."""
    import torch
    n_head, n_kv, hd = MODEL
    n_tok = 6
    r = synth.Rng(503)
    q = r.normal(n_tok * n_head * hd).reshape(n_tok, n_head, hd)
    k = r.normal(n_tok * n_kv * hd).reshape(n_tok, n_kv * hd)
    v = r.normal(n_tok * n_kv * hd).reshape(n_tok, n_kv * hd)
    dk = torch.zeros((n_tok, n_kv * hd), device=dev)
    dv = torch.zeros_like(dk)
    outs = []
    for t in range(n_tok):
        bh.kv_store(_t(k[t:t + 1], dev), _t(v[t:t + 1], dev), dk, dv, t)
        outs.append(_h(bh.attention(_t(q[t:t + 1], dev), t, dk, dv, n_kv)))
    ref = oracle.attention(q, 0, k, v, n_kv)
    assert rel_err(np.concatenate(outs), ref) <= TOL
    batch = _h(bh.attention(_t(q, dev), 0, dk, dv, n_kv))
    assert rel_err(batch, ref) <= TOL


@pytest.mark.parametrize("n_q,pos0,f16,n_head,n_kv,vscale,qscale", [
    (64, 4032, False, 24, 4, 1.0, 2.0),    # the bench's prefill case
    (64, 4032, True, 24, 4, 1.0, 2.0),
    (50, 17, False, 24, 4, 1.0, 2.0),      # ragged row tiles and position tiles
    (9, 300, False, 16, 2, 1.0, 2.0),      # grouping 8
    (40, 100, False, 8, 8, 1.0, 2.0),      # grouping 1
    (16, 500, False, 24, 4, 3e6, 1e-3),    # large v (scaled-down tiles), small q
    (16, 500, False, 24, 4, 1e-6, 10.0),   # tiny v, peaked attention (logits ~ N(0, 10^2))
    (33, 2000, True, 12, 4, 1.0, 0.05),    # f16 cache, near-flat attention
    # 8+ row tiles per kv head: the f32 cache is split into f16 hi / lo once
    (200, 37, False, 24, 4, 1.0, 2.0),     # ragged row and position tiles
    (176, 500, False, 24, 4, 3e6, 1e-3),   # large v, small q
    (176, 500, False, 24, 4, 1e-6, 10.0),  # tiny v, peaked attention
])
def test_attention_multi_query_matrix_cores(bh, oracle, synth, dev, n_q, pos0, f16, n_head, n_kv,
                                            vscale, qscale):
    """Many queries per kv head take the matrix-core path (f16 hi/lo
    products with power-of-two scaling); <= 1e-5 against the oracle's
    per-token loop, on magnitudes that stress the splits."""
    hd = 256
    _say("attention mq", n_q, pos0, "f16" if f16 else "f32", n_head, n_kv, vscale, qscale)
    q, kc, vc = _case(synth, n_q, pos0, n_head, n_kv, hd, 700 + n_q + pos0, qscale=qscale)
    vc = (vc * np.float32(vscale)).astype(np.float32)
    if f16:
        kc = kc.astype(np.float16).view(np.uint16)
        vc = vc.astype(np.float16).view(np.uint16)
    ref = oracle.attention(q, pos0, kc, vc, n_kv)
    got = _run(bh, dev, q, pos0, kc, vc, n_kv)
    err = rel_err(got, ref)
    _say("  rel", err)
    assert err <= TOL


@pytest.mark.parametrize("f16", [False, True])
def test_attention_prefill_2048_from_position_0(bh, oracle, synth, dev, f16):
    """The prefill shape behind config 4b's scores: 2048 causal queries from
    position 0 on the model's heads (src/forward.rs:273-375 run for a whole
    window, as GDev::prefill_batch does).  The whole batch runs in one call;
    sampled query rows (the first, chunk and tile edges, the last) are
    checked against the oracle's per-token loop at their own positions, and
    query 0 -- which sees position 0 alone, so its softmax is exactly 1 --
    must return v_0 of its kv head (to the f16 hi + lo products' 2^-21)."""
    n_head, n_kv, hd = MODEL
    n = 2048
    _say("attention prefill 2048", "f16" if f16 else "f32")
    q, kc, vc = _case(synth, n, 0, n_head, n_kv, hd, 911 + int(f16))
    if f16:
        kc = kc.astype(np.float16).view(np.uint16)
        vc = vc.astype(np.float16).view(np.uint16)
    got = _run(bh, dev, q, 0, kc, vc, n_kv)
    assert np.all(np.isfinite(got))
    v0 = (vc[0].view(np.float16).astype(np.float32) if f16 else vc[0]).reshape(n_kv, hd)
    grp = n_head // n_kv
    for h in range(n_head):
        assert rel_err(got[0, h], v0[h // grp]) <= 1e-6
    worst = 0.0
    for i in (1, 2, 63, 64, 127, 511, 1000, 1023, 1024, 1535, 2046, 2047):
        ref = oracle.attention(q[i:i + 1], i, kc[:i + 1], vc[:i + 1], n_kv)
        worst = max(worst, rel_err(got[i:i + 1], ref))
    _say("  rel (sampled rows)", worst)
    assert worst <= TOL


def test_attention_presplit_tile_scales(bh, oracle, synth, dev):
    """The pre-split f32 path (8+ row tiles per kv head) with V tiles whose
    magnitudes differ by up to 2^48 along the positions: each 32-position
    tile keeps its own power-of-two unit, and a block whose running unit
    has grown scales the tile's probabilities down instead.  <= 1e-5
    against the oracle's per-token loop."""
    n_head, n_kv, hd = MODEL
    n_q, pos0 = 192, 300
    q, kc, vc = _case(synth, n_q, pos0, n_head, n_kv, hd, 977)
    n = pos0 + n_q
    expo = np.round(24.0 * np.sin(np.arange(n) / 37.0)).astype(np.float32)
    vc = (vc * np.exp2(expo)[:, None]).astype(np.float32)
    ref = oracle.attention(q, pos0, kc, vc, n_kv)
    got = _run(bh, dev, q, pos0, kc, vc, n_kv)
    err = rel_err(got, ref)
    _say("  rel", err)
    assert err <= TOL
