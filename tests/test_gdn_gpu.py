"""GPU parity of the gated delta-net recurrence (bh_gdn_step) against the
oracle's restatement of src/gdn.rs:17-77 applied token by token.

Bar: max|gpu-ref| / max(|ref|, |gpu|) <= 1e-5 for attn and for the advanced
state.  The device sums each 128-long dot as 8 in-lane products and a fixed
16-lane tree where the reference adds in index order, and batches of 128 or
more tokens take the recurrence's closed form per 64-token chunk (a
triangular solve and matrix products), so the two differ by rounding only.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import rel_err
from gdndata import gdn_case

pytestmark = pytest.mark.gpu

TOL = 1e-5


def _say(*a):
    print(*a, flush=True)


def _t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev)


def _h(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def _run(bh, dev, case):
    q, k, v, gate, beta, st = case
    dst = _t(st, dev)
    attn = _h(bh.gdn_step(_t(q, dev), _t(k, dev), _t(v, dev), _t(gate, dev), _t(beta, dev), dst))
    return attn, _h(dst)


@pytest.mark.parametrize("n_tok,h_k,h_v,s", [
    (1, 16, 48, 128),     # the reference's decode step
    (7, 16, 48, 128),
    (256, 16, 48, 128),   # a prefill chunk through one launch
    (3, 2, 4, 128),       # fewer heads
    (5, 2, 6, 32),        # other head sizes: one lane per row
    (4, 3, 3, 40),
])
def test_gdn_step(bh, oracle, synth, dev, n_tok, h_k, h_v, s):
    _say("gdn_step", n_tok, h_k, h_v, s)
    case = gdn_case(synth, n_tok, h_k, h_v, s, 90 + n_tok + s)
    ref_attn, ref_st = oracle.gdn_step(*case)
    attn, st = _run(bh, dev, case)
    errs = rel_err(attn, ref_attn), rel_err(st, ref_st)
    _say("  rel", errs)
    assert max(errs) <= TOL


def test_gdn_step_unaligned_falls_back(bh, oracle, synth, dev):
    """s = 128 with q, k and the state not 32-byte aligned: the row-per-lane
    kernel gives the same results."""
    import torch
    n_tok, h_k, h_v, s = 2, 2, 4, 128
    q, k, v, gate, beta, st = gdn_case(synth, n_tok, h_k, h_v, s, 91)
    ref_attn, ref_st = oracle.gdn_step(q, k, v, gate, beta, st)

    def shifted(a):
        buf = torch.zeros(a.size + 1, dtype=torch.float32, device=dev)
        buf[1:] = _t(a.reshape(-1), dev)
        return buf[1:].view(a.shape)

    dq, dk, dst = shifted(q), shifted(k), shifted(st)
    attn = _h(bh.gdn_step(dq, dk, _t(v, dev), _t(gate, dev), _t(beta, dev), dst))
    assert max(rel_err(attn, ref_attn), rel_err(_h(dst), ref_st)) <= TOL


def test_gdn_step_chunks_equal_one_batch(bh, oracle, synth, dev):
    """Tokens in chunks with the state carried on the device = one batch."""
    n_tok, h_k, h_v, s = 9, 16, 48, 128
    q, k, v, gate, beta, st = gdn_case(synth, n_tok, h_k, h_v, s, 92)
    ref_attn, ref_st = oracle.gdn_step(q, k, v, gate, beta, st)
    dst = _t(st, dev)
    outs = []
    for lo, hi in ((0, 1), (1, 4), (4, 9)):
        sl = slice(lo, hi)
        outs.append(_h(bh.gdn_step(_t(q[sl], dev), _t(k[sl], dev), _t(v[sl], dev),
                                   _t(gate[sl], dev), _t(beta[sl], dev), dst)))
    assert rel_err(np.concatenate(outs), ref_attn) <= TOL
    assert rel_err(_h(dst), ref_st) <= TOL


def test_gdn_step_pure_decay_long_run(bh, synth, dev):
    """Size-independent property at a long run: beta = 0 leaves only the
    decay, so after T tokens M = M0 * prod_t expf(gate[t][h]) and the last
    attn row is that M times q / sqrt(s) (float64 check)."""
    n_tok, h_k, h_v, s = 1024, 16, 48, 128
    q, k, v, gate, beta, st = gdn_case(synth, n_tok, h_k, h_v, s, 93)
    gate = gate * np.float32(0.01)
    attn, got_st = _run(bh, dev, (q, k, v, gate, np.zeros_like(beta), st))
    f = np.ones(h_v)
    for t in range(n_tok):
        f *= np.exp(gate[t].astype(np.float32)).astype(np.float32).astype(np.float64)
    want_st = st.astype(np.float64) * f[:, None, None]
    assert rel_err(got_st, want_st) <= 1e-4  # 1024 f32 roundings of the product
    want = np.einsum("hji,hi->hj", want_st, q[-1][np.arange(h_v) % h_k].astype(np.float64))
    assert rel_err(attn[-1], want / np.sqrt(s)) <= 1e-4


def test_gdn_step_graph_replay_advances_state(bh, oracle, synth, dev):
    """Captured in a HIP graph, each replay advances the state like an eager
    call."""
    import torch
    n_tok, h_k, h_v, s = 3, 16, 48, 128
    q, k, v, gate, beta, st = gdn_case(synth, n_tok, h_k, h_v, s, 94)
    d = [_t(a, dev) for a in (q, k, v, gate, beta)]
    dst = _t(st, dev)
    attn = torch.empty_like(d[2])
    strm = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=strm):
        bh.gdn_step(*d, dst, attn=attn, stream=strm)
    torch.cuda.synchronize()
    dst.copy_(_t(st, dev))
    cur = st
    for rep in range(3):
        torch.cuda.synchronize()
        with torch.cuda.stream(strm):
            g.replay()
        torch.cuda.synchronize()
        ref_attn, cur = oracle.gdn_step(q, k, v, gate, beta, cur)
        assert rel_err(attn.cpu().numpy(), ref_attn) <= TOL, rep
        assert rel_err(dst.cpu().numpy(), cur) <= TOL, rep



@pytest.mark.parametrize("n_tok,h_k,h_v", [
    (128, 16, 48),   # the shortest batch of the chunked (matrix-core) path: 2 chunks
    (129, 16, 48),   # two chunks and one token
    (200, 16, 48),   # a ragged last chunk
    (2048, 16, 48),  # the prefill length of the metric: 32 chunks
    (130, 2, 6),     # q/k heads not a multiple of 8 (no XCD placement)
    (150, 3, 4),     # v-heads not a multiple of the q/k heads
])
def test_gdn_step_chunked(bh, oracle, synth, dev, n_tok, h_k, h_v):
    _say("gdn_step chunked", n_tok, h_k, h_v)
    case = gdn_case(synth, n_tok, h_k, h_v, 128, 300 + n_tok + h_v)
    ref_attn, ref_st = oracle.gdn_step(*case)
    attn, st = _run(bh, dev, case)
    errs = rel_err(attn, ref_attn), rel_err(st, ref_st)
    _say("  rel", errs)
    assert max(errs) <= TOL


def test_gdn_step_chunked_hard_inputs(bh, oracle, synth, dev):
    """The chunked path where its triangular solve and decays are stressed:
    keys of a head nearly identical, betas near 1, no decay on some heads, a
    -inf gate (the state is cleared) and gates whose decay underflows."""
    n_tok, h_k, h_v, s = 160, 16, 48, 128
    q, k, v, gate, beta, st = gdn_case(synth, n_tok, h_k, h_v, s, 96)
    r = synth.Rng(97)
    base = r.normal(h_k * s).reshape(1, h_k, s)
    k = base + np.float32(0.05) * r.normal(n_tok * h_k * s).reshape(n_tok, h_k, s)
    k = (k / np.linalg.norm(k, axis=-1, keepdims=True)).astype(np.float32)
    beta = (np.float32(0.99) + np.float32(0.01) * beta).astype(np.float32)
    gate = gate.copy()
    gate[:, :16] = 0.0
    gate[5, 16:32] = -np.inf
    gate[70:, 32:40] = -150.0
    ref_attn, ref_st = oracle.gdn_step(q, k, v, gate, beta, st)
    attn, got = _run(bh, dev, (q, k, v, gate, beta, st))
    errs = rel_err(attn, ref_attn), rel_err(got, ref_st)
    _say("  rel", errs)
    assert max(errs) <= TOL


def test_gdn_step_chunked_graph_replay(bh, oracle, synth, dev):
    """The chunked path (prepared matrices in library scratch) captured in a
    HIP graph after one eager call: each replay advances the state like an
    eager call."""
    import torch
    n_tok, h_k, h_v, s = 128, 16, 48, 128
    q, k, v, gate, beta, st = gdn_case(synth, n_tok, h_k, h_v, s, 98)
    d = [_t(a, dev) for a in (q, k, v, gate, beta)]
    dst = _t(st, dev)
    attn = torch.empty_like(d[2])
    strm = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(strm):
        bh.gdn_step(*d, dst, attn=attn, stream=strm)  # sizes the scratch outside capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=strm):
        bh.gdn_step(*d, dst, attn=attn, stream=strm)
    torch.cuda.synchronize()
    dst.copy_(_t(st, dev))
    cur = st
    for rep in range(3):
        torch.cuda.synchronize()
        with torch.cuda.stream(strm):
            g.replay()
        torch.cuda.synchronize()
        ref_attn, cur = oracle.gdn_step(q, k, v, gate, beta, cur)
        assert rel_err(attn.cpu().numpy(), ref_attn) <= TOL, rep
        assert rel_err(dst.cpu().numpy(), cur) <= TOL, rep
