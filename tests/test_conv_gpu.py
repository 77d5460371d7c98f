"""GPU parity of the causal conv1d + SiLU (bh_conv1d_silu, and the conv mode of
bh_gdn_prep_fused) against the oracle's per-token restatement of
src/forward.rs:508-533.

Bars: outputs max|gpu-ref|/max(|ref|,|gpu|) <= 1e-5 (the pre-activation is
the same f32 products and sums in the same order; the SiLU's expf is the
device's); the advanced conv cache bit for bit (it only moves inputs).
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import rel_err

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


def _inputs(synth, n_tok, ch, k, seed):
    r = synth.Rng(seed)
    x = r.normal(n_tok * ch).reshape(n_tok, ch)
    st = r.normal(ch * max(k - 1, 0)).reshape(ch, k - 1)
    w = r.normal(ch * k, 0.0, 0.5).reshape(ch, k)
    return x, st, w


@pytest.mark.parametrize("n_tok,ch,k", [
    (1, 10240, 4), (2, 10240, 4), (3, 40, 4),   # fewer tokens than taps: cache reads
    (4096, 10240, 4),                          # a prefill batch over the model's qkv width
    (7, 13, 4),                                # odd width: one lane per output
    (5, 64, 1), (5, 64, 2), (9, 48, 7),        # other tap counts (generic path)
])
def test_conv1d_silu(bh, oracle, synth, dev, n_tok, ch, k):
    _say("conv1d_silu", n_tok, ch, k)
    x, st, w = _inputs(synth, n_tok, ch, k, n_tok + ch + k)
    ref, ref_st = oracle.conv1d_silu(x, st, w)
    dst = _t(st, dev) if k > 1 else None
    got = _h(bh.conv1d_silu(_t(x, dev), dst, _t(w, dev)))
    err = rel_err(got, ref)
    _say("  rel", err)
    assert err <= TOL
    if k > 1:
        assert np.array_equal(_h(dst), ref_st)


def test_conv1d_silu_chunks_equal_one_batch(bh, oracle, synth, dev):
    """Running the tokens in chunks (the cache carried on the device) gives
    the outputs and final cache of one batch, as the per-token reference."""
    import torch
    n_tok, ch, k = 11, 64, 4
    x, st, w = _inputs(synth, n_tok, ch, k, 70)
    ref, ref_st = oracle.conv1d_silu(x, st, w)
    dst, dw = _t(st, dev), _t(w, dev)
    outs = []
    for lo, hi in ((0, 1), (1, 3), (3, 4), (4, 11)):
        outs.append(_h(bh.conv1d_silu(_t(x[lo:hi], dev), dst, dw)))
    assert rel_err(np.concatenate(outs), ref) <= TOL
    assert np.array_equal(_h(dst), ref_st)


def test_conv1d_graph_replay_advances_cache(bh, oracle, synth, dev):
    """Captured in a HIP graph, each replay advances the cache like an eager
    call would (state kernel inside the graph, no memset)."""
    import torch
    n_tok, ch, k = 6, 128, 4
    x, st, w = _inputs(synth, n_tok, ch, k, 71)
    dx, dst, dw = _t(x, dev), _t(st, dev), _t(w, dev)
    out = torch.empty_like(dx)
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        bh.conv1d_silu(dx, dst, dw, out=out, stream=s)
    torch.cuda.synchronize()
    dst.copy_(_t(st, dev))  # capture does not run the kernels: reset anyway
    cache = st
    for rep in range(3):
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            g.replay()
        torch.cuda.synchronize()
        ref, cache = oracle.conv1d_silu(x, cache, w)
        assert rel_err(out.cpu().numpy(), ref) <= TOL, rep
        assert np.array_equal(dst.cpu().numpy(), cache), rep


@pytest.mark.parametrize("shape", [
    (4096, 10240, 4096, 6144, 48),   # model layout: conv over qkv, q,k L2, 48 gates
    (3, 10240, 4096, 6144, 48),      # fewer tokens than taps
    (1, 10240, 4096, 6144, 48),      # one token: the new cache keeps two old entries
    (2, 10240, 4096, 6144, 48),      # two tokens: one old entry
    (3, 100, 60, 10, 5),             # odd widths: looped kernel
])
def test_gdn_prep_fused_with_conv(bh, oracle, synth, dev, shape):
    """bh_gdn_prep_fused in conv mode = conv1d_silu, then the per-head L2 of
    the first l2_dim channels, plus the gates, from the raw qkv."""
    import torch
    n_tok, ch, l2_dim, inner, n_head = shape
    head_dim = 128 if ch % 128 == 0 else 20
    _say("gdn_prep_fused+conv", shape)
    x, st, w = _inputs(synth, n_tok, ch, 4, 72)
    r = synth.Rng(73)
    dt = r.normal(n_tok * n_head).reshape(n_tok, n_head)
    bias = r.normal(n_head, 0.0, 0.5)
    A = (-np.exp(r.uniform(n_head) * 2.0)).astype(np.float32)
    beta = r.normal(n_tok * n_head).reshape(n_tok, n_head)
    z = r.normal(n_tok * inner).reshape(n_tok, inner)
    y = r.normal(n_tok * inner).reshape(n_tok, inner)
    d = {k: _t(v, dev) for k, v in dict(x=x, st=st, w=w, dt=dt, bias=bias, A=A, beta=beta,
                                        z=z, y=y).items()}
    conv_out = torch.empty_like(d["x"])
    gated = torch.empty_like(d["z"])
    gate = torch.empty_like(d["dt"])
    beta_o = torch.empty_like(d["beta"])
    args = bh.make_gdn_args(conv=d["x"], conv_out=conv_out, z=d["z"], y=d["y"],
                            gated_out=gated, alpha_raw=d["dt"], dt_bias=d["bias"],
                            ssm_a=d["A"], beta_raw=d["beta"], gate_out=gate, beta_out=beta_o,
                            n_tok=n_tok, conv_dim=ch, l2_dim=l2_dim, head_dim=head_dim,
                            inner_dim=inner, n_v_head=n_head, gate_mode=3, eps=1e-6,
                            conv_w=d["w"], conv_state=d["st"], conv_k=4)
    bh.gdn_prep_fused(args)
    act, ref_st = oracle.conv1d_silu(x, st, w)
    ref_conv = act.copy()
    ref_conv[:, :l2_dim] = oracle.l2_norm_rows(act[:, :l2_dim], head_dim, 1e-6).reshape(
        n_tok, l2_dim)
    errs = [rel_err(_h(conv_out), ref_conv), rel_err(_h(gated), oracle.unary(3, z, y)),
            rel_err(_h(gate), oracle.gdn_gate_prep(dt, bias, A, beta)[0]),
            rel_err(_h(beta_o), oracle.gdn_gate_prep(dt, bias, A, beta)[1])]
    _say("  rel", errs)
    assert max(errs) <= TOL
    assert np.array_equal(_h(d["st"]), ref_st)
