"""Writes tests/golden/golden_small.npz: seeded small inputs of every function
on the path and the CPU oracle's outputs for them (oracle/oracle.c, the
restatement of src/kernels.rs, src/rope.rs, src/gdn.rs and the composition
sites of src/forward.rs).

Run from the repository root after building the oracle:

    python tests/golden/make_golden.py

Inputs come from the SplitMix64 + Box-Muller generator of
ternary-bonsai-inference_amd/synth.py (the algorithm of src/sampler.rs:15-21),
so the file is reproducible bit for bit.  The fixture is data only (float32 /
int32 / uint8 / uint16 arrays, loaded with allow_pickle=False).  The tests
compare the HIP library against these outputs and check that the oracle
still reproduces them.
"""
from __future__ import annotations

import importlib.util
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REPO = HERE.parent.parent
OUT = HERE / "golden_small.npz"

SECTIONS = (11, 11, 10, 0)
EPS = 1e-6


def _load(name, path):
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def cases(oracle, synth) -> dict[str, np.ndarray]:
    """Every fixture array, keyed '<case>/<name>'.  Inputs first, outputs last."""
    R = synth.Rng
    f = {}

    def put(case, **arrs):
        for k, v in arrs.items():
            f[f"{case}/{k}"] = np.ascontiguousarray(v)

    # a1/a2 RMSNorm rows (config 1 row length)
    x = R(100).normal(4 * 5120).reshape(4, 5120)
    w = R(101).normal(5120, 1.0, 0.1)
    put("rms_rows", x=x, w=w, y=oracle.rms_norm_rows(x, w, 5120, EPS).reshape(4, 5120))
    # a2' residual add + norm
    x = R(102).normal(3 * 1024).reshape(3, 1024)
    r = R(103).normal(3 * 1024).reshape(3, 1024)
    w = R(104).normal(1024, 1.0, 0.1)
    s, y = oracle.add_rms_norm_rows(x, r, w, 1024, EPS)
    put("add_rms_rows", x=x, r=r, w=w, sum=s.reshape(3, 1024), y=y.reshape(3, 1024))
    # a3 L2 rows over 128-float heads, and SiLU first
    x = R(105).normal(5 * 512).reshape(5, 512)
    put("l2_rows", x=x, y=oracle.l2_norm_rows(x, 128, EPS).reshape(5, 512),
        y_silu=oracle.silu_l2_part(x, 512, 128, EPS))
    # a4 element-wise modes 0..4
    a = R(106).normal(777, 0.0, 4.0)
    b = R(107).normal(777)
    put("unary", a=a, b=b, **{f"mode{m}": oracle.unary(m, a, b) for m in range(5)})
    # a5 GDN gate prep
    alpha = R(108).normal(16 * 48).reshape(16, 48)
    bias = R(109).normal(48, 0.0, 0.5)
    ssm_a = -np.exp(R(110).uniform(48) * 2.0).astype(np.float32)
    beta_raw = R(111).normal(16 * 48).reshape(16, 48)
    gate, beta = oracle.gdn_gate_prep(alpha, bias, ssm_a, beta_raw)
    put("gdn_gate_prep", alpha=alpha, bias=bias, ssm_a=ssm_a, beta_raw=beta_raw, gate=gate,
        beta=beta)
    # a6 IMROPE on a few heads at mixed positions (sections [11,11,10,0])
    heads = R(112).normal(3 * 4 * 256).reshape(3, 4, 256)
    pos = np.array([[0, 0, 0, 0], [37, 5, 900, 2], [2047, 2047, 2047, 2047]], np.int32)
    rot = np.stack([np.stack([oracle.rope_imrope(heads[t, h], *pos[t], 64, SECTIONS, 1e7)
                              for h in range(4)]) for t in range(3)])
    put("rope_imrope", heads=heads, pos=pos, y=rot)
    # a6' attention pre-block: q/k RMSNorm + IMROPE, and the [q | gate] split
    n_tok = 8
    q = R(113).normal(n_tok * 24 * 256).reshape(n_tok, 24, 256)
    k = R(114).normal(n_tok * 4 * 256).reshape(n_tok, 4, 256)
    wq = R(115).normal(256, 1.0, 0.1)
    wk = R(116).normal(256, 1.0, 0.1)
    pos = np.repeat(np.arange(1000, 1000 + n_tok, dtype=np.int32)[:, None], 4, axis=1).copy()
    qo, ko, _ = oracle.qk_norm_rope(q, k, wq, wk, pos, 24, 4, 256, 64, SECTIONS, 1e7, EPS)
    qg = R(117).normal(4 * 24 * 512).reshape(4, 24, 512)
    qgo, kgo, go = oracle.qk_norm_rope(qg, k[:4], wq, wk, pos[:4], 24, 4, 256, 64, SECTIONS,
                                       1e7, EPS, q_head_stride=512, want_gate=True)
    put("qk_norm_rope", q=q, k=k, wq=wq, wk=wk, pos=pos, q_out=qo, k_out=ko, qg=qg,
        qg_out=qgo, kg_out=kgo, gate=go)
    # a7 softmax: masked attention rows, temperature, one wide row (split path)
    x = R(118).normal(6 * 2048, 0.0, 2.0).reshape(6, 2048)
    x[np.triu_indices(6, 1)[0], np.triu_indices(6, 1)[1] + 2042] = -np.inf
    xw = R(119).normal(20000, 0.0, 3.0)
    xw[::97] += 10.0
    inv_t = np.float32(1.0) / np.float32(0.7)
    put("softmax", x=x, y=oracle.softmax_rows(x, 2048).reshape(6, 2048), xw=xw,
        inv_temp=np.array([inv_t], np.float32), yw=oracle.softmax_rows(xw, 20000, inv_t))
    # a8/a9 PQ2_0 gather and gather + first RMSNorm (code 3 included)
    rng = R(120)
    table = synth.pq2_table(rng, 64, 5120)
    table[5, 2:34] = 0xFF       # a block of code 3 (+2 * scale)
    ids = np.array([0, 63, 5, 17, 17, 2, 40, 63, 1, 33], np.uint32)
    wn = R(121).normal(5120, 1.0, 0.1)
    emb, emb_norm = oracle.embed_gather(table, 5120, 64, ids, wn, EPS)
    put("pq2_gather", table=table, ids=ids, w=wn, y=emb, y_norm=emb_norm)
    # f2 causal conv1d + SiLU over a token batch
    xc = R(122).normal(9 * 256).reshape(9, 256)
    stc = R(123).normal(256 * 3).reshape(256, 3)
    wc = R(124).normal(256 * 4, 0.0, 0.5).reshape(256, 4)
    yc, st2 = oracle.conv1d_silu(xc, stc, wc)
    put("conv1d", x=xc, state=stc, w=wc, y=yc, state_out=st2)
    # f3 gated delta-net recurrence, 3 tokens, 1 k-head, 2 v-heads of 128
    from gdndata import gdn_case  # noqa: E402  (tests/ on sys.path)
    g = gdn_case(synth, 3, 1, 2, 128, 125)
    attn, st3 = oracle.gdn_step(*g)
    put("gdn_step", q=g[0], k=g[1], v=g[2], gate=g[3], beta=g[4], state=g[5], attn=attn,
        state_out=st3)
    # f4 attention over an f32 KV cache: 3 queries at positions 5..7
    n_head, n_kv, hd = 4, 2, 256
    qa = R(126).normal(3 * n_head * hd).reshape(3, n_head, hd)
    kc = R(127).normal(8 * n_kv * hd).reshape(8, n_kv * hd)
    vc = R(128).normal(8 * n_kv * hd).reshape(8, n_kv * hd)
    put("attention", q=qa, k_cache=kc, v_cache=vc, y=oracle.attention(qa, 5, kc, vc, n_kv))
    # f1 PQ2_0 products: 40 rows of 1024, three tokens (and one token = matvec)
    pay = synth.pq2_table(R(129), 40, 1024)
    xm = R(130).normal(3 * 1024).reshape(3, 1024)
    put("pq2_matmul", payload=pay, x=xm, y=oracle.pq2_matmul_n(pay, 1024, 40, xm),
        y1=oracle.pq2_matmul_n(pay, 1024, 40, xm[0]))
    return f


def main():
    sys.path.insert(0, str(REPO / "tests"))
    oracle = _load("bonsai_oracle", REPO / "oracle" / "oracle.py")
    synth = _load("bonsai_amd_synth", REPO / "ternary-bonsai-inference_amd" / "synth.py")
    f = cases(oracle, synth)
    np.savez_compressed(OUT, **f)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(f)} arrays)")


if __name__ == "__main__":
    main()
