"""Golden fixtures (tests/golden/golden_small.npz, written by
tests/golden/make_golden.py from the CPU oracle on seeded inputs).

CPU: the oracle still reproduces every stored output bit for bit (a change of
the restatement, its build flags or the libm it links shows up here).
GPU: every entry point of the path against the stored outputs -- the PQ2_0
gather and the gather + RMSNorm bit-exact, float kernels within the
reference's per-tensor metric (<= 1e-5; softmax <= 2e-5).
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from conftest import rel_err

GOLDEN = Path(__file__).resolve().parent / "golden" / "golden_small.npz"
TOL = 1e-5
TOL_SOFTMAX = 2e-5
SECTIONS = (11, 11, 10, 0)
EPS = 1e-6


@pytest.fixture(scope="module")
def gold():
    with np.load(GOLDEN, allow_pickle=False) as z:
        d = {k: z[k] for k in z.files}
    out = {}
    for key, v in d.items():
        case, name = key.split("/")
        out.setdefault(case, {})[name] = v
    return out


def _same(a, b):
    a, b = np.asarray(a), np.asarray(b)
    return a.shape == b.shape and np.array_equal(a.view(np.uint8), b.view(np.uint8))


# ---------------------------------------------------------------------------
# CPU: the oracle reproduces the fixtures
# ---------------------------------------------------------------------------

def test_fixture_covers_every_path_function(gold):
    assert set(gold) == {"rms_rows", "add_rms_rows", "l2_rows", "unary", "gdn_gate_prep",
                         "rope_imrope", "qk_norm_rope", "softmax", "pq2_gather", "conv1d",
                         "gdn_step", "attention", "pq2_matmul"}


def test_oracle_reproduces_golden(gold, oracle):
    g = gold["rms_rows"]
    assert _same(oracle.rms_norm_rows(g["x"], g["w"], 5120, EPS).reshape(g["y"].shape), g["y"])
    g = gold["add_rms_rows"]
    s, y = oracle.add_rms_norm_rows(g["x"], g["r"], g["w"], 1024, EPS)
    assert _same(s.reshape(g["sum"].shape), g["sum"]) and _same(y.reshape(g["y"].shape), g["y"])
    g = gold["l2_rows"]
    assert _same(oracle.l2_norm_rows(g["x"], 128, EPS).reshape(g["y"].shape), g["y"])
    assert _same(oracle.silu_l2_part(g["x"], 512, 128, EPS), g["y_silu"])
    g = gold["unary"]
    for m in range(5):
        assert _same(oracle.unary(m, g["a"], g["b"]), g[f"mode{m}"])
    g = gold["gdn_gate_prep"]
    gate, beta = oracle.gdn_gate_prep(g["alpha"], g["bias"], g["ssm_a"], g["beta_raw"])
    assert _same(gate, g["gate"]) and _same(beta, g["beta"])
    g = gold["rope_imrope"]
    for t in range(g["heads"].shape[0]):
        for h in range(g["heads"].shape[1]):
            assert _same(oracle.rope_imrope(g["heads"][t, h], *g["pos"][t], 64, SECTIONS, 1e7),
                         g["y"][t, h])
    g = gold["qk_norm_rope"]
    qo, ko, _ = oracle.qk_norm_rope(g["q"], g["k"], g["wq"], g["wk"], g["pos"], 24, 4, 256, 64,
                                    SECTIONS, 1e7, EPS)
    assert _same(qo, g["q_out"]) and _same(ko, g["k_out"])
    g = gold["softmax"]
    assert _same(oracle.softmax_rows(g["x"], 2048).reshape(g["y"].shape), g["y"])
    assert _same(oracle.softmax_rows(g["xw"], g["xw"].size, float(g["inv_temp"][0])), g["yw"])
    g = gold["pq2_gather"]
    e, en = oracle.embed_gather(g["table"], 5120, g["table"].shape[0], g["ids"], g["w"], EPS)
    assert _same(e, g["y"]) and _same(en, g["y_norm"])
    g = gold["conv1d"]
    y, st = oracle.conv1d_silu(g["x"], g["state"], g["w"])
    assert _same(y, g["y"]) and _same(st, g["state_out"])
    g = gold["gdn_step"]
    a, st = oracle.gdn_step(g["q"], g["k"], g["v"], g["gate"], g["beta"], g["state"])
    assert _same(a, g["attn"]) and _same(st, g["state_out"])
    g = gold["attention"]
    assert _same(oracle.attention(g["q"], 5, g["k_cache"], g["v_cache"], 2), g["y"])
    g = gold["pq2_matmul"]
    rows = g["y"].shape[1]
    assert _same(oracle.pq2_matmul_n(g["payload"], 1024, rows, g["x"]), g["y"])
    assert _same(oracle.pq2_matmul_n(g["payload"], 1024, rows, g["x"][0]), g["y1"])


def test_golden_reference_known_answers(gold):
    """Facts of the stored outputs that the reference's own tests assert
    (src/kernels.rs:840-853: masked entries are 0, rows sum to 1;
    src/rope.rs:96-114: position 0 is the identity)."""
    g = gold["softmax"]
    assert np.all(g["y"][np.isneginf(g["x"])] == 0.0)
    assert np.allclose(g["y"].astype(np.float64).sum(axis=1), 1.0, atol=1e-5)
    assert abs(float(g["yw"].astype(np.float64).sum()) - 1.0) < 1e-5
    r = gold["rope_imrope"]
    assert _same(r["y"][0], r["heads"][0])
    assert _same(r["y"][:, :, 64:], r["heads"][:, :, 64:])


# ---------------------------------------------------------------------------
# GPU: the HIP library against the fixtures
# ---------------------------------------------------------------------------

def _t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _h(t):
    return t.detach().cpu().numpy()


@pytest.mark.gpu
def test_golden_norms_and_gates(bh, gold, dev):
    g = gold["rms_rows"]
    assert rel_err(_h(bh.rms_norm_rows(_t(g["x"], dev), _t(g["w"], dev), EPS)), g["y"]) <= TOL
    g = gold["add_rms_rows"]
    s, y = bh.add_rms_norm_rows(_t(g["x"], dev), _t(g["r"], dev), _t(g["w"], dev), EPS)
    assert _same(_h(s), g["sum"]) and rel_err(_h(y), g["y"]) <= TOL
    g = gold["l2_rows"]
    x = _t(g["x"], dev)
    assert rel_err(_h(bh.l2_norm_rows(x, 128, EPS)), g["y"]) <= TOL
    assert rel_err(_h(bh.l2_norm_rows(x, 128, EPS, silu_first=True)), g["y_silu"]) <= TOL
    g = gold["unary"]
    a, b = _t(g["a"], dev), _t(g["b"], dev)
    for m in range(5):
        assert rel_err(_h(bh.unary(m, a, b)), g[f"mode{m}"]) <= TOL, m
    g = gold["gdn_gate_prep"]
    gate, beta = bh.gdn_gate_prep(_t(g["alpha"], dev), _t(g["bias"], dev), _t(g["ssm_a"], dev),
                                  _t(g["beta_raw"], dev))
    assert rel_err(_h(gate), g["gate"]) <= TOL and rel_err(_h(beta), g["beta"]) <= TOL


@pytest.mark.gpu
def test_golden_rope_and_qk(bh, gold, dev):
    import torch
    g = gold["rope_imrope"]
    h = _t(g["heads"], dev)
    bh.rope_imrope(h, _t(g["pos"], dev), 64, SECTIONS, 1e7)
    assert rel_err(_h(h), g["y"]) <= TOL
    g = gold["qk_norm_rope"]
    n_tok = g["pos"].shape[0]
    q, k = _t(g["q"], dev), _t(g["k"], dev)
    qo, ko = torch.empty_like(q), torch.empty_like(k)
    wq, wk, pos = _t(g["wq"], dev), _t(g["wk"], dev), _t(g["pos"], dev)
    bh.qk_norm_rope(bh.make_qk_args(q, qo, k, ko, wq, wk, pos, n_tok, 24, 4))
    assert rel_err(_h(qo), g["q_out"]) <= TOL and rel_err(_h(ko), g["k_out"]) <= TOL
    qg = _t(g["qg"], dev)
    n4 = g["qg"].shape[0]
    qgo = torch.empty((n4, 24, 256), device=dev)
    go = torch.empty_like(qgo)
    kgo = torch.empty((n4, 4, 256), device=dev)
    bh.qk_norm_rope(bh.make_qk_args(qg, qgo, k[:n4].contiguous(), kgo, wq, wk,
                                    pos[:n4].contiguous(), n4, 24, 4, q_head_stride=512,
                                    gate_out=go))
    assert rel_err(_h(qgo), g["qg_out"]) <= TOL and rel_err(_h(kgo), g["kg_out"]) <= TOL
    assert rel_err(_h(go), g["gate"]) <= TOL


@pytest.mark.gpu
def test_golden_softmax(bh, gold, dev):
    g = gold["softmax"]
    assert rel_err(_h(bh.softmax_rows(_t(g["x"], dev), 2048)), g["y"]) <= TOL_SOFTMAX
    got = bh.softmax_rows(_t(g["xw"], dev), g["xw"].size, float(g["inv_temp"][0]))
    assert rel_err(_h(got), g["yw"]) <= TOL_SOFTMAX


@pytest.mark.gpu
def test_golden_pq2_gather_bit_exact(bh, gold, dev):
    g = gold["pq2_gather"]
    table, ids = _t(g["table"], dev), _t(g["ids"], dev)
    n_rows = g["table"].shape[0]
    assert _same(_h(bh.pq2_embed_gather(table, 5120, n_rows, ids)), g["y"])
    e, en = bh.pq2_embed_gather(table, 5120, n_rows, ids, w=_t(g["w"], dev), eps=EPS)
    assert _same(_h(e), g["y"]) and _same(_h(en), g["y_norm"])


@pytest.mark.gpu
def test_golden_next_rows(bh, gold, dev):
    g = gold["conv1d"]
    st = _t(g["state"], dev)
    y = bh.conv1d_silu(_t(g["x"], dev), st, _t(g["w"], dev))
    assert rel_err(_h(y), g["y"]) <= TOL and _same(_h(st), g["state_out"])
    g = gold["gdn_step"]
    st = _t(g["state"], dev)
    a = bh.gdn_step(*(_t(g[n], dev) for n in ("q", "k", "v", "gate", "beta")), st)
    assert rel_err(_h(a), g["attn"]) <= TOL and rel_err(_h(st), g["state_out"]) <= TOL
    g = gold["attention"]
    y = bh.attention(_t(g["q"], dev), 5, _t(g["k_cache"], dev), _t(g["v_cache"], dev), 2)
    assert rel_err(_h(y), g["y"]) <= TOL
    g = gold["pq2_matmul"]
    pay, x = _t(g["payload"], dev), _t(g["x"], dev)
    rows = g["y"].shape[1]
    assert rel_err(_h(bh.pq2_matmul_n(pay, 1024, rows, x)), g["y"]) <= TOL
    assert rel_err(_h(bh.pq2_matmul_n(pay, 1024, rows, x[0].contiguous())), g["y1"]) <= TOL
