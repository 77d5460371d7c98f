"""GPU parity of the planar-quantized KV cache (src/kvquant.rs; the quantized
branches of src/forward.rs:99-140, 296-349): bh_kv_store_planar against the
oracle's append bit for bit (indices and norms), bh_attention_planar against
the oracle's attention over the same caches within 1e-5 (scores and P.V
summed in another order).  Every width 1..8, quantized and f32 V, one and
several queries, chunk and tile boundaries, zero and tiny vectors."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import rel_err

pytestmark = pytest.mark.gpu

HD = 256
TOL = 1e-5


def _say(*a):
    print(*a, flush=True)


def _t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _store(bh, dev, k, v, n_kv, bits, cap, quantize_v):
    import torch
    plen = bh.lib().bh_planar_packed_len(HD, bits)
    kq = torch.zeros((cap, n_kv, plen), dtype=torch.uint8, device=dev)
    kn = torch.zeros((cap, n_kv), device=dev)
    vq = torch.zeros_like(kq) if quantize_v else None
    vn = torch.zeros_like(kn) if quantize_v else None
    vf = None if quantize_v else torch.zeros((cap, n_kv * HD), device=dev)
    bh.kv_store_planar(_t(k, dev), _t(v, dev), 0, n_kv, bits, kq, kn, vq, vn, vf)
    return kq, kn, vq, vn, vf


@pytest.mark.parametrize("bits", range(1, 9))
def test_kv_store_planar_bit_exact(bh, oracle, synth, dev, bits):
    import torch
    n_kv, n = 4, 37
    r = synth.Rng(40 + bits)
    k = r.normal(n * n_kv * HD).reshape(n, n_kv * HD)
    v = r.normal(n * n_kv * HD).reshape(n, n_kv * HD) * np.float32(1e-3)
    k[3, :HD] = 0.0                                   # zero vector: norm 0, unit 0
    k[5, HD:2 * HD] *= np.float32(1e-20)              # tiny but nonzero
    k[6, :HD] *= np.float32(1e12)
    _say("store planar", bits)
    kq, kn, vq, vn, _ = _store(bh, dev, k, v, n_kv, bits, n, True)
    rkq, rkn, rvq, rvn, _ = oracle.kv_store_planar(k, v, n_kv, HD, bits, n, 0, True)
    torch.cuda.synchronize()
    assert np.array_equal(kq.cpu().numpy(), rkq)
    assert np.array_equal(kn.cpu().numpy().view(np.uint32), rkn.view(np.uint32))
    assert np.array_equal(vq.cpu().numpy(), rvq)
    assert np.array_equal(vn.cpu().numpy().view(np.uint32), rvn.view(np.uint32))


def test_kv_store_planar_f32_v_and_offset(bh, oracle, synth, dev):
    """planarNk: V rows copied in f32; rows land at positions pos0 .."""
    import torch
    n_kv, n, pos0, cap, bits = 4, 5, 9, 16, 4
    r = synth.Rng(77)
    k = r.normal(n * n_kv * HD).reshape(n, n_kv * HD)
    v = r.normal(n * n_kv * HD).reshape(n, n_kv * HD)
    plen = bh.lib().bh_planar_packed_len(HD, bits)
    kq = torch.zeros((cap, n_kv, plen), dtype=torch.uint8, device=dev)
    kn = torch.zeros((cap, n_kv), device=dev)
    vf = torch.zeros((cap, n_kv * HD), device=dev)
    bh.kv_store_planar(_t(k, dev), _t(v, dev), pos0, n_kv, bits, kq, kn, v_f32=vf)
    rkq, rkn, _, _, rvf = oracle.kv_store_planar(k, v, n_kv, HD, bits, cap, pos0, False)
    torch.cuda.synchronize()
    assert np.array_equal(kq.cpu().numpy(), rkq)
    assert np.array_equal(kn.cpu().numpy(), rkn)
    assert np.array_equal(vf.cpu().numpy(), rvf)


@pytest.mark.parametrize("bits,quantize_v,n_q,pos0,n_head,n_kv", [
    (4, True, 1, 0, 24, 4),
    (4, True, 1, 31, 24, 4),       # exactly one tile
    (4, True, 1, 32, 24, 4),       # a tile and one position
    (4, True, 1, 4095, 24, 4),     # the model's decode at ctx 4096
    (3, True, 1, 9000, 24, 4),     # several tiles per chunk, ragged last chunk
    (2, True, 1, 2000, 24, 4),     # 2-bit K and V
    (8, True, 1, 5000, 16, 2),     # 8-bit, groups of 8
    (2, False, 1, 700, 24, 4),     # V in f32 (planarNk)
    (8, True, 3, 100, 24, 4),      # several queries
    (1, True, 2, 63, 8, 8),        # one q head per kv head
    (5, True, 1, 300, 16, 2),      # groups of 8
    (6, False, 4, 50, 12, 4),
    # n_q * rep >= 48: the matrix-core path
    (4, True, 8, 500, 24, 4),      # 48 rows per kv head
    (3, True, 64, 4032, 24, 4),    # 64 queries at ctx 4096
    (7, True, 20, 33, 24, 4),      # index bits straddling dwords
    (2, False, 16, 100, 16, 2),    # V in f32, groups of 8
    (1, True, 50, 0, 8, 8),        # one q head per kv head, from position 0
    (8, True, 130, 70, 12, 4),     # more than one 128-row tile
])
def test_attention_planar(bh, oracle, synth, dev, bits, quantize_v, n_q, pos0, n_head, n_kv):
    n = pos0 + n_q
    r = synth.Rng(500 + bits + n)
    k = r.normal(n * n_kv * HD).reshape(n, n_kv * HD)
    v = r.normal(n * n_kv * HD).reshape(n, n_kv * HD)
    q = (r.normal(n_q * n_head * HD).reshape(n_q, n_head, HD) * np.float32(2.0)).astype(np.float32)
    _say("attention planar", bits, quantize_v, n_q, pos0, n_head, n_kv)
    kq, kn, vq, vn, vf = _store(bh, dev, k, v, n_kv, bits, n, quantize_v)
    got = bh.attention_planar(_t(q, dev), pos0, kq, kn, n_kv, bits, vq, vn, vf).cpu().numpy()
    rkq, rkn, rvq, rvn, rvf = oracle.kv_store_planar(k, v, n_kv, HD, bits, n, 0, quantize_v)
    ref = oracle.attention_planar(q, pos0, rkq, rkn, rvq, rvn, rvf, n_kv, bits, quantize_v)
    err = rel_err(got, ref)
    _say("  rel", err)
    assert err <= TOL


def test_attention_planar_graph_replay(bh, oracle, synth, dev):
    """Captured (planar kernel + merge with the inverse rotation, tables as
    kernel arguments) and replayed with new q contents."""
    import torch
    n_head, n_kv, bits, pos0 = 24, 4, 4, 2047
    n = pos0 + 1
    r = synth.Rng(91)
    k = r.normal(n * n_kv * HD).reshape(n, n_kv * HD)
    v = r.normal(n * n_kv * HD).reshape(n, n_kv * HD)
    kq, kn, vq, vn, _ = _store(bh, dev, k, v, n_kv, bits, n, True)
    rkq, rkn, rvq, rvn, rvf = oracle.kv_store_planar(k, v, n_kv, HD, bits, n, 0, True)
    qs = [r.normal(n_head * HD).reshape(1, n_head, HD) for _ in range(3)]
    qd = _t(qs[0], dev)
    out = torch.empty_like(qd)
    s = torch.cuda.Stream()
    bh.attention_planar(qd, pos0, kq, kn, n_kv, bits, vq, vn, out=out, stream=s)  # warm scratch
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        bh.attention_planar(qd, pos0, kq, kn, n_kv, bits, vq, vn, out=out, stream=s)
    for qi in qs:
        qd.copy_(_t(qi, dev))
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            g.replay()
        torch.cuda.synchronize()
        ref = oracle.attention_planar(qi, pos0, rkq, rkn, rvq, rvn, rvf, n_kv, bits, True)
        assert rel_err(out.cpu().numpy(), ref) <= TOL


def test_planar_argument_errors(bh):
    lib = bh.lib()
    assert lib.bh_planar_packed_len(256, 3) == 96
    assert lib.bh_kv_store_planar(None, None, 1, 1, 128, 4, None, None, None, None, None, 0,
                                  None) == bh.BH_ERR_SHAPE
    assert lib.bh_kv_store_planar(None, None, 1, 1, 256, 9, None, None, None, None, None, 0,
                                  None) == bh.BH_ERR_ARG
    assert lib.bh_attention_planar(None, 1, 0, None, None, None, None, None, 4, 24, 5, 256, None,
                                   None) == bh.BH_ERR_SHAPE


@pytest.mark.parametrize("bits", [2, 4])
def test_attention_planar_skips_zero_probability_inf_norm(bh, oracle, synth, dev, bits):
    """One query over two positions: position 0's key points along q (score
    ~ +2000), position 1's against it (~ -2000), so p_1 underflows to 0, and
    position 1's V row overflows to an infinite norm.  The reference skips
    p == 0 (src/forward.rs:335), so the output is finite: 1 x |v_0|-weighted
    centroids of v_0; the decode kernel must not form 0 x inf."""
    n_head, n_kv = 4, 1
    r = synth.Rng(77 + bits)
    q = (r.normal(n_head * HD).reshape(1, n_head, HD) * np.float32(2.0)).astype(np.float32)
    qd = q[0, 0] / np.linalg.norm(q[0, 0])
    k = np.stack([qd * 1e3, -qd * 1e3]).astype(np.float32)
    v = np.stack([r.normal(HD), r.normal(HD) * np.float32(1e30)]).astype(np.float32)
    kq, kn, vq, vn, vf = _store(bh, dev, k, v, n_kv, bits, 2, True)
    assert np.isinf(vn.cpu().numpy()[1, 0])
    got = bh.attention_planar(_t(q, dev), 1, kq, kn, n_kv, bits, vq, vn, vf).cpu().numpy()
    rkq, rkn, rvq, rvn, rvf = oracle.kv_store_planar(k, v, n_kv, HD, bits, 2, 0, True)
    ref = oracle.attention_planar(q, 1, rkq, rkn, rvq, rvn, rvf, n_kv, bits, True)
    assert np.all(np.isfinite(ref[0, 0])) and np.all(np.isfinite(got[0, 0]))
    assert rel_err(got[0, 0], ref[0, 0]) <= TOL
