"""HIP-graph capture of the entry points a serving loop would capture: the
fused gather + RMSNorm (two streams, fork/join) and the wide-row softmax
(three launches, library scratch).  Each graph is replayed several times with
eager work and synchronisation in between; every replay must reproduce the
eager result bit for bit."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _replay_check(make_out, run, dev, replays=4):
    import torch
    s = torch.cuda.Stream()
    eager = run(s)
    torch.cuda.synchronize()  # the work ran on `s`; clone only after it finished
    eager = [o.clone() for o in eager]
    torch.cuda.synchronize()
    outs = make_out()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        run(s, outs)
    for i in range(replays):
        for o in outs:
            o.fill_(float("nan"))
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            g.replay()
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            assert torch.equal(o.view(torch.int32), e.view(torch.int32)), f"replay {i} differs"
        # unrelated eager work between replays
        run(s)
        torch.cuda.synchronize()


def test_graph_gather_rms(bh, synth, dev):
    import torch
    table = _t(synth.pq2_table(synth.Rng(1), 300, 5120), dev)
    ids = _t((synth.Rng(2).u64(1000) % np.uint64(300)).astype(np.uint32), dev)
    w = _t(synth.Rng(3).normal(5120, 1.0, 0.1), dev)

    def make_out():
        return [torch.empty((1000, 5120), device=dev), torch.empty((1000, 5120), device=dev)]

    def run(s, outs=None):
        outs = outs or make_out()
        e, n = bh.pq2_embed_gather(table, 5120, 300, ids, w=w, out=outs[0], out_norm=outs[1],
                                   stream=s)
        return [e, n]

    _replay_check(make_out, run, dev)


def test_graph_softmax_wide(bh, synth, dev):
    import torch
    x = _t(synth.Rng(4).normal(16 * 248320, 0.0, 3.0).reshape(16, 248320), dev)

    def make_out():
        return [torch.empty_like(x)]

    def run(s, outs=None):
        outs = outs or make_out()
        return [bh.softmax_rows(x, 248320, 1.25, out=outs[0], stream=s)]

    _replay_check(make_out, run, dev)


def test_graph_qk_norm_rope(bh, synth, dev):
    import torch
    q = _t(synth.Rng(5).normal(64 * 24 * 256).reshape(64, 24, 256), dev)
    k = _t(synth.Rng(6).normal(64 * 4 * 256).reshape(64, 4, 256), dev)
    wq = _t(synth.Rng(7).normal(256, 1.0, 0.1), dev)
    wk = _t(synth.Rng(8).normal(256, 1.0, 0.1), dev)
    pos = _t(synth.positions(64), dev)

    def make_out():
        return [torch.empty_like(q), torch.empty_like(k)]

    def run(s, outs=None):
        outs = outs or make_out()
        bh.qk_norm_rope(bh.make_qk_args(q, outs[0], k, outs[1], wq, wk, pos, 64, 24, 4), stream=s)
        return outs

    _replay_check(make_out, run, dev)


def test_graph_softmax_survives_scratch_growth(bh, oracle, synth, dev):
    """A graph captured with the wide-row softmax keeps the library scratch
    address it recorded.  A later eager call needing more scratch (here about
    1.2 MB of row partials, above the 1 MB first allocation) makes the library
    switch to a larger buffer; the old one must stay alive, so every replay of
    the graph still matches the oracle."""
    import torch
    from conftest import rel_err
    xs = synth.Rng(40).normal(4 * 248320, 0.0, 3.0).reshape(4, 248320)
    ref = oracle.softmax_rows(xs, 248320, 1.25)
    x = _t(xs, dev)
    out = torch.empty_like(x)
    s = torch.cuda.Stream()
    torch.cuda.synchronize()  # x and out come from the default stream; the calls run on s
    bh.softmax_rows(x, 248320, 1.25, out=out, stream=s)  # eager: scratch exists before capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        bh.softmax_rows(x, 248320, 1.25, out=out, stream=s)
    first = None
    for i in range(3):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            g.replay()
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        assert rel_err(got, ref) < 2e-5, f"replay {i}"
        if first is None:
            first = got
        assert np.array_equal(got.view(np.uint32), first.view(np.uint32)), f"replay {i} differs"
        if i == 0:
            # 100 rows of 2^22: 1024 chunks per row -> 102400 partials x 12 B
            row = 1 << 22
            big = torch.randn((100, row), device=dev, generator=torch.Generator(dev).manual_seed(3))
            torch.cuda.synchronize()  # big comes from the default stream; the call runs on s
            bout = bh.softmax_rows(big, row, 1.0, stream=s)
            torch.cuda.synchronize()
            for r in (0, 99):
                assert rel_err(bout[r].cpu().numpy(),
                               oracle.softmax_rows(big[r].cpu().numpy(), row)) < 2e-5, r
            del big, bout
            torch.cuda.synchronize()


def test_scratch_release_frees_retired_buffers(bh, oracle, synth, dev):
    """Growing a scratch slot retires the old buffer; bh_scratch_release
    (for callers that know no captured graph still uses it) frees every
    retired buffer after synchronizing, and later calls work as before."""
    import torch
    from conftest import rel_err
    lib = bh.lib()
    before = lib.bh_scratch_retired_bytes()
    # a wide softmax needing more partials than any earlier call: the slot grows
    row = 1 << 22
    big = torch.randn((400, row // 4), device=dev, generator=torch.Generator(dev).manual_seed(4))
    bh.softmax_rows(big.reshape(100, row), row, 1.0)
    torch.cuda.synchronize()
    grown = lib.bh_scratch_retired_bytes()
    assert grown >= before
    assert lib.bh_scratch_release() == bh.BH_OK, bh.last_error()
    assert lib.bh_scratch_retired_bytes() == 0
    del big
    xs = synth.Rng(41).normal(3 * 248320, 0.0, 3.0).reshape(3, 248320)
    got = bh.softmax_rows(_t(xs, dev), 248320, 1.0).cpu().numpy()
    assert rel_err(got, oracle.softmax_rows(xs, 248320, 1.0)) < 2e-5


@pytest.mark.parametrize("n_q,pos0,f16", [(1, 4095, False), (3, 63, False), (1, 4095, True),
                                          (2, 700, True)])
def test_graph_attention_decode(bh, synth, dev, n_q, pos0, f16):
    """The decode attention (chunk partials in library scratch, then the
    chunk merge; for an f16 cache the matrix-core kernel): every replay,
    with eager calls in between, reproduces the eager result bit for bit."""
    import torch
    n_head, n_kv, hd = 24, 4, 256
    r = synth.Rng(77 + n_q)
    n = pos0 + n_q
    q = _t(r.normal(n_q * n_head * hd).reshape(n_q, n_head, hd).astype(np.float32), dev)
    kn = r.normal(n * n_kv * hd).reshape(n, n_kv * hd).astype(np.float32)
    vn = r.normal(n * n_kv * hd).reshape(n, n_kv * hd).astype(np.float32)
    if f16:
        kn = kn.astype(np.float16).view(np.uint16)
        vn = vn.astype(np.float16).view(np.uint16)
    kc, vc = _t(kn, dev), _t(vn, dev)

    def make_out():
        return [torch.empty_like(q)]

    def run(s, outs=None):
        outs = outs or make_out()
        bh.attention(q, pos0, kc, vc, n_kv, out=outs[0], stream=s)
        return outs

    _replay_check(make_out, run, dev)
