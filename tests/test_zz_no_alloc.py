"""bh_softmax_rows_noalloc, the entry point that allocates nothing: same
results as bh_softmax_rows bit for bit (both run the same kernels; only the
scratch of the wide-row path differs), on two calls in a row with the second
smaller, so the fixed array's leftover contents from the first call must not
leak into the second.  Also checked against the CPU oracle (softmax tolerance
2e-5, src/kernels.rs:175-202) and for the size limit of the fixed array."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from conftest import rel_err

pytestmark = pytest.mark.gpu


def _call(bh, fn, x, row_len, inv_t, out):
    import torch
    s = torch.cuda.current_stream().cuda_stream
    return fn(ctypes.c_void_p(x.data_ptr()), x.numel(), row_len, inv_t,
              ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(s))


@pytest.mark.parametrize("shapes", [
    [(64, 248320, 1 / 0.7), (3, 248320, 1.0)],   # wide rows: fixed scratch path
    [(40, 65536, 1.0), (2, 20000, 1.25)],        # second call: fewer chunks, ragged row
    [(512, 2048, 1.0), (7, 100, 2.0)],           # one-workgroup rows: no scratch at all
])
def test_noalloc_matches_softmax_rows(bh, oracle, synth, dev, shapes):
    import torch
    lib = bh.lib()
    for i, (rows, row_len, inv_t) in enumerate(shapes):
        print(f"noalloc call {i}: rows {rows} row_len {row_len}", flush=True)
        xs = synth.Rng(70 + i).normal(rows * row_len, 0.0, 3.0).reshape(rows, row_len)
        xs[0, : row_len // 3] = -np.inf  # a partly masked row
        x = torch.from_numpy(xs).to(dev)
        want = torch.empty_like(x)
        got = torch.full_like(x, float("nan"))
        assert _call(bh, lib.bh_softmax_rows, x, row_len, inv_t, want) == 0, bh.last_error()
        assert _call(bh, lib.bh_softmax_rows_noalloc, x, row_len, inv_t, got) == 0, \
            bh.last_error()
        torch.cuda.synchronize()
        g, w = got.cpu().numpy(), want.cpu().numpy()
        assert np.array_equal(g.view(np.uint32), w.view(np.uint32)), f"call {i}"
        assert rel_err(g[:8], oracle.softmax_rows(xs[:8], row_len, inv_t)) < 2e-5, f"call {i}"


def test_noalloc_rejects_inputs_beyond_its_scratch(bh, dev):
    import torch
    lib = bh.lib()
    # 1500 rows of 248320: 1500 * 61 chunks * 12 B > 1 MiB
    x = torch.zeros((1500, 248320), device=dev)
    st = _call(bh, lib.bh_softmax_rows_noalloc, x, 248320, 1.0, x)
    assert st == bh.BH_ERR_SHAPE
    assert "above the fixed 1048576" in bh.last_error()
    torch.cuda.synchronize()
