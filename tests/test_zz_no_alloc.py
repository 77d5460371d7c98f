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


_CAPTURE_SCRIPT = r'''
import ctypes, sys
import numpy as np
import torch
sys.path.insert(0, sys.argv[1])
from conftest import load_bonsai
bh = load_bonsai()
lib = bh.lib()
dev = torch.device("cuda:0")
rows, row_len, inv_t = 16, 248320, 1 / 0.7
x = torch.randn((rows, row_len), device=dev) * 3
want = torch.empty_like(x)
got = torch.full_like(x, float("nan"))
s = torch.cuda.Stream(device=dev)
def call(fn, out, stream):
    return fn(ctypes.c_void_p(x.data_ptr()), x.numel(), row_len, ctypes.c_float(inv_t),
              ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(stream.cuda_stream))
lib.bh_softmax_rows_noalloc.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_size_t,
                                        ctypes.c_float, ctypes.c_void_p, ctypes.c_void_p]
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g, stream=s):
    # the process's first no-allocation call: its scratch lookup happens here
    assert call(lib.bh_softmax_rows_noalloc, got, s) == 0, bh.last_error()
torch.cuda.synchronize()
assert call(lib.bh_softmax_rows, want, torch.cuda.current_stream()) == 0, bh.last_error()
torch.cuda.synchronize()
w = want.cpu().numpy().view(np.uint32)
for rep in range(3):
    got.fill_(float("nan"))
    x.mul_(1.0)  # eager work between replays
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    assert np.array_equal(got.cpu().numpy().view(np.uint32), w), f"replay {rep}"
print("capture ok")
'''


def test_noalloc_first_call_inside_graph_capture(dev):
    """The first wide-row no-allocation call of a process made inside a HIP
    graph capture (so the per-device scratch address is looked up during the
    capture); three replays, with eager work between them, each match
    bh_softmax_rows bit for bit.  Runs in a fresh process so no earlier call
    has done the lookup."""
    import subprocess
    import sys
    from pathlib import Path
    here = Path(__file__).resolve().parent
    res = subprocess.run([sys.executable, "-c", _CAPTURE_SCRIPT, str(here)], capture_output=True,
                         text=True, timeout=300)
    print(res.stdout[-2000:], res.stderr[-2000:])
    assert res.returncode == 0 and "capture ok" in res.stdout
