"""Benchmark of the fused layer kernels on one MI355X.

Headline (the JSON line's `value`): the attention pre-block -- per-head q/k
RMSNorm fused with IMROPE -- on config 2 of the benchmark definition:
q [2048, 24, 256], k [2048, 4, 256] fp32, rotary 64 with sections
[11,11,10,0], theta 1e7, positions 0..2047.  One step = one launch of
bh_qk_norm_rope over the whole batch.  `value` = algorithmic HBM bytes per
step / measured time, in GB/s.

The line also carries, for every kernel family of the hot path, the achieved
GB/s, fraction of the 8 TB/s HBM peak and rows/s ("kernels"), the roofline of
the dominant kernel and a CPU baseline: the C restatement of the reference
(oracle/) timed on this host, one core, on a bounded sample.

Inputs are synthetic (config distributions), already resident in HBM when the
timed region starts.  Buffer sets rotate so each config's working set exceeds
the 256 MB Infinity Cache (MALL); otherwise repeated launches would be served
from it and overstate HBM bandwidth.
"""
from __future__ import annotations

import argparse
import importlib.util
import json
import os
import re
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
PKG_DIR = REPO / "ternary-bonsai-inference_amd"
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense f16/bf16 MFMA
HBM_PEAK_GBS = 8000.0
ROTATE_BYTES = 600 * 2**20  # > 2x the 256 MB MALL


def _load(name: str, path: Path):
    if name in sys.modules:
        return sys.modules[name]
    is_pkg = path.name == "__init__.py"
    spec = importlib.util.spec_from_file_location(
        name, path, submodule_search_locations=[str(path.parent)] if is_pkg else None)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def n_sets(bytes_per_set: int, max_sets: int = 32) -> int:
    return max(1, min(max_sets, -(-ROTATE_BYTES // max(1, bytes_per_set))))


def time_launches(launch, n_rot: int, steps: int, warmup: int, stream) -> float:
    """Average ms per launch.  The W warmup launches run eagerly; the K timed
    launches are captured into one HIP graph (so the Python/ctypes launch
    cost does not space them out).  The graph is replayed once untimed
    (upload), then replayed again untimed directly before the timed replay,
    which sits between two HIP events recorded on the launch stream, with
    synchronisation on both sides.  The untimed replay keeps the GPU busy
    with the same kernel while the host submits the timed one, so the timed
    launches neither wait on the host nor start from an idle (clocked-down)
    memory system."""
    import torch
    for i in range(max(1, warmup)):
        launch(i % n_rot)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for i in range(steps):
            launch(i % n_rot)
    with torch.cuda.stream(stream):  # replay() launches on the current stream
        graph.replay()  # untimed: first replay uploads the graph
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        graph.replay()  # untimed: runs while the timed replay is submitted
        e0.record(stream)
        graph.replay()
        e1.record(stream)
    torch.cuda.synchronize()
    del graph
    return e0.elapsed_time(e1) / steps


# ---------------------------------------------------------------------------
# workloads: each returns (launch(i), n_rot, algorithmic bytes, rows, info)
# ---------------------------------------------------------------------------

def wl_qk_norm_rope(bh, synth, dev, stream, n_tok=2048):
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(1)
    nq, nk, hd = 24, 4, 256
    bytes_per = (n_tok * nq * hd * 4 + n_tok * nk * hd * 4) * 2 + 2 * hd * 4
    sets = []
    for _ in range(n_sets(bytes_per)):
        q = torch.randn((n_tok, nq, hd), device=dev, generator=g)
        k = torch.randn((n_tok, nk, hd), device=dev, generator=g)
        sets.append((q, torch.empty_like(q), k, torch.empty_like(k)))
    wq = 1 + 0.1 * torch.randn(hd, device=dev, generator=g)
    wk = 1 + 0.1 * torch.randn(hd, device=dev, generator=g)
    pos = torch.from_numpy(synth.positions(n_tok)).to(dev)
    args = [bh.make_qk_args(q, qo, k, ko, wq, wk, pos, n_tok, nq, nk) for q, qo, k, ko in sets]
    sh = stream.cuda_stream
    lib = bh.lib()
    import ctypes
    refs = [ctypes.byref(a) for a in args]

    def launch(i):
        st = lib.bh_qk_norm_rope(refs[i], sh)
        if st:
            bh.check(st)
    keep = (sets, wq, wk, pos, args)
    return launch, len(sets), bytes_per, n_tok, keep


def wl_rms_rows(bh, synth, dev, stream, rows=512, row_len=5120):
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    bytes_per = rows * row_len * 4 * 2 + row_len * 4
    sets = [(torch.randn((rows, row_len), device=dev, generator=g),
             torch.empty((rows, row_len), device=dev)) for _ in range(n_sets(bytes_per))]
    w = 1 + 0.1 * torch.randn(row_len, device=dev, generator=g)
    lib, sh = bh.lib(), stream.cuda_stream
    n = rows * row_len

    def launch(i):
        x, y = sets[i]
        st = lib.bh_rms_norm_rows(x.data_ptr(), n, w.data_ptr(), row_len, row_len, 1e-6,
                                  y.data_ptr(), sh)
        if st:
            bh.check(st)
    return launch, len(sets), bytes_per, rows, (sets, w)


def wl_gdn_prep(bh, synth, dev, stream, n_tok=4096, with_conv=False):
    """Config 3; with with_conv the causal conv1d (k = 4) runs in front, from
    the raw qkv and the cache (src/forward.rs:508-533): the same row bytes
    plus the taps and the cache read and written."""
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(2)
    C, H, K = 6144, 48, 4
    bytes_per = (n_tok * C * 4 * 2 + n_tok * H * 4 * 2 + 2 * H * 4 + n_tok * H * 4 * 2
                 + n_tok * C * 4 * 3)
    if with_conv:
        bytes_per += C * K * 4 + 2 * C * (K - 1) * 4
    taps = 0.5 * torch.randn((C, K), device=dev, generator=g) if with_conv else None
    A = -torch.exp(2 * torch.rand(H, device=dev, generator=g))
    bias = 0.5 * torch.randn(H, device=dev, generator=g)
    sets = []
    for _ in range(n_sets(bytes_per)):
        conv = torch.randn((n_tok, C), device=dev, generator=g)
        z = torch.randn((n_tok, C), device=dev, generator=g)
        y = torch.randn((n_tok, C), device=dev, generator=g)
        dt = torch.randn((n_tok, H), device=dev, generator=g)
        beta = torch.randn((n_tok, H), device=dev, generator=g)
        outs = [torch.empty_like(conv), torch.empty_like(z), torch.empty_like(dt),
                torch.empty_like(beta)]
        cache = torch.randn((C, K - 1), device=dev, generator=g) if with_conv else None
        sets.append((conv, z, y, dt, beta, outs, cache))
    args = [bh.make_gdn_args(conv=c, conv_out=o[0], z=z, y=y, gated_out=o[1], alpha_raw=dt,
                             dt_bias=bias, ssm_a=A, beta_raw=b, gate_out=o[2], beta_out=o[3],
                             n_tok=n_tok, conv_dim=C, l2_dim=C, head_dim=128, inner_dim=C,
                             n_v_head=H, gate_mode=bh.BH_SIGMOID_MUL, eps=1e-6,
                             conv_w=taps, conv_state=cache, conv_k=K)
            for c, z, y, dt, b, o, cache in sets]
    import ctypes
    refs = [ctypes.byref(a) for a in args]
    lib, sh = bh.lib(), stream.cuda_stream

    def launch(i):
        st = lib.bh_gdn_prep_fused(refs[i], sh)
        if st:
            bh.check(st)
    return launch, len(sets), bytes_per, n_tok, (sets, A, bias, args, taps)


def wl_conv1d(bh, synth, dev, stream, n_tok=4096, ch=10240, k=4):
    """Causal conv1d + SiLU (src/forward.rs:508-533) over a prefill batch of
    the model's qkv width: inputs read once, outputs written once, the taps
    and the cache (read and written)."""
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    bytes_per = 2 * n_tok * ch * 4 + ch * k * 4 + 2 * ch * (k - 1) * 4
    w = 0.5 * torch.randn((ch, k), device=dev, generator=g)
    sets = [(torch.randn((n_tok, ch), device=dev, generator=g),
             torch.randn((ch, k - 1), device=dev, generator=g),
             torch.empty((n_tok, ch), device=dev)) for _ in range(n_sets(bytes_per))]
    lib, sh = bh.lib(), stream.cuda_stream

    def launch(i):
        x, cache, out = sets[i]
        st = lib.bh_conv1d_silu(x.data_ptr(), cache.data_ptr(), w.data_ptr(), n_tok, ch, k,
                                out.data_ptr(), sh)
        if st:
            bh.check(st)
    return launch, len(sets), bytes_per, n_tok, (sets, w)


def wl_gdn_step(bh, synth, dev, stream, n_tok, h_k=16, h_v=48, s=128):
    """Gated delta-net recurrence (src/gdn.rs:17-77) over n_tok tokens of the
    model's heads: the state [48,128,128] read and written once, per token
    q, k [16,128], v, attn [48,128] and gate, beta [48]."""
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(8)
    per_tok = (2 * h_k * s + 2 * h_v * s + 2 * h_v) * 4
    bytes_per = 2 * h_v * s * s * 4 + n_tok * per_tok
    q = torch.nn.functional.normalize(torch.randn((n_tok, h_k, s), device=dev, generator=g), dim=-1)
    k = torch.nn.functional.normalize(torch.randn((n_tok, h_k, s), device=dev, generator=g), dim=-1)
    v = torch.randn((n_tok, h_v, s), device=dev, generator=g)
    gate = -torch.rand((n_tok, h_v), device=dev, generator=g)
    beta = torch.rand((n_tok, h_v), device=dev, generator=g)
    sets = [(0.1 * torch.randn((h_v, s, s), device=dev, generator=g),
             torch.empty((n_tok, h_v, s), device=dev)) for _ in range(n_sets(bytes_per))]
    lib, sh = bh.lib(), stream.cuda_stream

    def launch(i):
        st_, attn = sets[i]
        rc = lib.bh_gdn_step(q.data_ptr(), k.data_ptr(), v.data_ptr(), gate.data_ptr(),
                             beta.data_ptr(), st_.data_ptr(), attn.data_ptr(), n_tok, h_k, h_v,
                             s, sh)
        if rc:
            bh.check(rc)
    return launch, len(sets), bytes_per, n_tok, (sets, q, k, v, gate, beta)


def wl_softmax(bh, synth, dev, stream, rows, row_len, inv_t, causal=False, spikes=False):
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(3 if spikes else 4)
    bytes_per = rows * row_len * 4 * 2
    sets = []
    for _ in range(n_sets(bytes_per)):
        x = torch.randn((rows, row_len), device=dev, generator=g) * (3.0 if spikes else 2.0)
        if spikes:
            x += 10.0 * (torch.rand((rows, row_len), device=dev, generator=g) < 0.01)
        if causal:
            q = torch.arange(rows, device=dev) % row_len
            x.masked_fill_(torch.arange(row_len, device=dev)[None, :] > q[:, None],
                           float("-inf"))
        sets.append((x, torch.empty_like(x)))
    lib, sh = bh.lib(), stream.cuda_stream
    n = rows * row_len

    def launch(i):
        x, y = sets[i]
        st = lib.bh_softmax_rows(x.data_ptr(), n, row_len, inv_t, y.data_ptr(), sh)
        if st:
            bh.check(st)
    return launch, len(sets), bytes_per, rows, sets


def wl_gather_rms(bh, synth, dev, stream, n_tok=8192, vocab=248320, ne0=5120):
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    table = synth.torch_pq2_table(vocab, ne0, dev, generator=g)
    w = 1 + 0.1 * torch.randn(ne0, device=dev, generator=g)
    rb = table.shape[1]
    bytes_per = n_tok * rb + n_tok * 4 + ne0 * 4 + 2 * n_tok * ne0 * 4
    sets = []
    for _ in range(n_sets(2 * n_tok * ne0 * 4)):
        ids = torch.randint(0, vocab, (n_tok,), device=dev, generator=g, dtype=torch.int32)
        sets.append((ids, torch.empty((n_tok, ne0), device=dev),
                     torch.empty((n_tok, ne0), device=dev)))
    lib, sh = bh.lib(), stream.cuda_stream

    def launch(i):
        ids, e, nrm = sets[i]
        st = lib.bh_pq2_embed_gather_rms(table.data_ptr(), ne0, vocab, ids.data_ptr(), n_tok,
                                         w.data_ptr(), ne0, 1e-6, e.data_ptr(), nrm.data_ptr(),
                                         None, sh)
        if st:
            bh.check(st)
    return launch, len(sets), bytes_per, n_tok, (table, w, sets)


def wl_attention(bh, synth, dev, stream, n_q, pos0, f16, n_head=24, n_kv=4, hd=256):
    """Grouped-query attention over the KV cache (src/forward.rs:282-375) for
    n_q query tokens at positions pos0 .. on the model's heads (24 q / 4 kv x
    256).  Algorithmic bytes: the K and V rows of positions 0 .. pos0+n_q-1
    read once (f32 or f16 storage), q read and out written once."""
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(9)
    n_pos = pos0 + n_q
    esz = 2 if f16 else 4
    bytes_per = 2 * n_pos * n_kv * hd * esz + 2 * n_q * n_head * hd * 4
    dt = torch.float16 if f16 else torch.float32
    sets = []
    for _ in range(n_sets(bytes_per)):
        sets.append((torch.randn((n_q, n_head, hd), device=dev, generator=g),
                     torch.randn((n_pos, n_kv * hd), device=dev, generator=g).to(dt),
                     torch.randn((n_pos, n_kv * hd), device=dev, generator=g).to(dt),
                     torch.empty((n_q, n_head, hd), device=dev)))
    lib, sh = bh.lib(), stream.cuda_stream
    kvd = bh.BH_KV_F16 if f16 else bh.BH_KV_F32

    def launch(i):
        q, kc, vc, out = sets[i]
        st = lib.bh_attention(q.data_ptr(), n_q, pos0, kc.data_ptr(), vc.data_ptr(), kvd,
                              n_head, n_kv, hd, out.data_ptr(), sh)
        if st:
            bh.check(st)
    return launch, len(sets), bytes_per, n_q, sets


def wl_attention_planar(bh, synth, dev, stream, n_q, pos0, bits, quantize_v=True, n_head=24,
                        n_kv=4, hd=256):
    """Attention over a planar-quantized KV cache (BONSAI_KV=planarN,
    src/forward.rs:296-349, src/kvquant.rs) on the model's heads.  The caches
    are filled by bh_kv_store_planar at setup (untimed).  Algorithmic bytes:
    the packed rows and norms of K (and V, or V's f32 rows) of positions
    0 .. pos0+n_q-1 read once, q read and out written once."""
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(10)
    n_pos = pos0 + n_q
    plen = bh.lib().bh_planar_packed_len(hd, bits)
    kv_bytes = n_pos * n_kv * (plen + 4)
    bytes_per = kv_bytes + (kv_bytes if quantize_v else n_pos * n_kv * hd * 4) + \
        2 * n_q * n_head * hd * 4
    sets = []
    for _ in range(n_sets(bytes_per)):
        k = torch.randn((n_pos, n_kv * hd), device=dev, generator=g)
        v = torch.randn((n_pos, n_kv * hd), device=dev, generator=g)
        kq = torch.empty((n_pos, n_kv, plen), dtype=torch.uint8, device=dev)
        kn = torch.empty((n_pos, n_kv), device=dev)
        vq = torch.empty_like(kq) if quantize_v else None
        vn = torch.empty_like(kn) if quantize_v else None
        vf = None if quantize_v else torch.empty((n_pos, n_kv * hd), device=dev)
        bh.kv_store_planar(k, v, 0, n_kv, bits, kq, kn, vq, vn, vf, stream=stream)
        del k, v
        sets.append((torch.randn((n_q, n_head, hd), device=dev, generator=g), kq, kn, vq, vn, vf,
                     torch.empty((n_q, n_head, hd), device=dev)))
    torch.cuda.synchronize()
    lib, sh = bh.lib(), stream.cuda_stream
    ptr = lambda t: None if t is None else t.data_ptr()

    def launch(i):
        q, kq, kn, vq, vn, vf, out = sets[i]
        st = lib.bh_attention_planar(q.data_ptr(), n_q, pos0, kq.data_ptr(), kn.data_ptr(),
                                     ptr(vq), ptr(vn), ptr(vf), bits, n_head, n_kv, hd,
                                     out.data_ptr(), sh)
        if st:
            bh.check(st)
    return launch, len(sets), bytes_per, n_q, sets


def wl_pq2_matmul(bh, synth, dev, stream, n_rows, ne0, n_tok):
    """kernels::pq2_matmul_n / pq2_matvec_range (src/kernels.rs:283-423):
    Y[n_tok][n_rows] = X[n_tok][ne0] * W^T over a PQ2_0 weight tensor.  Each
    rotating set has its own weight tensor, so the weights stream from HBM
    (a decode step reads every matrix once).  Algorithmic bytes: the packed
    weights once, x and y once."""
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(6)
    rb = bh.pq2_row_bytes(ne0)
    bytes_per = n_rows * rb + n_tok * ne0 * 4 + n_tok * n_rows * 4
    sets = []
    for _ in range(n_sets(bytes_per)):
        table = synth.torch_pq2_table(n_rows, ne0, dev, generator=g).reshape(-1)
        x = torch.randn((n_tok, ne0), device=dev, generator=g)
        sets.append((table, x, torch.empty((n_tok, n_rows), device=dev)))
    lib, sh = bh.lib(), stream.cuda_stream

    def launch(i):
        table, x, y = sets[i]
        if n_tok == 1:
            st = lib.bh_pq2_matvec_range(table.data_ptr(), table.numel(), ne0, 0, n_rows,
                                         x.data_ptr(), ne0, y.data_ptr(), n_rows, sh)
        else:
            st = lib.bh_pq2_matmul_n(table.data_ptr(), table.numel(), ne0, 0, n_rows,
                                     x.data_ptr(), x.numel(), n_tok, y.data_ptr(), y.numel(), sh)
        if st:
            bh.check(st)
    return launch, len(sets), bytes_per, n_rows, sets


def measure_mm(name, n_rows, ne0, n_tok, bh, synth, dev, stream, steps, warmup):
    """A product entry: HBM GB/s as every entry, plus useful TFLOP/s (2 flops
    per weight and token) against the dense f16 MFMA peak; the x side runs
    as two f16 MFMAs (hi, lo), so half that peak is the useful ceiling."""
    rec = measure(name, wl_pq2_matmul(bh, synth, dev, stream, n_rows, ne0, n_tok), steps,
                  warmup, stream)
    tflops = 2.0 * n_tok * n_rows * ne0 / (rec["ms"] * 1e-3) / 1e12
    rec.update({"tokens": n_tok, "TFLOPs": round(tflops, 2),
                "frac_mfma_f16": round(tflops / MFMA_F16_PEAK_TFLOPS, 4)})
    return rec


def measure(name, wl, steps, warmup, stream, extra=None):
    import torch
    launch, n_rot, nbytes, rows, keep = wl
    ms = time_launches(launch, n_rot, steps, warmup, stream)
    gbs = nbytes / (ms * 1e-3) / 1e9
    rec = {"kernel": name, "ms": round(ms, 5), "GBps": round(gbs, 1),
           "frac_hbm": round(gbs / HBM_PEAK_GBS, 4), "bytes": nbytes, "rows": rows,
           "rows_per_s": round(rows / (ms * 1e-3), 1), "rotating_sets": n_rot}
    if extra:
        rec.update(extra)
    del keep
    torch.cuda.empty_cache()
    return rec


# ---------------------------------------------------------------------------
# CPU baseline: the oracle (C restatement of the reference), 1 thread
# ---------------------------------------------------------------------------

def _time_cpu(run, n_units: int, seconds: float):
    """Repeat run(lo, hi) over the whole sample on one thread for `seconds`,
    then split by units over the host's threads (the C oracle releases the
    GIL) for a quarter of that: (units/s one thread, units/s threaded,
    threads, repetitions one thread, repetitions threaded)."""
    import concurrent.futures
    reps, t0 = 0, time.perf_counter()
    while True:
        run(0, n_units)
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    try:
        n_thr = len(os.sched_getaffinity(0))
    except AttributeError:
        n_thr = os.cpu_count() or 1
    n_thr = max(1, min(n_thr, 16, n_units))  # the GPU box's CPU share is 16 cores
    cuts = [n_units * i // n_thr for i in range(n_thr + 1)]
    reps_mt, t1 = 0, time.perf_counter()
    with concurrent.futures.ThreadPoolExecutor(n_thr) as pool:
        while True:
            list(pool.map(run, cuts[:-1], cuts[1:]))
            reps_mt += 1
            el_mt = time.perf_counter() - t1
            if el_mt >= seconds / 4:
                break
    return n_units * reps / el, n_units * reps_mt / el_mt, n_thr, reps, reps_mt


def _cpu_entry(name, run, n_units, bytes_per_unit, rows_per_unit, seconds, sample):
    ups, ups_mt, n_thr, reps, reps_mt = _time_cpu(run, n_units, seconds)
    return {"config": name, "value": round(ups * bytes_per_unit / 1e9, 4), "unit": "GB/s",
            "cores": 1, "kind": "port", "rows_per_s": round(ups * rows_per_unit, 1),
            "sample": f"{sample}, {reps} repetitions in {seconds:.0f} s, 1 thread",
            "upper_bound_mt": {"value": round(ups_mt * bytes_per_unit / 1e9, 4), "unit": "GB/s",
                               "cores": n_thr, "rows_per_s": round(ups_mt * rows_per_unit, 1),
                               "sample": f"same sample split over {n_thr} threads, "
                                         f"{reps_mt} repetitions"}}


def cpu_baseline(bh, synth, oracle, seconds: float):
    """Time oracle.qk_norm_rope (src/forward.rs:237-270 restated) on the same
    config, repeating the 2048-token batch until `seconds` have passed: once on
    one thread (the reference's decode thread), then row-parallel over the
    host's cores for a quarter of that time (an upper bound for a threaded
    CPU path; the C call releases the GIL, tokens are split into contiguous
    slices, one per thread)."""
    n_tok, nq, nk, hd = 2048, 24, 4, 256
    r = synth.Rng(1)
    q = r.normal(n_tok * nq * hd).reshape(n_tok, nq, hd)
    k = r.normal(n_tok * nk * hd).reshape(n_tok, nk, hd)
    wq, wk = r.normal(hd, 1.0, 0.1), r.normal(hd, 1.0, 0.1)
    pos = synth.positions(n_tok)
    per_tok = (nq + nk) * hd * 4 * 2

    def run(lo, hi):
        oracle.qk_norm_rope(q[lo:hi], k[lo:hi], wq, wk, pos[lo:hi], nq, nk, hd, 64, bh.SECTIONS,
                            1e7, 1e-6)

    e = _cpu_entry("config 2", run, n_tok, per_tok, 1, seconds,
                   "oracle qk_norm_rope on the full config-2 batch (2048 tokens x 28 heads)")
    e.pop("config")
    return e


def cpu_baselines_other(bh, synth, oracle, seconds: float):
    """The CPU oracle (the reference's algorithm restated in C, one thread,
    then split by rows over the host's threads) on each other config of the
    benchmark, each on a bounded sample of its rows (said per entry);
    GB/s counts the config's algorithmic bytes per row."""
    import numpy as np
    out = []
    # config 1: rms_norm_rows [512, 5120] (src/kernels.rs:97-122)
    r = synth.Rng(0)
    x1, w1 = r.normal(512 * 5120).reshape(512, 5120), r.normal(5120, 1.0, 0.1)
    out.append(_cpu_entry(
        "config 1 rms_norm_rows [512,5120]",
        lambda lo, hi: oracle.rms_norm_rows(x1[lo:hi], w1, 5120, 1e-6), 512, 5120 * 8, 1,
        seconds, "oracle rms_norm_rows on all 512 rows"))
    # config 3: GDN prep [T, 6144] x 48 heads (src/forward.rs:497-507, 524, 539-540, 379)
    T3 = 512
    r = synth.Rng(2)
    conv, z, y = (r.normal(T3 * 6144).reshape(T3, 6144) for _ in range(3))
    dt, beta = r.normal(T3 * 48, 0.0, 0.5).reshape(T3, 48), r.normal(T3 * 48).reshape(T3, 48)
    bias = r.normal(48, 0.0, 0.5)
    A = -np.exp(2 * r.uniform(48)).astype(np.float32)
    per3 = 6144 * 4 * 2 + 48 * 4 * 2 + 48 * 4 * 2 + 6144 * 4 * 3

    def run3(lo, hi):
        oracle.silu_l2_part(conv[lo:hi], 6144, 128, 1e-6)
        oracle.unary(4, z[lo:hi], y[lo:hi])
        oracle.gdn_gate_prep(dt[lo:hi], bias, A, beta[lo:hi])
    out.append(_cpu_entry("config 3 gdn_prep [4096,6144]", run3, T3, per3, 1, seconds,
                          f"oracle silu_l2_part + sigmoid gate + gdn_gate_prep on {T3} of the "
                          "4096 tokens"))
    # config 4a: softmax_rows [64, 248320] at temperature 0.7 (src/kernels.rs:175-202)
    r = synth.Rng(3)
    n4a = 8 * 248320
    x4 = r.normal(n4a, 0.0, 3.0)
    x4[r.uniform(n4a) < 0.01] += np.float32(10.0)
    x4 = x4.reshape(8, 248320)
    inv_t = float(np.float32(1.0) / np.float32(0.7))
    out.append(_cpu_entry("config 4a softmax [64,248320] temp 0.7",
                          lambda lo, hi: oracle.softmax_rows(x4[lo:hi], 248320, inv_t), 8,
                          248320 * 8, 1, seconds, "oracle softmax_rows on 8 of the 64 rows"))
    # config 4b: causal softmax rows [24*2048, 2048]
    r = synth.Rng(4)
    xb = r.normal(2048 * 2048, 0.0, 2.0).reshape(2048, 2048)
    xb[np.triu(np.ones((2048, 2048), bool), 1)] = -np.inf
    out.append(_cpu_entry("config 4b softmax causal [24*2048,2048]",
                          lambda lo, hi: oracle.softmax_rows(xb[lo:hi], 2048), 2048, 2048 * 8, 1,
                          seconds, "oracle softmax_rows on one head's 2048 causal rows"))
    # config 5: gather + first RMSNorm (src/forward.rs:691, 701-702)
    # the full 248320-row table (338 MB, built on the device and copied to
    # host memory), so the CPU gathers rows that are not cache-resident,
    # as the GPU does
    import torch
    tab = synth.torch_pq2_table(248320, 5120, torch.device("cuda:0")).cpu().numpy()
    ids = (synth.Rng(6).u64(1024) % np.uint64(248320)).astype(np.uint32)
    w5 = synth.Rng(7).normal(5120, 1.0, 0.1)
    per5 = 1360 + 4 + 2 * 5120 * 4
    out.append(_cpu_entry("config 5 pq2_gather_rms [8192 ids, 248320x5120]",
                          lambda lo, hi: oracle.embed_gather(tab, 5120, 248320, ids[lo:hi], w5,
                                                             1e-6), 1024, per5, 1, seconds,
                          "oracle embed_gather + rms on 1024 uniform ids from the full "
                          "248320-row table (338 MB in host memory)"))
    del tab
    return out


def load_traffic():
    """HBM bytes per step of every bench entry (name -> bytes) from the
    committed rocprofv3 FETCH_SIZE / WRITE_SIZE runs of this bench
    (profiles/traffic_all_configs.json, commands inside), if recorded."""
    p = REPO / "profiles" / "traffic_all_configs.json"
    if not p.exists():
        return {}
    try:
        return {e["entry"]: e["hbm_bytes"] for e in json.loads(p.read_text())["entries"]}
    except (ValueError, OSError, KeyError):
        return {}


def measure_traffic_live(timeout_s: float = 90.0, budget_s: float = 240.0):
    """The headline kernel's HBM bytes per call measured now: two rocprofv3
    --pmc child runs of this bench (FETCH_SIZE, then WRITE_SIZE, headline
    only), each scaled by what the same counter reads for a 256 MiB device
    copy (two more child runs).  Returns (bytes, note) or (None, reason)."""
    import csv
    import glob
    import shutil
    import statistics
    import subprocess
    import tempfile
    prof = shutil.which("rocprofv3")
    if prof is None:
        return None, "rocprofv3 not found"
    env = dict(os.environ, TMPDIR="/tmp")
    me = [sys.executable, str(Path(__file__).resolve())]
    child = ["--headline-only", "--steps", "10", "--warmup", "2", "--cpu-seconds", "0",
             "--traffic", "committed"]
    runs = {"fetch": ("FETCH_SIZE", me + child),
            "write": ("WRITE_SIZE", me + child),
            "cfetch": ("FETCH_SIZE", me + ["--calibrate-copy", "256", "--steps", "5"]),
            "cwrite": ("WRITE_SIZE", me + ["--calibrate-copy", "256", "--steps", "5"])}
    vals = {}
    t0 = time.time()
    with tempfile.TemporaryDirectory(dir="/tmp") as tmp:
        for key, (counter, cmd) in runs.items():
            if time.time() - t0 > budget_s:
                return None, "counter runs over their time budget"
            d = os.path.join(tmp, key)
            try:
                subprocess.run([prof, "--pmc", counter, "--output-format", "csv", "-d", d, "-o", key,
                                "--"] + cmd, env=env, cwd="/tmp", capture_output=True,
                               timeout=timeout_s, check=True)
                f = glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)[0]
                rows = [r for r in csv.DictReader(open(f)) if r["Counter_Name"].startswith(counter)]
                if key.startswith("c"):
                    sel = [float(r["Counter_Value"]) for r in rows if "elementwise" in r["Kernel_Name"]
                           and int(r.get("Grid_Size") or r.get("Grid_Size_X") or 0) > 1000000]
                else:
                    sel = [float(r["Counter_Value"]) for r in rows
                           if "qk_norm_rope_kernel" in r["Kernel_Name"]]
                vals[key] = statistics.median(sel)
            except (OSError, subprocess.SubprocessError, IndexError, ValueError,
                    statistics.StatisticsError) as e:
                return None, f"live counter run {key} failed: {type(e).__name__}"
    copy = 256 * 2**20
    fbytes = vals["fetch"] * copy / vals["cfetch"]
    wbytes = vals["write"] * copy / vals["cwrite"]
    return int(fbytes + wbytes), ("live: rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE of this bench's "
                                  "headline in this run, scaled by a 256 MiB copy "
                                  f"(fetch {fbytes / 1e6:.1f} MB, write {wbytes / 1e6:.1f} MB)")


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--headline-only", action="store_true",
                    help="time only the headline kernel (profiling runs)")
    ap.add_argument("--only", default="",
                    help="after the headline, time only the entries whose name matches this regex")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="length of the CPU-baseline sample (0 disables)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB (counter calibration)")
    ap.add_argument("--traffic", choices=("live", "committed"), default="live",
                    help="live (default): measure the headline's HBM traffic in this run with "
                         "four short rocprofv3 counter child runs (falls back to the committed "
                         "figure if they fail); committed: read profiles/traffic_all_configs.json")
    args = ap.parse_args()
    # no nested counter runs when this process itself runs under rocprofv3
    profiled = any(k.startswith("ROCPROF") for k in os.environ)
    live = args.traffic == "live" and not args.calibrate_copy and args.gpus == 1 and not profiled
    live_traffic = measure_traffic_live() if live else (None, "")
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(every kernel is row-independent: multi-GPU runs would shard rows with no "
              "exchange)", file=sys.stderr)
        return 2

    import torch
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 2
    bh = _load("bonsai_amd", PKG_DIR / "__init__.py")
    synth = _load("bonsai_amd_synth", PKG_DIR / "synth.py")
    dev = torch.device("cuda:0")
    bh.lib()  # fail loudly if the HIP library is missing
    stream = torch.cuda.Stream(device=dev)

    if args.calibrate_copy:
        n = args.calibrate_copy * 2**20 // 4
        a = torch.randn(n, device=dev)
        b = torch.empty_like(a)
        with torch.cuda.stream(stream):
            for _ in range(args.steps):
                torch.mul(a, 1.0, out=b)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy_bytes_each_way": n * 4, "launches": args.steps}))
        return 0

    # bring clocks up before the first measurement: ~25 ms of 256 MB copies
    # (untimed; the first kernel measured in a cold process otherwise reads
    # up to 10% slow)
    warm_a = torch.empty(64 * 2**20, device=dev)
    warm_b = torch.empty_like(warm_a)
    for _ in range(300):
        warm_b.copy_(warm_a)
    torch.cuda.synchronize()
    del warm_a, warm_b

    with torch.cuda.stream(stream):
        head = measure("qk_norm_rope", wl_qk_norm_rope(bh, synth, dev, stream), args.steps,
                       args.warmup, stream)
        kernels = [head]
        if not args.headline_only:
            ksteps = max(10, args.steps // 4)
            np32 = __import__("numpy").float32
            rows_wl = {T: (lambda T=T: wl_rms_rows(bh, synth, dev, stream, T)) for T in (512, 2048, 8192)}
            entries = [
                ("rms_norm_rows T=512", rows_wl[512]),
                ("rms_norm_rows T=2048", rows_wl[2048]),
                ("rms_norm_rows T=8192", rows_wl[8192]),
                ("qk_norm_rope T=4096", lambda: wl_qk_norm_rope(bh, synth, dev, stream, 4096)),
                ("qk_norm_rope T=8192", lambda: wl_qk_norm_rope(bh, synth, dev, stream, 8192)),
                ("gdn_prep_fused T=2048", lambda: wl_gdn_prep(bh, synth, dev, stream, 2048)),
                ("gdn_prep_fused T=4096", lambda: wl_gdn_prep(bh, synth, dev, stream)),
                ("gdn_prep_fused + conv1d T=4096",
                 lambda: wl_gdn_prep(bh, synth, dev, stream, with_conv=True)),
                ("conv1d_silu [4096,10240] k=4", lambda: wl_conv1d(bh, synth, dev, stream)),
                ("softmax vocab [64,248320] temp 0.7",
                 lambda: wl_softmax(bh, synth, dev, stream, 64, 248320, float(1 / np32(0.7)),
                                    spikes=True)),
                ("softmax causal [24*2048,2048]",
                 lambda: wl_softmax(bh, synth, dev, stream, 24 * 2048, 2048, 1.0, causal=True)),
                ("pq2_gather_rms T=2048", lambda: wl_gather_rms(bh, synth, dev, stream, 2048)),
                ("pq2_gather_rms T=8192", lambda: wl_gather_rms(bh, synth, dev, stream)),
                ("gdn_step decode T=1", lambda: wl_gdn_step(bh, synth, dev, stream, 1)),
                ("gdn_step T=256", lambda: wl_gdn_step(bh, synth, dev, stream, 256)),
                ("gdn_step T=2048", lambda: wl_gdn_step(bh, synth, dev, stream, 2048)),
                ("attention decode ctx=4096 f32",
                 lambda: wl_attention(bh, synth, dev, stream, 1, 4095, False)),
                ("attention decode ctx=32768 f32",
                 lambda: wl_attention(bh, synth, dev, stream, 1, 32767, False)),
                ("attention decode ctx=32768 f16",
                 lambda: wl_attention(bh, synth, dev, stream, 1, 32767, True)),
                ("attention batch 64 queries ctx=4096 f32",
                 lambda: wl_attention(bh, synth, dev, stream, 64, 4032, False)),
                ("attention prefill 2048 queries from 0 f32",
                 lambda: wl_attention(bh, synth, dev, stream, 2048, 0, False)),
                ("attention decode ctx=32768 planar4",
                 lambda: wl_attention_planar(bh, synth, dev, stream, 1, 32767, 4)),
                ("attention decode ctx=4096 planar4",
                 lambda: wl_attention_planar(bh, synth, dev, stream, 1, 4095, 4)),
                ("attention batch 64 queries ctx=4096 planar4",
                 lambda: wl_attention_planar(bh, synth, dev, stream, 64, 4032, 4)),
            ]
            products = [  # (name, rows, ne0, tokens): decode matvecs and batched products
                ("pq2_matvec LM head [248320x5120] N=1", 248320, 5120, 1),
                ("pq2_matvec ffn_up [17408x5120] N=1", 17408, 5120, 1),
                ("pq2_matvec ffn_down [5120x17408] N=1", 5120, 17408, 1),
                ("pq2_matmul_n ffn_up [17408x5120] N=64", 17408, 5120, 64),
                ("pq2_matmul_n LM head [248320x5120] N=16", 248320, 5120, 16),
            ]
            for name, wl in entries:
                if re.search(args.only, name):
                    kernels.append(measure(name, wl(), ksteps, args.warmup, stream))
            for name, rows, ne0, n_tok in products:
                if re.search(args.only, name):
                    kernels.append(measure_mm(name, rows, ne0, n_tok, bh, synth, dev, stream,
                                              ksteps, args.warmup))
            for k in kernels:
                if k["kernel"].startswith("attention prefill 2048"):
                    # causal prefill: scores and P.V each 2 flops per (query, head,
                    # visible position, dim); query i sees i + 1 positions
                    n, heads, hd = 2048, 24, 256
                    flops = 2 * 2 * heads * hd * (n * (n + 1) // 2)
                    tf = flops / (k["ms"] * 1e-3) / 1e12
                    k.update({"useful_flops": flops, "TFLOPs": round(tf, 2),
                              "frac_mfma_f16": round(tf / MFMA_F16_PEAK_TFLOPS, 4),
                              "note": "f32 operands as f16 hi + lo: three MFMA products per "
                                      "useful one, so a third of the f16 peak is its ceiling"})

    cpu = None
    if args.cpu_seconds > 0:
        oracle = _load("bonsai_oracle", REPO / "oracle" / "oracle.py")
        cpu = cpu_baseline(bh, synth, oracle, args.cpu_seconds)
        if not args.headline_only:
            cpu["other_configs"] = cpu_baselines_other(bh, synth, oracle,
                                                       max(1.0, args.cpu_seconds / 4))

    traffic = load_traffic()
    for k in kernels:
        if k["kernel"] in traffic:
            k["traffic"] = traffic[k["kernel"]]
    traffic_source = ("profiles/traffic_all_configs.json: rocprofv3 --pmc FETCH_SIZE / "
                      "WRITE_SIZE runs of this bench, copy-calibrated (commands inside)")
    if live_traffic[0] is not None:
        traffic["qk_norm_rope"] = live_traffic[0]
        head["traffic"] = live_traffic[0]
        traffic_source = live_traffic[1]
    elif live:
        traffic_source += f" (live measurement not used: {live_traffic[1]})"
    ms = head["ms"]
    line = {
        "metric": "achieved HBM GB/s (% of 8 TB/s) per fused kernel; rows/s at T=2048",
        "value": head["GBps"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (config distributions, torch RNG on device)",
        "config": {"workload": "config 2: attention pre-block, q/k RMSNorm + IMROPE, "
                               "q [2048,24,256] k [2048,4,256] fp32, n_rot 64, sections "
                               "[11,11,10,0], theta 1e7, pos 0..2047",
                   "tokens": 2048, "head_rows": 2048 * 28},
        "rows_per_s": head["rows_per_s"],
        "roofline": {"bound": "hbm", "achieved": head["GBps"], "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(head["GBps"] / HBM_PEAK_GBS, 4),
                     "traffic": traffic.get("qk_norm_rope"), "traffic_source": traffic_source},
        "cpu_baseline": cpu,
        "kernels": kernels,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
