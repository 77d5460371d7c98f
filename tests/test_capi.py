"""C-ABI checks that need no GPU: the library loads, exports every symbol the
header declares, and rejects bad shapes with the reference's error text
before it touches the device (src/kernels.rs:97-109, 126-131, 175-180;
src/weights.rs:337-341)."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest


def test_library_exports_every_header_symbol(bh):
    lib = bh.lib()
    names = bh.header_symbols()
    assert len(names) == 41
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # and the Python binding declares a signature for each of them
    assert sorted(bh._SIGNATURES) == names


def test_version_and_row_bytes(bh):
    assert b"gfx950" in bh.lib().bh_version()
    assert bh.pq2_row_bytes(5120) == 1360
    assert bh.pq2_row_bytes(128) == 34
    assert bh.pq2_row_bytes(129) == 68
    assert bh.pq2_row_bytes(0) == 0


def test_rms_norm_rows_shape_errors(bh):
    lib = bh.lib()
    st = lib.bh_rms_norm_rows(None, 8, None, 2, 4, 1e-6, None, None)
    assert st == bh.BH_ERR_SHAPE
    assert bh.last_error() == "rms_norm_rows: weight len 2 != row_len 4"
    st = lib.bh_rms_norm_rows(None, 8, None, 3, 3, 1e-6, None, None)
    assert st == bh.BH_ERR_SHAPE
    assert bh.last_error() == "rms_norm_rows: x len 8 not divisible by row_len 3"
    # row_len 0 is an error, not a division by zero
    assert lib.bh_rms_norm_rows(None, 8, None, 0, 0, 1e-6, None, None) == bh.BH_ERR_SHAPE
    # empty input is fine and touches nothing
    assert lib.bh_rms_norm_rows(None, 0, None, 4, 4, 1e-6, None, None) == bh.BH_OK
    assert bh.last_error() == ""


def test_host_mirror_shape_errors_match(bh):
    lib = bh.lib()
    x = (ctypes.c_float * 8)()
    w = (ctypes.c_float * 2)()
    assert lib.bh_host_rms_norm_rows(x, 8, w, 2, 4, 1e-6, x) == bh.BH_ERR_SHAPE
    assert bh.last_error() == "rms_norm_rows: weight len 2 != row_len 4"
    assert lib.bh_host_l2_norm_rows(x, 8, 3, 1e-12, x) == bh.BH_ERR_SHAPE
    assert bh.last_error() == "l2_norm_rows: x len 8 not divisible by row_len 3"
    assert lib.bh_host_softmax_rows(x, 8, 3, x) == bh.BH_ERR_SHAPE
    assert bh.last_error() == "softmax_rows: x len 8 not divisible by row_len 3"
    assert lib.bh_host_map_inplace(x, 8, 7) == bh.BH_ERR_ARG


def test_other_shape_errors(bh):
    lib = bh.lib()
    assert lib.bh_l2_norm_rows(None, 10, 4, 1e-6, None, None) == bh.BH_ERR_SHAPE
    assert lib.bh_silu_l2_norm_rows(None, 10, 4, 1e-6, None, None) == bh.BH_ERR_SHAPE
    assert lib.bh_softmax_rows(None, 10, 4, 1.0, None, None) == bh.BH_ERR_SHAPE
    assert lib.bh_add_rms_norm_rows(None, None, 8, None, 3, 4, 1e-6, None, None,
                                    None) == bh.BH_ERR_SHAPE
    assert lib.bh_unary(9, None, None, 4, None, None) == bh.BH_ERR_ARG
    assert bh.last_error().startswith("unary: unknown mode")
    assert lib.bh_unary(bh.BH_SILU_MUL, None, None, 4, None, None) == bh.BH_ERR_ARG
    assert lib.bh_pq2_embed_gather_rms(None, 5120, 10, None, 4, None, 5000, 1e-6, None, None,
                                       None, None) == bh.BH_ERR_SHAPE
    assert bh.last_error() == "pq2_embed_gather_rms: weight len 5000 != ne0 5120"
    assert lib.bh_qk_norm_rope(None, None) == bh.BH_ERR_ARG


def test_rope_argument_errors(bh):
    lib = bh.lib()
    sec = (ctypes.c_int32 * 4)(11, 11, 10, 0)
    head = (ctypes.c_float * 8)()
    assert lib.bh_host_rope_imrope(head, 8, 0, 0, 0, 0, 3, sec, 1e7) == bh.BH_ERR_SHAPE
    assert lib.bh_host_rope_imrope(head, 8, 0, 0, 0, 0, 10, sec, 1e7) == bh.BH_ERR_SHAPE
    zero = (ctypes.c_int32 * 4)(0, 0, 0, 0)
    assert lib.bh_rope_imrope(None, 1, 1, 8, None, 4, zero, 1e7, None) == bh.BH_ERR_ARG
    args = bh.make_qk_args(None, None, None, None, None, None, None, 1, 1, 0, head_dim=256,
                           q_head_stride=256)
    args.gate_out = 16  # any non-NULL value: rejected before use
    assert lib.bh_qk_norm_rope(ctypes.byref(args), None) == bh.BH_ERR_SHAPE
    assert "gate_out needs q_head_stride" in bh.last_error()


def test_gdn_prep_argument_errors(bh):
    lib = bh.lib()
    a = bh.make_gdn_args(conv=None, conv_out=None, n_tok=1, conv_dim=512, l2_dim=200,
                         head_dim=128)
    a.conv_out = 16
    assert lib.bh_gdn_prep_fused(ctypes.byref(a), None) == bh.BH_ERR_SHAPE
    b = bh.make_gdn_args(n_tok=1, gate_mode=bh.BH_SILU)
    assert lib.bh_gdn_prep_fused(ctypes.byref(b), None) == bh.BH_ERR_ARG


def test_batch_embed_range_error_text(bh, synth):
    """src/weights.rs:337-341: the first out-of-range token is reported."""
    lib = bh.lib()
    table = synth.pq2_table(synth.Rng(1), 4, 256)
    toks = np.array([0, 4, 9], np.uint32)
    out = np.empty((3, 256), np.float32)
    st = lib.bh_host_batch_embed(table.ctypes.data, table.size, 256, 4, toks.ctypes.data, 3,
                                 out.ctypes.data)
    assert st == bh.BH_ERR_RANGE
    assert bh.last_error() == ("Weights: row_f32(token_embd.weight): row 4 out of range "
                               "(n_rows 4)")
    assert lib.bh_host_decode_pq2_0_row(table.ctypes.data, 10, 256, out.ctypes.data) == \
        bh.BH_ERR_SHAPE


def test_pq2_product_shape_errors(bh):
    """src/kernels.rs:239-256, 291-307, 349-364: the reference's Err texts,
    returned before any device work (the pointers are never read)."""
    lib = bh.lib()
    dummy = ctypes.c_void_p(16)
    # device entry points
    assert lib.bh_pq2_matvec_range(dummy, 1360, 5120, 0, 1, dummy, 5119, dummy, 1, None) == \
        bh.BH_ERR_SHAPE
    assert bh.last_error() == "pq2_matvec_range: x length 5119 != ne0 5120"
    assert lib.bh_pq2_matvec_range(dummy, 1360 * 4, 5120, 0, 4, dummy, 5120, dummy, 3, None) == \
        bh.BH_ERR_SHAPE
    assert bh.last_error() == "pq2_matvec_range: y too small"
    assert lib.bh_pq2_matvec_range(dummy, 1360 * 4, 5120, 2, 3, dummy, 5120, dummy, 3, None) == \
        bh.BH_ERR_SHAPE
    assert bh.last_error() == "pq2_matvec_range: rows 2..5 need 6800 bytes, payload is 5440"
    assert lib.bh_pq2_matvec_range(dummy, 1360, 5120, 2**63, 2**62, dummy, 5120, dummy,
                                   2**62, None) == bh.BH_ERR_SHAPE
    assert bh.last_error() == "pq2_matvec_range: row range byte length overflows"
    assert lib.bh_pq2_matmul_n(dummy, 68 * 12, 256, 0, 12, dummy, 767, 3, dummy, 36, None) == \
        bh.BH_ERR_SHAPE
    assert bh.last_error() == "pq2_matmul_n: x length 767 != n_tok 3 * ne0 256"
    assert lib.bh_pq2_matmul_n(dummy, 68 * 12, 256, 0, 12, dummy, 768, 3, dummy, 35, None) == \
        bh.BH_ERR_SHAPE
    assert bh.last_error() == "pq2_matmul_n: y too small"
    assert lib.bh_pq2_matmul_n(dummy, 68 * 12, 256, 1, 12, dummy, 768, 3, dummy, 36, None) == \
        bh.BH_ERR_SHAPE
    assert bh.last_error() == "pq2_matmul_n: row range exceeds payload"
    assert lib.bh_pq2_matmul_n(dummy, 68, 256, 2**63, 2**62, dummy, 256, 1, dummy, 2**62,
                               None) == bh.BH_ERR_SHAPE
    assert bh.last_error() == "pq2_matmul_n: overflow"
    # empty ranges succeed without touching anything
    assert lib.bh_pq2_matvec_range(None, 0, 5120, 0, 0, None, 5120, None, 0, None) == bh.BH_OK
    assert lib.bh_pq2_matmul_n(None, 0, 256, 0, 0, None, 0, 0, None, 0, None) == bh.BH_OK
    # host mirrors: same texts, dot_pq2_0_row's own
    raw = np.zeros(1360 * 2, np.uint8)
    x = np.zeros(5120, np.float32)
    out = np.zeros(4, np.float32)
    assert lib.bh_host_dot_pq2_0_row(raw.ctypes.data, raw.size, 5120, 0, x.ctypes.data, 5000,
                                     out.ctypes.data) == bh.BH_ERR_SHAPE
    assert bh.last_error() == "dot_pq2_0_row: x length 5000 != ne0 5120"
    assert lib.bh_host_dot_pq2_0_row(raw.ctypes.data, raw.size, 5120, 2, x.ctypes.data, 5120,
                                     out.ctypes.data) == bh.BH_ERR_SHAPE
    assert bh.last_error() == "dot_pq2_0_row: row 2 needs bytes 2720..4080, payload is 2720"
    assert lib.bh_host_pq2_matvec_range(raw.ctypes.data, raw.size, 5120, 1, 2, x.ctypes.data,
                                        5120, out.ctypes.data, 4) == bh.BH_ERR_SHAPE
    assert bh.last_error() == "pq2_matvec_range: rows 1..3 need 4080 bytes, payload is 2720"
    assert lib.bh_host_pq2_matmul_n(raw.ctypes.data, raw.size, 5120, 0, 2, x.ctypes.data, 5120,
                                    2, out.ctypes.data, 4) == bh.BH_ERR_SHAPE
    assert bh.last_error() == "pq2_matmul_n: x length 5120 != n_tok 2 * ne0 5120"


def test_conv1d_argument_errors(bh):
    """bh_conv1d_silu rejects a bad tap count, a missing cache and an output
    aliasing the input before touching the device."""
    lib = bh.lib()
    d = ctypes.c_void_p(64)
    assert lib.bh_conv1d_silu(d, d, d, 4, 16, 0, ctypes.c_void_p(128), None) == bh.BH_ERR_SHAPE
    assert "conv kernel size 0" in bh.last_error()
    assert lib.bh_conv1d_silu(d, d, d, 4, 16, 65, ctypes.c_void_p(128), None) == bh.BH_ERR_SHAPE
    assert lib.bh_conv1d_silu(d, None, d, 4, 16, 4, ctypes.c_void_p(128), None) == bh.BH_ERR_ARG
    assert lib.bh_conv1d_silu(d, d, d, 4, 16, 4, d, None) == bh.BH_ERR_ARG
    assert "must not alias" in bh.last_error()
    assert lib.bh_conv1d_silu(None, None, None, 0, 16, 4, None, None) == bh.BH_OK


def test_splitmix64_known_vector(synth):
    """SplitMix64 with seed 0: the published first outputs."""
    out = synth.splitmix64(0, 0, 3)
    assert [int(v) for v in out] == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4,
                                     0x06C45D188009454F]
    r = synth.Rng(0)
    assert int(r.u64(2)[1]) == 0x6E789E6AA1B965F4
    assert int(r.u64(1)[0]) == 0x06C45D188009454F


def test_synth_normal_moments(synth):
    x = synth.Rng(42).normal(200000, 1.0, 0.1)
    assert x.dtype == np.float32
    assert abs(x.mean() - 1.0) < 2e-3 and abs(x.std() - 0.1) < 2e-3


def test_pq2_pack_roundtrip(oracle, synth):
    rng = np.random.default_rng(0)
    codes = rng.integers(0, 4, size=(3, 300), dtype=np.uint8)
    sc = synth.f32_to_half(np.abs(rng.standard_normal(9)).astype(np.float32) * 0.02)
    packed = synth.pack_pq2_rows(codes, sc.reshape(3, 3))
    assert packed.shape == (3, oracle.pq2_row_bytes(300))
    scale = oracle.half_to_f32(sc).reshape(3, 3)
    for r in range(3):
        v = oracle.decode_pq2_0_row(packed[r], 300)
        expect = (codes[r].astype(np.float32) - 1) * np.repeat(scale[r], 128)[:300]
        assert np.array_equal(v, expect)


def test_pq2_table_distribution(oracle, synth):
    t = synth.pq2_table(synth.Rng(5), 64, 5120)
    v = np.stack([oracle.decode_pq2_0_row(t[r], 5120) for r in range(64)])
    sc = oracle.half_to_f32(t.reshape(64, 40, 34)[:, :, :2].copy().view(np.uint16)[..., 0])
    codes = np.round(v / np.repeat(sc, 128, axis=1)) + 1
    frac = [(codes == c).mean() for c in (0, 1, 2)]
    assert all(abs(f - p) < 0.01 for f, p in zip(frac, (0.3, 0.4, 0.3)))
    assert abs(np.abs(sc).mean() - 0.02 * np.sqrt(2 / np.pi)) < 5e-4


def test_gdn_step_argument_errors(bh):
    """bh_gdn_step checks shapes and pointers before touching the device;
    zero tokens is a no-op."""
    lib = bh.lib()
    assert lib.bh_gdn_step(None, None, None, None, None, None, None, 0, 16, 48, 128, None) == 0
    assert lib.bh_gdn_step(None, None, None, None, None, None, None, 1, 0, 48, 128,
                           None) == bh.BH_ERR_SHAPE
    assert bh.last_error() == "gdn_step: h_k, h_v and s must be positive"
    assert lib.bh_gdn_step(None, None, None, None, None, None, None, 1, 16, 48, 128,
                           None) == bh.BH_ERR_ARG
    assert bh.last_error() == "gdn_step: null pointer"


def test_host_gdn_step_short_slices(bh):
    """bh_host_gdn_step names the first short slice before any device work."""
    lib = bh.lib()
    need = dict(q=2048, k=2048, v=6144, gate=48, beta=48, state=48 * 128 * 128, attn=6144)
    for short in need:
        lens = [need[n] - (n == short) for n in need]
        args = []
        for ln in lens:
            args += [None, ln]
        assert lib.bh_host_gdn_step(*args) == bh.BH_ERR_SHAPE
        assert bh.last_error() == f"gdn_step: {short} len {need[short] - 1} < {need[short]}"


def test_attention_argument_errors(bh):
    lib = bh.lib()
    assert lib.bh_attention(None, 0, 0, None, None, 0, 24, 4, 256, None, None) == 0
    assert lib.bh_attention(None, 1, 0, None, None, 0, 24, 5, 256, None, None) == bh.BH_ERR_SHAPE
    assert "multiple of n_kv 5" in bh.last_error()
    assert lib.bh_attention(None, 1, 0, None, None, 2, 24, 4, 256, None, None) == bh.BH_ERR_ARG
    assert lib.bh_attention(None, 1, 0, None, None, 0, 24, 4, 256, None, None) == bh.BH_ERR_ARG
    assert bh.last_error() == "attention: null pointer"
    assert lib.bh_kv_store(None, None, 0, 1024, None, None, 0, 1, None) == 0
    assert lib.bh_kv_store(None, None, 1, 1024, None, None, 0, 1, None) == bh.BH_ERR_ARG
    assert lib.bh_kv_store(None, None, 1, 1024, None, None, 0, 7, None) == bh.BH_ERR_ARG


def test_host_byte_ranges_do_not_wrap(bh):
    """Sizes whose byte products overflow 64 bits are shape errors, not a
    wrapped length that passes the payload check (the reference's slice
    indexing would panic instead of reading past the buffer)."""
    lib = bh.lib()
    table = np.zeros(34 * 4, np.uint8)
    toks = np.zeros(1, np.uint32)
    out = np.empty(128, np.float32)
    huge = (1 << 64) // 34 + 1  # huge * 34 wraps to a small number
    st = lib.bh_host_batch_embed(table.ctypes.data, table.size, 128, huge, toks.ctypes.data, 1,
                                 out.ctypes.data)
    assert st == bh.BH_ERR_SHAPE and "overflows" in bh.last_error()
    x = np.zeros(128, np.float32)
    y = np.zeros(1, np.float32)
    st = lib.bh_host_dot_pq2_0_row(table.ctypes.data, table.size, 128, huge, x.ctypes.data, 128,
                                   y.ctypes.data)
    assert st == bh.BH_ERR_SHAPE and "overflows" in bh.last_error()
    # an ordinary out-of-payload row keeps the reference's text
    st = lib.bh_host_dot_pq2_0_row(table.ctypes.data, table.size, 128, 4, x.ctypes.data, 128,
                                   y.ctypes.data)
    assert st == bh.BH_ERR_SHAPE
    assert bh.last_error() == "dot_pq2_0_row: row 4 needs bytes 136..170, payload is 136"


def test_attention_scratch_size_does_not_wrap(bh):
    """n_q * n_head * n_max * 4 above 2^64 is rejected before any allocation
    (generic path: hd 64 is not the decode path's head size)."""
    lib = bh.lib()
    p = ctypes.c_void_p(16)  # never dereferenced: the call fails on the size first
    st = lib.bh_attention(p, 65535, (1 << 40) - 65535, p, p, 0, 65535, 1, 64, p, None)
    assert st == bh.BH_ERR_SHAPE and "overflows" in bh.last_error()


def test_rust_ffi_matches_header(bh):
    """rust/src/hip/mod.rs (the reference-side binding) declares only entry
    points the header has, each with the header's parameter count."""
    import re
    from pathlib import Path
    root = Path(__file__).resolve().parent.parent
    rs = (root / "rust" / "src" / "hip" / "mod.rs").read_text()
    hdr = re.sub(r"/\*.*?\*/", "", (root / "include" / "bonsai_hip.h").read_text(), flags=re.S)
    c_params = {}
    for m in re.finditer(r"\b(?:int|const char \*|size_t)\s*\**\s*(bh_\w+)\s*\(([^)]*)\)\s*;", hdr):
        args = m.group(2).strip()
        c_params[m.group(1)] = 0 if args in ("", "void") else args.count(",") + 1
    ext = rs[rs.index('extern "C"'):]
    ext = ext[:ext.index("\n}\n")]
    found = 0
    for m in re.finditer(r"fn (bh_\w+)\(([^)]*)\)", ext):
        name, args = m.group(1), m.group(2).strip()
        n = 0 if not args else args.rstrip(",").count(",") + 1
        assert name in c_params, name
        assert n == c_params[name], (name, n, c_params[name])
        found += 1
    assert found >= 20
