"""ctypes binding of oracle/liboracle.so (the C restatement in oracle.c).

TEST INFRASTRUCTURE ONLY: the checker the HIP library is compared against.
Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it.

Arrays are numpy; every function returns new arrays.  Each wraps the C
function of the same name, which cites the reference source it restates.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
LIB_PATH = ORACLE_DIR / "liboracle.so"

_vp = ctypes.c_void_p
_sz = ctypes.c_size_t
_f = ctypes.c_float
_i64 = ctypes.c_int64
_i32p = ctypes.POINTER(ctypes.c_int32)

_SIG = {
    "or_half_to_f32": (_f, [ctypes.c_uint16]),
    "or_f32_to_half": (ctypes.c_uint16, [_f]),
    "or_half_to_f32_n": (None, [_vp, _sz, _vp]),
    "or_f32_to_half_n": (None, [_vp, _sz, _vp]),
    "or_silu": (_f, [_f]),
    "or_softplus": (_f, [_f]),
    "or_sigmoid": (_f, [_f]),
    "or_unary": (None, [ctypes.c_int, _vp, _vp, _sz, _vp]),
    "or_rms_norm": (None, [_vp, _sz, _vp, _f, _vp]),
    "or_rms_norm_rows": (ctypes.c_int, [_vp, _sz, _vp, _sz, _sz, _f, _vp]),
    "or_add_rms_norm_rows": (ctypes.c_int, [_vp, _vp, _sz, _vp, _sz, _sz, _f, _vp, _vp]),
    "or_l2_norm_rows": (ctypes.c_int, [_vp, _sz, _sz, _f, _vp]),
    "or_softmax_rows": (ctypes.c_int, [_vp, _sz, _sz, _f, _vp]),
    "or_softmax_rows_ex": (ctypes.c_int, [_vp, _sz, _sz, _f, ctypes.c_int, _vp]),
    "or_rope_imrope": (None, [_vp, _sz, _i64, _i64, _i64, _i64, _sz, _i32p, _f]),
    "or_qk_norm_rope": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz,
                                       _sz, _sz, _sz, _i32p, _f, _f]),
    "or_pq2_row_bytes": (_sz, [_sz]),
    "or_decode_pq2_0_row": (None, [_vp, _sz, _vp]),
    "or_embed_gather": (ctypes.c_int, [_vp, _sz, _sz, _vp, _sz, _vp, _f, _vp, _vp, _vp]),
    "or_gdn_gate_prep": (None, [_vp, _vp, _vp, _vp, _sz, _sz, _vp, _vp]),
    "or_silu_l2_part": (ctypes.c_int, [_vp, _sz, _sz, _sz, _sz, _f, _vp]),
    "or_pq2_row_dot": (_f, [_vp, _sz, _vp]),
    "or_conv1d_silu": (None, [_vp, _vp, _vp, _sz, _sz, _sz, _vp]),
    "or_kv_store": (None, [_vp, _vp, _sz, _sz, _vp, _vp, _sz, ctypes.c_int]),
    "or_attention": (ctypes.c_int, [_vp, _sz, _sz, _vp, _vp, ctypes.c_int, _sz, _sz, _sz, _vp]),
    "or_gdn_step": (None, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz]),
    "or_planar_codebook": (None, [_sz, ctypes.c_uint, _vp]),
    "or_planar_distortion": (ctypes.c_double, [_sz, ctypes.c_uint]),
    "or_planar_givens": (None, [_sz, _vp, _vp]),
    "or_planar_packed_len": (_sz, [_sz, ctypes.c_uint]),
    "or_planar_pack": (None, [_vp, _sz, ctypes.c_uint, _vp]),
    "or_planar_unpack": (None, [_vp, _sz, ctypes.c_uint, _vp]),
    "or_planar_rotate": (None, [_vp, _sz, _vp, _vp, _vp]),
    "or_planar_quantize": (None, [_vp, _sz, ctypes.c_uint, _vp, _vp]),
    "or_planar_dequantize": (None, [_vp, _f, _sz, ctypes.c_uint, _vp]),
    "or_planar_dot_rotated": (_f, [_vp, _vp, _f, _sz, ctypes.c_uint]),
    "or_kv_store_planar": (None, [_vp, _vp, _sz, _sz, _sz, ctypes.c_uint, _vp, _vp, _vp, _vp, _vp,
                                  _sz]),
    "or_attention_planar": (ctypes.c_int, [_vp, _sz, _sz, _vp, _vp, _vp, _vp, _vp, ctypes.c_uint,
                                           _sz, _sz, _sz, _vp]),
    "or_pq2_matmul_n": (None, [_vp, _sz, ctypes.c_uint64, _sz, _vp, _sz, _vp]),
}

_LIB = None


class OracleShapeError(ValueError):
    pass


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise FileNotFoundError(f"{LIB_PATH} missing: run `make -C oracle`")
        h = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIG.items():
            fn = getattr(h, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = h
    return _LIB


def _c(a, dtype=np.float32):
    return np.ascontiguousarray(a, dtype=dtype)


def _p(a):
    return None if a is None else a.ctypes.data


def _sections(s):
    return (ctypes.c_int32 * 4)(*s)


def _st(code: int, what: str):
    if code == -1:
        raise OracleShapeError(what)
    if code == -2:
        raise IndexError(what)


def half_to_f32(h) -> np.ndarray:
    h = _c(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().or_half_to_f32_n(_p(h), h.size, _p(out))
    return out


def f32_to_half(v) -> np.ndarray:
    v = _c(v)
    out = np.empty(v.shape, np.uint16)
    lib().or_f32_to_half_n(_p(v), v.size, _p(out))
    return out


def silu(x: float) -> float:
    return lib().or_silu(x)


def softplus(x: float) -> float:
    return lib().or_softplus(x)


def sigmoid(x: float) -> float:
    return lib().or_sigmoid(x)


def unary(mode: int, a, b=None) -> np.ndarray:
    a = _c(a)
    b = None if b is None else _c(b)
    out = np.empty_like(a)
    lib().or_unary(mode, _p(a), _p(b), a.size, _p(out))
    return out


def rms_norm(x, w, eps: float) -> np.ndarray:
    x, w = _c(x), _c(w)
    out = np.empty_like(x)
    lib().or_rms_norm(_p(x), x.size, _p(w), eps, _p(out))
    return out


def rms_norm_rows(x, w, row_len: int, eps: float) -> np.ndarray:
    x, w = _c(x), _c(w)
    out = np.empty_like(x)
    _st(lib().or_rms_norm_rows(_p(x), x.size, _p(w), w.size, row_len, eps, _p(out)),
        "rms_norm_rows shape")
    return out


def add_rms_norm_rows(x, r, w, row_len: int, eps: float):
    x, r, w = _c(x), _c(r), _c(w)
    s = np.empty_like(x)
    out = np.empty_like(x)
    _st(lib().or_add_rms_norm_rows(_p(x), _p(r), x.size, _p(w), w.size, row_len, eps, _p(s),
                                   _p(out)), "add_rms_norm_rows shape")
    return s, out


def l2_norm_rows(x, row_len: int, eps: float) -> np.ndarray:
    x = _c(x)
    out = np.empty_like(x)
    _st(lib().or_l2_norm_rows(_p(x), x.size, row_len, eps, _p(out)), "l2_norm_rows shape")
    return out


def softmax_rows(x, row_len: int, inv_temp: float = 1.0, sampler_norm: bool = False) -> np.ndarray:
    x = _c(x)
    out = np.empty_like(x)
    if sampler_norm:
        _st(lib().or_softmax_rows_ex(_p(x), x.size, row_len, inv_temp, 1, _p(out)),
            "softmax_rows shape")
    else:
        _st(lib().or_softmax_rows(_p(x), x.size, row_len, inv_temp, _p(out)), "softmax_rows shape")
    return out


def rope_imrope(head, p_t, p_h, p_w, p_e, n_dims, sections, freq_base) -> np.ndarray:
    h = _c(head).copy()
    lib().or_rope_imrope(_p(h), h.size, p_t, p_h, p_w, p_e, n_dims, _sections(sections),
                         freq_base)
    return h


def qk_norm_rope(q, k, wq, wk, pos, n_q_head, n_k_head, head_dim, n_dims, sections,
                 freq_base, eps, q_head_stride=None, want_gate=False):
    q, wq, pos = _c(q), _c(wq), _c(pos, np.int32)
    n_tok = pos.shape[0]
    stride = head_dim if q_head_stride is None else q_head_stride
    q_out = np.empty((n_tok, n_q_head, head_dim), np.float32)
    gate = np.empty_like(q_out) if want_gate else None
    if n_k_head:
        k, wk = _c(k), _c(wk)
        k_out = np.empty((n_tok, n_k_head, head_dim), np.float32)
    else:
        k = wk = k_out = None
    _st(lib().or_qk_norm_rope(_p(q), _p(q_out), _p(gate), _p(k), _p(k_out), _p(wq), _p(wk),
                              _p(pos), n_tok, n_q_head, n_k_head, head_dim, stride, n_dims,
                              _sections(sections), freq_base, eps), "qk_norm_rope shape")
    return q_out, k_out, gate


def pq2_row_bytes(ne0: int) -> int:
    return int(lib().or_pq2_row_bytes(ne0))


def decode_pq2_0_row(raw, ne0: int) -> np.ndarray:
    raw = _c(raw, np.uint8)
    if raw.size < pq2_row_bytes(ne0):
        raise OracleShapeError("raw row too short")
    out = np.empty(ne0, np.float32)
    lib().or_decode_pq2_0_row(_p(raw), ne0, _p(out))
    return out


def embed_gather(table, ne0: int, n_rows: int, tokens, w=None, eps: float = 1e-6):
    table = _c(table, np.uint8)
    tokens = _c(tokens, np.uint32)
    out = np.empty((tokens.size, ne0), np.float32)
    out_norm = np.empty_like(out) if w is not None else None
    wv = _c(w) if w is not None else None
    bad = np.zeros(1, np.uint32)
    _st(lib().or_embed_gather(_p(table), ne0, n_rows, _p(tokens), tokens.size, _p(wv), eps,
                              _p(out), _p(out_norm), _p(bad)),
        f"row {int(bad[0])} out of range (n_rows {n_rows})")
    return (out, out_norm) if w is not None else out


def conv1d_silu(x, state, w):
    """Causal conv1d + SiLU over tokens (src/forward.rs:508-533): x [n_tok, ch],
    state [ch, k-1], w [ch, k] -> (out [n_tok, ch], new state)."""
    x, w = _c(x), _c(w)
    st = _c(state).copy()
    n_tok, ch = x.shape
    k = w.shape[1]
    if w.shape[0] != ch or st.shape != (ch, k - 1) or k < 1 or k > 64:
        raise OracleShapeError("conv1d_silu shape")
    out = np.empty_like(x)
    lib().or_conv1d_silu(_p(x), _p(st), _p(w), n_tok, ch, k, _p(out))
    return out, st


def gdn_step(q, k, v, gate, beta, state):
    """gdn_step (src/gdn.rs:17-77) over tokens: q, k [n_tok, h_k, s]; v
    [n_tok, h_v, s]; gate, beta [n_tok, h_v]; state [h_v, s, s] ->
    (attn [n_tok, h_v, s], new state)."""
    q, k, v, gate, beta = map(_c, (q, k, v, gate, beta))
    st = _c(state).copy()
    n_tok, h_k, s = q.shape
    h_v = v.shape[1]
    if k.shape != q.shape or v.shape != (n_tok, h_v, s) or gate.shape != (n_tok, h_v) or \
            beta.shape != (n_tok, h_v) or st.shape != (h_v, s, s):
        raise OracleShapeError("gdn_step shape")
    attn = np.empty_like(v)
    lib().or_gdn_step(_p(q), _p(k), _p(v), _p(gate), _p(beta), _p(st), _p(attn), n_tok, h_k,
                      h_v, s)
    return attn, st


def kv_store(k, v, k_cache, v_cache, pos0: int):
    """AttnCache::append / append_f16 (src/forward.rs:90-95, 120-125): rows
    k, v [n_tok, n_kv_elems] into copies of the caches [cap, n_kv_elems]
    (float32, or uint16 f16 bits) at positions pos0 ..; returns the copies."""
    k, v = _c(k), _c(v)
    f16 = k_cache.dtype == np.uint16
    kc = np.ascontiguousarray(k_cache).copy()
    vc = np.ascontiguousarray(v_cache).copy()
    n_tok, elems = k.shape
    if v.shape != k.shape or kc.shape != vc.shape or kc.shape[1] != elems or \
            pos0 + n_tok > kc.shape[0] or kc.dtype != vc.dtype:
        raise OracleShapeError("kv_store shape")
    lib().or_kv_store(_p(k), _p(v), n_tok, elems, _p(kc), _p(vc), pos0, int(f16))
    return kc, vc


def attention(q, pos0: int, k_cache, v_cache, n_kv: int):
    """The GQA block of full_attention_layer (src/forward.rs:282-375) for
    queries q [n_q, n_head, hd] at positions pos0 .. pos0 + n_q - 1 over
    caches [>= pos0 + n_q, n_kv * hd] (float32, or uint16 f16 bits);
    returns out [n_q, n_head, hd]."""
    q = _c(q)
    n_q, n_head, hd = q.shape
    f16 = k_cache.dtype == np.uint16
    kc, vc = np.ascontiguousarray(k_cache), np.ascontiguousarray(v_cache)
    if kc.shape != vc.shape or kc.dtype != vc.dtype or kc.shape[1] != n_kv * hd or \
            kc.shape[0] < pos0 + n_q or (f16 is False and kc.dtype != np.float32):
        raise OracleShapeError("attention shape")
    out = np.empty_like(q)
    if lib().or_attention(_p(q), n_q, pos0, _p(kc), _p(vc), int(f16), n_head, n_kv, hd,
                          _p(out)) != 0:
        raise OracleShapeError("attention heads")
    return out


def pq2_row_dot(raw, ne0: int, x) -> float:
    """row_dot_scalar (src/kernels.rs:633-653) of one packed row with x."""
    raw, x = _c(raw, np.uint8), _c(x)
    if raw.size < pq2_row_bytes(ne0) or x.size != ne0:
        raise OracleShapeError("pq2_row_dot shape")
    return float(lib().or_pq2_row_dot(_p(raw), ne0, _p(x)))


def pq2_matmul_n(payload, ne0: int, n_rows: int, x, base_row: int = 0) -> np.ndarray:
    """pq2_matmul_n (src/kernels.rs:340-423): x [n_tok][ne0] -> y [n_tok][n_rows];
    a 1-D x gives pq2_matvec_range's y [n_rows]."""
    payload = _c(payload, np.uint8)
    x = _c(x)
    one = x.ndim == 1
    x2 = x.reshape(1, -1) if one else x
    n_tok = x2.shape[0]
    if x2.shape[1] != ne0 or payload.size < (base_row + n_rows) * pq2_row_bytes(ne0):
        raise OracleShapeError("pq2_matmul_n shape")
    y = np.empty((n_tok, n_rows), np.float32)
    lib().or_pq2_matmul_n(_p(payload), ne0, base_row, n_rows, _p(x2), n_tok, _p(y))
    return y[0] if one else y


def gdn_gate_prep(alpha_raw, dt_bias, ssm_a, beta_raw):
    alpha_raw, dt_bias, ssm_a, beta_raw = map(_c, (alpha_raw, dt_bias, ssm_a, beta_raw))
    n_tok, n_head = alpha_raw.shape
    gate = np.empty_like(alpha_raw)
    beta = np.empty_like(beta_raw)
    lib().or_gdn_gate_prep(_p(alpha_raw), _p(dt_bias), _p(ssm_a), _p(beta_raw), n_tok, n_head,
                           _p(gate), _p(beta))
    return gate, beta


def silu_l2_part(conv, l2_dim: int, head_dim: int, eps: float) -> np.ndarray:
    conv = _c(conv)
    n_tok, conv_dim = conv.shape
    out = np.empty_like(conv)
    _st(lib().or_silu_l2_part(_p(conv), n_tok, conv_dim, l2_dim, head_dim, eps, _p(out)),
        "silu_l2_part shape")
    return out


# ---- planar-quantized KV cache (src/kvquant.rs) ----------------------------

def planar_codebook(d: int, bits: int) -> np.ndarray:
    """codebook (src/kvquant.rs:105-118): 2^bits Lloyd-Max centroids, f32."""
    out = np.empty(1 << bits, np.float32)
    lib().or_planar_codebook(d, bits, _p(out))
    return out


def planar_distortion(d: int, bits: int) -> float:
    """kvquant_expected_distortion (src/kvquant.rs:854-880)."""
    return float(lib().or_planar_distortion(d, bits))


def planar_givens(d: int):
    """givens_table (src/kvquant.rs:124-146): (cos, sin) f32 per pair."""
    n = (d + 1) // 2
    c, s = np.empty(n, np.float32), np.empty(n, np.float32)
    lib().or_planar_givens(d, _p(c), _p(s))
    return c, s


def planar_packed_len(hd: int, bits: int) -> int:
    return int(lib().or_planar_packed_len(hd, bits))


def planar_pack(idx, bits: int) -> np.ndarray:
    idx = _c(idx, np.uint8)
    out = np.empty((idx.size * bits + 7) // 8, np.uint8)
    lib().or_planar_pack(_p(idx), idx.size, bits, _p(out))
    return out


def planar_unpack(packed, n: int, bits: int) -> np.ndarray:
    packed = _c(packed, np.uint8)
    if packed.size < (n * bits + 7) // 8:
        raise OracleShapeError("planar_unpack: packed too short")
    out = np.empty(n, np.uint8)
    lib().or_planar_unpack(_p(packed), n, bits, _p(out))
    return out


def planar_rotate(x) -> np.ndarray:
    """PlanarQuant::rotate (src/kvquant.rs:356-366) with the fixed table."""
    x = _c(x)
    c, s = planar_givens(x.size)
    out = np.empty(x.size + (x.size & 1), np.float32)
    lib().or_planar_rotate(_p(x), x.size, _p(c), _p(s), _p(out))
    return out


def planar_quantize(x, bits: int):
    """PlanarQuant::quantize (src/kvquant.rs:381-396): (packed, norm)."""
    x = _c(x)
    packed = np.empty(planar_packed_len(x.size, bits), np.uint8)
    norm = np.empty(1, np.float32)
    lib().or_planar_quantize(_p(x), x.size, bits, _p(packed), _p(norm))
    return packed, float(norm[0])


def planar_dequantize(packed, norm: float, hd: int, bits: int) -> np.ndarray:
    """PlanarQuant::dequantize (src/kvquant.rs:399-413)."""
    packed = _c(packed, np.uint8)
    out = np.empty(hd, np.float32)
    lib().or_planar_dequantize(_p(packed), norm, hd, bits, _p(out))
    return out


def planar_dot_rotated(q_rot, packed, norm: float, hd: int, bits: int) -> float:
    q_rot, packed = _c(q_rot), _c(packed, np.uint8)
    return float(lib().or_planar_dot_rotated(_p(q_rot), _p(packed), norm, hd, bits))


def kv_store_planar(k, v, n_kv: int, hd: int, bits: int, cap: int, pos0: int = 0,
                    quantize_v: bool = True, caches=None):
    """AttnCache::append_k_quantized / append_v_quantized / append_v
    (src/forward.rs:99-140) for rows k, v [n_tok, n_kv * hd] at positions
    pos0 ..; returns (kq [cap, n_kv, plen] u8, kn [cap, n_kv] f32, vq, vn,
    v_f32 [cap, n_kv * hd]) -- copies of `caches` when given."""
    k, v = _c(k), _c(v)
    n_tok = k.shape[0]
    plen = planar_packed_len(hd, bits)
    if caches is None:
        caches = (np.zeros((cap, n_kv, plen), np.uint8), np.zeros((cap, n_kv), np.float32),
                  np.zeros((cap, n_kv, plen), np.uint8), np.zeros((cap, n_kv), np.float32),
                  np.zeros((cap, n_kv * hd), np.float32))
    kq, kn, vq, vn, vf = (np.ascontiguousarray(a).copy() for a in caches)
    if k.shape != (n_tok, n_kv * hd) or v.shape != k.shape or pos0 + n_tok > kq.shape[0]:
        raise OracleShapeError("kv_store_planar shape")
    lib().or_kv_store_planar(_p(k), _p(v), n_tok, n_kv, hd, bits, _p(kq), _p(kn),
                             _p(vq) if quantize_v else None, _p(vn) if quantize_v else None,
                             _p(vf), pos0)
    return kq, kn, vq, vn, vf


def attention_planar(q, pos0: int, kq, kn, vq, vn, v_f32, n_kv: int, bits: int,
                     quantize_v: bool = True) -> np.ndarray:
    """The quantized-cache branches of full_attention_layer
    (src/forward.rs:296-349) for queries q [n_q, n_head, hd] at positions
    pos0 ..; V from vq / vn when quantize_v, else from v_f32."""
    q = _c(q)
    n_q, n_head, hd = q.shape
    kq, kn = _c(kq, np.uint8), _c(kn)
    vq, vn, vf = _c(vq, np.uint8), _c(vn), _c(v_f32)
    out = np.empty_like(q)
    if lib().or_attention_planar(_p(q), n_q, pos0, _p(kq), _p(kn), _p(vq) if quantize_v else None,
                                 _p(vn) if quantize_v else None, _p(vf), bits, n_head, n_kv, hd,
                                 _p(out)) != 0:
        raise OracleShapeError("attention_planar heads")
    return out
