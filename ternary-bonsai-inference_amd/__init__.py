"""Python binding of the bonsai HIP library (ctypes over the C ABI).

The product is lib/libbonsai_hip.so with the C ABI of include/bonsai_hip.h;
this module only loads it and offers torch-tensor conveniences for tests and
benchmarks (torch provides device memory and streams; every computation runs
in the library's HIP kernels).  There is no CPU fallback: if the library is
missing, `lib()` raises.

The package directory name contains dashes, so import it by path:

    spec = importlib.util.spec_from_file_location(
        "bonsai_amd", "ternary-bonsai-inference_amd/__init__.py")
"""
from __future__ import annotations

import ctypes
import os
import re
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
LIB_PATH = PKG_DIR / "lib" / "libbonsai_hip.so"
HEADER_PATH = REPO_DIR / "include" / "bonsai_hip.h"

BH_OK = 0
BH_ERR_SHAPE = -1
BH_ERR_RANGE = -2
BH_ERR_HIP = -3
BH_ERR_ARG = -4

BH_SILU = 0
BH_SIGMOID = 1
BH_SOFTPLUS = 2
BH_SILU_MUL = 3
BH_SIGMOID_MUL = 4

BH_SOFTMAX_SAMPLER_NORM = 1  # bh_softmax_rows_ex flag

# Ternary-Bonsai-27B constants (reference src/gdev.rs:21-37, src/weights.rs:42-62)
N_EMBD = 5120
N_HEAD = 24
N_HEAD_KV = 4
HEAD_DIM = 256
N_ROT = 64
SECTIONS = (11, 11, 10, 0)
FREQ_BASE = 1e7
EPS = 1e-6
N_VOCAB = 248320
GDN_HV = 48
GDN_STATE = 128

_c_size = ctypes.c_size_t
_c_float = ctypes.c_float
_c_int = ctypes.c_int
_vp = ctypes.c_void_p


class BonsaiError(RuntimeError):
    """A non-zero status from the library, with bh_last_error()'s message."""

    def __init__(self, status: int, message: str):
        super().__init__(f"status {status}: {message}")
        self.status = status
        self.message = message


class GdnPrepArgs(ctypes.Structure):
    """bh_gdn_prep_args (include/bonsai_hip.h)."""

    _fields_ = [
        ("conv", _vp), ("conv_out", _vp), ("z", _vp), ("y", _vp), ("gated_out", _vp),
        ("alpha_raw", _vp), ("dt_bias", _vp), ("ssm_a", _vp), ("beta_raw", _vp),
        ("gate_out", _vp), ("beta_out", _vp),
        ("n_tok", _c_size), ("conv_dim", _c_size), ("l2_dim", _c_size), ("head_dim", _c_size),
        ("inner_dim", _c_size), ("n_v_head", _c_size), ("gate_mode", _c_int), ("eps", _c_float),
        ("conv_w", _vp), ("conv_state", _vp), ("conv_k", _c_size),
    ]


class QkNormRopeArgs(ctypes.Structure):
    """bh_qk_norm_rope_args (include/bonsai_hip.h)."""

    _fields_ = [
        ("q", _vp), ("q_out", _vp), ("gate_out", _vp), ("k", _vp), ("k_out", _vp),
        ("wq", _vp), ("wk", _vp), ("pos", _vp),
        ("n_tok", _c_size), ("n_q_head", _c_size), ("n_k_head", _c_size), ("head_dim", _c_size),
        ("q_head_stride", _c_size), ("n_dims", _c_size),
        ("sections", ctypes.c_int32 * 4), ("freq_base", _c_float), ("eps", _c_float),
    ]


_SIGNATURES = {
    "bh_last_error": (ctypes.c_char_p, []),
    "bh_version": (ctypes.c_char_p, []),
    "bh_scratch_retired_bytes": (ctypes.c_size_t, []),
    "bh_scratch_release": (_c_int, []),
    "bh_pq2_row_bytes": (_c_size, [_c_size]),
    "bh_rms_norm": (_c_int, [_vp, _vp, _c_size, _c_float, _vp, _vp]),
    "bh_rms_norm_rows": (_c_int, [_vp, _c_size, _vp, _c_size, _c_size, _c_float, _vp, _vp]),
    "bh_add_rms_norm_rows": (_c_int, [_vp, _vp, _c_size, _vp, _c_size, _c_size, _c_float, _vp,
                                      _vp, _vp]),
    "bh_l2_norm_rows": (_c_int, [_vp, _c_size, _c_size, _c_float, _vp, _vp]),
    "bh_silu_l2_norm_rows": (_c_int, [_vp, _c_size, _c_size, _c_float, _vp, _vp]),
    "bh_unary": (_c_int, [_c_int, _vp, _vp, _c_size, _vp, _vp]),
    "bh_gdn_gate_prep": (_c_int, [_vp, _vp, _vp, _vp, _c_size, _c_size, _vp, _vp, _vp]),
    "bh_gdn_prep_fused": (_c_int, [ctypes.POINTER(GdnPrepArgs), _vp]),
    "bh_softmax_rows": (_c_int, [_vp, _c_size, _c_size, _c_float, _vp, _vp]),
    "bh_softmax_rows_noalloc": (_c_int, [_vp, _c_size, _c_size, _c_float, _vp, _vp]),
    "bh_softmax_rows_ex": (_c_int, [_vp, _c_size, _c_size, _c_float, _c_int, _vp, _vp]),
    "bh_rope_imrope": (_c_int, [_vp, _c_size, _c_size, _c_size, _vp, _c_size,
                                ctypes.POINTER(ctypes.c_int32), _c_float, _vp]),
    "bh_qk_norm_rope": (_c_int, [ctypes.POINTER(QkNormRopeArgs), _vp]),
    "bh_pq2_embed_gather": (_c_int, [_vp, _c_size, _c_size, _vp, _c_size, _vp, _vp, _vp]),
    "bh_pq2_embed_gather_rms": (_c_int, [_vp, _c_size, _c_size, _vp, _c_size, _vp, _c_size,
                                         _c_float, _vp, _vp, _vp, _vp]),
    "bh_host_rms_norm": (_c_int, [_vp, _c_size, _vp, _c_float, _vp]),
    "bh_host_rms_norm_rows": (_c_int, [_vp, _c_size, _vp, _c_size, _c_size, _c_float, _vp]),
    "bh_host_l2_norm_rows": (_c_int, [_vp, _c_size, _c_size, _c_float, _vp]),
    "bh_host_map_inplace": (_c_int, [_vp, _c_size, _c_int]),
    "bh_host_softmax_rows": (_c_int, [_vp, _c_size, _c_size, _vp]),
    "bh_host_rope_imrope": (_c_int, [_vp, _c_size, ctypes.c_int64, ctypes.c_int64,
                                     ctypes.c_int64, ctypes.c_int64, _c_size,
                                     ctypes.POINTER(ctypes.c_int32), _c_float]),
    "bh_host_decode_pq2_0_row": (_c_int, [_vp, _c_size, _c_size, _vp]),
    "bh_host_batch_embed": (_c_int, [_vp, _c_size, _c_size, _c_size, _vp, _c_size, _vp]),
    "bh_conv1d_silu": (_c_int, [_vp, _vp, _vp, _c_size, _c_size, _c_size, _vp, _vp]),
    "bh_host_gdn_step": (_c_int, [_vp, _c_size, _vp, _c_size, _vp, _c_size, _vp, _c_size, _vp,
                                  _c_size, _vp, _c_size, _vp, _c_size]),
    "bh_kv_store": (_c_int, [_vp, _vp, _c_size, _c_size, _vp, _vp, _c_size, _c_int, _vp]),
    "bh_attention": (_c_int, [_vp, _c_size, _c_size, _vp, _vp, _c_int, _c_size, _c_size, _c_size,
                              _vp, _vp]),
    "bh_gdn_step": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_size, _c_size, _c_size,
                             _c_size, _vp]),
    "bh_planar_packed_len": (_c_size, [_c_size, ctypes.c_uint]),
    "bh_kv_store_planar": (_c_int, [_vp, _vp, _c_size, _c_size, _c_size, ctypes.c_uint, _vp, _vp,
                                    _vp, _vp, _vp, _c_size, _vp]),
    "bh_attention_planar": (_c_int, [_vp, _c_size, _c_size, _vp, _vp, _vp, _vp, _vp,
                                     ctypes.c_uint, _c_size, _c_size, _c_size, _vp, _vp]),
    "bh_pq2_matvec_range": (_c_int, [_vp, _c_size, _c_size, ctypes.c_uint64, _c_size, _vp,
                                     _c_size, _vp, _c_size, _vp]),
    "bh_pq2_matmul_n": (_c_int, [_vp, _c_size, _c_size, ctypes.c_uint64, _c_size, _vp, _c_size,
                                 _c_size, _vp, _c_size, _vp]),
    "bh_host_dot_pq2_0_row": (_c_int, [_vp, _c_size, _c_size, ctypes.c_uint64, _vp, _c_size,
                                       _vp]),
    "bh_host_pq2_matvec_range": (_c_int, [_vp, _c_size, _c_size, ctypes.c_uint64, _c_size, _vp,
                                          _c_size, _vp, _c_size]),
    "bh_host_pq2_matmul_n": (_c_int, [_vp, _c_size, _c_size, ctypes.c_uint64, _c_size, _vp,
                                      _c_size, _c_size, _vp, _c_size]),
}

_LIB = None


def header_symbols() -> list[str]:
    """Every function name declared in include/bonsai_hip.h."""
    text = HEADER_PATH.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(bh_[a-z0-9_]+)\s*\(", text)))


def lib() -> ctypes.CDLL:
    """Load lib/libbonsai_hip.so (raises if it has not been built)."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        raise FileNotFoundError(
            f"{LIB_PATH} is missing: run __graft_entry__.build() (hipcc for gfx950) first")
    try:  # share torch's HIP runtime when torch is present (same soname)
        import torch  # noqa: F401
    except ImportError:
        pass
    handle = ctypes.CDLL(str(LIB_PATH), mode=ctypes.RTLD_LOCAL)
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = handle
    return handle


def last_error() -> str:
    return lib().bh_last_error().decode()


def check(status: int) -> None:
    if status != BH_OK:
        raise BonsaiError(status, last_error())


def pq2_row_bytes(ne0: int) -> int:
    return int(lib().bh_pq2_row_bytes(ne0))


# ---------------------------------------------------------------------------
# torch-tensor conveniences (device tensors, current torch stream)
# ---------------------------------------------------------------------------

def _ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(stream=None) -> int:
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


def _f32(t, name: str):
    import torch
    if t.dtype != torch.float32 or not t.is_cuda or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous float32 CUDA tensor")
    return t


def rms_norm_rows(x, w, eps: float = EPS, out=None, stream=None):
    import torch
    _f32(x, "x"), _f32(w, "w")
    out = torch.empty_like(x) if out is None else out
    check(lib().bh_rms_norm_rows(x.data_ptr(), x.numel(), w.data_ptr(), w.numel(), w.numel(),
                                 eps, out.data_ptr(), _stream(stream)))
    return out


def add_rms_norm_rows(x, residual, w, eps: float = EPS, sum_out=None, out=None, stream=None):
    import torch
    sum_out = torch.empty_like(x) if sum_out is None else sum_out
    out = torch.empty_like(x) if out is None else out
    check(lib().bh_add_rms_norm_rows(x.data_ptr(), residual.data_ptr(), x.numel(), w.data_ptr(),
                                     w.numel(), w.numel(), eps, sum_out.data_ptr(),
                                     out.data_ptr(), _stream(stream)))
    return sum_out, out


def l2_norm_rows(x, row_len: int, eps: float = EPS, out=None, silu_first=False, stream=None):
    import torch
    _f32(x, "x")
    out = torch.empty_like(x) if out is None else out
    fn = lib().bh_silu_l2_norm_rows if silu_first else lib().bh_l2_norm_rows
    check(fn(x.data_ptr(), x.numel(), row_len, eps, out.data_ptr(), _stream(stream)))
    return out


def unary(mode: int, a, b=None, out=None, stream=None):
    import torch
    out = torch.empty_like(a) if out is None else out
    check(lib().bh_unary(mode, a.data_ptr(), _ptr(b), a.numel(), out.data_ptr(),
                         _stream(stream)))
    return out


def softmax_rows(x, row_len: int, inv_temp: float = 1.0, out=None, stream=None,
                 noalloc: bool = False, sampler_norm: bool = False):
    """bh_softmax_rows; with noalloc=True bh_softmax_rows_noalloc (fixed
    library scratch, no device allocation by the library); with
    sampler_norm=True bh_softmax_rows_ex(BH_SOFTMAX_SAMPLER_NORM), the
    sampler's f64 normalisation (src/sampler.rs:118-126)."""
    import torch
    _f32(x, "x")
    if noalloc and sampler_norm:
        raise ValueError("softmax_rows: noalloc has no sampler normalisation")
    out = torch.empty_like(x) if out is None else out
    if sampler_norm:
        check(lib().bh_softmax_rows_ex(x.data_ptr(), x.numel(), row_len, inv_temp,
                                       BH_SOFTMAX_SAMPLER_NORM, out.data_ptr(), _stream(stream)))
        return out
    fn = lib().bh_softmax_rows_noalloc if noalloc else lib().bh_softmax_rows
    check(fn(x.data_ptr(), x.numel(), row_len, inv_temp, out.data_ptr(), _stream(stream)))
    return out


def gdn_gate_prep(alpha_raw, dt_bias, ssm_a, beta_raw, stream=None):
    import torch
    n_tok, n_head = alpha_raw.shape
    gate = torch.empty_like(alpha_raw)
    beta = torch.empty_like(beta_raw)
    check(lib().bh_gdn_gate_prep(alpha_raw.data_ptr(), dt_bias.data_ptr(), ssm_a.data_ptr(),
                                 beta_raw.data_ptr(), n_tok, n_head, gate.data_ptr(),
                                 beta.data_ptr(), _stream(stream)))
    return gate, beta


def make_gdn_args(conv=None, conv_out=None, z=None, y=None, gated_out=None, alpha_raw=None,
                  dt_bias=None, ssm_a=None, beta_raw=None, gate_out=None, beta_out=None,
                  n_tok=0, conv_dim=0, l2_dim=0, head_dim=GDN_STATE, inner_dim=0,
                  n_v_head=0, gate_mode=BH_SILU_MUL, eps=EPS, conv_w=None, conv_state=None,
                  conv_k=0) -> GdnPrepArgs:
    """With conv_w (and conv_state, conv_k), `conv` is the raw qkv and the
    causal conv1d runs in front of the SiLU (src/forward.rs:508-533)."""
    return GdnPrepArgs(_ptr(conv), _ptr(conv_out), _ptr(z), _ptr(y), _ptr(gated_out),
                       _ptr(alpha_raw), _ptr(dt_bias), _ptr(ssm_a), _ptr(beta_raw),
                       _ptr(gate_out), _ptr(beta_out), n_tok, conv_dim, l2_dim, head_dim,
                       inner_dim, n_v_head, gate_mode, eps, _ptr(conv_w), _ptr(conv_state),
                       conv_k if conv_w is not None else 0)


def gdn_prep_fused(args: GdnPrepArgs, stream=None) -> None:
    check(lib().bh_gdn_prep_fused(ctypes.byref(args), _stream(stream)))


def make_qk_args(q, q_out, k, k_out, wq, wk, pos, n_tok, n_q_head, n_k_head,
                 head_dim=HEAD_DIM, q_head_stride=None, n_dims=N_ROT, sections=SECTIONS,
                 freq_base=FREQ_BASE, eps=EPS, gate_out=None) -> QkNormRopeArgs:
    return QkNormRopeArgs(_ptr(q), _ptr(q_out), _ptr(gate_out), _ptr(k), _ptr(k_out), _ptr(wq),
                          _ptr(wk), _ptr(pos), n_tok, n_q_head, n_k_head, head_dim,
                          head_dim if q_head_stride is None else q_head_stride, n_dims,
                          (ctypes.c_int32 * 4)(*sections), freq_base, eps)


def qk_norm_rope(args: QkNormRopeArgs, stream=None) -> None:
    check(lib().bh_qk_norm_rope(ctypes.byref(args), _stream(stream)))


def rope_imrope(heads, pos, n_dims=N_ROT, sections=SECTIONS, freq_base=FREQ_BASE, stream=None):
    """In place on heads [n_tok, n_head, head_dim]; pos int32 [n_tok, 4]."""
    n_tok, n_head, head_dim = heads.shape
    sec = (ctypes.c_int32 * 4)(*sections)
    check(lib().bh_rope_imrope(heads.data_ptr(), n_tok, n_head, head_dim, pos.data_ptr(), n_dims,
                               sec, freq_base, _stream(stream)))
    return heads


def pq2_embed_gather(table, ne0: int, n_rows: int, ids, out=None, w=None, eps: float = EPS,
                     out_norm=None, bad_id=None, stream=None):
    """Gather ids from a packed PQ2_0 table (uint8 device tensor); with w, also
    returns the fused RMSNorm rows."""
    import torch
    n = ids.numel()
    out = torch.empty((n, ne0), dtype=torch.float32, device=ids.device) if out is None else out
    if w is None:
        check(lib().bh_pq2_embed_gather(table.data_ptr(), ne0, n_rows, ids.data_ptr(), n,
                                        out.data_ptr(), _ptr(bad_id), _stream(stream)))
        return out
    out_norm = torch.empty_like(out) if out_norm is None else out_norm
    check(lib().bh_pq2_embed_gather_rms(table.data_ptr(), ne0, n_rows, ids.data_ptr(), n,
                                        w.data_ptr(), w.numel(), eps, out.data_ptr(),
                                        out_norm.data_ptr(), _ptr(bad_id), _stream(stream)))
    return out, out_norm


def conv1d_silu(x, state, w, out=None, stream=None):
    """Causal conv1d + SiLU (src/forward.rs:508-533) over x [n_tok, ch] with
    the cache state [ch, k-1] (advanced in place) and taps w [ch, k]."""
    import torch
    n_tok, ch = x.shape
    k = w.shape[1]
    out = torch.empty_like(x) if out is None else out
    check(lib().bh_conv1d_silu(x.data_ptr(), _ptr(state), w.data_ptr(), n_tok, ch, k,
                               out.data_ptr(), _stream(stream)))
    return out


BH_KV_F32, BH_KV_F16 = 0, 1


def _kv_dtype(cache):
    import torch
    if cache.dtype == torch.float32:
        return BH_KV_F32
    if cache.dtype in (torch.float16, torch.int16, torch.uint16):
        return BH_KV_F16
    raise TypeError(f"KV cache dtype {cache.dtype}: f32 or 16-bit f16 storage")


def kv_store(k, v, k_cache, v_cache, pos0: int, stream=None):
    """AttnCache::append / append_f16 (src/forward.rs:90-95, 120-125): rows
    k, v [n_tok, n_kv_elems] f32 into the caches [cap, n_kv_elems] (f32, or
    16-bit tensors holding f16 bits) at positions pos0 .."""
    n_tok, elems = k.shape
    check(lib().bh_kv_store(k.data_ptr(), v.data_ptr(), n_tok, elems, k_cache.data_ptr(),
                            v_cache.data_ptr(), pos0, _kv_dtype(k_cache), _stream(stream)))


def attention(q, pos0: int, k_cache, v_cache, n_kv: int, out=None, stream=None):
    """The GQA block of full_attention_layer (src/forward.rs:282-375) for
    queries q [n_q, n_head, hd] at positions pos0 ..; caches [cap, n_kv*hd]."""
    import torch
    n_q, n_head, hd = q.shape
    out = torch.empty_like(q) if out is None else out
    check(lib().bh_attention(q.data_ptr(), n_q, pos0, k_cache.data_ptr(), v_cache.data_ptr(),
                             _kv_dtype(k_cache), n_head, n_kv, hd, out.data_ptr(),
                             _stream(stream)))
    return out


def _ptr(t):
    return None if t is None else t.data_ptr()


def kv_store_planar(k, v, pos0: int, n_kv: int, bits: int, kq, kn, vq=None, vn=None, v_f32=None,
                    stream=None):
    """AttnCache::append_k_quantized / append_v_quantized / append_v
    (src/forward.rs:99-140): rows k, v [n_tok, n_kv * 256] into the planar
    caches kq [cap, n_kv, plen] u8, kn [cap, n_kv] f32 (and vq / vn, or the
    f32 v_f32 [cap, n_kv * 256] when vq is None), in place."""
    n_tok = k.shape[0]
    check(lib().bh_kv_store_planar(k.data_ptr(), v.data_ptr(), n_tok, n_kv, 256, bits,
                                   kq.data_ptr(), kn.data_ptr(), _ptr(vq), _ptr(vn), _ptr(v_f32),
                                   pos0, _stream(stream)))


def attention_planar(q, pos0: int, kq, kn, n_kv: int, bits: int, vq=None, vn=None, v_f32=None,
                     out=None, stream=None):
    """The quantized-cache branches of full_attention_layer
    (src/forward.rs:296-349) for q [n_q, n_head, 256] at positions pos0 ..."""
    import torch
    n_q, n_head, hd = q.shape
    out = torch.empty_like(q) if out is None else out
    check(lib().bh_attention_planar(q.data_ptr(), n_q, pos0, kq.data_ptr(), kn.data_ptr(),
                                    _ptr(vq), _ptr(vn), _ptr(v_f32), bits, n_head, n_kv, hd,
                                    out.data_ptr(), _stream(stream)))
    return out


def gdn_step(q, k, v, gate, beta, state, attn=None, stream=None):
    """Gated delta-net recurrence (src/gdn.rs:17-77 per token) over device
    tensors q, k [n_tok, h_k, s], v [n_tok, h_v, s], gate, beta [n_tok, h_v];
    state [h_v, s, s] is advanced in place; returns attn [n_tok, h_v, s]."""
    import torch
    n_tok, h_k, s = q.shape
    h_v = v.shape[1]
    attn = torch.empty_like(v) if attn is None else attn
    check(lib().bh_gdn_step(q.data_ptr(), k.data_ptr(), v.data_ptr(), gate.data_ptr(),
                            beta.data_ptr(), state.data_ptr(), attn.data_ptr(), n_tok, h_k, h_v,
                            s, _stream(stream)))
    return attn


def pq2_matmul_n(payload, ne0: int, n_rows: int, x, base_row: int = 0, out=None, stream=None):
    """kernels::pq2_matmul_n (src/kernels.rs:340-423) on device tensors:
    payload uint8 (the tensor's whole PQ2_0 data), x [n_tok, ne0] f32 ->
    y [n_tok, n_rows]; a 1-D x runs pq2_matvec_range and returns y [n_rows]."""
    import torch
    if x.dim() == 1:
        y = torch.empty(n_rows, dtype=torch.float32, device=x.device) if out is None else out
        check(lib().bh_pq2_matvec_range(payload.data_ptr(), payload.numel(), ne0, base_row,
                                        n_rows, x.data_ptr(), x.numel(), y.data_ptr(),
                                        y.numel(), _stream(stream)))
        return y
    n_tok = x.shape[0]
    y = torch.empty((n_tok, n_rows), dtype=torch.float32, device=x.device) if out is None else out
    check(lib().bh_pq2_matmul_n(payload.data_ptr(), payload.numel(), ne0, base_row, n_rows,
                                x.data_ptr(), x.numel(), n_tok, y.data_ptr(), y.numel(),
                                _stream(stream)))
    return y


def env_info() -> dict:
    return {"lib": str(LIB_PATH), "version": lib().bh_version().decode(),
            "pid": os.getpid()}
