//! HIP (MI355X / gfx950) versions of the kernels in src/kernels.rs and
//! src/rope.rs, bound through the C ABI of include/bonsai_hip.h.
use std::ffi::CStr;
use std::os::raw::{c_char, c_int, c_uint, c_void};

pub type Stream = *mut c_void; // hipStream_t; null = default stream

#[repr(C)]
pub struct QkNormRopeArgs {
    pub q: *const f32, pub q_out: *mut f32, pub gate_out: *mut f32,
    pub k: *const f32, pub k_out: *mut f32,
    pub wq: *const f32, pub wk: *const f32, pub pos: *const i32,
    pub n_tok: usize, pub n_q_head: usize, pub n_k_head: usize, pub head_dim: usize,
    pub q_head_stride: usize, pub n_dims: usize,
    pub sections: [i32; 4], pub freq_base: f32, pub eps: f32,
}

#[repr(C)]
pub struct GdnPrepArgs {
    pub conv: *const f32, pub conv_out: *mut f32,
    pub z: *const f32, pub y: *const f32, pub gated_out: *mut f32,
    pub alpha_raw: *const f32, pub dt_bias: *const f32, pub ssm_a: *const f32,
    pub beta_raw: *const f32, pub gate_out: *mut f32, pub beta_out: *mut f32,
    pub n_tok: usize, pub conv_dim: usize, pub l2_dim: usize, pub head_dim: usize,
    pub inner_dim: usize, pub n_v_head: usize, pub gate_mode: c_int, pub eps: f32,
    // optional causal conv1d in front (null conv_w: off)
    pub conv_w: *const f32, pub conv_state: *mut f32, pub conv_k: usize,
}

extern "C" {
    fn bh_last_error() -> *const c_char;
    // host-slice mirrors (exact kernels.rs / rope.rs shapes)
    fn bh_host_rms_norm(x: *const f32, n: usize, w: *const f32, eps: f32, out: *mut f32) -> c_int;
    fn bh_host_rms_norm_rows(x: *const f32, x_len: usize, w: *const f32, w_len: usize,
                             row_len: usize, eps: f32, out: *mut f32) -> c_int;
    fn bh_host_l2_norm_rows(x: *const f32, x_len: usize, row_len: usize, eps: f32,
                            out: *mut f32) -> c_int;
    fn bh_host_map_inplace(x: *mut f32, n: usize, mode: c_int) -> c_int;
    fn bh_host_softmax_rows(x: *const f32, x_len: usize, row_len: usize, out: *mut f32) -> c_int;
    fn bh_host_rope_imrope(head: *mut f32, head_len: usize, p_t: i64, p_h: i64, p_w: i64,
                           p_e: i64, n_dims: usize, sections: *const i32, freq_base: f32) -> c_int;
    fn bh_host_decode_pq2_0_row(raw: *const u8, raw_len: usize, ne0: usize, out: *mut f32) -> c_int;
    fn bh_host_batch_embed(payload: *const u8, payload_len: usize, ne0: usize, n_rows: usize,
                           tokens: *const u32, n_tok: usize, out: *mut f32) -> c_int;
    fn bh_host_dot_pq2_0_row(payload: *const u8, payload_len: usize, ne0: usize, row: u64,
                             x: *const f32, x_len: usize, out: *mut f32) -> c_int;
    fn bh_host_pq2_matvec_range(payload: *const u8, payload_len: usize, ne0: usize,
                                base_row: u64, n_rows: usize, x: *const f32, x_len: usize,
                                y: *mut f32, y_len: usize) -> c_int;
    fn bh_host_pq2_matmul_n(payload: *const u8, payload_len: usize, ne0: usize, base_row: u64,
                            n_rows: usize, x: *const f32, x_len: usize, n_tok: usize,
                            y: *mut f32, y_len: usize) -> c_int;
    fn bh_host_gdn_step(q: *const f32, q_len: usize, k: *const f32, k_len: usize,
                        v: *const f32, v_len: usize, gate: *const f32, gate_len: usize,
                        beta: *const f32, beta_len: usize, state: *mut f32, state_len: usize,
                        attn: *mut f32, attn_len: usize) -> c_int;
    // device entry points (for a device-resident forward pass)
    pub fn bh_qk_norm_rope(args: *const QkNormRopeArgs, stream: Stream) -> c_int;
    pub fn bh_gdn_prep_fused(args: *const GdnPrepArgs, stream: Stream) -> c_int;
    pub fn bh_softmax_rows(x: *const f32, x_len: usize, row_len: usize, inv_temp: f32,
                           out: *mut f32, stream: Stream) -> c_int;
    // with flags: BH_SOFTMAX_SAMPLER_NORM = 1 normalises as src/sampler.rs:118-126
    pub fn bh_softmax_rows_ex(x: *const f32, x_len: usize, row_len: usize, inv_temp: f32,
                              flags: c_int, out: *mut f32, stream: Stream) -> c_int;
    // the same, allocating nothing (fixed library scratch; for graph capture)
    pub fn bh_softmax_rows_noalloc(x: *const f32, x_len: usize, row_len: usize, inv_temp: f32,
                                   out: *mut f32, stream: Stream) -> c_int;
    pub fn bh_pq2_embed_gather_rms(table: *const u8, ne0: usize, n_rows: usize, ids: *const u32,
                                   n_ids: usize, w: *const f32, w_len: usize, eps: f32,
                                   out_embed: *mut f32, out_norm: *mut f32, bad_id: *mut u32,
                                   stream: Stream) -> c_int;
    pub fn bh_conv1d_silu(x: *const f32, state: *mut f32, w: *const f32, n_tok: usize, ch: usize,
                          k: usize, out: *mut f32, stream: Stream) -> c_int;
    pub fn bh_pq2_matvec_range(payload: *const u8, payload_len: usize, ne0: usize,
                               base_row: u64, n_rows: usize, x: *const f32, x_len: usize,
                               y: *mut f32, y_len: usize, stream: Stream) -> c_int;
    pub fn bh_pq2_matmul_n(payload: *const u8, payload_len: usize, ne0: usize, base_row: u64,
                           n_rows: usize, x: *const f32, x_len: usize, n_tok: usize,
                           y: *mut f32, y_len: usize, stream: Stream) -> c_int;
    pub fn bh_gdn_step(q: *const f32, k: *const f32, v: *const f32, gate: *const f32,
                       beta: *const f32, state: *mut f32, attn: *mut f32, n_tok: usize,
                       h_k: usize, h_v: usize, s: usize, stream: Stream) -> c_int;
    pub fn bh_kv_store(k: *const f32, v: *const f32, n_tok: usize, n_kv_elems: usize,
                       k_cache: *mut c_void, v_cache: *mut c_void, pos0: usize, kv_dtype: c_int,
                       stream: Stream) -> c_int;
    pub fn bh_attention(q: *const f32, n_q: usize, pos0: usize, k_cache: *const c_void,
                        v_cache: *const c_void, kv_dtype: c_int, n_head: usize, n_kv: usize,
                        hd: usize, out: *mut f32, stream: Stream) -> c_int;
    pub fn bh_planar_packed_len(hd: usize, bits: c_uint) -> usize;
    pub fn bh_kv_store_planar(k: *const f32, v: *const f32, n_tok: usize, n_kv: usize, hd: usize,
                              bits: c_uint, kq: *mut u8, kn: *mut f32, vq: *mut u8, vn: *mut f32,
                              v_f32: *mut f32, pos0: usize, stream: Stream) -> c_int;
    pub fn bh_attention_planar(q: *const f32, n_q: usize, pos0: usize, kq: *const u8,
                               kn: *const f32, vq: *const u8, vn: *const f32, v_f32: *const f32,
                               bits: c_uint, n_head: usize, n_kv: usize, hd: usize, out: *mut f32,
                               stream: Stream) -> c_int;
    // (remaining bh_* device entry points: see include/bonsai_hip.h)
}

fn last_error() -> String {
    unsafe { CStr::from_ptr(bh_last_error()).to_string_lossy().into_owned() }
}

fn ok_or_err(st: c_int) -> Result<(), String> {
    if st == 0 { Ok(()) } else { Err(last_error()) }
}

fn must(st: c_int) {
    // the infallible reference functions (rms_norm, map_inplace, ...) have no
    // Err path; a HIP failure there is a panic, like an out-of-bounds index
    if st != 0 { panic!("bonsai_hip: {}", last_error()); }
}

pub fn rms_norm(x: &[f32], w: &[f32], eps: f32) -> Vec<f32> {
    let mut out = vec![0.0f32; x.len()];
    assert!(w.len() >= x.len());
    must(unsafe { bh_host_rms_norm(x.as_ptr(), x.len(), w.as_ptr(), eps, out.as_mut_ptr()) });
    out
}

pub fn rms_norm_inplace(x: &mut [f32], w: &[f32], eps: f32) {
    let y = rms_norm(x, w, eps);
    x.copy_from_slice(&y);
}

pub fn rms_norm_rows(x: &[f32], w: &[f32], row_len: usize, eps: f32) -> Result<Vec<f32>, String> {
    let mut out = vec![0.0f32; x.len()];
    ok_or_err(unsafe {
        bh_host_rms_norm_rows(x.as_ptr(), x.len(), w.as_ptr(), w.len(), row_len, eps, out.as_mut_ptr())
    })?;
    Ok(out)
}

pub fn l2_norm_rows(x: &[f32], row_len: usize, eps: f32) -> Result<Vec<f32>, String> {
    let mut out = vec![0.0f32; x.len()];
    ok_or_err(unsafe { bh_host_l2_norm_rows(x.as_ptr(), x.len(), row_len, eps, out.as_mut_ptr()) })?;
    Ok(out)
}

#[derive(Clone, Copy)]
pub enum Act { Silu = 0, Sigmoid = 1, Softplus = 2 }

pub fn map_inplace(x: &mut [f32], f: Act) {
    must(unsafe { bh_host_map_inplace(x.as_mut_ptr(), x.len(), f as c_int) });
}

pub fn softmax_rows(x: &[f32], row_len: usize) -> Result<Vec<f32>, String> {
    let mut out = vec![0.0f32; x.len()];
    ok_or_err(unsafe { bh_host_softmax_rows(x.as_ptr(), x.len(), row_len, out.as_mut_ptr()) })?;
    Ok(out)
}

pub fn rope_imrope(head: &mut [f32], p_t: i64, p_h: i64, p_w: i64, p_e: i64, n_dims: usize,
                   sections: [i32; 4], freq_base: f32) {
    must(unsafe {
        bh_host_rope_imrope(head.as_mut_ptr(), head.len(), p_t, p_h, p_w, p_e, n_dims,
                            sections.as_ptr(), freq_base)
    });
}

pub fn decode_pq2_0_row(raw: &[u8], ne0: usize) -> Vec<f32> {
    let mut out = vec![0.0f32; ne0];
    must(unsafe { bh_host_decode_pq2_0_row(raw.as_ptr(), raw.len(), ne0, out.as_mut_ptr()) });
    out
}

/// prefill::batch_embed over the token_embd PQ2_0 payload.
pub fn batch_embed(payload: &[u8], ne0: usize, n_rows: usize, tokens: &[u32])
    -> Result<Vec<f32>, String> {
    let mut out = vec![0.0f32; tokens.len() * ne0];
    ok_or_err(unsafe {
        bh_host_batch_embed(payload.as_ptr(), payload.len(), ne0, n_rows, tokens.as_ptr(),
                            tokens.len(), out.as_mut_ptr())
    })?;
    Ok(out)
}
// kernels::dot_pq2_0_row (src/kernels.rs:233)
pub fn dot_pq2_0_row(payload: &[u8], ne0: usize, row: u64, x: &[f32]) -> Result<f32, String> {
    let mut out = 0.0f32;
    ok_or_err(unsafe { bh_host_dot_pq2_0_row(payload.as_ptr(), payload.len(), ne0, row,
                                             x.as_ptr(), x.len(), &mut out) })?;
    Ok(out)
}

// kernels::pq2_matvec_range (src/kernels.rs:283)
pub fn pq2_matvec_range(payload: &[u8], ne0: usize, base_row: u64, n_rows: usize, x: &[f32],
                        y: &mut [f32]) -> Result<(), String> {
    ok_or_err(unsafe { bh_host_pq2_matvec_range(payload.as_ptr(), payload.len(), ne0, base_row,
                                                n_rows, x.as_ptr(), x.len(), y.as_mut_ptr(),
                                                y.len()) })
}

// kernels::pq2_matmul_n (src/kernels.rs:340)
pub fn pq2_matmul_n(payload: &[u8], ne0: usize, base_row: u64, n_rows: usize, x: &[f32],
                    n_tok: usize, y: &mut [f32]) -> Result<(), String> {
    ok_or_err(unsafe { bh_host_pq2_matmul_n(payload.as_ptr(), payload.len(), ne0, base_row,
                                            n_rows, x.as_ptr(), x.len(), n_tok,
                                            y.as_mut_ptr(), y.len()) })
}

// gdn::gdn_step (src/gdn.rs:17): same slices, state advanced in place.  The
// reference panics on a short slice (indexing); so does this wrapper.
pub fn gdn_step(q: &[f32], k: &[f32], v: &[f32], gate: &[f32], beta: &[f32],
                state: &mut [f32], attn: &mut [f32]) {
    must(unsafe { bh_host_gdn_step(q.as_ptr(), q.len(), k.as_ptr(), k.len(), v.as_ptr(),
                                   v.len(), gate.as_ptr(), gate.len(), beta.as_ptr(),
                                   beta.len(), state.as_mut_ptr(), state.len(),
                                   attn.as_mut_ptr(), attn.len()) })
}
