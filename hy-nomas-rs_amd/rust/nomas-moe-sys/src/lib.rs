//! Raw bindings of `include/nomas_moe.h`, one `extern "C"` item per entry
//! point, in the header's order and with its C types (`int` = `c_int`,
//! `int64_t` = `i64`, `uint64_t` = `u64`, `const T *` = `*const T`, `T *` =
//! `*mut T`).  See the header for the contract of each call; every `c_int`
//! result is `NOMAS_OK` or a `NOMAS_ERR_*` status with the message in
//! `nomas_moe_last_error()`.
#![allow(non_camel_case_types)]

use std::os::raw::{c_char, c_int, c_void};

// enum nomas_status
pub const NOMAS_OK: c_int = 0;
pub const NOMAS_ERR_INVALID_CONFIG: c_int = 1;
pub const NOMAS_ERR_INVALID_ARGUMENT: c_int = 2;
pub const NOMAS_ERR_WEIGHT_KEY: c_int = 3;
pub const NOMAS_ERR_IO: c_int = 4;
pub const NOMAS_ERR_HIP: c_int = 5;
pub const NOMAS_ERR_OUT_OF_MEMORY: c_int = 6;
pub const NOMAS_ERR_STATE: c_int = 7;
pub const NOMAS_ERR_INTERNAL: c_int = 8;

// enum nomas_dtype (DataType, nomas-core config.rs:30-39)
pub const NOMAS_F32: c_int = 0;
pub const NOMAS_BF16: c_int = 1;
pub const NOMAS_F16: c_int = 2;

/// MoeConfig (nomas-core config.rs:202-213), field for field.
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct nomas_moe_config {
    pub experts: i64,
    pub top_k: i64,
    pub shared_dense: f64,
    pub seed: u64,
}

/// Opaque MoE handle.
#[repr(C)]
pub struct nomas_moe_t {
    _private: [u8; 0],
}

/// Opaque dense feed-forward handle.
#[repr(C)]
pub struct nomas_ffn_t {
    _private: [u8; 0],
}

extern "C" {
    pub fn nomas_moe_config_validate(cfg: *const nomas_moe_config) -> c_int;
    pub fn nomas_moe_from_random(cfg: *const nomas_moe_config, path: *const c_char, dim: i64,
                                 hidden: i64, dtype: c_int, seed: u64, device: c_int,
                                 out: *mut *mut nomas_moe_t) -> c_int;
    pub fn nomas_moe_from_safetensors(cfg: *const nomas_moe_config, files: *const *const c_char,
                                      n_files: i64, path: *const c_char, dim: i64, hidden: i64,
                                      dtype: c_int, device: c_int,
                                      out: *mut *mut nomas_moe_t) -> c_int;
    pub fn nomas_moe_from_host(cfg: *const nomas_moe_config, dim: i64, hidden: i64, dtype: c_int,
                               device: c_int, router_w: *const c_void, gate_w: *const c_void,
                               gate_b: *const c_void, up_w: *const c_void, up_b: *const c_void,
                               down_w: *const c_void, down_b: *const c_void,
                               dense_gate_w: *const c_void, dense_gate_b: *const c_void,
                               dense_up_w: *const c_void, dense_up_b: *const c_void,
                               dense_down_w: *const c_void, dense_down_b: *const c_void,
                               out: *mut *mut nomas_moe_t) -> c_int;
    pub fn nomas_moe_forward(h: *mut nomas_moe_t, x: *const c_void, y: *mut c_void, rows: i64,
                             stream: *mut c_void) -> c_int;
    pub fn nomas_moe_forward_noalloc(h: *mut nomas_moe_t, x: *const c_void, y: *mut c_void,
                                     rows: i64, stream: *mut c_void) -> c_int;
    pub fn nomas_moe_forward_block(h: *mut nomas_moe_t, x: *const c_void, out: *mut c_void,
                                   rows: i64, seq: i64, norm_w: *const f32, eps: f64,
                                   shift: *const f32, scale: *const f32, gate: *const f32,
                                   stream: *mut c_void) -> c_int;
    pub fn nomas_moe_forward_host(h: *mut nomas_moe_t, x: *const c_void, y: *mut c_void,
                                  rows: i64) -> c_int;
    pub fn nomas_moe_n_params(h: *const nomas_moe_t) -> i64;
    pub fn nomas_moe_routing(h: *mut nomas_moe_t, idx: *mut i32, w: *mut f32, counts: *mut i32,
                             gap: *mut f32) -> c_int;
    pub fn nomas_moe_dims(h: *const nomas_moe_t, dim: *mut i64, hidden: *mut i64,
                          experts: *mut i64, top_k: *mut i64, dtype: *mut c_int) -> c_int;
    pub fn nomas_moe_set_profiling(h: *mut nomas_moe_t, enable: c_int) -> c_int;
    pub fn nomas_moe_stage_times(h: *mut nomas_moe_t, ms6: *mut f32) -> c_int;
    pub fn nomas_moe_uses_mfma(h: *const nomas_moe_t) -> c_int;
    pub fn nomas_moe_destroy(h: *mut nomas_moe_t);

    pub fn nomas_ffn_from_random(path: *const c_char, dim: i64, hidden: i64, dtype: c_int,
                                 seed: u64, device: c_int, out: *mut *mut nomas_ffn_t) -> c_int;
    pub fn nomas_ffn_from_safetensors(files: *const *const c_char, n_files: i64,
                                      path: *const c_char, dim: i64, hidden: i64, dtype: c_int,
                                      device: c_int, out: *mut *mut nomas_ffn_t) -> c_int;
    pub fn nomas_ffn_from_host(dim: i64, hidden: i64, dtype: c_int, device: c_int,
                               gate_w: *const c_void, gate_b: *const c_void, up_w: *const c_void,
                               up_b: *const c_void, down_w: *const c_void, down_b: *const c_void,
                               out: *mut *mut nomas_ffn_t) -> c_int;
    pub fn nomas_ffn_forward(h: *mut nomas_ffn_t, x: *const c_void, y: *mut c_void, rows: i64,
                             stream: *mut c_void) -> c_int;
    pub fn nomas_ffn_forward_host(h: *mut nomas_ffn_t, x: *const c_void, y: *mut c_void,
                                  rows: i64) -> c_int;
    pub fn nomas_ffn_n_params(h: *const nomas_ffn_t) -> i64;
    pub fn nomas_ffn_set_profiling(h: *mut nomas_ffn_t, enable: c_int) -> c_int;
    pub fn nomas_ffn_stage_times(h: *mut nomas_ffn_t, ms6: *mut f32) -> c_int;
    pub fn nomas_ffn_uses_mfma(h: *const nomas_ffn_t) -> c_int;
    pub fn nomas_ffn_destroy(h: *mut nomas_ffn_t);

    pub fn nomas_norm_modulate(dtype: c_int, x: *const c_void, h: *mut c_void, rows: i64,
                               dim: i64, seq: i64, norm_w: *const f32, eps: f64,
                               shift: *const f32, scale: *const f32,
                               stream: *mut c_void) -> c_int;
    pub fn nomas_gated_residual(dtype: c_int, x: *const c_void, y: *const c_void,
                                gate: *const f32, out: *mut c_void, rows: i64, dim: i64,
                                seq: i64, stream: *mut c_void) -> c_int;

    pub fn nomas_moe_last_error() -> *const c_char;
    pub fn nomas_path_seed(seed: u64, path: *const c_char) -> u64;
    pub fn nomas_randn_affine(seed: u64, mean: f64, std: f64, n: i64, out: *mut f32);
    pub fn nomas_f32_to_bf16(input: *const f32, out: *mut u16, n: i64);
    pub fn nomas_f32_to_f16(input: *const f32, out: *mut u16, n: i64);
}
