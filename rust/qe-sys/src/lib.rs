//! Raw binding of libqe.so, the C ABI declared in include/qe.h: one `extern "C"` item per entry
//! point, with the header's argument order and types (u64 for uint64_t, *mut c_void for a HIP
//! stream or device pointer). Every call returns a status (QE_OK == 0) and never aborts;
//! `qe_last_error` gives the message of the calling thread's last failure.
//!
//! The safe engine over it, with the methods of the reference's MetalModel / MetalKVCache
//! (metal_infrence_engine/src/metal_inference.rs:129-316), is `hip_inference`.
#![allow(non_camel_case_types)]

use std::ffi::{c_char, c_int, c_void};

pub mod hip_inference;

pub const QE_OK: c_int = 0;
pub const QE_ERR_IO: c_int = 1;
pub const QE_ERR_FORMAT: c_int = 2;
pub const QE_ERR_TENSOR: c_int = 3;
pub const QE_ERR_POS: c_int = 4;
pub const QE_ERR_ARG: c_int = 5;
pub const QE_ERR_UNSUPPORTED: c_int = 6;
pub const QE_ERR_HIP: c_int = 7;
pub const QE_ERR_NO_DEVICE: c_int = 8;
pub const QE_ERR_KERNEL: c_int = 9;

pub const QE_KV_F32: c_int = 0;
pub const QE_KV_BF16: c_int = 1;

/// A draft source's failure return (qe_draft_fn).
pub const QE_DRAFT_ERROR: u32 = 0xFFFF_FFFF;

/// `qe_config`: the config.json fields the forward pass reads (cpu_inference.rs:20-33).
#[repr(C)]
#[derive(Clone, Copy, Debug, Default, PartialEq)]
pub struct qe_config {
    pub hidden_size: u64,
    pub intermediate_size: u64,
    pub num_hidden_layers: u64,
    pub num_attention_heads: u64,
    pub num_key_value_heads: u64,
    pub head_dim: u64,
    pub vocab_size: u64,
    pub rms_norm_eps: f32,
    pub rope_theta: f32,
    pub eos_token_id: u32,
}

/// `qe_lookup_stats`: counts of a speculative decode.
#[repr(C)]
#[derive(Clone, Copy, Debug, Default, PartialEq, Eq)]
pub struct qe_lookup_stats {
    pub passes: u64,
    pub drafted: u64,
    pub accepted: u64,
    pub single_steps: u64,
    pub plain_steps: u64,
}

/// Opaque model handle.
#[repr(C)]
pub struct qe_model {
    _private: [u8; 0],
}

/// Opaque KV cache handle.
#[repr(C)]
pub struct qe_kv {
    _private: [u8; 0],
}

/// Called once per finished decode step with that step's greedy token, in order.
pub type qe_on_token = Option<unsafe extern "C" fn(user: *mut c_void, token: u32)>;

/// A draft source: up to k_max tokens to follow history[0..n) into draft_out; returns their
/// count, or QE_DRAFT_ERROR.
pub type qe_draft_fn =
    Option<unsafe extern "C" fn(user: *mut c_void, history: *const u32, n: u64, k_max: u32, draft_out: *mut u32) -> u32>;

#[link(name = "qe")]
extern "C" {
    pub fn qe_last_error() -> *const c_char;

    // model: MetalModel::load_model / config (metal_inference.rs:157-170)
    pub fn qe_model_load(safetensors_path: *const c_char, out: *mut *mut qe_model) -> c_int;
    pub fn qe_model_free(model: *mut qe_model);
    pub fn qe_model_config(model: *const qe_model, out: *mut qe_config) -> c_int;
    pub fn qe_model_stream(model: *const qe_model) -> *mut c_void;
    // bench.rs:106-119 byte formula
    pub fn qe_weight_bytes_per_token(model: *const qe_model) -> u64;
    pub fn qe_kv_bytes_at(model: *const qe_model, pos: u64, kv_dtype: c_int) -> u64;
    pub fn qe_model_fused_layers(model: *const qe_model) -> c_int;

    // KV cache: MetalKVCache::new (metal_inference.rs:129-137)
    pub fn qe_kv_new(model: *mut qe_model, max_seq: u64, kv_dtype: c_int, out: *mut *mut qe_kv) -> c_int;
    pub fn qe_kv_free(kv: *mut qe_kv);
    pub fn qe_kv_max_seq(kv: *const qe_kv) -> u64;
    pub fn qe_kv_len(kv: *const qe_kv) -> u64;

    // MetalModel::forward (metal_inference.rs:284-291), the prompt loop (bench.rs:174-176) and
    // MetalModel::decode (metal_inference.rs:293-316)
    pub fn qe_forward(model: *mut qe_model, token: u32, pos: u64, kv: *mut qe_kv, logits_out: *mut f32) -> c_int;
    pub fn qe_prefill(model: *mut qe_model, ids: *const u32, n: u64, start_pos: u64, kv: *mut qe_kv,
                      last_logits: *mut f32) -> c_int;
    pub fn qe_decode(model: *mut qe_model, first: u32, start_pos: u64, steps: u64, kv: *mut qe_kv,
                     on_token: qe_on_token, user: *mut c_void, logits_per_step: *mut f32) -> c_int;

    // multi-token forward on the matrix cores (no reference counterpart)
    pub fn qe_prefill_batch(model: *mut qe_model, ids: *const u32, n: u64, start_pos: u64, kv: *mut qe_kv,
                            chunk: u32, last_logits: *mut f32) -> c_int;
    pub fn qe_verify(model: *mut qe_model, ids: *const u32, k: u64, start_pos: u64, kv: *mut qe_kv,
                     logits_out: *mut f32) -> c_int;
    pub fn qe_verify_greedy(model: *mut qe_model, ids: *const u32, k: u64, start_pos: u64, kv: *mut qe_kv,
                            tokens_out: *mut u32) -> c_int;

    // speculative greedy decode (README.md:109-111 names it as the next step)
    pub fn qe_decode_lookup(model: *mut qe_model, context: *const u32, n_context: u64, first: u32, start_pos: u64,
                            steps: u64, kv: *mut qe_kv, k_max: u32, ngram: u32, on_token: qe_on_token,
                            user: *mut c_void, stats: *mut qe_lookup_stats) -> c_int;
    pub fn qe_decode_drafted(model: *mut qe_model, context: *const u32, n_context: u64, first: u32, start_pos: u64,
                             steps: u64, kv: *mut qe_kv, k_max: u32, draft: qe_draft_fn, draft_user: *mut c_void,
                             adaptive: c_int, on_token: qe_on_token, user: *mut c_void,
                             stats: *mut qe_lookup_stats) -> c_int;
    pub fn qe_lookup_draft(history: *const u32, n: u64, ngram: u32, k_max: u32, draft_out: *mut u32) -> u64;

    // per-stage kernel timing (no reference counterpart: README.md:64-71)
    pub fn qe_profile_step(model: *mut qe_model, token: u32, pos: u64, kv: *mut qe_kv, us_out: *mut f32,
                           launches_out: *mut u32, names_out: *mut *const c_char, max_stages: u32,
                           n_out: *mut u32) -> c_int;

    // synthetic inputs
    pub fn qe_write_random_checkpoint(dir: *const c_char, seed: u64, cfg: *const qe_config) -> c_int;
    pub fn qe_random_prompt(seed: u64, n: u64, vocab: u32, out: *mut u32);

    // isolated device ops on caller-owned device memory (stream may be null)
    pub fn qe_op_matvec_bf16(w: *const c_void, x: *const f32, out: *mut f32, rows: u64, cols: u64,
                             stream: *mut c_void) -> c_int;
    pub fn qe_op_gemm_bf16(a: *const f32, w: *const c_void, c: *mut f32, m: u64, n: u64, k: u64,
                           stream: *mut c_void) -> c_int;
    pub fn qe_op_attention_work_bytes(n_heads: u64, n_kv_heads: u64, n_pos: u64) -> u64;
    pub fn qe_op_attention(q: *const f32, k: *const f32, v: *const f32, out: *mut f32, n_pos: u64, kv_stride: u64,
                           n_heads: u64, n_kv_heads: u64, n_splits: u32, work: *mut c_void,
                           stream: *mut c_void) -> c_int;
    pub fn qe_op_attention_static(q: *const f32, k: *const f32, v: *const f32, out: *mut f32, n_pos: u64,
                                  kv_stride: u64, n_heads: u64, n_kv_heads: u64, n_splits: u32,
                                  stream: *mut c_void) -> c_int;
    pub fn qe_op_argmax(logits: *const f32, rows: u64, n: u64, tokens_out: *mut u32, stream: *mut c_void) -> c_int;
    pub fn qe_op_read_sum(src: *const f32, n: u64, partial: *mut f32, grid: u32, stream: *mut c_void) -> c_int;
    pub fn qe_op_read_sum_nt(src: *const f32, n: u64, partial: *mut f32, grid: u32, stream: *mut c_void) -> c_int;
}
