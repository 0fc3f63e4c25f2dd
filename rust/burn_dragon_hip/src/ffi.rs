//! Raw bindings of include/bdh_hip.h (the C ABI of libbdh_hip).  Every
//! function returns a bdh_status: BDH_OK (0), BDH_UNSUPPORTED (1, the
//! reference's `None`), BDH_EINVAL (-1) or BDH_EHIP (-2); bdh_last_error()
//! gives the message.  All tensor pointers are device pointers; `stream` is a
//! hipStream_t (null: the default stream).
#![allow(non_camel_case_types)]

use std::os::raw::{c_char, c_void};

pub const BDH_OK: i32 = 0;
pub const BDH_UNSUPPORTED: i32 = 1;
pub const BDH_EINVAL: i32 = -1;
pub const BDH_EHIP: i32 = -2;
pub const BDH_F32: i32 = 0;
pub const BDH_BF16: i32 = 1;
pub const BDH_ROPE_SEQUENTIAL: i32 = 0;
pub const BDH_ROPE_FIXED: i32 = 1;
pub const BDH_KERNEL_PREFILL: i32 = 0;
pub const BDH_KERNEL_DECODE: i32 = 1;
pub const BDH_CALIB_READ: i32 = 0;
pub const BDH_CALIB_COPY: i32 = 1;
pub const BDH_CALIB_RMW: i32 = 2;
pub const BDH_CALIB_RMW_ROWS: i32 = 3;
pub const BDH_CALIB_MFMA_16X16X32_BF16: i32 = 0;
pub const BDH_CALIB_MFMA_32X32X16_BF16: i32 = 1;
pub const BDH_CALIB_MFMA_32X32X2_F32: i32 = 2;

#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct bdh_rope {
    pub mode: i32,
    pub _pad: i32,
    pub pos0: i64,
    pub theta: f32,
}

#[repr(C)]
#[derive(Clone, Copy, Debug, Default, PartialEq, Eq)]
pub struct bdh_recurrent_plan {
    pub batch: i64,
    pub heads: i64,
    pub value_heads: i64,
    pub time: i64,
    pub latent: i64,
    pub embd: i64,
}

#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct bdh_layer_plan {
    pub batch: i64,
    pub heads: i64,
    pub time: i64,
    pub latent: i64,
    pub embd: i64,
}

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct bdh_layer_options {
    pub relu_threshold: f32,
    pub _pad: i32,
    pub latent_mask: *const f32,
}

#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct bdh_layer_state_desc {
    pub batch: i64,
    pub heads: i64,
    pub latent: i64,
    pub embd: i64,
    pub persist_sequence_state: i32,
    pub retain_terminal_sequence_state: i32,
}

#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct bdh_profile_snapshot {
    pub calls: u64,
    pub launches: u64,
    pub total_ns: u64,
    pub setup_ns: u64,
    pub copy_ns: u64,
    pub dispatch_ns: u64,
    pub transient_allocations: u64,
    pub metadata_upload_bytes: u64,
    pub metadata_reuse_hits: u64,
    pub metadata_reuse_bytes: u64,
    pub resident_rollout_steps: u64,
}

#[link(name = "bdh_hip")]
extern "C" {
    pub fn bdh_rope_freqs(latent: i64, theta: f32, freqs_out: *mut f32) -> i32;
    pub fn bdh_recurrent_plan_new(batch: i64, heads: i64, value_heads: i64, time: i64, latent: i64,
                                  embd: i64, out: *mut bdh_recurrent_plan) -> i32;
    pub fn bdh_supports_backend() -> i32;
    pub fn bdh_recurrent_attention_fwd(plan: *const bdh_recurrent_plan, dtype: i32,
                                       query: *const c_void, value: *const c_void,
                                       rho_in: *const f32, decay: *const f32,
                                       context_out: *mut f32, rho_out: *mut f32, chunk: i32,
                                       stream: *mut c_void) -> i32;
    pub fn bdh_recurrent_attention_rope_fwd(plan: *const bdh_recurrent_plan, dtype: i32,
                                            x: *const c_void, value: *const c_void,
                                            rho_in: *const f32, decay: *const f32,
                                            rope: *const bdh_rope, context_out: *mut f32,
                                            rho_out: *mut f32, chunk: i32,
                                            stream: *mut c_void) -> i32;
    pub fn bdh_decode_step(batch: i64, heads: i64, value_heads: i64, latent: i64, embd: i64,
                           x: *const f32, value: *const f32, rho: *mut f32, decay: *const f32,
                           rope: *const bdh_rope, a_out: *mut f32, active_idx_out: *mut i32,
                           active_cnt_out: *mut i32, stream: *mut c_void) -> i32;
    pub fn bdh_decode_step_noalloc(batch: i64, heads: i64, value_heads: i64, latent: i64,
                                   embd: i64, x: *const f32, value: *const f32, rho: *mut f32,
                                   decay: *const f32, rope: *const bdh_rope, a_out: *mut f32,
                                   active_idx_out: *mut i32, active_cnt_out: *mut i32,
                                   stream: *mut c_void) -> i32;
    pub fn bdh_dense_causal_attention_fwd(plan: *const bdh_recurrent_plan, dtype: i32,
                                          query: *const c_void, value: *const c_void,
                                          decay: *const f32, context_out: *mut f32,
                                          stream: *mut c_void) -> i32;
    pub fn bdh_dense_causal_attention_vjp(plan: *const bdh_recurrent_plan, query: *const f32,
                                          value: *const f32, decay: *const f32, rho0: *const f32,
                                          grad_output: *const f32, grad_query: *mut f32,
                                          grad_value: *mut f32, grad_decay: *mut f32,
                                          grad_rho0: *mut f32, stream: *mut c_void) -> i32;
    pub fn bdh_recurrent_attention_vjp(plan: *const bdh_recurrent_plan, query: *const f32,
                                       value: *const f32, rho_in: *const f32, decay: *const f32,
                                       grad_context: *const f32, grad_query: *mut f32,
                                       grad_value: *mut f32, grad_rho: *mut f32,
                                       grad_decay: *mut f32, stream: *mut c_void) -> i32;
    pub fn bdh_lowrank_pack_weights(heads: i64, latent: i64, embd: i64, encoder: *const f32,
                                    encoder_v: *const f32, decoder: *const f32,
                                    encoder_packed: *mut c_void, encoder_v_packed: *mut c_void,
                                    decoder_packed: *mut c_void, stream: *mut c_void) -> i32;
    pub fn bdh_lowrank_layer_fwd(plan: *const bdh_layer_plan, current: *const f32,
                                 encoder_packed: *const c_void, encoder_v_packed: *const c_void,
                                 decoder_packed: *const c_void, rope: *const bdh_rope,
                                 rho_in: *const f32, next_out: *mut f32, rho_out: *mut f32,
                                 stream: *mut c_void) -> i32;
    pub fn bdh_lowrank_layer_fwd_ex(plan: *const bdh_layer_plan, current: *const f32,
                                    encoder_packed: *const c_void, encoder_v_packed: *const c_void,
                                    decoder_packed: *const c_void, rope: *const bdh_rope,
                                    rho_in: *const f32, next_out: *mut f32, rho_out: *mut f32,
                                    options: *const bdh_layer_options, stream: *mut c_void) -> i32;
    pub fn bdh_embed_norm(tokens: *const i32, n_tokens: i64, embed: *const f32, vocab: i64,
                          embd: i64, out: *mut f32, stream: *mut c_void) -> i32;
    pub fn bdh_lm_head_pack(embd: i64, vocab: i64, lm_head: *const f32, packed: *mut c_void,
                            stream: *mut c_void) -> i32;
    pub fn bdh_lm_logits(hidden: *const f32, rows: i64, embd: i64, lm_head_packed: *const c_void,
                         vocab: i64, logits: *mut f32, stream: *mut c_void) -> i32;
    pub fn bdh_state_record_save(path: *const c_char, position: i64, n_layers: i32,
                                 layers: *const bdh_layer_state_desc, rho: *const *const f32,
                                 stream: *mut c_void) -> i32;
    pub fn bdh_state_record_info(path: *const c_char, position: *mut i64, n_layers: *mut i32,
                                 layers: *mut bdh_layer_state_desc, max_layers: i32) -> i32;
    pub fn bdh_state_record_load(path: *const c_char, n_layers: i32,
                                 layers: *const bdh_layer_state_desc, rho: *const *mut f32,
                                 stream: *mut c_void) -> i32;
    pub fn bdh_profile_enable(enabled: i32);
    pub fn bdh_profile_reset();
    pub fn bdh_profile_get(out: *mut bdh_profile_snapshot);
    pub fn bdh_profile_kernel_timing(enabled: i32) -> i32;
    pub fn bdh_profile_kernel_get(kind: i32, total_ms: *mut f64, launches: *mut i64) -> i32;
    pub fn bdh_scratch_release(stream: *mut c_void) -> i32;
    pub fn bdh_selftest_rot8(x: *const c_void, cs: *const c_void, out_bf16_asm: *mut c_void,
                             out_bf16_builtin: *mut c_void, out_f32_asm: *mut f32,
                             out_f32_builtin: *mut f32, n_chunks: i64, stream: *mut c_void) -> i32;
    pub fn bdh_calib_hbm(kind: i32, buf: *mut c_void, buf2: *mut c_void, bytes: i64,
                         rows: *const i32, n_rows: i64, stream: *mut c_void) -> i32;
    pub fn bdh_calib_mfma(kind: i32, iters: i64, sink: *mut f32, flop_out: *mut f64,
                          stream: *mut c_void) -> i32;
    pub fn bdh_last_error() -> *const c_char;
    pub fn bdh_version() -> *const c_char;
}
