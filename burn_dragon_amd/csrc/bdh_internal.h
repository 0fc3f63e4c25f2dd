// Host-side internal interfaces between the translation units of libbdh_hip.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <string>

#include "bdh_common.h"
#include "bdh_hip.h"

namespace bdh {

// Thread-local error message; returns the status for `return fail(...)`.
bdh_status fail(bdh_status st, const std::string& msg);
bdh_status hip_fail(hipError_t e, const char* what);

#define BDH_HIP_TRY(expr)                                   \
  do {                                                      \
    hipError_t _e = (expr);                                 \
    if (_e != hipSuccess) return ::bdh::hip_fail(_e, #expr); \
  } while (0)

// Scratch per (device, stream), one buffer per slot, grown on demand (never shrunk).
enum ScratchSlot {
  SLOT_SCORES = 0,   // causal score partials    [KS, S, n_iv, Lp, Lp] f32
  SLOT_VT,           // transposed values        [B*Hv, Tp/32, Dp, 32] bf16
  SLOT_ROTATED,      // rotated queries [S, T, N]: f32 (fp32 path) or bf16 (bf16 path)
  SLOT_READOUT,      // readout partials (bf16 path) [rd_kr, S, Lp, D] f32
  SLOT_RHO_A,        // states between intervals (bf16 path) [S, N, D] f32
  SLOT_RHO_B,
  SLOT_LAYER_CUR,    // layer input as bf16          [B, T, D]
  SLOT_LAYER_XY,     // x, then y over it (bf16)     [B, H, T, N]
  SLOT_LAYER_Q,      // rotated queries (bf16)       [B, H, T, N]
  SLOT_LAYER_ATTN,   // attention output (f32)       [B, H, T, D]
  SLOT_LAYER_AN,     // its LayerNorm (bf16)         [B, H, T, D]
  SLOT_LAYER_Z,      // decoder split-K partials     [ks, B*T, D] f32
  SLOT_LAYER_RHO,    // a successor state not kept   [B, H, N, D] f32
  SLOT_DECODE_PART,  // decode range readouts        [S, G, D] f32
  SLOT_DECODE_IDX,   // decode range active lists    [S, N] int32
  SLOT_DECODE_CNT,   // decode range active counts   [S, G] int32
  SLOT_VJP_S,        // VJP scores tril(QQ^T) * D    [S, T, T] f32
  SLOT_VJP_GS,       // VJP tril(G V^T)              [S, T, T] f32
  SLOT_VJP_M,        // VJP GS*D + its transpose     [S, T, T] f32
  SLOT_VJP_TD,       // VJP per-head grad_v, IC, G*d^t  3 x [S, T, D] f32
  SLOT_VJP_PART,     // VJP decay partials           [S] f64
  SLOT_GEMM_PART,    // fp32 GEMM split-K partials   [P, batch, M, N] f32
  SLOT_VJP_RHO,      // VJP states at interval starts [n_iv - 1, S, N, D] f32
  SLOT_VJP_GAMMA,    // VJP state gradients          2 x [S, N, D] f32
  SLOT_SNAP,         // states at interval starts (bf16 path) [n_iv, S, D, N] bf16
  SLOT_COUNT
};
// Scratch of the calling stream (see api.hip): grows on first use of a
// larger shape, refused (BDH_UNSUPPORTED) while the stream is capturing.
bdh_status scratch(hipStream_t st, int slot, size_t bytes, void** out, bool zero_on_alloc = false);
// Frees the scratch kept for `st` on the current device (after the stream's
// queued work), including buffers retired while a graph held them.
bdh_status scratch_release(hipStream_t st);
// True when `st` is being captured into a graph.
bdh_status stream_capturing(hipStream_t st, bool* capturing);

// Compute units of the current device (256 on MI355X), cached per device.
int device_cus();

// Kernel timing (bdh_profile_kernel_timing): ktime_begin records a start
// event on `st` and returns a handle (-1 when timing is off); ktime_end
// records the matching stop event.
int ktime_begin(int kind, hipStream_t st);
void ktime_end(int handle, hipStream_t st);

// Device copy of the RoPE frequency table for (latent, theta), cached per
// device; the first use uploads it (refused during capture of `st`).
bdh_status rope_freqs_device(int64_t latent, float theta, hipStream_t st, const float** out);
// Host computation of the same table (attention.rs:552-576).
void rope_freqs_host(int64_t latent, float theta, float* out);

// --- launchers (rope.hip) ---------------------------------------------------
// out[s, t, :] = rope(x[s, t, :], pos(t)) in f32, exact op order.
hipError_t launch_rope_rotate_f32(const float* x, const float* freqs, float* out, int64_t S,
                                  int64_t T, int64_t N, int64_t pos0, int fixed, hipStream_t st);

// --- fp32 path (prefill_f32.hip) -------------------------------------------
struct F32Args {
  const float* q;       // rotated queries [S, T, N]
  const float* v;       // [B, Hv, T, D]
  const float* rho_in;  // [S, N, D] or null
  const float* decay;   // [H] or null
  float* ctx;           // [S, T, D]
  float* rho_out;       // [S, N, D]
  float* scores;        // scratch [S, Lmax, Lmax]
  float* part;          // scratch for the GEMMs' split-K partials (f32_path_part_elems floats)
  int64_t B, H, Hv, T, N, D, Lmax;
  bool state;           // false: context only (single interval, no rho)
  // Context-only calls on pre-rotated queries: gram partials in bf16 (half
  // the partial traffic; the scores then carry ~9 significant bits).
  bool part16 = false;
};
size_t f32_path_part_elems(const F32Args& a);
hipError_t run_f32_path(const F32Args& a, hipStream_t st, uint64_t* launches);

// --- bf16 MFMA path (prefill_bf16.hip) --------------------------------------
struct Bf16Args {
  const bf16_t* x;      // [S, T, N] (unrotated when rope != null)
  const bf16_t* v;      // [B, Hv, T, D]
  const float* rho_in;  // [S, N, D] or null
  const float* decay;   // [H] or null
  const float* freqs;   // device RoPE frequencies or null (query pre-rotated)
  int64_t pos0;
  int fixed;
  float* ctx;           // [S, T, D]
  float* rho_out;       // [S, N, D]
  int64_t B, H, Hv, T, N, D;
  int64_t L;            // state-carry interval (multiple of 128)
  bool state;           // false: context only (single interval, no rho)
  // Context-only calls on pre-rotated queries: gram partials in bf16 (half
  // the partial traffic; the scores then carry ~9 significant bits).
  bool part16 = false;
};
bool bf16_shape_supported(int64_t N, int64_t D, const char** why);
bdh_status run_bf16_path(const Bf16Args& a, hipStream_t st, uint64_t* launches);

// --- low-rank layer body (layer_bf16.hip) ------------------------------------
struct LayerArgs {
  const float* cur;     // [B, T, D]
  const bf16_t* enc;    // packed encoder   [H, N, D]
  const bf16_t* encv;   // packed encoder_v [H, N, D]
  const bf16_t* dec;    // packed decoder   [H*N/128, D, 128] (chunk-major)
  const float* freqs;   // device RoPE frequencies or null
  int64_t pos0;
  int fixed;
  float* next;          // [B, T, D]
  const float* rho_in;  // [B, H, N, D] carried state, or null (zeros)
  float* rho_out;       // [B, H, N, D] or null; == rho_in with T = 1: sparse decode step
  int64_t B, H, T, N, D;
  int64_t state_interval;  // state-carry interval when rho_out is set
  float relu_th = 0.0f;    // ReLU threshold of both projections
  const float* mask = nullptr;  // latent mask [N] of both projections, or null
};
bool layer_shape_supported(int64_t N, int64_t D, const char** why);
bdh_status pack_lowrank_weights(int64_t H, int64_t N, int64_t D, const float* enc,
                                const float* encv, const float* dec, bf16_t* enc_p,
                                bf16_t* encv_p, bf16_t* dec_p, hipStream_t st);
bdh_status run_layer(const LayerArgs& a, hipStream_t st, uint64_t* launches);
bdh_status embed_norm(const int32_t* tokens, int64_t n, const float* embed, int64_t vocab,
                      int64_t D, float* out, hipStream_t st);
bdh_status pack_lm_head(int64_t D, int64_t V, const float* head, bf16_t* packed, hipStream_t st);
bdh_status lm_logits(const float* hidden, int64_t M, int64_t D, const bf16_t* head, int64_t V,
                     float* logits, hipStream_t st);

// --- decode (decode.hip) ------------------------------------------------------
// One token per stream (T = 1).  rho_in == rho (not null) and no decay:
// the sparse step (only the active rows are read and written).  Otherwise
// the dense step: every row of rho_in (zeros when null) is read and written
// to rho, rho = (rho_in + rot(x)^T v) * decay, in place or not.
struct DecodeArgs {
  const float* x;       // [S, N]
  const float* v;       // [B, Hv, D]
  const float* rho_in;  // [S, N, D] or null (zeros)
  float* rho;           // [S, N, D] successor state
  const float* decay;   // [H] or null (ones)
  const float* freqs;   // null -> x already rotated
  float pos;
  float* a_out;         // [S, D]
  int32_t* idx_out;     // [S, N] or null
  int32_t* cnt_out;     // [S] or null
  int64_t B, H, Hv, N, D;
  // Buffers for the range readouts and lists of a split stream; null: the
  // stream's scratch.
  void* part_buf = nullptr;
  size_t part_bytes = 0;
};
bdh_status run_decode(const DecodeArgs& a, hipStream_t st, uint64_t* launches);

// --- attention VJP (vjp.hip), fp32 ---------------------------------------------
struct VjpArgs {
  const float* q;       // [S, T, N] (Q = K)
  const float* v;       // [B, Hv, T, D]
  const float* decay;   // [H] or null (ones)
  const float* rho0;    // [S, N, D] or null
  const float* g;       // context gradient [S, T, D]
  float* grad_q;        // [S, T, N]
  float* grad_v;        // [B, Hv, T, D]
  float* grad_decay;    // [H] or null (not computed)
  float* grad_rho0;     // [S, N, D] or null (not computed)
  int64_t B, H, Hv, T, N, D;
  bool recurrent_eps;   // decay guard of the recurrent backward, else d + 1e-12
};
bdh_status run_attention_vjp(const VjpArgs& a, hipStream_t st, uint64_t* launches);
// Bytes of range buffers run_decode needs for a.
size_t decode_part_bytes(const DecodeArgs& a);

}  // namespace bdh
