/*
 * bdh_hip.h -- C ABI of the MI355X (gfx950) recurrent linear-attention
 * forward path of burn_dragon ("BDH"), implemented in hand-written HIP.
 *
 * Every entry point replaces one function of the reference's Burn custom-op
 * surface (crates/burn_dragon_kernel, re-exported at src/lib.rs:40-56);
 * the comment above each declaration cites it.  Conventions:
 *   - all tensor arguments are DEVICE pointers owned by the caller, dense
 *     row-major (C-contiguous) in the reference's layouts:
 *       query / x  [B, H, T, N]       value [B, Hv, T, D], Hv in {1, H}
 *       rho        [B, H, N, D] f32   context [B, H, T, D] f32
 *       decay      [H] f32            (NULL = ones: RoPE, no ALiBi)
 *   - `stream` is a hipStream_t (NULL = the default stream); launches are
 *     asynchronous on it, nothing synchronises the host;
 *   - the library never allocates or frees caller memory.  It keeps its own
 *     scratch per (device, stream), grown on the first call of a larger
 *     shape on that stream.  Growth is refused (BDH_UNSUPPORTED) while the
 *     stream is being captured into a graph: run the largest shape once
 *     eagerly on the capturing stream first.  A buffer a captured graph may
 *     still use is never freed before bdh_scratch_release, and the first
 *     eager call on a stream after a capture on it takes fresh buffers, so a
 *     replay (on any stream) never shares scratch with eager work.  Graphs
 *     captured on one stream share that stream's buffers: their replays
 *     must not overlap each other.  A stream's scratch (GB-scale at long
 *     shapes) lives until bdh_scratch_release(stream): call it before a
 *     stream is destroyed, or a later stream given the same handle inherits
 *     the set;
 *   - errors are status codes, never aborts.  BDH_UNSUPPORTED is the
 *     reference's `None` ("use the Burn-op reference instead");
 *     bdh_last_error() gives the message (thread-local).
 *   - calls on different streams may run concurrently (each stream has its
 *     own scratch); calls on one stream are ordered by it.
 */
#ifndef BDH_HIP_H
#define BDH_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
  BDH_OK = 0,
  BDH_UNSUPPORTED = 1, /* reference returns None: caller falls back */
  BDH_EINVAL = -1,     /* malformed arguments (null outputs, bad enum) */
  BDH_EHIP = -2        /* a HIP runtime call failed */
} bdh_status;

typedef enum { BDH_F32 = 0, BDH_BF16 = 1 } bdh_dtype;

/* RoPE positions: RecurrentPositionMode (dragon_support.rs), mirrored by
 * rotate_positions / rotate_positions_fixed (attention.rs:339-349). */
typedef enum { BDH_ROPE_SEQUENTIAL = 0, BDH_ROPE_FIXED = 1 } bdh_rope_mode;

typedef struct {
  int32_t mode;  /* bdh_rope_mode */
  int32_t _pad;
  int64_t pos0;  /* first position (Sequential) or the position (Fixed) */
  float theta;   /* FusedKernelConfig::rope_theta, default 65536 (config.rs:79) */
} bdh_rope;

/* Host copy of the RoPE frequency table the kernels use (f32, latent
 * entries): Attention::build_freqs, Rope arm
 * (crates/burn_dragon_core/src/model/attention.rs:552-576). */
bdh_status bdh_rope_freqs(int64_t latent, float theta, float* freqs_out);

/* Shape plan.  Replaces CompiledRecurrentAttentionPlan::new
 * (crates/burn_dragon_kernel/src/recurrent.rs:107-139); integers instead of
 * the reference's uploaded f32 meta tensor, nothing is sent to the device. */
typedef struct {
  int64_t batch, heads, value_heads, time, latent, embd;
} bdh_recurrent_plan;

/* Validates like try_fused_recurrent_attention_wgpu (recurrent.rs:187-195):
 * any zero dim or value_heads not in {1, heads} -> BDH_UNSUPPORTED. */
bdh_status bdh_recurrent_plan_new(int64_t batch, int64_t heads, int64_t value_heads,
                                  int64_t time, int64_t latent, int64_t embd,
                                  bdh_recurrent_plan* out);

/* Replaces supports_backend (recurrent.rs:151-173, exported as
 * supports_recurrent_backend): 1 when the current device is gfx950 and the
 * kernels are loadable, else 0. */
int32_t bdh_supports_backend(void);

/* Replaces try_fused_recurrent_attention_wgpu_with_plan (recurrent.rs:221-359)
 * and, with plan built per call, try_fused_recurrent_attention_wgpu
 * (recurrent.rs:175-219).  query is already rotated (the reference applies
 * RoPE before the call, sequence_dispatch.rs:97-104).
 *   ctx_t = x_t . rho_t ;  rho_{t+1} = (rho_t + x_t^T v_t) * decay
 * rho_in NULL -> zeros (recurrent.rs:243-246).  rho_out may equal rho_in
 * (in place); otherwise rho_in is not written (the reference's private copy,
 * recurrent.rs:259).  dtype applies to query and value: BDH_F32 runs the
 * fp32 path, BDH_BF16 the MFMA path (fp32 accumulate, fp32 rho/context).
 * chunk: the row chunk of the MFMA path, the reference's
 * dense_score_row_chunk (config.rs:46; linear.rs:117-118): rho is
 * materialised every `chunk` tokens and the carries inside a row chunk go
 * through causal score blocks of 128 tokens.  0 = auto: 512 (the
 * reference's default, config.rs:10), with or without decay; otherwise a
 * multiple of 128 up to 4096 (BDH_UNSUPPORTED otherwise).  The result does
 * not depend on it beyond rounding; the fp32 path materialises rho every 256
 * tokens whatever it is.
 * time == 1 with BDH_F32 (the reference's decode call, sequence_dispatch.rs
 * :109-124; it selects kernels by T, forward_runtime.rs:235-256) runs the
 * one-token step of bdh_decode_step: with rho_out == rho_in and no decay
 * only the active rows of rho are read and written; otherwise one pass
 * copies every row of rho_in (zeros when NULL) to rho_out with the update.
 * All tensor pointers must be 16-byte aligned (BDH_EINVAL otherwise). */
bdh_status bdh_recurrent_attention_fwd(const bdh_recurrent_plan* plan, int32_t dtype,
                                       const void* query, const void* value,
                                       const float* rho_in, const float* decay,
                                       float* context_out, float* rho_out,
                                       int32_t chunk, void* stream);

/* RoPE-fused variant: x is the UNROTATED sparse activation; RoPE
 * (attention.rs:488-576, f32 phase op order) is applied inside the kernels.
 * Otherwise identical to bdh_recurrent_attention_fwd.  Replaces the pair
 * rotate_positions[_fixed] + try_fused_recurrent_attention_wgpu_with_plan
 * inside DragonModel::recurrent_attention_with_plan
 * (crates/burn_dragon_core/src/model/dragon/sequence_dispatch.rs:83-136). */
bdh_status bdh_recurrent_attention_rope_fwd(const bdh_recurrent_plan* plan, int32_t dtype,
                                            const void* x, const void* value,
                                            const float* rho_in, const float* decay,
                                            const bdh_rope* rope, float* context_out,
                                            float* rho_out, int32_t chunk, void* stream);

/* Decode step (T = 1), fp32, rho updated in place.  Same result as
 * bdh_recurrent_attention_rope_fwd with time = 1 and rho_out == rho_in:
 *   A = { i : x_i != 0  or  (x_{i^1} != 0 and frac(pos * f_i) != 0) }
 *   a = rot(x) . rho (read before the update) ;  rho = (rho + rot(x)^T v) * decay
 * decay NULL (RoPE models): only the rows in A change, and only they are
 * read and written (the sparse row gather).  decay [H] f32 (ALiBi, e.g.
 * exp(-slope), attention.rs:201-208): every row is scaled, so every row is
 * streamed once (recurrent.rs:415, linear.rs:53-56).
 * x [B,H,N], value [B,Hv,D], rho [B,H,N,D], a_out [B,H,D].
 * rope NULL: x is already rotated and A = { i : x_i != 0 }.
 * active_idx_out [B,H,N] int32 (ascending, padded with -1) and
 * active_cnt_out [B,H] int32 may be NULL.  This is the per-token call of the
 * reference's decode drivers (dragon.rs:1749-1808, generation.rs:458) through
 * recurrent_attention_with_plan at T = 1 (sequence_dispatch.rs:109-124).
 * Pointers must be 4-byte aligned; 16-byte aligned rows with embd % 4 == 0
 * take the float4 kernels. */
bdh_status bdh_decode_step(int64_t batch, int64_t heads, int64_t value_heads,
                           int64_t latent, int64_t embd, const float* x,
                           const float* value, float* rho, const float* decay,
                           const bdh_rope* rope, float* a_out, int32_t* active_idx_out,
                           int32_t* active_cnt_out, void* stream);

/* bdh_decode_step without any device allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments and results as bdh_decode_step; its buffers (the RoPE frequency
 * tables and the row-range readouts and lists) live in one 16 MiB device
 * array per GPU, kept until the process ends.  Limits: latent <= 2^20, and
 * the range buffers of the shape within 8 MiB (BDH_UNSUPPORTED beyond,
 * with the reason in bdh_last_error).  Every call on a GPU shares that
 * GPU's range buffers, so calls that overlap on one GPU (different streams
 * or threads) race.  The first call with a new (latent, theta) uploads its
 * frequency table into a slot of an 8 MiB table region (synchronously on
 * `stream`; refused during capture); slots are never overwritten, so a
 * graph captured at one key stays valid after calls at other keys, and a
 * key that no longer fits the region is refused. */
bdh_status bdh_decode_step_noalloc(int64_t batch, int64_t heads, int64_t value_heads,
                                   int64_t latent, int64_t embd, const float* x,
                                   const float* value, float* rho, const float* decay,
                                   const bdh_rope* rope, float* a_out, int32_t* active_idx_out,
                                   int32_t* active_cnt_out, void* stream);

/* Replaces try_fused_dense_causal_attention_wgpu[_with_plan]
 * (crates/burn_dragon_kernel/src/dense_causal_attention.rs:162-261):
 *   ctx = tril(-1)(Q Q^T * decay^(r-c)) V      (no state), decay [H] required.
 * time > 1024 -> BDH_UNSUPPORTED as in the reference (:44, :179). */
bdh_status bdh_dense_causal_attention_fwd(const bdh_recurrent_plan* plan, int32_t dtype,
                                          const void* query, const void* value,
                                          const float* decay, float* context_out,
                                          void* stream);

/* VJP of the dense causal attention, fp32 (the reference's backward runs in
 * f32).  Replaces dense_causal_attention_vjp and
 * dense_causal_attention_vjp_with_initial_rho
 * (crates/burn_dragon_kernel/src/dense_causal_attention/backward_runtime.rs
 * :16-148): for ctx = tril(-1)(Q Q^T * d^(r-c)) V + (Q * d^t) rho0 and the
 * context gradient G [B,H,T,D]:
 *   grad_query [B,H,T,N], grad_value [B,Hv,T,D] (summed over heads when
 *   Hv = 1), grad_decay [H] (sum((G V^T * gap) * S) / (d + 1e-12) and the
 *   state term), grad_rho0 [B,H,N,D] = (Q * d^t)^T G.
 * decay NULL = ones; rho0 NULL = no state (grad_rho0 must then be NULL);
 * grad_decay and grad_rho0 may be NULL (not computed).  Any time: beyond
 * 1024 tokens the sequence runs as 1024-token intervals with the interval
 * states recomputed forward and their gradients carried back (scratch of
 * (time / 1024) x [B,H,N,D] f32).  Pointers 4-byte aligned. */
bdh_status bdh_dense_causal_attention_vjp(const bdh_recurrent_plan* plan, const float* query,
                                          const float* value, const float* decay, const float* rho0,
                                          const float* grad_output, float* grad_query,
                                          float* grad_value, float* grad_decay, float* grad_rho0,
                                          void* stream);

/* Backward of the recurrent attention with respect to its context output
 * (FusedRecurrentAttentionBackward, crates/burn_dragon_kernel/src/recurrent/
 * backward_runtime.rs:336-502, 1155-1239: grad query / value / decay from the
 * state history and the reverse-time adjoint, and the initial state's
 * gradient).  The same closed form as bdh_dense_causal_attention_vjp, with the
 * recurrent kernel's decay guard (|d| < 1e-8 -> 1e-8, :458-465).
 * rho_in NULL = zeros (grad_rho must then be NULL); decay NULL = ones. */
bdh_status bdh_recurrent_attention_vjp(const bdh_recurrent_plan* plan, const float* query,
                                       const float* value, const float* rho_in, const float* decay,
                                       const float* grad_context, float* grad_query,
                                       float* grad_value, float* grad_rho, float* grad_decay,
                                       void* stream);

/* Low-rank BDH layer body around the recurrent attention, bf16 MFMA with
 * fp32 accumulation.  Replaces lowrank_residual_step_impl
 * (crates/burn_dragon_core/src/model/residual_stream.rs:323-572), dropout
 * off; bdh_lowrank_layer_fwd takes its default options (no ReLU threshold,
 * no sparse latent mask), bdh_lowrank_layer_fwd_ex the options below:
 *   x    = ReLU(cur E_h - th) * mask            per head h, [B,H,T,N]
 *   a    = LN(attention(rope(x), value = cur))  (sequence_dispatch.rs:83-136)
 *   y    = (ReLU(a Ev_h - th) * mask) * x
 *   next = LN(cur + LN(decode_y_neuron_tail(y, Dec)))   (:309-321)
 * LN = DragonNorm LayerNorm with gamma = 1, beta = 0, eps = 1e-5 (norm.rs:302-328).
 * current, next_out [B,T,D] f32 (Burn's [B,1,T,D]); weights packed by
 * bdh_lowrank_pack_weights; rope may be NULL (no rotation).
 * rho_in [B,H,N,D] f32 is the layer's carried state (LayerState.rho, read
 * by recurrent_attention_with_plan, sequence_dispatch.rs:83-136; dragon.rs
 * :3437-3446 passes each layer its own state), NULL = zeros.  rho_out
 * [B,H,N,D] f32 receives the successor state, or NULL when it is not
 * retained; it may equal rho_in (in place).  With time == 1 and
 * rho_out == rho_in the attention is the sparse decode step of
 * bdh_decode_step (only the rho rows of the token's active neurons are
 * read and written); otherwise it is the MFMA prefill path.
 * Needs latent % 256 == 0 and embd % 64 == 0, embd <= 2048; all pointers
 * 16-byte aligned. */
typedef struct {
  int64_t batch, heads, time, latent, embd;
} bdh_layer_plan;

/* The layer's weights in the operand layouts of bdh_lowrank_layer_fwd:
 * encoder, encoder_v [H,D,N] f32 (Burn [1,H,D,N]) -> [H,N,D] bf16;
 * decoder [H*N, D] f32 -> chunk-major [H*N/128, D, 128] bf16 (its
 * transpose in blocks of 128 latents, so that the decoder product reads
 * one contiguous block per chunk).  Outputs are caller-owned device
 * buffers of H*N*D bf16 elements each; H*N must be a multiple of 128.
 * Pack once per weight set (the reference shares the weights across
 * layers, dragon.rs:3358). */
bdh_status bdh_lowrank_pack_weights(int64_t heads, int64_t latent, int64_t embd,
                                    const float* encoder, const float* encoder_v,
                                    const float* decoder, void* encoder_packed,
                                    void* encoder_v_packed, void* decoder_packed,
                                    void* stream);

bdh_status bdh_lowrank_layer_fwd(const bdh_layer_plan* plan, const float* current,
                                 const void* encoder_packed, const void* encoder_v_packed,
                                 const void* decoder_packed, const bdh_rope* rope,
                                 const float* rho_in, float* next_out, float* rho_out,
                                 void* stream);

/* Options of the layer's two low-rank projections, as the fused projection
 * of the reference applies them (relu_lowrank.rs reference_forward,
 * crates/burn_dragon_core/src/kernel/relu_lowrank.rs:100-135, called with
 * the layer's threshold and mask at residual_stream.rs:377-410, 440-470):
 *   relu_threshold  FusedKernelConfig::relu_threshold (config.rs:64): th,
 *                   subtracted before the ReLU (0 = none);
 *   latent_mask     [latent] f32 device pointer, 16-byte aligned, or NULL:
 *                   the sparse latent mask (BlockPattern1d::mask,
 *                   block_sparse.rs:49-64: 1 on active blocks, 0 elsewhere;
 *                   any values are applied as given), shared by the heads.
 * The layer passes no bias to its projections, so there is none here. */
typedef struct {
  float relu_threshold;
  int32_t _pad;
  const float* latent_mask;
} bdh_layer_options;

/* bdh_lowrank_layer_fwd with options (NULL = the defaults).  Same
 * arguments otherwise; a non-finite threshold or a misaligned mask is
 * BDH_EINVAL. */
bdh_status bdh_lowrank_layer_fwd_ex(const bdh_layer_plan* plan, const float* current,
                                    const void* encoder_packed, const void* encoder_v_packed,
                                    const void* decoder_packed, const bdh_rope* rope,
                                    const float* rho_in, float* next_out, float* rho_out,
                                    const bdh_layer_options* options, void* stream);

/* The model's input: out = LN(embed[token]) per token, the embedding lookup
 * followed by DragonModel's input norm (dragon.rs:3352, norm.rs:302-328).
 * tokens [n] int32, embed [vocab, embd] f32, out [n, embd] f32 (device).
 * Ids outside [0, vocab) give a zero row.  embd % 64 == 0, embd <= 2048. */
bdh_status bdh_embed_norm(const int32_t* tokens, int64_t n_tokens, const float* embed,
                          int64_t vocab, int64_t embd, float* out, void* stream);

/* lm_head [embd, vocab] f32 (dragon.rs:898-905) -> packed [vocab, embd] bf16
 * for bdh_lm_logits (caller-owned, vocab*embd elements). */
bdh_status bdh_lm_head_pack(int64_t embd, int64_t vocab, const float* lm_head, void* packed,
                            void* stream);

/* logits [rows, vocab] f32 = hidden [rows, embd] @ lm_head, bf16 MFMA with
 * fp32 accumulation: project_hidden_to_logits (dragon.rs:4033-4055). */
bdh_status bdh_lm_logits(const float* hidden, int64_t rows, int64_t embd,
                         const void* lm_head_packed, int64_t vocab, float* logits,
                         void* stream);

/* Streaming-state record: the model position and each layer's carried rho
 * with its sequence-state flags, saved from / loaded into device memory.
 * Replaces, for the state this path carries, StreamingRuntimeStateRecord /
 * LayerRuntimeStateRecord (crates/burn_dragon_language/src/train/
 * runtime_checkpoint.rs:16-112) over LayerState / ModelState
 * (crates/burn_dragon_core/src/model/state.rs:7-30); Burn's bincode record
 * cannot be written without Burn, so the file is this library's own
 * little-endian layout (magic "BDHRHO01", version 1, n_layers, position,
 * 64-byte layer entries, f32 rho blocks at 4096-byte offsets, a CRC32C per
 * block).  A layer whose four dims are 0 has no rho (None).  Copies run on
 * `stream` through pinned staging buffers (device-to-host overlapped with
 * the file write); both calls return once the file / the device buffers are
 * complete.  load rejects a record whose layer count or shapes differ from
 * `layers` (BDH_EINVAL), and verifies every layer's checksum from the file
 * before it writes any device memory: a corrupt or truncated record returns
 * BDH_EINVAL with every rho buffer unchanged.  (A file rewritten while the
 * load runs is still reported, but after its copy.)  info reads the header
 * only, so the caller can allocate. */
typedef struct {
  int64_t batch, heads, latent, embd;
  int32_t persist_sequence_state, retain_terminal_sequence_state;
} bdh_layer_state_desc;

bdh_status bdh_state_record_save(const char* path, int64_t position, int32_t n_layers,
                                 const bdh_layer_state_desc* layers, const float* const* rho,
                                 void* stream);
bdh_status bdh_state_record_info(const char* path, int64_t* position, int32_t* n_layers,
                                 bdh_layer_state_desc* layers, int32_t max_layers);
bdh_status bdh_state_record_load(const char* path, int32_t n_layers,
                                 const bdh_layer_state_desc* layers, float* const* rho,
                                 void* stream);

/* Profiling counters with the field names of KernelProfileSnapshot
 * (crates/burn_dragon_kernel/src/profiling.rs:3-16), filled per entry-point
 * call as recurrent.rs:206-215, 344-356 fills them; collected only while
 * enabled (the reference's DragonModel_STAGE_PROFILE switch,
 * profiling.rs:50-51).  Host wall-clock nanoseconds: total_ns, setup_ns
 * (validation and table lookup), dispatch_ns (the rest); copy_ns stays 0
 * (no separate rho copy: the reference's private copy, recurrent.rs:259, is
 * fused into the kernel writing rho_out).  transient_allocations: device
 * buffers the call allocated (scratch growth, a first-use table; 0 once a
 * shape is warm).  metadata_upload_bytes: host-to-device bytes of tables
 * (RoPE frequencies on first use; plans upload nothing).
 * metadata_reuse_hits / _bytes: table lookups that found it resident.
 * resident_rollout_steps: one-token steps that updated rho in place through
 * the sparse row gather. */
typedef struct {
  uint64_t calls, launches;
  uint64_t total_ns, setup_ns, copy_ns, dispatch_ns;
  uint64_t transient_allocations;
  uint64_t metadata_upload_bytes, metadata_reuse_hits, metadata_reuse_bytes;
  uint64_t resident_rollout_steps;
} bdh_profile_snapshot;

void bdh_profile_enable(int32_t enabled);
/* recurrent_profile_reset / recurrent_profile_snapshot (recurrent.rs:57-63). */
void bdh_profile_reset(void);
void bdh_profile_get(bdh_profile_snapshot* out);

/* Device time of the dominant kernel of each path, from HIP events recorded
 * on the launch stream right before and after each of its launches.  No
 * counterpart in the reference: a measurement hook for benchmarks (the
 * roofline of one kernel).  Enabling (or disabling) clears what was
 * recorded.  kind: BDH_KERNEL_PREFILL = prefill_mfma_kernel (gram, readout
 * and state units), BDH_KERNEL_DECODE = decode_kernel.  bdh_profile_kernel_get
 * waits for the recorded launches and returns their summed milliseconds and
 * their count. */
typedef enum { BDH_KERNEL_PREFILL = 0, BDH_KERNEL_DECODE = 1 } bdh_kernel_kind;
bdh_status bdh_profile_kernel_timing(int32_t enabled);
bdh_status bdh_profile_kernel_get(int32_t kind, double* total_ms, int64_t* launches);

/* Frees the scratch the library keeps for `stream` on the current device,
 * after the stream's queued work.  No counterpart in the reference (Burn's
 * allocator owns its buffers): call it when a stream is retired, and only
 * after destroying every graph captured on it that calls this library. */
bdh_status bdh_scratch_release(void* stream);

/* Check hook, no counterpart in the reference: runs the hand-written RoPE
 * rotation of the bf16 prefill (4 bf16 (even, odd) pairs per 16-byte chunk
 * rotated by 4 packed bf16 (cos, sin) words) and the same rotation written
 * with the compiler's dot-product builtin, on n_chunks chunks: rotated bf16
 * chunks (RNE) and the 8 f32 results per chunk of each.  Used by the tests to
 * hold the assembly block to the builtin bit for bit. */
bdh_status bdh_selftest_rot8(const void* x, const void* cs, void* out_bf16_asm,
                             void* out_bf16_builtin, float* out_f32_asm, float* out_f32_builtin,
                             int64_t n_chunks, void* stream);

/* HBM calibration hook, no counterpart in the reference: one launch of a
 * plain bandwidth kernel over `bytes` (a multiple of 1024) of device memory,
 * the ceilings the decode step's bytes per second are read against.
 *   BDH_CALIB_READ      read buf (buf2: a 16-byte sink, never written for
 *                       finite data)
 *   BDH_CALIB_COPY      buf -> buf2
 *   BDH_CALIB_RMW       buf[i] += (1, 0, 0, 0) in place
 *   BDH_CALIB_RMW_ROWS  the same on the 1 KiB rows rows[0..n_rows) of buf,
 *                       one wavefront per row (four in flight), written
 *                       back with non-temporal stores as the decode step
 *                       does; indices outside [0, bytes / 1024) are
 *                       skipped. */
typedef enum {
  BDH_CALIB_READ = 0,
  BDH_CALIB_COPY = 1,
  BDH_CALIB_RMW = 2,
  BDH_CALIB_RMW_ROWS = 3
} bdh_calib_kind;
bdh_status bdh_calib_hbm(int32_t kind, void* buf, void* buf2, int64_t bytes, const int32_t* rows,
                         int64_t n_rows, void* stream);

/* MFMA calibration hook, no counterpart in the reference: one launch of
 * `iters` rounds of one MFMA shape on register operands (independent
 * accumulator chains per wave: 8 for 16x16x32, 4 for the 32x32 shapes; two
 * waves per SIMD on every CU), the matrix core rate the prefill kernels
 * (bf16 shapes) and the fp32 path's GEMMs (32x32x2 f32) are read against.
 * *flop_out receives the launch's FLOP (2 m n k per MFMA); sink is a 4-byte
 * buffer that is never written for these operands. */
typedef enum {
  BDH_CALIB_MFMA_16X16X32_BF16 = 0,
  BDH_CALIB_MFMA_32X32X16_BF16 = 1,
  BDH_CALIB_MFMA_32X32X2_F32 = 2
} bdh_calib_mfma_kind;
bdh_status bdh_calib_mfma(int32_t kind, int64_t iters, float* sink, double* flop_out, void* stream);

/* Thread-local message of the last non-OK status of this thread. */
const char* bdh_last_error(void);

/* Library version string. */
const char* bdh_version(void);

#ifdef __cplusplus
}
#endif
#endif /* BDH_HIP_H */
