/*
 * bdh_oracle.h -- CPU restatement of burn_dragon's recurrent linear-attention
 * forward path.  TEST INFRASTRUCTURE ONLY: the parity tests, the smoke check
 * and the CPU-baseline leg of bench.py call it as the checker.  The product
 * path (libbdh_hip.so) never links, loads or calls anything in this directory.
 *
 * Every function cites the reference source it restates (paths relative to the
 * burn_dragon v0.21.8 checkout).  Layouts are the reference's, row-major,
 * contiguous:
 *   query / x   [B, H, T, N]      ("latent" N neurons per head)
 *   value       [B, Hv, T, D]     Hv in {1, H}; Hv == 1 is shared across heads
 *   rho         [B, H, N, D]
 *   context     [B, H, T, D]
 *   decay       [H]               (NULL means ones, i.e. RoPE / no ALiBi)
 */
#ifndef BDH_ORACLE_H
#define BDH_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* RoPE frequency table, f32, op order of Attention::build_freqs
 * (crates/burn_dragon_core/src/model/attention.rs:552-576, Rope arm). */
void bdh_oracle_rope_freqs(int64_t latent, float theta, float* freqs_out);

/* RoPE rotation in f32, op order of Attention::rotate_with_positions + rope
 * (attention.rs:540-550, 488-501).  Positions are pos0 + t (mode 0,
 * RecurrentPositionMode::Sequential -> rotate_positions, attention.rs:339-341,
 * 512-523) or pos0 for every t (mode 1, Fixed -> rotate_fixed, :525-538).
 * x and out are [rows, T, N]; rows = B*H.  out may not alias x. */
void bdh_oracle_rope_rotate(const float* x, int64_t rows, int64_t T, int64_t N,
                            int64_t pos0, int32_t mode, float theta, float* out);

/* Structural active set of one rotated row (position p):
 *   i is active  <=>  x[i] != 0  or  (x[i^1] != 0 and frac(p*f_i) != 0).
 * This is the set of rows where rot(x)_i is not identically zero; it is the
 * row set the sparse decode kernel gathers.  Writes ascending indices into
 * idx_out (capacity N) and returns the count. */
int32_t bdh_oracle_active_rows(const float* x, int64_t N, int64_t pos,
                               const float* freqs, int32_t* idx_out);

/* Recurrent forward, f32, op-for-op mirror of recurrent_attention_reference
 * (crates/burn_dragon_core/src/model/sequence/linear.rs:18-60):
 *   per t: ctx_t[e] = sum_l (rho[l,e] * q_t[l])   (sequential over l, f32)
 *          rho = rho + q_t[l] * v_t[e];  if decay: rho = rho * decay[h]
 * rho0 may be NULL (zeros).  ctx_out [B,H,T,D], rho_out [B,H,N,D]. */
void bdh_oracle_recurrent_f32(const float* q, const float* v, const float* rho0,
                              const float* decay, int64_t B, int64_t H,
                              int64_t Hv, int64_t T, int64_t N, int64_t D,
                              float* ctx_out, float* rho_out);

/* Same recurrence carried in f64 (inputs are f32 values, exact in f64). */
void bdh_oracle_recurrent_f64(const float* q, const float* v, const float* rho0,
                              const float* decay, int64_t B, int64_t H,
                              int64_t Hv, int64_t T, int64_t N, int64_t D,
                              double* ctx_out, double* rho_out);

/* Dense-score (parallel) form in f64, recurrent_attention_dense_score_reference
 * _full_maybe_final (linear.rs:221-322) with final rho (linear.rs:324-364):
 *   ctx = tril(-1)(Q Q^T * d^(r-c)) V + (Q * d^r) rho0
 *   rho = rho0 * d^T + (Q * d^(T-r))^T V
 * Either output pointer may be NULL. */
void bdh_oracle_dense_score_f64(const float* q, const float* v, const float* rho0,
                                const float* decay, int64_t B, int64_t H,
                                int64_t Hv, int64_t T, int64_t N, int64_t D,
                                double* ctx_out, double* rho_out);

/* One decode step (T = 1) with RoPE at position pos, f32, op order of
 * sequence_dispatch.rs:97-124 -> linear.rs:43-57 at T = 1:
 *   r = rope(x, pos);  a[e] = sum_l r[l] * rho[l,e];  rho += r^T v
 * x [B,H,N], v [B,Hv,D], rho [B,H,N,D] updated in place, a_out [B,H,D].
 * active_idx_out [B,H,N] (ascending, rest -1) and active_cnt_out [B,H] may be
 * NULL.  Rows outside the structural active set are left bit-identical. */
void bdh_oracle_decode_step_f32(const float* x, const float* v, float* rho,
                                int64_t B, int64_t H, int64_t Hv, int64_t N,
                                int64_t D, int64_t pos, float theta,
                                float* a_out, int32_t* active_idx_out,
                                int32_t* active_cnt_out);

/* bf16 round-to-nearest-even, returned as f32 (exact). */
void bdh_oracle_round_bf16(const float* in, float* out, int64_t n);

/* CPU baseline: the Burn NdArray reference's op sequence for the recurrence
 * (linear.rs:43-57) with materialised [B,H,N,D] temporaries per op, OpenMP
 * over (b,h).  Same outputs as bdh_oracle_recurrent_f32.  threads <= 0 uses
 * the OpenMP default.  Returns wall seconds. */
double bdh_oracle_ndarray_recurrent_f32(const float* q, const float* v,
                                        const float* rho0, const float* decay,
                                        int64_t B, int64_t H, int64_t Hv,
                                        int64_t T, int64_t N, int64_t D,
                                        float* ctx_out, float* rho_out,
                                        int32_t threads);

/* CPU baseline, dense-score form (linear.rs:241, 321) without state or
 * decay: scores = (Q Q^T).tril(-1) materialised as [T, T], context =
 * scores V, fp32, OpenMP over (b,h).  Returns wall seconds. */
double bdh_oracle_ndarray_dense_f32(const float* q, const float* v, int64_t B,
                                    int64_t H, int64_t Hv, int64_t T, int64_t N,
                                    int64_t D, float* ctx_out, int32_t threads);

#ifdef __cplusplus
}
#endif
#endif
