/*
 * bdh_oracle.c -- CPU restatement of burn_dragon's recurrent linear-attention
 * forward path.  TEST INFRASTRUCTURE ONLY (checker for tests/, smoke() and the
 * CPU-baseline leg of bench.py); the product library never uses it.
 *
 * Built with -ffp-contract=off and without -ffast-math so that every f32
 * multiply and add rounds separately, as the reference's element-wise Burn
 * NdArray ops do.  See bdh_oracle.h for the citation of each function.
 */
#include "bdh_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <omp.h>

/* 2.0 * PI as the reference evaluates it in f32 (attention.rs:546, 565). */
static const float TWO_PI_F32 = 2.0f * 3.14159265358979323846f;

void bdh_oracle_rope_freqs(int64_t latent, float theta, float* freqs_out) {
  /* attention.rs:559-563:
   *   exponent = ((idx as f32 / 2.0).floor() * 2.0) / latent as f32
   *   value    = 1.0 / theta.powf(exponent) / (2.0 * PI)                    */
  for (int64_t idx = 0; idx < latent; ++idx) {
    float exponent = (floorf((float)idx / 2.0f) * 2.0f) / (float)latent;
    float inv = 1.0f / powf(theta, exponent);
    freqs_out[idx] = inv / TWO_PI_F32;
  }
}

/* phase = (raw - floor(raw)) * 2pi with raw = p * f   (attention.rs:544-546) */
static inline float rope_frac(float p, float f) {
  float raw = p * f;
  return raw - floorf(raw);
}

static void rope_row(const float* x, float* out, int64_t N, float p,
                     const float* freqs) {
  /* attention.rs:488-501: rotated = stack([-odd, even]); values*cos + rotated*sin */
  for (int64_t k = 0; k + 1 < N; k += 2) {
    float ph0 = rope_frac(p, freqs[k]) * TWO_PI_F32;
    float ph1 = rope_frac(p, freqs[k + 1]) * TWO_PI_F32;
    float c0 = cosf(ph0), s0 = sinf(ph0);
    float c1 = cosf(ph1), s1 = sinf(ph1);
    float even = x[k], odd = x[k + 1];
    float a0 = even * c0;
    float b0 = (-odd) * s0;
    float a1 = odd * c1;
    float b1 = even * s1;
    out[k] = a0 + b0;
    out[k + 1] = a1 + b1;
  }
}

void bdh_oracle_rope_rotate(const float* x, int64_t rows, int64_t T, int64_t N,
                            int64_t pos0, int32_t mode, float theta, float* out) {
  float* freqs = (float*)malloc(sizeof(float) * (size_t)N);
  bdh_oracle_rope_freqs(N, theta, freqs);
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t t = 0; t < T; ++t) {
      float p = (float)(mode == 1 ? pos0 : pos0 + t);
      rope_row(x + (r * T + t) * N, out + (r * T + t) * N, N, p, freqs);
    }
  }
  free(freqs);
}

int32_t bdh_oracle_active_rows(const float* x, int64_t N, int64_t pos,
                               const float* freqs, int32_t* idx_out) {
  int32_t cnt = 0;
  float p = (float)pos;
  for (int64_t i = 0; i < N; ++i) {
    int64_t partner = i ^ 1;
    int on = x[i] != 0.0f;
    if (!on && partner < N && x[partner] != 0.0f) on = rope_frac(p, freqs[i]) != 0.0f;
    if (on) idx_out[cnt++] = (int32_t)i;
  }
  return cnt;
}

static inline int64_t vhead(int64_t Hv, int64_t h) { return Hv == 1 ? 0 : h; }

void bdh_oracle_recurrent_f32(const float* q, const float* v, const float* rho0,
                              const float* decay, int64_t B, int64_t H,
                              int64_t Hv, int64_t T, int64_t N, int64_t D,
                              float* ctx_out, float* rho_out) {
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t b = 0; b < B; ++b) {
    for (int64_t h = 0; h < H; ++h) {
      float* rho = rho_out + (b * H + h) * N * D;
      if (rho0) memcpy(rho, rho0 + (b * H + h) * N * D, sizeof(float) * (size_t)(N * D));
      else memset(rho, 0, sizeof(float) * (size_t)(N * D));
      float* acc = (float*)malloc(sizeof(float) * (size_t)D);
      const float d = decay ? decay[h] : 1.0f;
      for (int64_t t = 0; t < T; ++t) {
        const float* qt = q + ((b * H + h) * T + t) * N;
        const float* vt = v + ((b * Hv + vhead(Hv, h)) * T + t) * D;
        for (int64_t e = 0; e < D; ++e) acc[e] = 0.0f;
        for (int64_t l = 0; l < N; ++l) {
          const float x = qt[l];
          float* row = rho + l * D;
          /* Zero rows add (+/-)0 to the sum and to rho: skipping them keeps
           * every nonzero result bit-identical.  With decay every row scales. */
          if (x == 0.0f && !decay) continue;
          for (int64_t e = 0; e < D; ++e) {
            float prod = row[e] * x;          /* rho.clone() * x_t_latent */
            acc[e] = acc[e] + prod;           /* .sum_dim(2), sequential in l */
            float upd = x * vt[e];            /* x_t_latent * v_t */
            float nr = row[e] + upd;          /* rho + ... */
            if (decay) nr = nr * d;           /* rho * decay */
            row[e] = nr;
          }
        }
        float* ct = ctx_out + ((b * H + h) * T + t) * D;
        for (int64_t e = 0; e < D; ++e) ct[e] = acc[e];
      }
      free(acc);
    }
  }
}

void bdh_oracle_recurrent_f64(const float* q, const float* v, const float* rho0,
                              const float* decay, int64_t B, int64_t H,
                              int64_t Hv, int64_t T, int64_t N, int64_t D,
                              double* ctx_out, double* rho_out) {
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t b = 0; b < B; ++b) {
    for (int64_t h = 0; h < H; ++h) {
      double* rho = rho_out + (b * H + h) * N * D;
      for (int64_t i = 0; i < N * D; ++i)
        rho[i] = rho0 ? (double)rho0[(b * H + h) * N * D + i] : 0.0;
      double* acc = (double*)malloc(sizeof(double) * (size_t)D);
      const double d = decay ? (double)decay[h] : 1.0;
      for (int64_t t = 0; t < T; ++t) {
        const float* qt = q + ((b * H + h) * T + t) * N;
        const float* vt = v + ((b * Hv + vhead(Hv, h)) * T + t) * D;
        for (int64_t e = 0; e < D; ++e) acc[e] = 0.0;
        for (int64_t l = 0; l < N; ++l) {
          const double x = (double)qt[l];
          double* row = rho + l * D;
          if (x == 0.0 && !decay) continue;
          for (int64_t e = 0; e < D; ++e) {
            acc[e] += row[e] * x;
            row[e] = (row[e] + x * (double)vt[e]) * d;
          }
        }
        double* ct = ctx_out + ((b * H + h) * T + t) * D;
        for (int64_t e = 0; e < D; ++e) ct[e] = acc[e];
      }
      free(acc);
    }
  }
}

void bdh_oracle_dense_score_f64(const float* q, const float* v, const float* rho0,
                                const float* decay, int64_t B, int64_t H,
                                int64_t Hv, int64_t T, int64_t N, int64_t D,
                                double* ctx_out, double* rho_out) {
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t b = 0; b < B; ++b) {
    for (int64_t h = 0; h < H; ++h) {
      const float* Q = q + (b * H + h) * T * N;
      const float* V = v + (b * Hv + vhead(Hv, h)) * T * D;
      const float* R0 = rho0 ? rho0 + (b * H + h) * N * D : NULL;
      const double d = decay ? (double)decay[h] : 1.0;
      if (ctx_out) {
        double* C = ctx_out + (b * H + h) * T * D;
        for (int64_t r = 0; r < T; ++r) {
          double* cr = C + r * D;
          for (int64_t e = 0; e < D; ++e) cr[e] = 0.0;
          /* tril(-1)(Q Q^T * d^(r-c)) V   (linear.rs:240-242, 262, 321) */
          for (int64_t c = 0; c < r; ++c) {
            double s = 0.0;
            for (int64_t l = 0; l < N; ++l) s += (double)Q[r * N + l] * (double)Q[c * N + l];
            s *= pow(d, (double)(r - c));
            for (int64_t e = 0; e < D; ++e) cr[e] += s * (double)V[c * D + e];
          }
          /* (Q * d^r) rho0   (linear.rs:264-272, 294-299) */
          if (R0) {
            double w = pow(d, (double)r);
            for (int64_t l = 0; l < N; ++l) {
              double ql = (double)Q[r * N + l] * w;
              if (ql == 0.0) continue;
              for (int64_t e = 0; e < D; ++e) cr[e] += ql * (double)R0[l * D + e];
            }
          }
        }
      }
      if (rho_out) {
        /* rho0 * d^T + (Q * d^(T-r))^T V   (linear.rs:274-281, 300-306) */
        double* P = rho_out + (b * H + h) * N * D;
        double carry = pow(d, (double)T);
        for (int64_t i = 0; i < N * D; ++i) P[i] = R0 ? (double)R0[i] * carry : 0.0;
        for (int64_t r = 0; r < T; ++r) {
          double w = pow(d, (double)(T - r));
          for (int64_t l = 0; l < N; ++l) {
            double ql = (double)Q[r * N + l] * w;
            if (ql == 0.0) continue;
            for (int64_t e = 0; e < D; ++e) P[l * D + e] += ql * (double)V[r * D + e];
          }
        }
      }
    }
  }
}

void bdh_oracle_decode_step_f32(const float* x, const float* v, float* rho,
                                int64_t B, int64_t H, int64_t Hv, int64_t N,
                                int64_t D, int64_t pos, float theta,
                                float* a_out, int32_t* active_idx_out,
                                int32_t* active_cnt_out) {
  float* freqs = (float*)malloc(sizeof(float) * (size_t)N);
  bdh_oracle_rope_freqs(N, theta, freqs);
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t b = 0; b < B; ++b) {
    for (int64_t h = 0; h < H; ++h) {
      const int64_t s = b * H + h;
      float* r = (float*)malloc(sizeof(float) * (size_t)N);
      int32_t* idx = (int32_t*)malloc(sizeof(int32_t) * (size_t)N);
      rope_row(x + s * N, r, N, (float)pos, freqs);
      int32_t cnt = bdh_oracle_active_rows(x + s * N, N, pos, freqs, idx);
      const float* vt = v + (b * Hv + vhead(Hv, h)) * D;
      float* a = a_out + s * D;
      float* R = rho + s * N * D;
      for (int64_t e = 0; e < D; ++e) a[e] = 0.0f;
      for (int32_t j = 0; j < cnt; ++j) {
        const int64_t l = idx[j];
        const float xl = r[l];
        float* row = R + l * D;
        for (int64_t e = 0; e < D; ++e) {
          float prod = row[e] * xl;
          a[e] = a[e] + prod;
          float upd = xl * vt[e];
          row[e] = row[e] + upd;
        }
      }
      if (active_idx_out) {
        int32_t* out = active_idx_out + s * N;
        for (int64_t i = 0; i < N; ++i) out[i] = i < cnt ? idx[i] : -1;
      }
      if (active_cnt_out) active_cnt_out[s] = cnt;
      free(idx);
      free(r);
    }
  }
  free(freqs);
}

void bdh_oracle_round_bf16(const float* in, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    uint32_t u;
    memcpy(&u, &in[i], 4);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x7fffffu)) {
      u |= 0x400000u; /* quiet NaN stays NaN */
    } else {
      u += 0x7fffu + ((u >> 16) & 1u);
    }
    u &= 0xffff0000u;
    memcpy(&out[i], &u, 4);
  }
}

double bdh_oracle_ndarray_recurrent_f32(const float* q, const float* v,
                                        const float* rho0, const float* decay,
                                        int64_t B, int64_t H, int64_t Hv,
                                        int64_t T, int64_t N, int64_t D,
                                        float* ctx_out, float* rho_out,
                                        int32_t threads) {
  if (threads > 0) omp_set_num_threads(threads);
  double t0 = omp_get_wtime();
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t b = 0; b < B; ++b) {
    for (int64_t h = 0; h < H; ++h) {
      const size_t nd = (size_t)(N * D);
      float* rho = rho_out + (b * H + h) * N * D;
      if (rho0) memcpy(rho, rho0 + (b * H + h) * N * D, sizeof(float) * nd);
      else memset(rho, 0, sizeof(float) * nd);
      /* The two [N, D] temporaries Burn NdArray materialises per token:
       * rho.clone() * x_t_latent  and  x_t_latent * v_t  (linear.rs:49-54). */
      float* prod = (float*)malloc(sizeof(float) * nd);
      float* outer = (float*)malloc(sizeof(float) * nd);
      const float d = decay ? decay[h] : 1.0f;
      for (int64_t t = 0; t < T; ++t) {
        const float* qt = q + ((b * H + h) * T + t) * N;
        const float* vt = v + ((b * Hv + vhead(Hv, h)) * T + t) * D;
        float* ct = ctx_out + ((b * H + h) * T + t) * D;
        for (int64_t l = 0; l < N; ++l)
          for (int64_t e = 0; e < D; ++e) prod[l * D + e] = rho[l * D + e] * qt[l];
        for (int64_t e = 0; e < D; ++e) ct[e] = 0.0f;           /* sum_dim(2) */
        for (int64_t l = 0; l < N; ++l)
          for (int64_t e = 0; e < D; ++e) ct[e] = ct[e] + prod[l * D + e];
        for (int64_t l = 0; l < N; ++l)
          for (int64_t e = 0; e < D; ++e) outer[l * D + e] = qt[l] * vt[e];
        for (size_t i = 0; i < nd; ++i) rho[i] = rho[i] + outer[i];
        if (decay)
          for (size_t i = 0; i < nd; ++i) rho[i] = rho[i] * d;
      }
      free(outer);
      free(prod);
    }
  }
  return omp_get_wtime() - t0;
}

/* CPU baseline, dense-score form without state or decay: the NdArray op
 * sequence of linear.rs:241 and 321 with its [T, T] temporary materialised,
 * scores = (Q Q^T).tril(-1), context = scores V, fp32, OpenMP over (b, h).
 * Returns the wall time in seconds. */
double bdh_oracle_ndarray_dense_f32(const float* q, const float* v, int64_t B,
                                    int64_t H, int64_t Hv, int64_t T, int64_t N,
                                    int64_t D, float* ctx_out, int32_t threads) {
  if (threads > 0) omp_set_num_threads(threads);
  double t0 = omp_get_wtime();
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t b = 0; b < B; ++b) {
    for (int64_t h = 0; h < H; ++h) {
      const float* Q = q + (b * H + h) * T * N;
      const float* V = v + (b * Hv + vhead(Hv, h)) * T * D;
      float* C = ctx_out + (b * H + h) * T * D;
      float* S = (float*)malloc(sizeof(float) * (size_t)(T * T));
      for (int64_t r = 0; r < T; ++r)
        for (int64_t c = 0; c < T; ++c) {
          float s = 0.0f;
          for (int64_t l = 0; l < N; ++l) s += Q[r * N + l] * Q[c * N + l];
          S[r * T + c] = s;
        }
      for (int64_t r = 0; r < T; ++r)           /* tril(-1) */
        for (int64_t c = r; c < T; ++c) S[r * T + c] = 0.0f;
      for (int64_t r = 0; r < T; ++r) {
        float* cr = C + r * D;
        for (int64_t e = 0; e < D; ++e) cr[e] = 0.0f;
        for (int64_t c = 0; c < T; ++c) {
          const float s = S[r * T + c];
          for (int64_t e = 0; e < D; ++e) cr[e] += s * V[c * D + e];
        }
      }
      free(S);
    }
  }
  return omp_get_wtime() - t0;
}
