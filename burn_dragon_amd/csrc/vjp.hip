// VJP of the causal linear attention (context gradient), fp32 on gfx950.
//
// The reference has two backward paths with one closed form: the dense
// causal VJP (kernel/src/dense_causal_attention/backward_runtime.rs:36-148)
// and the recurrent backward (kernel/src/recurrent/backward_runtime.rs,
// state history and a reverse-time adjoint).  With Q = K = query, G the
// context gradient, D[r, c] = d^(r-c) and gap = r - c below the diagonal:
//   S      = tril(-1)(Q Q^T) * D            [T, T]   gemm, TRIL_DECAY epilogue
//   GS     = tril(-1)(G V^T)                [T, T]   gemm, TRIL epilogue
//   M      = GS * D + (GS * D)^T            [T, T]   elementwise
//   grad_q = M Q  [+ (G rho0^T) * d^t]      [T, N]   gemm (+ ROWSCALE_ACC)
//   grad_v = S^T G                          [T, D]   gemm, heads summed for Hv = 1
//   grad_d = sum((GS * gap) * S) / sd  [+ sum((G * IC) * t) / sd],
//            IC = (Q rho0) * d^t                      gemm ROWSCALE + reduction
//   grad_rho0 = Q^T (G * d^t)               [N, D]   gemm
// Every product is a batched fp32 GEMM on v_mfma_f32_32x32x2f32 (exact fp32
// products, fp32 accumulation; bdh_gemm_f32.h) with generic strides, so
// transposed operands need no copy.  Reductions are per stream and then per head in a
// fixed order: the result is deterministic.
#include "bdh_gemm_f32.h"

namespace bdh {
namespace {

using gf32::dpowf;
using gf32::gemm;
using gf32::GemmF32;
using gf32::E_ROWSCALE;
using gf32::E_ROWSCALE_ACC;
using gf32::E_STORE;
using gf32::E_TRIL;
using gf32::E_TRIL_DECAY;

// M[s, r, c] = W[r, c] + W[c, r], W[r, c] = r > c ? GS[r, c] d^(r - c) : 0.
__global__ __launch_bounds__(256) void msym_kernel(const float* __restrict__ gs, float* __restrict__ m,
                                                   const float* __restrict__ decay, int H, int T) {
  const int64_t s = blockIdx.y;
  const float d = decay ? decay[s % H] : 1.0f;
  const float* G = gs + s * (int64_t)T * T;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < (int64_t)T * T; i += (int64_t)gridDim.x * 256) {
    const int r = (int)(i / T), c = (int)(i - (int64_t)r * T);
    float v = 0.0f;
    if (r > c) v = G[i] * dpowf(d, r - c);
    else if (c > r) v = G[(int64_t)c * T + r] * dpowf(d, c - r);
    m[s * (int64_t)T * T + i] = v;
  }
}

// Per-stream partial of the decay gradient, in the reference's element op
// order: ((GS * gap) * S) / sd over the lower triangle, plus, with a state,
// ((G * IC) * t) / sd over [T, D].  Accumulated in f64, reduced in a fixed
// order.
__global__ __launch_bounds__(256) void decay_partial_kernel(const float* __restrict__ gs,
                                                            const float* __restrict__ sc,
                                                            const float* __restrict__ g,
                                                            const float* __restrict__ ic,
                                                            const float* __restrict__ decay, int H,
                                                            int T, int D, int recurrent_eps,
                                                            double* __restrict__ part) {
  __shared__ double red[256];
  const int64_t s = blockIdx.x;
  float d = decay ? decay[s % H] : 1.0f;
  float sd;
  if (recurrent_eps) sd = (d < 1e-8f && d > -1e-8f) ? 1e-8f : d;
  else sd = d + 1e-12f;
  double acc = 0.0;
  const float* GS = gs + s * (int64_t)T * T;
  const float* SC = sc + s * (int64_t)T * T;
  for (int64_t i = threadIdx.x; i < (int64_t)T * T; i += 256) {
    const int r = (int)(i / T), c = (int)(i - (int64_t)r * T);
    if (r > c) acc += (double)(((GS[i] * (float)(r - c)) * SC[i]) / sd);
  }
  if (ic) {
    const float* Gs = g + s * (int64_t)T * D;
    const float* I = ic + s * (int64_t)T * D;
    for (int64_t i = threadIdx.x; i < (int64_t)T * D; i += 256) {
      const int t = (int)(i / D);
      acc += (double)(((Gs[i] * I[i]) * (float)t) / sd);
    }
  }
  red[threadIdx.x] = acc;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if ((int)threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
    __syncthreads();
  }
  if (threadIdx.x == 0) part[s] = red[0];
}

// grad_decay[h] = sum over batch (in order) of the stream partials.
__global__ __launch_bounds__(256) void decay_final_kernel(const double* __restrict__ part,
                                                          float* __restrict__ out, int B, int H) {
  const int h = blockIdx.x * 256 + threadIdx.x;
  if (h >= H) return;
  double acc = 0.0;
  for (int b = 0; b < B; ++b) acc += part[(int64_t)b * H + h];
  out[h] = (float)acc;
}

// gv[b, 0, t, e] = sum over heads (in order) of gvh[b, h, t, e].
__global__ __launch_bounds__(256) void head_sum_kernel(const float* __restrict__ gvh, float* __restrict__ gv,
                                                       int64_t B, int H, int64_t TD) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= B * TD) return;
  const int64_t b = i / TD, j = i - b * TD;
  float acc = 0.0f;
  for (int h = 0; h < H; ++h) acc += gvh[(b * H + h) * TD + j];
  gv[i] = acc;
}

// gp[s, t, e] = g[s, t, e] * d^t.
__global__ __launch_bounds__(256) void rowscale_kernel(const float* __restrict__ g, float* __restrict__ gp,
                                                       const float* __restrict__ decay, int H, int T, int D,
                                                       int64_t total) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  const int64_t s = i / ((int64_t)T * D);
  const int t = (int)((i / D) % T);
  const float d = decay ? decay[s % H] : 1.0f;
  gp[i] = g[i] * dpowf(d, t);
}

inline unsigned cdivu(int64_t a, int64_t b) { return (unsigned)((a + b - 1) / b); }

}  // namespace

bdh_status run_attention_vjp(const VjpArgs& a, hipStream_t st, uint64_t* launches) {
  const int64_t B = a.B, H = a.H, Hv = a.Hv, T = a.T, N = a.N, D = a.D, S = B * H;
  const int64_t TT = T * T;
  void *ps = nullptr, *pgs = nullptr, *pm = nullptr, *ptd = nullptr, *ppart = nullptr;
  bdh_status s = scratch(st, SLOT_VJP_S, (size_t)(S * TT) * sizeof(float), &ps);
  if (s != BDH_OK) return s;
  s = scratch(st, SLOT_VJP_GS, (size_t)(S * TT) * sizeof(float), &pgs);
  if (s != BDH_OK) return s;
  s = scratch(st, SLOT_VJP_M, (size_t)(S * TT) * sizeof(float), &pm);
  if (s != BDH_OK) return s;
  // [S, T, D] buffers: per-head grad_v (Hv = 1), IC, G * d^t
  s = scratch(st, SLOT_VJP_TD, (size_t)(3 * S * T * D) * sizeof(float), &ptd);
  if (s != BDH_OK) return s;
  s = scratch(st, SLOT_VJP_PART, (size_t)S * sizeof(double), &ppart);
  if (s != BDH_OK) return s;
  // Split-K partials of the products over N (S and IC) and over T (grad_v).
  size_t pe = gf32::split_k_elems(S, (int)T, (int)T, (int)N);
  const size_t pe_ic = gf32::split_k_elems(S, (int)T, (int)D, (int)N);
  const size_t pe_gv = gf32::split_k_elems(S, (int)T, (int)D, (int)T);
  pe = pe > pe_ic ? pe : pe_ic;
  pe = pe > pe_gv ? pe : pe_gv;
  float* part = nullptr;
  if (pe) {
    void* pp = nullptr;
    s = scratch(st, SLOT_GEMM_PART, pe * sizeof(float), &pp);
    if (s != BDH_OK) return s;
    part = (float*)pp;
  }
  float* Sc = (float*)ps;
  float* GS = (float*)pgs;
  float* Msym = (float*)pm;
  float* gvh = (float*)ptd;
  float* ic = gvh + S * T * D;
  float* gp = ic + S * T * D;
  uint64_t n = 0;

  // Strides: query / grad_out / grad_q by stream (b*H + h); value by
  // (b, h) with a zero head stride when Hv = 1.
  const int64_t sVi = Hv == 1 ? 0 : T * D;
  GemmF32 g{};
  g.H = (int)H;
  g.decay = a.decay;
  // S = tril(-1)(Q Q^T) * D
  g.A = a.q; g.sAo = H * T * N; g.sAi = T * N; g.sAm = N; g.sAk = 1;
  g.B = a.q; g.sBo = H * T * N; g.sBi = T * N; g.sBn = N; g.sBk = 1;
  g.C = Sc; g.sCo = H * TT; g.sCi = TT; g.sCm = T; g.sCn = 1;
  g.M = (int)T; g.N = (int)T; g.K = (int)N;
  BDH_HIP_TRY(gemm<E_TRIL_DECAY>(g, S, st, part, pe, &n));
  // GS = tril(-1)(G V^T)
  g.A = a.g; g.sAo = H * T * D; g.sAi = T * D; g.sAm = D; g.sAk = 1;
  g.B = a.v; g.sBo = Hv * T * D; g.sBi = sVi; g.sBn = D; g.sBk = 1;
  g.C = GS;
  g.K = (int)D;
  BDH_HIP_TRY(gemm<E_TRIL>(g, S, st, part, pe, &n));
  // M = GS * D + (GS * D)^T
  hipLaunchKernelGGL(msym_kernel, dim3(cdivu(TT, 256 * 16) , (unsigned)S), dim3(256), 0, st, (const float*)GS,
                     Msym, a.decay, (int)H, (int)T);
  BDH_HIP_TRY(hipGetLastError());
  ++n;
  // grad_q = M Q
  g.A = Msym; g.sAo = H * TT; g.sAi = TT; g.sAm = T; g.sAk = 1;
  g.B = a.q; g.sBo = H * T * N; g.sBi = T * N; g.sBn = 1; g.sBk = N;
  g.C = a.grad_q; g.sCo = H * T * N; g.sCi = T * N; g.sCm = N; g.sCn = 1;
  g.M = (int)T; g.N = (int)N; g.K = (int)T;
  BDH_HIP_TRY(gemm<E_STORE>(g, S, st, part, pe, &n));
  // grad_v = S^T G (per head; summed over heads for shared values)
  g.A = Sc; g.sAo = H * TT; g.sAi = TT; g.sAm = 1; g.sAk = T;
  g.B = a.g; g.sBo = H * T * D; g.sBi = T * D; g.sBn = 1; g.sBk = D;
  if (Hv == 1) {
    g.C = gvh; g.sCo = H * T * D; g.sCi = T * D;
  } else {
    g.C = a.grad_v; g.sCo = H * T * D; g.sCi = T * D;
  }
  g.sCm = D; g.sCn = 1;
  g.M = (int)T; g.N = (int)D; g.K = (int)T;
  BDH_HIP_TRY(gemm<E_STORE>(g, S, st, part, pe, &n));
  if (Hv == 1) {
    hipLaunchKernelGGL(head_sum_kernel, dim3(cdivu(B * T * D, 256)), dim3(256), 0, st, (const float*)gvh,
                       a.grad_v, B, (int)H, T * D);
    BDH_HIP_TRY(hipGetLastError());
    ++n;
  }
  if (a.rho0) {
    // IC = (Q rho0) * d^t  (the decay gradient's state term)
    g.A = a.q; g.sAo = H * T * N; g.sAi = T * N; g.sAm = N; g.sAk = 1;
    g.B = a.rho0; g.sBo = H * N * D; g.sBi = N * D; g.sBn = 1; g.sBk = D;
    g.C = ic; g.sCo = H * T * D; g.sCi = T * D; g.sCm = D; g.sCn = 1;
    g.M = (int)T; g.N = (int)D; g.K = (int)N;
    BDH_HIP_TRY(gemm<E_ROWSCALE>(g, S, st, part, pe, &n));
    // grad_q += (G rho0^T) * d^t
    g.A = a.g; g.sAo = H * T * D; g.sAi = T * D; g.sAm = D; g.sAk = 1;
    g.B = a.rho0; g.sBo = H * N * D; g.sBi = N * D; g.sBn = D; g.sBk = 1;
    g.C = a.grad_q; g.sCo = H * T * N; g.sCi = T * N; g.sCm = N; g.sCn = 1;
    g.M = (int)T; g.N = (int)N; g.K = (int)D;
    BDH_HIP_TRY(gemm<E_ROWSCALE_ACC>(g, S, st, part, pe, &n));
    if (a.grad_rho0) {
      // grad_rho0 = Q^T (G * d^t)
      hipLaunchKernelGGL(rowscale_kernel, dim3(cdivu(S * T * D, 256)), dim3(256), 0, st, a.g, gp, a.decay,
                         (int)H, (int)T, (int)D, S * T * D);
      BDH_HIP_TRY(hipGetLastError());
      g.A = a.q; g.sAo = H * T * N; g.sAi = T * N; g.sAm = 1; g.sAk = N;
      g.B = gp; g.sBo = H * T * D; g.sBi = T * D; g.sBn = 1; g.sBk = D;
      g.C = a.grad_rho0; g.sCo = H * N * D; g.sCi = N * D; g.sCm = D; g.sCn = 1;
      g.M = (int)N; g.N = (int)D; g.K = (int)T;
      BDH_HIP_TRY(gemm<E_STORE>(g, S, st, part, pe, &n));
      ++n;
    }
  }
  if (a.grad_decay) {
    hipLaunchKernelGGL(decay_partial_kernel, dim3((unsigned)S), dim3(256), 0, st, (const float*)GS,
                       (const float*)Sc, a.g, a.rho0 ? (const float*)ic : nullptr, a.decay, (int)H, (int)T,
                       (int)D, a.recurrent_eps ? 1 : 0, (double*)ppart);
    BDH_HIP_TRY(hipGetLastError());
    hipLaunchKernelGGL(decay_final_kernel, dim3(cdivu(H, 256)), dim3(256), 0, st, (const double*)ppart,
                       a.grad_decay, (int)B, (int)H);
    BDH_HIP_TRY(hipGetLastError());
    n += 2;
  }
  if (launches) *launches += n;
  return BDH_OK;
}

}  // namespace bdh
