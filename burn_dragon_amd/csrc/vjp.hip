// VJP of the causal linear attention (context gradient), fp32 on gfx950.
//
// The reference has two backward paths with one closed form: the dense
// causal VJP (kernel/src/dense_causal_attention/backward_runtime.rs:36-148)
// and the recurrent backward (kernel/src/recurrent/backward_runtime.rs,
// state history and a reverse-time adjoint).  With Q = K = query, G the
// context gradient, D[r, c] = d^(r-c) and gap = r - c below the diagonal, one
// interval of L tokens starting from the state rho_iv gives
//   S      = tril(-1)(Q Q^T) * D            [L, L]   gemm, TRIL_DECAY epilogue
//   GS     = tril(-1)(G V^T)                [L, L]   gemm, TRIL epilogue
//   M      = GS * D + (GS * D)^T            [L, L]   elementwise
//   grad_q = M Q  [+ (G rho_iv^T) * d^t]    [L, N]   gemm (+ ROWSCALE_ACC)
//   grad_v = S^T G                          [L, D]   gemm, heads summed for Hv = 1
//   grad_d = sum((GS * gap) * S) / sd  [+ sum((G * IC) * t) / sd],
//            IC = (Q rho_iv) * d^t                    gemm ROWSCALE + reduction
// Longer sequences run as intervals of at most 1024 tokens with the state
// history and a reverse scan (the reference's recurrent backward does the
// same per token): the states rho_iv are recomputed forward, then, from the
// last interval back, Gamma_iv = dL/d rho_iv = Q^T (G * d^t) + d^L Gamma_{iv+1}
// carries the later intervals' gradient into each interval through
// rho_{iv+1} = rho_iv d^L + (Q * d^(L-t))^T V:
//   grad_q += d^(L-t) (V Gamma_{iv+1}^T)      gemm, ROWREV_ACC epilogue
//   grad_v += d^(L-t) (Q Gamma_{iv+1})        gemm P, then a scaled add
//   grad_d += sum (L-t) d^(L-t) P V / sd + L d^L <rho_iv, Gamma_{iv+1}> / sd
// and grad_rho0 = Gamma_0.
// Every product is a batched fp32 GEMM on the fp32 MFMAs (exact fp32
// products, fp32 accumulation; bdh_gemm_f32.h) with generic strides, so
// transposed operands need no copy.  Reductions are per stream (f64) and then
// per head in a fixed order: the result is deterministic.
#include "bdh_gemm_f32.h"

namespace bdh {
namespace {

using gf32::dpowf;
using gf32::gemm;
using gf32::GemmF32;
using gf32::E_CARRY;
using gf32::E_ROWREV_ACC;
using gf32::E_ROWSCALE;
using gf32::E_ROWSCALE_ACC;
using gf32::E_STORE;
using gf32::E_TRIL;
using gf32::E_TRIL_DECAY;

constexpr int64_t kVjpInterval = 1024;  // tokens per interval of the reverse scan
constexpr int kCrossBlocks = 64;        // workgroups per stream of the state-term reduction

__device__ __forceinline__ float decay_sd(float d, int recurrent_eps) {
  if (recurrent_eps) return (d < 1e-8f && d > -1e-8f) ? 1e-8f : d;
  return d + 1e-12f;
}

// M[s, r, c] = W[r, c] + W[c, r], W[r, c] = r > c ? GS[r, c] d^(r - c) : 0,
// over the leading L x L of ld x ld blocks.
__global__ __launch_bounds__(256) void msym_kernel(const float* __restrict__ gs, float* __restrict__ m,
                                                   const float* __restrict__ decay, int H, int L, int ld) {
  const int64_t s = blockIdx.y;
  const float d = decay ? decay[s % H] : 1.0f;
  const float* G = gs + s * (int64_t)ld * ld;
  float* Mo = m + s * (int64_t)ld * ld;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < (int64_t)L * L; i += (int64_t)gridDim.x * 256) {
    const int r = (int)(i / L), c = (int)(i - (int64_t)r * L);
    float v = 0.0f;
    if (r > c) v = G[(int64_t)r * ld + c] * dpowf(d, r - c);
    else if (c > r) v = G[(int64_t)c * ld + r] * dpowf(d, c - r);
    Mo[(int64_t)r * ld + c] = v;
  }
}

__global__ __launch_bounds__(256) void zero_f64_kernel(double* __restrict__ p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0.0;
}

// Adds stream s's decay-gradient terms of one interval to part[s], in the
// reference's element op order: ((GS * gap) * S) / sd over the lower
// triangle, plus, with a state, ((G * IC) * t) / sd over [L, D].  f64 sums,
// fixed order.
__global__ __launch_bounds__(256) void decay_partial_kernel(const float* __restrict__ gs,
                                                            const float* __restrict__ sc, int ld,
                                                            const float* __restrict__ g, int64_t g_stride,
                                                            const float* __restrict__ ic,
                                                            const float* __restrict__ decay, int H, int L,
                                                            int D, int recurrent_eps,
                                                            double* __restrict__ part) {
  __shared__ double red[256];
  const int64_t s = blockIdx.x;
  const float sd = decay_sd(decay ? decay[s % H] : 1.0f, recurrent_eps);
  double acc = 0.0;
  const float* GS = gs + s * (int64_t)ld * ld;
  const float* SC = sc + s * (int64_t)ld * ld;
  for (int64_t i = threadIdx.x; i < (int64_t)L * L; i += 256) {
    const int r = (int)(i / L), c = (int)(i - (int64_t)r * L);
    if (r > c) acc += (double)(((GS[(int64_t)r * ld + c] * (float)(r - c)) * SC[(int64_t)r * ld + c]) / sd);
  }
  if (ic) {
    const float* Gs = g + s * g_stride;
    const float* I = ic + s * (int64_t)ld * D;
    for (int64_t i = threadIdx.x; i < (int64_t)L * D; i += 256) {
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
  if (threadIdx.x == 0) part[s] += red[0];
}

// The decay terms through the next state, per stream and block of a fixed
// split: block j < kCrossBlocks sums L d^L rho_iv * Gamma / sd over its slice
// of [N, D]; block kCrossBlocks sums (L - t) d^(L - t) P[t, e] V[t, e] / sd.
// Results go to cpart[s, j] (f64), folded in order by cross_fold_kernel.
__global__ __launch_bounds__(256) void decay_cross_kernel(const float* __restrict__ p, int ld,
                                                          const float* __restrict__ v, int64_t sVo,
                                                          int64_t sVi, const float* __restrict__ rho,
                                                          const float* __restrict__ gamma,
                                                          const float* __restrict__ decay, int H, int L,
                                                          int64_t ND, int D, int recurrent_eps,
                                                          double* __restrict__ cpart) {
  __shared__ double red[256];
  const int64_t s = blockIdx.y;
  const int j = blockIdx.x;
  const int64_t b = s / H, h = s - b * H;
  const float d = decay ? decay[h] : 1.0f;
  const float sd = decay_sd(d, recurrent_eps);
  double acc = 0.0;
  if (j < kCrossBlocks) {
    if (rho) {
      const float w = (float)L * dpowf(d, L);
      const int64_t per = (ND + kCrossBlocks - 1) / kCrossBlocks;
      const int64_t lo = j * per, hi = lo + per < ND ? lo + per : ND;
      const float* R = rho + s * ND;
      const float* Gm = gamma + s * ND;
      for (int64_t i = lo + threadIdx.x; i < hi; i += 256) acc += (double)((R[i] * Gm[i]) * w / sd);
    }
  } else {
    const float* P = p + s * (int64_t)ld * D;
    const float* V = v + b * sVo + h * sVi;
    for (int64_t i = threadIdx.x; i < (int64_t)L * D; i += 256) {
      const int t = (int)(i / D);
      acc += (double)(((P[i] * V[i]) * ((float)(L - t) * dpowf(d, L - t))) / sd);
    }
  }
  red[threadIdx.x] = acc;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if ((int)threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
    __syncthreads();
  }
  if (threadIdx.x == 0) cpart[s * (kCrossBlocks + 1) + j] = red[0];
}

__global__ __launch_bounds__(256) void cross_fold_kernel(const double* __restrict__ cpart,
                                                         double* __restrict__ part, int64_t S) {
  const int64_t s = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (s >= S) return;
  double acc = 0.0;
  for (int j = 0; j <= kCrossBlocks; ++j) acc += cpart[s * (kCrossBlocks + 1) + j];
  part[s] += acc;
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

// gv[b, t, e] (one value head, rows of stride gv_stride per batch from the
// slice's first token) = sum over heads (in order) of gvh[b*H + h, t, e]
// (ld rows a stream).
__global__ __launch_bounds__(256) void head_sum_kernel(const float* __restrict__ gvh, int ld,
                                                       float* __restrict__ gv, int64_t gv_stride, int64_t B,
                                                       int H, int L, int D) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t LD = (int64_t)L * D;
  if (i >= B * LD) return;
  const int64_t b = i / LD, j = i - b * LD;
  float acc = 0.0f;
  for (int h = 0; h < H; ++h) acc += gvh[(b * H + h) * (int64_t)ld * D + j];
  gv[b * gv_stride + j] = acc;
}

// gp[s, t, e] = g[s, t, e] * d^t over the interval (g rows of stride
// g_stride per stream, gp of ld * D).
__global__ __launch_bounds__(256) void rowscale_kernel(const float* __restrict__ g, int64_t g_stride,
                                                       float* __restrict__ gp, int ld,
                                                       const float* __restrict__ decay, int H, int L,
                                                       int D, int64_t S) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t LD = (int64_t)L * D;
  if (i >= S * LD) return;
  const int64_t s = i / LD, j = i - s * LD;
  const int t = (int)(j / D);
  const float d = decay ? decay[s % H] : 1.0f;
  gp[s * (int64_t)ld * D + j] = g[s * g_stride + j] * dpowf(d, t);
}

// dst[s, t, e] += d^(L - t) P[s, t, e] (dst rows of stride dst_stride per
// stream, P of ld * D).
__global__ __launch_bounds__(256) void add_rowrev_kernel(float* __restrict__ dst, int64_t dst_stride,
                                                         const float* __restrict__ P, int ld,
                                                         const float* __restrict__ decay, int H, int L,
                                                         int D, int64_t S) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t LD = (int64_t)L * D;
  if (i >= S * LD) return;
  const int64_t s = i / LD, j = i - s * LD;
  const int t = (int)(j / D);
  const float d = decay ? decay[s % H] : 1.0f;
  dst[s * dst_stride + j] += P[s * (int64_t)ld * D + j] * dpowf(d, L - t);
}

inline unsigned cdivu(int64_t a, int64_t b) { return (unsigned)((a + b - 1) / b); }

}  // namespace

bdh_status run_attention_vjp(const VjpArgs& a, hipStream_t st, uint64_t* launches) {
  const int64_t B = a.B, H = a.H, Hv = a.Hv, T = a.T, N = a.N, D = a.D, S = B * H;
  const int64_t Lv = T < kVjpInterval ? T : kVjpInterval;
  const int64_t n_iv = (T + Lv - 1) / Lv;
  const int64_t LL = Lv * Lv, ND = N * D;
  const bool want_d = a.grad_decay != nullptr;
  void *ps = nullptr, *pgs = nullptr, *pm = nullptr, *ptd = nullptr, *ppart = nullptr;
  void *prho = nullptr, *pgam = nullptr;
  bdh_status s = scratch(st, SLOT_VJP_S, (size_t)(S * LL) * sizeof(float), &ps);
  if (s != BDH_OK) return s;
  s = scratch(st, SLOT_VJP_GS, (size_t)(S * LL) * sizeof(float), &pgs);
  if (s != BDH_OK) return s;
  s = scratch(st, SLOT_VJP_M, (size_t)(S * LL) * sizeof(float), &pm);
  if (s != BDH_OK) return s;
  // [S, Lv, D] buffers: per-head grad_v (Hv = 1), IC, G * d^t, P = Q Gamma
  s = scratch(st, SLOT_VJP_TD, (size_t)(4 * S * Lv * D) * sizeof(float), &ptd);
  if (s != BDH_OK) return s;
  // decay partials [S] and the state-term partials [S, kCrossBlocks + 1], f64
  s = scratch(st, SLOT_VJP_PART, (size_t)(S * (kCrossBlocks + 2)) * sizeof(double), &ppart);
  if (s != BDH_OK) return s;
  if (n_iv > 1) {
    // states at the interval starts 1 .. n_iv - 1, and two Gamma buffers
    s = scratch(st, SLOT_VJP_RHO, (size_t)((n_iv - 1) * S * ND) * sizeof(float), &prho);
    if (s != BDH_OK) return s;
    s = scratch(st, SLOT_VJP_GAMMA, (size_t)(2 * S * ND) * sizeof(float), &pgam);
    if (s != BDH_OK) return s;
  }
  // Split-K partials of the products over N (S, IC, P) and over L (grad_v).
  size_t pe = gf32::split_k_elems(S, (int)Lv, (int)Lv, (int)N);
  const size_t pe_ic = gf32::split_k_elems(S, (int)Lv, (int)D, (int)N);
  const size_t pe_gv = gf32::split_k_elems(S, (int)Lv, (int)D, (int)Lv);
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
  float* ic = gvh + S * Lv * D;
  float* gp = ic + S * Lv * D;
  float* Pq = gp + S * Lv * D;
  double* dpart = (double*)ppart;
  double* cpart = dpart + S;
  float* states = (float*)prho;
  float* gam[2] = {(float*)pgam, pgam ? (float*)pgam + S * ND : nullptr};
  uint64_t n = 0;

  // Strides: query / grad_out / grad_q by stream (b*H + h); value by
  // (b, h) with a zero head stride when Hv = 1.
  const int64_t sVo = Hv * T * D, sVi = Hv == 1 ? 0 : T * D;
  if (want_d) {
    hipLaunchKernelGGL(zero_f64_kernel, dim3(cdivu(S, 256)), dim3(256), 0, st, dpart, S);
    BDH_HIP_TRY(hipGetLastError());
    ++n;
  }
  // Forward: the states at the interval starts.
  for (int64_t iv = 0; iv + 1 < n_iv; ++iv) {
    const int64_t t0 = iv * Lv;
    GemmF32 g{};
    g.H = (int)H;
    g.decay = a.decay;
    g.A = a.q + t0 * N; g.sAo = H * T * N; g.sAi = T * N; g.sAm = 1; g.sAk = N;
    g.B = a.v + t0 * D; g.sBo = sVo; g.sBi = sVi; g.sBn = 1; g.sBk = D;
    g.C = states + iv * S * ND; g.sCo = H * ND; g.sCi = ND; g.sCm = D; g.sCn = 1;
    g.src = iv == 0 ? a.rho0 : states + (iv - 1) * S * ND;
    g.M = (int)N; g.N = (int)D; g.K = (int)Lv;
    g.kpow = (int)Lv;
    BDH_HIP_TRY((gemm<E_CARRY, true>(g, S, st, nullptr, 0, &n)));
  }

  // Reverse scan over the intervals.
  const float* gam_next = nullptr;
  for (int64_t iv = n_iv - 1; iv >= 0; --iv) {
    const int64_t t0 = iv * Lv;
    const int64_t L = (T - t0 < Lv) ? T - t0 : Lv;
    const float* rho_iv = iv == 0 ? a.rho0 : states + (iv - 1) * S * ND;
    const float* Q = a.q + t0 * N;
    const float* G = a.g + t0 * D;
    const float* V = a.v + t0 * D;
    float* GQ = a.grad_q + t0 * N;
    GemmF32 g{};
    g.H = (int)H;
    g.decay = a.decay;
    // S = tril(-1)(Q Q^T) * D
    g.A = Q; g.sAo = H * T * N; g.sAi = T * N; g.sAm = N; g.sAk = 1;
    g.B = Q; g.sBo = H * T * N; g.sBi = T * N; g.sBn = N; g.sBk = 1;
    g.C = Sc; g.sCo = H * LL; g.sCi = LL; g.sCm = Lv; g.sCn = 1;
    g.M = (int)L; g.N = (int)L; g.K = (int)N;
    BDH_HIP_TRY(gemm<E_TRIL_DECAY>(g, S, st, part, pe, &n));
    // GS = tril(-1)(G V^T)
    g.A = G; g.sAo = H * T * D; g.sAi = T * D; g.sAm = D; g.sAk = 1;
    g.B = V; g.sBo = sVo; g.sBi = sVi; g.sBn = D; g.sBk = 1;
    g.C = GS;
    g.K = (int)D;
    BDH_HIP_TRY(gemm<E_TRIL>(g, S, st, part, pe, &n));
    // M = GS * D + (GS * D)^T
    hipLaunchKernelGGL(msym_kernel, dim3(cdivu(L * L, 256 * 16), (unsigned)S), dim3(256), 0, st,
                       (const float*)GS, Msym, a.decay, (int)H, (int)L, (int)Lv);
    BDH_HIP_TRY(hipGetLastError());
    ++n;
    // grad_q = M Q
    g.A = Msym; g.sAo = H * LL; g.sAi = LL; g.sAm = Lv; g.sAk = 1;
    g.B = Q; g.sBo = H * T * N; g.sBi = T * N; g.sBn = 1; g.sBk = N;
    g.C = GQ; g.sCo = H * T * N; g.sCi = T * N; g.sCm = N; g.sCn = 1;
    g.M = (int)L; g.N = (int)N; g.K = (int)L;
    BDH_HIP_TRY(gemm<E_STORE>(g, S, st, part, pe, &n));
    // grad_v = S^T G (per head into gvh when heads share the value)
    float* gvt = Hv == 1 ? gvh : a.grad_v + t0 * D;
    const int64_t gvt_stride = Hv == 1 ? Lv * D : T * D;
    g.A = Sc; g.sAo = H * LL; g.sAi = LL; g.sAm = 1; g.sAk = Lv;
    g.B = G; g.sBo = H * T * D; g.sBi = T * D; g.sBn = 1; g.sBk = D;
    g.C = gvt; g.sCo = H * gvt_stride; g.sCi = gvt_stride; g.sCm = D; g.sCn = 1;
    g.M = (int)L; g.N = (int)D; g.K = (int)L;
    BDH_HIP_TRY(gemm<E_STORE>(g, S, st, part, pe, &n));
    if (rho_iv) {
      // IC = (Q rho_iv) * d^t  (the decay gradient's state term)
      g.A = Q; g.sAo = H * T * N; g.sAi = T * N; g.sAm = N; g.sAk = 1;
      g.B = rho_iv; g.sBo = H * ND; g.sBi = ND; g.sBn = 1; g.sBk = D;
      g.C = ic; g.sCo = H * Lv * D; g.sCi = Lv * D; g.sCm = D; g.sCn = 1;
      g.M = (int)L; g.N = (int)D; g.K = (int)N;
      if (want_d) BDH_HIP_TRY(gemm<E_ROWSCALE>(g, S, st, part, pe, &n));
      // grad_q += (G rho_iv^T) * d^t
      g.A = G; g.sAo = H * T * D; g.sAi = T * D; g.sAm = D; g.sAk = 1;
      g.B = rho_iv; g.sBo = H * ND; g.sBi = ND; g.sBn = D; g.sBk = 1;
      g.C = GQ; g.sCo = H * T * N; g.sCi = T * N; g.sCm = N; g.sCn = 1;
      g.M = (int)L; g.N = (int)N; g.K = (int)D;
      BDH_HIP_TRY(gemm<E_ROWSCALE_ACC>(g, S, st, part, pe, &n));
    }
    if (gam_next) {
      // P = Q Gamma_{iv+1}; grad_v += d^(L-t) P
      g.A = Q; g.sAo = H * T * N; g.sAi = T * N; g.sAm = N; g.sAk = 1;
      g.B = gam_next; g.sBo = H * ND; g.sBi = ND; g.sBn = 1; g.sBk = D;
      g.C = Pq; g.sCo = H * Lv * D; g.sCi = Lv * D; g.sCm = D; g.sCn = 1;
      g.M = (int)L; g.N = (int)D; g.K = (int)N;
      BDH_HIP_TRY(gemm<E_STORE>(g, S, st, part, pe, &n));
      hipLaunchKernelGGL(add_rowrev_kernel, dim3(cdivu(S * L * D, 256)), dim3(256), 0, st, gvt, gvt_stride,
                         (const float*)Pq, (int)Lv, a.decay, (int)H, (int)L, (int)D, S);
      BDH_HIP_TRY(hipGetLastError());
      ++n;
      // grad_q += d^(L-t) (V Gamma_{iv+1}^T)
      g.A = V; g.sAo = sVo; g.sAi = sVi; g.sAm = D; g.sAk = 1;
      g.B = gam_next; g.sBo = H * ND; g.sBi = ND; g.sBn = D; g.sBk = 1;
      g.C = GQ; g.sCo = H * T * N; g.sCi = T * N; g.sCm = N; g.sCn = 1;
      g.M = (int)L; g.N = (int)N; g.K = (int)D;
      g.kpow = (int)L;
      BDH_HIP_TRY(gemm<E_ROWREV_ACC>(g, S, st, part, pe, &n));
      g.kpow = 0;
    }
    if (Hv == 1) {
      hipLaunchKernelGGL(head_sum_kernel, dim3(cdivu(B * L * D, 256)), dim3(256), 0, st, (const float*)gvh,
                         (int)Lv, a.grad_v + t0 * D, T * D, B, (int)H, (int)L, (int)D);
      BDH_HIP_TRY(hipGetLastError());
      ++n;
    }
    if (want_d) {
      hipLaunchKernelGGL(decay_partial_kernel, dim3((unsigned)S), dim3(256), 0, st, (const float*)GS,
                         (const float*)Sc, (int)Lv, G, T * D, rho_iv ? (const float*)ic : nullptr, a.decay,
                         (int)H, (int)L, (int)D, a.recurrent_eps ? 1 : 0, dpart);
      BDH_HIP_TRY(hipGetLastError());
      ++n;
      if (gam_next) {
        hipLaunchKernelGGL(decay_cross_kernel, dim3(kCrossBlocks + 1, (unsigned)S), dim3(256), 0, st,
                           (const float*)Pq, (int)Lv, V, sVo, sVi, rho_iv, gam_next, a.decay, (int)H,
                           (int)L, ND, (int)D, a.recurrent_eps ? 1 : 0, cpart);
        BDH_HIP_TRY(hipGetLastError());
        hipLaunchKernelGGL(cross_fold_kernel, dim3(cdivu(S, 256)), dim3(256), 0, st, (const double*)cpart,
                           dpart, S);
        BDH_HIP_TRY(hipGetLastError());
        n += 2;
      }
    }
    // Gamma_iv = Q^T (G * d^t) + d^L Gamma_{iv+1}: needed by the interval
    // before, or as grad_rho0 for the first.
    float* gam_out = iv > 0 ? gam[iv & 1] : a.grad_rho0;
    if (gam_out) {
      hipLaunchKernelGGL(rowscale_kernel, dim3(cdivu(S * L * D, 256)), dim3(256), 0, st, G, T * D, gp,
                         (int)Lv, a.decay, (int)H, (int)L, (int)D, S);
      BDH_HIP_TRY(hipGetLastError());
      ++n;
      g = GemmF32{};
      g.H = (int)H;
      g.decay = a.decay;
      g.A = Q; g.sAo = H * T * N; g.sAi = T * N; g.sAm = 1; g.sAk = N;
      g.B = gp; g.sBo = H * Lv * D; g.sBi = Lv * D; g.sBn = 1; g.sBk = D;
      g.C = gam_out; g.sCo = H * ND; g.sCi = ND; g.sCm = D; g.sCn = 1;
      g.src = gam_next;
      g.M = (int)N; g.N = (int)D; g.K = (int)L;
      g.kpow = (int)L;
      BDH_HIP_TRY(gemm<E_CARRY>(g, S, st, part, pe, &n));
    }
    gam_next = gam_out;
  }
  if (want_d) {
    hipLaunchKernelGGL(decay_final_kernel, dim3(cdivu(H, 256)), dim3(256), 0, st, (const double*)dpart,
                       a.grad_decay, (int)B, (int)H);
    BDH_HIP_TRY(hipGetLastError());
    ++n;
  }
  if (launches) *launches += n;
  return BDH_OK;
}

}  // namespace bdh
