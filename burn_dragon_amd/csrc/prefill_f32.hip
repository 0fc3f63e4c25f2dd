// fp32 path of the recurrent forward (any shape, decay, shared or per-head
// values).  It evaluates the same closed form as the reference's dense-score
// executor (linear.rs:221-400), one state-carry interval of L tokens at a time:
//   S      = tril(-1)(Q Q^T * d^(r-c))                       [gram]
//   ctx    = S V + (Q * d^r) rho                              [context]
//   rho'   = rho * d^L + (Q * d^(L-r))^T V                     [state]
// with r, c token offsets inside the interval.  Each product is a batched
// fp32 GEMM on the matrix cores (bdh_gemm_f32.h: v_mfma_f32_16x16x4f32,
// exact fp32 products and fp32 accumulation), the masks and decay powers in
// its epilogue or operand loads:
//   gram     A = B = Q (rows t, k over N), epilogue tril(-1) * d^(r-c)
//   context  A = S (k limited to the causal part of the row block), B = V;
//            then A = Q, B = rho, epilogue += acc * d^r
//   state    A = Q^T (rows n, k over t, loaded d^(L-t)-scaled), B = V,
//            epilogue acc + rho * d^L (in place when rho_out is rho)
#include "bdh_gemm_f32.h"

namespace bdh {

using namespace gf32;

// Split-K partials of the gram and readout (K = N) and of S V (K = L).
size_t f32_path_part_elems(const F32Args& a) {
  const int64_t S = a.B * a.H;
  const int L = (int)(a.T < a.Lmax ? a.T : a.Lmax);
  const size_t g = split_k_elems(S, L, L, (int)a.N), r = split_k_elems(S, L, (int)a.D, (int)a.N);
  const size_t sv = split_k_elems(S, L, (int)a.D, L);
  const size_t m = g > r ? g : r;
  return m > sv ? m : sv;
}

hipError_t run_f32_path(const F32Args& a, hipStream_t st, uint64_t* launches) {
  const int64_t S = a.B * a.H, H = a.H, T = a.T, N = a.N, D = a.D, Lm = a.Lmax;
  const size_t pe = f32_path_part_elems(a);
  const int64_t sVo = a.Hv * T * D, sVi = a.Hv == 1 ? 0 : T * D;
  const float* rho_cur = a.rho_in;
  uint64_t n = 0;
  for (int64_t t0 = 0; t0 < T; t0 += Lm) {
    const int64_t L = (T - t0 < Lm) ? T - t0 : Lm;
    GemmF32 g{};
    g.H = (int)H;
    g.decay = a.decay;
    // S = tril(-1)(Q Q^T) * d^(r-c)  ->  scores [S, Lm, Lm]
    g.A = a.q + t0 * N; g.sAo = H * T * N; g.sAi = T * N; g.sAm = N; g.sAk = 1;
    g.B = a.q + t0 * N; g.sBo = H * T * N; g.sBi = T * N; g.sBn = N; g.sBk = 1;
    g.C = a.scores; g.sCo = H * Lm * Lm; g.sCi = Lm * Lm; g.sCm = Lm; g.sCn = 1;
    g.M = (int)L; g.N = (int)L; g.K = (int)N;
    hipError_t e = gemm<E_TRIL_DECAY>(g, S, st, a.part, pe, &n);
    if (e != hipSuccess) return e;
    // ctx = S V
    g = GemmF32{};
    g.H = (int)H;
    g.decay = a.decay;
    g.A = a.scores; g.sAo = H * Lm * Lm; g.sAi = Lm * Lm; g.sAm = Lm; g.sAk = 1;
    g.B = a.v + t0 * D; g.sBo = sVo; g.sBi = sVi; g.sBn = 1; g.sBk = D;
    g.C = a.ctx + t0 * D; g.sCo = H * T * D; g.sCi = T * D; g.sCm = D; g.sCn = 1;
    g.M = (int)L; g.N = (int)D; g.K = (int)L;
    g.kcausal = 1;
    e = gemm<E_STORE>(g, S, st, a.part, pe, &n);
    if (e != hipSuccess) return e;
    if (rho_cur) {
      // ctx += (Q * d^r) rho
      g.A = a.q + t0 * N; g.sAo = H * T * N; g.sAi = T * N; g.sAm = N; g.sAk = 1;
      g.B = rho_cur; g.sBo = H * N * D; g.sBi = N * D; g.sBn = 1; g.sBk = D;
      g.K = (int)N;
      g.kcausal = 0;
      e = gemm<E_ROWSCALE_ACC>(g, S, st, a.part, pe, &n);
      if (e != hipSuccess) return e;
    }
    if (a.state) {
      // rho' = rho * d^L + (Q * d^(L-t))^T V
      g = GemmF32{};
      g.H = (int)H;
      g.decay = a.decay;
      g.A = a.q + t0 * N; g.sAo = H * T * N; g.sAi = T * N; g.sAm = 1; g.sAk = N;
      g.B = a.v + t0 * D; g.sBo = sVo; g.sBi = sVi; g.sBn = 1; g.sBk = D;
      g.C = a.rho_out; g.sCo = H * N * D; g.sCi = N * D; g.sCm = D; g.sCn = 1;
      g.src = rho_cur;
      g.M = (int)N; g.N = (int)D; g.K = (int)L;
      g.kpow = (int)L;
      e = gemm<E_CARRY, true>(g, S, st, nullptr, 0, &n);
      if (e != hipSuccess) return e;
      rho_cur = a.rho_out;
    }
  }
  if (launches) *launches += n;
  return hipSuccess;
}

}  // namespace bdh
