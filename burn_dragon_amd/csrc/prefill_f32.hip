// fp32 path of the recurrent forward (any shape, decay, shared or per-head
// values).  It evaluates the same closed form as the reference's dense-score
// executor (linear.rs:221-400), one state-carry interval of L tokens at a time:
//   S      = tril(-1)(Q Q^T * d^(r-c))                       [gram]
//   ctx    = S V + (Q * d^r) rho                              [context]
//   rho'   = rho * d^L + (Q * d^(L-r))^T V                     [state]
// with r, c token offsets inside the interval.  The three are LDS-tiled fp32
// FMA kernels (64x64 tiles, 256 threads, 4x4 outputs per thread).
#include "bdh_internal.h"

namespace bdh {
namespace {

constexpr int FT = 64;
constexpr int FK = 16;

// acc += A(64 x K) * B(K x 64).  fa(m, k) / fb(k, n) return the element or 0
// out of range.  *_KCONTIG picks the thread->element map that keeps global
// reads contiguous for a K-contiguous or M/N-contiguous operand.
template <bool A_KCONTIG, bool B_KCONTIG, class FA, class FB>
__device__ __forceinline__ void tile_mm(float (&acc)[4][4], FA fa, FB fb, int K,
                                        float (*smA)[FT + 4], float (*smB)[FT + 4]) {
  const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
  for (int k0 = 0; k0 < K; k0 += FK) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = tid + i * 256;
      int m, k;
      if (A_KCONTIG) { m = e >> 4; k = e & 15; } else { k = e >> 6; m = e & 63; }
      smA[k][m] = fa(m, k0 + k);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = tid + i * 256;
      int n, k;
      if (B_KCONTIG) { n = e >> 4; k = e & 15; } else { k = e >> 6; n = e & 63; }
      smB[k][n] = fb(k0 + k, n);
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < FK; ++k) {
      const float4 a = *reinterpret_cast<const float4*>(&smA[k][ty * 4]);
      const float4 b = *reinterpret_cast<const float4*>(&smB[k][tx * 4]);
      const float av[4] = {a.x, a.y, a.z, a.w};
      const float bv[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(av[i], bv[j], acc[i][j]);
    }
    __syncthreads();
  }
}

__device__ __forceinline__ const float* value_base(const float* v, int64_t s, int64_t H,
                                                   int64_t Hv, int64_t T, int64_t D) {
  const int64_t b = s / H, h = s - b * H;
  return v + (b * Hv + (Hv == 1 ? 0 : h)) * T * D;
}

__device__ __forceinline__ float dpow(const float* decay, int64_t h, float e) {
  return decay ? powf(decay[h], e) : 1.0f;
}

__global__ __launch_bounds__(256) void gram_f32_kernel(const float* __restrict__ q,
                                                       float* __restrict__ scores,
                                                       const float* __restrict__ decay,
                                                       int64_t H, int64_t T, int64_t N,
                                                       int64_t t0, int64_t L, int64_t ldS) {
  const int jt = blockIdx.x, it = blockIdx.y;
  if (jt > it) return;  // strictly above the diagonal: never read
  const int64_t s = blockIdx.z;
  const int64_t i0 = (int64_t)it * FT, j0 = (int64_t)jt * FT;
  __shared__ float smA[FK][FT + 4];
  __shared__ float smB[FK][FT + 4];
  const float* Q = q + (s * T + t0) * N;
  float acc[4][4] = {};
  auto fa = [&](int m, int k) -> float {
    return (i0 + m < L && k < N) ? Q[(i0 + m) * N + k] : 0.0f;
  };
  auto fb = [&](int k, int n) -> float {
    return (j0 + n < L && k < N) ? Q[(j0 + n) * N + k] : 0.0f;
  };
  tile_mm<true, true>(acc, fa, fb, (int)N, smA, smB);
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int64_t h = s % H;
  float* Sg = scores + s * ldS * ldS;
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    const int64_t ti = i0 + ty * 4 + a;
    if (ti >= L) continue;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int64_t tj = j0 + tx * 4 + b;
      if (tj >= L) continue;
      Sg[ti * ldS + tj] = tj < ti ? acc[a][b] * dpow(decay, h, (float)(ti - tj)) : 0.0f;
    }
  }
}

__global__ __launch_bounds__(256) void ctx_f32_kernel(
    const float* __restrict__ q, const float* __restrict__ v, const float* __restrict__ scores,
    const float* __restrict__ rho, const float* __restrict__ decay, float* __restrict__ ctx,
    int64_t H, int64_t Hv, int64_t T, int64_t N, int64_t D, int64_t t0, int64_t L,
    int64_t ldS) {
  const int64_t e0 = (int64_t)blockIdx.x * FT, i0 = (int64_t)blockIdx.y * FT;
  const int64_t s = blockIdx.z;
  __shared__ float smA[FK][FT + 4];
  __shared__ float smB[FK][FT + 4];
  const float* V = value_base(v, s, H, Hv, T, D) + t0 * D;
  const float* Sg = scores + s * ldS * ldS;
  float acc[4][4] = {};
  const int64_t kend = (i0 + FT < L) ? i0 + FT : L;
  auto fs = [&](int m, int k) -> float {
    return (i0 + m < L && k < kend) ? Sg[(i0 + m) * ldS + k] : 0.0f;
  };
  auto fv = [&](int k, int n) -> float {
    return (k < kend && e0 + n < D) ? V[k * D + e0 + n] : 0.0f;
  };
  tile_mm<true, false>(acc, fs, fv, (int)kend, smA, smB);
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int64_t h = s % H;
  if (rho) {
    float acc2[4][4] = {};
    const float* Q = q + (s * T + t0) * N;
    const float* R = rho + s * N * D;
    auto fq = [&](int m, int k) -> float {
      return (i0 + m < L && k < N) ? Q[(i0 + m) * N + k] : 0.0f;
    };
    auto fr = [&](int k, int n) -> float {
      return (k < N && e0 + n < D) ? R[(int64_t)k * D + e0 + n] : 0.0f;
    };
    tile_mm<true, false>(acc2, fq, fr, (int)N, smA, smB);
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const float w = dpow(decay, h, (float)(i0 + ty * 4 + a));
#pragma unroll
      for (int b = 0; b < 4; ++b) acc[a][b] = fmaf(w, acc2[a][b], acc[a][b]);
    }
  }
  float* C = ctx + (s * T + t0) * D;
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    const int64_t ti = i0 + ty * 4 + a;
    if (ti >= L) continue;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int64_t e = e0 + tx * 4 + b;
      if (e < D) C[ti * D + e] = acc[a][b];
    }
  }
}

__global__ __launch_bounds__(256) void state_f32_kernel(
    const float* __restrict__ q, const float* __restrict__ v, const float* rho_in,
    float* rho_out, const float* __restrict__ decay, int64_t H, int64_t Hv, int64_t T,
    int64_t N, int64_t D, int64_t t0, int64_t L) {
  const int64_t e0 = (int64_t)blockIdx.x * FT, n0 = (int64_t)blockIdx.y * FT;
  const int64_t s = blockIdx.z;
  const int64_t h = s % H;
  __shared__ float smA[FK][FT + 4];
  __shared__ float smB[FK][FT + 4];
  const float* Q = q + (s * T + t0) * N;
  const float* V = value_base(v, s, H, Hv, T, D) + t0 * D;
  float acc[4][4] = {};
  auto fq = [&](int m, int k) -> float {
    if (n0 + m >= N || k >= L) return 0.0f;
    const float x = Q[(int64_t)k * N + n0 + m];
    return decay ? x * dpow(decay, h, (float)(L - k)) : x;
  };
  auto fv = [&](int k, int n) -> float {
    return (k < L && e0 + n < D) ? V[(int64_t)k * D + e0 + n] : 0.0f;
  };
  tile_mm<false, false>(acc, fq, fv, (int)L, smA, smB);
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const float carry = dpow(decay, h, (float)L);
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    const int64_t n = n0 + ty * 4 + a;
    if (n >= N) continue;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int64_t e = e0 + tx * 4 + b;
      if (e >= D) continue;
      const int64_t idx = (s * N + n) * D + e;
      const float prev = rho_in ? rho_in[idx] * carry : 0.0f;
      rho_out[idx] = prev + acc[a][b];
    }
  }
}

inline unsigned cdiv(int64_t a, int64_t b) { return (unsigned)((a + b - 1) / b); }

}  // namespace

hipError_t run_f32_path(const F32Args& a, hipStream_t st, uint64_t* launches) {
  const int64_t S = a.B * a.H;
  const float* rho_cur = a.rho_in;
  for (int64_t t0 = 0; t0 < a.T; t0 += a.Lmax) {
    const int64_t L = (a.T - t0 < a.Lmax) ? a.T - t0 : a.Lmax;
    const unsigned nt = cdiv(L, FT);
    hipLaunchKernelGGL(gram_f32_kernel, dim3(nt, nt, (unsigned)S), dim3(256), 0, st, a.q,
                       a.scores, a.decay, a.H, a.T, a.N, t0, L, a.Lmax);
    hipLaunchKernelGGL(ctx_f32_kernel, dim3(cdiv(a.D, FT), nt, (unsigned)S), dim3(256), 0, st,
                       a.q, a.v, a.scores, rho_cur, a.decay, a.ctx, a.H, a.Hv, a.T, a.N, a.D,
                       t0, L, a.Lmax);
    if (a.state)
      hipLaunchKernelGGL(state_f32_kernel, dim3(cdiv(a.D, FT), cdiv(a.N, FT), (unsigned)S),
                         dim3(256), 0, st, a.q, a.v, rho_cur, a.rho_out, a.decay, a.H, a.Hv,
                         a.T, a.N, a.D, t0, L);
    if (launches) *launches += a.state ? 3 : 2;
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    rho_cur = a.rho_out;
  }
  return hipSuccess;
}

}  // namespace bdh
