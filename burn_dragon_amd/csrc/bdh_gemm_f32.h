// Batched fp32 GEMM on gfx950 matrix cores (v_mfma_f32_32x32x2f32: exact
// fp32 products, fp32 accumulation) with the epilogues of the recurrence's
// closed form.  Used by the fp32 forward (prefill_f32.hip) and the backward
// (vjp.hip).
//
//   C(m, n) = sum_k A(m, k) B(n, k),  batch b = (b / H, b % H):
//   X(i, j) = X + (b / H) * sXo + (b % H) * sXi + i * sXr + j * sXc
//
// Workgroups of 256 threads own 128 x 128 output tiles, each wave a 64 x 64
// block (2 x 2 MFMA blocks, 64 accumulators a lane).  K steps are 16 deep:
// the operands of step k + 1 are loaded into registers (16-byte loads where
// the operand is contiguous along k or along its rows) while step k is
// multiplied from LDS; LDS holds two steps, so one barrier a step suffices.
// A long K with few tiles is split into P ranges (split-K): each range's
// workgroup writes its raw sums to a partial buffer, and a reduce kernel
// adds the P partials in range order (deterministic) and applies the
// epilogue.
#pragma once

#include "bdh_internal.h"

namespace bdh {
namespace gf32 {

enum Epi {
  E_STORE = 0,     // C = acc
  E_TRIL,          // C = n < m ? acc : 0
  E_TRIL_DECAY,    // C = n < m ? acc * d^(m-n) : 0
  E_ROWSCALE,      // C = acc * d^m
  E_ROWSCALE_ACC,  // C += acc * d^m
  E_CARRY,         // C = acc + src * d^kpow (src null: acc)
  E_ROWREV_ACC     // C += acc * d^(kpow - m)
};

struct GemmF32 {
  const float* A;
  const float* B;
  float* C;
  const float* src;     // E_CARRY: addend with C's strides (may equal C)
  int64_t sAo, sAi, sAm, sAk;
  int64_t sBo, sBi, sBn, sBk;
  int64_t sCo, sCi, sCm, sCn;
  int M, N, K, H;
  int kpow;             // E_CARRY: carry power; KSCALE: A(m, k) *= d^(kpow - k)
  int kcausal;          // K of row block m0 limited to m0 + 128 (operand A lower triangular)
  const float* decay;   // [H] or null (ones)
  int a_vec, b_vec;     // 16-byte loads allowed (host-checked alignment)
  float* part;          // split-K partials [ksplit, batch, M, N] (ksplit > 1)
  int ksplit;
  int64_t batch;
};

constexpr int GT = 128;   // tile edge
constexpr int GK = 16;               // k step (32 measured slower: 2.24 against 2.17 ms, fp32 C2 shape)
constexpr int FE = GK / 2;           // operand elements a thread stages per step (128 x GK / 256)
constexpr int TPK = 256 / GK;        // threads per k row in the row-contiguous loader
constexpr int GP = 130;   // LDS row pitch (floats): k rows 8 apart fall on different banks

__device__ __forceinline__ float dpowf(float d, int e) { return powf(d, (float)e); }

__device__ __forceinline__ floatx16 mfma_f32(float a, float b, const floatx16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// FE elements of a 128 x GK operand tile for thread t, rows r0.. (R valid),
// k from kb (K valid):
//   k-contiguous (sk == 1): row t >> 1, k (t & 1) * FE .. + FE - 1;
//   row-contiguous (sr == 1): k t / TPK, rows (t % TPK) * FE .. + FE - 1;
//   otherwise as k-contiguous, element by element.
struct Frag {
  float v[FE];
};

__device__ __forceinline__ void load_frag(const float* X, int64_t sr, int64_t sk, int r0, int R, int kb,
                                          int K, bool vec, int t, Frag& f) {
  if (sr == 1 && sk != 1) {
    const int k = kb + t / TPK, r = r0 + (t % TPK) * FE;
    const float* p = X + (int64_t)k * sk + r;
    if (vec && k < K && r + FE <= R) {
#pragma unroll
      for (int q = 0; q < FE / 4; ++q) {
        const float4 a = *reinterpret_cast<const float4*>(p + 4 * q);
        f.v[4 * q] = a.x; f.v[4 * q + 1] = a.y; f.v[4 * q + 2] = a.z; f.v[4 * q + 3] = a.w;
      }
    } else {
#pragma unroll
      for (int e = 0; e < FE; ++e) f.v[e] = (k < K && r + e < R) ? p[e] : 0.0f;
    }
  } else {
    const int r = r0 + (t >> 1), k = kb + (t & 1) * FE;
    const float* p = X + (int64_t)r * sr + (int64_t)k * sk;
    if (vec && sk == 1 && r < R && k + FE <= K) {
#pragma unroll
      for (int q = 0; q < FE / 4; ++q) {
        const float4 a = *reinterpret_cast<const float4*>(p + 4 * q);
        f.v[4 * q] = a.x; f.v[4 * q + 1] = a.y; f.v[4 * q + 2] = a.z; f.v[4 * q + 3] = a.w;
      }
    } else {
#pragma unroll
      for (int e = 0; e < FE; ++e) f.v[e] = (r < R && k + e < K) ? p[(int64_t)e * sk] : 0.0f;
    }
  }
}

// Writes thread t's FE elements to the [k][row] LDS tile.
__device__ __forceinline__ void store_frag(float* L, int64_t sr, int64_t sk, int t, const Frag& f) {
  if (sr == 1 && sk != 1) {
    float* p = L + (t / TPK) * GP + (t % TPK) * FE;
#pragma unroll
    for (int e = 0; e < FE; ++e) p[e] = f.v[e];
  } else {
    float* p = L + ((t & 1) * FE) * GP + (t >> 1);
#pragma unroll
    for (int e = 0; e < FE; ++e) p[e * GP] = f.v[e];
  }
}

// The k index of element e of thread t's fragment (relative to the step).
__device__ __forceinline__ int frag_k(int64_t sr, int64_t sk, int t, int e) {
  return (sr == 1 && sk != 1) ? t / TPK : (t & 1) * FE + e;
}

template <int EPI>
__device__ __forceinline__ void epilogue(const GemmF32& g, int64_t bo, int64_t bi, float d, float carry, int m,
                                         int n, float v) {
  float* C = g.C + bo * g.sCo + bi * g.sCi;
  if (EPI == E_TRIL) v = n < m ? v : 0.0f;
  if (EPI == E_TRIL_DECAY) v = n < m ? (g.decay ? v * dpowf(d, m - n) : v) : 0.0f;
  if ((EPI == E_ROWSCALE || EPI == E_ROWSCALE_ACC) && g.decay) v *= dpowf(d, m);
  if (EPI == E_ROWREV_ACC && g.decay) v *= dpowf(d, g.kpow - m);
  const int64_t o = (int64_t)m * g.sCm + (int64_t)n * g.sCn;
  if (EPI == E_ROWSCALE_ACC || EPI == E_ROWREV_ACC) v += C[o];
  if (EPI == E_CARRY && g.src) v += g.src[bo * g.sCo + bi * g.sCi + o] * carry;
  C[o] = v;
}

template <int EPI, bool KSCALE>
__global__ __launch_bounds__(256) void gemm_f32_kernel(GemmF32 g) {
  __shared__ float As[2][GK * GP];
  __shared__ float Bs[2][GK * GP];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int wm = w >> 1, wn = w & 1;
  const int P = g.ksplit > 1 ? g.ksplit : 1;
  const int kp = (int)(blockIdx.z % P);
  const int64_t b = blockIdx.z / P, bo = b / g.H, bi = b - bo * g.H;
  const int m0 = blockIdx.y * GT, n0 = blockIdx.x * GT;
  const float d = g.decay ? g.decay[bi] : 1.0f;
  const bool tril = EPI == E_TRIL || EPI == E_TRIL_DECAY;
  if (tril && n0 >= m0 + GT) {
    // Every (m, n) of the tile has n > m: all masked (with split-K the
    // reduce writes the zeros).
    if (P > 1) return;
    float* C = g.C + bo * g.sCo + bi * g.sCi;
    for (int i = t; i < GT * GT; i += 256) {
      const int m = m0 + i / GT, n = n0 + i % GT;
      if (m < g.M && n < g.N) C[(int64_t)m * g.sCm + (int64_t)n * g.sCn] = 0.0f;
    }
    return;
  }
  const float* A = g.A + bo * g.sAo + bi * g.sAi + (int64_t)m0 * g.sAm;
  const float* B = g.B + bo * g.sBo + bi * g.sBi + (int64_t)n0 * g.sBn;
  // This workgroup's K range [k_lo, Kt): range kp of P, whole steps.
  const int Kfull = g.kcausal ? min(g.K, m0 + GT) : g.K;
  const int chunk = ((Kfull + P - 1) / P + GK - 1) / GK * GK;
  const int k_lo = min(Kfull, kp * chunk);
  const int Kt = min(Kfull, k_lo + chunk);
  const int Ma = g.M - m0, Nb = g.N - n0;

  floatx16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = zero16();

  Frag fa, fb;
  auto load = [&](int kb) {
    load_frag(A, g.sAm, g.sAk, 0, Ma, kb, Kt, g.a_vec, t, fa);
    load_frag(B, g.sBn, g.sBk, 0, Nb, kb, Kt, g.b_vec, t, fb);
    if (KSCALE && g.decay) {
      // Padding past K stays 0 (no power of a zero decay with a negative exponent).
#pragma unroll
      for (int e = 0; e < FE; ++e) {
        const int k = kb + frag_k(g.sAm, g.sAk, t, e);
        if (k < Kt) fa.v[e] *= dpowf(d, g.kpow - k);
      }
    }
  };
  auto store = [&](int buf) {
    store_frag(As[buf], g.sAm, g.sAk, t, fa);
    store_frag(Bs[buf], g.sBn, g.sBk, t, fb);
  };
  const int nks = (Kt - k_lo + GK - 1) / GK;
  if (nks > 0) {
    load(k_lo);
    store(0);
  }
  __syncthreads();
  for (int ks = 0; ks < nks; ++ks) {
    const int buf = ks & 1;
    if (ks + 1 < nks) load(k_lo + (ks + 1) * GK);
    const float* Ab = As[buf];
    const float* Bb = Bs[buf];
#pragma unroll
    for (int kk = 0; kk < GK; kk += 2) {
      const int kr = (kk + (lane >> 5)) * GP;
      const float a0 = Ab[kr + wm * 64 + (lane & 31)];
      const float a1 = Ab[kr + wm * 64 + 32 + (lane & 31)];
      const float b0 = Bb[kr + wn * 64 + (lane & 31)];
      const float b1 = Bb[kr + wn * 64 + 32 + (lane & 31)];
      acc[0][0] = mfma_f32(a0, b0, acc[0][0]);
      acc[0][1] = mfma_f32(a0, b1, acc[0][1]);
      acc[1][0] = mfma_f32(a1, b0, acc[1][0]);
      acc[1][1] = mfma_f32(a1, b1, acc[1][1]);
    }
    if (ks + 1 < nks) store(buf ^ 1);
    __syncthreads();
  }

  const float carry = (EPI == E_CARRY && g.decay) ? dpowf(d, g.kpow) : 1.0f;
  float* Pp = P > 1 ? g.part + ((int64_t)kp * g.batch + b) * (int64_t)g.M * g.N : nullptr;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + wm * 64 + i * 32 + acc_row(lane, r), n = n0 + wn * 64 + j * 32 + (lane & 31);
        if (m >= g.M || n >= g.N) continue;
        if (P > 1) Pp[(int64_t)m * g.N + n] = acc[i][j][r];
        else epilogue<EPI>(g, bo, bi, d, carry, m, n, acc[i][j][r]);
      }
}

// Split-K: sums the P partials of each (b, m, n) in range order and applies
// the epilogue (masked elements are written without reading partials, which
// the skipped tiles did not write).
template <int EPI>
__global__ __launch_bounds__(256) void gemm_reduce_kernel(GemmF32 g) {
  const int64_t MN = (int64_t)g.M * g.N, total = g.batch * MN;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  const int64_t b = i / MN, bo = b / g.H, bi = b - bo * g.H;
  const int m = (int)((i - b * MN) / g.N), n = (int)(i - b * MN - (int64_t)m * g.N);
  const float d = g.decay ? g.decay[bi] : 1.0f;
  const float carry = (EPI == E_CARRY && g.decay) ? dpowf(d, g.kpow) : 1.0f;
  float v = 0.0f;
  if (!((EPI == E_TRIL || EPI == E_TRIL_DECAY) && n >= m)) {
    for (int kp = 0; kp < g.ksplit; ++kp) v += g.part[kp * total + i];
  }
  epilogue<EPI>(g, bo, bi, d, carry, m, n, v);
}

// 16-byte loads need the operand's base, batch strides and the stride of
// the non-contiguous index to keep 4-float alignment.
inline bool vec_ok(const float* X, int64_t so, int64_t si, int64_t sr, int64_t sk) {
  if (((uintptr_t)X & 15) != 0 || so % 4 != 0 || si % 4 != 0) return false;
  if (sk == 1) return sr % 4 == 0;
  if (sr == 1) return sk % 4 == 0;
  return false;
}

// Ranges of K to split into: the fewest (a power of two, up to 16) that give
// the launch two workgroups per CU, each range keeping at least 512 of K.
// (Choosing the count from the gram's working tiles only, 3 of its 4 at the
// fp32 C2 shape, was slower: 5 ranges 523 us, 16 ranges 384 us, against 351
// us with 4: the masked tiles' workgroups, which exit at once, still take
// dispatch slots.  Aiming at four workgroups per CU, which registers and LDS
// allow, gave the gram and readout 8 ranges and no gain: 362 and 332 us; a
// grid of the gram's working tiles only, 8 ranges, 3 workgroups on every
// CU: 352 us.  Counters put the GEMMs' MFMAs 46-66 % busy whatever the
// occupancy.)
inline int split_k_ranges(int64_t tiles, int K) {
  int p = 1;
  const int64_t want = 2 * (int64_t)device_cus();
  while (p < 16 && tiles * p < want && K / (2 * p) >= 512) p *= 2;
  return p;
}

// C = epilogue(A B^T) over `batch` products.  With `part` (part_elems floats)
// a long K may be split; the partials need ksplit * batch * M * N floats.
template <int EPI, bool KSCALE = false>
hipError_t gemm(GemmF32 g, int64_t batch, hipStream_t st, float* part = nullptr, size_t part_elems = 0,
                uint64_t* launches = nullptr) {
  if (g.M <= 0 || g.N <= 0 || batch <= 0) return hipSuccess;
  g.a_vec = vec_ok(g.A, g.sAo, g.sAi, g.sAm, g.sAk);
  g.b_vec = vec_ok(g.B, g.sBo, g.sBi, g.sBn, g.sBk);
  g.batch = batch;
  const int64_t tiles = ((g.N + GT - 1) / GT) * ((g.M + GT - 1) / GT) * batch;
  int p = part ? split_k_ranges(tiles, g.K) : 1;
  while (p > 1 && (size_t)p * (size_t)batch * (size_t)g.M * (size_t)g.N > part_elems) p /= 2;
  g.ksplit = p;
  g.part = p > 1 ? part : nullptr;
  const dim3 grid((unsigned)((g.N + GT - 1) / GT), (unsigned)((g.M + GT - 1) / GT), (unsigned)(batch * p));
  hipLaunchKernelGGL((gemm_f32_kernel<EPI, KSCALE>), grid, dim3(256), 0, st, g);
  if (p > 1) {
    const int64_t total = batch * (int64_t)g.M * g.N;
    hipLaunchKernelGGL(gemm_reduce_kernel<EPI>, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, g);
  }
  if (launches) *launches += p > 1 ? 2 : 1;
  return hipGetLastError();
}

// Partial floats the split-K of a [batch, M, N] product at depth K may use.
inline size_t split_k_elems(int64_t batch, int M, int N, int K) {
  const int64_t tiles = ((N + GT - 1) / GT) * (int64_t)((M + GT - 1) / GT) * batch;
  const int p = split_k_ranges(tiles, K);
  return p > 1 ? (size_t)p * (size_t)batch * (size_t)M * (size_t)N : 0;
}

}  // namespace gf32
}  // namespace bdh
