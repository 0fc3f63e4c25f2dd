// Batched fp32 GEMM on gfx950 matrix cores (v_mfma_f32_16x16x4f32 and
// v_mfma_f32_32x32x2f32: exact fp32 products, fp32 accumulation) with the
// epilogues of the recurrence's closed form.  Used by the fp32 forward
// (prefill_f32.hip) and the backward (vjp.hip).  Two kernels: the
// direct-load kernel further down for operands contiguous along k or along
// their rows (the common case), and this register-staged one for the rest.
//
//   C(m, n) = sum_k A(m, k) B(n, k),  batch b = (b / H, b % H):
//   X(i, j) = X + (b / H) * sXo + (b % H) * sXi + i * sXr + j * sXc
//
// Register-staged kernel: workgroups of 256 threads own 128 x 128 output
// tiles, each wave a 64 x 64 block (2 x 2 MFMA blocks of
// v_mfma_f32_32x32x2f32, 64 accumulators a lane).  K steps are 16 deep:
// the operands of step k + 1 are loaded into registers (16-byte loads where
// the operand is contiguous along k or along its rows) while step k is
// multiplied from LDS; LDS holds two steps, so one barrier a step suffices.
// A long K with few tiles is split into P ranges (split-K): each range's
// workgroup writes its raw sums to a partial buffer, and a reduce kernel
// adds the P partials in range order (deterministic) and applies the
// epilogue.
#pragma once

#include <type_traits>

#include "bdh_internal.h"
#include "bdh_mfma.h"

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
  int tri;              // direct-load grid of the tiles on or below the diagonal only (M == N, split-K)
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

// The epilogue's addend: C itself (the accumulating kinds), src (E_CARRY),
// or none.
template <int EPI>
__device__ __forceinline__ const float* epi_addend(const GemmF32& g, int64_t bo, int64_t bi) {
  if (EPI == E_ROWSCALE_ACC || EPI == E_ROWREV_ACC) return g.C + bo * g.sCo + bi * g.sCi;
  if (EPI == E_CARRY && g.src) return g.src + bo * g.sCo + bi * g.sCi;
  return nullptr;
}

// Output value of (m, n) from the sum v and the addend x (when the kind has one).
template <int EPI>
__device__ __forceinline__ float epi_value(const GemmF32& g, float d, float carry, int m, int n, float v, float x) {
  if (EPI == E_TRIL) v = n < m ? v : 0.0f;
  if (EPI == E_TRIL_DECAY) v = n < m ? (g.decay ? v * dpowf(d, m - n) : v) : 0.0f;
  if ((EPI == E_ROWSCALE || EPI == E_ROWSCALE_ACC) && g.decay) v *= dpowf(d, m);
  if (EPI == E_ROWREV_ACC && g.decay) v *= dpowf(d, g.kpow - m);
  if (EPI == E_ROWSCALE_ACC || EPI == E_ROWREV_ACC) v += x;
  if (EPI == E_CARRY && g.src) v += x * carry;
  return v;
}

template <int EPI>
__device__ __forceinline__ void epilogue(const GemmF32& g, int64_t bo, int64_t bi, float d, float carry, int m,
                                         int n, float v) {
  float* C = g.C + bo * g.sCo + bi * g.sCi;
  const float* X = epi_addend<EPI>(g, bo, bi);
  const int64_t o = (int64_t)m * g.sCm + (int64_t)n * g.sCn;
  C[o] = epi_value<EPI>(g, d, carry, m, n, v, X ? X[o] : 0.0f);
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

// --- Direct-load kernel: the shapes the fp32 forward and backward run ----
// The product and epilogues of gemm_f32_kernel, with the operand tiles
// fetched by direct global -> LDS loads (global_load_lds_dwordx4) into a
// ring of DST stages, DST - 1 of them in flight while one is multiplied:
// the register-staged kernel above has one step in flight, and its MFMAs
// sat 46-66 % busy.  Each operand is either
//   KC, contiguous along k (sk == 1): tile [128 rows][16 k] of 64-byte
//       rows, 16-byte chunk c of row r stored at chunk c ^ ((r >> 1) & 3);
//   RC, contiguous along its rows (sr == 1): tile [16 k][128 rows] of
//       512-byte rows, chunk c of k row k stored at chunk c ^ 4 ((k >> 2) & 3).
// The swizzles keep the fragment reads free of bank conflicts; a DMA writes
// lane l's 16 bytes to LDS at M0 + 16 l, so it applies them by the choice of
// the global chunk each lane fetches.  Rows past the operand's end re-read
// its last row (KC) or chunk (RC): their sums are never written.
// MFMA: v_mfma_f32_16x16x4f32, lane l = 16 g + i holding row (column) i of a
// 16 x 16 block in k slot g.  The 4 MFMAs j = 0..3 of a 16-deep step give
// slot g the k index 4 g + j for both operands, so a KC operand reads its 4
// values in one 16-byte read and an RC operand in two 2-dword reads (k rows
// 4 g + j, 512 bytes apart).  A wave owns a 64 x 64 block: 4 x 4 MFMA
// blocks, 64 MFMAs a step.
// Workgroup ids are remapped so that each XCD (id % 8) takes a contiguous
// range of tiles: the tiles of one batch and K range, which share operand
// rows, then run on one L2.
// (Reading a step's fragments while the step before is multiplied, with the
// DMAs spread between its MFMA groups behind sched_barrier fences, was
// slower: the fp32 C2 gram 225 against 215 us, with 212 VGPRs against 136.)
constexpr int DST = 4;               // ring stages
constexpr int DTILE = GT * GK * 4;   // bytes of one operand tile (8 KiB)
constexpr int DSTAGE = 2 * DTILE;    // A tile, then B tile
constexpr int DSCALE = 1024;         // KSCALE: most k of one workgroup (LDS table of d^(kpow - k))

typedef float floatx2 __attribute__((ext_vector_type(2)));

// Byte offset from a tile's global base of what lane `lane` of DMA
// instruction i (8 per tile) fetches; R = rows of the tile inside the operand.
__device__ __forceinline__ uint32_t dma_src(bool kc, int64_t sr, int64_t sk, int R, int i, int lane) {
  if (kc) {
    const int r = 16 * i + (lane >> 2);
    const int c = (lane & 3) ^ ((r >> 1) & 3);
    return (uint32_t)((int64_t)min(r, R - 1) * sr * 4 + c * 16);
  }
  const int k = 2 * i + (lane >> 5);
  const int c = min((lane & 31) ^ (4 * ((k >> 2) & 3)), R / 4 - 1);
  return (uint32_t)((int64_t)k * sk * 4 + c * 16);
}

// KC fragments: v[mi] = k slots 4 g .. 4 g + 3 of row 16 mi + i of the wave's
// block (a = the lane's address of mi = 0).
__device__ __forceinline__ void dread_kc(uint32_t a, floatx4 (&v)[4]) {
  asm volatile("ds_read_b128 %0, %1 offset:0" : "=v"(v[0]) : "v"(a));
  asm volatile("ds_read_b128 %0, %1 offset:1024" : "=v"(v[1]) : "v"(a));
  asm volatile("ds_read_b128 %0, %1 offset:2048" : "=v"(v[2]) : "v"(a));
  asm volatile("ds_read_b128 %0, %1 offset:3072" : "=v"(v[3]) : "v"(a));
}
// RC fragments: v[mi][h] = k rows 4 g + 2 h and 4 g + 2 h + 1 of column
// 16 mi + i (a[mi] = the lane's address of k row 4 g).
__device__ __forceinline__ void dread_rc(const uint32_t (&a)[4], floatx2 (&v)[4][2]) {
#pragma unroll
  for (int mi = 0; mi < 4; ++mi) {
    asm volatile("ds_read2st64_b32 %0, %1 offset0:0 offset1:2" : "=v"(v[mi][0]) : "v"(a[mi]));
    asm volatile("ds_read2st64_b32 %0, %1 offset0:4 offset1:6" : "=v"(v[mi][1]) : "v"(a[mi]));
  }
}
__device__ __forceinline__ void dtie(floatx4 (&v)[4]) {
  asm volatile("" : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]));
}
__device__ __forceinline__ void dtie(floatx2 (&v)[4][2]) {
  asm volatile("" : "+v"(v[0][0]), "+v"(v[0][1]), "+v"(v[1][0]), "+v"(v[1][1]), "+v"(v[2][0]), "+v"(v[2][1]),
               "+v"(v[3][0]), "+v"(v[3][1]));
}
__device__ __forceinline__ float dval(const floatx4 (&v)[4], int mi, int j) { return v[mi][j]; }
__device__ __forceinline__ float dval(const floatx2 (&v)[4][2], int mi, int j) { return v[mi][j >> 1][j & 1]; }

template <bool KC>
using DFrag = typename std::conditional<KC, floatx4[4], floatx2[4][2]>::type;

template <int EPI, bool KSCALE, bool AKC, bool BKC>
__global__ __launch_bounds__(256, 2) void gemm_f32_dma_kernel(GemmF32 g, int ntx, int nty) {
  __shared__ __attribute__((aligned(16))) char lds[DST * DSTAGE + (KSCALE ? 4 * DSCALE : 0)];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int wm = w >> 1, wn = w & 1, gq = lane >> 4, li = lane & 15;
  // XCD-contiguous work order (the launch has a multiple of 8 workgroups).
  const int nwg = (int)gridDim.x, id = (int)blockIdx.x;
  int wk = (nwg & 7) ? id : (id & 7) * (nwg >> 3) + (id >> 3);
  int tx, ty;
  int64_t z;
  if (g.tri) {
    // Tiles (ty, tx <= ty) in row order, nty (nty + 1) / 2 of them a batch.
    const int per = nty * (nty + 1) / 2;
    z = wk / per;
    int r = wk - (int)z * per;
    ty = 0;
    while (r > ty) {
      r -= ty + 1;
      ++ty;
    }
    tx = r;
  } else {
    tx = wk % ntx;
    wk /= ntx;
    ty = wk % nty;
    z = wk / nty;
  }
  const int P = g.ksplit > 1 ? g.ksplit : 1;
  const int kp = (int)(z % P);
  const int64_t b = z / P, bo = b / g.H, bi = b - bo * g.H;
  const int m0 = ty * GT, n0 = tx * GT;
  const float d = g.decay ? g.decay[bi] : 1.0f;
  const bool tril = EPI == E_TRIL || EPI == E_TRIL_DECAY;
  if (tril && n0 >= m0 + GT) {
    if (P > 1) return;
    float* C = g.C + bo * g.sCo + bi * g.sCi;
    for (int i = t; i < GT * GT; i += 256) {
      const int m = m0 + i / GT, n = n0 + i % GT;
      if (m < g.M && n < g.N) C[(int64_t)m * g.sCm + (int64_t)n * g.sCn] = 0.0f;
    }
    return;
  }
  const int Kfull = g.kcausal ? min(g.K, m0 + GT) : g.K;
  const int chunk = ((Kfull + P - 1) / P + GK - 1) / GK * GK;
  const int k_lo = min(Kfull, kp * chunk);
  const int Kt = min(Kfull, k_lo + chunk);
  const int nks = (Kt - k_lo) / GK;  // the host sends K % GK == 0 here
  const int Ma = min(GT, g.M - m0), Nb = min(GT, g.N - n0);
  const char* Ag = reinterpret_cast<const char*>(g.A + bo * g.sAo + bi * g.sAi + (int64_t)m0 * g.sAm +
                                                 (int64_t)k_lo * g.sAk);
  const char* Bg = reinterpret_cast<const char*>(g.B + bo * g.sBo + bi * g.sBi + (int64_t)n0 * g.sBn +
                                                 (int64_t)k_lo * g.sBk);
  const int64_t a_step = (int64_t)GK * g.sAk * 4, b_step = (int64_t)GK * g.sBk * 4;
  uint32_t va[2], vb[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    va[j] = dma_src(AKC, g.sAm, g.sAk, Ma, w + 4 * j, lane);
    vb[j] = dma_src(BKC, g.sBn, g.sBk, Nb, w + 4 * j, lane);
  }
  const uint32_t l0 = mfma::lds_addr(lds);
  auto issue = [&](int s) {
    const uint32_t st = l0 + (uint32_t)((s % DST) * DSTAGE);
#pragma unroll
    for (int j = 0; j < 2; ++j) mfma::dma16(Ag + s * a_step, va[j], st + (uint32_t)((w + 4 * j) * 1024));
#pragma unroll
    for (int j = 0; j < 2; ++j) mfma::dma16(Bg + s * b_step, vb[j], st + (uint32_t)(DTILE + (w + 4 * j) * 1024));
  };

  const bool ksc = KSCALE && g.decay != nullptr;
  float* sct = reinterpret_cast<float*>(lds + DST * DSTAGE);
  if (ksc) {
    for (int k = t; k < Kt - k_lo; k += 256) sct[k] = dpowf(d, g.kpow - (k_lo + k));
    __syncthreads();
  }

  // Lane addresses of the fragments, relative to a stage.
  const uint32_t a_kc = (uint32_t)((wm * 64 + li) * 64 + ((gq ^ ((li >> 1) & 3)) << 4));
  const uint32_t b_kc = (uint32_t)(DTILE + (wn * 64 + li) * 64 + ((gq ^ ((li >> 1) & 3)) << 4));
  uint32_t a_rc[4], b_rc[4];
#pragma unroll
  for (int mi = 0; mi < 4; ++mi) {
    a_rc[mi] = (uint32_t)(2048 * gq + 256 * wm + 64 * (mi ^ gq) + 4 * li);
    b_rc[mi] = (uint32_t)(DTILE + 2048 * gq + 256 * wn + 64 * (mi ^ gq) + 4 * li);
  }

  floatx4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = zero4();

  // A whole tile's epilogue addends are loaded during the last K steps (the
  // rows of block rows 0-1 in step nks - 3, of 2-3 in step nks - 2, once no
  // DMA is left to issue), so that their latency hides behind those steps.
  constexpr bool ADDEND = EPI == E_ROWSCALE_ACC || EPI == E_ROWREV_ACC || EPI == E_CARRY;
  const bool whole = P == 1 && m0 + GT <= g.M && n0 + GT <= g.N;
  const float* X = epi_addend<EPI>(g, bo, bi);
  float xv[ADDEND ? 4 : 1][4][4];
  auto load_addends = [&](int mi0) {
#pragma unroll
    for (int mi = mi0; mi < mi0 + 2; ++mi)
#pragma unroll
      for (int ni = 0; ni < 4; ++ni)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = m0 + wm * 64 + 16 * mi + 4 * gq + r, n = n0 + wn * 64 + 16 * ni + li;
          xv[ADDEND ? mi : 0][ni][r] = X[(int64_t)m * g.sCm + (int64_t)n * g.sCn];
        }
  };
  const bool early = ADDEND && whole && X != nullptr && nks >= DST - 1;

  // Reads and MFMAs of stage s (after the wait that it has landed).
  auto step = [&](int s) {
    const uint32_t st = l0 + (uint32_t)((s % DST) * DSTAGE);
    DFrag<AKC> fa;
    DFrag<BKC> fb;
    if constexpr (AKC) {
      dread_kc(st + a_kc, fa);
    } else {
      const uint32_t ad[4] = {st + a_rc[0], st + a_rc[1], st + a_rc[2], st + a_rc[3]};
      dread_rc(ad, fa);
    }
    if constexpr (BKC) {
      dread_kc(st + b_kc, fb);
    } else {
      const uint32_t bd[4] = {st + b_rc[0], st + b_rc[1], st + b_rc[2], st + b_rc[3]};
      dread_rc(bd, fb);
    }
    floatx4 sc = floatx4{1.0f, 1.0f, 1.0f, 1.0f};
    if (KSCALE && ksc) {
      const uint32_t sa = mfma::lds_addr(sct) + (uint32_t)(64 * s + 16 * gq);
      asm volatile("ds_read_b128 %0, %1" : "=v"(sc) : "v"(sa));
    }
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(sc));
    dtie(fa);
    dtie(fb);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float av[4], bv[4];
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) {
        av[mi] = dval(fa, mi, j);
        if (KSCALE) av[mi] *= sc[j];
        bv[mi] = dval(fb, mi, j);
      }
#pragma unroll
      for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int ni = 0; ni < 4; ++ni)
          acc[mi][ni] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[mi], bv[ni], acc[mi][ni], 0, 0, 0);
    }
  };

  // Stage s has landed once at most the vector memory operations issued
  // after it are in flight: the DMAs of later stages (4 a stage) and, in the
  // last two steps of the early-addend tail, the addend loads (32 a step; 63
  // is the counter's most, one load short).
  for (int s = 0; s < DST - 1 && s < nks; ++s) issue(s);
  int s = 0;
  for (; s + DST - 1 < nks; ++s) {
    mfma::dma_wait_barrier<4 * (DST - 2)>();
    // Into the slot of stage s - 1, which every wave finished reading before the barrier.
    issue(s + DST - 1);
    step(s);
  }
  static_assert(DST == 4, "the tails below wait for 2, 1, 0 later stages");
  if (early) {
    // nks >= 3: the last three stages, none left to issue.
    mfma::dma_wait_barrier<8>();
    load_addends(0);
    step(s);
    mfma::dma_wait_barrier<36>();
    load_addends(2);
    step(s + 1);
    mfma::dma_wait_barrier<63>();
    step(s + 2);
  } else {
    for (; s < nks; ++s) {
      const int later = nks - 1 - s;
      if (later >= 2) mfma::dma_wait_barrier<8>();
      else if (later == 1) mfma::dma_wait_barrier<4>();
      else mfma::dma_wait_barrier<0>();
      step(s);
    }
  }

  const float carry = (EPI == E_CARRY && g.decay) ? dpowf(d, g.kpow) : 1.0f;
  float* Pp = P > 1 ? g.part + ((int64_t)kp * g.batch + b) * (int64_t)g.M * g.N : nullptr;
  // Block (mi, ni), register r: row 16 mi + 4 g + r, column 16 ni + i.
  if (whole) {
    float* C = g.C + bo * g.sCo + bi * g.sCi;
    if (ADDEND && X != nullptr && !early) {
      load_addends(0);
      load_addends(2);
    }
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
      for (int ni = 0; ni < 4; ++ni)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = m0 + wm * 64 + 16 * mi + 4 * gq + r, n = n0 + wn * 64 + 16 * ni + li;
          const float x = (ADDEND && X) ? xv[ADDEND ? mi : 0][ni][r] : 0.0f;
          C[(int64_t)m * g.sCm + (int64_t)n * g.sCn] = epi_value<EPI>(g, d, carry, m, n, acc[mi][ni][r], x);
        }
    return;
  }
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
#pragma unroll
    for (int ni = 0; ni < 4; ++ni)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + wm * 64 + 16 * mi + 4 * gq + r, n = n0 + wn * 64 + 16 * ni + li;
        if (m >= g.M || n >= g.N) continue;
        if (P > 1) Pp[(int64_t)m * g.N + n] = acc[mi][ni][r];
        else epilogue<EPI>(g, bo, bi, d, carry, m, n, acc[mi][ni][r]);
      }
}

// 16-byte loads need the operand's base, batch strides and the stride of
// the non-contiguous index to keep 4-float alignment.
inline bool vec_ok(const float* X, int64_t so, int64_t si, int64_t sr, int64_t sk) {
  if (((uintptr_t)X & 15) != 0 || so % 4 != 0 || si % 4 != 0) return false;
  if (sk == 1) return sr % 4 == 0;
  if (sr == 1) return sk % 4 == 0;
  return false;
}

// Layout of an operand for the direct-load kernel: 1 = contiguous along k
// (KC), 0 = contiguous along its rows (RC, R rows a multiple of 4), -1 = not
// served (no 16-byte alignment, neither index contiguous, or a tile's DMA
// offsets past 32 bits).
inline int dma_layout(const float* X, int64_t so, int64_t si, int64_t sr, int64_t sk, int R) {
  if (!vec_ok(X, so, si, sr, sk)) return -1;
  if (sk == 1 && (int64_t)(GT - 1) * sr * 4 + 64 <= (int64_t)UINT32_MAX) return 1;
  if (sr == 1 && R % 4 == 0 && (int64_t)(GK - 1) * sk * 4 + 512 <= (int64_t)UINT32_MAX) return 0;
  return -1;
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

// Ranges for the direct-load kernel: as many as fit its workgroups of the
// working tiles into the CUs' two slots (up to 16), each at least 128 deep;
// a short K (< 1024) only when the tiles fill under a quarter of the CUs.
// (At the fp32 C2 shape: the gram's 96 working tiles 5 ranges, 480
// workgroups; the readout 4; S V, K = 256 on 128 tiles, none: 2 ranges took
// 19.9 us and their reduce 10.6 us, against 22.7 us unsplit.)
inline int split_k_ranges_dma(int64_t work_tiles, int K) {
  if (K < 1024 && work_tiles * 4 >= (int64_t)device_cus()) return 1;
  int64_t p = 2 * (int64_t)device_cus() / (work_tiles > 0 ? work_tiles : 1);
  p = p < 16 ? p : 16;
  p = p < K / 128 ? p : K / 128;
  return p > 1 ? (int)p : 1;
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
  const int ntx = (g.N + GT - 1) / GT, nty = (g.M + GT - 1) / GT;
  const int akc = dma_layout(g.A, g.sAo, g.sAi, g.sAm, g.sAk, g.M), bkc = dma_layout(g.B, g.sBo, g.sBi, g.sBn, g.sBk, g.N);
  const bool dma = akc >= 0 && bkc >= 0 && g.K % GK == 0 && (!KSCALE || g.K <= DSCALE);
  const bool tril = EPI == E_TRIL || EPI == E_TRIL_DECAY;
  const int64_t tri_tiles = (int64_t)nty * (nty + 1) / 2 * batch;
  const size_t per = (size_t)batch * (size_t)g.M * (size_t)g.N;
  int p = 1;
  if (part && dma) {
    p = split_k_ranges_dma(tril && g.M == g.N && !g.kcausal ? tri_tiles : tiles, g.K);
    if ((size_t)p * per > part_elems) p = (int)(part_elems / per);
  } else if (part) {
    p = split_k_ranges(tiles, g.K);
    while (p > 1 && (size_t)p * per > part_elems) p /= 2;
  }
  if (p < 1) p = 1;
  g.ksplit = p;
  g.part = p > 1 ? part : nullptr;
  // Masked tiles are left out of the grid only with split-K, whose reduce
  // writes their zeros.
  g.tri = dma && tril && g.M == g.N && !g.kcausal && p > 1;
  if (dma) {
    const int64_t nwg = (g.tri ? tri_tiles : tiles) * p;
    if (nwg > INT32_MAX) return hipErrorInvalidValue;
    const dim3 grid((unsigned)nwg);
    if (akc && bkc)
      hipLaunchKernelGGL((gemm_f32_dma_kernel<EPI, KSCALE, true, true>), grid, dim3(256), 0, st, g, ntx, nty);
    else if (akc)
      hipLaunchKernelGGL((gemm_f32_dma_kernel<EPI, KSCALE, true, false>), grid, dim3(256), 0, st, g, ntx, nty);
    else if (bkc)
      hipLaunchKernelGGL((gemm_f32_dma_kernel<EPI, KSCALE, false, true>), grid, dim3(256), 0, st, g, ntx, nty);
    else
      hipLaunchKernelGGL((gemm_f32_dma_kernel<EPI, KSCALE, false, false>), grid, dim3(256), 0, st, g, ntx, nty);
  } else {
    const dim3 grid((unsigned)ntx, (unsigned)nty, (unsigned)(batch * p));
    hipLaunchKernelGGL((gemm_f32_kernel<EPI, KSCALE>), grid, dim3(256), 0, st, g);
  }
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
  const int64_t nty = (M + GT - 1) / GT;
  int p = split_k_ranges(tiles, K);
  // Either kernel's count; the direct-load one's is largest with the
  // triangular grid of a square masked product.
  const int pd = split_k_ranges_dma(M == N ? nty * (nty + 1) / 2 * batch : tiles, K);
  p = p > pd ? p : pd;
  return p > 1 ? (size_t)p * (size_t)batch * (size_t)M * (size_t)N : 0;
}

}  // namespace gf32
}  // namespace bdh
