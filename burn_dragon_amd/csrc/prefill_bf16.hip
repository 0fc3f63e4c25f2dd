// bf16 MFMA chunked prefill on gfx950 (fp32 accumulate, fp32 rho / context).
//
// The sequence is split into state-carry intervals of L tokens (L a multiple
// of the 128-token chunk).  Inside an interval the carried state of chunk c,
// rho_c = rho_in + sum_{c'<c} Q_c'^T V_c', is applied through the chunk-pair
// score blocks Q_c Q_c'^T, so rho is materialised once per interval instead
// of once per chunk:
//   gram   S = tril(-1)(Q Q^T * d^(r-c)) for every interval (one launch; it
//          does not depend on rho), 256x256 MFMA tiles, split along N into
//          KS fixed partial buffers that ctx sums in a fixed order
//   ctx    O = tril(S) V + (Q * d^r) rho_in              64x256 MFMA tiles
//   state  rho_out = rho_in * d^L + (Q * d^(L-r))^T V    256x256 MFMA tiles
// RoPE is applied to Q tiles between HBM and LDS: each (even, odd) bf16 pair
// is rotated with two v_dot2_f32_bf16 against a packed bf16 (cos, sin) table
// entry of its (token, pair), then repacked to bf16.  Rotated queries are
// never written to memory.  All products are v_mfma_f32_32x32x16_bf16.
#include "bdh_internal.h"

namespace bdh {
namespace {

constexpr int GT = 256;        // gram / state tile edge
constexpr int BK = 64;         // k step
constexpr int LDP = BK + 8;    // padded LDS pitch (bf16) of K-contiguous tiles
constexpr int NT = 256;        // threads of the 256-tile kernels (4 waves, 128x128 each)

__device__ __forceinline__ uint4 ldg16(const void* p) {
  return *reinterpret_cast<const uint4*>(p);
}

// (even, odd) bf16 pair rotated by the packed bf16 (cos, sin) word csw:
//   re = e*c - o*s = dot2((e,o), (c,-s)) ; ro = e*s + o*c = dot2((e,o), (s,c))
__device__ __forceinline__ void rot_pair(uint32_t xw, uint32_t csw, float& re, float& ro) {
  const bf16x2 xv = __builtin_bit_cast(bf16x2, xw);
  const bf16x2 cms = __builtin_bit_cast(bf16x2, csw ^ 0x80000000u);
  const bf16x2 sc = __builtin_bit_cast(bf16x2, __builtin_amdgcn_alignbit(csw, csw, 16));
  re = __builtin_amdgcn_fdot2_f32_bf16(xv, cms, 0.0f, false);
  ro = __builtin_amdgcn_fdot2_f32_bf16(xv, sc, 0.0f, false);
}

// 8 bf16 (4 pairs) rotated (ROPE) and/or scaled by w, as f32.
template <bool ROPE>
__device__ __forceinline__ void prep8_f32(uint4 raw, uint4 cs, float w, bool scale,
                                          float (&out)[8]) {
  const uint32_t in[4] = {raw.x, raw.y, raw.z, raw.w};
  const uint32_t c[4] = {cs.x, cs.y, cs.z, cs.w};
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    float re, ro;
    if (ROPE) {
      rot_pair(in[p], c[p], re, ro);
    } else {
      re = bf16_lo(in[p]);
      ro = bf16_hi(in[p]);
    }
    if (scale) {
      re *= w;
      ro *= w;
    }
    out[2 * p] = re;
    out[2 * p + 1] = ro;
  }
}

// Same, repacked to 8 bf16 (RNE).  Without RoPE and scaling it is a copy.
template <bool ROPE>
__device__ __forceinline__ uint4 prep8(uint4 raw, uint4 cs, float w, bool scale) {
  if (!ROPE && !scale) return raw;
  float v[8];
  prep8_f32<ROPE>(raw, cs, w, scale, v);
  return make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                    pack_bf16x2(v[6], v[7]));
}

// XOR swizzle of the 8-element groups of a 64-wide transposed tile row n:
// 16-byte fragment reads of rows n..n+7 hit distinct bank groups.
__device__ __forceinline__ int swz(int n, int g) { return g ^ (n & 7) ^ ((n >> 3) & 7); }

__device__ __forceinline__ float decay_pow(const float* decay, int64_t h, float e) {
  return decay ? powf(decay[h], e) : 1.0f;
}

// ---------------------------------------------------------------------------
// gram: partial[kp, s, iv] = lower-triangular Q Q^T over the kp-th N range.
struct GramArgs {
  const bf16_t* x;
  const uint32_t* cs;   // packed bf16 (cos, sin) [T, N/2] or null
  float* part;          // [KS, S, n_iv, Lp, Lp]
  const float* decay;
  int64_t H, T, N, L, Lp, S, n_iv;
  int ks, tiles_per_iv, nb;
};

template <bool ROPE>
__global__ __launch_bounds__(NT) void gram_kernel(GramArgs a) {
  const int iv = blockIdx.x / a.tiles_per_iv;
  const int tile = blockIdx.x - iv * a.tiles_per_iv;
  const int kp = blockIdx.y;
  const int64_t s = blockIdx.z;
  int bi = 0;
  while ((bi + 1) * (bi + 2) / 2 <= tile) ++bi;
  const int bj = tile - bi * (bi + 1) / 2;
  const bool diag = bi == bj;
  const int64_t t0 = (int64_t)iv * a.L;
  const int64_t Lc = (a.T - t0 < a.L) ? a.T - t0 : a.L;
  const int64_t ri = (int64_t)bi * GT, rj = (int64_t)bj * GT;
  if (ri >= Lc) return;  // tile beyond the ragged last interval: never read

  __shared__ __attribute__((aligned(16))) bf16_t As[2][GT * LDP];
  __shared__ __attribute__((aligned(16))) bf16_t Bs[2][GT * LDP];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;  // 128-row half, 128-col half
  const int64_t half = a.N / 2;
  const bf16_t* X = a.x + (s * a.T + t0) * a.N;
  const uint32_t* CS = ROPE ? a.cs + t0 * half : nullptr;

  // Per-wave 32x32 sub-tiles that are entirely masked (above the diagonal or
  // beyond the interval) skip their MFMAs.
  bool on[4][4];
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) {
      const int64_t r_lo = ri + wm * 128 + mi * 32, c_lo = rj + wn * 128 + ni * 32;
      on[mi][ni] = r_lo < Lc && c_lo < Lc && c_lo < r_lo + 32;
    }

  uint4 ra[8], rb[8], ca[8], cb[8];
  const int kv = tid & 7;
  auto load = [&](int kt) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int row = (tid + i * NT) >> 3;
      const int64_t k = (int64_t)kt * BK + kv * 8;
      const int64_t ti = ri + row;
      const bool vi = ti < Lc;
      ra[i] = vi ? ldg16(X + ti * a.N + k) : make_uint4(0, 0, 0, 0);
      if (ROPE) ca[i] = vi ? ldg16(CS + ti * half + k / 2) : make_uint4(0, 0, 0, 0);
      if (!diag) {
        const int64_t tj = rj + row;
        const bool vj = tj < Lc;
        rb[i] = vj ? ldg16(X + tj * a.N + k) : make_uint4(0, 0, 0, 0);
        if (ROPE) cb[i] = vj ? ldg16(CS + tj * half + k / 2) : make_uint4(0, 0, 0, 0);
      }
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int row = (tid + i * NT) >> 3;
      *reinterpret_cast<uint4*>(&As[buf][row * LDP + kv * 8]) = prep8<ROPE>(ra[i], ca[i], 1.0f, false);
      if (!diag)
        *reinterpret_cast<uint4*>(&Bs[buf][row * LDP + kv * 8]) = prep8<ROPE>(rb[i], cb[i], 1.0f, false);
    }
  };

  floatx16 acc[4][4];
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = zero16();

  const int nk = (int)(a.N / BK);
  const int kb = (int)((int64_t)nk * kp / a.ks), ke = (int)((int64_t)nk * (kp + 1) / a.ks);
  if (kb < ke) {
    load(kb);
    store(0);
    __syncthreads();
    for (int kt = kb; kt < ke; ++kt) {
      const int buf = (kt - kb) & 1;
      if (kt + 1 < ke) load(kt + 1);
      const bf16_t* Ab = As[buf];
      const bf16_t* Bb = diag ? As[buf] : Bs[buf];
#pragma unroll
      for (int kk = 0; kk < BK / 16; ++kk) {
        const int ko = kk * 16 + 8 * (lane >> 5);
        bf16x8 af[4], bfr[4];
#pragma unroll
        for (int mi = 0; mi < 4; ++mi)
          af[mi] = *reinterpret_cast<const bf16x8*>(&Ab[(wm * 128 + mi * 32 + (lane & 31)) * LDP + ko]);
#pragma unroll
        for (int ni = 0; ni < 4; ++ni)
          bfr[ni] = *reinterpret_cast<const bf16x8*>(&Bb[(wn * 128 + ni * 32 + (lane & 31)) * LDP + ko]);
#pragma unroll
        for (int mi = 0; mi < 4; ++mi)
#pragma unroll
          for (int ni = 0; ni < 4; ++ni)
            if (on[mi][ni]) acc[mi][ni] = mfma32(af[mi], bfr[ni], acc[mi][ni]);
      }
      if (kt + 1 < ke) store(buf ^ 1);
      __syncthreads();
    }
  }

  const int64_t h = s % a.H;
  float* P = a.part + (((int64_t)kp * a.S + s) * a.n_iv + iv) * a.Lp * a.Lp;
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
#pragma unroll
    for (int ni = 0; ni < 4; ++ni)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t ti = ri + wm * 128 + mi * 32 + acc_row(lane, r);
        const int64_t tj = rj + wn * 128 + ni * 32 + acc_col(lane);
        if (ti < Lc && tj < Lc) {
          const float v = tj < ti ? acc[mi][ni][r] * decay_pow(a.decay, h, (float)(ti - tj)) : 0.0f;
          P[ti * a.Lp + tj] = v;
        }
      }
}

// ---------------------------------------------------------------------------
// state: rho_out[n0:n0+256, d0:d0+256] = rho_in * d^L + (Q * d^(L-r))^T V
struct StateArgs {
  const bf16_t* x;
  const uint32_t* cs;
  const bf16_t* vt;   // [B*Hv, D, Tp]
  const float* rho_in;
  float* rho_out;
  const float* decay;
  int64_t H, Hv, T, N, D, t0, L, Tp;
};

template <bool ROPE>
__global__ __launch_bounds__(NT) void state_kernel(StateArgs a) {
  const int64_t n0 = (int64_t)blockIdx.x * GT;
  const int64_t d0 = (int64_t)blockIdx.y * GT;
  const int64_t s = blockIdx.z;
  __shared__ __attribute__((aligned(16))) bf16_t As[2][GT * BK];    // [n][t], swizzled
  __shared__ __attribute__((aligned(16))) bf16_t Bs[2][GT * LDP];   // [d][t]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;  // 128 rows of n, 128 cols of d
  const int64_t half = a.N / 2;
  const int64_t b = s / a.H, h = s - b * a.H;
  const bf16_t* X = a.x + (s * a.T + a.t0) * a.N;
  const uint32_t* CS = ROPE ? a.cs + a.t0 * half : nullptr;
  const bf16_t* VT = a.vt + (b * a.Hv + (a.Hv == 1 ? 0 : h)) * a.D * a.Tp;
  const float dv = a.decay ? a.decay[h] : 1.0f;
  const bool scale = a.decay != nullptr;

  bool on[4];
#pragma unroll
  for (int ni = 0; ni < 4; ++ni) on[ni] = d0 + wn * 128 + ni * 32 < a.D;

  uint4 ra[8], ca[8], rbv[8];
  float wa[8];
  auto load = [&](int kt) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int v = tid + i * NT;
      const int tt = v >> 5, nv = v & 31;
      const int64_t tl = (int64_t)kt * BK + tt;
      const bool ok = tl < a.L;
      const int64_t n = n0 + nv * 8;
      ra[i] = ok ? ldg16(X + tl * a.N + n) : make_uint4(0, 0, 0, 0);
      if (ROPE) ca[i] = ok ? ldg16(CS + tl * half + n / 2) : make_uint4(0, 0, 0, 0);
      wa[i] = scale ? powf(dv, (float)(a.L - tl)) : 1.0f;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int v = tid + i * NT;
      const int dd = v >> 3, kv = v & 7;
      const int64_t d = d0 + dd;
      rbv[i] = d < a.D ? ldg16(VT + d * a.Tp + a.t0 + (int64_t)kt * BK + kv * 8)
                       : make_uint4(0, 0, 0, 0);
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int v = tid + i * NT;
      const int tt = v >> 5, nv = v & 31;
      float vals[8];
      prep8_f32<ROPE>(ra[i], ca[i], wa[i], scale, vals);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int n = nv * 8 + e;
        As[buf][n * BK + swz(n, tt >> 3) * 8 + (tt & 7)] = (bf16_t)vals[e];
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int v = tid + i * NT;
      const int dd = v >> 3, kv = v & 7;
      *reinterpret_cast<uint4*>(&Bs[buf][dd * LDP + kv * 8]) = rbv[i];
    }
  };

  floatx16 acc[4][4];
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = zero16();

  const int nk = (int)((a.L + BK - 1) / BK);
  load(0);
  store(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) load(kt + 1);
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      const int g = kk * 2 + (lane >> 5);
      bf16x8 af[4], bfr[4];
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) {
        const int n = wm * 128 + mi * 32 + (lane & 31);
        af[mi] = *reinterpret_cast<const bf16x8*>(&As[buf][n * BK + swz(n, g) * 8]);
      }
#pragma unroll
      for (int ni = 0; ni < 4; ++ni)
        bfr[ni] = *reinterpret_cast<const bf16x8*>(
            &Bs[buf][(wn * 128 + ni * 32 + (lane & 31)) * LDP + kk * 16 + 8 * (lane >> 5)]);
#pragma unroll
      for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int ni = 0; ni < 4; ++ni)
          if (on[ni]) acc[mi][ni] = mfma32(af[mi], bfr[ni], acc[mi][ni]);
    }
    if (kt + 1 < nk) store(buf ^ 1);
    __syncthreads();
  }

  const float carry = scale ? powf(dv, (float)a.L) : 1.0f;
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
#pragma unroll
    for (int ni = 0; ni < 4; ++ni)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t n = n0 + wm * 128 + mi * 32 + acc_row(lane, r);
        const int64_t d = d0 + wn * 128 + ni * 32 + acc_col(lane);
        if (d < a.D) {
          const int64_t idx = (s * a.N + n) * a.D + d;
          const float prev = a.rho_in ? a.rho_in[idx] * carry : 0.0f;
          a.rho_out[idx] = prev + acc[mi][ni][r];
        }
      }
}

// ---------------------------------------------------------------------------
// ctx: O[rows r0..r0+64, e0..e0+256] of interval iv.
struct CtxArgs {
  const bf16_t* x;
  const uint32_t* cs;
  const bf16_t* vt;
  const float* part;   // gram partials [KS, S, n_iv, Lp, Lp]
  const float* rho;
  const float* decay;
  float* ctx;
  int64_t H, Hv, T, N, D, t0, L, Lp, Tp, S, n_iv, iv;
  int ks;
};

constexpr int CTX_ROWS = 64;
// LDS carve (bytes): part 1 uses Ahi, Alo [64 x LDP] and Bv [256 x LDP];
// part 2 reuses the space for Aq [64 x LDP] and Br [256 x BK] (swizzled).
constexpr int CTX_A_BYTES = CTX_ROWS * LDP * 2;
constexpr int CTX_B_BYTES = 256 * LDP * 2;
constexpr int CTX_LDS = 2 * CTX_A_BYTES + CTX_B_BYTES;

template <bool ROPE, bool HAS_RHO>
__global__ __launch_bounds__(256) void ctx_kernel(CtxArgs a) {
  const int64_t r0 = (int64_t)blockIdx.x * CTX_ROWS;
  const int64_t e0 = (int64_t)blockIdx.y * 256;
  const int64_t s = blockIdx.z;
  __shared__ __attribute__((aligned(16))) char lds[CTX_LDS];
  bf16_t* Ahi = reinterpret_cast<bf16_t*>(lds);
  bf16_t* Alo = reinterpret_cast<bf16_t*>(lds + CTX_A_BYTES);
  bf16_t* Bv = reinterpret_cast<bf16_t*>(lds + 2 * CTX_A_BYTES);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t b = s / a.H, h = s - b * a.H;
  const bf16_t* VT = a.vt + (b * a.Hv + (a.Hv == 1 ? 0 : h)) * a.D * a.Tp;
  const int64_t pstride = a.S * a.n_iv * a.Lp * a.Lp;
  const float* P0 = a.part + (s * a.n_iv + a.iv) * a.Lp * a.Lp;
  const int64_t ecol = e0 + wave * 64;  // this wave's 64 output columns
  const bool wave_on = ecol < a.D;

  floatx16 acc[2][2];
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int ni = 0; ni < 2; ++ni) acc[mi][ni] = zero16();

  // ---- part 1: tril(S) V with S = sum of the KS partials, split bf16 hi + lo
  const int64_t kend = (r0 + CTX_ROWS < a.L) ? r0 + CTX_ROWS : a.L;
  for (int64_t k0 = 0; k0 < kend; k0 += BK) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int v = tid + i * 256;
      const int m = v >> 4, c4 = v & 15;
      const int64_t row = r0 + m, col = k0 + c4 * 4;
      float4 sv = make_float4(0, 0, 0, 0);
      if (row < a.L && col < kend) {
        for (int kp = 0; kp < a.ks; ++kp) {
          const float4 pv = *reinterpret_cast<const float4*>(P0 + kp * pstride + row * a.Lp + col);
          sv.x += pv.x;
          sv.y += pv.y;
          sv.z += pv.z;
          sv.w += pv.w;
        }
        // columns >= kend lie outside the written score blocks
        if (col + 1 >= kend) sv.y = 0.0f;
        if (col + 2 >= kend) sv.z = 0.0f;
        if (col + 3 >= kend) sv.w = 0.0f;
      }
      const float hx = bf16_round(sv.x), hy = bf16_round(sv.y), hz = bf16_round(sv.z), hw = bf16_round(sv.w);
      const uint2 hv = make_uint2(pack_bf16x2(hx, hy), pack_bf16x2(hz, hw));
      const uint2 lv = make_uint2(pack_bf16x2(sv.x - hx, sv.y - hy), pack_bf16x2(sv.z - hz, sv.w - hw));
      *reinterpret_cast<uint2*>(&Ahi[m * LDP + c4 * 4]) = hv;
      *reinterpret_cast<uint2*>(&Alo[m * LDP + c4 * 4]) = lv;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int v = tid + i * 256;
      const int dd = v >> 3, kv = v & 7;
      const int64_t d = e0 + dd;
      const uint4 val = d < a.D ? ldg16(VT + d * a.Tp + a.t0 + k0 + kv * 8) : make_uint4(0, 0, 0, 0);
      *reinterpret_cast<uint4*>(&Bv[dd * LDP + kv * 8]) = val;
    }
    __syncthreads();
    if (wave_on) {
#pragma unroll
      for (int kk = 0; kk < BK / 16; ++kk) {
        const int ko = kk * 16 + 8 * (lane >> 5);
        bf16x8 ah[2], al[2], bv[2];
#pragma unroll
        for (int mi = 0; mi < 2; ++mi) {
          ah[mi] = *reinterpret_cast<const bf16x8*>(&Ahi[(mi * 32 + (lane & 31)) * LDP + ko]);
          al[mi] = *reinterpret_cast<const bf16x8*>(&Alo[(mi * 32 + (lane & 31)) * LDP + ko]);
        }
#pragma unroll
        for (int ni = 0; ni < 2; ++ni)
          bv[ni] = *reinterpret_cast<const bf16x8*>(&Bv[(wave * 64 + ni * 32 + (lane & 31)) * LDP + ko]);
#pragma unroll
        for (int mi = 0; mi < 2; ++mi)
#pragma unroll
          for (int ni = 0; ni < 2; ++ni) {
            acc[mi][ni] = mfma32(ah[mi], bv[ni], acc[mi][ni]);
            acc[mi][ni] = mfma32(al[mi], bv[ni], acc[mi][ni]);
          }
      }
    }
    __syncthreads();
  }

  // ---- part 2: (Q * d^r) rho_in ----
  if (HAS_RHO) {
    bf16_t* Aq = Ahi;                                           // [64][LDP]
    bf16_t* Br = reinterpret_cast<bf16_t*>(lds + CTX_A_BYTES);  // [256][BK] swizzled
    const int64_t half = a.N / 2;
    const bf16_t* X = a.x + (s * a.T + a.t0) * a.N;
    const uint32_t* CS = ROPE ? a.cs + a.t0 * half : nullptr;
    const float* R = a.rho + s * a.N * a.D;
    const float dv = a.decay ? a.decay[h] : 1.0f;
    const bool scale = a.decay != nullptr;
    for (int64_t k0 = 0; k0 < a.N; k0 += BK) {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int v = tid + i * 256;
        const int m = v >> 3, kv = v & 7;
        const int64_t row = r0 + m;
        const bool ok = row < a.L;
        const int64_t k = k0 + kv * 8;
        const uint4 raw = ok ? ldg16(X + row * a.N + k) : make_uint4(0, 0, 0, 0);
        uint4 c = make_uint4(0, 0, 0, 0);
        if (ROPE && ok) c = ldg16(CS + row * half + k / 2);
        const float w = scale ? powf(dv, (float)row) : 1.0f;
        *reinterpret_cast<uint4*>(&Aq[m * LDP + kv * 8]) = prep8<ROPE>(raw, c, w, scale);
      }
#pragma unroll 4
      for (int i = 0; i < 16; ++i) {
        const int v = tid + i * 256;
        const int l = v >> 6, e4 = v & 63;
        const int64_t d = e0 + e4 * 4;
        float4 rv = make_float4(0, 0, 0, 0);
        if (d < a.D) rv = *reinterpret_cast<const float4*>(R + (k0 + l) * a.D + d);
        const float vals[4] = {rv.x, rv.y, rv.z, rv.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int e = e4 * 4 + q;
          Br[e * BK + swz(e, l >> 3) * 8 + (l & 7)] = (bf16_t)vals[q];
        }
      }
      __syncthreads();
      if (wave_on) {
#pragma unroll
        for (int kk = 0; kk < BK / 16; ++kk) {
          const int g = kk * 2 + (lane >> 5);
          bf16x8 aq[2], br[2];
#pragma unroll
          for (int mi = 0; mi < 2; ++mi)
            aq[mi] = *reinterpret_cast<const bf16x8*>(&Aq[(mi * 32 + (lane & 31)) * LDP + kk * 16 + 8 * (lane >> 5)]);
#pragma unroll
          for (int ni = 0; ni < 2; ++ni) {
            const int e = wave * 64 + ni * 32 + (lane & 31);
            br[ni] = *reinterpret_cast<const bf16x8*>(&Br[e * BK + swz(e, g) * 8]);
          }
#pragma unroll
          for (int mi = 0; mi < 2; ++mi)
#pragma unroll
            for (int ni = 0; ni < 2; ++ni) acc[mi][ni] = mfma32(aq[mi], br[ni], acc[mi][ni]);
        }
      }
      __syncthreads();
    }
  }

  float* C = a.ctx + (s * a.T + a.t0) * a.D;
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int ni = 0; ni < 2; ++ni)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = r0 + mi * 32 + acc_row(lane, r);
        const int64_t d = ecol + ni * 32 + acc_col(lane);
        if (row < a.L && d < a.D) C[row * a.D + d] = acc[mi][ni][r];
      }
}

// ---------------------------------------------------------------------------
// vt[bv, d, t] = v[bv, t, d] for t < T, 0 for T <= t < Tp.
__global__ __launch_bounds__(256) void transpose_v_kernel(const bf16_t* __restrict__ v,
                                                          bf16_t* __restrict__ vt, int64_t T,
                                                          int64_t D, int64_t Tp) {
  __shared__ bf16_t tile[32][33];
  const int64_t bv = blockIdx.z;
  const int64_t t0 = (int64_t)blockIdx.x * 32, d0 = (int64_t)blockIdx.y * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
  for (int r = ty; r < 32; r += 8) {
    const int64_t t = t0 + r, d = d0 + tx;
    tile[r][tx] = (t < T && d < D) ? v[(bv * T + t) * D + d] : (bf16_t)0.0f;
  }
  __syncthreads();
  for (int r = ty; r < 32; r += 8) {
    const int64_t d = d0 + r, t = t0 + tx;
    if (d < D && t < Tp) vt[(bv * D + d) * Tp + t] = tile[tx][r];
  }
}

// Packed bf16 (cos, sin) of the RoPE phase of (token, pair): low half cos.
__global__ __launch_bounds__(256) void rope_table_bf16_kernel(const float* __restrict__ freqs,
                                                              uint32_t* __restrict__ cs, int64_t T,
                                                              int64_t half, int64_t pos_first,
                                                              int fixed) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= T * half) return;
  const int64_t t = i / half;
  const int64_t k = i - t * half;
  const float p = (float)(fixed ? pos_first : pos_first + t);
  float sn, c;
  sincosf(rope_phase(p, freqs[2 * k]), &sn, &c);
  cs[i] = pack_bf16x2(c, sn);
}

inline unsigned cdiv(int64_t a, int64_t b) { return (unsigned)((a + b - 1) / b); }

}  // namespace

bool bf16_shape_supported(int64_t N, int64_t D, const char** why) {
  if (N % GT != 0) {
    if (why) *why = "bf16 MFMA path needs latent % 256 == 0";
    return false;
  }
  if (D % 32 != 0) {
    if (why) *why = "bf16 MFMA path needs embd % 32 == 0";
    return false;
  }
  return true;
}

bdh_status run_bf16_path(const Bf16Args& a, hipStream_t st, uint64_t* launches) {
  const int64_t S = a.B * a.H;
  const int64_t half = a.N / 2;
  const int64_t Tp = ((a.T + BK - 1) / BK) * BK;
  const int64_t L = a.L;
  const int64_t n_iv = (a.T + L - 1) / L;
  const int64_t Lc0 = a.T < L ? a.T : L;
  const int64_t Lp = ((Lc0 + GT - 1) / GT) * GT;
  const int nb = (int)(Lp / GT);
  const int tiles_per_iv = nb * (nb + 1) / 2;
  // Split the gram along N until there are ~3 workgroups per CU.
  const int64_t tiles = tiles_per_iv * n_iv * S;
  int ks = (int)((768 + tiles - 1) / tiles);
  const int nk = (int)(a.N / BK);
  if (ks > 8) ks = 8;
  if (ks > nk) ks = nk;
  if (ks < 1) ks = 1;

  void *vt = nullptr, *part = nullptr, *cs = nullptr;
  bdh_status stt = scratch(SLOT_VT, (size_t)(a.B * a.Hv * a.D * Tp) * sizeof(bf16_t), &vt);
  if (stt != BDH_OK) return stt;
  stt = scratch(SLOT_SCORES, (size_t)(ks * S * n_iv * Lp * Lp) * sizeof(float), &part);
  if (stt != BDH_OK) return stt;
  if (a.freqs) {
    stt = scratch(SLOT_ROPE_TABLE, (size_t)(a.T * half) * sizeof(uint32_t), &cs);
    if (stt != BDH_OK) return stt;
  }

  hipLaunchKernelGGL(transpose_v_kernel, dim3(cdiv(Tp, 32), cdiv(a.D, 32), (unsigned)(a.B * a.Hv)),
                     dim3(256), 0, st, a.v, (bf16_t*)vt, a.T, a.D, Tp);
  uint64_t n_launch = 1;
  BDH_HIP_TRY(hipGetLastError());
  if (a.freqs) {
    hipLaunchKernelGGL(rope_table_bf16_kernel, dim3(cdiv(a.T * half, 256)), dim3(256), 0, st,
                       a.freqs, (uint32_t*)cs, a.T, half, a.pos0, a.fixed);
    BDH_HIP_TRY(hipGetLastError());
    ++n_launch;
  }

  GramArgs g{a.x, (const uint32_t*)cs, (float*)part, a.decay, a.H, a.T, a.N, L, Lp, S, n_iv,
             ks, tiles_per_iv, nb};
  const dim3 ggrid((unsigned)(tiles_per_iv * n_iv), (unsigned)ks, (unsigned)S);
  if (a.freqs) hipLaunchKernelGGL(gram_kernel<true>, ggrid, dim3(NT), 0, st, g);
  else hipLaunchKernelGGL(gram_kernel<false>, ggrid, dim3(NT), 0, st, g);
  BDH_HIP_TRY(hipGetLastError());
  ++n_launch;

  const float* rho_cur = a.rho_in;
  for (int64_t iv = 0; iv < n_iv; ++iv) {
    const int64_t t0 = iv * L;
    const int64_t Lc = (a.T - t0 < L) ? a.T - t0 : L;
    CtxArgs c{a.x, (const uint32_t*)cs, (const bf16_t*)vt, (const float*)part, rho_cur, a.decay,
              a.ctx, a.H, a.Hv, a.T, a.N, a.D, t0, Lc, Lp, Tp, S, n_iv, iv, ks};
    const dim3 cgrid(cdiv(Lc, CTX_ROWS), cdiv(a.D, 256), (unsigned)S);
    if (a.freqs) {
      if (rho_cur) hipLaunchKernelGGL((ctx_kernel<true, true>), cgrid, dim3(256), 0, st, c);
      else hipLaunchKernelGGL((ctx_kernel<true, false>), cgrid, dim3(256), 0, st, c);
    } else {
      if (rho_cur) hipLaunchKernelGGL((ctx_kernel<false, true>), cgrid, dim3(256), 0, st, c);
      else hipLaunchKernelGGL((ctx_kernel<false, false>), cgrid, dim3(256), 0, st, c);
    }
    BDH_HIP_TRY(hipGetLastError());
    ++n_launch;
    if (!a.state) continue;
    StateArgs sa{a.x, (const uint32_t*)cs, (const bf16_t*)vt, rho_cur, a.rho_out, a.decay,
                 a.H, a.Hv, a.T, a.N, a.D, t0, Lc, Tp};
    const dim3 sgrid((unsigned)(a.N / GT), cdiv(a.D, GT), (unsigned)S);
    if (a.freqs) hipLaunchKernelGGL(state_kernel<true>, sgrid, dim3(NT), 0, st, sa);
    else hipLaunchKernelGGL(state_kernel<false>, sgrid, dim3(NT), 0, st, sa);
    BDH_HIP_TRY(hipGetLastError());
    ++n_launch;
    rho_cur = a.rho_out;
  }
  if (launches) *launches += n_launch;
  return BDH_OK;
}

}  // namespace bdh
