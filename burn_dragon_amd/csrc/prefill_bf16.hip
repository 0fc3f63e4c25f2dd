// bf16 MFMA chunked prefill on gfx950 (fp32 accumulate, fp32 rho / context).
//
// The sequence is processed in state-carry intervals of L tokens (a multiple
// of the 128-token chunk).  Inside an interval the carried state of chunk c,
// rho_c = rho_in + sum_{c'<c} Q_c'^T V_c', is applied through the chunk-pair
// score blocks Q_c Q_c'^T, so rho is materialised once per interval rather
// than once per chunk:
//   gram   S[c,c'] = Q_c Q_c'^T (c' <= c; strict lower mask and d^(r-c) on
//          the diagonal blocks)                          128x128 MFMA tiles
//   ctx    O = tril(S) V + (Q * d^r) rho_in              64x256 MFMA tiles
//   state  rho_out = rho_in * d^L + (Q * d^(L-r))^T V    128x256 MFMA tiles
// RoPE is applied to the Q tiles on their way from HBM to LDS (f32 rotation
// from a per-(token, pair) cos/sin table, then bf16), so rotated queries are
// never written to memory.  All MFMAs are v_mfma_f32_32x32x16_bf16.
#include "bdh_internal.h"

namespace bdh {
namespace {

constexpr int CB = 128;        // chunk / gram tile
constexpr int BK = 64;         // k step
constexpr int LDP = BK + 8;    // padded LDS pitch (bf16) of K-contiguous tiles

__device__ __forceinline__ uint4 ldg16(const void* p) {
  return *reinterpret_cast<const uint4*>(p);
}

// Rotates the 4 (even, odd) pairs of an 8 x bf16 vector with their table
// entries (cos, sin) and scales by w; returns 8 x bf16 (RNE).
__device__ __forceinline__ uint4 rotate8(uint4 raw, float4 cs01, float4 cs23, float w) {
  const uint32_t in[4] = {raw.x, raw.y, raw.z, raw.w};
  const float c[4] = {cs01.x, cs01.z, cs23.x, cs23.z};
  const float s[4] = {cs01.y, cs01.w, cs23.y, cs23.w};
  uint32_t out[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const float e = bf16_lo(in[p]), o = bf16_hi(in[p]);
    const float ne = fmaf(e, c[p], -o * s[p]) * w;
    const float no = fmaf(o, c[p], e * s[p]) * w;
    out[p] = pack_bf16x2(ne, no);
  }
  return make_uint4(out[0], out[1], out[2], out[3]);
}

__device__ __forceinline__ uint4 scale8(uint4 raw, float w) {
  const uint32_t in[4] = {raw.x, raw.y, raw.z, raw.w};
  uint32_t out[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) out[p] = pack_bf16x2(bf16_lo(in[p]) * w, bf16_hi(in[p]) * w);
  return make_uint4(out[0], out[1], out[2], out[3]);
}

// Unpacked rotated/scaled values of an 8-vector (for transposed LDS writes).
__device__ __forceinline__ void rotate8_f32(uint4 raw, float4 cs01, float4 cs23, float w,
                                           bool rope, float (&out)[8]) {
  const uint32_t in[4] = {raw.x, raw.y, raw.z, raw.w};
  const float c[4] = {cs01.x, cs01.z, cs23.x, cs23.z};
  const float s[4] = {cs01.y, cs01.w, cs23.y, cs23.w};
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const float e = bf16_lo(in[p]), o = bf16_hi(in[p]);
    if (rope) {
      out[2 * p] = fmaf(e, c[p], -o * s[p]) * w;
      out[2 * p + 1] = fmaf(o, c[p], e * s[p]) * w;
    } else {
      out[2 * p] = e * w;
      out[2 * p + 1] = o * w;
    }
  }
}

// XOR swizzle of the 8-element groups of a 64-wide transposed tile row n:
// conflict-free 16-byte fragment reads (rows n..n+7 hit distinct groups) and
// at most 2-way conflicts on the column-wise 2-byte writes.
__device__ __forceinline__ int swz(int n, int g) { return g ^ (n & 7) ^ ((n >> 3) & 7); }

__device__ __forceinline__ float decay_pow(const float* decay, int64_t h, float e) {
  return decay ? powf(decay[h], e) : 1.0f;
}

// ---------------------------------------------------------------------------
struct GramArgs {
  const bf16_t* x;
  const float2* cs;
  float* scores;
  const float* decay;
  int64_t H, T, N, t0, L, ldS;
};

template <bool ROPE>
__global__ __launch_bounds__(256) void gram_bf16_kernel(GramArgs a) {
  const int pair = blockIdx.x;
  const int64_t s = blockIdx.y;
  int bi = (int)((sqrtf(8.0f * pair + 1.0f) - 1.0f) * 0.5f);
  while ((bi + 1) * (bi + 2) / 2 <= pair) ++bi;
  while (bi * (bi + 1) / 2 > pair) --bi;
  const int bj = pair - bi * (bi + 1) / 2;
  const bool diag = bi == bj;

  __shared__ __attribute__((aligned(16))) bf16_t As[2][CB * LDP];
  __shared__ __attribute__((aligned(16))) bf16_t Bs[2][CB * LDP];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const bool skip = diag && wn > wm;  // whole 64x64 quadrant above the diagonal
  const int64_t half = a.N / 2;
  const bf16_t* X = a.x + (s * a.T + a.t0) * a.N;
  const int64_t ri = (int64_t)bi * CB, rj = (int64_t)bj * CB;

  uint4 ra[4], rb[4];
  float4 ca[4][2], cb[4][2];
  const int kv = tid & 7;
  auto load = [&](int kt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = (tid + i * 256) >> 3;
      const int64_t k = (int64_t)kt * BK + kv * 8;
      const int64_t ti = ri + row;
      const bool vi = ti < a.L;
      ra[i] = vi ? ldg16(X + ti * a.N + k) : make_uint4(0, 0, 0, 0);
      if (ROPE) {
        const float4* c = reinterpret_cast<const float4*>(a.cs + ti * half + k / 2);
        ca[i][0] = vi ? c[0] : make_float4(0, 0, 0, 0);
        ca[i][1] = vi ? c[1] : make_float4(0, 0, 0, 0);
      }
      if (!diag) {
        const int64_t tj = rj + row;
        const bool vj = tj < a.L;
        rb[i] = vj ? ldg16(X + tj * a.N + k) : make_uint4(0, 0, 0, 0);
        if (ROPE) {
          const float4* c = reinterpret_cast<const float4*>(a.cs + tj * half + k / 2);
          cb[i][0] = vj ? c[0] : make_float4(0, 0, 0, 0);
          cb[i][1] = vj ? c[1] : make_float4(0, 0, 0, 0);
        }
      }
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = (tid + i * 256) >> 3;
      const uint4 va = ROPE ? rotate8(ra[i], ca[i][0], ca[i][1], 1.0f) : ra[i];
      *reinterpret_cast<uint4*>(&As[buf][row * LDP + kv * 8]) = va;
      if (!diag) {
        const uint4 vb = ROPE ? rotate8(rb[i], cb[i][0], cb[i][1], 1.0f) : rb[i];
        *reinterpret_cast<uint4*>(&Bs[buf][row * LDP + kv * 8]) = vb;
      }
    }
  };

  floatx16 acc[2][2];
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int ni = 0; ni < 2; ++ni) acc[mi][ni] = zero16();

  const int nk = (int)(a.N / BK);
  load(0);
  store(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) load(kt + 1);
    if (!skip) {
      const bf16_t* Ab = As[buf];
      const bf16_t* Bb = diag ? As[buf] : Bs[buf];
#pragma unroll
      for (int kk = 0; kk < BK / 16; ++kk) {
        const int ko = kk * 16 + 8 * (lane >> 5);
        bf16x8 af[2], bfr[2];
#pragma unroll
        for (int mi = 0; mi < 2; ++mi)
          af[mi] = *reinterpret_cast<const bf16x8*>(&Ab[(wm * 64 + mi * 32 + (lane & 31)) * LDP + ko]);
#pragma unroll
        for (int ni = 0; ni < 2; ++ni)
          bfr[ni] = *reinterpret_cast<const bf16x8*>(&Bb[(wn * 64 + ni * 32 + (lane & 31)) * LDP + ko]);
#pragma unroll
        for (int mi = 0; mi < 2; ++mi)
#pragma unroll
          for (int ni = 0; ni < 2; ++ni) acc[mi][ni] = mfma32(af[mi], bfr[ni], acc[mi][ni]);
      }
    }
    if (kt + 1 < nk) store(buf ^ 1);
    __syncthreads();
  }

  const int64_t h = s % a.H;
  float* Sg = a.scores + s * a.ldS * a.ldS;
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int ni = 0; ni < 2; ++ni)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t ti = ri + wm * 64 + mi * 32 + acc_row(lane, r);
        const int64_t tj = rj + wn * 64 + ni * 32 + acc_col(lane);
        if (ti < a.L && tj < a.L) {
          const float v = tj < ti ? acc[mi][ni][r] * decay_pow(a.decay, h, (float)(ti - tj)) : 0.0f;
          Sg[ti * a.ldS + tj] = v;
        }
      }
}

// ---------------------------------------------------------------------------
struct StateArgs {
  const bf16_t* x;
  const float2* cs;
  const bf16_t* vt;   // [B*Hv, D, Tp]
  const float* rho_in;
  float* rho_out;
  const float* decay;
  int64_t H, Hv, T, N, D, t0, L, Tp;
};

template <bool ROPE>
__global__ __launch_bounds__(256) void state_bf16_kernel(StateArgs a) {
  const int64_t n0 = (int64_t)blockIdx.x * 128;
  const int64_t d0 = (int64_t)blockIdx.y * 256;
  const int64_t s = blockIdx.z;
  __shared__ __attribute__((aligned(16))) bf16_t As[2][128 * BK];    // [n][t], swizzled
  __shared__ __attribute__((aligned(16))) bf16_t Bs[2][256 * LDP];   // [d][t]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t half = a.N / 2;
  const int64_t b = s / a.H, h = s - b * a.H;
  const bf16_t* X = a.x + (s * a.T + a.t0) * a.N;
  const bf16_t* VT = a.vt + (b * a.Hv + (a.Hv == 1 ? 0 : h)) * a.D * a.Tp;
  const float dv = a.decay ? a.decay[h] : 1.0f;

  uint4 ra[4];
  float4 ca[4][2];
  float wa[4];
  uint4 rbv[8];
  auto load = [&](int kt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int v = tid + i * 256;
      const int tt = v >> 4, nv = v & 15;
      const int64_t tl = (int64_t)kt * BK + tt;
      const bool ok = tl < a.L;
      const int64_t n = n0 + nv * 8;
      ra[i] = ok ? ldg16(X + tl * a.N + n) : make_uint4(0, 0, 0, 0);
      if (ROPE) {
        const float4* c = reinterpret_cast<const float4*>(a.cs + tl * half + n / 2);
        ca[i][0] = ok ? c[0] : make_float4(0, 0, 0, 0);
        ca[i][1] = ok ? c[1] : make_float4(0, 0, 0, 0);
      }
      wa[i] = a.decay ? powf(dv, (float)(a.L - tl)) : 1.0f;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int v = tid + i * 256;
      const int dd = v >> 3, kv = v & 7;
      const int64_t d = d0 + dd;
      rbv[i] = d < a.D ? ldg16(VT + d * a.Tp + a.t0 + (int64_t)kt * BK + kv * 8)
                       : make_uint4(0, 0, 0, 0);
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int v = tid + i * 256;
      const int tt = v >> 4, nv = v & 15;
      float vals[8];
      rotate8_f32(ra[i], ca[i][0], ca[i][1], wa[i], ROPE, vals);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int n = nv * 8 + e;
        As[buf][n * BK + swz(n, tt >> 3) * 8 + (tt & 7)] = (bf16_t)vals[e];
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int v = tid + i * 256;
      const int dd = v >> 3, kv = v & 7;
      *reinterpret_cast<uint4*>(&Bs[buf][dd * LDP + kv * 8]) = rbv[i];
    }
  };

  floatx16 acc[2][4];
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
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
      bf16x8 af[2], bfr[4];
#pragma unroll
      for (int mi = 0; mi < 2; ++mi) {
        const int n = wm * 64 + mi * 32 + (lane & 31);
        af[mi] = *reinterpret_cast<const bf16x8*>(&As[buf][n * BK + swz(n, g) * 8]);
      }
#pragma unroll
      for (int ni = 0; ni < 4; ++ni)
        bfr[ni] = *reinterpret_cast<const bf16x8*>(
            &Bs[buf][(wn * 128 + ni * 32 + (lane & 31)) * LDP + kk * 16 + 8 * (lane >> 5)]);
#pragma unroll
      for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 4; ++ni)
          if (d0 + wn * 128 + ni * 32 < a.D) acc[mi][ni] = mfma32(af[mi], bfr[ni], acc[mi][ni]);
    }
    if (kt + 1 < nk) store(buf ^ 1);
    __syncthreads();
  }

  const float carry = a.decay ? powf(dv, (float)a.L) : 1.0f;
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int ni = 0; ni < 4; ++ni)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t n = n0 + wm * 64 + mi * 32 + acc_row(lane, r);
        const int64_t d = d0 + wn * 128 + ni * 32 + acc_col(lane);
        if (d < a.D) {
          const int64_t idx = (s * a.N + n) * a.D + d;
          const float prev = a.rho_in ? a.rho_in[idx] * carry : 0.0f;
          a.rho_out[idx] = prev + acc[mi][ni][r];
        }
      }
}

// ---------------------------------------------------------------------------
struct CtxArgs {
  const bf16_t* x;
  const float2* cs;
  const bf16_t* vt;
  const float* scores;
  const float* rho;
  const float* decay;
  float* ctx;
  int64_t H, Hv, T, N, D, t0, L, ldS, Tp;
};

constexpr int CTX_ROWS = 64;
// LDS carve (bytes): part 1 uses Ahi, Alo [64 x LDP] and Bv [256 x LDP];
// part 2 reuses the same space for Aq [64 x LDP] and Br [256 x BK] (swizzled).
constexpr int CTX_A_BYTES = CTX_ROWS * LDP * 2;
constexpr int CTX_B_BYTES = 256 * LDP * 2;
constexpr int CTX_LDS = 2 * CTX_A_BYTES + CTX_B_BYTES;

template <bool ROPE, bool HAS_RHO>
__global__ __launch_bounds__(256) void ctx_bf16_kernel(CtxArgs a) {
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
  const float* Sg = a.scores + s * a.ldS * a.ldS;
  const int64_t ecol = e0 + wave * 64;  // this wave's 64 output columns
  const bool wave_on = ecol < a.D;

  floatx16 acc[2][2];
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int ni = 0; ni < 2; ++ni) acc[mi][ni] = zero16();

  // ---- part 1: tril(S) V with S split into bf16 hi + lo ----
  const int64_t kend = (r0 + CTX_ROWS < a.L) ? r0 + CTX_ROWS : a.L;
  for (int64_t k0 = 0; k0 < kend; k0 += BK) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int v = tid + i * 256;
      const int m = v >> 4, c4 = v & 15;
      const int64_t row = r0 + m, col = k0 + c4 * 4;
      float4 sv = make_float4(0, 0, 0, 0);
      if (row < a.L && col < kend) {
        // columns >= kend are outside the written score blocks: mask each lane
        sv = *reinterpret_cast<const float4*>(Sg + row * a.ldS + col);
        if (col + 1 >= kend) sv.y = 0.0f;
        if (col + 2 >= kend) sv.z = 0.0f;
        if (col + 3 >= kend) sv.w = 0.0f;
      }
      const float hx = bf16_round(sv.x), hy = bf16_round(sv.y), hz = bf16_round(sv.z), hw = bf16_round(sv.w);
      uint2 hv = make_uint2(pack_bf16x2(hx, hy), pack_bf16x2(hz, hw));
      uint2 lv = make_uint2(pack_bf16x2(sv.x - hx, sv.y - hy), pack_bf16x2(sv.z - hz, sv.w - hw));
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
    bf16_t* Aq = Ahi;                                        // [64][LDP]
    bf16_t* Br = reinterpret_cast<bf16_t*>(lds + CTX_A_BYTES);  // [256][BK] swizzled
    const int64_t half = a.N / 2;
    const bf16_t* X = a.x + (s * a.T + a.t0) * a.N;
    const float* R = a.rho + s * a.N * a.D;
    const float dv = a.decay ? a.decay[h] : 1.0f;
    for (int64_t k0 = 0; k0 < a.N; k0 += BK) {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int v = tid + i * 256;
        const int m = v >> 3, kv = v & 7;
        const int64_t row = r0 + m;
        const bool ok = row < a.L;
        const int64_t k = k0 + kv * 8;
        uint4 raw = ok ? ldg16(X + row * a.N + k) : make_uint4(0, 0, 0, 0);
        const float w = a.decay ? powf(dv, (float)row) : 1.0f;
        uint4 val;
        if (ROPE) {
          const float4* c = reinterpret_cast<const float4*>(a.cs + row * half + k / 2);
          const float4 c0 = ok ? c[0] : make_float4(0, 0, 0, 0);
          const float4 c1 = ok ? c[1] : make_float4(0, 0, 0, 0);
          val = rotate8(raw, c0, c1, w);
        } else {
          val = a.decay ? scale8(raw, w) : raw;
        }
        *reinterpret_cast<uint4*>(&Aq[m * LDP + kv * 8]) = val;
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

inline unsigned cdiv(int64_t a, int64_t b) { return (unsigned)((a + b - 1) / b); }

}  // namespace

bool bf16_shape_supported(int64_t N, int64_t D, const char** why) {
  if (N % 128 != 0) {
    if (why) *why = "bf16 MFMA path needs latent % 128 == 0";
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
  const int64_t Lc0 = a.T < L ? a.T : L;
  const int64_t ldS = ((Lc0 + CB - 1) / CB) * CB;

  void *vt = nullptr, *scores = nullptr, *cs = nullptr;
  bdh_status stt = scratch(SLOT_VT, (size_t)(a.B * a.Hv * a.D * Tp) * sizeof(bf16_t), &vt);
  if (stt != BDH_OK) return stt;
  stt = scratch(SLOT_SCORES, (size_t)(S * ldS * ldS) * sizeof(float), &scores);
  if (stt != BDH_OK) return stt;
  if (a.freqs) {
    stt = scratch(SLOT_ROPE_TABLE, (size_t)(ldS * half) * sizeof(float2), &cs);
    if (stt != BDH_OK) return stt;
  }

  hipLaunchKernelGGL(transpose_v_kernel, dim3(cdiv(Tp, 32), cdiv(a.D, 32), (unsigned)(a.B * a.Hv)),
                     dim3(256), 0, st, a.v, (bf16_t*)vt, a.T, a.D, Tp);
  uint64_t n_launch = 1;
  BDH_HIP_TRY(hipGetLastError());

  const float* rho_cur = a.rho_in;
  for (int64_t t0 = 0; t0 < a.T; t0 += L) {
    const int64_t Lc = (a.T - t0 < L) ? a.T - t0 : L;
    if (a.freqs) {
      BDH_HIP_TRY(launch_rope_table(a.freqs, (float2*)cs, Lc, half,
                                    a.fixed ? a.pos0 : a.pos0 + t0, a.fixed, st));
      ++n_launch;
    }
    const int nb = (int)((Lc + CB - 1) / CB);
    GramArgs g{a.x, (const float2*)cs, (float*)scores, a.decay, a.H, a.T, a.N, t0, Lc, ldS};
    const dim3 ggrid((unsigned)(nb * (nb + 1) / 2), (unsigned)S);
    if (a.freqs) hipLaunchKernelGGL(gram_bf16_kernel<true>, ggrid, dim3(256), 0, st, g);
    else hipLaunchKernelGGL(gram_bf16_kernel<false>, ggrid, dim3(256), 0, st, g);
    BDH_HIP_TRY(hipGetLastError());

    CtxArgs c{a.x, (const float2*)cs, (const bf16_t*)vt, (const float*)scores, rho_cur,
              a.decay, a.ctx, a.H, a.Hv, a.T, a.N, a.D, t0, Lc, ldS, Tp};
    const dim3 cgrid(cdiv(Lc, CTX_ROWS), cdiv(a.D, 256), (unsigned)S);
    if (a.freqs) {
      if (rho_cur) hipLaunchKernelGGL((ctx_bf16_kernel<true, true>), cgrid, dim3(256), 0, st, c);
      else hipLaunchKernelGGL((ctx_bf16_kernel<true, false>), cgrid, dim3(256), 0, st, c);
    } else {
      if (rho_cur) hipLaunchKernelGGL((ctx_bf16_kernel<false, true>), cgrid, dim3(256), 0, st, c);
      else hipLaunchKernelGGL((ctx_bf16_kernel<false, false>), cgrid, dim3(256), 0, st, c);
    }
    BDH_HIP_TRY(hipGetLastError());

    n_launch += 2;
    if (!a.state) continue;
    StateArgs sa{a.x, (const float2*)cs, (const bf16_t*)vt, rho_cur, a.rho_out, a.decay,
                 a.H, a.Hv, a.T, a.N, a.D, t0, Lc, Tp};
    const dim3 sgrid((unsigned)(a.N / 128), cdiv(a.D, 256), (unsigned)S);
    if (a.freqs) hipLaunchKernelGGL(state_bf16_kernel<true>, sgrid, dim3(256), 0, st, sa);
    else hipLaunchKernelGGL(state_bf16_kernel<false>, sgrid, dim3(256), 0, st, sa);
    BDH_HIP_TRY(hipGetLastError());
    ++n_launch;
    rho_cur = a.rho_out;
  }
  if (launches) *launches += n_launch;
  return BDH_OK;
}

}  // namespace bdh
