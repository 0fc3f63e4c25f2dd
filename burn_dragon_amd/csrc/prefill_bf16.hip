// bf16 MFMA chunked prefill on gfx950 (fp32 accumulate, fp32 rho / context):
// orchestration, context kernel, value transpose and RoPE table.
//
// The sequence is split into state-carry intervals of L tokens (L a multiple
// of the 128-token chunk).  Inside an interval the carried state of chunk c,
// rho_c = rho_iv + sum_{c'<c} Q_c'^T V_c', is applied through the chunk-pair
// score blocks Q_c Q_c'^T, so rho is materialised once per interval instead
// of once per chunk.  Per interval iv (state rho_iv at its start):
//   gram    S = tril(-1)(Q Q^T * d^(r-c)), split along N into KS partial
//           buffers (all intervals, in the first launch: it needs no rho)
//   readout (Q * d^r) rho_iv, split along N into rd_kr partial buffers
//   state   rho_{iv+1} = rho_iv * d^L + (Q * d^(L-r))^T V
//   ctx     O = tril(S) V + readout    (this file; sums the partials in a
//           fixed order, S split into bf16 hi + lo)
// gram, readout and state units share one launch per interval
// (mfma_prefill.hip); the states between intervals alternate between two
// scratch buffers and the last one lands in rho_out.
// RoPE is applied to Q tiles between HBM and LDS, each lane computing the
// (cos, sin) of its pairs from the f32 phase; with one interval rotated
// queries are never written to memory.
#include <cstdlib>
#include <type_traits>

#include "bdh_bf16.h"

namespace bdh {
namespace {

constexpr int CK = 32;         // k step of the context kernel: 64-byte LDS rows
constexpr int CTX_ROWS = 64;   // output rows of one workgroup
constexpr int CTX_COLS = 256;  // output columns of a wide workgroup (4 waves x 64); narrow: 128

// Element offset of 16-byte chunk c (0..3) of a 64-byte LDS row r, XOR
// swizzled with bits 1..2 of the row: conflict-free for MFMA fragment reads
// (8 consecutive rows of one chunk per LDS cycle) and for row-segment writes.
__device__ __forceinline__ int cofs(int r, int c) { return r * CK + ((c ^ ((r >> 1) & 3)) << 3); }

// O = tril(S) V for every interval in [iv0, iv0 + n_ivc) at once: S is the
// sum of the KS gram partials of its interval, which the first prefill
// launch writes for all intervals.  (The readout of a carried state is added
// per interval by readout_add_kernel.)
struct CtxArgs {
  const bf16_t* vt;      // v^T [B*Hv, Tp/32, Dp, 32]
  const float* part;     // gram partials [KS, S, n_iv, Lp, Lp]
  float* ctx;            // [S, T, D]
  int64_t H, Hv, T, D, L, Lp, Tp, Dp, S, n_iv;
  int iv0, n_ivc;        // intervals covered by this launch
  int nrb;               // CTX_ROWS row blocks per interval: ceil(min(L, T) / 64)
  // Readout partials added to the context of intervals iv >= rd_iv0 (null:
  // none): rd [rd_kr, S, T, D], summed in split order.
  const float* rd;
  int rd_kr;
  int64_t rd_iv0;
  int part16;            // part holds bf16 partials (snap_wide_kernel's part16)
};

// Workgroup id -> (row block, interval, stream): row blocks heaviest first
// (row block rb contracts over 64 (rb + 1) columns), then interval, then
// stream.  blockIdx.y is the column block: 4 waves x WC columns (WC = 64, or
// 32 when the wide blocks would leave CUs with fewer than two workgroups).
template <int KS, int WC, bool P16>
__global__ __launch_bounds__(256, 2) void ctx_kernel(CtxArgs a) {
  constexpr int NI = WC / 32, COLS = 4 * WC;
  const int nz = (int)(a.S * a.n_ivc);
  const int id = blockIdx.x;
  const int rb = a.nrb - 1 - id / nz;
  const int z = id - (id / nz) * nz;
  const int64_t iv = a.iv0 + z / a.S, s = z % a.S;
  const int64_t t0 = iv * a.L;
  const int64_t Lc = (a.T - t0 < a.L) ? a.T - t0 : a.L;
  const int64_t r0 = (int64_t)rb * CTX_ROWS;
  if (r0 >= Lc) return;  // a ragged last interval has fewer row blocks
  const int64_t e0 = (int64_t)blockIdx.y * COLS;

  __shared__ __attribute__((aligned(16))) bf16_t Ahi[CTX_ROWS * CK];
  __shared__ __attribute__((aligned(16))) bf16_t Alo[CTX_ROWS * CK];
  __shared__ __attribute__((aligned(16))) bf16_t Bv[COLS * CK];

  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int64_t b = s / a.H, h = s - b * a.H;
  const bf16_t* VT = a.vt + (b * a.Hv + (a.Hv == 1 ? 0 : h)) * a.Dp * a.Tp + (t0 >> 5) * (a.Dp * 32);
  const int64_t pstride = a.S * a.n_iv * a.Lp * a.Lp;
  const float* P0 = a.part + (s * a.n_iv + iv) * a.Lp * a.Lp;
  const int64_t ecol = e0 + wave * WC;  // this wave's WC output columns
  const bool wave_on = ecol < a.D;
  // Columns [0, kend) of the score rows r0 .. r0+63 are written by the gram
  // (zero on and above the diagonal); past kend nothing is read.
  const int64_t kend = (r0 + CTX_ROWS < Lc) ? r0 + CTX_ROWS : Lc;
  const int nk = (int)((kend + CK - 1) / CK);

  // Loaders.  Scores: 8 lanes per 32-column row segment (4 floats each),
  // rows m and m + 32.  v^T: 4 lanes per 64-byte row segment of the step,
  // rows dv + 64 i (v^T is zero past D up to Dp, a multiple of 256, so no
  // column test).
  const int sm = tid >> 3, sc = tid & 7;
  const int dv = tid >> 2, kc = tid & 3;
  // bf16 partials stay packed (two words per 4 scores) until they are summed.
  struct Stage {
    std::conditional_t<P16, uint2, float4> p[2][KS];
    uint4 v[NI * 2];
  } st;
  auto score4 = [&](int i, int kp) -> float4 {
    if constexpr (P16) {
      const uint2 w = st.p[i][kp];
      return make_float4(bf16_lo(w.x), bf16_hi(w.x), bf16_lo(w.y), bf16_hi(w.y));
    } else {
      return st.p[i][kp];
    }
  };
  const bf16_t* P16b = reinterpret_cast<const bf16_t*>(a.part) + (s * a.n_iv + iv) * a.Lp * a.Lp;
  auto load = [&](int kt) {
    const int64_t k0 = (int64_t)kt * CK;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int64_t row = r0 + sm + 32 * i, col = k0 + sc * 4;
      const bool in = row < Lc && col < kend;
#pragma unroll
      for (int kp = 0; kp < KS; ++kp) {
        if constexpr (P16)
          st.p[i][kp] = in ? *reinterpret_cast<const uint2*>(P16b + kp * pstride + row * a.Lp + col) : make_uint2(0, 0);
        else
          st.p[i][kp] = in ? *reinterpret_cast<const float4*>(P0 + kp * pstride + row * a.Lp + col)
                           : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      }
    }
#pragma unroll
    for (int i = 0; i < NI * 2; ++i) st.v[i] = ldg16(VT + (k0 >> 5) * (a.Dp * 32) + (e0 + dv + 64 * i) * 32 + kc * 8);
  };
  auto store = [&](int kt) {
    const int64_t k0 = (int64_t)kt * CK;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      float4 sv = score4(i, 0);
#pragma unroll
      for (int kp = 1; kp < KS; ++kp) {
        const float4 pv = score4(i, kp);
        sv.x += pv.x;
        sv.y += pv.y;
        sv.z += pv.z;
        sv.w += pv.w;
      }
      // a step that runs past kend (ragged interval) reads zeros there
      const int64_t col = k0 + sc * 4;
      if (col + 1 >= kend) sv.y = 0.0f;
      if (col + 2 >= kend) sv.z = 0.0f;
      if (col + 3 >= kend) sv.w = 0.0f;
      const float hx = bf16_round(sv.x), hy = bf16_round(sv.y), hz = bf16_round(sv.z), hw = bf16_round(sv.w);
      const int o = cofs(sm + 32 * i, sc >> 1) + (sc & 1) * 4;
      *reinterpret_cast<uint2*>(&Ahi[o]) = make_uint2(pack_bf16x2(hx, hy), pack_bf16x2(hz, hw));
      *reinterpret_cast<uint2*>(&Alo[o]) =
          make_uint2(pack_bf16x2(sv.x - hx, sv.y - hy), pack_bf16x2(sv.z - hz, sv.w - hw));
    }
#pragma unroll
    for (int i = 0; i < NI * 2; ++i) *reinterpret_cast<uint4*>(&Bv[cofs(dv + 64 * i, kc)]) = st.v[i];
  };

  floatx16 acc[2][NI];
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) acc[mi][ni] = zero16();

  load(0);
  for (int kt = 0; kt < nk; ++kt) {
    store(kt);
    __syncthreads();
    if (kt + 1 < nk) load(kt + 1);
    if (wave_on) {
#pragma unroll
      for (int kk = 0; kk < CK / 16; ++kk) {
        const int c = 2 * kk + (lane >> 5);
        bf16x8 ah[2], al[2], bv[NI];
#pragma unroll
        for (int mi = 0; mi < 2; ++mi) {
          ah[mi] = *reinterpret_cast<const bf16x8*>(&Ahi[cofs(mi * 32 + (lane & 31), c)]);
          al[mi] = *reinterpret_cast<const bf16x8*>(&Alo[cofs(mi * 32 + (lane & 31), c)]);
        }
#pragma unroll
        for (int ni = 0; ni < NI; ++ni)
          bv[ni] = *reinterpret_cast<const bf16x8*>(&Bv[cofs(wave * WC + ni * 32 + (lane & 31), c)]);
#pragma unroll
        for (int mi = 0; mi < 2; ++mi)
#pragma unroll
          for (int ni = 0; ni < NI; ++ni) {
            acc[mi][ni] = mfma32(ah[mi], bv[ni], acc[mi][ni]);
            acc[mi][ni] = mfma32(al[mi], bv[ni], acc[mi][ni]);
          }
      }
    }
    __syncthreads();
  }

  if (!wave_on) return;
  float* C = a.ctx + (s * a.T + t0) * a.D;
  if (a.rd != nullptr && iv >= a.rd_iv0) {
    // Readout partials added in split order, every load of a partial issued
    // before any context store: loads after a store that the compiler cannot
    // prove distinct would each wait out a memory round trip.
    const float* RD = a.rd + (s * a.T + t0) * a.D;
    const int64_t rd_stride = a.S * a.T * a.D;
    for (int kp = 0; kp < a.rd_kr; ++kp) {
      float rv[2][NI][16];
#pragma unroll
      for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < NI; ++ni)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int64_t row = r0 + mi * 32 + acc_row(lane, r);
            const int64_t d = ecol + ni * 32 + acc_col(lane);
            rv[mi][ni][r] = row < Lc && d < a.D ? RD[kp * rd_stride + row * a.D + d] : 0.0f;
          }
#pragma unroll
      for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < NI; ++ni)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[mi][ni][r] += rv[mi][ni][r];
    }
  }
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int ni = 0; ni < NI; ++ni)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = r0 + mi * 32 + acc_row(lane, r);
        const int64_t d = ecol + ni * 32 + acc_col(lane);
        if (row < Lc && d < a.D) C[row * a.D + d] = acc[mi][ni][r];
      }
}

template <int WC, bool P16>
hipError_t launch_ctx_wc(const CtxArgs& c, int ks, hipStream_t st) {
  const int cols = 4 * WC;
  const dim3 grid((unsigned)(c.nrb * c.S * c.n_ivc), (unsigned)((c.D + cols - 1) / cols));
  switch (ks) {
    case 1: hipLaunchKernelGGL((ctx_kernel<1, WC, P16>), grid, dim3(256), 0, st, c); break;
    case 2: hipLaunchKernelGGL((ctx_kernel<2, WC, P16>), grid, dim3(256), 0, st, c); break;
    case 4: hipLaunchKernelGGL((ctx_kernel<4, WC, P16>), grid, dim3(256), 0, st, c); break;
    case 8: hipLaunchKernelGGL((ctx_kernel<8, WC, P16>), grid, dim3(256), 0, st, c); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// Measured at C2 (256 wide workgroups): narrow 24.2 us against 26.6; at C4
// and C5 (512 and more wide workgroups) narrow is slower.
hipError_t launch_ctx(const CtxArgs& c, int ks, hipStream_t st) {
  const int64_t wide = c.nrb * c.S * c.n_ivc * ((c.D + CTX_COLS - 1) / CTX_COLS);
  if (c.part16) {
    if (wide < 2 * (int64_t)device_cus()) return launch_ctx_wc<32, true>(c, ks, st);
    return launch_ctx_wc<64, true>(c, ks, st);
  }
  if (wide < 2 * (int64_t)device_cus()) return launch_ctx_wc<32, false>(c, ks, st);
  return launch_ctx_wc<64, false>(c, ks, st);
}

// ctx[s, t0 + t, :] += sum over the rd_kr readout partials (fixed order),
// one float4 of columns per thread.
__global__ __launch_bounds__(256) void readout_add_kernel(const float* __restrict__ rd, float* __restrict__ ctx,
                                                          int64_t S, int64_t T, int64_t D, int64_t t0,
                                                          int64_t Lc, int64_t Lp, int kr) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // (s, t, d4)
  const int64_t d4n = D / 4;
  if (i >= S * Lc * d4n) return;
  const int64_t s = i / (Lc * d4n);
  const int64_t rem = i - s * Lc * d4n;
  const int64_t t = rem / d4n, d = (rem - t * d4n) * 4;
  float4 v = *reinterpret_cast<const float4*>(&ctx[(s * T + t0 + t) * D + d]);
  for (int kp = 0; kp < kr; ++kp) {
    const float4 r = *reinterpret_cast<const float4*>(&rd[((kp * S + s) * Lp + t) * D + d]);
    v.x += r.x;
    v.y += r.y;
    v.z += r.z;
    v.w += r.w;
  }
  *reinterpret_cast<float4*>(&ctx[(s * T + t0 + t) * D + d]) = v;
}

// v^T, step-major: element (bv, d, t) at bv Dp Tp + (t / 32) Dp 32 + d 32 +
// t % 32, = v[bv, t, d] for t < T, d < D and 0 for T <= t < Tp or D <= d < Dp.
// One 32-token step of every column is then one contiguous Dp x 64-byte
// block, so a consumer's 64-byte row segments of a step come in 1 KiB runs
// per wave load (with rows of Tp tokens they were 64-byte pieces 2 Tp bytes
// apart).  One 64 x 64 tile (tokens t0 .., columns d0 ..): 16-byte loads of v
// rows (8 columns; D is a multiple of 32, so 8 columns are all inside D or
// all past it) into LDS, 16-byte stores of 8 tokens (Tp is a multiple of
// 128).  Zeros past T and D.
constexpr int VT_TILE = 64;
__device__ __forceinline__ void transpose_v_tile(const bf16_t* __restrict__ v, bf16_t* __restrict__ vt,
                                                 int64_t T, int64_t D, int64_t Tp, int64_t Dp,
                                                 int64_t bv, int64_t t0, int64_t d0) {
  __shared__ __attribute__((aligned(16))) uint32_t tile[VT_TILE][VT_TILE / 2 + 1];  // [t][d pair]
  const int tid = threadIdx.x;
  for (int i = tid; i < VT_TILE * 8; i += 256) {
    const int r = i >> 3, c = (i & 7) * 8;
    const int64_t t = t0 + r, d = d0 + c;
    uint4 e = make_uint4(0, 0, 0, 0);
    if (t < T && d < D) e = *reinterpret_cast<const uint4*>(v + (bv * T + t) * D + d);
    tile[r][c / 2] = e.x;
    tile[r][c / 2 + 1] = e.y;
    tile[r][c / 2 + 2] = e.z;
    tile[r][c / 2 + 3] = e.w;
  }
  __syncthreads();
  for (int i = tid; i < VT_TILE * 8; i += 256) {
    const int r = i >> 3, c = (i & 7) * 8;  // v^T row d0 + r, tokens t0 + c ..
    const int64_t d = d0 + r, t = t0 + c;
    if (d >= Dp || t >= Tp) continue;
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t a = tile[c + 2 * j][r >> 1], b = tile[c + 2 * j + 1][r >> 1];
      // element r of tokens c + 2j and c + 2j + 1: the low or high half of their words
      w[j] = (r & 1) ? ((a >> 16) | (b & 0xffff0000u)) : ((a & 0xffffu) | (b << 16));
    }
    *reinterpret_cast<uint4*>(vt + bv * Dp * Tp + (t >> 5) * (Dp * 32) + d * 32 + (t & 31)) =
        make_uint4(w[0], w[1], w[2], w[3]);
  }
}

__global__ __launch_bounds__(256) void transpose_v_kernel(const bf16_t* __restrict__ v,
                                                          bf16_t* __restrict__ vt, int64_t T,
                                                          int64_t D, int64_t Tp, int64_t Dp) {
  transpose_v_tile(v, vt, T, D, Tp, Dp, blockIdx.z, (int64_t)blockIdx.x * VT_TILE,
                   (int64_t)blockIdx.y * VT_TILE);
}

// q[s, t, :] = rope(x[s, t, :]) in bf16: phase frac(p f) in the reference's
// f32 op order, cos / sin by v_cos_f32 / v_sin_f32 of it, the rotation in f32
// in the op order of attention.rs:488-501, then rounded to bf16.  Workgroup b
// covers 2048 elements (8 a lane) of the ROT_ROWS rows row0 + ROT_ROWS (b /
// segs) + r (r < ROT_ROWS, rows < row_end): one frequency load and ROT_ROWS
// x loads in flight per lane, rows and positions workgroup-uniform (scalar
// arithmetic).  q is written with streaming stores: it is read by later
// launches, after far more than the caches hold has passed through them.
constexpr int ROT_SEG = 2048;
constexpr int ROT_ROWS = 4;
__global__ __launch_bounds__(256) void rope_rotate_bf16_kernel(const bf16_t* __restrict__ x,
                                                               const float* __restrict__ freqs,
                                                               bf16_t* __restrict__ q, int64_t row0,
                                                               int64_t row_end, int64_t segs, int64_t T,
                                                               int64_t N, int64_t pos_first, int fixed) {
  const int64_t b = blockIdx.x / segs;
  const int64_t n = (blockIdx.x - b * segs) * ROT_SEG + threadIdx.x * 8;
  const int64_t rb = row0 + b * ROT_ROWS;
  if (n >= N) return;  // N % 8 == 0: a lane's 8 elements are all in the row or all past it
  const float4 f0 = *reinterpret_cast<const float4*>(freqs + n);
  const float4 f1 = *reinterpret_cast<const float4*>(freqs + n + 4);
  const float f[4] = {f0.x, f0.z, f1.x, f1.z};  // one frequency per pair
  uint4 raw[ROT_ROWS];
#pragma unroll
  for (int r = 0; r < ROT_ROWS; ++r)
    if (rb + r < row_end) raw[r] = *reinterpret_cast<const uint4*>(x + (rb + r) * N + n);
#pragma unroll
  for (int r = 0; r < ROT_ROWS; ++r) {
    const int64_t row = rb + r;
    if (row >= row_end) break;
    const float p = (float)(fixed ? pos_first : pos_first + row % T);
    const uint32_t in[4] = {raw[r].x, raw[r].y, raw[r].z, raw[r].w};
    uint32_t out[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float fr = rope_frac(p, f[k]);
      float e, o;
      rope_pair_exact(bf16_lo(in[k]), bf16_hi(in[k]), __builtin_amdgcn_cosf(fr),
                      __builtin_amdgcn_sinf(fr), e, o);
      out[k] = pack_bf16x2(e, o);
    }
    __builtin_nontemporal_store(u32x4{out[0], out[1], out[2], out[3]},
                                reinterpret_cast<u32x4*>(q + row * N + n));
  }
}

inline unsigned cdiv(int64_t a, int64_t b) { return (unsigned)((a + b - 1) / b); }

}  // namespace

// Intervals from which a RoPE prefill rotates x in a pass of its own rather
// than in every launch's tile loads.
#ifndef BDH_PREROT_MIN_IV
#define BDH_PREROT_MIN_IV 2
#endif

bool bf16_shape_supported(int64_t N, int64_t D, const char** why) {
  if (N % T256 != 0) {
    if (why) *why = "bf16 MFMA path needs latent % 256 == 0";
    return false;
  }
  if (D % 32 != 0) {
    if (why) *why = "bf16 MFMA path needs embd % 32 == 0";
    return false;
  }
  return true;
}

// Compute units of the current device (256 on MI355X), cached per device.
int device_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

// Largest bf16 state-snapshot buffer of the state-carry form; past it the
// per-interval launch chain runs (two f32 states).
constexpr size_t kCarrySnapMax = (size_t)8 << 30;

namespace {
// Two or more intervals, no decay: v^T, the state-carry kernel (which also
// rotates x once and writes q), one launch of every interval's gram tiles
// and readouts (from the bf16 snapshots), then the context kernel, which
// adds the readout partials.  Four launches whatever the interval count.
bdh_status run_carry_path(const Bf16Args& a, hipStream_t st, uint64_t* launches, int64_t S, int64_t Tp,
                          int64_t Dp, int64_t n_iv, int64_t Lp, int nb, int nk) {
  const bool rope = a.freqs != nullptr;
  const int64_t L = a.L;
  const int64_t rd_iv0 = a.rho_in ? 0 : 1;
  // Gram and readout tiles run in 8-wave workgroups (snap_wide.hip, one per
  // CU); an interval's readout tiles join its gram group (same N range, same
  // XCD, dispatched together): they read the same q rows.  N splits: 1 or 2,
  // whichever gives the fewer steps in rounds of units over the CUs, 1 on a
  // tie (every split writes, and the context kernel re-reads, one more set
  // of partials).  Measured at C4: chunk 1024 (a tie) 0.83 ms with 1 split,
  // 0.88 with 2; chunk 512 0.875 with 2, 0.889 with 1; 4 splits (the fewest
  // rounds at 512 and 1024) made the context kernel read twice as much
  // (chunk 512: 157 against 58 us) and the call 0.93-0.98 ms; 3 splits at
  // chunk 512 (4 rounds of 86 steps against 3 of 128) took the gram/readout
  // and carry launches 0.614 -> 0.602 ms but the call 0.745 -> 0.777 ms.
  const int ndb256 = (int)cdiv(a.D, T256);
  const int rd_pg = nb * ndb256;
  const int64_t slots = device_cus();
  const int64_t upg = (int64_t)nb * (nb - 1) / 2 + nb + rd_pg;
  auto rounds = [&](int k) { return (S * n_iv * k * upg + slots - 1) / slots * (nk / k); };
  const int ks = (nk % 2 == 0 && rounds(2) < rounds(1)) ? 2 : 1;
  const int kr = ks;

  void *vt = nullptr, *part = nullptr, *snap = nullptr, *rdp = nullptr, *q = nullptr;
  bdh_status stt = scratch(st, SLOT_VT, (size_t)(a.B * a.Hv * Dp * Tp) * sizeof(bf16_t), &vt);
  if (stt != BDH_OK) return stt;
  stt = scratch(st, SLOT_SCORES, (size_t)(ks * S * n_iv * Lp * Lp) * sizeof(float), &part);
  if (stt != BDH_OK) return stt;
  stt = scratch(st, SLOT_SNAP, (size_t)(n_iv * S * a.D * a.N) * sizeof(bf16_t), &snap);
  if (stt != BDH_OK) return stt;
  stt = scratch(st, SLOT_READOUT, (size_t)(kr * S * a.T * a.D) * sizeof(float), &rdp);
  if (stt != BDH_OK) return stt;
  if (rope) {
    stt = scratch(st, SLOT_ROTATED, (size_t)(S * a.T * a.N) * sizeof(bf16_t), &q);
    if (stt != BDH_OK) return stt;
  }

  hipLaunchKernelGGL(transpose_v_kernel, dim3(cdiv(Tp, VT_TILE), cdiv(Dp, VT_TILE), (unsigned)(a.B * a.Hv)),
                     dim3(256), 0, st, a.v, (bf16_t*)vt, a.T, a.D, Tp, Dp);
  BDH_HIP_TRY(hipGetLastError());

  CarryArgs c{};
  c.x = a.x;
  c.freqs = a.freqs;
  c.pos0 = a.pos0;
  c.fixed = a.fixed;
  c.H = a.H; c.Hv = a.Hv; c.T = a.T; c.N = a.N; c.D = a.D; c.S = S; c.L = L; c.Tp = Tp; c.Dp = Dp;
  c.vt = (const bf16_t*)vt;
  c.rho_in = a.rho_in;
  c.rho_out = a.rho_out;
  c.snap = (bf16_t*)snap;
  c.q = (bf16_t*)q;
  c.decay = a.decay;
  int kt = ktime_begin(BDH_KERNEL_PREFILL, st);
  BDH_HIP_TRY(launch_prefill_carry(c, st));
  ktime_end(kt, st);

  PrefillArgs p{};
  p.x = rope ? (const bf16_t*)q : a.x;
  p.freqs = nullptr;
  p.pos0 = a.pos0;
  p.fixed = a.fixed;
  p.decay = a.decay;
  p.H = a.H; p.Hv = a.Hv; p.T = a.T; p.N = a.N; p.D = a.D; p.S = S;
  p.part = (float*)part;
  p.L = L; p.Lp = Lp; p.n_iv = n_iv;
  p.ks = ks; p.nb = nb;
  p.gram_groups = (int)(S * ks * n_iv);
  p.rd_pg = rd_pg;
  p.gram_ids = snap_wide_ids(p.gram_groups, nb, p.rd_pg);
  p.vt = (const bf16_t*)vt;
  p.Tp = Tp; p.Dp = Dp;
  p.state_units = 0;
  p.rd_part = (float*)rdp;
  p.rd_kr = kr;
  p.rd_units = 0;
  p.rd_snap = (const bf16_t*)snap;
  p.rd_iv0 = rd_iv0;
  p.add_units = 0;
  kt = ktime_begin(BDH_KERNEL_PREFILL, st);
  BDH_HIP_TRY(launch_snap_wide(p, st));
  ktime_end(kt, st);

  CtxArgs cx{(const bf16_t*)vt, (const float*)part, a.ctx, a.H, a.Hv, a.T, a.D, L, Lp, Tp, Dp, S,
             n_iv, 0, (int)n_iv, (int)cdiv(L, CTX_ROWS), (const float*)rdp, kr, rd_iv0};
  BDH_HIP_TRY(launch_ctx(cx, ks, st));
  if (launches) *launches += 4;
  return BDH_OK;
}

// Context only (no state, no carried state), queries already rotated, no
// decay: v^T, the gram tiles, the context kernel.  The tiles run in 4-wave
// workgroups of 128 x 128 blocks a wave (wide_gram.hip) where the shape
// suits them (whole 256-row blocks, an even step count per N range), else in
// 8-wave workgroups (snap_wide.hip, the tiles of the state-carry form without
// readouts).  Measured at C5 (same box): 4-wave tiles 10.97-11.06 ms a
// forward against 11.18-11.22 ms.  N splits:
// the fewest of 1, 2 or 4 with the fewest steps in rounds of units over the
// CUs.  (The layer's attention runs here: the layer rotates q in its GEMM
// epilogue.)
bdh_status run_gram_path(const Bf16Args& a, hipStream_t st, uint64_t* launches, int64_t S, int64_t Tp,
                         int64_t Dp, int64_t Lp, int nb, int nk) {
  const int64_t L = a.L;
  const int64_t slots = device_cus();
  const int64_t upg = (int64_t)nb * (nb - 1) / 2 + nb;
  auto rounds = [&](int k) { return (S * k * upg + slots - 1) / slots * (nk / k); };
  int ks = 1;
  for (int cand = 2; cand <= 4 && nk % (2 * cand) == 0; cand *= 2)
    if (rounds(cand) < rounds(ks)) ks = cand;

  void *vt = nullptr, *part = nullptr;
  bdh_status stt = scratch(st, SLOT_VT, (size_t)(a.B * a.Hv * Dp * Tp) * sizeof(bf16_t), &vt);
  if (stt != BDH_OK) return stt;
  const size_t pbytes = a.part16 ? sizeof(bf16_t) : sizeof(float);
  stt = scratch(st, SLOT_SCORES, (size_t)(ks * S * Lp * Lp) * pbytes, &part);
  if (stt != BDH_OK) return stt;

  hipLaunchKernelGGL(transpose_v_kernel, dim3(cdiv(Tp, VT_TILE), cdiv(Dp, VT_TILE), (unsigned)(a.B * a.Hv)),
                     dim3(256), 0, st, a.v, (bf16_t*)vt, a.T, a.D, Tp, Dp);
  BDH_HIP_TRY(hipGetLastError());

  PrefillArgs p{};
  p.part16 = a.part16 ? 1 : 0;
  p.x = a.x;
  p.H = a.H; p.Hv = a.Hv; p.T = a.T; p.N = a.N; p.D = a.D; p.S = S;
  p.part = (float*)part;
  p.L = L; p.Lp = Lp; p.n_iv = 1;
  p.ks = ks; p.nb = nb;
  p.gram_groups = (int)(S * ks);
  p.rd_pg = 0;
  p.gram_ids = snap_wide_ids(p.gram_groups, nb, 0);
  p.vt = (const bf16_t*)vt;
  p.Tp = Tp; p.Dp = Dp;
  const bool wide = wide_gram_fits(p);
  if (wide) p.gram_ids = wide_gram_ids(p.gram_groups, nb);
  const int kt = ktime_begin(BDH_KERNEL_PREFILL, st);
  BDH_HIP_TRY(wide ? launch_wide_gram(p, st) : launch_snap_wide(p, st));
  ktime_end(kt, st);

  const int64_t Lc0 = a.T < L ? a.T : L;
  CtxArgs cx{(const bf16_t*)vt, (const float*)part, a.ctx, a.H, a.Hv, a.T, a.D, L, Lp, Tp, Dp, S,
             1, 0, 1, (int)cdiv(Lc0, CTX_ROWS), nullptr, 0, 0, p.part16};
  BDH_HIP_TRY(launch_ctx(cx, ks, st));
  if (launches) *launches += 3;
  return BDH_OK;
}

// The wave-role launch is parity-green but no faster at C2, so it is off
// unless BDH_PREFILL_ROLES=1 is set in the environment (read at each call):
// with two N splits it takes 270 us against 270-274 us for the 4-wave launch
// on the same box (four splits: 279-283 us).  One workgroup per CU gives up
// what two 4-wave workgroups per CU have, a gram unit's rotation overlapping
// a state unit's memory stream on the same CU; and the one producer wave per
// SIMD needs ~2400 cycles (37 VALU instructions a row group) to rotate an
// off-diagonal tile's step, which the MFMA waves multiply in ~1050.
bool roles_prefill_enabled() {
  const char* e = getenv("BDH_PREFILL_ROLES");
  return e != nullptr && e[0] == '1';
}

// One interval with RoPE, no decay and no carried state, T a multiple of
// 256: the wave-role launch of gram and state units (roles_prefill.hip),
// then the context kernel.  N splits: the fewest for which an off-diagonal
// gram unit stays within the launch's work per CU, counted in producer
// steps (off-diagonal gram 1.5, diagonal 1, state 1.1 plus 4 for its rho
// write), with at least 16 steps per range (C2: 2, measured against 4 and
// 8).  Returns BDH_UNSUPPORTED (nothing launched) where the launch does not
// apply.
bdh_status run_roles_path(const Bf16Args& a, hipStream_t st, uint64_t* launches, int64_t S, int64_t Tp,
                          int64_t Dp, int64_t Lp, int nb, int nk) {
  const int st_units = a.state ? prefill_roles_state_units(S, a.N, Dp) : 0;
  const double gram = (double)S * nk * (nb * (nb - 1) / 2 * 1.5 + nb);
  const double stw = (double)st_units * ((double)(a.T / 32) * 1.1 + 4.0);
  const double per = (gram + stw) / (double)device_cus();
  const double heavy = nb > 1 ? 1.5 : 1.0;
  int ks = 1;
  for (int cand = 1; cand <= 8 && nk % (2 * cand) == 0 && (cand == 1 || nk / cand >= 16); cand *= 2) {
    ks = cand;
    if (heavy * nk / cand <= per) break;
  }
  PrefillArgs p{};
  p.x = a.x;
  p.freqs = a.freqs;
  p.pos0 = a.pos0;
  p.fixed = a.fixed;
  p.H = a.H; p.Hv = a.Hv; p.T = a.T; p.N = a.N; p.D = a.D; p.S = S;
  p.L = a.L; p.Lp = Lp; p.n_iv = 1;
  p.ks = ks; p.nb = nb;
  p.gram_groups = (int)(S * ks);
  p.gram_ids = prefill_roles_gram_ids(p.gram_groups, nb);
  p.Tp = Tp; p.Dp = Dp;
  p.rho_out = a.rho_out;
  p.st_t0 = 0; p.st_Lc = a.T;
  p.state_units = st_units;
  p.rho_stream = 1;
  if (!prefill_roles_fits(p)) return BDH_UNSUPPORTED;

  void *vt = nullptr, *part = nullptr;
  bdh_status stt = scratch(st, SLOT_VT, (size_t)(a.B * a.Hv * Dp * Tp) * sizeof(bf16_t), &vt);
  if (stt != BDH_OK) return stt;
  stt = scratch(st, SLOT_SCORES, (size_t)(ks * S * Lp * Lp) * sizeof(float), &part);
  if (stt != BDH_OK) return stt;
  p.vt = (const bf16_t*)vt;
  p.part = (float*)part;
  hipLaunchKernelGGL(transpose_v_kernel, dim3(cdiv(Tp, VT_TILE), cdiv(Dp, VT_TILE), (unsigned)(a.B * a.Hv)),
                     dim3(256), 0, st, a.v, (bf16_t*)vt, a.T, a.D, Tp, Dp);
  BDH_HIP_TRY(hipGetLastError());
  const int kt = ktime_begin(BDH_KERNEL_PREFILL, st);
  BDH_HIP_TRY(launch_prefill_roles(p, st));
  ktime_end(kt, st);
  CtxArgs c{(const bf16_t*)vt, (const float*)part, a.ctx, a.H, a.Hv, a.T, a.D, a.L, Lp, Tp, Dp, S,
            1, 0, 1, (int)cdiv(a.T, CTX_ROWS), nullptr, 0, 0};
  BDH_HIP_TRY(launch_ctx(c, ks, st));
  if (launches) *launches += 3;
  return BDH_OK;
}
}  // namespace

bdh_status run_bf16_path(const Bf16Args& a, hipStream_t st, uint64_t* launches) {
  // The MFMA kernels address one stream's x, its RoPE table rows and one
  // v^T slab with 32-bit byte offsets.
  if (a.T * a.N * 2 >= (int64_t)1 << 31 || a.D * (a.T + 64) * 2 >= (int64_t)1 << 31)
    return fail(BDH_UNSUPPORTED, "bf16 MFMA path needs time * latent < 2^30 per stream");
  const int64_t S = a.B * a.H;
  // v^T: tokens padded to a multiple of 128 (a state unit's steps cover its
  // interval rounded up to 128 tokens), columns to a multiple of 256 (whole
  // 256-row tiles).
  const int64_t Tp = ((a.T + 127) / 128) * 128;
  const int64_t Dp = ((a.D + T256 - 1) / T256) * T256;
  const int64_t L = a.L;
  const int64_t n_iv = (a.T + L - 1) / L;
  const int64_t Lc0 = a.T < L ? a.T : L;
  const int64_t Lp = ((Lc0 + T256 - 1) / T256) * T256;
  const int nb = (int)(Lp / T256);
  const int nk = (int)(a.N / 32);  // 32-deep gram steps
  const int state_units = prefill_state_units(S, a.N, a.D);
  // (The readout units address a snapshot's rows with 32-bit offsets.)
  if (a.state && n_iv >= 2 && a.D * a.N * 2 < ((int64_t)1 << 31) &&
      (size_t)(n_iv * S * a.N * a.D) * sizeof(bf16_t) <= kCarrySnapMax)
    return run_carry_path(a, st, launches, S, Tp, Dp, n_iv, Lp, nb, nk);
  if (!a.state && a.rho_in == nullptr && a.freqs == nullptr && a.decay == nullptr && n_iv == 1)
    return run_gram_path(a, st, launches, S, Tp, Dp, Lp, nb, nk);
  if (n_iv == 1 && a.freqs != nullptr && a.decay == nullptr && a.rho_in == nullptr && a.T % T256 == 0 &&
      roles_prefill_enabled()) {
    const bdh_status r = run_roles_path(a, st, launches, S, Tp, Dp, Lp, nb, nk);
    if (r != BDH_UNSUPPORTED) return r;
  }

  // N splits of the gram: the fewest for which the longest gram unit stays
  // within ~85% of the first launch's average work per workgroup slot (two
  // per CU; every split writes, and the context kernel re-reads, one more
  // partial score buffer).  Work is counted in 32-deep steps of one 256x128
  // tile; a state unit costs its token steps plus ~4 for its rho write.
  const double gram_work = (double)S * n_iv * nb * (nb + 1) * nk;
  const double state_work = a.state ? state_units * (((Lc0 + 63) / 64) * 2 + 4.0) : 0.0;
  const double per_slot = (gram_work + state_work) / (2.0 * device_cus());
  // Every N range must be an even number of steps (nk is a multiple of 8, so
  // ks = 1, 2 and 4 always qualify).
  int ks = 1;
  for (int cand = 1; cand <= 8 && nk % (2 * cand) == 0; cand *= 2) {
    ks = cand;
    if ((double)nk / cand <= 0.85 * per_slot) break;
  }

  // Readout splits: the fewest for which one readout unit stays within the
  // average work per workgroup slot of its launch (readout + state units).
  const bool carried = a.rho_in != nullptr || n_iv > 1;
  int rd_kr = 1;
  if (carried) {
    const double rd1 = (double)prefill_readout_units(S, L, a.D, 1) * nk;
    const double st = a.state ? state_units * (((L + 63) / 64) * 2 + 4.0) : 0.0;
    const double slot = (rd1 + st) / (2.0 * device_cus());
    for (int cand = 1; cand <= 16 && nk % (2 * cand) == 0; cand *= 2) {
      rd_kr = cand;
      if ((double)nk / cand <= 1.25 * slot) break;
    }
  }

  void *vt = nullptr, *part = nullptr, *rdp = nullptr, *rho_a = nullptr, *rho_b = nullptr;
  bdh_status stt = scratch(st, SLOT_VT, (size_t)(a.B * a.Hv * Dp * Tp) * sizeof(bf16_t), &vt);
  if (stt != BDH_OK) return stt;
  stt = scratch(st, SLOT_SCORES, (size_t)(ks * S * n_iv * Lp * Lp) * sizeof(float), &part);
  if (stt != BDH_OK) return stt;
  // With two or more intervals every launch would re-rotate its x tiles;
  // rotating x once (one read and one write of x) lets every launch run the
  // rotation-free units instead.
  const bool prerot = a.freqs != nullptr && a.state && n_iv >= BDH_PREROT_MIN_IV;
  void* xr = nullptr;
  if (prerot) {
    stt = scratch(st, SLOT_ROTATED, (size_t)(S * a.T * a.N) * sizeof(bf16_t), &xr);
    if (stt != BDH_OK) return stt;
  }
  if (carried) {
    // Two buffers: interval iv's partials go to buffer iv % 2, and their add
    // runs in the next launch, beside that launch's own readout units.
    stt = scratch(st, SLOT_READOUT, (size_t)(2 * rd_kr * S * Lp * a.D) * sizeof(float), &rdp);
    if (stt != BDH_OK) return stt;
  }
  if (a.state && n_iv > 1) {
    stt = scratch(st, SLOT_RHO_A, (size_t)(S * a.N * a.D) * sizeof(float), &rho_a);
    if (stt != BDH_OK) return stt;
    if (n_iv > 2) {
      stt = scratch(st, SLOT_RHO_B, (size_t)(S * a.N * a.D) * sizeof(float), &rho_b);
      if (stt != BDH_OK) return stt;
    }
  }
  const bool rope = a.freqs != nullptr && !prerot;

  uint64_t n_launch = 1;
  hipLaunchKernelGGL(transpose_v_kernel, dim3(cdiv(Tp, VT_TILE), cdiv(Dp, VT_TILE), (unsigned)(a.B * a.Hv)),
                     dim3(256), 0, st, a.v, (bf16_t*)vt, a.T, a.D, Tp, Dp);
  BDH_HIP_TRY(hipGetLastError());
  if (prerot) {
    // Launches of at most 2^22 workgroups (2^30 work-items) each.
    const int64_t segs = cdiv(a.N, ROT_SEG);
    const int64_t rows_per = (((int64_t)1 << 22) / segs) * ROT_ROWS;
    for (int64_t r0 = 0; r0 < S * a.T; r0 += rows_per) {
      const int64_t rows = S * a.T - r0 < rows_per ? S * a.T - r0 : rows_per;
      hipLaunchKernelGGL(rope_rotate_bf16_kernel, dim3((unsigned)(cdiv(rows, ROT_ROWS) * segs)), dim3(256),
                         0, st, a.x, a.freqs, (bf16_t*)xr, r0, r0 + rows, segs, a.T, a.N, a.pos0, a.fixed);
      BDH_HIP_TRY(hipGetLastError());
      ++n_launch;
    }
  }

  PrefillArgs p{};
  p.x = prerot ? (const bf16_t*)xr : a.x;
  p.freqs = rope ? a.freqs : nullptr;
  p.pos0 = a.pos0;
  p.fixed = a.fixed;
  p.decay = a.decay;
  p.H = a.H; p.Hv = a.Hv; p.T = a.T; p.N = a.N; p.D = a.D; p.S = S;
  p.part = (float*)part;
  p.L = L; p.Lp = Lp; p.n_iv = n_iv;
  p.ks = ks; p.nb = nb;
  p.gram_groups = (int)(S * ks * n_iv);
  p.vt = (const bf16_t*)vt;
  p.Tp = Tp; p.Dp = Dp;
  p.rd_part = (float*)rdp;
  p.rd_kr = rd_kr;
  p.add_units = 0;

  // rho_iv for iv = 0 .. n_iv: rho_in, then the scratch buffers A, B, A, ...,
  // and rho_out for the last.  The readout and state units of interval iv
  // both read rho_iv; the state units write rho_{iv+1}, a different buffer
  // except for a single in-place interval, where they run after the readout.
  // The readout add of interval iv runs as add units in the tail of launch
  // iv + 1 (slots freed by its finished units); the last interval's add is
  // a kernel of its own.
  const int64_t rd_buf = rd_kr * S * Lp * a.D;
  int64_t pend_t0 = -1, pend_Lc = 0;
  int pend_buf = 0;
  p.add_ctx = a.ctx;
  const float* cur = a.rho_in;
  for (int64_t iv = 0; iv < n_iv; ++iv) {
    const int buf = (int)(iv & 1);
    p.rd_part = (float*)rdp + buf * rd_buf;
    p.add_units = 0;
    if (pend_t0 >= 0) {
      p.add_src = (const float*)rdp + pend_buf * rd_buf;
      p.add_t0 = pend_t0;
      p.add_Lc = pend_Lc;
      const int64_t f4 = S * pend_Lc * (a.D / 4);
      p.add_units = (int)cdiv(f4, 256);  // one float4 of context per thread
      pend_t0 = -1;
    }
    const int64_t t0 = iv * L;
    const int64_t Lc = (a.T - t0 < L) ? a.T - t0 : L;
    float* next = iv == n_iv - 1 ? a.rho_out : (float*)(iv % 2 == 0 ? rho_a : rho_b);
    const bool in_place = cur != nullptr && (const float*)next == cur;
    p.gram_ids = iv == 0 ? prefill_gram_ids(p.gram_groups, nb) : 0;
    p.rd_rho = cur;
    p.rd_t0 = t0;
    p.rd_Lc = Lc;
    p.rd_units = cur ? prefill_readout_units(S, Lc, a.D, rd_kr) : 0;
    p.rho_in = cur;
    p.rho_out = next;
    p.st_t0 = t0;
    p.st_Lc = Lc;
    p.state_units = (a.state && !in_place) ? state_units : 0;
    p.rho_stream = next == a.rho_out;
    int kt = ktime_begin(BDH_KERNEL_PREFILL, st);
    BDH_HIP_TRY(launch_prefill_mfma(p, rope, st));
    ktime_end(kt, st);
    ++n_launch;
    if (a.state && in_place) {
      PrefillArgs q = p;
      q.gram_ids = 0;
      q.rd_units = 0;
      q.add_units = 0;
      q.state_units = state_units;
      kt = ktime_begin(BDH_KERNEL_PREFILL, st);
      BDH_HIP_TRY(launch_prefill_mfma(q, rope, st));
      ktime_end(kt, st);
      ++n_launch;
    }
    if (iv == 0) {
      // tril(S) V of every interval: the gram partials are all written by
      // the first launch.
      CtxArgs c{(const bf16_t*)vt, (const float*)part, a.ctx, a.H, a.Hv, a.T, a.D, L, Lp, Tp, Dp, S,
                n_iv, 0, (int)(a.state ? n_iv : 1), (int)cdiv(Lc0, CTX_ROWS), nullptr, 0, 0};
      BDH_HIP_TRY(launch_ctx(c, ks, st));
      ++n_launch;
    }
    if (cur) {
      if (a.state && iv + 1 < n_iv) {
        pend_t0 = t0;
        pend_Lc = Lc;
        pend_buf = buf;
      } else {
        hipLaunchKernelGGL(readout_add_kernel, dim3(cdiv(S * Lc * (a.D / 4), 256)), dim3(256), 0, st,
                           (const float*)p.rd_part, a.ctx, S, a.T, a.D, t0, Lc, Lp, rd_kr);
        BDH_HIP_TRY(hipGetLastError());
        ++n_launch;
      }
    }
    if (!a.state) break;  // dense mode: one interval, no state
    cur = next;
  }
  if (launches) *launches += n_launch;
  return BDH_OK;
}

}  // namespace bdh
