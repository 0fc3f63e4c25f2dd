// Causal score blocks of the bf16 chunked prefill (gfx950 MFMA):
//   part[kp, s, iv][r, c] = (c < r) * d^(r-c) * sum_{n in range kp} q_r[n] q_c[n]
// for the lower-triangular 256x256 tiles of every state-carry interval iv,
// with q = RoPE(x) applied to each tile on its way from HBM to LDS.
// One workgroup = one (tile, N-range kp, stream): 8 waves, each accumulating
// a 64x128 block with v_mfma_f32_32x32x16_bf16; 32-wide k steps staged in
// double-buffered LDS.  Diagonal tiles load one operand (A == B) and their
// two waves that lie wholly above the diagonal skip the MFMAs.  The KS
// partials are summed by the context kernel in a fixed order.
#include "bdh_bf16.h"

namespace bdh {
namespace {

constexpr int NT = T256_THREADS;
constexpr int BK = T256_BK;
constexpr int LDP = T256_LDP;
constexpr int VPT = T256 * (BK / 8) / NT;  // 16-byte vectors per thread per operand

struct TileCtx {
  const bf16_t* X;      // interval's first token row
  const uint32_t* CS;   // table row of the interval's first token
  int64_t N, half, Lc, ri, rj;
};

// Straight-line body for one tile; DIAG tiles use A as both operands.
template <bool ROPE, bool DIAG>
__device__ __forceinline__ void gram_tile(const TileCtx& t, int kb, int ke, bf16_t (*As)[T256 * LDP],
                                          bf16_t (*Bs)[T256 * LDP], floatx16 (&acc)[2][4]) {
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int wm = wave >> 1, wn = wave & 1;  // rows 64*wm.., cols 128*wn..
  // Waves wholly above the diagonal (diag tiles) or past the interval end.
  const bool active = (!DIAG || wn * 128 < wm * 64 + 64) && t.ri + wm * 64 < t.Lc &&
                      t.rj + wn * 128 < t.Lc;

  struct Stage {
    uint4 ra[VPT], rb[VPT], ca[VPT], cb[VPT];
  };
  const int kv = tid & 3;
  auto load = [&](Stage& S, int kt) {
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int row = (tid + i * NT) >> 2;
      const int64_t k = (int64_t)kt * BK + kv * 8;
      // Rows past the interval re-read the last valid row: the scores of
      // such rows and columns are never written, so no masking is needed
      // (and none may be: a select here would wait for the load).
      const int64_t ti = t.ri + row;
      const int64_t tic = ti < t.Lc ? ti : t.Lc - 1;
      S.ra[i] = ldg16(t.X + tic * t.N + k);
      if (ROPE) S.ca[i] = ldg16(t.CS + tic * t.half + k / 2);
      if (!DIAG) {
        const int64_t tj = t.rj + row;
        const int64_t tjc = tj < t.Lc ? tj : t.Lc - 1;
        S.rb[i] = ldg16(t.X + tjc * t.N + k);
        if (ROPE) S.cb[i] = ldg16(t.CS + tjc * t.half + k / 2);
      }
    }
  };
  auto store = [&](const Stage& S, int buf) {
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int row = (tid + i * NT) >> 2;
      *reinterpret_cast<uint4*>(&As[buf][row * LDP + kv * 8]) = prep8<ROPE>(S.ra[i], S.ca[i], 1.0f, false);
      if (!DIAG)
        *reinterpret_cast<uint4*>(&Bs[buf][row * LDP + kv * 8]) = prep8<ROPE>(S.rb[i], S.cb[i], 1.0f, false);
    }
  };
  auto compute = [&](int buf) {
    if (active) {
      const bf16_t* Ab = As[buf];
      const bf16_t* Bb = DIAG ? As[buf] : Bs[buf];
#pragma unroll
      for (int kk = 0; kk < BK / 16; ++kk) {
        const int ko = kk * 16 + 8 * (lane >> 5);
        bf16x8 af[2], bfr[4];
#pragma unroll
        for (int mi = 0; mi < 2; ++mi)
          af[mi] = *reinterpret_cast<const bf16x8*>(&Ab[(wm * 64 + mi * 32 + (lane & 31)) * LDP + ko]);
#pragma unroll
        for (int ni = 0; ni < 4; ++ni)
          bfr[ni] = *reinterpret_cast<const bf16x8*>(&Bb[(wn * 128 + ni * 32 + (lane & 31)) * LDP + ko]);
#pragma unroll
        for (int mi = 0; mi < 2; ++mi)
#pragma unroll
          for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = mfma32(af[mi], bfr[ni], acc[mi][ni]);
      }
    }
  };

  // Pipeline: LDS holds step kt (buffer (kt - kb) & 1); the register ring
  // holds steps kt+1 and kt+2 in flight.
  Stage s0, s1;
  load(s0, kb);
  if (kb + 1 < ke) load(s1, kb + 1);
  store(s0, 0);
  __syncthreads();
  for (int kt = kb; kt < ke; kt += 2) {
    if (kt + 2 < ke) load(s0, kt + 2);
    compute(0);
    if (kt + 1 < ke) store(s1, 1);
    __syncthreads();
    if (kt + 1 >= ke) break;
    if (kt + 3 < ke) load(s1, kt + 3);
    compute(1);
    if (kt + 2 < ke) store(s0, 0);
    __syncthreads();
  }
}

// Workgroups are numbered so that the tiles of one (stream, N range) group
// get ids congruent mod 8: the dispatcher sends id i to XCD i % 8, so those
// tiles, which read the same x rows, share one XCD's L2.
template <bool ROPE>
__global__ __launch_bounds__(NT) void gram_kernel(GramArgs a) {
  const int G = a.tiles_per_iv * (int)a.n_iv;  // tiles per (stream, kp) group
  const int lid = blockIdx.x;
  const int rest = lid >> 3;
  const int64_t q = (int64_t)(rest / G) * 8 + (lid & 7);
  if (q >= a.S * a.ks) return;
  const int gt = rest - (rest / G) * G;
  const int iv = gt / a.tiles_per_iv;
  const int tile = gt - iv * a.tiles_per_iv;
  const int kp = (int)(q % a.ks);
  const int64_t s = q / a.ks;
  int bi = 0;
  while ((bi + 1) * (bi + 2) / 2 <= tile) ++bi;
  const int bj = tile - bi * (bi + 1) / 2;
  const int64_t t0 = (int64_t)iv * a.L;
  const int64_t Lc = (a.T - t0 < a.L) ? a.T - t0 : a.L;
  const int64_t ri = (int64_t)bi * T256, rj = (int64_t)bj * T256;
  if (ri >= Lc) return;  // tile beyond a ragged last interval: never read

  __shared__ __attribute__((aligned(16))) bf16_t As[2][T256 * LDP];
  __shared__ __attribute__((aligned(16))) bf16_t Bs[2][T256 * LDP];

  const int64_t half = a.N / 2;
  TileCtx tc{a.x + (s * a.T + t0) * a.N, ROPE ? a.cs + t0 * half : nullptr, a.N, half, Lc, ri, rj};

  floatx16 acc[2][4];
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = zero16();

  const int nk = (int)(a.N / BK);
  const int kb = (int)((int64_t)nk * kp / a.ks), ke = (int)((int64_t)nk * (kp + 1) / a.ks);
  if (kb < ke) {
    if (bi == bj) gram_tile<ROPE, true>(tc, kb, ke, As, Bs, acc);
    else gram_tile<ROPE, false>(tc, kb, ke, As, Bs, acc);
  }

  const int lane = threadIdx.x & 63, wave = wave_id();
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t h = s % a.H;
  float* P = a.part + (((int64_t)kp * a.S + s) * a.n_iv + iv) * a.Lp * a.Lp;
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int ni = 0; ni < 4; ++ni)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t ti = ri + wm * 64 + mi * 32 + acc_row(lane, r);
        const int64_t tj = rj + wn * 128 + ni * 32 + acc_col(lane);
        if (ti < Lc && tj < Lc) {
          const float v = tj < ti ? acc[mi][ni][r] * decay_pow(a.decay, h, (float)(ti - tj)) : 0.0f;
          P[ti * a.Lp + tj] = v;
        }
      }
}

}  // namespace

hipError_t launch_gram(const GramArgs& g, bool rope, hipStream_t st) {
  const int64_t groups = (g.S * g.ks + 7) / 8;
  const dim3 grid((unsigned)(groups * g.tiles_per_iv * g.n_iv * 8));
  if (rope) hipLaunchKernelGGL(gram_kernel<true>, grid, dim3(NT), 0, st, g);
  else hipLaunchKernelGGL(gram_kernel<false>, grid, dim3(NT), 0, st, g);
  return hipGetLastError();
}

}  // namespace bdh
