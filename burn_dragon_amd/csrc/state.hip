// State update of the bf16 chunked prefill (gfx950 MFMA), one interval:
//   rho_out[n, d] = rho_in[n, d] * d^L + sum_t q_t[n] * d^(L-t) * v_t[d]
// with q = RoPE(x) applied on the way from HBM to LDS.  One workgroup owns a
// 256 (n) x 256 (d) tile of rho and runs over the interval's tokens in
// 32-token steps: 8 waves, each accumulating a 64x128 block with
// v_mfma_f32_32x32x16_bf16.  The contraction runs over tokens, which are the
// slow index of both x and v: v comes pre-transposed ([d][t]), and the
// rotated x tile is written transposed into LDS ([n][t], 16-byte groups XOR
// swizzled so that fragment reads are conflict-free).
// Global loads run two steps ahead of the MFMAs through a two-slot register
// ring (LDS double buffer + 2 staged steps), so a step's HBM latency is
// covered by the two steps computed before it is needed.
#include "bdh_bf16.h"

namespace bdh {
namespace {

constexpr int NT = T256_THREADS;
constexpr int BK = T256_BK;
constexpr int LDP = T256_LDP;
constexpr int VB = T256 * (BK / 8) / NT;   // v vectors per thread per step
// Each thread stages a 2-token x 8-neuron block of x per step (one token
// pair, one 16-byte neuron group) and writes it transposed as 8 packed
// bf16x2 (token pair) words.
static_assert((BK / 2) * (T256 / 8) == NT, "one x block per thread per step");

// Physical 8-token group of logical group g (0..3) in row n of the [n][32]
// tile: rows n..n+7 read at distinct 16-byte bank groups.
__device__ __forceinline__ int swz4(int n, int g) { return g ^ ((n >> 1) & 3) ^ ((n >> 3) & 3); }

struct Stage {
  uint4 ra[2], ca[2], rb[VB];
  float wa[2];
};

template <bool ROPE>
__global__ __launch_bounds__(NT) void state_kernel(StateArgs a) {
  const int64_t n0 = (int64_t)blockIdx.x * T256;
  const int64_t d0 = (int64_t)blockIdx.y * T256;
  const int64_t s = blockIdx.z;
  __shared__ __attribute__((aligned(16))) bf16_t As[2][T256 * BK];    // [n][t], swizzled
  __shared__ __attribute__((aligned(16))) bf16_t Bs[2][T256 * LDP];   // [d][t]

  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int wm = wave >> 1, wn = wave & 1;  // n rows 64*wm.., d cols 128*wn..
  const int64_t half = a.N / 2;
  const int64_t b = s / a.H, h = s - b * a.H;
  const bf16_t* X = a.x + (s * a.T + a.t0) * a.N;
  const uint32_t* CS = ROPE ? a.cs + a.t0 * half : nullptr;
  const bf16_t* VT = a.vt + (b * a.Hv + (a.Hv == 1 ? 0 : h)) * a.D * a.Tp;
  const float dv = a.decay ? a.decay[h] : 1.0f;
  const bool scale = a.decay != nullptr;
  // v columns past D are zero-filled in LDS, so partially covered waves
  // compute zeros there; waves with no column below D skip the MFMAs.
  const bool active = d0 + wn * 128 < a.D;

  // x block of this thread: tokens 2*tp, 2*tp+1 of the step, neurons 8*nv..
  const int tp = tid & 15, nv = tid >> 4;
  const bool kt_partial = (a.L % BK) != 0;  // last step runs past the interval
  auto load = [&](Stage& S, int kt) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      // Tokens past the interval re-read the last valid row; their weight
      // is 0, applied when the step is written to LDS (a select on the
      // loaded value here would make the load wait).
      const int64_t tl = (int64_t)kt * BK + 2 * tp + i;
      const int64_t tlc = tl < a.L ? tl : a.L - 1;
      const int64_t n = n0 + nv * 8;
      S.ra[i] = ldg16(X + tlc * a.N + n);
      if (ROPE) S.ca[i] = ldg16(CS + tlc * half + n / 2);
      S.wa[i] = tl < a.L ? (scale ? powf(dv, (float)(a.L - tl)) : 1.0f) : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < VB; ++i) {
      // v columns past D re-read the last column: they only feed output
      // columns that are never written.
      const int v = tid + i * NT;
      const int dd = v >> 2, kv = v & 3;
      const int64_t d = d0 + dd;
      const int64_t dc = d < a.D ? d : a.D - 1;
      S.rb[i] = ldg16(VT + dc * a.Tp + a.t0 + (int64_t)kt * BK + kv * 8);
    }
  };
  auto store = [&](const Stage& S, int buf) {
    float v0[8], v1[8];
    const bool masked = scale || kt_partial;
    prep8_f32<ROPE>(S.ra[0], S.ca[0], S.wa[0], masked, v0);
    prep8_f32<ROPE>(S.ra[1], S.ca[1], S.wa[1], masked, v1);
    const int tt = 2 * tp;  // even token of the pair; both share a 16-byte group
    uint32_t* Aw = reinterpret_cast<uint32_t*>(As[buf]);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int n = nv * 8 + e;
      Aw[(n * BK + swz4(n, tt >> 3) * 8 + (tt & 7)) >> 1] = pack_bf16x2(v0[e], v1[e]);
    }
#pragma unroll
    for (int i = 0; i < VB; ++i) {
      const int v = tid + i * NT;
      const int dd = v >> 2, kv = v & 3;
      *reinterpret_cast<uint4*>(&Bs[buf][dd * LDP + kv * 8]) = S.rb[i];
    }
  };

  floatx16 acc[2][4];
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = zero16();

  auto compute = [&](int buf) {
    if (!active) return;
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      const int g = kk * 2 + (lane >> 5);
      bf16x8 af[2], bfr[4];
#pragma unroll
      for (int mi = 0; mi < 2; ++mi) {
        const int n = wm * 64 + mi * 32 + (lane & 31);
        af[mi] = *reinterpret_cast<const bf16x8*>(&As[buf][n * BK + swz4(n, g) * 8]);
      }
#pragma unroll
      for (int ni = 0; ni < 4; ++ni)
        bfr[ni] = *reinterpret_cast<const bf16x8*>(
            &Bs[buf][(wn * 128 + ni * 32 + (lane & 31)) * LDP + kk * 16 + 8 * (lane >> 5)]);
#pragma unroll
      for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = mfma32(af[mi], bfr[ni], acc[mi][ni]);
    }
  };

  // Pipeline: LDS holds step kt (buffer kt & 1); the register ring holds
  // steps kt+1 and kt+2 in flight.
  const int nk = (int)((a.L + BK - 1) / BK);
  Stage s0, s1;
  load(s0, 0);
  if (nk > 1) load(s1, 1);
  store(s0, 0);
  __syncthreads();
  for (int kt = 0; kt < nk; kt += 2) {
    if (kt + 2 < nk) load(s0, kt + 2);
    compute(0);
    if (kt + 1 < nk) store(s1, 1);
    __syncthreads();
    if (kt + 1 >= nk) break;
    if (kt + 3 < nk) load(s1, kt + 3);
    compute(1);
    if (kt + 2 < nk) store(s0, 0);
    __syncthreads();
  }

  const float carry = scale ? powf(dv, (float)a.L) : 1.0f;
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

inline unsigned cdiv(int64_t a, int64_t b) { return (unsigned)((a + b - 1) / b); }

}  // namespace

hipError_t launch_state(const StateArgs& a, bool rope, hipStream_t st) {
  const dim3 grid((unsigned)(a.N / T256), cdiv(a.D, T256), (unsigned)a.S);
  if (rope) hipLaunchKernelGGL(state_kernel<true>, grid, dim3(NT), 0, st, a);
  else hipLaunchKernelGGL(state_kernel<false>, grid, dim3(NT), 0, st, a);
  return hipGetLastError();
}

}  // namespace bdh
