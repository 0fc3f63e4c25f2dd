// State-carry kernel of the multi-interval bf16 prefill (gfx950 MFMA).
//
// With two or more state-carry intervals the state at each interval start,
// rho_iv = rho_in + sum_{iv' < iv} Q_iv'^T V_iv', is what the readouts of
// interval iv need.  Without decay the update of a (stream, 128-neuron,
// 256-column) block of rho depends only on that block, so one workgroup owns
// the block and walks every token of the call with it in its accumulators:
//   - per 32-token step it loads x (and rotates it: q = RoPE(x), each x
//     element read and rotated once per call), writes q for the gram and
//     readout units of the next launch (first column block only), stages
//     q^T and v^T in LDS and accumulates q^T v with v_mfma_f32_16x16x32_bf16;
//   - at each interval boundary it writes its block of rho_iv as bf16,
//     transposed ([d][n]: the operand layout of the readout units);
//   - at the end it writes the final rho in f32.
// The readouts of every interval and the gram tiles then run in one launch
// (prefill_mfma_kernel), with no chain of per-interval launches and no f32
// state round trips between intervals.
//
// Loads run P steps ahead in registers (one workgroup per CU when the call
// has few streams, so the loads, not a second workgroup, hide the latency);
// LDS double-buffers one step's q^T and v^T.
#include "bdh_mfma.h"

namespace bdh {
namespace {

using namespace mfma;

constexpr int CARRY_N = T256 / 2;  // neurons per block
constexpr int CARRY_P = 4;         // steps of loads in flight

template <bool ROPE, bool QOUT>
__device__ __forceinline__ void carry_unit(const CarryArgs& a, bf16_t* lds, int64_t s, int64_t n0,
                                           int64_t d0) {
  const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
  const int wm = w >> 1, wn = w & 1;  // n rows 64 wm .., d columns 128 wn ..
  const int64_t b = s / a.H, h = s - b * a.H;
  const int64_t rowb = a.N * 2;  // bytes per x row
  const char* X = reinterpret_cast<const char*>(a.x + s * a.T * a.N);
  const char* VT = reinterpret_cast<const char*>(a.vt + (b * a.Hv + (a.Hv == 1 ? 0 : h)) * a.Dp * a.Tp);
  bf16_t* Q = QOUT ? a.q + s * a.T * a.N : nullptr;

  // x loader: tokens 2 tp, 2 tp + 1 of the step x neurons n0 + 8 nv .. + 7;
  // tokens past T re-read row T - 1 (their v^T columns are zero).
  const int tp = tid & 15, nv = tid >> 4;
  const uint32_t xcol = (uint32_t)((n0 + 8 * nv) * 2);
  // v^T loader: 4 lanes per 64-byte segment of a row d, rows vb + 64 i (a
  // step's rows are contiguous).
  const int kc = tid & 3, vb = tid >> 2;
  const int64_t vstep = a.Dp * 64;  // bytes of one 32-token step of v^T
  const uint32_t vlane = (uint32_t)(vb * 64 + kc * 16);
  float fq[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (ROPE) load_freq4(a.freqs + n0 + 8 * nv, fq);

  struct Stage {
    uint4 xr[2], vr[4];
  };
  auto load = [&](Stage& st, int kt) {
    const int64_t tb = (int64_t)kt * BK;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int64_t t = tb + 2 * tp + i;
      st.xr[i] = ldg16_off(X, (uint32_t)((t < a.T ? t : a.T - 1) * rowb) + xcol);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) st.vr[i] = ldg16_off(VT + (int64_t)kt * vstep + (d0 + 64 * i) * 64, vlane);
  };
  auto store = [&](const Stage& st, int kt, int buf) {
    bf16_t* A = lds + buf * BUF;             // q^T [n][t], 128 rows
    bf16_t* B = lds + buf * BUF + 128 * BK;  // v^T [d][t], 256 rows
    // Tokens past T hold row T - 1 (see load) and are rotated at its
    // position, so their q is row T - 1's and is stored there again (the
    // same bytes): every step issues the same memory operations, and the
    // compiler's waits for a stage loaded CARRY_P steps ago stay exact.
    const int64_t t = (int64_t)kt * BK + 2 * tp;
    const int64_t ta = t < a.T ? t : a.T - 1, tb = t + 1 < a.T ? t + 1 : a.T - 1;
    uint4 q0 = st.xr[0], q1 = st.xr[1];
    if (ROPE) {
      // Sums of integers below 2^24 are exact in f32.
      const float pa = (float)(a.fixed ? a.pos0 : a.pos0 + ta);
      const float pb = (float)(a.fixed ? a.pos0 : a.pos0 + tb);
      q0 = rot8_bf16(q0, rope_cs4(pa, fq));
      q1 = rot8_bf16(q1, rope_cs4(pb, fq));
    }
    if (QOUT) {
      // Read by the next launch after ~1 GB of other traffic: streaming stores.
      __builtin_nontemporal_store(u32x4{q0.x, q0.y, q0.z, q0.w},
                                  reinterpret_cast<u32x4*>(Q + ta * a.N + n0 + 8 * nv));
      __builtin_nontemporal_store(u32x4{q1.x, q1.y, q1.z, q1.w},
                                  reinterpret_cast<u32x4*>(Q + tb * a.N + n0 + 8 * nv));
    }
    // q^T: word (neuron e, tokens 2 tp, 2 tp + 1) from the two tokens' words.
    const uint32_t u0[4] = {q0.x, q0.y, q0.z, q0.w}, u1[4] = {q1.x, q1.y, q1.z, q1.w};
    uint32_t* Aw = reinterpret_cast<uint32_t*>(A);
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      Aw[(lds_off(8 * nv + 2 * p, tp >> 2) + 2 * (tp & 3)) >> 1] = (u0[p] & 0xffffu) | (u1[p] << 16);
      Aw[(lds_off(8 * nv + 2 * p + 1, tp >> 2) + 2 * (tp & 3)) >> 1] = (u0[p] >> 16) | (u1[p] & 0xffff0000u);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) *reinterpret_cast<uint4*>(&B[lds_off(vb + 64 * i, kc)]) = st.vr[i];
  };

  const bool active = d0 + 128 * wn < a.D;
  floatx4 acc[4][8];
  // Accumulator element (mi, ni, r): n = n0 + 64 wm + 16 mi + 4 (lane >> 4) + r,
  // d = d0 + 128 wn + 16 ni + (lane & 15).
  const int64_t nl = n0 + 64 * wm + 4 * (lane >> 4);
  const int64_t dl = d0 + 128 * wn + (lane & 15);
  if (a.rho_in && active) {
    const float* R = a.rho_in + s * a.N * a.D;
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
      for (int ni = 0; ni < 8; ++ni)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int64_t d = dl + 16 * ni;
          acc[mi][ni][r] = d < a.D ? R[(nl + 16 * mi + r) * a.D + d] : 0.0f;
        }
  } else {
    zero_acc(acc);
  }
  // rho_iv of this block as bf16 into snap[iv] ([d][n]): each lane holds 4
  // consecutive neurons of one column, one 8-byte store per 16 x 16 block.
  auto snapshot = [&](int64_t iv) {
    if (!active) return;
    bf16_t* S0 = a.snap + (iv * a.S + s) * a.D * a.N;
#pragma unroll
    for (int ni = 0; ni < 8; ++ni)
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) {  // the 4 stores of a column's 128 bytes in a row
        const int64_t d = dl + 16 * ni;
        if (d < a.D)
          *reinterpret_cast<uint2*>(S0 + d * a.N + nl + 16 * mi) =
              make_uint2(pack_bf16x2(acc[mi][ni][0], acc[mi][ni][1]),
                         pack_bf16x2(acc[mi][ni][2], acc[mi][ni][3]));
      }
  };

  const int nk = (int)(a.Tp / BK);  // a multiple of 4 (Tp: T rounded up to 128)
  const int spi = (int)(a.L / BK);  // steps per interval, a multiple of 4
  Stage st[CARRY_P];
#pragma unroll
  for (int j = 0; j < CARRY_P; ++j) load(st[j], j);  // nk >= 4
  if (a.rho_in) snapshot(0);
  for (int kt = 0; kt < nk; kt += CARRY_P) {
#pragma unroll
    for (int j = 0; j < CARRY_P; ++j) {
      const int k = kt + j;
      store(st[j], k, k & 1);
      // Also orders this buffer's writes after every wave's MFMA reads of
      // step k - 2 (which finished before the previous step's barrier).
      __syncthreads();
      // Past the end the last step is loaded again (unused): no branch, so
      // the wait for each stage covers only its own loads.
      load(st[j], k + CARRY_P < nk ? k + CARRY_P : nk - 1);
      if (active) mma_64x128(lds + (k & 1) * BUF, lds + (k & 1) * BUF + 128 * BK, lane, 64 * wm, 128 * wn, acc);
    }
    // Interval boundaries fall on multiples of spi steps (CARRY_P divides spi).
    if ((kt + CARRY_P) % spi == 0 && kt + CARRY_P < nk) snapshot((kt + CARRY_P) / spi);
  }
  __syncthreads();  // the epilogue reuses the LDS buffers

  epilogue_64x128(acc, lds, w, lane, [&](int row, int col, float4 v) {
    const int64_t n = n0 + 64 * wm + row, d = d0 + 128 * wn + col;
    if (d >= a.D) return;
    __builtin_nontemporal_store(floatx4{v.x, v.y, v.z, v.w},
                                reinterpret_cast<floatx4*>(&a.rho_out[(s * a.N + n) * a.D + d]));
  });
}

template <bool ROPE>
__global__ __launch_bounds__(NT, 1) void prefill_carry_kernel(CarryArgs a) {
  __shared__ __attribute__((aligned(16))) bf16_t lds[2 * BUF];
  const int nt = (int)(a.N / CARRY_N);
  const int dt = (int)(a.Dp / T256);
  const int units = (int)(a.S * nt * dt);
  // Units of one stream share its v^T: when the count allows, give each XCD
  // (workgroup id i runs on XCD i % 8) a contiguous range of units, so a
  // stream's v^T is fetched into few L2s.
  int u = blockIdx.x;
  if (units % 8 == 0) u = (u % 8) * (units / 8) + u / 8;
  const int64_t s = u / (nt * dt);
  const int rem = u - (int)s * nt * dt;
  const int64_t n0 = (int64_t)(rem / dt) * CARRY_N, d0 = (int64_t)(rem % dt) * T256;
  if (ROPE && d0 == 0) carry_unit<ROPE, true>(a, lds, s, n0, d0);
  else carry_unit<ROPE, false>(a, lds, s, n0, d0);
}

}  // namespace

int prefill_carry_units(int64_t S, int64_t N, int64_t Dp) { return (int)(S * (N / CARRY_N) * (Dp / T256)); }

hipError_t launch_prefill_carry(const CarryArgs& a, hipStream_t st) {
  const unsigned grid = (unsigned)prefill_carry_units(a.S, a.N, a.Dp);
  if (a.freqs) hipLaunchKernelGGL((prefill_carry_kernel<true>), dim3(grid), dim3(NT), 0, st, a);
  else hipLaunchKernelGGL((prefill_carry_kernel<false>), dim3(grid), dim3(NT), 0, st, a);
  return hipGetLastError();
}

}  // namespace bdh
