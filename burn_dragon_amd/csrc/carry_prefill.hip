// State-carry kernel of the multi-interval bf16 prefill (gfx950 MFMA).
//
// With two or more state-carry intervals the state at each interval start,
// rho_iv = rho_in d^(t_iv) + sum_{iv' < iv} (Q_iv' * d^(end - t))^T V_iv'
// (d = 1 without decay), is what the readouts of interval iv need.  The
// update of a (stream, 128-neuron, 256-column) block of rho depends only on
// that block, so one workgroup owns the block and walks every token of the
// call with it in its accumulators:
//   - per 32-token step it loads x (and rotates it: q = RoPE(x), each x
//     element read and rotated once per call), writes q for the gram and
//     readout units of the next launch (first column block only), stages
//     q^T and v^T in LDS and accumulates q^T v with v_mfma_f32_16x16x32_bf16;
//   - at each interval boundary it writes its block of rho_iv as bf16,
//     transposed ([d][n]: the operand layout of the readout units), and with
//     decay scales the block by d^Lc, Lc the new interval's length, while
//     each token's q^T row is weighted by d^(end - t), end the token's
//     interval end (recurrent.rs:415 over an interval; linear.rs:105-197);
//   - at the end it writes the final rho in f32.
// The readouts of every interval and the gram tiles then run in one launch
// (snap_wide_kernel), with no chain of per-interval launches and no f32
// state round trips between intervals.
//
// Roles (512 threads, 8 waves, one workgroup per CU): waves 0..3 own the
// 64 x 128 accumulator blocks, multiply and store q; waves 4..7 fetch x and
// v^T (direct-to-LDS ring) and rotate x.  With one barrier per 32-token
// step, a SIMD's multiplying wave runs its MFMAs while its loading wave does
// the rotation's VALU and LDS work.  The loading waves issue loads only, so
// their waits can count DMAs in flight (loads complete in order; a store
// issued later may complete before them).
#include "bdh_mfma.h"

namespace bdh {
namespace {

using namespace mfma;

constexpr int CARRY_NT = 512;
constexpr int CARRY_N = T256 / 2;  // neurons per block
constexpr int CARRY_R = 5;         // ring stages
// LDS bytes: ring stages of raw x [32 tokens][128 neurons] (8 KiB) + v^T
// [256 columns][32 tokens] (16 KiB), then the double-buffered q^T [128][32].
constexpr int CARRY_STAGE = 24 * 1024;
constexpr int CARRY_XT = CARRY_R * CARRY_STAGE;
constexpr int CARRY_LDS = CARRY_XT + 2 * 8 * 1024;

// Step k (one barrier B_k at its start):
//   loaders   DMA of step k + 4 into the slot of step k - 1, then x of step
//             k + 1 rotated: q^T into buffer (k + 1) & 1 and (with q) q back
//             in place in its slot;
//   multiply  q^T buffer k & 1 x v^T of slot k into the accumulators, then
//             q of step k (rotated during step k - 1) from slot k to HBM.
// B_k needs stage k + 1 landed (its x is rotated during step k) and every
// LDS access of step k - 1 finished: slot k - 1 and q^T buffer (k + 1) & 1
// are rewritten during step k.  A loading wave issues 6 DMAs per step;
// stage k + 1's (step k - 3) are followed by those of steps k - 2 and k - 1,
// so waiting for at most 12 in flight leaves it landed (steps 1 and 2 need
// prologue stages only, all waited for).
constexpr int CARRY_WAIT = 12;

template <int N>
__device__ __forceinline__ void lds_dma_wait_barrier() {
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}
__device__ __forceinline__ void plain_barrier() { asm volatile("s_barrier" ::: "memory"); }

// The loading waves (rw = wave - 4).
template <bool ROPE, bool QOUT, bool DECAY>
__device__ __forceinline__ void carry_loader(const CarryArgs& a, char* lds, int64_t s, int64_t n0, int64_t d0,
                                             int rw, int lane) {
  const int rtid = rw * 64 + lane;
  const int64_t b = s / a.H, h = s - b * a.H;
  const int64_t rowb = a.N * 2;  // bytes per x row
  const char* X = reinterpret_cast<const char*>(a.x + s * a.T * a.N);
  const char* VT = reinterpret_cast<const char*>(a.vt + (b * a.Hv + (a.Hv == 1 ? 0 : h)) * a.Dp * a.Tp) + d0 * 64;
  const int64_t vstep = a.Dp * 64;  // bytes of one 32-token step of v^T
  const int nk = (int)(a.Tp / BK);  // a multiple of 4 (Tp: T rounded up to 128)

  // DMA lanes.  x: 1 KiB blocks of 4 rows x 256 bytes (128 neurons); wave rw
  // fetches blocks rw and rw + 4; LDS chunk c of row r holds global chunk
  // c ^ (r & 15), so that the readers below (16 rows, one chunk column) hit
  // distinct banks.  v^T: 1 KiB blocks of 16 rows x 64 bytes, blocks rw + 4 j;
  // the lane writing slot c of row r fetches chunk c ^ ((r >> 1) & 3), the
  // swizzle of the MFMA operand layout (lds_off).
  int xrow[2];
  uint32_t xcol[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    xrow[j] = 4 * (rw + 4 * j) + (lane >> 4);
    xcol[j] = (uint32_t)((n0 + 8 * ((lane & 15) ^ (xrow[j] & 15))) * 2);
  }
  uint32_t voff[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = 16 * (rw + 4 * j) + (lane >> 2);
    voff[j] = (uint32_t)(r * 64 + (((lane & 3) ^ ((r >> 1) & 3)) * 16));
  }
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_addr(lds));
  auto issue = [&](int kt, int slot) {
    const int64_t tb = (int64_t)kt * BK;
    const uint32_t base = lds0 + (uint32_t)(slot * CARRY_STAGE);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t t = tb + xrow[j];
      dma16(X, (uint32_t)((t < a.T ? t : a.T - 1) * rowb) + xcol[j], base + (uint32_t)((rw + 4 * j) * 1024));
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
      dma16(VT + (int64_t)kt * vstep, voff[j], base + 8192u + (uint32_t)((rw + 4 * j) * 1024));
  };

  // Rotation lanes: tokens 2 tp, 2 tp + 1 of the step x neurons n0 + 8 nv ..
  const int tp = rtid & 15, nv = rtid >> 4;
  float fq[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (ROPE) load_freq4(a.freqs + n0 + 8 * nv, fq);
  // (cos, sin) of the lane's 4 pairs at its two tokens of the step rotated
  // next: from frac(pos f) for step 0 (positions clamped to T - 1 as the
  // rows are), then advanced by e(32 f) a step, one complex multiply a pair
  // instead of a phase, a cosine and a sine (the steps run in order).
  float ca[4], sa[4], cb[4], sb[4], ec[4], es[4];
  if (ROPE) {
    const int64_t ta = 2 * tp < a.T ? 2 * tp : a.T - 1, tb = 2 * tp + 1 < a.T ? 2 * tp + 1 : a.T - 1;
    const float pa = (float)(a.fixed ? a.pos0 : a.pos0 + ta);
    const float pb = (float)(a.fixed ? a.pos0 : a.pos0 + tb);
    const float dstep = a.fixed ? 0.0f : (float)BK;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float fa = rope_frac(pa, fq[j]), fb = rope_frac(pb, fq[j]), fe = rope_frac(dstep, fq[j]);
      ca[j] = __builtin_amdgcn_cosf(fa);
      sa[j] = __builtin_amdgcn_sinf(fa);
      cb[j] = __builtin_amdgcn_cosf(fb);
      sb[j] = __builtin_amdgcn_sinf(fb);
      ec[j] = __builtin_amdgcn_cosf(fe);
      es[j] = __builtin_amdgcn_sinf(fe);
    }
  }
  // q^T of step k (tokens 2 tp, 2 tp + 1 of neuron 8 nv + e) into buffer k & 1.
  const float dk = DECAY ? a.decay[h] : 1.0f;
  const float l2d = DECAY ? decay_log2(dk) : 0.0f;
  // Weight of token t's row of q^T: d^(end - t), end the end of t's
  // interval; tokens past T (zero v^T columns) weigh 0, so no power of d
  // beyond its interval is formed.
  auto weight = [&](int64_t t) -> float {
    if (t >= a.T) return 0.0f;
    const int64_t e = (t / a.L + 1) * a.L;
    return decay_pow_int(dk, l2d, (int)((e < a.T ? e : a.T) - t));
  };
  auto rotate = [&](int kt, int slot) {
    char* R = lds + slot * CARRY_STAGE;
    const int r0 = 2 * tp, r1 = 2 * tp + 1;
    uint4* X0 = reinterpret_cast<uint4*>(R + r0 * 256 + ((nv ^ (r0 & 15)) << 4));
    uint4* X1 = reinterpret_cast<uint4*>(R + r1 * 256 + ((nv ^ (r1 & 15)) << 4));
    const uint4 x0 = *X0, x1 = *X1;
    uint4 q0 = x0, q1 = x1;    // rotated: the rows the gram and readout tiles read
    uint4 c0 = make_uint4(0, 0, 0, 0), c1 = c0;
    const int64_t t = (int64_t)kt * BK + 2 * tp;
    if (ROPE) {
      // Tokens past T hold row T - 1 (see issue) and are rotated at their
      // own positions; their v^T columns are zero, so they add nothing to
      // rho, and their q rows are not stored.
      c0 = make_uint4(pack_bf16x2(ca[0], sa[0]), pack_bf16x2(ca[1], sa[1]), pack_bf16x2(ca[2], sa[2]),
                      pack_bf16x2(ca[3], sa[3]));
      c1 = make_uint4(pack_bf16x2(cb[0], sb[0]), pack_bf16x2(cb[1], sb[1]), pack_bf16x2(cb[2], sb[2]),
                      pack_bf16x2(cb[3], sb[3]));
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float na = ca[j] * ec[j] - sa[j] * es[j], ma = sa[j] * ec[j] + ca[j] * es[j];
        const float nb = cb[j] * ec[j] - sb[j] * es[j], mb = sb[j] * ec[j] + cb[j] * es[j];
        ca[j] = na;
        sa[j] = ma;
        cb[j] = nb;
        sb[j] = mb;
      }
    }
    uint4 u0, u1;  // the q^T source rows: rotated and, with decay, weighted
    if (DECAY) {
      // Weighted from the f32 rotation, rounded once.
      float f0[8], f1[8];
      prep8_f32<ROPE>(x0, c0, 1.0f, false, f0);
      prep8_f32<ROPE>(x1, c1, 1.0f, false, f1);
      if (ROPE) {
        q0 = make_uint4(pack_bf16x2(f0[0], f0[1]), pack_bf16x2(f0[2], f0[3]), pack_bf16x2(f0[4], f0[5]),
                        pack_bf16x2(f0[6], f0[7]));
        q1 = make_uint4(pack_bf16x2(f1[0], f1[1]), pack_bf16x2(f1[2], f1[3]), pack_bf16x2(f1[4], f1[5]),
                        pack_bf16x2(f1[6], f1[7]));
      }
      const float w0 = weight(t), w1 = weight(t + 1);
      u0 = make_uint4(pack_bf16x2(f0[0] * w0, f0[1] * w0), pack_bf16x2(f0[2] * w0, f0[3] * w0),
                      pack_bf16x2(f0[4] * w0, f0[5] * w0), pack_bf16x2(f0[6] * w0, f0[7] * w0));
      u1 = make_uint4(pack_bf16x2(f1[0] * w1, f1[1] * w1), pack_bf16x2(f1[2] * w1, f1[3] * w1),
                      pack_bf16x2(f1[4] * w1, f1[5] * w1), pack_bf16x2(f1[6] * w1, f1[7] * w1));
    } else {
      if (ROPE) {
        q0 = rot8_bf16(x0, c0);
        q1 = rot8_bf16(x1, c1);
      }
      u0 = q0;
      u1 = q1;
    }
    if (QOUT) {  // back in place for the q stores (each thread rewrites only what it read)
      *X0 = q0;
      *X1 = q1;
    }
    // q^T: word (neuron e, tokens 2 tp, 2 tp + 1) from the two tokens' words.
    const uint32_t w0[4] = {u0.x, u0.y, u0.z, u0.w}, w1[4] = {u1.x, u1.y, u1.z, u1.w};
    uint32_t* Aw = reinterpret_cast<uint32_t*>(lds + CARRY_XT + (kt & 1) * 8192);
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      Aw[(lds_off(8 * nv + 2 * p, tp >> 2) + 2 * (tp & 3)) >> 1] = (w0[p] & 0xffffu) | (w1[p] << 16);
      Aw[(lds_off(8 * nv + 2 * p + 1, tp >> 2) + 2 * (tp & 3)) >> 1] = (w0[p] >> 16) | (w1[p] & 0xffff0000u);
    }
  };
  // Every load above has completed before the ring starts (the compiler cannot
  // see the DMAs, so it must not be left waiting for older loads inside it).
  __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
#pragma unroll
  for (int j = 0; j < CARRY_R - 1; ++j) issue(j, j);  // nk >= 4 = CARRY_R - 1
  lds_dma_wait_barrier<0>();                          // prologue stages landed
  rotate(0, 0);
  for (int k = 0; k < nk; ++k) {
    lds_dma_wait_barrier<CARRY_WAIT>();  // B_k
    // Step k + 4 into the slot of step k - 1; past the end the last step is
    // fetched again (unused), so every step issues the same operations.
    issue(k + CARRY_R - 1 < nk ? k + CARRY_R - 1 : nk - 1, (k + CARRY_R - 1) % CARRY_R);
    if (k + 1 < nk) rotate(k + 1, (k + 1) % CARRY_R);
  }
  lds_dma_wait_barrier<0>();  // the epilogue reuses the ring
#pragma unroll
  for (int i = 0; i < 8; ++i) __syncthreads();  // the multiplying waves' epilogue barriers
}

// The multiplying waves (w = 0..3): rows n0 + 64 wm .., columns d0 + 128 wn ..
template <bool QOUT, bool DECAY>
__device__ __forceinline__ void carry_mma(const CarryArgs& a, char* lds, int64_t s, int64_t n0, int64_t d0, int w,
                                          int lane) {
  const int wm = w >> 1, wn = w & 1;
  const int nk = (int)(a.Tp / BK);  // a multiple of 4 (Tp: T rounded up to 128)
  const int spi = (int)(a.L / BK);  // steps per interval
  const bool active = d0 + 128 * wn < a.D;
  floatx4 acc[4][8];
  // Accumulator element (mi, ni, r): n = n0 + 64 wm + 16 mi + 4 (lane >> 4) + r,
  // d = d0 + 128 wn + 16 ni + (lane & 15).
  const int64_t nl = n0 + 64 * wm + 4 * (lane >> 4);
  const int64_t dl = d0 + 128 * wn + (lane & 15);
  if (a.rho_in && active) {
    const float* Rin = a.rho_in + s * a.N * a.D;
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
      for (int ni = 0; ni < 8; ++ni)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int64_t d = dl + 16 * ni;
          acc[mi][ni][r] = d < a.D ? Rin[(nl + 16 * mi + r) * a.D + d] : 0.0f;
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
  // With decay: the carried block times d^Lc at the start of interval iv
  // (Lc its length), the weighted q^T rows of the interval being added after.
  const float dk = DECAY ? a.decay[s % a.H] : 1.0f;
  const float l2d = DECAY ? decay_log2(dk) : 0.0f;
  auto carry_scale = [&](int64_t iv) {
    if (!DECAY) return;
    const int64_t t0 = iv * a.L;
    const float f = decay_pow_int(dk, l2d, (int)(a.T - t0 < a.L ? a.T - t0 : a.L));
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
      for (int ni = 0; ni < 8; ++ni)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[mi][ni][r] *= f;
  };
  if (a.rho_in) {
    snapshot(0);
    carry_scale(0);
  }
  bf16_t* Q = QOUT ? a.q + s * a.T * a.N : nullptr;
  // q rows of step k from its ring slot (rotated in place) to HBM: lane
  // (lane & 15) stores chunk c of rows 4 (w + 4 j) + (lane >> 4), so each
  // store instruction writes 4 whole 256-byte row pieces (the rotation
  // lanes' own layout would write 64-byte pieces, each 128-byte line then
  // completed by another wave later, which costs HBM write bytes).  Rows
  // past T (row T - 1's x rotated at their own positions) are not stored.
  auto store_q = [&](int kt, int slot) {
    const char* R = lds + slot * CARRY_STAGE;
    const int c = lane & 15;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int r = 4 * (w + 4 * j) + (lane >> 4);
      const uint4 v = *reinterpret_cast<const uint4*>(R + r * 256 + ((c ^ (r & 15)) << 4));
      const int64_t t = (int64_t)kt * BK + r;
      // Read by the next launch after ~1 GB of other traffic: streaming stores.
      if (t < a.T)
        __builtin_nontemporal_store(u32x4{v.x, v.y, v.z, v.w}, reinterpret_cast<u32x4*>(Q + t * a.N + n0 + 8 * c));
    }
  };


  plain_barrier();  // the loaders' prologue stages landed
  for (int k = 0; k < nk; ++k) {
    plain_barrier();  // B_k: q^T of step k written, stage k landed
    if (active)
      mma_64x128_dsasm(reinterpret_cast<const bf16_t*>(lds + CARRY_XT + (k & 1) * 8192),
                       reinterpret_cast<const bf16_t*>(lds + (k % CARRY_R) * CARRY_STAGE + 8192), lane, 64 * wm,
                       128 * wn, acc);
    if (QOUT) store_q(k, k % CARRY_R);
    if ((k + 1) % spi == 0 && k + 1 < nk) {
      snapshot((k + 1) / spi);
      carry_scale((k + 1) / spi);
    }
  }
  lds_dma_wait_barrier<0>();  // the epilogue reuses the ring

  epilogue_64x128(acc, reinterpret_cast<bf16_t*>(lds), w, lane, [&](int row, int col, float4 v) {
    const int64_t n = n0 + 64 * wm + row, d = d0 + 128 * wn + col;
    if (d >= a.D) return;
    __builtin_nontemporal_store(floatx4{v.x, v.y, v.z, v.w},
                                reinterpret_cast<floatx4*>(&a.rho_out[(s * a.N + n) * a.D + d]));
  });
}

template <bool ROPE, bool QOUT, bool DECAY>
__device__ __forceinline__ void carry_unit(const CarryArgs& a, char* lds, int64_t s, int64_t n0, int64_t d0) {
  const int lane = threadIdx.x & 63, w = wave_id();
  if (w >= 4) carry_loader<ROPE, QOUT, DECAY>(a, lds, s, n0, d0, w - 4, lane);
  else carry_mma<QOUT, DECAY>(a, lds, s, n0, d0, w, lane);
}

template <bool ROPE, bool DECAY>
__global__ __launch_bounds__(CARRY_NT, 1) void prefill_carry_kernel(CarryArgs a) {
  __shared__ __attribute__((aligned(16))) char lds[CARRY_LDS];
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
  if (ROPE && d0 == 0) carry_unit<ROPE, true, DECAY>(a, lds, s, n0, d0);
  else carry_unit<ROPE, false, DECAY>(a, lds, s, n0, d0);
}

}  // namespace

int prefill_carry_units(int64_t S, int64_t N, int64_t Dp) { return (int)(S * (N / CARRY_N) * (Dp / T256)); }

hipError_t launch_prefill_carry(const CarryArgs& a, hipStream_t st) {
  const unsigned grid = (unsigned)prefill_carry_units(a.S, a.N, a.Dp);
  if (a.decay) {
    if (a.freqs) hipLaunchKernelGGL((prefill_carry_kernel<true, true>), dim3(grid), dim3(CARRY_NT), 0, st, a);
    else hipLaunchKernelGGL((prefill_carry_kernel<false, true>), dim3(grid), dim3(CARRY_NT), 0, st, a);
  } else {
    if (a.freqs) hipLaunchKernelGGL((prefill_carry_kernel<true, false>), dim3(grid), dim3(CARRY_NT), 0, st, a);
    else hipLaunchKernelGGL((prefill_carry_kernel<false, false>), dim3(grid), dim3(CARRY_NT), 0, st, a);
  }
  return hipGetLastError();
}

}  // namespace bdh
