// Gram and readout tiles of the state-carry form (two or more intervals, q
// already rotated) in 512-thread workgroups (8 waves, one per CU).  With
// decay d the epilogues apply the closed form's powers: d^(r - c) to the
// score (r, c) below the diagonal, d^r to readout row r (r, c local to the
// interval: linear.rs:105-197).
//
// Every operand row comes from HBM (or L2) through a four-stage direct-load
// LDS ring, so what bounds these tiles is the operand traffic per MFMA.  A
// wave owns a 64 x 128 block of v_mfma_f32_16x16x32_bf16 accumulators, and
// the workgroup's 4 x 2 waves cover a 256 x 256 tile:
//   diagonal gram tile  rows = columns = 256 tokens of the interval: 256 rows
//                       loaded per step (the 4-wave launch loads 512 for the
//                       same scores: a 256 x 128 tile and a pair of 128 x 128
//                       diagonal blocks);
//   off-diagonal tile   256 + 256 token rows;
//   readout tile        256 token rows (q) + 256 state rows (rho_iv^T from
//                       the bf16 snapshot): all 256 columns of D at once,
//                       where the 4-wave launch loads the q rows once per
//                       128-column block.
// A group (stream, interval, N range) holds its interval's readout tiles,
// then its off-diagonal and diagonal gram tiles; group ids are laid out so
// that a group runs on one XCD (workgroup id i runs on XCD i % 8).
// Outputs are the 4-wave launch's: gram partials [KS, S, n_iv, Lp, Lp] (tril
// masked) and readout partials [KS, S, T, D], reduced by the context kernel.
#include "bdh_mfma.h"

namespace bdh {
namespace {

using namespace mfma;

constexpr int SW_NT = 512;                  // 8 waves
constexpr int SW_STAGE = 2 * T256 * BK;     // bf16 elements of one stage: 512 rows of 32
constexpr int SW_LDS = 4 * SW_STAGE;        // four stages (128 KiB); the epilogue reuses them

enum { K_DIAG = 0, K_OFF = 1, K_READ = 2 };

// Tile of interval iv, N range kp: A = token rows ri .. ri+255 of the
// interval; B = token rows rj .. (K_OFF), the A rows (K_DIAG), or state
// rows d0 .. d0+255 of snap[iv] (K_READ).  Stage rows 0..255 hold A, 256..511
// B.  Wave w fetches 16-row blocks w + 8 j of the stage (j < 2: A, j >= 2:
// B); the lane writing LDS slot c of row r fetches global chunk
// c ^ ((r >> 1) & 3), the swizzle of lds_off.  Token rows past a ragged
// interval (!WHOLE) re-read its last row, state rows past D re-read row
// D - 1; neither is stored.
template <int KIND, bool WHOLE>
__device__ __forceinline__ void snap_wide_unit(const PrefillArgs& a, bf16_t* lds, int64_t s, int kp, int64_t iv,
                                               int64_t ri, int64_t rj) {
  const int lane = threadIdx.x & 63, w = wave_id();
  const int wr = w >> 1, wc = w & 1;  // rows 64 wr .., columns 128 wc .. of the tile
  const int64_t t0 = iv * a.L;
  const int64_t Lc = (a.T - t0 < a.L) ? a.T - t0 : a.L;
  const int64_t rowb = a.N * 2;  // bytes per q row and per snapshot row
  const char* X = reinterpret_cast<const char*>(a.x + (s * a.T + t0) * a.N);
  const char* R = KIND == K_READ ? reinterpret_cast<const char*>(a.rd_snap + (iv * a.S + s) * a.D * a.N) : X;
  const int nk = (int)(a.N / BK);
  const int kb = (int)((int64_t)nk * kp / a.ks), ke = (int)((int64_t)nk * (kp + 1) / a.ks);
  constexpr int NB = KIND == K_DIAG ? 2 : 4;  // 16-row blocks a wave fetches per step
  const uint32_t gc = (uint32_t)((lane & 3) ^ ((lane >> 3) & 3));
  uint32_t voff[NB];
  int64_t vbase[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    const int blk = w + 8 * j;
    const int64_t rr = 16 * (blk & 15);  // first row of the block within its 256
    if (KIND == K_READ && j >= 2) {
      const int64_t d = rj + rr + (lane >> 2);
      vbase[j] = 0;
      voff[j] = (uint32_t)((d < a.D ? d : a.D - 1) * rowb) + gc * 16;
    } else {
      const int64_t r0 = j < 2 ? ri : rj;
      if (WHOLE) {
        vbase[j] = (r0 + rr) * rowb;
        voff[j] = (uint32_t)((lane >> 2) * rowb) + gc * 16;
      } else {
        const int64_t t = r0 + rr + (lane >> 2);
        vbase[j] = 0;
        voff[j] = (uint32_t)((t < Lc ? t : Lc - 1) * rowb) + gc * 16;
      }
    }
  }
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_addr(lds));
  auto issue1 = [&](int kt, int stg, int j) {
    dma16((KIND == K_READ && j >= 2 ? R : X) + vbase[j] + (int64_t)kt * 64, voff[j],
          lds0 + (uint32_t)(stg * SW_STAGE * 2 + (w + 8 * j) * 1024));
  };
  auto issue = [&](int kt, int stg) {
#pragma unroll
    for (int j = 0; j < NB; ++j) issue1(kt, stg, j);
  };

  floatx4 acc[4][8];
  zero_acc(acc);
  const int64_t wr0 = ri + 64 * wr, wc0 = rj + 128 * wc;
  bool active;
  if (KIND == K_DIAG) active = wr0 + 63 > wc0 && wr0 < Lc && wc0 < Lc;
  else if (KIND == K_OFF) active = wr0 < Lc;  // every column lies below every row
  else active = wr0 < Lc && wc0 < a.D;
  const int brow = KIND == K_DIAG ? 128 * wc : T256 + 128 * wc;

  // Ring of 4 stages, step kt in stage (kt - kb) & 3.  At step kt the barrier
  // confirms stage kt + 1 (DMAs issued two steps earlier); each wave then
  // starts the fragment reads of step kt + 1 and multiplies step kt from the
  // fragments it read during step kt - 1, so LDS reads overlap MFMAs.  The
  // DMA of step kt + 3 goes into the stage of step kt - 1, whose fragments
  // every wave waited for (at the top of step kt - 1) before this barrier.
  // Past the end the last step is fetched again (unused), so every step
  // leaves NB DMAs in flight and reads a landed stage.  A multiplying wave
  // issues its NB DMAs between its MFMA groups: issued together after the
  // barrier, the 8 waves' 32 KiB of DMAs queue in the texture address unit
  // and hold every wave's MFMAs back by hundreds of cycles.
  __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): no compiler-visible load left in flight
  auto clampk = [&](int k) { return k < ke ? k : ke - 1; };
  issue(kb, 0);
  issue(clampk(kb + 1), 1);
  issue(clampk(kb + 2), 2);
  dma_wait_barrier<2 * NB>();  // stage kb landed
  u32x4 fa[4], fb[8], ga[4], gb[8];
  // Fragment bases in stage 0 (a stage is SW_STAGE * 2 bytes further on).
  const uint32_t fa0 = frag_64x128_base(lds, lane, 64 * wr), fb0 = frag_64x128_base(lds, lane, brow);
  constexpr uint32_t SB = SW_STAGE * 2;
  if (active) {
    frag_64x128_read<0>(fa0, fb0, fa, fb);
    frag_64x128_read<1>(fa0, fb0, fa, fb);
    frag_64x128_read<2>(fa0, fb0, fa, fb);
    frag_64x128_read<3>(fa0, fb0, fa, fb);
    frag_64x128_read<4>(fa0, fb0, fa, fb);
    frag_64x128_read<5>(fa0, fb0, fa, fb);
    frag_64x128_read<6>(fa0, fb0, fa, fb);
    frag_64x128_read<7>(fa0, fb0, fa, fb);
    frag_64x128_read<8>(fa0, fb0, fa, fb);
    frag_64x128_read<9>(fa0, fb0, fa, fb);
    frag_64x128_read<10>(fa0, fb0, fa, fb);
    frag_64x128_read<11>(fa0, fb0, fa, fb);
  }
  int stg = 0;  // stage of step kt
  constexpr int GPD = 8 / NB;  // MFMA groups per DMA
  for (int kt = kb; kt < ke; kt += 2) {
    dma_wait_barrier<NB>();
    int kn = clampk(kt + 3), sn = (stg + 3) & 3;
    stg = (stg + 1) & 3;
    if (active) {
      frags_64x128_wait(fa, fb);
      const uint32_t na = fa0 + stg * SB, nb = fb0 + stg * SB;
      mma_64x128_frags(fa, fb, acc, [&](auto gc) {
        constexpr int g = decltype(gc)::value;
        if constexpr (g < 6) {
          frag_64x128_read<2 * g>(na, nb, ga, gb);
          frag_64x128_read<2 * g + 1>(na, nb, ga, gb);
        }
        if constexpr (g % GPD == GPD - 1) issue1(kn, sn, g / GPD);
      });
    } else {
      issue(kn, sn);
    }
    if (kt + 1 >= ke) break;
    dma_wait_barrier<NB>();
    kn = clampk(kt + 4);
    sn = (stg + 3) & 3;
    stg = (stg + 1) & 3;
    if (active) {
      frags_64x128_wait(ga, gb);
      const uint32_t na = fa0 + stg * SB, nb = fb0 + stg * SB;
      mma_64x128_frags(ga, gb, acc, [&](auto gc) {
        constexpr int g = decltype(gc)::value;
        if constexpr (g < 6) {
          frag_64x128_read<2 * g>(na, nb, fa, fb);
          frag_64x128_read<2 * g + 1>(na, nb, fa, fb);
        }
        if constexpr (g % GPD == GPD - 1) issue1(kn, sn, g / GPD);
      });
    } else {
      issue(kn, sn);
    }
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the last (unused) fragment reads
  dma_wait_barrier<0>();  // the epilogue reuses the ring

  const float dk = a.decay ? a.decay[s % a.H] : 1.0f;
  const float l2d = a.decay ? decay_log2(dk) : 0.0f;
  if (KIND == K_READ) {
    float* P = a.rd_part + ((int64_t)kp * a.S + s) * a.T * a.D + t0 * a.D;
    epilogue_64x128(acc, lds, w, lane, [&](int row, int col, float4 v) {
      const int64_t t = wr0 + row, d = wc0 + col;
      if (!active || t >= Lc || d >= a.D) return;
      if (a.decay) {
        const float f = decay_pow_int(dk, l2d, (int)t);
        v.x *= f;
        v.y *= f;
        v.z *= f;
        v.w *= f;
      }
      __builtin_nontemporal_store(floatx4{v.x, v.y, v.z, v.w}, reinterpret_cast<floatx4*>(&P[t * a.D + d]));
    });
  } else {
    // Scores of rows ti < Lc and columns tj < Lc, 0 on and above the
    // diagonal (the context kernel reads them up to its row block's end).
    float* P = a.part + (((int64_t)kp * a.S + s) * a.n_iv + iv) * a.Lp * a.Lp;
    epilogue_64x128(acc, lds, w, lane, [&](int row, int col, float4 v) {
      const int64_t ti = wr0 + row, tj = wc0 + col;
      if (!active || ti >= Lc) return;
      float e[4] = {tj < ti ? v.x : 0.0f, tj + 1 < ti ? v.y : 0.0f, tj + 2 < ti ? v.z : 0.0f,
                    tj + 3 < ti ? v.w : 0.0f};
      if (a.decay) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (tj + j < ti) e[j] *= decay_pow_int(dk, l2d, (int)(ti - tj - j));
      }
      if (a.part16) {
        // bf16 partials (RNE): half the bytes written here and read by the
        // context kernel.
        bf16_t* dst = reinterpret_cast<bf16_t*>(a.part) + ((((int64_t)kp * a.S + s) * a.n_iv + iv) * a.Lp + ti) * a.Lp + tj;
        if (tj + 3 < Lc) {
          __builtin_nontemporal_store(u32x2{pack_bf16x2(e[0], e[1]), pack_bf16x2(e[2], e[3])},
                                      reinterpret_cast<u32x2*>(dst));
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (tj + j < Lc) dst[j] = (bf16_t)e[j];
        }
        return;
      }
      float* dst = P + ti * a.Lp + tj;
      if (tj + 3 < Lc) {
        __builtin_nontemporal_store(floatx4{e[0], e[1], e[2], e[3]}, reinterpret_cast<floatx4*>(dst));
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (tj + j < Lc) dst[j] = e[j];
      }
    });
  }
}

template <int KIND>
__device__ __forceinline__ void snap_wide_dispatch(const PrefillArgs& a, bf16_t* lds, int64_t s, int kp,
                                                   int64_t iv, int64_t ri, int64_t rj, bool whole) {
  if (whole) snap_wide_unit<KIND, true>(a, lds, s, kp, iv, ri, rj);
  else snap_wide_unit<KIND, false>(a, lds, s, kp, iv, ri, rj);
}

// Group g = (stream, N range, interval), interval fastest; units of a group:
// rd_pg readout tiles (row block, 256-column block), the nb (nb - 1) / 2
// off-diagonal gram tiles, the nb diagonal ones.
__global__ __launch_bounds__(SW_NT, 1) void snap_wide_kernel(PrefillArgs a) {
  __shared__ __attribute__((aligned(16))) bf16_t lds[SW_LDS];
  const int nod = a.nb * (a.nb - 1) / 2;
  const int tpg = a.rd_pg + nod + a.nb;
  const int id = blockIdx.x;
  const int blk = id / (8 * tpg), rem = id - blk * 8 * tpg;
  int u = rem >> 3;
  const int g = blk * 8 + (rem & 7);
  if (g >= a.gram_groups) return;
  const int64_t iv = g % a.n_iv;
  const int q = (int)(g / a.n_iv);
  const int kp = q % a.ks;
  const int64_t s = q / a.ks;
  const int64_t t0 = iv * a.L;
  const int64_t Lc = (a.T - t0 < a.L) ? a.T - t0 : a.L;
  if (u < a.rd_pg) {
    const int ndb = (int)((a.D + T256 - 1) / T256);
    const int64_t ri = (int64_t)(u / ndb) * T256, d0 = (int64_t)(u % ndb) * T256;
    if (iv < a.rd_iv0 || ri >= Lc) return;
    snap_wide_dispatch<K_READ>(a, lds, s, kp, iv, ri, d0, ri + T256 <= Lc);
    return;
  }
  u -= a.rd_pg;
  if (u < nod) {
    int bi = 1;
    while (bi * (bi + 1) / 2 <= u) ++bi;  // row block of off-diagonal tile u
    const int bj = u - bi * (bi - 1) / 2;
    const int64_t ri = (int64_t)bi * T256, rj = (int64_t)bj * T256;
    if (ri >= Lc) return;  // past a ragged last interval: never read
    snap_wide_dispatch<K_OFF>(a, lds, s, kp, iv, ri, rj, ri + T256 <= Lc);
    return;
  }
  const int64_t ri = (int64_t)(u - nod) * T256;
  if (ri >= Lc) return;
  snap_wide_dispatch<K_DIAG>(a, lds, s, kp, iv, ri, ri, ri + T256 <= Lc);
}

}  // namespace

int snap_wide_ids(int groups, int nb, int rd_pg) {
  const int tpg = rd_pg + nb * (nb - 1) / 2 + nb;
  return ((groups + 7) / 8) * 8 * tpg;
}

hipError_t launch_snap_wide(const PrefillArgs& a, hipStream_t st) {
  if (a.gram_ids == 0) return hipSuccess;
  hipLaunchKernelGGL(snap_wide_kernel, dim3((unsigned)a.gram_ids), dim3(SW_NT), 0, st, a);
  return hipGetLastError();
}

}  // namespace bdh
