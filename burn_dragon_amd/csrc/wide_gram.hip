// Gram tiles of a context-only call on pre-rotated queries (one interval,
// whole 256-row blocks, no decay) in 256-thread workgroups, one per CU: each
// of the 4 waves owns a 128 x 128 block of v_mfma_f32_16x16x32_bf16
// accumulators (256 accumulator registers; one wave a SIMD), the workgroup a
// 256 x 256 tile.  Against the 8-wave tiles of snap_wide.hip (64 x 128 a
// wave) a step reads 64 instead of 96 KiB of fragments from LDS beside its
// 32 KiB of direct loads, for the same 1024 MFMA cycles a SIMD.
//   diagonal tile      rows = columns = 256 tokens: 256 rows loaded a step,
//                      the wave of rows 0..127 x columns 128..255 idle;
//   off-diagonal tile  256 + 256 token rows.
// The ring and its waits follow snap_wide.hip: four stages, direct loads
// three steps ahead, one barrier a step, each wave reading the next step's
// fragments while it multiplies the current one, with the reads and the
// direct loads spread between its 8 groups of 8 MFMAs.  Outputs: the gram
// partials [KS, S, 1, Lp, Lp] (bf16 with part16), tril-masked, which the
// context kernel sums.  The closed form is the reference's (linear.rs:221-322).
#include "bdh_mfma.h"

namespace bdh {
namespace {

using namespace mfma;

constexpr int WG4_NT = 256;
constexpr int WG4_STAGE = 2 * T256 * BK;  // bf16 elements of one stage: A rows 0..255, B rows 256..511
constexpr int WG4_LDS = 4 * WG4_STAGE;    // four stages (128 KiB); the epilogue reuses them

// Fragment I of a 128 x 128 block: I < 8 the A rows 16 I.., else the B rows
// 16 (I - 8)..; a and b from frag_64x128_base.
template <int I>
__device__ __forceinline__ void frag128_read(uint32_t a, uint32_t b, u32x4 (&af)[8], u32x4 (&bf)[8]) {
  if constexpr (I < 8)
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(af[I]) : "v"(a), "n"(I * 1024));
  else
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(bf[I - 8]) : "v"(b), "n"((I - 8) * 1024));
}
// The next step's 16 fragment reads spread over MFMA groups 0..5 (three a
// group, one in group 5), so that they have landed before the next step's
// wait.
template <int G>
__device__ __forceinline__ void frag128_reads(uint32_t a, uint32_t b, u32x4 (&af)[8], u32x4 (&bf)[8]) {
  if constexpr (3 * G < 16) frag128_read<3 * G>(a, b, af, bf);
  if constexpr (3 * G + 1 < 16) frag128_read<3 * G + 1>(a, b, af, bf);
  if constexpr (3 * G + 2 < 16) frag128_read<3 * G + 2>(a, b, af, bf);
}
__device__ __forceinline__ void frags128_wait(u32x4 (&af)[8], u32x4 (&bf)[8]) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(af[0]), "+v"(af[1]), "+v"(af[2]), "+v"(af[3]), "+v"(af[4]), "+v"(af[5]), "+v"(af[6]),
                 "+v"(af[7]), "+v"(bf[0]), "+v"(bf[1]), "+v"(bf[2]), "+v"(bf[3]), "+v"(bf[4]), "+v"(bf[5]),
                 "+v"(bf[6]), "+v"(bf[7]));
}
// The step's 64 MFMAs in 8 groups (group G: B fragment G with the 8 A
// fragments); between(integral_constant<G>) runs after group G, fenced so
// that the scheduler keeps it there.  The MFMAs are asm with the
// accumulator tied in place ("+a"): with every AGPR holding an accumulator,
// the builtin form lets the register allocator rotate accumulators through
// v_accvgpr moves between MFMAs (about 150 a step).  Fragments come from
// LDS reads behind an lgkmcnt wait, and srcA/B are read at issue, so the
// only hazard left to cover by hand is the epilogue's read of the results.
template <int G, class Between>
__device__ __forceinline__ void mma128_group(const u32x4 (&af)[8], const u32x4 (&bf)[8], floatx4 (&acc)[8][8],
                                             Between& between) {
#pragma unroll
  for (int mi = 0; mi < 8; ++mi)
    asm("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(acc[mi][G]) : "v"(af[mi]), "v"(bf[G]));
  __builtin_amdgcn_sched_barrier(0);
  between(std::integral_constant<int, G>{});
  __builtin_amdgcn_sched_barrier(0);
}
template <class Between, int... G>
__device__ __forceinline__ void mma128_groups(const u32x4 (&af)[8], const u32x4 (&bf)[8], floatx4 (&acc)[8][8],
                                              Between& between, std::integer_sequence<int, G...>) {
  (mma128_group<G>(af, bf, acc, between), ...);
}
template <class Between>
__device__ __forceinline__ void mma128_frags(u32x4 (&af)[8], u32x4 (&bf)[8], floatx4 (&acc)[8][8],
                                             Between&& between) {
  __builtin_amdgcn_sched_barrier(0);
  mma128_groups(af, bf, acc, between, std::make_integer_sequence<int, 8>{});
}

// The block's scores through the wave's own 16 x 132-float slab of LDS
// (rows 16 mi .. of the block at a time), emit(row, col, lo, hi) getting
// columns col .. col + 7 of one row (col = 8 (lane & 15)), 4 rows a call.
// The slab is the wave's alone and the ring is idle by then, so no
// workgroup barrier: lgkmcnt waits order the wave's own writes and reads.
template <class Emit>
__device__ __forceinline__ void wave_epilogue8(const floatx4 (&acc)[8][8], bf16_t* lds, int w, int lane,
                                               Emit&& emit) {
  constexpr int EP = 132;
  float* E = reinterpret_cast<float*>(lds) + w * 16 * EP;
#pragma unroll
  for (int mi = 0; mi < 8; ++mi) {
#pragma unroll
    for (int ni = 0; ni < 8; ++ni)
#pragma unroll
      for (int r = 0; r < 4; ++r) E[acc16_row(lane, r) * EP + ni * 16 + acc16_col(lane)] = acc[mi][ni][r];
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int rr = 0; rr < 16; rr += 4) {
      const int row = rr + (lane >> 4), col = 8 * (lane & 15);
      emit(mi * 16 + row, col, *reinterpret_cast<const float4*>(&E[row * EP + col]),
           *reinterpret_cast<const float4*>(&E[row * EP + col + 4]));
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  }
}

// Tile of stream s, N range kp: A = token rows ri .. ri + 255, B = token rows
// rj .. (off diagonal) or the A rows (diagonal).  Wave w fetches the 16-row
// blocks w + 4 j of the stage (j < 4: A, j >= 4: B); the lane writing LDS
// slot c of row r fetches global chunk c ^ ((r >> 1) & 3), the swizzle of
// lds_off.
template <bool DIAG>
__device__ __forceinline__ void wide_gram_unit(const PrefillArgs& a, bf16_t* lds, int64_t s, int kp, int64_t ri,
                                               int64_t rj) {
  constexpr int NB = DIAG ? 4 : 8;  // 16-row blocks a wave fetches a step
  const int lane = threadIdx.x & 63, w = wave_id();
  const int wr = w >> 1, wc = w & 1;  // rows 128 wr .., columns 128 wc .. of the tile
  const int64_t rowb = a.N * 2;
  const char* X = reinterpret_cast<const char*>(a.x + s * a.T * a.N);
  const int nk = (int)(a.N / BK);
  // Uniform step bounds (readfirstlane), so that the loop counter and the
  // direct loads' addresses live in scalar registers.
  const int kb = __builtin_amdgcn_readfirstlane((int)((int64_t)nk * kp / a.ks));
  const int ke = __builtin_amdgcn_readfirstlane((int)((int64_t)nk * (kp + 1) / a.ks));
  const uint32_t gc = (uint32_t)((lane & 3) ^ ((lane >> 3) & 3));
  const uint32_t voff = (uint32_t)((lane >> 2) * rowb) + gc * 16;
  int64_t vbase[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    const int blk = w + 4 * j;
    vbase[j] = (blk < 16 ? ri + 16 * blk : rj + 16 * (blk - 16)) * rowb;
  }
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_addr(lds));
  auto issue1 = [&](int kt, int stg, int j) {
    dma16(X + vbase[j] + (int64_t)kt * 64, voff, lds0 + (uint32_t)(stg * WG4_STAGE * 2 + (w + 4 * j) * 1024));
  };
  auto issue = [&](int kt, int stg) {
#pragma unroll
    for (int j = 0; j < NB; ++j) issue1(kt, stg, j);
  };
  floatx4 acc[8][8];
#pragma unroll
  for (int mi = 0; mi < 8; ++mi)
#pragma unroll
    for (int ni = 0; ni < 8; ++ni) acc[mi][ni] = zero4();
  const bool active = !DIAG || 128 * wr + 127 > 128 * wc;
  const int brow = DIAG ? 128 * wc : T256 + 128 * wc;
  __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): no compiler-visible load left in flight
  auto clampk = [&](int k) { return k < ke ? k : ke - 1; };
  issue(kb, 0);
  issue(clampk(kb + 1), 1);
  issue(clampk(kb + 2), 2);
  dma_wait_barrier<2 * NB>();  // stage kb landed
  u32x4 fa[8], fb[8], ga[8], gb[8];
  const uint32_t fa0 = frag_64x128_base(lds, lane, 128 * wr), fb0 = frag_64x128_base(lds, lane, brow);
  constexpr uint32_t SB = WG4_STAGE * 2;
  if (active) {
    frag128_read<0>(fa0, fb0, fa, fb);
    frag128_read<1>(fa0, fb0, fa, fb);
    frag128_read<2>(fa0, fb0, fa, fb);
    frag128_read<3>(fa0, fb0, fa, fb);
    frag128_read<4>(fa0, fb0, fa, fb);
    frag128_read<5>(fa0, fb0, fa, fb);
    frag128_read<6>(fa0, fb0, fa, fb);
    frag128_read<7>(fa0, fb0, fa, fb);
    frag128_read<8>(fa0, fb0, fa, fb);
    frag128_read<9>(fa0, fb0, fa, fb);
    frag128_read<10>(fa0, fb0, fa, fb);
    frag128_read<11>(fa0, fb0, fa, fb);
    frag128_read<12>(fa0, fb0, fa, fb);
    frag128_read<13>(fa0, fb0, fa, fb);
    frag128_read<14>(fa0, fb0, fa, fb);
    frag128_read<15>(fa0, fb0, fa, fb);
  }
  int stg = 0;  // stage of step kt
  constexpr int GPD = 8 / NB;  // MFMA groups per direct load
  if (!active) {
    // The idle wave of a diagonal tile: its share of the direct loads and
    // the barriers only (a loop of its own, so that the accumulators never
    // cross a branch).
    for (int kt = kb; kt < ke; ++kt) {
      dma_wait_barrier<NB>();
      issue(clampk(kt + 3), (stg + 3) & 3);
      stg = (stg + 1) & 3;
    }
  } else {
    // Step kt: the barrier confirms stage kt + 1; the wave reads step kt + 1's
    // fragments (3 a group, groups 0..5) into the other set while it multiplies step kt,
    // and issues step kt + 3's direct loads into the stage of step kt - 1.
    // ke - kb is even: the loop has one exit.
    for (int kt = kb; kt < ke; kt += 2) {
      dma_wait_barrier<NB>();
      int kn = clampk(kt + 3), sn = (stg + 3) & 3;
      stg = (stg + 1) & 3;
      frags128_wait(fa, fb);
      uint32_t na = fa0 + stg * SB, nb = fb0 + stg * SB;
      mma128_frags(fa, fb, acc, [&](auto gcst) {
        constexpr int g = decltype(gcst)::value;
        frag128_reads<g>(na, nb, ga, gb);
        if constexpr (g % GPD == GPD - 1) issue1(kn, sn, g / GPD);
      });
      dma_wait_barrier<NB>();
      kn = clampk(kt + 4);
      sn = (stg + 3) & 3;
      stg = (stg + 1) & 3;
      frags128_wait(ga, gb);
      na = fa0 + stg * SB;
      nb = fb0 + stg * SB;
      mma128_frags(ga, gb, acc, [&](auto gcst) {
        constexpr int g = decltype(gcst)::value;
        frag128_reads<g>(na, nb, fa, fb);
        if constexpr (g % GPD == GPD - 1) issue1(kn, sn, g / GPD);
      });
    }
  }
  // The last (unused) fragment reads land in fa / fb: the wait names them,
  // so that their registers are not reused before it.  Then wait states for
  // the epilogue's reads of accumulators written by the asm MFMAs (whose
  // hazards the compiler does not track).
  frags128_wait(fa, fb);
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
  dma_wait_barrier<0>();  // the epilogue reuses the ring

  // Scores (ti, tj), 0 on and above the diagonal.
  const int64_t Lp = a.Lp;
  const int64_t wr0 = ri + 128 * wr, wc0 = rj + 128 * wc;
  if (!active) return;  // the idle wave of a diagonal tile writes nothing (no barrier follows)
  wave_epilogue8(acc, lds, w, lane, [&](int row, int col, float4 lo, float4 hi) {
    const int64_t ti = wr0 + row, tj = wc0 + col;
    const float e[8] = {tj < ti ? lo.x : 0.0f,     tj + 1 < ti ? lo.y : 0.0f, tj + 2 < ti ? lo.z : 0.0f,
                        tj + 3 < ti ? lo.w : 0.0f, tj + 4 < ti ? hi.x : 0.0f, tj + 5 < ti ? hi.y : 0.0f,
                        tj + 6 < ti ? hi.z : 0.0f, tj + 7 < ti ? hi.w : 0.0f};
    const int64_t o = (((int64_t)kp * a.S + s) * Lp + ti) * Lp + tj;
    // Streaming stores: the partials are read once, by the context kernel.
    if (a.part16) {
      __builtin_nontemporal_store(u32x4{pack_bf16x2(e[0], e[1]), pack_bf16x2(e[2], e[3]), pack_bf16x2(e[4], e[5]),
                                        pack_bf16x2(e[6], e[7])},
                                  reinterpret_cast<u32x4*>(reinterpret_cast<bf16_t*>(a.part) + o));
    } else {
      __builtin_nontemporal_store(floatx4{e[0], e[1], e[2], e[3]}, reinterpret_cast<floatx4*>(a.part + o));
      __builtin_nontemporal_store(floatx4{e[4], e[5], e[6], e[7]}, reinterpret_cast<floatx4*>(a.part + o + 4));
    }
  });
}

// Group g = (stream, N range); its units: the nb (nb - 1) / 2 off-diagonal
// tiles, then the nb diagonal ones.  Ids in blocks of 8 groups, id = unit * 8
// + (group & 7) inside a block: a group's tiles (which read the same rows)
// run on one XCD (workgroup id i runs on XCD i % 8).
__global__ __launch_bounds__(WG4_NT, 1) void wide_gram_kernel(PrefillArgs a) {
  __shared__ __attribute__((aligned(16))) bf16_t lds[WG4_LDS];
  const int nod = a.nb * (a.nb - 1) / 2;
  const int tpg = nod + a.nb;
  const int id = blockIdx.x;
  const int blk = id / (8 * tpg), rem = id - blk * 8 * tpg;
  const int u = rem >> 3;
  const int g = blk * 8 + (rem & 7);
  if (g >= a.gram_groups) return;
  const int kp = g % a.ks;
  const int64_t s = g / a.ks;
  if (u < nod) {
    int bi = 1;
    while (bi * (bi + 1) / 2 <= u) ++bi;  // row block of off-diagonal tile u
    const int bj = u - bi * (bi - 1) / 2;
    wide_gram_unit<false>(a, lds, s, kp, (int64_t)bi * T256, (int64_t)bj * T256);
    return;
  }
  const int64_t ri = (int64_t)(u - nod) * T256;
  wide_gram_unit<true>(a, lds, s, kp, ri, ri);
}

}  // namespace

bool wide_gram_fits(const PrefillArgs& a) {
  return a.n_iv == 1 && a.decay == nullptr && a.freqs == nullptr && a.rd_pg == 0 && a.T % T256 == 0 &&
         a.Lp == a.T && a.N % 64 == 0 && (a.N / BK) % (2 * a.ks) == 0;
}

int wide_gram_ids(int groups, int nb) {
  const int tpg = nb * (nb - 1) / 2 + nb;
  return ((groups + 7) / 8) * 8 * tpg;
}

hipError_t launch_wide_gram(const PrefillArgs& a, hipStream_t st) {
  if (a.gram_ids == 0) return hipSuccess;
  hipLaunchKernelGGL(wide_gram_kernel, dim3((unsigned)a.gram_ids), dim3(WG4_NT), 0, st, a);
  return hipGetLastError();
}

}  // namespace bdh
