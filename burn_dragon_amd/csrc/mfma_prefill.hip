// Gram, readout and state products of the bf16 chunked prefill (gfx950
// MFMA), in one launch.  Each workgroup computes a 256x128 (gram, readout)
// or 128x256 (state) output tile of a bf16 product with fp32 accumulation:
// 4 waves, each owning a 64x128 block of v_mfma_f32_16x16x32_bf16
// accumulators.  Two workgroups share a CU (48 KB of LDS and up to 256
// registers per lane each), so while one waits on its loads, rotates its next
// tile or synchronises, the other's MFMAs keep the matrix cores busy.
//
//   gram unit   S_kp[r, c] = sum_{n in range kp} q_r[n] q_c[n] for one
//               256-row x 128-column tile touching an interval's lower
//               triangle, written (masked to c < r, times d^(r-c)) to the
//               partial buffer kp; contraction over neurons.  Waves whose 64
//               rows lie wholly above the diagonal skip the MFMAs.
//   state unit  rho_out[n, d] = rho_in[n, d] * d^Lc + sum_t q_t[n] d^(Lc-t) v_t[d]
//               for a 128-neuron x 256-column block; contraction over tokens,
//               so the rotated x tile is written transposed ([n][t]) to LDS.
//   readout unit (q_t d^t) . rho_in for 256 rows x 128 columns over one N
//               range (split-K partial); rho is read as fp32 rows and
//               written transposed as bf16 to LDS.
//
// q = RoPE(x) is applied between HBM and LDS: each lane computes the packed
// bf16 (cos, sin) words of its 4 pairs from the f32 phase frac(p f) (v_cos /
// v_sin take revolutions; the gram tiles advance it from one row group to the
// next by a complex multiply) and rotates with v_dot2.  K steps are 32 deep; LDS
// holds two steps (double buffer) and the loads of later steps are in flight
// while step k is multiplied (the RoPE gram tiles' x two steps ahead).  Every
// unit runs an even number of steps (the host guarantees it), so the step
// loop has a single exit; with a mid-loop exit the compiler moves the
// accumulators between AGPRs and VGPRs on every iteration.
// Units are ordered heaviest first (gram tiles, readout blocks, then state
// blocks), so the state units' HBM-bound rho writes fill the tail.
#include "bdh_mfma.h"

namespace bdh {
namespace {

using namespace mfma;

// ---------------------------------------------------------------------------
// gram unit: rows ri .. ri+255 (A) x columns rj .. rj+127 (B) of interval iv,
// N range [kb, ke) in BK steps.  PAIR: two diagonal 128 x 128 blocks, rows
// and columns ri .. ri+127 (waves 0, 1) and rj .. rj+127 (waves 2, 3; rj < 0:
// none), each the lower part of a 256-row block's last 128-column tile.
// INNER: the 128 columns are tokens of the tile's own 256 rows (rj - ri = 0
// or 128; pairs are inner too), so only the 4 A groups are loaded.
template <bool ROPE, bool DECAY, bool WHOLE, bool INNER, bool PAIR = false>
__device__ __forceinline__ void gram_unit(const PrefillArgs& a, bf16_t* lds, int64_t s, int kp,
                                          int64_t iv, int64_t ri, int64_t rj) {
  const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
  const int64_t t0 = iv * a.L;
  const int64_t Lc = (a.T - t0 < a.L) ? a.T - t0 : a.L;
  const int64_t rowb = a.N * 2;  // bytes per x row
  const char* X = reinterpret_cast<const char*>(a.x + (s * a.T + t0) * a.N);
  const int nk = (int)(a.N / BK);
  // RoPE units: uniform step bounds (readfirstlane), so that the loop
  // counter and the direct loads' addresses live in scalar registers (the
  // other units' loops already keep them there, and are worse with it).
  int kb = (int)((int64_t)nk * kp / a.ks), ke = (int)((int64_t)nk * (kp + 1) / a.ks);
  if constexpr (ROPE) {
    kb = __builtin_amdgcn_readfirstlane(kb);
    ke = __builtin_amdgcn_readfirstlane(ke);
  }

  // Loader: 4 lanes per 64-byte row segment; group g < 4 covers A rows
  // rb + 64 g, g = 4, 5 cover B rows rb + 64 (g - 4).  WHOLE tiles (inside
  // the interval) use uniform row bases and one per-lane offset.  Tiles that
  // cross the end of a ragged interval re-read its last row for the rows past
  // it: their scores are never written (and a select on the loaded value
  // would stall the load).
  // A tile whose 128 columns are tokens of its own 256 rows (rj - ri = 0 or
  // 128) takes its B operand from the A rows already in LDS: groups 4 and 5
  // load nothing.  The row offset is a multiple of 8, so a row's swizzle is
  // the same seen from either base.
  constexpr bool inner = PAIR || INNER;
  constexpr int groups = inner ? 4 : 6;
  const int64_t rj2 = PAIR ? (rj < 0 ? ri : rj) : rj;  // second block (a pair's absent one re-reads the first)
  const int kc = tid & 3, rb = tid >> 2;
  const uint32_t lane_off = (uint32_t)(rb * rowb + kc * 16);
  // Uniform base and per-lane offset of group g's 16 bytes of step kt in a
  // [token][N] array.
  auto at = [&](int g, int kt, uint32_t& off) -> int64_t {
    const int64_t kofs = (int64_t)kt * 64;  // 32 bf16 of x
    const int64_t r0 = PAIR ? (g < 2 ? ri + 64 * g : rj2 + 64 * (g - 2))
                            : (g < 4 ? ri + 64 * g : rj + 64 * (g - 4));
    if (WHOLE) {
      off = lane_off;
      return r0 * rowb + kofs;
    }
    const int64_t t = r0 + rb;
    off = (uint32_t)((t < Lc ? t : Lc - 1) * rowb + kc * 16);
    return kofs;
  };
  // RoPE: the position of each group's row for this lane (constant over the
  // steps) and the step's 4 pair frequencies (neurons 32 kt + 8 kc + 2 j).
  float pg[6];
#pragma unroll
  for (int g = 0; g < 6; ++g) {
    const int64_t r0 = PAIR ? (g < 2 ? ri + 64 * g : rj2 + 64 * (g - 2))
                            : (g < 4 ? ri + 64 * g : rj + 64 * (g - 4));
    const int64_t t = WHOLE ? r0 + rb : (r0 + rb < Lc ? r0 + rb : Lc - 1);
    pg[g] = ROPE ? rope_pos(a, t0 + t) : 0.0f;
  }
  floatx4 acc[4][8];
  zero_acc(acc);
  // Waves whose 64 rows end at or before the tile's first column compute
  // nothing that is kept; nor do waves starting past a ragged interval.
  // Each wave's rows start at wr0 and its columns at wc0.
  const int64_t wc0 = PAIR ? (w < 2 ? ri : rj2) : rj;
  const int64_t wr0 = PAIR ? wc0 + 64 * (w & 1) : ri + 64 * w;
  const bool active = PAIR ? (wr0 < Lc && (w < 2 || rj >= 0)) : (wr0 + 64 > rj + 1 && wr0 < Lc);
  const int brow = PAIR ? 128 * (w >> 1) : inner ? (int)(rj - ri) : T256;  // LDS row of the first B row
  if (!ROPE) {
    // Operands need no rotation: a three-stage LDS ring filled by direct
    // loads two steps ahead, one barrier per step, no register staging.
    // Stage rows are those of the register path (A rows 0..255, B rows
    // 256..383), swizzled the same way: the lane writing LDS slot c of row r
    // fetches global chunk c ^ ((r >> 1) & 3).  Wave w issues the DMAs of
    // 16-row blocks w, w + 4, ... (groups of them per step).
    const uint32_t gc = (uint32_t)((lane & 3) ^ ((lane >> 3) & 3));
    uint32_t voff[groups];
    int64_t vbase[groups];
#pragma unroll
    for (int j = 0; j < groups; ++j) {
      const int blk = w + 4 * j;  // 16-row block of the stage
      const int g = blk >> 2;
      const int64_t r0 = PAIR ? (g < 2 ? ri + 64 * g : rj2 + 64 * (g - 2))
                              : (g < 4 ? ri + 64 * g : rj + 64 * (g - 4));
      const int64_t t = r0 + 16 * (blk & 3) + (lane >> 2);
      if (WHOLE) {
        vbase[j] = (r0 + 16 * (blk & 3)) * rowb;
        voff[j] = (uint32_t)((lane >> 2) * rowb) + gc * 16;
      } else {
        vbase[j] = 0;
        voff[j] = (uint32_t)((t < Lc ? t : Lc - 1) * rowb) + gc * 16;
      }
    }
    constexpr int STAGE = groups * 64 * BK;  // bf16 elements of one stage
    const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_addr(lds));
    auto issue = [&](int kt, int stg) {
      const char* gb = X + (int64_t)kt * 64;
#pragma unroll
      for (int j = 0; j < groups; ++j)
        dma16(gb + vbase[j], voff[j], lds0 + (uint32_t)(stg * STAGE * 2 + (w + 4 * j) * 1024));
    };
    // A compiler-visible wait: loads of other unit kinds that share this
    // kernel's registers are then known complete, so the compiler adds no
    // waits inside the ring loop (it cannot see the DMAs, only their
    // destination-less assembly).
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
    issue(kb, 0);
    issue(kb + 1 < ke ? kb + 1 : kb, 1);
    int stg = 0;
    for (int kt = kb; kt < ke; ++kt) {
      dma_wait_barrier<groups>();
      // Step kt + 2 goes to the stage read in step kt - 1, which every wave
      // has finished; past the end the last step is fetched again (unused),
      // so that every step leaves the same number of DMAs in flight.
      issue(kt + 2 < ke ? kt + 2 : ke - 1, stg == 0 ? 2 : stg - 1);
      if (active) mma_64x128_dsasm(lds + stg * STAGE, lds + stg * STAGE, lane, 64 * w, brow, acc);
      stg = stg == 2 ? 0 : stg + 1;
    }
    dma_wait_barrier<0>();  // the epilogue reuses the ring
  } else {
    // RoPE: each lane's raw x chunks and the step's frequencies arrive by
    // direct loads two steps ahead in lane-private LDS slots (the third
    // buffer; the frequencies after it).  At the top of a step the lane reads
    // the next step's slots into registers and refills them with the step
    // after; after the MFMAs it rotates what it read into the other operand
    // buffer.  The loads then have a whole step to land, where loads into
    // registers one step ahead had only the MFMA phase (C2: 258 -> 253 us).
    // A lane reads back only what its own loads wrote (wave w's load of group
    // g fills rows 64 g + 16 w + l/4, chunk l & 3 for lane l: that lane's
    // (rb, kc)), so the slots need waits but no barrier.  (Rotating each
    // group between the MFMA groups instead was slower: 266 us.)
    struct Stage {
      uint4 xr[6];
      float fq[4];
    } st;
    const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_addr(lds));
    const uint32_t raw0 = lds0 + (uint32_t)(2 * BUF * 2);
    const uint32_t fq0 = lds0 + (uint32_t)(3 * BUF * 2 + w * 256);
    const char* rawp = reinterpret_cast<const char*>(lds + 2 * BUF) + w * 1024 + 16 * lane;
    const float* fqp = reinterpret_cast<const float*>(lds + 3 * BUF) + w * 64 + 4 * kc;
    // Step kt's x chunks, then its 16 pair frequencies (lane l: the even
    // neuron 32 kt + 2 (l & 15); lanes 4 kc .. 4 kc + 3 are this lane's).
    auto issue = [&](int kt) {
#pragma unroll
      for (int g = 0; g < 6; ++g) {
        if (g >= groups) break;
        uint32_t off;
        const int64_t o = at(g, kt, off);
        dma16(X + o, off, raw0 + (uint32_t)((g * 4 + w) * 1024));
      }
      dma4(a.freqs + (int64_t)kt * BK, (uint32_t)(8 * (lane & 15)), fq0);
    };
    // The slots into registers; they may be refilled once this returns.
    auto pull = [&]() {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
      for (int g = 0; g < 6; ++g) {
        if (g >= groups) break;
        st.xr[g] = *reinterpret_cast<const uint4*>(rawp + g * 4096);
      }
      const float4 f = *reinterpret_cast<const float4*>(fqp);
      st.fq[0] = f.x;
      st.fq[1] = f.y;
      st.fq[2] = f.z;
      st.fq[3] = f.w;
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    };
    // Packed (cos, sin) words of each group's row for the step in st,
    // computed before the MFMAs of the current step (the rotation itself
    // follows them).  A lane's rows in groups g and g + 1 of one operand lie
    // 64 tokens apart (0 with fixed positions), so only the first group of
    // each operand takes its phase from frac(p f) and two transcendentals;
    // the others advance it by one complex multiply with e(64 f).  (C2: 253 ->
    // 249 us; the advance alone, after the MFMAs, gained nothing.)  Rows past
    // a ragged interval take advanced phases instead of their clamped row's:
    // their scores are never stored.
    uint4 csw[6];
    auto phases = [&]() {
      float c[4], sn[4], ec[4], es[4];
      const float dstep = a.fixed ? 0.0f : 64.0f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float fe = rope_frac(dstep, st.fq[j]);
        ec[j] = __builtin_amdgcn_cosf(fe);
        es[j] = __builtin_amdgcn_sinf(fe);
      }
      constexpr int anchor2 = PAIR ? 2 : 4;
#pragma unroll
      for (int g = 0; g < 6; ++g) {
        if (g >= groups) break;
        if (g == 0 || g == anchor2) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float fr = rope_frac(pg[g], st.fq[j]);
            c[j] = __builtin_amdgcn_cosf(fr);
            sn[j] = __builtin_amdgcn_sinf(fr);
          }
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float nc = c[j] * ec[j] - sn[j] * es[j];
            const float ns = sn[j] * ec[j] + c[j] * es[j];
            c[j] = nc;
            sn[j] = ns;
          }
        }
        csw[g] = make_uint4(pack_bf16x2(c[0], sn[0]), pack_bf16x2(c[1], sn[1]), pack_bf16x2(c[2], sn[2]),
                            pack_bf16x2(c[3], sn[3]));
      }
    };
    auto store = [&](int buf) {
      bf16_t* base = lds + buf * BUF;  // A rows 0..255, then B rows 256..383
#pragma unroll
      for (int g = 0; g < 6; ++g) {
        if (g >= groups) break;
        *reinterpret_cast<uint4*>(&base[lds_off(64 * g + rb, kc)]) = rot8_bf16(st.xr[g], csw[g]);
      }
    };
    auto compute = [&](int buf) {
      if (active) mma_64x128(lds + buf * BUF, lds + buf * BUF, lane, 64 * w, brow, acc);
    };
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): no compiler-visible load left in flight
    auto clampk = [&](int k) { return k < ke ? k : ke - 1; };
    issue(kb);
    pull();
    issue(clampk(kb + 1));
    phases();
    store(0);
    __syncthreads();
    // Past the end the last step is fetched again (unused).
    for (int kt = kb; kt < ke; kt += 2) {
      pull();  // step kt + 1 (ke - kb is even)
      issue(clampk(kt + 2));
      phases();
      compute(0);
      store(1);
      __syncthreads();
      pull();  // step kt + 2
      issue(clampk(kt + 3));
      phases();
      compute(1);
      if (kt + 2 < ke) store(0);
      __syncthreads();
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the unused loads, before the epilogue reuses LDS
    __syncthreads();
  }

  // Scores of rows ti < Lc and columns tj < Lc: times d^(ti - tj) below
  // the diagonal, 0 on and above it.  Waves that computed nothing still
  // take part in the epilogue's barriers.
  const float dk = DECAY ? a.decay[s % a.H] : 1.0f;
  const float l2d = DECAY ? decay_log2(dk) : 0.0f;
  float* P = a.part + (((int64_t)kp * a.S + s) * a.n_iv + iv) * a.Lp * a.Lp;
  epilogue_64x128(acc, lds, w, lane, [&](int row, int col, float4 v) {
    const int64_t ti = wr0 + row, tj = wc0 + col;
    if (!active || ti >= Lc) return;
    float e[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j)
      e[j] = tj + j < ti ? (DECAY ? e[j] * decay_pow_int(dk, l2d, (int)(ti - tj - j)) : e[j]) : 0.0f;
    float* dst = P + ti * a.Lp + tj;
    // Streaming stores: the partials are read once, by the context kernel
    // after this launch (C2: 0.369 -> 0.351 ms per prefill).
    if (tj + 3 < Lc) {
      __builtin_nontemporal_store(floatx4{e[0], e[1], e[2], e[3]}, reinterpret_cast<floatx4*>(dst));
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (tj + j < Lc) dst[j] = e[j];
    }
  });
}

// ---------------------------------------------------------------------------
// state unit: rho block (n0 .. n0+127, d0 .. d0+255) of stream s over tokens
// [st_t0, st_t0 + st_Lc).
template <bool ROPE, bool DECAY, bool WHOLE>
__device__ __forceinline__ void state_unit(const PrefillArgs& a, bf16_t* lds, int64_t s,
                                           int64_t n0, int64_t d0) {
  const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
  const int wm = w >> 1, wn = w & 1;  // n rows 64*wm.., d cols 128*wn..
  const int64_t b = s / a.H, h = s - b * a.H;
  const int64_t t0 = a.st_t0, Lc = a.st_Lc;
  const int64_t rowb = a.N * 2;  // bytes per x row
  const char* X = reinterpret_cast<const char*>(a.x + s * a.T * a.N);
  const char* VT = reinterpret_cast<const char*>(a.vt + (b * a.Hv + (a.Hv == 1 ? 0 : h)) * a.Dp * a.Tp);
  const float dk = DECAY ? a.decay[h] : 1.0f;
  const float l2d = DECAY ? decay_log2(dk) : 0.0f;

  // x loader: lane block of 2 tokens (2 tp, 2 tp + 1) x 8 neurons (8 nv ..).
  // In a unit whose steps run past T (ragged last interval, !WHOLE), tokens
  // past T re-read row T-1: their v^T columns are zero-padded, so they add 0.
  const int tp = tid & 15, nv = tid >> 4;
  const uint32_t xlane = (uint32_t)(2 * tp * rowb + (n0 + 8 * nv) * 2);
  // v^T loader: 4 lanes per 64-byte segment of a row d, rows vb + 64 i (v^T
  // has Dp = D rounded up to 256 rows, zero past D; a step's rows are
  // contiguous).
  const int kc = tid & 3, vb = tid >> 2;
  const int64_t vstep = a.Dp * 64;  // bytes of one 32-token step of v^T
  const uint32_t vlane = (uint32_t)(vb * 64 + kc * 16);
  // Uniform base and per-lane offset of token tb + i's 16 bytes for this
  // lane in the [token][N] x.
  auto at = [&](int kt, int i, uint32_t& off) -> int64_t {
    const int64_t tb = t0 + (int64_t)kt * BK;
    if (WHOLE) {
      off = xlane;
      return (tb + i) * rowb;
    }
    const int64_t t = tb + 2 * tp + i;
    off = (uint32_t)((t < a.T ? t : a.T - 1) * rowb + (n0 + 8 * nv) * 2);
    return 0;
  };
  // RoPE: the lane's 4 pair frequencies are those of its 8 neurons, the same
  // in every step.
  float fq[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (ROPE) load_freq4(a.freqs + n0 + 8 * nv, fq);
  const float pbase = ROPE ? rope_pos(a, t0) : 0.0f;  // position of the interval's first token
  struct Stage {
    uint4 xr[2], vr[4];
  } st;
  int cur = 0;  // step held in st
  auto load = [&](int kt) {
    cur = kt;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      uint32_t off;
      const int64_t o = at(kt, i, off);
      st.xr[i] = ldg16_off(X + o, off);
    }
    const int64_t tb = t0 + (int64_t)kt * BK;
#pragma unroll
    for (int i = 0; i < 4; ++i) st.vr[i] = ldg16_off(VT + (tb >> 5) * vstep + (d0 + 64 * i) * 64, vlane);
  };
  auto store = [&](int buf) {
    bf16_t* A = lds + buf * BUF;             // [n][t], 128 rows
    bf16_t* B = lds + buf * BUF + 128 * BK;  // [d][t], 256 rows
    float f0[8], f1[8];
    float w0 = 1.0f, w1 = 1.0f;
    const int64_t tl = (int64_t)cur * BK + 2 * tp;  // tokens tl, tl + 1 of the interval
    if (DECAY) {
      w0 = tl < Lc ? decay_pow_int(dk, l2d, (int)(Lc - tl)) : 0.0f;
      w1 = tl + 1 < Lc ? decay_pow_int(dk, l2d, (int)(Lc - tl - 1)) : 0.0f;
    }
    uint4 c0 = make_uint4(0, 0, 0, 0), c1 = c0;
    if (ROPE) {
      // Tokens past T (ragged last interval) add zero: any position will do.
      // Sums of integers below 2^24 are exact in f32.
      const float p0 = a.fixed ? pbase : pbase + (float)(int)tl;
      c0 = rope_cs4(p0, fq);
      c1 = rope_cs4(a.fixed ? pbase : p0 + 1.0f, fq);
    }
    prep8_f32<ROPE>(st.xr[0], c0, w0, DECAY, f0);
    prep8_f32<ROPE>(st.xr[1], c1, w1, DECAY, f1);
    uint32_t* Aw = reinterpret_cast<uint32_t*>(A);
#pragma unroll
    for (int e = 0; e < 8; ++e)
      Aw[(lds_off(8 * nv + e, tp >> 2) + 2 * (tp & 3)) >> 1] = pack_bf16x2(f0[e], f1[e]);
#pragma unroll
    for (int i = 0; i < 4; ++i) *reinterpret_cast<uint4*>(&B[lds_off(vb + 64 * i, kc)]) = st.vr[i];
  };

  floatx4 acc[4][8];
  zero_acc(acc);
  const bool active = d0 + wn * 128 < a.D;
  const int nk = (int)(((Lc + 63) / 64) * 2);  // even; steps past Lc read zero v columns
  auto compute = [&](int buf) {
    if (active) mma_64x128(lds + buf * BUF, lds + buf * BUF + 128 * BK, lane, 64 * wm, 128 * wn, acc);
  };
  run_steps(0, nk, load, store, compute);

  // Columns past D (zero v^T rows) are computed and never written; D is a
  // multiple of 32, so a float4 of columns is all in or all out.
  const float carry = DECAY ? decay_pow_int(dk, l2d, (int)Lc) : 1.0f;
  epilogue_64x128(acc, lds, w, lane, [&](int row, int col, float4 v) {
    const int64_t n = n0 + 64 * wm + row, d = d0 + 128 * wn + col;
    if (d >= a.D) return;
    const int64_t idx = (s * a.N + n) * a.D + d;
    if (a.rho_in) {
      const float4 pv = *reinterpret_cast<const float4*>(&a.rho_in[idx]);
      v.x += pv.x * carry;
      v.y += pv.y * carry;
      v.z += pv.z * carry;
      v.w += pv.w * carry;
    }
    // The caller's final state is not read again here: a streaming store
    // keeps the x rows that the gram tiles share in the caches (C2: 0.390 ->
    // 0.369 ms).  A state between intervals is read by the next launch and
    // stays cached.
    if (a.rho_stream)
      __builtin_nontemporal_store(floatx4{v.x, v.y, v.z, v.w}, reinterpret_cast<floatx4*>(&a.rho_out[idx]));
    else
      *reinterpret_cast<float4*>(&a.rho_out[idx]) = v;
  });
}

// ---------------------------------------------------------------------------
// readout unit: partial (Q * d^r) rho of rows r0 .. r0+255 of the interval
// [rd_t0, rd_t0 + rd_Lc) and columns d0 .. d0+127, over the kp-th N range,
// written to rd_part[kp].  A = the interval's rotated, decay-weighted x rows
// (loaded as in the gram); B = rho^T, converted from the fp32 state rows and
// written transposed ([d][n]) to LDS.
template <bool ROPE, bool DECAY, bool WHOLE>
__device__ __forceinline__ void readout_unit(const PrefillArgs& a, bf16_t* lds, int64_t s, int kp,
                                             int64_t r0, int64_t d0) {
  const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
  const int64_t t0 = a.rd_t0, Lc = a.rd_Lc;
  const int64_t rowb = a.N * 2;  // bytes per x row
  const char* X = reinterpret_cast<const char*>(a.x + (s * a.T + t0) * a.N);
  const float* R = a.rd_rho + s * a.N * a.D;
  const int nk = (int)(a.N / BK);
  const int kb = (int)((int64_t)nk * kp / a.rd_kr), ke = (int)((int64_t)nk * (kp + 1) / a.rd_kr);
  const float dk = DECAY ? a.decay[s % a.H] : 1.0f;
  const float l2d = DECAY ? decay_log2(dk) : 0.0f;

  // x loader (group g: rows rb + 64 g), as in the gram unit; rows past a
  // ragged interval re-read its last row and are never stored.
  const int kc = tid & 3, rb = tid >> 2;
  const uint32_t lane_off = (uint32_t)(rb * rowb + kc * 16);
  float wr[4], pg[4];
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    wr[g] = DECAY ? decay_pow_int(dk, l2d, (int)(r0 + rb + 64 * g)) : 1.0f;
    const int64_t t = r0 + 64 * g + rb;
    pg[g] = ROPE ? rope_pos(a, t0 + (WHOLE || t < Lc ? t : Lc - 1)) : 0.0f;
  }
  // rho loader: lane block of 2 state rows (2 np, 2 np + 1) x 8 columns
  // (8 dv ..); columns past D re-read the last 8 and are never stored.
  const int np = tid & 15, dv = tid >> 4;
  const int64_t dcol = d0 + 8 * dv <= a.D - 8 ? d0 + 8 * dv : a.D - 8;
  struct Stage {
    uint4 xr[4];
    float fq[4];
    float4 rr[4];
  } st;
  auto load = [&](int kt) {
    const int64_t kofs = (int64_t)kt * 64;  // 32 bf16 of x
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      if (WHOLE) {
        const int64_t o = (r0 + 64 * g) * rowb + kofs;
        st.xr[g] = ldg16_off(X + o, lane_off);
      } else {
        const int64_t t = r0 + 64 * g + rb;
        const uint32_t o = (uint32_t)((t < Lc ? t : Lc - 1) * rowb + kc * 16);
        st.xr[g] = ldg16_off(X + kofs, o);
      }
    }
    if (ROPE) load_freq4(a.freqs + (int64_t)kt * BK + kc * 8, st.fq);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const float* row = R + ((int64_t)kt * BK + 2 * np + i) * a.D + dcol;
      st.rr[2 * i] = *reinterpret_cast<const float4*>(row);
      st.rr[2 * i + 1] = *reinterpret_cast<const float4*>(row + 4);
    }
  };
  auto store = [&](int buf) {
    bf16_t* A = lds + buf * BUF;             // x rows 0..255
    bf16_t* B = lds + buf * BUF + T256 * BK; // rho^T rows (columns d) 0..127
#pragma unroll
    for (int g = 0; g < 4; ++g)
      *reinterpret_cast<uint4*>(&A[lds_off(64 * g + rb, kc)]) =
          prep8<ROPE>(st.xr[g], ROPE ? rope_cs4(pg[g], st.fq) : make_uint4(0, 0, 0, 0), wr[g], DECAY);
    const float r0v[8] = {st.rr[0].x, st.rr[0].y, st.rr[0].z, st.rr[0].w,
                          st.rr[1].x, st.rr[1].y, st.rr[1].z, st.rr[1].w};
    const float r1v[8] = {st.rr[2].x, st.rr[2].y, st.rr[2].z, st.rr[2].w,
                          st.rr[3].x, st.rr[3].y, st.rr[3].z, st.rr[3].w};
    uint32_t* Bw = reinterpret_cast<uint32_t*>(B);
#pragma unroll
    for (int e = 0; e < 8; ++e)
      Bw[(lds_off(8 * dv + e, np >> 2) + 2 * (np & 3)) >> 1] = pack_bf16x2(r0v[e], r1v[e]);
  };

  floatx4 acc[4][8];
  zero_acc(acc);
  const bool active = r0 + 64 * w < Lc;
  run_steps(kb, ke, load, store, [&](int buf) {
    if (active) mma_64x128(lds + buf * BUF, lds + buf * BUF + T256 * BK, lane, 64 * w, 0, acc);
  });
  float* P = a.rd_part + ((int64_t)kp * a.S + s) * a.Lp * a.D;
  epilogue_64x128(acc, lds, w, lane, [&](int row, int col, float4 v) {
    const int64_t t = r0 + 64 * w + row, d = d0 + col;
    if (t < Lc && d < a.D) *reinterpret_cast<float4*>(&P[t * a.D + d]) = v;
  });
}

// ---------------------------------------------------------------------------
// add unit aid: a contiguous share of the previous interval's (s, t, float4)
// context elements; the partials are summed in split order onto ctx (the
// order of readout_add_kernel).
__device__ __forceinline__ void add_unit(const PrefillArgs& a, int aid) {
  const int64_t d4n = a.D / 4, total = a.S * a.add_Lc * d4n;
  const int64_t per = (total + a.add_units - 1) / a.add_units;
  const int64_t b = (int64_t)aid * per, e = b + per < total ? b + per : total;
  for (int64_t i = b + threadIdx.x; i < e; i += NT) {
    const int64_t s = i / (a.add_Lc * d4n);
    const int64_t rem = i - s * a.add_Lc * d4n;
    const int64_t t = rem / d4n, d = (rem - t * d4n) * 4;
    float* dst = a.add_ctx + (s * a.T + a.add_t0 + t) * a.D + d;
    float4 v = *reinterpret_cast<const float4*>(dst);
    const float* src = a.add_src + (s * a.Lp + t) * a.D + d;
    const int64_t stride = a.S * a.Lp * a.D;
    int kp = 0;
    for (; kp + 4 <= a.rd_kr; kp += 4) {  // four partials' loads in flight
      float4 r[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) r[j] = *reinterpret_cast<const float4*>(src + (kp + j) * stride);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v.x += r[j].x;
        v.y += r[j].y;
        v.z += r[j].z;
        v.w += r[j].w;
      }
    }
    for (; kp < a.rd_kr; ++kp) {
      const float4 r = *reinterpret_cast<const float4*>(src + kp * stride);
      v.x += r.x;
      v.y += r.y;
      v.z += r.z;
      v.w += r.w;
    }
    *reinterpret_cast<float4*>(dst) = v;
  }
}

// ---------------------------------------------------------------------------
// Gram units of one interval.  Units u < nb^2 are the tiles of 256-row block
// rbk (of nb) x 128-column block cbk for cbk <= 2 rbk, row block by row
// block.  The block's last column tile (cbk = 2 rbk + 1) has work only in its
// lower 128 rows, a diagonal 128 x 128 block; those blocks go two to a unit
// (rows 2j and 2j + 1), units nb^2 .. nb^2 + ceil(nb / 2) - 1, so that a
// group's units carry about equal work.
// Gram ids: blocks of 8 groups; inside a block, id = unit * 8 + (group & 7),
// so the units of one group (which read the same x rows) have ids congruent
// mod 8 and run on one XCD (the dispatcher sends id i to XCD i % 8).
__device__ __forceinline__ int units_per_group(int nb) { return nb * nb + (nb + 1) / 2; }

__device__ __forceinline__ void tile_of(int u, int& rbk, int& cbk) {
  rbk = 0;
  while ((rbk + 1) * (rbk + 1) <= u) ++rbk;
  cbk = u - rbk * rbk;
}

template <bool ROPE, bool DECAY>
__global__ __launch_bounds__(NT, 2) void prefill_mfma_kernel(PrefillArgs a) {
  // Three operand buffers (the direct-load ring of the gram without RoPE; with
  // RoPE two operand buffers and the lane-private x slots), then the RoPE
  // gram's frequency slots (256 bytes a wave).
  __shared__ __attribute__((aligned(16))) bf16_t lds[3 * BUF + 512];
  const int id = blockIdx.x;
  if (id < a.gram_ids) {
    const int tpg = units_per_group(a.nb);
    const int blk = id / (8 * tpg), rem = id - blk * 8 * tpg;
    const int u = rem >> 3;
    const int g = blk * 8 + (rem & 7);
    if (g >= a.gram_groups) return;
    const int64_t iv = g % a.n_iv;
    const int q = (int)(g / a.n_iv);
    const int kp = q % a.ks;
    const int64_t s = q / a.ks;
    const int64_t t0 = iv * a.L;
    const int64_t Lc = (a.T - t0 < a.L) ? a.T - t0 : a.L;
    if (u >= a.nb * a.nb) {
      // Pair of diagonal blocks of row blocks 2j and 2j + 1.
      const int j = u - a.nb * a.nb;
      const int64_t ra = (int64_t)(2 * j) * T256 + T256 / 2;
      int64_t rb = (int64_t)(2 * j + 1) * T256 + T256 / 2;
      if (ra >= Lc) return;  // past a ragged last interval: never read
      if (2 * j + 1 >= a.nb || rb >= Lc) rb = -1;
      if (ra + T256 / 2 <= Lc && (rb < 0 || rb + T256 / 2 <= Lc))
        gram_unit<ROPE, DECAY, true, true, true>(a, lds, s, kp, iv, ra, rb);
      else
        gram_unit<ROPE, DECAY, false, true, true>(a, lds, s, kp, iv, ra, rb);
      return;
    }
    int rbk, cbk;
    tile_of(u, rbk, cbk);
    const int64_t ri = (int64_t)rbk * T256, rj = (int64_t)cbk * (T256 / 2);
    if (ri >= Lc || rj >= Lc) return;  // tile past a ragged last interval: never read
    const bool inner = rj >= ri && rj + T256 / 2 <= ri + T256;
    if (ri + T256 <= Lc) {
      if (inner) gram_unit<ROPE, DECAY, true, true>(a, lds, s, kp, iv, ri, rj);
      else gram_unit<ROPE, DECAY, true, false>(a, lds, s, kp, iv, ri, rj);
    } else {
      if (inner) gram_unit<ROPE, DECAY, false, true>(a, lds, s, kp, iv, ri, rj);
      else gram_unit<ROPE, DECAY, false, false>(a, lds, s, kp, iv, ri, rj);
    }
  } else if (id < a.gram_ids + a.rd_units) {
    // readout unit: (stream, 256-row block, 128-column block, N range), N range fastest
    int rid = id - a.gram_ids;
    const int kp = rid % a.rd_kr;
    rid /= a.rd_kr;
    const int ndb = (int)((a.D + T256 / 2 - 1) / (T256 / 2));
    const int64_t d0 = (int64_t)(rid % ndb) * (T256 / 2);
    rid /= ndb;
    const int nrb = (int)((a.rd_Lc + T256 - 1) / T256);
    const int64_t r0 = (int64_t)(rid % nrb) * T256;
    const int64_t s = rid / nrb;
    if (r0 + T256 <= a.rd_Lc) readout_unit<ROPE, DECAY, true>(a, lds, s, kp, r0, d0);
    else readout_unit<ROPE, DECAY, false>(a, lds, s, kp, r0, d0);
  } else {
    const int sid = id - a.gram_ids - a.rd_units;
    if (sid >= a.state_units) {
      if (sid - a.state_units < a.add_units) add_unit(a, sid - a.state_units);
      return;
    }
    const int nt = (int)(a.N / (T256 / 2));
    const int dt = (int)((a.D + T256 - 1) / T256);
    const int64_t s = sid / (nt * dt);
    const int rem = sid - (int)s * nt * dt;
    const int64_t n0 = (int64_t)(rem / dt) * (T256 / 2), d0 = (int64_t)(rem % dt) * T256;
    // Steps cover round_up(Lc, 64) tokens; they stay inside T unless the
    // interval is a ragged last one.
    if (a.st_t0 + ((a.st_Lc + 63) / 64) * 64 <= a.T) state_unit<ROPE, DECAY, true>(a, lds, s, n0, d0);
    else state_unit<ROPE, DECAY, false>(a, lds, s, n0, d0);
  }
}

}  // namespace

int prefill_gram_ids(int groups, int nb) {
  const int tpg = nb * nb + (nb + 1) / 2;
  return ((groups + 7) / 8) * 8 * tpg;
}

int prefill_state_units(int64_t S, int64_t N, int64_t D) {
  return (int)(S * (N / (T256 / 2)) * ((D + T256 - 1) / T256));
}

int prefill_readout_units(int64_t S, int64_t Lc, int64_t D, int kr) {
  return (int)(S * ((Lc + T256 - 1) / T256) * ((D + T256 / 2 - 1) / (T256 / 2)) * kr);
}

hipError_t launch_prefill_mfma(const PrefillArgs& a, bool rope, hipStream_t st) {
  const unsigned grid = (unsigned)(a.gram_ids + a.rd_units + a.state_units + a.add_units);
  if (grid == 0) return hipSuccess;
  const bool decay = a.decay != nullptr;
  if (rope) {
    if (decay) hipLaunchKernelGGL((prefill_mfma_kernel<true, true>), dim3(grid), dim3(NT), 0, st, a);
    else hipLaunchKernelGGL((prefill_mfma_kernel<true, false>), dim3(grid), dim3(NT), 0, st, a);
  } else {
    if (decay) hipLaunchKernelGGL((prefill_mfma_kernel<false, true>), dim3(grid), dim3(NT), 0, st, a);
    else hipLaunchKernelGGL((prefill_mfma_kernel<false, false>), dim3(grid), dim3(NT), 0, st, a);
  }
  return hipGetLastError();
}

}  // namespace bdh
