// Gram and state products of a one-interval RoPE prefill (no decay, no
// carried state in, T a multiple of 256) in 768-thread workgroups with wave
// roles, one workgroup per CU:
//   waves 0..7   MFMA waves, each a 64 x 128 block of
//                v_mfma_f32_16x16x32_bf16 accumulators; together a 256 x 256
//                output tile;
//   waves 8..11  producer waves: fetch the raw x rows (and frequencies) two
//                steps ahead into lane-private LDS slots by direct loads,
//                compute the (cos, sin) words, rotate, and write the step's
//                operand stage; the state units' v^T goes straight to the
//                stage by direct loads.
// The roles meet through per-wave progress counters in LDS (wave_wait_min):
// producers count the steps whose stage is written, MFMA waves the steps
// whose fragments they have read; no workgroup barrier follows the start.
// On each SIMD two MFMA waves' matrix work then overlaps one producer's
// rotation (VALU) instead of the phases alternating inside one wave.
//
//   gram unit   (stream, N range kp, 256-row block rb, 256-column block cb,
//               cb <= rb): the tile of sum_{n in kp} q_r[n] q_c[n], masked to
//               c < r, into the partial buffer kp [KS, S, 1, Lp, Lp] that the
//               context kernel sums.  A diagonal tile (cb = rb) loads its 256
//               rows once for both operands; the 256-row x 128-column tiles
//               of the 4-wave launch (mfma_prefill.hip) load 1536 rows per
//               stream and step where these load 1024.
//   state unit  (stream, 256-neuron block, 256-column block):
//               rho_out[n, d] = sum_t q_t[n] v_t[d]; the producers write the
//               rotated x transposed ([n][t]) into the stage.
// The closed form is the reference's (linear.rs:221-322, one interval);
// the rotation is attention.rs:488-501 as in the 4-wave launch.
#include "bdh_mfma.h"

namespace bdh {
namespace {

using namespace mfma;

constexpr int RP_MW = 8;                    // MFMA waves
constexpr int RP_PW = 4;                    // producer waves
constexpr int RP_NT = 64 * (RP_MW + RP_PW);
constexpr int RP_STAGE = 2 * T256 * BK * 2; // bytes of one stage: 512 rows of 32 bf16 (A 0..255, B 256..511)
constexpr int RP_RING = 3;                  // stages
constexpr int RP_RAW = T256 * BK * 2;       // a state unit's raw x of one step: 4 chunks x 16 B per producer lane
constexpr int RP_EP = 132;                  // epilogue staging row pitch (floats)
constexpr int RP_LDS = RP_RING * RP_STAGE + 2 * RP_RAW;
static_assert(RP_MW * 16 * RP_EP * 4 <= RP_RING * RP_STAGE, "epilogue staging fits the ring");
static_assert(RP_MW == 8 && RP_PW == 4, "the progress counters are read 8 and 4 at a time");

enum { RK_DIAG = 0, RK_OFF = 1, RK_STATE = 2 };

// acc[mi][ni] += A[arow + 16 mi] x B[brow + 16 ni]^T over one 32-deep step.
// With 3 waves a SIMD a wave has 168 registers: the 4 A fragments stay while
// the B fragments are read one ahead of their MFMAs.
__device__ __forceinline__ void mma_64x128_lean(const bf16_t* A, const bf16_t* B, int lane, int arow, int brow,
                                                floatx4 (&acc)[4][8]) {
  bf16x8 af[4], b[2];
  b[0] = frag(B, brow, lane);
#pragma unroll
  for (int mi = 0; mi < 4; ++mi) af[mi] = frag(A, arow + 16 * mi, lane);
#pragma unroll
  for (int ni = 0; ni < 8; ++ni) {
    if (ni + 1 < 8) b[(ni + 1) & 1] = frag(B, brow + 16 * (ni + 1), lane);
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) acc[mi][ni] = mfma16(af[mi], b[ni & 1], acc[mi][ni]);
  }
}

// MFMA wave of a unit of J steps: multiply each stage once the producers
// have written it, then write the block through a private LDS region.
// emit(row, col, v): row 0..63, col 0..124 (multiple of 4) of the block.
template <int KIND, class Emit>
__device__ __forceinline__ void roles_multiply(char* lds, uint32_t landed, uint32_t consumed, int J, Emit&& emit) {
  const int lane = threadIdx.x & 63, w = wave_id();
  const int wr = w >> 1, wc = w & 1;
  const int arow = 64 * wr, brow = KIND == RK_DIAG ? 128 * wc : T256 + 128 * wc;
  // A diagonal tile's blocks whose 64 rows end before their first column
  // hold nothing below the diagonal: no MFMAs, nothing written.
  const bool active = KIND != RK_DIAG || 64 * wr + 63 > 128 * wc;
  uint32_t seen = 0;
  if (!active) {
    // Keep the protocol: the step counts as read once it has landed.
    for (int j = 0; j < J; ++j) {
      wave_wait_min<4>(landed, (uint32_t)(j + 1), seen);
      wave_count_set(consumed + 4 * w, (uint32_t)(j + 1), lane);
    }
    return;
  }
  floatx4 acc[4][8];
  zero_acc(acc);
  int slot = 0;
  for (int j = 0; j < J; ++j) {
    wave_wait_min<4>(landed, (uint32_t)(j + 1), seen);
    const bf16_t* S = reinterpret_cast<const bf16_t*>(lds + slot * RP_STAGE);
    mma_64x128_lean(S, S, lane, arow, brow, acc);
    // The fragment reads have returned: the stage may be rewritten.
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    wave_count_set(consumed + 4 * w, (uint32_t)(j + 1), lane);
    slot = slot == RP_RING - 1 ? 0 : slot + 1;
  }
  // Every MFMA wave has read every stage, and the producers' last direct
  // loads (J + 1) have landed: the ring and the slots are free.
  uint32_t seen_c = 0, seen_l = seen;
  wave_wait_min<8>(consumed, (uint32_t)J, seen_c);
  wave_wait_min<4>(landed, (uint32_t)(J + 1), seen_l);
  float* E = reinterpret_cast<float*>(lds) + w * 16 * RP_EP;
#pragma unroll
  for (int mi = 0; mi < 4; ++mi) {
#pragma unroll
    for (int ni = 0; ni < 8; ++ni)
#pragma unroll
      for (int r = 0; r < 4; ++r) E[acc16_row(lane, r) * RP_EP + ni * 16 + acc16_col(lane)] = acc[mi][ni][r];
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int rr = 0; rr < 16; rr += 2) {
      const int row = rr + (lane >> 5), col = 4 * (lane & 31);
      emit(mi * 16 + row, col, *reinterpret_cast<const float4*>(&E[row * RP_EP + col]));
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  }
}

// Producer wave of a gram unit: A rows r0 .. r0 + 255, B rows r1 .. (off
// diagonal; a diagonal tile's B rows are its A rows), N steps [kb, ke).
// Lane (kc = lane & 3, rr = 16 p + lane / 4) owns chunk kc of row rr of each
// 64-row group g (g < 4: A rows, g >= 4: B rows).  Its raw x chunks and the
// step's 4 pair frequencies are loaded into registers two steps ahead (three
// register sets; the compiler places the waits), so the only LDS traffic a
// step adds to the MFMA waves' fragment reads is its stage writes.  The
// (cos, sin) words: the first group of each operand from frac(pos f), the
// next ones advanced by e(64 f), as the 4-wave gram tiles compute them.
template <int KIND>
__device__ __forceinline__ void roles_produce_gram(const PrefillArgs& a, char* lds, uint32_t landed,
                                                   uint32_t consumed, int64_t s, int kb, int ke, int64_t r0,
                                                   int64_t r1) {
  constexpr int NG = KIND == RK_OFF ? 8 : 4;
  const int lane = threadIdx.x & 63, p = wave_id() - RP_MW;
  const int kc = lane & 3, rr = 16 * p + (lane >> 2);
  const int64_t rowb = a.N * 2;
  const char* X = reinterpret_cast<const char*>(a.x + s * a.T * a.N);
  const uint32_t voff = (uint32_t)((lane >> 2) * rowb + kc * 16);
  auto gtok = [&](int g) -> int64_t { return (g < 4 ? r0 + 64 * g : r1 + 64 * (g - 4)) + 16 * p; };
  struct Raw {
    uint4 x[NG];
    float f[4];
  };
  // Step kt's raw chunks and the frequencies of its pairs 16 kt + 4 kc ..
  // (the even neurons 32 kt + 8 kc + 2 q).
  auto load = [&](Raw& r, int kt) {
#pragma unroll
    for (int g = 0; g < NG; ++g) r.x[g] = ldg16_off(X + gtok(g) * rowb + (int64_t)kt * 64, voff);
    const float* fp = a.freqs + (int64_t)kt * BK + 8 * kc;
#pragma unroll
    for (int q = 0; q < 4; ++q) r.f[q] = fp[2 * q];
  };
  const float pA = rope_pos(a, r0 + rr), pB = rope_pos(a, r1 + rr);
  const float dstep = a.fixed ? 0.0f : 64.0f;
  const int J = ke - kb;
  uint32_t seen = 0;
  int slot = 0;
  // Step j from cur; the loads of step j + 2 go to nxt2 first.
  auto step = [&](int j, const Raw& cur, Raw& nxt2) {
    const int kn = kb + j + 2 < ke ? kb + j + 2 : ke - 1;  // past the end the last step again (unused)
    load(nxt2, kn);
    float ec[4], es[4], c[4], sn[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float fe = rope_frac(dstep, cur.f[q]);
      ec[q] = __builtin_amdgcn_cosf(fe);
      es[q] = __builtin_amdgcn_sinf(fe);
    }
    // The stage of step j held step j - RP_RING: every MFMA wave has read it.
    if (j >= RP_RING) wave_wait_min<8>(consumed, (uint32_t)(j - RP_RING + 1), seen);
    bf16_t* stg = reinterpret_cast<bf16_t*>(lds + slot * RP_STAGE);
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      if (g == 0 || g == 4) {
        const float pos = g == 0 ? pA : pB;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float fr = rope_frac(pos, cur.f[q]);
          c[q] = __builtin_amdgcn_cosf(fr);
          sn[q] = __builtin_amdgcn_sinf(fr);
        }
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float nc = c[q] * ec[q] - sn[q] * es[q];
          const float ns = sn[q] * ec[q] + c[q] * es[q];
          c[q] = nc;
          sn[q] = ns;
        }
      }
      const uint4 cs = make_uint4(pack_bf16x2(c[0], sn[0]), pack_bf16x2(c[1], sn[1]), pack_bf16x2(c[2], sn[2]),
                                  pack_bf16x2(c[3], sn[3]));
      const int row = (g < 4 ? 0 : T256) + 64 * (g & 3) + rr;
      *reinterpret_cast<uint4*>(&stg[lds_off(row, kc)]) = rot8_bf16(cur.x[g], cs);
    }
    // The stage writes are done.
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    wave_count_set(landed + 4 * p, (uint32_t)(j + 1), lane);
    slot = slot == RP_RING - 1 ? 0 : slot + 1;
  };
  Raw ra, rb, rc;
  load(ra, kb);
  load(rb, kb + 1 < ke ? kb + 1 : ke - 1);
  // Whole rounds of the three sets without branches (so that the compiler's
  // waits inside the loop count exactly the loads in flight), then the rest.
  int j = 0;
  for (; j + 3 <= J; j += 3) {
    step(j, ra, rc);
    step(j + 1, rb, ra);
    step(j + 2, rc, rb);
  }
  if (j < J) step(j, ra, rc);
  if (j + 1 < J) step(j + 1, rb, ra);
  wave_count_set(landed + 4 * p, (uint32_t)(J + 1), lane);
}

// Producer wave of a state unit: neurons n0 .. n0 + 255 (stage A rows, as
// [n][t]), columns d0 .. d0 + 255 (stage B rows: v^T, direct loads), tokens
// in J steps of 32 (J even).  Lane (tp = lane & 15, oc = 4 p + lane / 16)
// owns tokens 2 tp, 2 tp + 1 of neuron octets oc and oc + 16 of each
// 128-neuron half.  The x of step j + 1 is read halfway through step j, as
// in the gram producer.
__device__ __forceinline__ void roles_produce_state(const PrefillArgs& a, char* lds, uint32_t landed,
                                                    uint32_t consumed, int64_t s, int64_t n0, int64_t d0, int J) {
  const int lane = threadIdx.x & 63, p = wave_id() - RP_MW;
  const int tp = lane & 15, oc = 4 * p + (lane >> 4);
  const int64_t b = s / a.H, h = s - b * a.H;
  const int64_t rowb = a.N * 2;
  const char* X = reinterpret_cast<const char*>(a.x + s * a.T * a.N);
  const char* VT = reinterpret_cast<const char*>(a.vt + (b * a.Hv + (a.Hv == 1 ? 0 : h)) * a.Dp * a.Tp);
  const int64_t vstep = a.Dp * 64;  // bytes of one 32-token step of v^T
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_addr(lds));
  const uint32_t raw0 = lds0 + RP_RING * RP_STAGE;
  const char* raw_l = lds + RP_RING * RP_STAGE + p * 1024 + 16 * lane;  // + slot * RP_RAW + c * 4096
  // Chunk c = 2 hh + i: token 2 tp + i, neurons n0 + 128 hh + 8 oc .. + 7.
  const uint32_t xoff0 = (uint32_t)((2 * tp) * rowb + 16 * (lane >> 4));
  const uint32_t xoff1 = xoff0 + (uint32_t)rowb;
  auto issue_x = [&](int kt, int sl) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int hh = c >> 1, i = c & 1;
      dma16(X + (int64_t)kt * BK * rowb + (n0 + 128 * hh) * 2 + 64 * p, i ? xoff1 : xoff0,
            raw0 + (uint32_t)(sl * RP_RAW + (c * 4 + p) * 1024));
    }
  };
  // v^T: 16-row block bk = p + 4 i of the stage's B rows; the lane writing
  // LDS chunk c of row r fetches global chunk c ^ ((r >> 1) & 3).
  const uint32_t vgc = (uint32_t)((lane & 3) ^ ((lane >> 3) & 3));
  const uint32_t voff = (uint32_t)((lane >> 2) * 64) + vgc * 16;
  auto issue_v = [&](int kt, int sl) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int bk = p + 4 * i;
      dma16(VT + (int64_t)kt * vstep + (d0 + 16 * bk) * 64, voff,
            lds0 + (uint32_t)(sl * RP_STAGE + (T256 + 16 * bk) * 64));
    }
  };
  struct Raw {
    uint4 x[4];
  };
  auto read_raw = [&](Raw& r, int sl) {
#pragma unroll
    for (int c = 0; c < 4; ++c) r.x[c] = *reinterpret_cast<const uint4*>(raw_l + sl * RP_RAW + c * 4096);
  };
  // The (cos, sin) words come from the phase of each token (as the 4-wave
  // state units compute them), so a state carried across calls is the same
  // bit for bit whichever launch computed it.
  float fq[2][4];
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) load_freq4(a.freqs + n0 + 128 * hh + 8 * oc, fq[hh]);
  const float pbase = rope_pos(a, 0);
  __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): the frequencies are in
  issue_x(0, 0);
  issue_x(1 < J ? 1 : J - 1, 1);
  asm volatile("s_waitcnt vmcnt(4)" ::: "memory");  // step 0's x landed
  Raw ra, rb;
  read_raw(ra, 0);
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  uint32_t seen = 0;
  auto step = [&](int j, const Raw& cur, Raw& nxt) {
    const int sl = j & 1, rs = j % RP_RING;
    // The stage of step j held step j - RP_RING: every MFMA wave has read it.
    if (j >= RP_RING) wave_wait_min<8>(consumed, (uint32_t)(j - RP_RING + 1), seen);
    issue_v(j, rs);
    issue_x(j + 2 < J ? j + 2 : J - 1, sl);  // raw slot sl was read during step j - 1
    // Tokens of this step (positions exact in f32 below 2^24).
    const float p0 = a.fixed ? pbase : pbase + (float)(32 * j + 2 * tp);
    const float p1 = a.fixed ? pbase : p0 + 1.0f;
    uint32_t* Aw = reinterpret_cast<uint32_t*>(lds + rs * RP_STAGE);
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      float f0[8], f1[8];
      rot8_f32(cur.x[2 * hh], rope_cs4(p0, fq[hh]), f0);
      rot8_f32(cur.x[2 * hh + 1], rope_cs4(p1, fq[hh]), f1);
#pragma unroll
      for (int e = 0; e < 8; ++e)
        Aw[(lds_off(128 * hh + 8 * oc + e, tp >> 2) + 2 * (tp & 3)) >> 1] = pack_bf16x2(f0[e], f1[e]);
      if (hh == 0) {
        // Step j + 1's x has landed once only step j's v^T and step j + 2's x
        // are in flight.
        asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
        read_raw(nxt, sl ^ 1);
      }
    }
    // Step j's v^T has landed once only step j + 2's x is in flight; the
    // stage writes and the next step's x reads are done.
    asm volatile("s_waitcnt vmcnt(4)\n\ts_waitcnt lgkmcnt(0)" ::: "memory");
    wave_count_set(landed + 4 * p, (uint32_t)(j + 1), lane);
  };
  for (int j = 0; j < J; j += 2) {
    step(j, ra, rb);
    step(j + 1, rb, ra);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  wave_count_set(landed + 4 * p, (uint32_t)(J + 1), lane);
}

// Gram ids: groups (stream, N range) in blocks of 8; inside a block id =
// unit * 8 + (group & 7), so the tiles of one group (which read the same x
// rows) run on one XCD (workgroup id i runs on XCD i % 8).  Units: the
// nb (nb - 1) / 2 off-diagonal tiles first (the heavier), then the nb
// diagonal ones.  State units follow the gram ids.
__global__ __launch_bounds__(RP_NT, 1) void prefill_roles_kernel(PrefillArgs a) {
  __shared__ __attribute__((aligned(16))) char lds[RP_LDS];
  // [0, 4) steps written, per producer wave; [4, 12) steps read, per MFMA wave.
  __shared__ __attribute__((aligned(16))) uint32_t counts[12];
  if (threadIdx.x < 12) counts[threadIdx.x] = 0;
  __syncthreads();
  const uint32_t landed = lds_addr(&counts[0]), consumed = lds_addr(&counts[4]);
  const bool producer = wave_id() >= RP_MW;
  const int id = blockIdx.x;
  if (id < a.gram_ids) {
    const int noff = a.nb * (a.nb - 1) / 2, tpg = noff + a.nb;
    const int blk = id / (8 * tpg), rem = id - blk * 8 * tpg;
    const int u = rem >> 3, g = blk * 8 + (rem & 7);
    if (g >= a.gram_groups) return;
    const int kp = g % a.ks;
    const int64_t s = g / a.ks;
    const int nk = (int)(a.N / BK);
    const int kb = (int)((int64_t)nk * kp / a.ks), ke = (int)((int64_t)nk * (kp + 1) / a.ks);
    float* P = a.part + ((int64_t)kp * a.S + s) * a.Lp * a.Lp;
    int rb, cb;
    if (u < noff) {
      rb = 1;
      while (rb * (rb + 1) / 2 <= u) ++rb;
      cb = u - rb * (rb - 1) / 2;
    } else {
      rb = cb = u - noff;
    }
    const int64_t r0 = (int64_t)rb * T256, r1 = (int64_t)cb * T256, Lp = a.Lp;
    // Scores (ti, tj): kept below the diagonal, 0 on and above it.
    auto emit = [=](int wr, int wc) {
      return [=](int row, int col, float4 v) {
        const int64_t ti = r0 + 64 * wr + row, tj = r1 + 128 * wc + col;
        const floatx4 e{tj < ti ? v.x : 0.0f, tj + 1 < ti ? v.y : 0.0f, tj + 2 < ti ? v.z : 0.0f,
                        tj + 3 < ti ? v.w : 0.0f};
        // Streaming stores: read once, by the context kernel.
        __builtin_nontemporal_store(e, reinterpret_cast<floatx4*>(P + ti * Lp + tj));
      };
    };
    const int w = wave_id();
    if (rb != cb) {
      if (producer) roles_produce_gram<RK_OFF>(a, lds, landed, consumed, s, kb, ke, r0, r1);
      else roles_multiply<RK_OFF>(lds, landed, consumed, ke - kb, emit(w >> 1, w & 1));
    } else {
      if (producer) roles_produce_gram<RK_DIAG>(a, lds, landed, consumed, s, kb, ke, r0, r0);
      else roles_multiply<RK_DIAG>(lds, landed, consumed, ke - kb, emit(w >> 1, w & 1));
    }
    return;
  }
  const int sid = id - a.gram_ids;
  if (sid >= a.state_units) return;
  const int nt = (int)(a.N / T256), dt = (int)(a.Dp / T256);
  const int64_t s = sid / (nt * dt);
  const int rem = sid - (int)s * nt * dt;
  const int64_t n0 = (int64_t)(rem / dt) * T256, d0 = (int64_t)(rem % dt) * T256;
  const int J = (int)(a.T / BK);
  if (producer) {
    roles_produce_state(a, lds, landed, consumed, s, n0, d0, J);
    return;
  }
  const int w = wave_id(), wr = w >> 1, wc = w & 1;
  roles_multiply<RK_STATE>(lds, landed, consumed, J, [&](int row, int col, float4 v) {
    const int64_t n = n0 + 64 * wr + row, d = d0 + 128 * wc + col;
    if (d >= a.D) return;
    float* dst = a.rho_out + (s * a.N + n) * a.D + d;
    // The caller's final state is not read again here.
    if (a.rho_stream) __builtin_nontemporal_store(floatx4{v.x, v.y, v.z, v.w}, reinterpret_cast<floatx4*>(dst));
    else *reinterpret_cast<float4*>(dst) = v;
  });
}

}  // namespace

bool prefill_roles_fits(const PrefillArgs& a) {
  return a.n_iv == 1 && a.freqs != nullptr && a.decay == nullptr && a.rho_in == nullptr && a.T % T256 == 0 &&
         a.N % T256 == 0 && a.Dp % T256 == 0 && (a.N / BK) % (2 * a.ks) == 0;
}

int prefill_roles_gram_ids(int groups, int nb) {
  const int tpg = nb * (nb - 1) / 2 + nb;
  return ((groups + 7) / 8) * 8 * tpg;
}

int prefill_roles_state_units(int64_t S, int64_t N, int64_t Dp) { return (int)(S * (N / T256) * (Dp / T256)); }

hipError_t launch_prefill_roles(const PrefillArgs& a, hipStream_t st) {
  const unsigned grid = (unsigned)(a.gram_ids + a.state_units);
  if (grid == 0) return hipSuccess;
  hipLaunchKernelGGL(prefill_roles_kernel, dim3(grid), dim3(RP_NT), 0, st, a);
  return hipGetLastError();
}

}  // namespace bdh
