// BDH low-rank layer body around the recurrent attention, bf16 MFMA with
// fp32 accumulation (residual_stream.rs:323-572, vanilla options: no ReLU
// threshold, no sparse latent mask, dropout off at inference):
//
//   x    = ReLU(cur E_h)                 [B, H, T, N]   (GEMM X, which also
//                                                         writes q = rope(x))
//   a    = LN(attn(q, v = cur))          [B, H, T, D]   (prefill_bf16.hip, ln_rows)
//   y    = ReLU(a Ev_h) * x              [B, H, T, N]   (GEMM Y, written over x)
//   z    = y' Dec, y' = [B*T, H*N]       [B, T, D]      (GEMM Z, split-K partials;
//                                                         with T % 256 == 0 and D <= 256
//                                                         one launch computes y tile by
//                                                         tile and never stores it)
//   next = LN(cur + LN(z))               [B, T, D]      (residual_kernel)
//
// LN is DragonNorm's LayerNorm arm with gamma = 1, beta = 0, eps = 1e-5 and
// the biased variance (norm.rs:302-328).  The three GEMMs share the
// 256 x 128 MFMA tile of the prefill units (bdh_mfma.h); their operands are
// K-contiguous bf16 rows: cur and the LN'd attention rows (K = D), the
// packed weights (encoders [H, N, D], decoder [D, H*N]) and y (K = H*N,
// contiguous inside a head's N).
#include "bdh_mfma.h"

namespace bdh {
namespace {

using namespace mfma;

enum { G_X = 0, G_Y = 1, G_Z = 2, G_L = 3 };

// The packed decoder is chunk-major, [H N / 128, D, 128]: the transpose
// [D, H N] cut into 128-latent chunks, each a contiguous 64 KiB block at
// D = 256.  The decoder products read one 32-latent step of D rows at a
// time: with the plain transpose those rows lie 64 KiB apart (C5), the same
// L2 sets for every row, and the fused Y + Z launch fetched 3.8 GB past L2
// for 1.1 GB of operands.  Element (d, k) of the transpose:
__host__ __device__ constexpr int64_t dec_off(int64_t d, int64_t k, int64_t D) {
  return (k / 128) * D * 128 + d * 128 + (k % 128);
}

typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

struct LayerGemmArgs {
  const bf16_t* a;    // X, L: rows [M, D]; Y: LN'd attention [B, H, T, D]; Z: y [B, H, T, N]
  const bf16_t* b;    // X: encoder [H*N, D]; Y: encoder_v [H*N, D]; Z: decoder [D, H*N];
                      // L: lm_head [V, D]
  bf16_t* xy;         // X: x out; Y: x in, y out (same place); [B, H, T, N]
  bf16_t* q;          // X: rope(x) out [B, H, T, N], or null (no rotation)
  float* xf;          // X: x out in f32 [B, H, T, N], or null
  const float* freqs; // X: RoPE frequencies [N] (with q)
  int64_t pos0;       // X: position of token 0
  int fixed;          // X: every token at pos0
  float* zpart;       // Z: partials [ks, M, D]; L: logits [M, V]
  int64_t B, H, T, N, D, M;  // M = B * T
  int64_t V;          // L: vocabulary
  int mt, ct, ks;     // tiles along M and along the output columns; Z: K splits
  float relu_th;      // X, Y: ReLU threshold (subtracted before the ReLU)
  const float* mask;  // X, Y: latent mask [N] (times the ReLU), or null (ones)
  const bf16_t* dec;  // Y fused into Z (layer_yz_kernel): decoder [D, H*N]
};

// The activation of the reference's low-rank projection (relu_lowrank.rs
// reference_forward, kernel/relu_lowrank.rs:100-135): subtract the
// threshold, ReLU, times the latent mask.
__device__ __forceinline__ float lowrank_act(float v, float th, float m) { return fmaxf(v - th, 0.0f) * m; }

// One output tile.  Tile id -> (row tile, column tile, K split).  X and Y
// (whose launches are mostly their [B, H, T, N] stores): column tiles
// fastest, so workgroups side by side write neighbouring 256-byte pieces of
// the same rows (C5: GEMM X 738 -> 655 us, Y unchanged, against row tiles
// fastest, where they wrote one piece each of rows 16 KB apart).  Z and L: row tiles
// fastest, so the row tiles that share a column tile's B rows run side by
// side.
template <int KIND>
__device__ __forceinline__ void gemm_tile(const LayerGemmArgs& g, bf16_t* lds, int id) {
  const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
  int mtile, ctile, kp = 0;
  if (KIND == G_X || KIND == G_Y) {
    ctile = id % g.ct;
    mtile = id / g.ct;
  } else {
    mtile = id % g.mt;
    id /= g.mt;
    ctile = id % g.ct;
    kp = id / g.ct;
  }
  const int64_t m0 = (int64_t)mtile * T256, c0 = (int64_t)ctile * (T256 / 2);
  const int64_t K = KIND == G_Z ? g.H * g.N : g.D;
  const int nk = (int)(K / BK);
  const int kb = KIND == G_Z ? (int)((int64_t)nk * kp / g.ks) : 0;
  const int ke = KIND == G_Z ? (int)((int64_t)nk * (kp + 1) / g.ks) : nk;
  const int64_t h = (KIND == G_X || KIND == G_Y) ? c0 / g.N : 0;  // head of the column tile
  const int64_t ncols = KIND == G_Z ? g.D : KIND == G_L ? g.V : g.H * g.N;

  // Loader: 4 lanes per 64-byte row segment; groups 0..3 are A rows
  // m0 + rb + 64 g, groups 4 and 5 are B rows c0 + rb + 64 (g - 4).  Rows
  // past M (or past D for Z's B rows) re-read the last row and are never
  // stored.
  const int kc = tid & 3, rb = tid >> 2;
  const bf16_t* arow[4];
  const bf16_t* brow[2];
#pragma unroll
  for (int gi = 0; gi < 4; ++gi) {
    int64_t m = m0 + rb + 64 * gi;
    m = m < g.M ? m : g.M - 1;
    const int64_t bb = m / g.T, t = m - bb * g.T;
    if (KIND == G_X || KIND == G_L) arow[gi] = g.a + m * g.D;
    else if (KIND == G_Y) arow[gi] = g.a + ((bb * g.H + h) * g.T + t) * g.D;
    else arow[gi] = g.a + (bb * g.H * g.T + t) * g.N;
    arow[gi] += kc * 8;
  }
#pragma unroll
  for (int gi = 0; gi < 2; ++gi) {
    int64_t c = c0 + rb + 64 * gi;
    c = c < ncols ? c : ncols - 1;
    brow[gi] = g.b + (KIND == G_Z ? c * 128 : c * K) + kc * 8;
  }
  uint4 st[6];
  auto load = [&](int kt) {
    const int64_t k0 = (int64_t)kt * BK;
    // Z: k runs over (head, neuron); a 32-deep step stays inside one head.
    const int64_t aoff = KIND == G_Z ? (k0 / g.N) * g.T * g.N + k0 % g.N : k0;
#pragma unroll
    for (int gi = 0; gi < 4; ++gi) st[gi] = ldg16(arow[gi] + aoff);
#pragma unroll
    for (int gi = 0; gi < 2; ++gi) st[4 + gi] = ldg16(brow[gi] + (KIND == G_Z ? dec_off(0, k0, g.D) : k0));
  };
  auto store = [&](int buf) {
    bf16_t* base = lds + buf * BUF;  // A rows 0..255, then B rows 256..383
#pragma unroll
    for (int gi = 0; gi < 6; ++gi) *reinterpret_cast<uint4*>(&base[lds_off(64 * gi + rb, kc)]) = st[gi];
  };

  floatx4 acc[4][8];
  zero_acc(acc);
  run_steps(kb, ke, load, store, [&](int buf) {
    mma_64x128(lds + buf * BUF, lds + buf * BUF, lane, 64 * w, T256, acc);
  });

  if (KIND == G_Y) {
    // As epilogue8_64x128 (8 columns per lane: 16-byte x reads and y
    // stores), with the 4 x reads of a 16-row slice issued before any y
    // store: y overwrites x in place, so the compiler could not move one
    // row's load above another row's store, and each read would be a round
    // trip of its own.
    constexpr int EP = 132;
    float* E = reinterpret_cast<float*>(lds) + w * 16 * EP;
    const int col = 8 * (lane & 15);
    const int64_t c = c0 + col, n = c - h * g.N;
    float mk[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) mk[j] = g.mask ? g.mask[n + j] : 1.0f;
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) {
#pragma unroll
      for (int ni = 0; ni < 8; ++ni)
#pragma unroll
        for (int r = 0; r < 4; ++r) E[acc16_row(lane, r) * EP + ni * 16 + acc16_col(lane)] = acc[mi][ni][r];
      __syncthreads();
      bf16_t* dst[4];
      uint4 xv[4];
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        int64_t m = m0 + 64 * w + mi * 16 + 4 * rr + (lane >> 4);
        m = m < g.M ? m : g.M - 1;  // rows past M re-read the last row, never stored
        const int64_t bb = m / g.T, t = m - bb * g.T;
        dst[rr] = g.xy + ((bb * g.H + h) * g.T + t) * g.N + n;
        xv[rr] = *reinterpret_cast<const uint4*>(dst[rr]);
      }
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int row = 4 * rr + (lane >> 4);
        const float4 lo = *reinterpret_cast<const float4*>(&E[row * EP + col]);
        const float4 hi = *reinterpret_cast<const float4*>(&E[row * EP + col + 4]);
        const uint32_t xw[4] = {xv[rr].x, xv[rr].y, xv[rr].z, xv[rr].w};
        const float a[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
        uint32_t yw[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          yw[j] = pack_bf16x2(lowrank_act(a[2 * j], g.relu_th, mk[2 * j]) * bf16_lo(xw[j]),
                              lowrank_act(a[2 * j + 1], g.relu_th, mk[2 * j + 1]) * bf16_hi(xw[j]));
        if (m0 + 64 * w + mi * 16 + row < g.M)
          *reinterpret_cast<uint4*>(dst[rr]) = make_uint4(yw[0], yw[1], yw[2], yw[3]);
      }
      __syncthreads();
    }
    return;
  }

  if (KIND == G_X) {
    // x = ReLU(acc) and q = rope(x): 8 columns per lane and call, one 16-byte
    // streaming store each (GBs at C5, read back only by later launches).  A
    // lane's columns (pairs (n, n+1) .. (n+6, n+7)) are the same in every
    // call, so their frequencies are loaded once per tile.
    float fq[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    const int64_t n0 = c0 + 8 * (lane & 15) - h * g.N;
    if (g.q) {
#pragma unroll
      for (int j = 0; j < 4; ++j) fq[j] = g.freqs[n0 + 2 * j];
    }
    float mk[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) mk[j] = g.mask ? g.mask[n0 + j] : 1.0f;
    epilogue8_64x128(acc, lds, w, lane, [&](int row, int col, float4 lo, float4 hi) {
      const int64_t m = m0 + 64 * w + row, c = c0 + col;
      if (m >= g.M) return;
      const int64_t bb = m / g.T, t = m - bb * g.T, n = c - h * g.N;
      const int64_t o = ((bb * g.H + h) * g.T + t) * g.N + n;
      const float th = g.relu_th;
      const float r[8] = {lowrank_act(lo.x, th, mk[0]), lowrank_act(lo.y, th, mk[1]), lowrank_act(lo.z, th, mk[2]),
                          lowrank_act(lo.w, th, mk[3]), lowrank_act(hi.x, th, mk[4]), lowrank_act(hi.y, th, mk[5]),
                          lowrank_act(hi.z, th, mk[6]), lowrank_act(hi.w, th, mk[7])};
      __builtin_nontemporal_store(u32x4{pack_bf16x2(r[0], r[1]), pack_bf16x2(r[2], r[3]),
                                        pack_bf16x2(r[4], r[5]), pack_bf16x2(r[6], r[7])},
                                  reinterpret_cast<u32x4*>(g.xy + o));
      if (g.xf) {
        *reinterpret_cast<float4*>(g.xf + o) = make_float4(r[0], r[1], r[2], r[3]);
        *reinterpret_cast<float4*>(g.xf + o + 4) = make_float4(r[4], r[5], r[6], r[7]);
      }
      if (g.q) {
        // Phase frac(p f) in the reference's f32 op order, cos / sin by
        // v_cos_f32 / v_sin_f32 (argument in revolutions); the rotation in
        // the op order of attention.rs:488-501.
        const float p = (float)(g.fixed ? g.pos0 : g.pos0 + t);
        float qv[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float fr = rope_frac(p, fq[j]);
          rope_pair_exact(r[2 * j], r[2 * j + 1], __builtin_amdgcn_cosf(fr), __builtin_amdgcn_sinf(fr),
                          qv[2 * j], qv[2 * j + 1]);
        }
        __builtin_nontemporal_store(u32x4{pack_bf16x2(qv[0], qv[1]), pack_bf16x2(qv[2], qv[3]),
                                          pack_bf16x2(qv[4], qv[5]), pack_bf16x2(qv[6], qv[7])},
                                    reinterpret_cast<u32x4*>(g.q + o));
      }
    });
    return;
  }

  epilogue_64x128(acc, lds, w, lane, [&](int row, int col, float4 v) {
    const int64_t m = m0 + 64 * w + row, c = c0 + col;
    if (m >= g.M) return;
    if (KIND == G_Z) {
      if (c < g.D) *reinterpret_cast<float4*>(&g.zpart[((int64_t)kp * g.M + m) * g.D + c]) = v;
      return;
    }
    // KIND == G_L: logits
    float* dst = g.zpart + m * g.V + c;
    if (c + 3 < g.V && (g.V & 3) == 0) {
      *reinterpret_cast<float4*>(dst) = v;
    } else {
      const float e[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (c + j < g.V) dst[j] = e[j];
    }
  });
}

// Persistent: each workgroup walks tiles blockIdx.x, + gridDim.x, ...; a
// tile's epilogue stores drain while the next tile's loads and MFMAs run.
template <int KIND>
__global__ __launch_bounds__(NT, 2) void layer_gemm_kernel(LayerGemmArgs g) {
  __shared__ __attribute__((aligned(16))) bf16_t lds[2 * BUF];
  const int total = g.mt * g.ct * (KIND == G_Z ? g.ks : 1);
  for (int id = blockIdx.x; id < total; id += gridDim.x) gemm_tile<KIND>(g, lds, id);
}

// ---- GEMM X in wave roles -------------------------------------------------
// x = act(cur E_h) and q = rope(x) are 2 GB of stores per C5 layer against
// 24 MB of operands: the launch is a write stream.  In layer_gemm_kernel a
// tile's K loop waits for its loads with the one counter that also counts
// the previous tile's stores (gfx9 has no separate store counter), so every
// tile first drains 128 KB of stores.  Here one 1024-thread workgroup per CU
// splits the work by wave, and no wave both loads and stores:
//   waves 0-3 (MFMA): multiply each 32-deep step of the cur tile, taken from
//     a 3-slot LDS ring, with the workgroup's 128-latent encoder chunk, which
//     stays in LDS for all its tiles; per 128 x 128 tile they write act(x)
//     in f32 to a staging tile.  No global memory access at all (the
//     optional latent mask aside).
//   waves 4-7 (DMA): fetch the encoder chunk once and then each step's cur
//     rows straight into the ring (global_load_lds_dwordx4), waiting only
//     for their own DMAs.
//   waves 8-15 (store): per tile, read the staging tile, form x in bf16 and
//     q = rope(x) (the f32 rotation in the reference's op order) and store
//     both, 16 bytes a lane.
// The waves hand work over through per-wave progress counters in LDS, not
// workgroup barriers: steps landed (per DMA wave), steps read (per MFMA
// wave), tiles staged (per MFMA wave), tiles read from staging (per store
// wave).  A DMA wave refills a ring slot once every MFMA wave has read it;
// an MFMA wave multiplies a step once every DMA wave has landed it, and
// writes a tile's staging once every store wave has read the previous one;
// a store wave reads a tile once every MFMA wave has staged it
// (tests/test_x_roles_protocol.py models the protocol on the CPU: random
// interleavings finish with no slot or staging part read stale).
// The product is computed transposed, E_chunk cur^T, so each accumulator
// register of a lane holds 4 consecutive latents of one token.  The
// workgroup owns one column tile (latent chunk) and walks the row tiles in
// order, so at any time the workgroups write neighbouring 256-byte pieces of
// the same rows.  Needs T % 128 == 0, N % 128 == 0, 64 <= D <= 256 with
// D % 32 == 0, and at most one column tile per CU (C5: 256 column tiles on
// 256 CUs).  Measured at C5 (GEMM X of layer_gemm_kernel: 688 us): 766 us
// with 4 MFMA waves that also issued the DMAs, 4 store waves and a barrier
// per K step (the store waves held the barriers); 620 us with 8 store waves
// and no 64-bit divisions in the loops; 601 us with 8 MFMA waves meeting
// through an LDS counter and the store waves free between tiles; 540 us
// with the DMAs in waves of their own; 520 us with polls skipped where an
// earlier read already showed the step; 512 us with counters instead of the
// two workgroup barriers per tile that all waves passed before.  An
// s_memtime trace at 512 us: a K step ~920 cycles for an MFMA wave (16
// MFMAs and their fragment reads ~540, the counter poll ~220), a tile ~9.2 k
// cycles, the store waves idle about half of it.  Slower, not kept: the poll issued with the step's
// fragment reads, the MFMAs after all of them (538 us); the DMA waves
// passing the tile barriers right after the next tile's first step had
// landed (vmcnt(0) there; 576 us with both); the landed counters read behind
// each step's MFMAs for the next step (523 us: the DMA waves, one step
// ahead, had rarely signalled it by then); 8 MFMA waves (64 x 32 blocks, two
// a SIMD) with 4 store waves (535 us).  Reading each step's fragments
// behind the previous step's MFMAs needs a second fragment set: with 4
// store waves (12 waves, 168 VGPRs) the MFMA waves spilled 157 registers,
// among them fragment registers stored to scratch before their read had
// completed (tests/asm_waits.py reports exactly that); not run.
constexpr int XR_T = 128;                      // tile edge (tokens and latents)
constexpr int XR_EBLK = XR_T * BK * 2;         // bytes of one 32-deep block of 128 rows
constexpr int XR_EMAX = (T256 / BK) * XR_EBLK; // encoder chunk, D <= 256
constexpr int XR_RING = 3;
constexpr int XR_STG = XR_T * XR_T * 4;        // f32 staging tile
constexpr int XR_MW = 4;                       // MFMA waves
constexpr int XR_DW = 4;                       // DMA waves
constexpr int XR_SW = 8;                       // store waves
static_assert(XR_MW == 4 && XR_DW == 4, "the progress counters are read 4 at a time");
constexpr int XR_PC = 32 / XR_SW;              // 16-byte pieces of x (and of q) a store lane writes per tile
constexpr int XR_LDS = XR_EMAX + XR_RING * XR_EBLK + XR_STG;

// acc[mi][ni] += A[arow + 16 mi] x B[brow + 16 ni]^T over one 32-deep step
// (4 x 2 MFMA blocks), fragment reads in assembly as mma_64x64_dsasm.
__device__ __forceinline__ void mma_64x32_dsasm(const bf16_t* A, const bf16_t* B, int lane, int arow, int brow,
                                                floatx4 (&acc)[4][2]) {
  typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
  const uint32_t a = lds_addr(A) + (uint32_t)(2 * lds_off(arow + (lane & 15), lane >> 4));
  const uint32_t b = lds_addr(B) + (uint32_t)(2 * lds_off(brow + (lane & 15), lane >> 4));
  u32x4_t af[4], bf[2];
  asm volatile("ds_read_b128 %0, %1 offset:0" : "=v"(bf[0]) : "v"(b));
  asm volatile("ds_read_b128 %0, %1 offset:1024" : "=v"(bf[1]) : "v"(b));
  asm volatile("ds_read_b128 %0, %1 offset:0" : "=v"(af[0]) : "v"(a));
  asm volatile("ds_read_b128 %0, %1 offset:1024" : "=v"(af[1]) : "v"(a));
  asm volatile("ds_read_b128 %0, %1 offset:2048" : "=v"(af[2]) : "v"(a));
  asm volatile("ds_read_b128 %0, %1 offset:3072" : "=v"(af[3]) : "v"(a));
  auto mm = [&](int mi, int ni) {
    acc[mi][ni] = mfma16(__builtin_bit_cast(bf16x8, af[mi]), __builtin_bit_cast(bf16x8, bf[ni]), acc[mi][ni]);
  };
  asm volatile("s_waitcnt lgkmcnt(3)" : "+v"(bf[0]), "+v"(bf[1]), "+v"(af[0]));
  mm(0, 0);
  mm(0, 1);
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(af[1]), "+v"(af[2]), "+v"(af[3]));
#pragma unroll
  for (int mi = 1; mi < 4; ++mi) {
    mm(mi, 0);
    mm(mi, 1);
  }
}

// Byte offset of f32 staging element (t, n): 16-byte chunk n / 4 of the
// 512-byte row t stored at chunk (n / 4) ^ (t & 15), so the MFMA waves' 16
// rows a write and the store waves' rows fall on distinct banks.
__device__ __forceinline__ uint32_t xr_stg(int t, int n) {
  return (uint32_t)(t * 512 + ((((n >> 2) ^ (t & 15))) << 4) + 4 * (n & 3));
}

template <bool PLAIN>
__global__ __launch_bounds__(64 * (XR_MW + XR_DW + XR_SW), 1) void layer_x_roles_kernel(LayerGemmArgs g, int rg_count) {
  __shared__ __attribute__((aligned(16))) char lds[XR_LDS];
  // Progress counters, each written by one wave: [0, 4) K steps landed, per
  // DMA wave; [4, 8) K steps read, per MFMA wave; [8, 12) tiles staged, per
  // MFMA wave; [12, 20) tiles read from staging, per store wave.
  __shared__ __attribute__((aligned(16))) uint32_t counts[20];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  if (tid < 20) counts[tid] = 0;
  __syncthreads();
  const int ct = (int)(g.H * g.N / XR_T), mt = (int)(g.M / XR_T);
  const int ctile = (int)blockIdx.x % ct, rg = (int)blockIdx.x / ct;
  const int ntile = (mt - rg + rg_count - 1) / rg_count;  // row tiles rg, rg + rg_count, ...
  const int nk = (int)(g.D / BK);
  const int J = ntile * nk;  // K steps of the workgroup
  const int64_t c0 = (int64_t)ctile * XR_T, h = c0 / g.N, n0 = c0 - h * g.N;
  char* const E = lds;
  char* const ring = lds + XR_EMAX;
  char* const stg = lds + XR_EMAX + XR_RING * XR_EBLK;
  const int gq = lane >> 4, li = lane & 15;
  const uint32_t landed = lds_addr(&counts[0]), consumed = lds_addr(&counts[4]);
  const uint32_t staged = lds_addr(&counts[8]), freed = lds_addr(&counts[12]);

  if (w < XR_MW) {
    // ---- MFMA waves: wave w owns latents 64 (w / 2) .. + 63 and tokens
    // 64 (w % 2) .. + 63 of the tile ----
    const int wm = w >> 1, wt = w & 1;
    float mk[4][4];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
      for (int r = 0; r < 4; ++r) mk[mi][r] = (!PLAIN && g.mask) ? g.mask[n0 + 64 * wm + 16 * mi + 4 * gq + r] : 1.0f;
    const float th = g.relu_th;
    floatx4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = zero4();
    int slot = 0, tile = 0;
    uint32_t seen = 0, seen_freed = 0;
    for (int j = 0, sk = 0; j < J; ++j) {
      // Step j (and, before step 0, the encoder chunk) has landed.
      wave_wait_min<4>(landed, (uint32_t)(j + 1), seen);
      mma_64x64_dsasm(reinterpret_cast<const bf16_t*>(E + sk * XR_EBLK),
                      reinterpret_cast<const bf16_t*>(ring + slot * XR_EBLK), lane, 64 * wm, 64 * wt, acc);
      // The fragment reads are complete (waited inside): the slot is free.
      wave_count_set(consumed + 4 * w, (uint32_t)(j + 1), lane);
      slot = slot == XR_RING - 1 ? 0 : slot + 1;
      if (++sk == nk) {
        sk = 0;
        // The store waves have read the previous tile's staging.
        wave_wait_min<8>(freed, (uint32_t)tile, seen_freed);
        // The tile's act(x), f32, into the staging tile: block (mi, ni),
        // register r is latent 64 wm + 16 mi + 4 gq + r of token
        // 64 wt + 16 ni + li.
#pragma unroll
        for (int mi = 0; mi < 4; ++mi)
#pragma unroll
          for (int ni = 0; ni < 4; ++ni) {
            const int t = 64 * wt + 16 * ni + li, n = 64 * wm + 16 * mi + 4 * gq;
            float4 v;
            if (PLAIN) {
              v = make_float4(fmaxf(acc[mi][ni][0], 0.0f), fmaxf(acc[mi][ni][1], 0.0f), fmaxf(acc[mi][ni][2], 0.0f),
                              fmaxf(acc[mi][ni][3], 0.0f));
            } else {
              v = make_float4(lowrank_act(acc[mi][ni][0], th, mk[mi][0]), lowrank_act(acc[mi][ni][1], th, mk[mi][1]),
                              lowrank_act(acc[mi][ni][2], th, mk[mi][2]), lowrank_act(acc[mi][ni][3], th, mk[mi][3]));
            }
            *reinterpret_cast<float4*>(stg + xr_stg(t, n)) = v;
            acc[mi][ni] = zero4();
          }
        // The staging writes are done (LDS order), then the tile is staged.
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        wave_count_set(staged + 4 * w, (uint32_t)(++tile), lane);
      }
    }
    return;
  }

  if (w < XR_MW + XR_DW) {
    // ---- DMA waves: wave dw issues instructions dw and dw + 4 of each
    // step's 8 (cur rows 16 i .. 16 i + 15) ----
    const int dw = w - XR_MW;
    const uint32_t lE = lds_addr(E), lR = lds_addr(ring);
    // Instruction i of a 128-row block covers rows 16 i .. 16 i + 15, lane l
    // row 16 i + l / 4, LDS chunk l & 3 = global chunk (l & 3) ^ ((row >> 1)
    // & 3) (the lds_off swizzle).
    auto src = [&](int i) {
      const int r = 16 * i + (lane >> 2);
      const int c = (lane & 3) ^ ((r >> 1) & 3);
      return (uint32_t)(r * g.D * 2 + c * 16);
    };
    const bf16_t* Eg = g.b + c0 * g.D;
    for (int idx = dw; idx < nk * 8; idx += XR_DW) {
      const int sblk = idx >> 3, i = idx & 7;
      dma16(Eg, src(i) + (uint32_t)(sblk * 64), lE + (uint32_t)(sblk * XR_EBLK + i * 1024));
    }
    const uint32_t cs0 = src(dw), cs1 = src(dw + XR_DW);
    const bf16_t* cg = g.a + (int64_t)rg * XR_T * g.D;
    const int64_t cstep = (int64_t)rg_count * XR_T * g.D;
    int sk = 0, slot = 0;
    uint32_t seen = 0;
    for (int j = 0; j < J; ++j) {
      // Slot j % 3 held step j - 3: free once every MFMA wave has read it.
      if (j >= XR_RING) wave_wait_min<4>(consumed, (uint32_t)(j - XR_RING + 1), seen);
      const uint32_t d = lR + (uint32_t)(slot * XR_EBLK);
      dma16(cg, cs0 + (uint32_t)(sk * 64), d + (uint32_t)(dw * 1024));
      dma16(cg, cs1 + (uint32_t)(sk * 64), d + (uint32_t)((dw + XR_DW) * 1024));
      slot = slot == XR_RING - 1 ? 0 : slot + 1;
      if (++sk == nk) {
        sk = 0;
        cg += cstep;
      }
      // Step j - 1 (this wave's part; with step 0 the encoder chunk) has
      // landed once only step j's 2 DMAs are in flight.
      if (j > 0) {
        asm volatile("s_waitcnt vmcnt(2)" ::: "memory");
        wave_count_set(landed + 4 * dw, (uint32_t)j, lane);
      }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    wave_count_set(landed + 4 * dw, (uint32_t)J, lane);  // step J - 1
    return;
  }

  // ---- store waves ----
  const int sw = w - XR_MW - XR_DW;
  // Piece u (0 .. XR_PC - 1) of a tile: token row (128 / XR_SW) sw + 4 u + gq,
  // latents 8 li .. 8 li + 7.
  float fq[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (g.q) {
#pragma unroll
    for (int j = 0; j < 4; ++j) fq[j] = g.freqs[n0 + 8 * li + 2 * j];
  }
  int64_t obase = 0, pbase = 0;  // of the staged tile: offset of its token 0, that token's position
  auto store_piece = [&](int u) {
    const int tl = (XR_T / XR_SW) * sw + 4 * u + gq;
    const int64_t o = obase + (int64_t)tl * g.N;
    const int64_t t = pbase + tl;
    const float4 lo = *reinterpret_cast<const float4*>(stg + xr_stg(tl, 8 * li));
    const float4 hi = *reinterpret_cast<const float4*>(stg + xr_stg(tl, 8 * li + 4));
    const float r[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
    __builtin_nontemporal_store(u32x4{pack_bf16x2(r[0], r[1]), pack_bf16x2(r[2], r[3]), pack_bf16x2(r[4], r[5]),
                                      pack_bf16x2(r[6], r[7])},
                                reinterpret_cast<u32x4*>(g.xy + o));
    if (g.q) {
      // Phase frac(p f) in the reference's f32 op order, cos / sin by
      // v_cos_f32 / v_sin_f32 (argument in revolutions); the rotation in the
      // op order of attention.rs:488-501 (as layer_gemm_kernel<G_X>).
      const float p = (float)(g.fixed ? g.pos0 : g.pos0 + t);
      float qv[8];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float fr = rope_frac(p, fq[j]);
        rope_pair_exact(r[2 * j], r[2 * j + 1], __builtin_amdgcn_cosf(fr), __builtin_amdgcn_sinf(fr), qv[2 * j],
                        qv[2 * j + 1]);
      }
      __builtin_nontemporal_store(u32x4{pack_bf16x2(qv[0], qv[1]), pack_bf16x2(qv[2], qv[3]),
                                        pack_bf16x2(qv[4], qv[5]), pack_bf16x2(qv[6], qv[7])},
                                  reinterpret_cast<u32x4*>(g.q + o));
    }
  };
  // Per tile: once every MFMA wave has staged it, the tile's pieces are read
  // from staging, formed and stored; then this wave's freed counter says so.
  int64_t row0 = (int64_t)rg * XR_T;  // first token row (b * T + t) of the tile
  uint32_t seen = 0;
  for (int i = 0; i < ntile; ++i) {
    wave_wait_min<4>(staged, (uint32_t)(i + 1), seen);
    // A tile lies inside one sequence (T % 128 == 0).
    const int64_t bb = row0 / g.T, t0 = row0 - bb * g.T;
    obase = ((bb * g.H + h) * g.T + t0) * g.N + n0 + 8 * li;
    pbase = t0;
    row0 += (int64_t)rg_count * XR_T;
#pragma unroll
    for (int u = 0; u < XR_PC; ++u) store_piece(u);
    // The pieces' staging reads are complete (their values went into the
    // stores) and precede this write in LDS order.
    wave_count_set(freed + 4 * sw, (uint32_t)(i + 1), lane);
  }
}

// ---- GEMM Y fused into GEMM Z --------------------------------------------
// With T a multiple of 256 and D <= 256 the layer never writes y.  One
// workgroup (8 waves, one per CU) owns a 256-token tile (one sequence) and a
// range of 128-latent chunks of H N, and per chunk
//   Y^T  = Ev_chunk a_h^T        [128 latents x 256 tokens], K = D
//   y    = act(Y) * x            bf16, into LDS as the next product's A operand
//   z   += y Dec_chunk^T         [256 tokens x D], K = 128
// with z in the accumulators across the chunks, written at the end as the
// split-K partial [kp, M, D] that the residual kernel sums in order.  Y is
// computed transposed so that each accumulator register of a lane holds 4
// consecutive latents of one token: one 8-byte read of x and one 8-byte
// write of y.  y is rounded to bf16 exactly as GEMM Y stores it.
// Operands stream through a 3-slot direct-load ring two steps ahead (a step
// is 32 deep: a Y step loads 256 a_h rows and 128 Ev rows, a z step 256
// decoder rows); x lands in the y buffer itself, in pairs of 32-latent
// blocks as soon as the previous chunk's z steps have read them.  (A 4-slot ring, three
// steps ahead in all 160 KiB of LDS, was slower: C5 1.08 against 0.98 ms
// per launch.  So was a wave-role form like layer_x_roles_kernel, one
// 512-thread workgroup per CU with 4 MFMA waves and 4 DMA waves handing a
// 6-slot ring and the y buffer over through LDS counters: parity-green,
// 816 against 780 us at C5.  A chunk took ~13.6 k cycles of an MFMA wave for
// 4.1 k of MFMAs: the y epilogue ~2.4 k, fragment read latency and counter
// polls every step; with one workgroup per CU no other workgroup's MFMAs
// cover them, and the MFMA waves' 242 VGPRs leave no room to read the next
// step's fragments early.)
constexpr int YZ_C = T256 / 2;  // latents per chunk
constexpr int YZ_RING = 3;
constexpr int YZ_PREF = YZ_RING - 1;  // steps loaded ahead

// Tile geometry of the launch with NW waves: TM = 32 NW tokens.
template <int NW>
struct YZGeom {
  static constexpr int NT = 64 * NW;
  static constexpr int TM = 32 * NW;                   // token rows of the tile
  static constexpr int SLOT = (TM + YZ_C) * BK * 2;    // ring slot: a_h rows, then Ev rows (z: decoder rows)
  static constexpr int KB = TM * BK * 2;               // one 32-latent block of y
  static constexpr int YBUF = YZ_RING * SLOT;
  static constexpr int LDS = YBUF + 4 * KB;
  static constexpr int YDMA = (TM / 16 + 8) / NW;      // DMAs a wave issues per Y stage
  static constexpr int ZDMA = 16 / NW;                 // per z stage (256 decoder rows)
  static constexpr int XDMA = TM / 16 / NW;            // per 32-latent x block
};

// Wait until at most n of this wave's DMAs are in flight, then a barrier.
__device__ __forceinline__ void yz_wait_barrier(int n) {
  switch (n) {
    case 1: dma_wait_barrier<1>(); break;
    case 2: dma_wait_barrier<2>(); break;
    case 3: dma_wait_barrier<3>(); break;
    case 4: dma_wait_barrier<4>(); break;
    case 5: dma_wait_barrier<5>(); break;
    case 6: dma_wait_barrier<6>(); break;
    case 7: dma_wait_barrier<7>(); break;
    case 8: dma_wait_barrier<8>(); break;
    default: dma_wait_barrier<0>(); break;
  }
}

// PLAIN: no threshold and no mask (act = ReLU; the same bits as the general
// form with th = 0, m = 1, two VALU instructions a value fewer).
template <int NW, bool PLAIN>
__global__ __launch_bounds__(64 * NW, 8 / NW) void layer_yz_kernel(LayerGemmArgs g) {
  using Geo = YZGeom<NW>;
  constexpr int TM = Geo::TM;
  __shared__ __attribute__((aligned(16))) char lds[Geo::LDS];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  // Workgroup id i runs on XCD i % 8.  With 8 | mt an XCD takes mt / 8
  // token tiles with all ks latent ranges: its L2 then holds those tiles'
  // a_h rows (re-read at every chunk) and the ks chunks' weights being
  // streamed (C5: 1 MB + 512 KB).  Giving an XCD one latent range and 32
  // token tiles instead put 4 MB of a_h rows on its 4 MB L2.
  const int id = (int)blockIdx.x;
  int kp, mtile;
  if (g.mt % 8 == 0) {
    const int slot = id >> 3;
    mtile = (id & 7) * (g.mt >> 3) + slot / g.ks;
    kp = slot % g.ks;
  } else {
    kp = id / g.mt;
    mtile = id - kp * g.mt;
  }
  const int64_t HN = g.H * g.N;
  const int nc = (int)(HN / YZ_C), cpn = (int)(g.N / YZ_C);  // chunks, chunks per head
  const int jb = (int)((int64_t)nc * kp / g.ks), je = (int)((int64_t)nc * (kp + 1) / g.ks);
  const int ny = (int)(g.D / BK), per = ny + 4;  // Y steps, then 4 z steps, per chunk
  const int64_t m0 = (int64_t)mtile * TM, bb = m0 / g.T, t0 = m0 - bb * g.T;
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_addr(lds));
  // DMA lanes (16 rows of 64 bytes per instruction): the lane writing slot
  // c of row r fetches chunk c ^ ((r >> 1) & 3), the swizzle of lds_off.
  // Block b of 16 rows goes to wave b % NW.
  const uint32_t gc16 = (uint32_t)(((lane & 3) ^ ((lane >> 3) & 3)) * 16);
  const uint32_t rsub = (uint32_t)(lane >> 2);
  const uint32_t rowA = (uint32_t)(g.D * 2), rowX = (uint32_t)(g.N * 2), rowDec = YZ_C * 2;  // row pitches, bytes
  // Per-lane offsets of the wave's first row (16 w + rsub); the wave's
  // further blocks, 16 NW rows on each, go through the (uniform) base.
  const uint32_t offA = (16 * w + rsub) * rowA + gc16, offX = (16 * w + rsub) * rowX + gc16;
  const int64_t stepA = 16 * NW * (int64_t)rowA, stepX = 16 * NW * (int64_t)rowX;
  uint32_t offD[Geo::ZDMA];  // decoder rows, clamped to D - 1
#pragma unroll
  for (int i = 0; i < Geo::ZDMA; ++i) {
    const uint32_t d = 16 * (w + NW * i) + rsub;
    offD[i] = (d < (uint32_t)g.D ? d : (uint32_t)g.D - 1) * rowDec + gc16;
  }

  // Operand bases of chunk j (one division per chunk, none per step).
  struct Bases {
    const char* A;   // a_h rows of the token tile, head of the chunk
    const char* E;   // Ev rows of the chunk
    const char* Dc;  // the chunk's decoder block [D, 128]
    const char* X;   // x rows of the token tile at the chunk's first latent
    int64_t n0;      // first latent of the chunk in its head
  };
  auto bases = [&](int j) {
    Bases c;
    const int64_t h = j / cpn;
    c.n0 = (int64_t)(j - h * cpn) * YZ_C;
    c.A = reinterpret_cast<const char*>(g.a + ((bb * g.H + h) * g.T + t0) * g.D);
    c.E = reinterpret_cast<const char*>(g.b + (int64_t)j * YZ_C * g.D);
    c.Dc = reinterpret_cast<const char*>(g.dec + (int64_t)j * g.D * YZ_C);
    c.X = reinterpret_cast<const char*>(g.xy + ((bb * g.H + h) * g.T + t0) * g.N + c.n0);
    return c;
  };
  // x block kb (latents 32 kb ..) of a chunk into the y buffer.
  auto issue_x = [&](const Bases& c, int kb) {
    const uint32_t base = lds0 + (uint32_t)(Geo::YBUF + kb * Geo::KB);
#pragma unroll
    for (int i = 0; i < Geo::XDMA; ++i)
      dma16_nt(c.X + kb * 64 + i * stepX, offX, base + (uint32_t)((w + NW * i) * 1024));
  };
  // Ring stage of step s of a chunk into slot `slot`: a Y step (s < ny) a_h
  // rows 0..TM-1 then Ev rows TM..TM+127, a z step the 256 decoder rows.
  auto issue_stage = [&](const Bases& c, int s, int slot) {
    const uint32_t base = lds0 + (uint32_t)(slot * Geo::SLOT);
    if (s < ny) {
#pragma unroll
      for (int i = 0; i < TM / 16 / NW; ++i)
        dma16(c.A + s * 64 + i * stepA, offA, base + (uint32_t)((w + NW * i) * 1024));
#pragma unroll
      for (int i = 0; i < 8 / NW; ++i)
        dma16(c.E + s * 64 + i * (16 * NW * (int64_t)rowA), offA, base + (uint32_t)((TM / 16 + w + NW * i) * 1024));
    } else {
#pragma unroll
      for (int i = 0; i < Geo::ZDMA; ++i)
        dma16(c.Dc + (s - ny) * 64, offD[i], base + (uint32_t)((w + NW * i) * 1024));
    }
  };
  static_assert(YZ_PREF == 2, "the waits below count one step ahead");
  // DMAs a wave issues at the top of a step, after its barrier: x blocks 0
  // and 1 of the next chunk at z step 2 (the z steps before have read those
  // blocks of y) and blocks 2 and 3 of the current chunk at its first Y step
  // (the prologue loads chunk jb's four; issued in pairs, the two 64-byte
  // halves of each 128-byte line are requested together); then the ring
  // stage of the step YZ_PREF = 2 ahead.  At the top of step (j, s) the wave
  // has issued after that step's stage (issued at the top of the step 2
  // back, after that step's x): the x DMAs of step (j, s - 1) and the stage
  // of the next step; waiting for at most that many leaves the stage (and
  // every x block issued before it) landed.  At the first z step the
  // epilogue needs the chunk's blocks 2 and 3 (issued at its first Y step,
  // at least 2 steps back): there the x count is 0 anyway.
  auto pending = [&](int j, int s) {
    int n = 0;
    if (s == 1 && j > jb) n += 2 * Geo::XDMA;           // x at (j, 0)
    if (s == ny + 3 && j + 1 < je) n += 2 * Geo::XDMA;  // x at (j, ny + 2)
    if (s + 1 < per) n += s + 1 < ny ? Geo::YDMA : Geo::ZDMA;  // stage of (j, s + 1)
    else if (j + 1 < je) n += Geo::YDMA;                // stage of (j + 1, 0)
    return n;
  };

  floatx4 accz[4][8];
  zero_acc(accz);
  const int yc = w & 1, ym = w >> 1;  // Y^T block: latents 64 yc .., tokens 64 ym ..
  const int zm = w >> 1, zd = w & 1;  // z block: tokens 64 zm .., columns 128 zd ..
  const float th = g.relu_th;
  char* const ybuf = lds + Geo::YBUF;
  // The two waves of a SIMD issue their DMAs and their MFMAs in opposite
  // orders, so that one issues MFMAs while the other's DMAs wait in the
  // texture unit's queue (8 waves: w and w + 4; 4 waves, two workgroups a
  // CU: the workgroups' barriers are independent).  Issuing the DMAs
  // between the MFMA groups instead (4 waves) was slower: 1.48 against 0.77
  // ms at C5, the stages landing later and 15 VGPRs spilled.
  const bool dma_first = NW == 8 ? w < 4 : true;
  __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): no compiler-visible load left in flight
  Bases cur = bases(jb);
  if (jb < je) {
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) issue_x(cur, kb);
    issue_stage(cur, 0, 0);
    issue_stage(cur, 1, 1);  // ny >= 2
  }
  int slot = 0;  // ring slot of the current step
  for (int j = jb; j < je; ++j) {
    const Bases nxt = bases(j + 1 < je ? j + 1 : j);
    // Stage of the step 2 ahead of (j, s), into the slot the step before
    // (j, s) used.
    auto prefetch = [&](int s) {
      const int t = s + YZ_PREF, sl = slot == 0 ? YZ_RING - 1 : slot - 1;
      if (t < per) issue_stage(cur, t, sl);
      else if (j + 1 < je) issue_stage(nxt, t - per, sl);
    };
    floatx4 accy[4][4];
#pragma unroll
    for (int ci = 0; ci < 4; ++ci)
#pragma unroll
      for (int mj = 0; mj < 4; ++mj) accy[ci][mj] = zero4();
    for (int s = 0; s < ny; ++s) {
      yz_wait_barrier(pending(j, s));
      const bf16_t* sp = reinterpret_cast<const bf16_t*>(lds + slot * Geo::SLOT);
      auto dmas = [&]() {
        if (s == 0 && j > jb) {
          issue_x(cur, 2);
          issue_x(cur, 3);
        }
        prefetch(s);
      };
      if (dma_first) dmas();
      mma_64x64_dsasm(sp + TM * BK, sp, lane, 64 * yc, 64 * ym, accy);
      if (!dma_first) dmas();
      slot = slot == YZ_RING - 1 ? 0 : slot + 1;
    }
    for (int kz = 0; kz < 4; ++kz) {
      yz_wait_barrier(pending(j, ny + kz));
      auto dmas = [&]() {
        if (kz == 2 && j + 1 < je) {
          issue_x(nxt, 0);
          issue_x(nxt, 1);
        }
        prefetch(ny + kz);
      };
      if (dma_first || kz == 0) dmas();
      if (kz == 0) {
        // y = act(Y) * x over the x block in place (each lane rewrites only
        // what it reads; the 4 reads of a latent group are issued before
        // its writes), then a barrier before any wave reads y.
#pragma unroll
        for (int ci = 0; ci < 4; ++ci) {
          const int cl = 64 * yc + 16 * ci + 4 * (lane >> 4);  // latents cl .. cl + 3 of the chunk
          float mk[4] = {1.0f, 1.0f, 1.0f, 1.0f};
          if (!PLAIN) {
#pragma unroll
            for (int r = 0; r < 4; ++r) mk[r] = g.mask ? g.mask[cur.n0 + cl + r] : 1.0f;
          }
          auto act = [&](float v, int r) { return PLAIN ? fmaxf(v, 0.0f) : lowrank_act(v, th, mk[r]); };
          char* const yb = ybuf + (cl >> 5) * Geo::KB + 8 * ((cl >> 2) & 1);
          uint2 xv[4];
#pragma unroll
          for (int mj = 0; mj < 4; ++mj) {
            const int ml = 64 * ym + 16 * mj + (lane & 15);
            xv[mj] = *reinterpret_cast<const uint2*>(yb + 2 * lds_off(ml, (cl >> 3) & 3));
          }
#pragma unroll
          for (int mj = 0; mj < 4; ++mj) {
            const int ml = 64 * ym + 16 * mj + (lane & 15);
            const floatx4 v = accy[ci][mj];
            *reinterpret_cast<uint2*>(yb + 2 * lds_off(ml, (cl >> 3) & 3)) =
                make_uint2(pack_bf16x2(act(v[0], 0) * bf16_lo(xv[mj].x), act(v[1], 1) * bf16_hi(xv[mj].x)),
                           pack_bf16x2(act(v[2], 2) * bf16_lo(xv[mj].y), act(v[3], 3) * bf16_hi(xv[mj].y)));
          }
        }
        __syncthreads();
      }
      const bf16_t* sp = reinterpret_cast<const bf16_t*>(lds + slot * Geo::SLOT);
      mma_64x128_dsasm(reinterpret_cast<const bf16_t*>(ybuf + kz * Geo::KB), sp, lane, 64 * zm, 128 * zd, accz);
      if (!dma_first && kz > 0) dmas();
      slot = slot == YZ_RING - 1 ? 0 : slot + 1;
    }
    cur = nxt;
  }
  dma_wait_barrier<0>();  // the epilogue reuses the ring
  epilogue_64x128(accz, reinterpret_cast<bf16_t*>(lds), w, lane, [&](int row, int col, float4 v) {
    const int64_t m = m0 + 64 * zm + row, d = 128 * zd + col;
    if (d < g.D) *reinterpret_cast<float4*>(&g.zpart[((int64_t)kp * g.M + m) * g.D + d]) = v;
  });
}

// ---- few-row GEMMs (M <= 64 token rows, e.g. one generated token per
// sequence) ---------------------------------------------------------------
// The 256 x 128 tile would run 8 (K = 256) or more dependent 32-deep steps on
// mostly empty rows.  Here a workgroup owns one 16-column block and a K
// range; its 4 waves split the range, each loading its steps' operands
// straight into MFMA fragment registers (8 steps' loads in flight, no LDS
// staging), and sum their accumulators through LDS in wave order.  Up to 4
// 16-row blocks; rows past M re-read row M - 1 and are never stored.
constexpr int SK_MAXM = 64;
constexpr int SK_CHUNK = 8;  // 32-deep steps loaded at once per wave

template <int KIND, int MB>  // MB = 16-row blocks: 1, 2 or 4
__global__ __launch_bounds__(256) void skinny_gemm_kernel(LayerGemmArgs g) {
  // X, Y (K = D, H N columns): each wave owns a 16-column block and all of
  // K.  Z (K = H N) and the logits (few columns): the workgroup owns one
  // column block and a K range, which its 4 waves split and sum through LDS
  // in wave order.  (X, Y: 13 and 15 -> 11 us at C5 decode.)
  constexpr bool WAVECOL = KIND == G_X || KIND == G_Y;
  __shared__ floatx4 red[WAVECOL ? 1 : 4][MB][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t ncols = KIND == G_Z ? g.D : KIND == G_L ? g.V : g.H * g.N;
  const int64_t K = KIND == G_Z ? g.H * g.N : g.D;
  const int ncb = (int)((ncols + 15) / 16);
  const int cblk = WAVECOL ? (int)blockIdx.x * 4 + w : (int)(blockIdx.x % ncb);
  const int kp = WAVECOL ? 0 : (int)(blockIdx.x / ncb);
  if (WAVECOL && cblk >= ncb) return;  // no barriers in this mode
  const int64_t c0 = (int64_t)cblk * 16;
  const int64_t h = (KIND == G_X || KIND == G_Y) ? c0 / g.N : 0;
  // Steps of this wave: all K/32 (WAVECOL), or part p of 4 * ks equal parts.
  const int64_t nk = K / 32, parts = 4 * (int64_t)g.ks, p = (int64_t)kp * 4 + w;
  const int kb = WAVECOL ? 0 : (int)(nk * p / parts);
  const int ke = WAVECOL ? (int)nk : (int)(nk * (p + 1) / parts);
  const int kl = 8 * (lane >> 4);  // this lane's 8 k values within a step
  int64_t cb = c0 + (lane & 15);
  cb = cb < ncols ? cb : ncols - 1;
  const bf16_t* brow = g.b + (KIND == G_Z ? cb * 128 : cb * K) + kl;
  const bf16_t* arow[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    int64_t m = 16 * mb + (lane & 15);
    m = m < g.M ? m : g.M - 1;
    const int64_t bb = m / g.T, t = m - bb * g.T;
    if (KIND == G_X || KIND == G_L) arow[mb] = g.a + m * g.D + kl;
    else if (KIND == G_Y) arow[mb] = g.a + ((bb * g.H + h) * g.T + t) * g.D + kl;
    else arow[mb] = g.a + (bb * g.H * g.T + t) * g.N + kl;
  }
  floatx4 acc[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) acc[mb] = zero4();
  for (int k0 = kb; k0 < ke; k0 += SK_CHUNK) {
    const int n = ke - k0 < SK_CHUNK ? ke - k0 : SK_CHUNK;
    bf16x8 bq[SK_CHUNK], aq[SK_CHUNK][MB];
#pragma unroll
    for (int s = 0; s < SK_CHUNK; ++s) {
      if (s >= n) break;
      const int64_t k = (int64_t)(k0 + s) * 32;
      // Z: k runs over (head, neuron); a 32-deep step stays inside one head.
      const int64_t aoff = KIND == G_Z ? (k / g.N) * g.T * g.N + k % g.N : k;
      bq[s] = *reinterpret_cast<const bf16x8*>(brow + (KIND == G_Z ? dec_off(0, k, g.D) : k));
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) aq[s][mb] = *reinterpret_cast<const bf16x8*>(arow[mb] + aoff);
    }
#pragma unroll
    for (int s = 0; s < SK_CHUNK; ++s) {
      if (s >= n) break;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) acc[mb] = mfma16(aq[s][mb], bq[s], acc[mb]);
    }
  }
  const int64_t c = c0 + (lane & 15);
  const int64_t n = c - h * g.N;
  const float mk = (WAVECOL && g.mask) ? g.mask[n < g.N ? n : g.N - 1] : 1.0f;
  // Epilogue of the 16 x 16 block of row block mb (lane: rows
  // 4 (lane >> 4) + r, column lane & 15).
  auto emit = [&](int mb, const floatx4& v) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t m = 16 * mb + acc16_row(lane, r);
      float val = v[r];
      if (KIND == G_X) {
        // Every lane joins the partner exchange before any row test.
        const float x = lowrank_act(val, g.relu_th, mk);
        const float xp = __shfl_xor(x, 1, 64);  // column c ^ 1 of the same row
        if (m >= g.M) continue;
        const int64_t bb = m / g.T, t = m - bb * g.T;
        const int64_t o = ((bb * g.H + h) * g.T + t) * g.N + n;
        g.xy[o] = (bf16_t)x;
        if (g.xf) g.xf[o] = x;
        if (g.q) {
          const float p = (float)(g.fixed ? g.pos0 : g.pos0 + t);
          const int64_t ne = n & ~(int64_t)1;
          const float fr = rope_frac(p, g.freqs[ne]);
          const float e = (n & 1) ? xp : x, od = (n & 1) ? x : xp;
          float qe, qo;
          rope_pair_exact(e, od, __builtin_amdgcn_cosf(fr), __builtin_amdgcn_sinf(fr), qe, qo);
          g.q[o] = (bf16_t)((n & 1) ? qo : qe);
        }
      } else {
        if (m >= g.M) continue;
        if (KIND == G_Y) {
          const int64_t bb = m / g.T, t = m - bb * g.T;
          bf16_t* dst = g.xy + ((bb * g.H + h) * g.T + t) * g.N + n;
          *dst = (bf16_t)(lowrank_act(val, g.relu_th, mk) * (float)*dst);
        } else if (KIND == G_Z) {
          g.zpart[((int64_t)kp * g.M + m) * g.D + c] = val;
        } else if (c < g.V) {
          g.zpart[m * g.V + c] = val;
        }
      }
    }
  };
  if (WAVECOL) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) emit(mb, acc[mb]);
    return;
  }
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) red[w][mb][lane] = acc[mb];
  __syncthreads();
  // Wave mb finishes row block mb: the 4 wave partials in order.
  if (w >= MB) return;
  floatx4 v = red[0][w][lane];
#pragma unroll
  for (int ww = 1; ww < 4; ++ww) v = v + red[ww][w][lane];
  emit(w, v);
}

// Wave-wide sum (fixed butterfly order: the same result in every lane).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

constexpr int LN_MAX = 32;  // D / 64 values per lane (D <= 2048)

// LayerNorm of one D-row held 64-strided across the wave's lanes, in place:
// (v - mean) / sqrt(var + eps), biased variance, two passes.
template <int PER>
__device__ __forceinline__ void ln_wave(float (&v)[LN_MAX], int D) {
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < PER; ++i) s += v[i];
  const float mean = wave_sum(s) / (float)D;
  float q = 0.0f;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    v[i] -= mean;
    q += v[i] * v[i];
  }
  const float den = sqrtf(wave_sum(q) / (float)D + 1e-5f);
#pragma unroll
  for (int i = 0; i < PER; ++i) v[i] /= den;
}

// out_bf16[r, :] = LN(in[r, :]) for `rows` rows of D (one wave per row).
template <int PER>
__global__ __launch_bounds__(256) void ln_rows_kernel(const float* __restrict__ in,
                                                      bf16_t* __restrict__ out, int64_t rows,
                                                      int D) {
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= rows) return;
  float v[LN_MAX];
#pragma unroll
  for (int i = 0; i < PER; ++i) v[i] = in[r * D + lane + 64 * i];
  ln_wave<PER>(v, D);
#pragma unroll
  for (int i = 0; i < PER; ++i) out[r * D + lane + 64 * i] = (bf16_t)v[i];
}

// next[m, :] = LN(cur[m, :] + LN(z[m, :])), z = sum of the ks partials in
// a fixed order (one wave per token row).
template <int PER>
__global__ __launch_bounds__(256) void residual_kernel(const float* __restrict__ zpart,
                                                       const float* __restrict__ cur,
                                                       float* __restrict__ next, int64_t M,
                                                       int D, int ks) {
  const int64_t m = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (m >= M) return;
  float v[LN_MAX];
  const float* z = zpart + m * D + lane;
#pragma unroll
  for (int i = 0; i < PER; ++i) v[i] = z[64 * i];
  // Partials in order kp = 1, 2, ...; the loads of U splits are issued
  // before their adds.
  constexpr int U = PER <= 8 ? 4 : 1;
  const int64_t zs = M * D;
  int kp = 1;
  for (; kp + U <= ks; kp += U) {
    float t[U][PER];
#pragma unroll
    for (int j = 0; j < U; ++j)
#pragma unroll
      for (int i = 0; i < PER; ++i) t[j][i] = z[(kp + j) * zs + 64 * i];
#pragma unroll
    for (int j = 0; j < U; ++j)
#pragma unroll
      for (int i = 0; i < PER; ++i) v[i] += t[j][i];
  }
  for (; kp < ks; ++kp)
#pragma unroll
    for (int i = 0; i < PER; ++i) v[i] += z[kp * zs + 64 * i];
  ln_wave<PER>(v, D);
#pragma unroll
  for (int i = 0; i < PER; ++i) v[i] += cur[m * D + lane + 64 * i];
  ln_wave<PER>(v, D);
#pragma unroll
  for (int i = 0; i < PER; ++i) next[m * D + lane + 64 * i] = v[i];
}

// out[i, :] = LN(embed[tokens[i], :]) (one wave per token); ids outside
// [0, vocab) give a zero row (LN of zeros is zeros).
template <int PER>
__global__ __launch_bounds__(256) void embed_norm_kernel(const int32_t* __restrict__ tokens,
                                                         const float* __restrict__ embed,
                                                         float* __restrict__ out, int64_t n,
                                                         int64_t vocab, int D) {
  const int64_t i = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (i >= n) return;
  const int32_t id = tokens[i];
  const bool ok = id >= 0 && (int64_t)id < vocab;
  float v[LN_MAX];
#pragma unroll
  for (int k = 0; k < PER; ++k) v[k] = ok ? embed[(int64_t)id * D + lane + 64 * k] : 0.0f;
  ln_wave<PER>(v, D);
#pragma unroll
  for (int k = 0; k < PER; ++k) out[i * D + lane + 64 * k] = v[k];
}

__global__ __launch_bounds__(256) void to_bf16_kernel(const float* __restrict__ in,
                                                      bf16_t* __restrict__ out, int64_t n) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i >= n) return;
  if (i + 4 <= n) {
    const float4 v = *reinterpret_cast<const float4*>(in + i);
    *reinterpret_cast<uint2*>(out + i) = make_uint2(pack_bf16x2(v.x, v.y), pack_bf16x2(v.z, v.w));
  } else {
    for (int64_t j = i; j < n; ++j) out[j] = (bf16_t)in[j];
  }
}

// out[b, c, r] = bf16(in[b, r, c]) for [batches, rows, cols] (32 x 32 tiles);
// chunked (one batch, rows a multiple of 128): out[dec_off(c, r, cols)], the
// chunk-major decoder.
__global__ __launch_bounds__(256) void transpose_bf16_kernel(const float* __restrict__ in,
                                                             bf16_t* __restrict__ out,
                                                             int64_t rows, int64_t cols, bool chunked) {
  __shared__ float tile[32][33];
  const int64_t b = blockIdx.z;
  const int64_t r0 = (int64_t)blockIdx.y * 32, c0 = (int64_t)blockIdx.x * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
  for (int k = ty; k < 32; k += 8) {
    const int64_t r = r0 + k, c = c0 + tx;
    tile[k][tx] = (r < rows && c < cols) ? in[(b * rows + r) * cols + c] : 0.0f;
  }
  __syncthreads();
  for (int k = ty; k < 32; k += 8) {
    const int64_t c = c0 + k, r = r0 + tx;
    if (c < cols && r < rows) out[chunked ? dec_off(c, r, cols) : (b * cols + c) * rows + r] = (bf16_t)tile[tx][k];
  }
}

inline unsigned cdiv(int64_t a, int64_t b) { return (unsigned)((a + b - 1) / b); }

// Few-row GEMM launch: one workgroup per (16-column block, K split).
template <int KIND>
hipError_t launch_skinny(const LayerGemmArgs& g, hipStream_t st) {
  const int64_t ncols = KIND == G_Z ? g.D : KIND == G_L ? g.V : g.H * g.N;
  const int64_t blocks = (KIND == G_X || KIND == G_Y) ? cdiv(cdiv(ncols, 16), 4)
                                                      : cdiv(ncols, 16) * (int64_t)(KIND == G_Z ? g.ks : 1);
  const dim3 grid((unsigned)blocks);
  if (g.M <= 16) hipLaunchKernelGGL((skinny_gemm_kernel<KIND, 1>), grid, dim3(256), 0, st, g);
  else if (g.M <= 32) hipLaunchKernelGGL((skinny_gemm_kernel<KIND, 2>), grid, dim3(256), 0, st, g);
  else hipLaunchKernelGGL((skinny_gemm_kernel<KIND, 4>), grid, dim3(256), 0, st, g);
  return hipGetLastError();
}

template <int KIND>
hipError_t launch_gemm(const LayerGemmArgs& g, hipStream_t st) {
  if (g.M <= SK_MAXM) return launch_skinny<KIND>(g, st);
  const int64_t total = (int64_t)g.mt * g.ct * (KIND == G_Z ? g.ks : 1);
  const int64_t slots = 2 * (int64_t)device_cus();  // two workgroups per CU
  const unsigned grid = (unsigned)(total < slots ? total : slots);
  hipLaunchKernelGGL(layer_gemm_kernel<KIND>, dim3(grid), dim3(NT), 0, st, g);
  return hipGetLastError();
}

// Row-tile groups of the two-role GEMM X (layer_x_roles_kernel), or 0 where
// the shape needs layer_gemm_kernel<G_X>: x wanted in f32 (the decode step),
// few rows, T or N not a multiple of 128, D not a multiple of 32, under 64
// or above 256, or more 128-latent column tiles than CUs.  A workgroup per column
// tile and group; the groups split the row tiles.
int x_roles_groups(const LayerGemmArgs& g) {
  if (g.xf || g.M <= SK_MAXM || g.T % XR_T != 0 || g.N % XR_T != 0 || g.D % BK != 0 || g.D < 2 * BK ||
      g.D > T256)
    return 0;
  const int64_t ct = g.H * g.N / XR_T, mt = g.M / XR_T, cus = device_cus();
  if (ct > cus) return 0;
  const int64_t r = cus / ct;
  return (int)(r < mt ? r : mt);
}

hipError_t launch_x(const LayerGemmArgs& g, hipStream_t st) {
  const int groups = x_roles_groups(g);
  if (groups == 0) return launch_gemm<G_X>(g, st);
  const dim3 grid((unsigned)(g.H * g.N / XR_T * groups));
  if (g.relu_th == 0.0f && g.mask == nullptr)
    hipLaunchKernelGGL(layer_x_roles_kernel<true>, grid, dim3(64 * (XR_MW + XR_DW + XR_SW)), 0, st, g, groups);
  else
    hipLaunchKernelGGL(layer_x_roles_kernel<false>, grid, dim3(64 * (XR_MW + XR_DW + XR_SW)), 0, st, g, groups);
  return hipGetLastError();
}

// Split count of the fused Y + Z launch over the 128-latent chunks, or 0
// where the shape needs GEMM Y and GEMM Z apart: T a multiple of 256 (a
// token tile inside one sequence), D a multiple of 64 up to 256 (the z tile),
// DMA offsets within 32 bits.  About one workgroup per CU, with at least 4
// chunks each where the chunks allow (C5: 64 token tiles x 4 splits of 64).
constexpr int YZ_NW = 4;  // waves of the fused launch: 128-token tiles, two workgroups a CU
constexpr int YZ_TM = YZGeom<YZ_NW>::TM;

int yz_splits(int64_t M, int64_t H, int64_t T, int64_t N, int64_t D) {
  if (M <= SK_MAXM || T % YZ_TM != 0 || D % 64 != 0 || D > T256) return 0;
  const int64_t HN = H * N;
  if (HN % YZ_C != 0 || (int64_t)YZ_TM * N * 2 >= ((int64_t)1 << 32)) return 0;
  const int64_t tiles = M / YZ_TM, nc = HN / YZ_C;
  int64_t ks = (int64_t)device_cus() * (8 / YZ_NW) / tiles;
  if (ks > nc / 4) ks = nc / 4;
  return (int)(ks < 1 ? 1 : ks);
}

hipError_t launch_yz(const LayerGemmArgs& g, hipStream_t st) {
  const dim3 grid((unsigned)(g.mt * g.ks)), block(64 * YZ_NW);
  if (g.relu_th == 0.0f && g.mask == nullptr) hipLaunchKernelGGL((layer_yz_kernel<YZ_NW, true>), grid, block, 0, st, g);
  else hipLaunchKernelGGL((layer_yz_kernel<YZ_NW, false>), grid, block, 0, st, g);
  return hipGetLastError();
}

template <int PER>
hipError_t launch_ln(const float* in, bf16_t* out, int64_t rows, int D, hipStream_t st) {
  hipLaunchKernelGGL(ln_rows_kernel<PER>, dim3(cdiv(rows, 4)), dim3(256), 0, st, in, out, rows, D);
  return hipGetLastError();
}

template <int PER>
hipError_t launch_residual(const float* z, const float* cur, float* next, int64_t M, int D, int ks,
                           hipStream_t st) {
  hipLaunchKernelGGL(residual_kernel<PER>, dim3(cdiv(M, 4)), dim3(256), 0, st, z, cur, next, M, D,
                     ks);
  return hipGetLastError();
}

// PER = D / 64 as a compile-time count (D a multiple of 64, at most 2048).
template <template <int> class F, class... Args>
hipError_t dispatch_per(int D, Args... args) {
  switch (D / 64) {
#define BDH_PER(p) \
  case p:          \
    return F<p>::run(args...);
    BDH_PER(1) BDH_PER(2) BDH_PER(3) BDH_PER(4) BDH_PER(5) BDH_PER(6) BDH_PER(7) BDH_PER(8)
    BDH_PER(9) BDH_PER(10) BDH_PER(11) BDH_PER(12) BDH_PER(13) BDH_PER(14) BDH_PER(15)
    BDH_PER(16) BDH_PER(17) BDH_PER(18) BDH_PER(19) BDH_PER(20) BDH_PER(21) BDH_PER(22)
    BDH_PER(23) BDH_PER(24) BDH_PER(25) BDH_PER(26) BDH_PER(27) BDH_PER(28) BDH_PER(29)
    BDH_PER(30) BDH_PER(31) BDH_PER(32)
#undef BDH_PER
    default:
      return hipErrorInvalidValue;
  }
}
template <int PER>
struct LnF {
  static hipError_t run(const float* in, bf16_t* out, int64_t rows, int D, hipStream_t st) {
    return launch_ln<PER>(in, out, rows, D, st);
  }
};
template <int PER>
struct EmbF {
  static hipError_t run(const int32_t* tokens, const float* embed, float* out, int64_t n,
                        int64_t vocab, int D, hipStream_t st) {
    hipLaunchKernelGGL(embed_norm_kernel<PER>, dim3(cdiv(n, 4)), dim3(256), 0, st, tokens, embed,
                       out, n, vocab, D);
    return hipGetLastError();
  }
};
template <int PER>
struct ResF {
  static hipError_t run(const float* z, const float* cur, float* next, int64_t M, int D, int ks,
                        hipStream_t st) {
    return launch_residual<PER>(z, cur, next, M, D, ks, st);
  }
};

}  // namespace

bool layer_shape_supported(int64_t N, int64_t D, const char** why) {
  if (!bf16_shape_supported(N, D, why)) return false;
  if (D % 64 != 0 || D > 64 * LN_MAX) {
    if (why) *why = "layer needs embd % 64 == 0 and embd <= 2048";
    return false;
  }
  return true;
}

bdh_status pack_lowrank_weights(int64_t H, int64_t N, int64_t D, const float* enc,
                                const float* encv, const float* dec, bf16_t* enc_p,
                                bf16_t* encv_p, bf16_t* dec_p, hipStream_t st) {
  // encoders [H, D, N] -> [H, N, D]; decoder [H*N, D] -> [H*N/128, D, 128]
  const dim3 ge(cdiv(N, 32), cdiv(D, 32), (unsigned)H);
  hipLaunchKernelGGL(transpose_bf16_kernel, ge, dim3(256), 0, st, enc, enc_p, D, N, false);
  hipLaunchKernelGGL(transpose_bf16_kernel, ge, dim3(256), 0, st, encv, encv_p, D, N, false);
  const dim3 gd(cdiv(D, 32), cdiv(H * N, 32), 1);
  hipLaunchKernelGGL(transpose_bf16_kernel, gd, dim3(256), 0, st, dec, dec_p, H * N, D, true);
  BDH_HIP_TRY(hipGetLastError());
  return BDH_OK;
}

bdh_status embed_norm(const int32_t* tokens, int64_t n, const float* embed, int64_t vocab,
                      int64_t D, float* out, hipStream_t st) {
  BDH_HIP_TRY(dispatch_per<EmbF>((int)D, tokens, embed, out, n, vocab, (int)D, st));
  return BDH_OK;
}

bdh_status pack_lm_head(int64_t D, int64_t V, const float* head, bf16_t* packed, hipStream_t st) {
  // [D, V] -> [V, D]
  hipLaunchKernelGGL(transpose_bf16_kernel, dim3(cdiv(V, 32), cdiv(D, 32), 1), dim3(256), 0, st,
                     head, packed, D, V, false);
  BDH_HIP_TRY(hipGetLastError());
  return BDH_OK;
}

bdh_status lm_logits(const float* hidden, int64_t M, int64_t D, const bf16_t* head, int64_t V,
                     float* logits, hipStream_t st) {
  void* hb = nullptr;
  bdh_status s = scratch(st, SLOT_LAYER_CUR, (size_t)(M * D) * sizeof(bf16_t), &hb);
  if (s != BDH_OK) return s;
  hipLaunchKernelGGL(to_bf16_kernel, dim3(cdiv(M * D, 1024)), dim3(256), 0, st, hidden,
                     (bf16_t*)hb, M * D);
  BDH_HIP_TRY(hipGetLastError());
  LayerGemmArgs g{};
  g.a = (const bf16_t*)hb;
  g.b = head;
  g.zpart = logits;
  g.B = 1; g.H = 1; g.T = M; g.N = 1; g.D = D; g.M = M; g.V = V;
  g.mt = (int)cdiv(M, T256);
  g.ct = (int)cdiv(V, T256 / 2);
  g.ks = 1;
  BDH_HIP_TRY(launch_gemm<G_L>(g, st));
  return BDH_OK;
}

bdh_status run_layer(const LayerArgs& a, hipStream_t st, uint64_t* launches) {
  const int64_t S = a.B * a.H, M = a.B * a.T, HN = a.H * a.N;
  // One token carried in place: the sparse decode step touches only the rho
  // rows of the token's active neurons, where the MFMA path would read and
  // write all of rho.
  const bool decode = a.T == 1 && a.rho_in != nullptr && a.rho_in == a.rho_out;
  void *curb = nullptr, *xy = nullptr, *attn = nullptr, *an = nullptr, *zp = nullptr;
  // Decoder split-K.  256 x 128 tiles: the fewest splits (each an even
  // number of 32-deep steps) that give at least two workgroups per CU, at
  // most 16.  Few rows: about 8 steps per wave (32 per workgroup), at most 64.
  const int64_t nkz = HN / 32;
  // GEMM Y fused into GEMM Z (y never reaches HBM) where the shape allows.
  const int ks_yz = decode ? 0 : yz_splits(M, a.H, a.T, a.N, a.D);
  int ks = 1;
  if (ks_yz > 0) {
    ks = ks_yz;
  } else if (M <= SK_MAXM) {
    while (ks < 64 && nkz / (2 * ks) >= 32) ks *= 2;
  } else {
    const int64_t tiles_z = (int64_t)cdiv(M, T256) * cdiv(a.D, T256 / 2);
    for (int cand = 1; cand <= 16 && nkz % (2 * cand) == 0; cand *= 2) {
      ks = cand;
      if (tiles_z * cand >= 512) break;
    }
  }
  bdh_status s = scratch(st, SLOT_LAYER_CUR, (size_t)(M * a.D) * sizeof(bf16_t), &curb);
  if (s != BDH_OK) return s;
  s = scratch(st, SLOT_LAYER_XY, (size_t)(S * a.T * a.N) * sizeof(bf16_t), &xy);
  if (s != BDH_OK) return s;
  // q: rope(x) in bf16 for the MFMA attention, or x in f32 for the decode
  // step (which rotates as it gathers).
  void* q = nullptr;
  if (decode) {
    s = scratch(st, SLOT_LAYER_Q, (size_t)(S * a.N) * sizeof(float), &q);
    if (s != BDH_OK) return s;
  } else if (a.freqs) {
    s = scratch(st, SLOT_LAYER_Q, (size_t)(S * a.T * a.N) * sizeof(bf16_t), &q);
    if (s != BDH_OK) return s;
  }
  s = scratch(st, SLOT_LAYER_ATTN, (size_t)(S * a.T * a.D) * sizeof(float), &attn);
  if (s != BDH_OK) return s;
  s = scratch(st, SLOT_LAYER_AN, (size_t)(S * a.T * a.D) * sizeof(bf16_t), &an);
  if (s != BDH_OK) return s;
  s = scratch(st, SLOT_LAYER_Z, (size_t)(ks * M * a.D) * sizeof(float), &zp);
  if (s != BDH_OK) return s;
  // A carried state whose successor is not kept still needs the state path
  // (readout of rho_in); its rho goes to scratch.
  float* rho_out = a.rho_out;
  if (!decode && a.rho_in && !rho_out) {
    void* r = nullptr;
    s = scratch(st, SLOT_LAYER_RHO, (size_t)(S * a.N * a.D) * sizeof(float), &r);
    if (s != BDH_OK) return s;
    rho_out = (float*)r;
  }

  hipLaunchKernelGGL(to_bf16_kernel, dim3(cdiv(M * a.D, 1024)), dim3(256), 0, st, a.cur,
                     (bf16_t*)curb, M * a.D);
  BDH_HIP_TRY(hipGetLastError());
  LayerGemmArgs g{};
  g.B = a.B; g.H = a.H; g.T = a.T; g.N = a.N; g.D = a.D; g.M = M;
  g.mt = (int)cdiv(M, T256);
  g.ct = (int)(HN / (T256 / 2));
  g.ks = 1;
  g.a = (const bf16_t*)curb;
  g.b = a.enc;
  g.xy = (bf16_t*)xy;
  g.q = decode ? nullptr : (bf16_t*)q;
  g.xf = decode ? (float*)q : nullptr;
  g.freqs = a.freqs;
  g.pos0 = a.pos0;
  g.fixed = a.fixed;
  g.relu_th = a.relu_th;
  g.mask = a.mask;
  BDH_HIP_TRY(launch_x(g, st));
  g.q = nullptr;
  g.xf = nullptr;

  uint64_t n_attn = 0;
  if (decode) {
    // a = rope(x) . rho, then rho[A] += rope(x)[A]^T cur for the token's
    // active set A, in f32 (value = the f32 layer input).
    DecodeArgs d;
    d.x = (const float*)q;
    d.v = a.cur;
    d.rho_in = a.rho_out;
    d.rho = a.rho_out;
    d.decay = nullptr;
    d.freqs = a.freqs;
    d.pos = (float)a.pos0;
    d.a_out = (float*)attn;
    d.idx_out = nullptr;
    d.cnt_out = nullptr;
    d.B = a.B; d.H = a.H; d.Hv = 1; d.N = a.N; d.D = a.D;
    s = run_decode(d, st, &n_attn);
    if (s != BDH_OK) return s;
  } else {
    // The attention reads the rotated queries GEMM X wrote (or x itself
    // without RoPE), so it runs without a RoPE table.
    Bf16Args b;
    b.x = (const bf16_t*)(q ? q : xy);
    b.v = (const bf16_t*)curb;
    b.rho_in = a.rho_in;
    b.decay = nullptr;
    b.freqs = nullptr;
    b.pos0 = 0;
    b.fixed = 0;
    b.ctx = (float*)attn;
    b.rho_out = rho_out;
    b.B = a.B; b.H = a.H; b.Hv = 1; b.T = a.T; b.N = a.N; b.D = a.D;
    b.state = rho_out != nullptr;
    b.L = b.state ? a.state_interval : ((a.T + 127) / 128) * 128;
    b.part16 = true;
    s = run_bf16_path(b, st, &n_attn);
    if (s != BDH_OK) return s;
  }

  BDH_HIP_TRY(dispatch_per<LnF>((int)a.D, (const float*)attn, (bf16_t*)an, S * a.T, (int)a.D, st));
  g.a = (const bf16_t*)an;
  g.b = a.encv;
  if (ks_yz > 0) {
    g.dec = a.dec;
    g.mt = (int)(M / YZ_TM);
    g.ks = ks;
    g.zpart = (float*)zp;
    BDH_HIP_TRY(launch_yz(g, st));
  } else {
    BDH_HIP_TRY(launch_gemm<G_Y>(g, st));
    g.a = (const bf16_t*)xy;
    g.b = a.dec;
    g.ct = (int)cdiv(a.D, T256 / 2);
    g.ks = ks;
    g.zpart = (float*)zp;
    BDH_HIP_TRY(launch_gemm<G_Z>(g, st));
  }
  BDH_HIP_TRY(dispatch_per<ResF>((int)a.D, (const float*)zp, a.cur, a.next, M, (int)a.D, ks, st));
  if (launches) *launches += (ks_yz > 0 ? 5 : 6) + n_attn;
  return BDH_OK;
}

}  // namespace bdh
