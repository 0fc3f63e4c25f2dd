// Shared pieces of the bf16 MFMA prefill kernels (gram, state, ctx).
#pragma once

#include "bdh_internal.h"

namespace bdh {

// Tile edge of the MFMA units: 256 rows of gram / readout tiles and of
// v^T padding, 128 = T256 / 2 their column blocks and state neuron blocks.
constexpr int T256 = 256;

__device__ __forceinline__ uint4 ldg16(const void* p) {
  return *reinterpret_cast<const uint4*>(p);
}
// 16-byte load at a wave-uniform base plus a 32-bit per-lane byte offset: the
// base stays in SGPRs and no 64-bit address math is done per lane.
__device__ __forceinline__ uint4 ldg16_off(const void* base, uint32_t byte_off) {
  return *reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(base) + byte_off);
}

// RoPE rotation of 4 (even, odd) bf16 pairs x.{x,y,z,w} by the packed bf16
// (cos, sin) words cs.{x,y,z,w} (rope_cs4 below):
//   re = e*c - o*s = (e, o) . (c, s) with the high product negated (neg_hi)
//   ro = o*c + e*s = (o, e) . (c, s), (o, e) = x rotated by 16 bits
// Written in assembly for the three-operand v_dot2_f32_bf16 and its neg_hi
// modifier (4 VALU instructions a pair; the builtin selects v_dot2c, which
// needs a zeroed accumulator copy and an explicit negation, 7 a pair).  The
// hardware needs 3 wait states between a v_dot2 that writes a VGPR and
// another VALU instruction that reads it, and the compiler cannot see inside
// the assembly, so every such read below is at least 3 instructions (with
// the s_nop, 5) after its write, and the f32 form ends with s_nop 2.  Results
// match the builtin dot product bit for bit (fp32 dot, round to nearest even
// on packing).
__device__ __forceinline__ uint4 rot8_bf16(uint4 x, uint4 cs) {
  uint4 o;
  float t0, t1, t2, t3, t4, t5, t6, t7;
  uint32_t w0, w1, w2, w3;
  asm("v_alignbit_b32 %12, %16, %16, 16\n\t"
      "v_alignbit_b32 %13, %17, %17, 16\n\t"
      "v_alignbit_b32 %14, %18, %18, 16\n\t"
      "v_alignbit_b32 %15, %19, %19, 16\n\t"
      "v_dot2_f32_bf16 %4, %16, %20, 0 neg_hi:[0,1,0]\n\t"
      "v_dot2_f32_bf16 %5, %12, %20, 0\n\t"
      "v_dot2_f32_bf16 %6, %17, %21, 0 neg_hi:[0,1,0]\n\t"
      "v_dot2_f32_bf16 %7, %13, %21, 0\n\t"
      "v_dot2_f32_bf16 %8, %18, %22, 0 neg_hi:[0,1,0]\n\t"
      "v_dot2_f32_bf16 %9, %14, %22, 0\n\t"
      "v_dot2_f32_bf16 %10, %19, %23, 0 neg_hi:[0,1,0]\n\t"
      "v_dot2_f32_bf16 %11, %15, %23, 0\n\t"
      "s_nop 1\n\t"
      "v_cvt_pk_bf16_f32 %0, %4, %5\n\t"
      "v_cvt_pk_bf16_f32 %1, %6, %7\n\t"
      "v_cvt_pk_bf16_f32 %2, %8, %9\n\t"
      "v_cvt_pk_bf16_f32 %3, %10, %11"
      : "=v"(o.x), "=v"(o.y), "=v"(o.z), "=v"(o.w), "=&v"(t0), "=&v"(t1), "=&v"(t2), "=&v"(t3),
        "=&v"(t4), "=&v"(t5), "=&v"(t6), "=&v"(t7), "=&v"(w0), "=&v"(w1), "=&v"(w2), "=&v"(w3)
      : "v"(x.x), "v"(x.y), "v"(x.z), "v"(x.w), "v"(cs.x), "v"(cs.y), "v"(cs.z), "v"(cs.w));
  return o;
}

// Same rotation, results left in f32: out[2p] = re, out[2p + 1] = ro of pair p.
__device__ __forceinline__ void rot8_f32(uint4 x, uint4 cs, float (&out)[8]) {
  uint32_t w0, w1, w2, w3;
  asm("v_alignbit_b32 %8, %12, %12, 16\n\t"
      "v_alignbit_b32 %9, %13, %13, 16\n\t"
      "v_alignbit_b32 %10, %14, %14, 16\n\t"
      "v_alignbit_b32 %11, %15, %15, 16\n\t"
      "v_dot2_f32_bf16 %0, %12, %16, 0 neg_hi:[0,1,0]\n\t"
      "v_dot2_f32_bf16 %1, %8, %16, 0\n\t"
      "v_dot2_f32_bf16 %2, %13, %17, 0 neg_hi:[0,1,0]\n\t"
      "v_dot2_f32_bf16 %3, %9, %17, 0\n\t"
      "v_dot2_f32_bf16 %4, %14, %18, 0 neg_hi:[0,1,0]\n\t"
      "v_dot2_f32_bf16 %5, %10, %18, 0\n\t"
      "v_dot2_f32_bf16 %6, %15, %19, 0 neg_hi:[0,1,0]\n\t"
      "v_dot2_f32_bf16 %7, %11, %19, 0\n\t"
      "s_nop 2"
      : "=&v"(out[0]), "=&v"(out[1]), "=&v"(out[2]), "=&v"(out[3]), "=&v"(out[4]), "=&v"(out[5]),
        "=&v"(out[6]), "=&v"(out[7]), "=&v"(w0), "=&v"(w1), "=&v"(w2), "=&v"(w3)
      : "v"(x.x), "v"(x.y), "v"(x.z), "v"(x.w), "v"(cs.x), "v"(cs.y), "v"(cs.z), "v"(cs.w));
}

// 8 bf16 (4 pairs) rotated (ROPE) and/or scaled by w, as f32.
template <bool ROPE>
__device__ __forceinline__ void prep8_f32(uint4 raw, uint4 cs, float w, bool scale,
                                          float (&out)[8]) {
  if (ROPE) {
    rot8_f32(raw, cs, out);
  } else {
    const uint32_t in[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      out[2 * p] = bf16_lo(in[p]);
      out[2 * p + 1] = bf16_hi(in[p]);
    }
  }
  if (scale) {
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] *= w;
  }
}

// Same, repacked to 8 bf16 (RNE).  Without RoPE and scaling it is a copy.
template <bool ROPE>
__device__ __forceinline__ uint4 prep8(uint4 raw, uint4 cs, float w, bool scale) {
  if (!ROPE && !scale) return raw;
  if (ROPE && !scale) return rot8_bf16(raw, cs);
  float v[8];
  prep8_f32<ROPE>(raw, cs, w, scale, v);
  return make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                    pack_bf16x2(v[6], v[7]));
}

__device__ __forceinline__ float decay_pow(const float* decay, int64_t h, float e) {
  return decay ? powf(decay[h], e) : 1.0f;
}

// d^e for an integer e >= 0, as the reference's repeated products give it
// (recurrent.rs:415): 1 at e = 0 (d = 0 included), exp2(e log2 |d|)
// otherwise, negated for d < 0 and odd e.  l2a = log2|d| (-inf for d = 0,
// where exp2 gives the 0 of 0^e, e > 0).
__device__ __forceinline__ float decay_log2(float d) { return log2f(fabsf(d)); }
__device__ __forceinline__ float decay_pow_int(float d, float l2a, int e) {
  if (e == 0) return 1.0f;
  const float m = exp2f((float)e * l2a);
  return (d < 0.0f && (e & 1)) ? -m : m;
}

// --- launch interface of the gram + state kernel (mfma_prefill.hip) --------
// One launch runs up to three kinds of work unit, heaviest first:
//   gram units  (stream, N range kp, interval iv, 256-row x 128-column tile
//               touching the interval's lower triangle): part[kp, s, iv] =
//               the tile of tril(-1)(Q Q^T * d^(r-c)) summed over the kp-th
//               N range;
//   state units (stream, 128-neuron block, 256-column block) of the
//               interval [st_t0, st_t0 + st_Lc):
//               rho_out = rho_in * d^Lc + (Q * d^(Lc-r))^T V.
//   readout units (stream, 256-row block, 128-column block, N range) of
//               the interval [rd_t0, rd_t0 + rd_Lc):
//               rd_part[kr] = (Q * d^r) rho_iv over the kr-th N range.
// Any kind may be absent (gram_ids, rd_units or state_units == 0).
struct PrefillArgs {
  const bf16_t* x;      // [S, T, N]
  const float* freqs;   // RoPE frequencies [N] (rotating kernels), or null (x pre-rotated)
  int64_t pos0;         // position of token 0 (Sequential), or of every token (fixed)
  int fixed;
  const float* decay;   // [H] or null
  int64_t H, Hv, T, N, D, S;
  // gram units
  float* part;          // [KS, S, n_iv, Lp, Lp] (bf16 with part16, snap_wide_kernel only)
  int part16;
  int64_t L, Lp, n_iv;
  int ks, nb;           // N splits (N/32 a multiple of 4 ks); 256-row blocks per interval
  int gram_groups;      // S * ks * n_iv
  int gram_ids;         // workgroup ids of the gram groups (prefill_gram_ids / snap_wide_ids)
  // state units
  const bf16_t* vt;     // v^T [B*Hv, Tp/32, Dp, 32] (step-major), zero past (D, T); Dp = D rounded up to 256
  const float* rho_in;  // [S, N, D] or null
  float* rho_out;       // [S, N, D]
  int64_t st_t0, st_Lc, Tp, Dp;  // Tp >= st_t0 + st_Lc rounded up to 64
  int state_units;      // prefill_state_units(S, N, D), or 0
  int rho_stream;       // rho_out is the caller's final state (streaming stores)
  // readout units: partial (Q * d^r) rho_iv for the interval
  // [rd_t0, rd_t0 + rd_Lc), rho_iv the state at its start
  const float* rd_rho;  // [S, N, D]
  float* rd_part;       // [rd_kr, S, Lp, D] partials over the rd_kr N ranges
  int64_t rd_t0, rd_Lc;
  int rd_kr;            // N splits (N/32 a multiple of 2 rd_kr)
  int rd_units;         // prefill_readout_units(S, rd_Lc, D, rd_kr), or 0
  // add units: ctx[s, add_t0 + t, :] += sum of the previous interval's rd_kr
  // readout partials (add_src, same layout as rd_part), run in this launch's
  // tail
  const float* add_src;
  float* add_ctx;       // [S, T, D]
  int64_t add_t0, add_Lc;
  int add_units;
  // snapshot mode (snap_wide.hip; rd_snap set, x pre-rotated, no decay):
  // rd_pg readout tiles per gram group, for every interval iv >= rd_iv0, over
  // the group's N range (rd_kr = ks): rd_part [rd_kr, S, T, D] = q rho_iv,
  // rho_iv from rd_snap [n_iv, S, D, N] bf16 (prefill_carry_kernel)
  const bf16_t* rd_snap;
  int64_t rd_iv0;
  int rd_pg;
};

// --- launch interface of the state-carry kernel (carry_prefill.hip) --------
// One workgroup per (stream, 128-neuron block, 256-column block) walks every
// token of the call with its block of rho in registers (no decay):
// rho_{iv+1} = rho_iv + Q_iv^T V_iv.  It writes snap[iv] = rho_iv as bf16
// [d][n] for every interval with a carried state (iv >= 1, and iv = 0 when
// rho_in is set), the final rho in f32, and, when it rotates, q = RoPE(x).
struct CarryArgs {
  const bf16_t* x;      // [S, T, N]
  const float* freqs;   // RoPE frequencies [N], or null (x already rotated; q unused)
  int64_t pos0;
  int fixed;
  int64_t H, Hv, T, N, D, S, L, Tp, Dp;  // L a multiple of 128; Tp = T rounded up to 128
  const bf16_t* vt;     // v^T [B*Hv, Tp/32, Dp, 32] (step-major), zero past (D, T)
  const float* rho_in;  // [S, N, D] or null
  float* rho_out;       // [S, N, D] (may be rho_in)
  bf16_t* snap;         // [n_iv, S, D, N]
  bf16_t* q;            // [S, T, N] rotated queries (freqs set)
  const float* decay;   // [H] or null (ones)
};
int prefill_carry_units(int64_t S, int64_t N, int64_t Dp);
// Gram and readout tiles of the state-carry form in 8-wave workgroups
// (snap_wide.hip): PrefillArgs in snapshot mode (rd_snap, rd_iv0, rd_pg =
// readout tiles per group = 256-row blocks x 256-column blocks, rd_kr = ks),
// gram_ids = snap_wide_ids(groups, nb, rd_pg).  With rd_pg = 0 (no readout
// tiles) it is the gram of a context-only call on pre-rotated queries.
int snap_wide_ids(int groups, int nb, int rd_pg);
hipError_t launch_snap_wide(const PrefillArgs& a, hipStream_t st);
// Gram tiles of a context-only call (wide_gram.hip): PrefillArgs as for
// snap_wide with rd_pg = 0, in 4-wave workgroups (a 128 x 128 block a wave);
// wide_gram_fits says whether a's shape suits them (one interval, no decay,
// pre-rotated queries, whole 256-row blocks, an even step count per N
// range), gram_ids = wide_gram_ids(groups, nb).
bool wide_gram_fits(const PrefillArgs& a);
int wide_gram_ids(int groups, int nb);
hipError_t launch_wide_gram(const PrefillArgs& a, hipStream_t st);
hipError_t launch_prefill_carry(const CarryArgs& a, hipStream_t st);

// RoPE position of token t of the call (attention.rs:488-501 with the
// Sequential or Fixed positions of the call): exact in f32 below 2^24.
__device__ __forceinline__ float rope_pos(const PrefillArgs& a, int64_t t) {
  return (float)(a.fixed ? a.pos0 : a.pos0 + t);
}
// Frequencies of the 4 (even, odd) pairs of 8 neurons starting at f (one per
// pair: the even neuron's; 16-byte aligned).
__device__ __forceinline__ void load_freq4(const float* f, float (&out)[4]) {
  const float4 a = *reinterpret_cast<const float4*>(f);
  const float4 b = *reinterpret_cast<const float4*>(f + 4);
  out[0] = a.x;
  out[1] = a.z;
  out[2] = b.x;
  out[3] = b.z;
}
// Packed bf16 (cos, sin) words of the 4 pairs at position p: the phase
// frac(p f) in the reference's f32 op order; v_cos_f32 / v_sin_f32 take
// their argument in revolutions (error ~1e-6, far below the bf16 rounding).
__device__ __forceinline__ uint4 rope_cs4(float p, const float (&f)[4]) {
  uint32_t w[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float fr = rope_frac(p, f[j]);
    w[j] = pack_bf16x2(__builtin_amdgcn_cosf(fr), __builtin_amdgcn_sinf(fr));
  }
  return make_uint4(w[0], w[1], w[2], w[3]);
}
hipError_t launch_prefill_mfma(const PrefillArgs& a, bool rope, hipStream_t st);
// Gram and state units of a one-interval RoPE call without decay or carried
// state, T a multiple of 256, in 768-thread workgroups with wave roles
// (roles_prefill.hip): PrefillArgs with n_iv = 1, gram_ids =
// prefill_roles_gram_ids(S * ks, nb), state_units =
// prefill_roles_state_units(S, N, Dp) or 0; partials as launch_prefill_mfma's.
bool prefill_roles_fits(const PrefillArgs& a);
int prefill_roles_gram_ids(int groups, int nb);
int prefill_roles_state_units(int64_t S, int64_t N, int64_t Dp);
hipError_t launch_prefill_roles(const PrefillArgs& a, hipStream_t st);
// Workgroup ids a gram launch needs for `groups` groups of nb-block
// intervals (ids are laid out so that one group's tiles share an XCD).
int prefill_gram_ids(int groups, int nb);
// State units of one interval.
int prefill_state_units(int64_t S, int64_t N, int64_t D);
// Readout units of one interval of Lc rows.
int prefill_readout_units(int64_t S, int64_t Lc, int64_t D, int kr);

}  // namespace bdh
