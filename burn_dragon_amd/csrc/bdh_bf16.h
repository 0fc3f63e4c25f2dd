// Shared pieces of the bf16 MFMA prefill kernels (gram, state, ctx).
#pragma once

#include "bdh_internal.h"

namespace bdh {

// Score-block (gram) and state tiles are 256 x 256.
constexpr int T256 = 256;

__device__ __forceinline__ uint4 ldg16(const void* p) {
  return *reinterpret_cast<const uint4*>(p);
}
// 16-byte load at a wave-uniform base plus a 32-bit per-lane byte offset: the
// base stays in SGPRs and no 64-bit address math is done per lane.
__device__ __forceinline__ uint4 ldg16_off(const void* base, uint32_t byte_off) {
  return *reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(base) + byte_off);
}

// (even, odd) bf16 pair rotated by the packed bf16 (cos, sin) word csw:
//   re = e*c - o*s = dot2((e, o), (c, -s)) ; ro = e*s + o*c = dot2((e, o), (s, c))
// Through the compiler builtin only: written as inline assembly, a
// v_dot2_f32_bf16 result read two instructions later came back stale on
// gfx950 (the compiler cannot see the instruction's latency there).
__device__ __forceinline__ void rot_pair(uint32_t xw, uint32_t csw, float& re, float& ro) {
  const bf16x2 xv = __builtin_bit_cast(bf16x2, xw);
  const bf16x2 cms = __builtin_bit_cast(bf16x2, csw ^ 0x80000000u);
  const bf16x2 sc = __builtin_bit_cast(bf16x2, __builtin_amdgcn_alignbit(csw, csw, 16));
  re = __builtin_amdgcn_fdot2_f32_bf16(xv, cms, 0.0f, false);
  ro = __builtin_amdgcn_fdot2_f32_bf16(xv, sc, 0.0f, false);
}

// 8 bf16 (4 pairs) rotated (ROPE) and/or scaled by w, as f32.
template <bool ROPE>
__device__ __forceinline__ void prep8_f32(uint4 raw, uint4 cs, float w, bool scale,
                                          float (&out)[8]) {
  const uint32_t in[4] = {raw.x, raw.y, raw.z, raw.w};
  const uint32_t c[4] = {cs.x, cs.y, cs.z, cs.w};
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    float re, ro;
    if (ROPE) {
      rot_pair(in[p], c[p], re, ro);
    } else {
      re = bf16_lo(in[p]);
      ro = bf16_hi(in[p]);
    }
    if (scale) {
      re *= w;
      ro *= w;
    }
    out[2 * p] = re;
    out[2 * p + 1] = ro;
  }
}

// Same, repacked to 8 bf16 (RNE).  Without RoPE and scaling it is a copy.
template <bool ROPE>
__device__ __forceinline__ uint4 prep8(uint4 raw, uint4 cs, float w, bool scale) {
  if (!ROPE && !scale) return raw;
  float v[8];
  prep8_f32<ROPE>(raw, cs, w, scale, v);
  return make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                    pack_bf16x2(v[6], v[7]));
}

__device__ __forceinline__ float decay_pow(const float* decay, int64_t h, float e) {
  return decay ? powf(decay[h], e) : 1.0f;
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
  const uint32_t* cs;   // packed bf16 (cos, sin) [T, N/2], or null (x pre-rotated)
  const float* decay;   // [H] or null
  int64_t H, Hv, T, N, D, S;
  // gram units
  float* part;          // [KS, S, n_iv, Lp, Lp]
  int64_t L, Lp, n_iv;
  int ks, nb;           // N splits (N/32 a multiple of 4 ks); 256-row blocks per interval
  int gram_groups;      // S * ks * n_iv
  int gram_ids;         // workgroup ids reserved for gram units (prefill_gram_ids)
  // state units
  const bf16_t* vt;     // [B*Hv, Dp, Tp], zero past (D, T); Dp = D rounded up to 256
  const float* rho_in;  // [S, N, D] or null
  float* rho_out;       // [S, N, D]
  int64_t st_t0, st_Lc, Tp, Dp;  // Tp >= st_t0 + st_Lc rounded up to 64
  int state_units;      // prefill_state_units(S, N, D), or 0
  // readout units: partial (Q * d^r) rho_iv for the interval
  // [rd_t0, rd_t0 + rd_Lc), rho_iv the state at its start
  const float* rd_rho;  // [S, N, D]
  float* rd_part;       // [rd_kr, S, Lp, D] partials over the rd_kr N ranges
  int64_t rd_t0, rd_Lc;
  int rd_kr;            // N splits (N/32 a multiple of 2 rd_kr)
  int rd_units;         // prefill_readout_units(S, rd_Lc, D, rd_kr), or 0
};
hipError_t launch_prefill_mfma(const PrefillArgs& a, bool rope, hipStream_t st);
// Workgroup ids a gram launch needs for `groups` groups of nb-block
// intervals (ids are laid out so that one group's tiles share an XCD).
int prefill_gram_ids(int groups, int nb);
// State units of one interval.
int prefill_state_units(int64_t S, int64_t N, int64_t D);
// Readout units of one interval of Lc rows.
int prefill_readout_units(int64_t S, int64_t Lc, int64_t D, int kr);

}  // namespace bdh
