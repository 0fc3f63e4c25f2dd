// Shared pieces of the bf16 MFMA prefill kernels (gram, state, ctx).
#pragma once

#include "bdh_internal.h"

namespace bdh {

// Tile geometry of the 256x256 gram / state kernels: 8 waves (2 per SIMD),
// each owning a 64x128 block of the tile (2 x 4 MFMA 32x32 accumulators).
constexpr int T256 = 256;
constexpr int T256_THREADS = 512;
constexpr int T256_BK = 32;                // k step
constexpr int T256_LDP = T256_BK + 8;      // padded LDS pitch (bf16), 80 B rows

__device__ __forceinline__ uint4 ldg16(const void* p) {
  return *reinterpret_cast<const uint4*>(p);
}

// (even, odd) bf16 pair rotated by the packed bf16 (cos, sin) word csw:
//   re = e*c - o*s = dot2((e,o), (c,-s)) ; ro = e*s + o*c = dot2((e,o), (s,c))
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

// --- launch interfaces ---------------------------------------------------------
struct GramArgs {
  const bf16_t* x;
  const uint32_t* cs;   // packed bf16 (cos, sin) [T, N/2] or null
  float* part;          // [KS, S, n_iv, Lp, Lp]
  const float* decay;
  int64_t H, T, N, L, Lp, S, n_iv;
  int ks, tiles_per_iv;
};
hipError_t launch_gram(const GramArgs& g, bool rope, hipStream_t st);

struct StateArgs {
  const bf16_t* x;
  const uint32_t* cs;
  const bf16_t* vt;   // [B*Hv, D, Tp]
  const float* rho_in;
  float* rho_out;
  const float* decay;
  int64_t H, Hv, T, N, D, t0, L, Tp, S;
};
hipError_t launch_state(const StateArgs& a, bool rope, hipStream_t st);

}  // namespace bdh
