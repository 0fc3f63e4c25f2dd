// Device-side helpers shared by the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __bf16 bf16_t;
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

// 2.0 * PI as the reference evaluates it in f32 (attention.rs:546, 565).
#define BDH_TWO_PI_F32 6.28318548202514648f

namespace bdh {

// --- RoPE phase, op order of attention.rs:544-546 --------------------------
//   raw = p * f ; phase = (raw - floor(raw)) * (2 pi)
// Every op rounds separately: contraction is off in these bodies (an FMA
// would subtract floor() from the unrounded product).  The active-row test
// frac != 0 must agree bit for bit with the reference's f32 arithmetic.
// raw - floor(raw) is exact for finite raw >= 0 (positions and frequencies
// are never negative), so v_fract_f32, which computes it in one instruction
// (and clamps below 1.0 only where the difference would round to 1.0), gives
// the same bits as the reference's two operations.
__device__ __forceinline__ float rope_frac(float p, float f) {
#pragma clang fp contract(off)
  const float raw = p * f;
  return __builtin_amdgcn_fractf(raw);
}
__device__ __forceinline__ float rope_phase(float p, float f) {
#pragma clang fp contract(off)
  return rope_frac(p, f) * BDH_TWO_PI_F32;
}

// Rotation of one (even, odd) pair, op order of attention.rs:488-501:
//   even' = even*cos + (-odd)*sin ; odd' = odd*cos + even*sin
__device__ __forceinline__ void rope_pair_exact(float even, float odd, float c, float s,
                                                float& out_even, float& out_odd) {
#pragma clang fp contract(off)
  out_even = even * c + (-odd) * s;
  out_odd = odd * c + even * s;
}

// bf16 <-> f32.  f32 -> bf16 is round-to-nearest-even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  bf16x2 r;
  r.x = (bf16_t)a;
  r.y = (bf16_t)b;
  return __builtin_bit_cast(uint32_t, r);
}
__device__ __forceinline__ float bf16_round(float a) { return (float)(bf16_t)a; }

// --- MFMA 32x32x16 bf16 (gfx950) ---------------------------------------------
// Operand fragments (8 bf16 per lane): lane l covers row/col (l & 31) and
// k = 8*(l >> 5) .. +7 of the 16-deep slice.  Accumulator (16 f32 per lane):
// col = l & 31, row = 8*(r >> 2) + 4*(l >> 5) + (r & 3).
__device__ __forceinline__ floatx16 mfma32(const bf16x8& a, const bf16x8& b, const floatx16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ int acc_row(int lane, int r) { return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3); }
__device__ __forceinline__ int acc_col(int lane) { return lane & 31; }

// --- MFMA 16x16x32 bf16 (gfx950) ---------------------------------------------
// Operand fragments (8 bf16 per lane): lane l covers row/col (l & 15) and
// k = 8*(l >> 4) .. +7 of the 32-deep slice.  Accumulator (4 f32 per lane):
// col = l & 15, row = 4*(l >> 4) + r.
__device__ __forceinline__ floatx4 mfma16(const bf16x8& a, const bf16x8& b, const floatx4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ int acc16_row(int lane, int r) { return 4 * (lane >> 4) + r; }
__device__ __forceinline__ int acc16_col(int lane) { return lane & 15; }
__device__ __forceinline__ floatx4 zero4() { return floatx4{0.0f, 0.0f, 0.0f, 0.0f}; }

// Wavefront index within the workgroup as a scalar (SGPR) value, so that
// branches on it are uniform scalar branches rather than exec-mask ones.
__device__ __forceinline__ int wave_id() {
  return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
}

__device__ __forceinline__ floatx16 zero16() {
  floatx16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.0f;
  return z;
}

}  // namespace bdh
