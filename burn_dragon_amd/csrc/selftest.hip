// Check hook for the hand-written RoPE rotation (rot8_bf16 / rot8_f32 in
// bdh_bf16.h): the assembly block places its hazard wait states by hand, so
// its results are compared, bit for bit, with the same rotation written with
// the compiler's dot-product builtin (which schedules its own waits).
#include "bdh_bf16.h"

namespace bdh {
namespace {

__device__ __forceinline__ bf16x2 as_bf16x2(uint32_t w) { return __builtin_bit_cast(bf16x2, w); }

// (e, o) . (c, -s) and (o, e) . (c, s) per pair with __builtin_amdgcn_fdot2_f32_bf16.
__device__ __forceinline__ void rot8_builtin(uint4 x, uint4 cs, float (&out)[8]) {
  const uint32_t xs[4] = {x.x, x.y, x.z, x.w}, ts[4] = {cs.x, cs.y, cs.z, cs.w};
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const uint32_t swapped = (xs[p] >> 16) | (xs[p] << 16);
    const uint32_t neg_s = ts[p] ^ 0x80000000u;  // (c, -s): flip the high half's sign
    out[2 * p] = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(xs[p]), as_bf16x2(neg_s), 0.0f, false);
    out[2 * p + 1] = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(swapped), as_bf16x2(ts[p]), 0.0f, false);
  }
}

__global__ __launch_bounds__(256) void rot8_selftest_kernel(const uint4* __restrict__ x,
                                                            const uint4* __restrict__ cs,
                                                            uint4* __restrict__ bf_asm,
                                                            uint4* __restrict__ bf_ref,
                                                            float* __restrict__ f_asm,
                                                            float* __restrict__ f_ref, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const uint4 xv = x[i], cv = cs[i];
  bf_asm[i] = rot8_bf16(xv, cv);
  float a[8], r[8];
  rot8_f32(xv, cv, a);
  rot8_builtin(xv, cv, r);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    f_asm[i * 8 + e] = a[e];
    f_ref[i * 8 + e] = r[e];
  }
  bf_ref[i] = make_uint4(pack_bf16x2(r[0], r[1]), pack_bf16x2(r[2], r[3]), pack_bf16x2(r[4], r[5]),
                         pack_bf16x2(r[6], r[7]));
}

}  // namespace
}  // namespace bdh

using namespace bdh;

extern "C" bdh_status bdh_selftest_rot8(const void* x, const void* cs, void* out_bf16_asm,
                                        void* out_bf16_builtin, float* out_f32_asm,
                                        float* out_f32_builtin, int64_t n_chunks, void* stream) {
  if (!x || !cs || !out_bf16_asm || !out_bf16_builtin || !out_f32_asm || !out_f32_builtin)
    return fail(BDH_EINVAL, "null pointer");
  if (n_chunks <= 0 || n_chunks > ((int64_t)1 << 30)) return fail(BDH_EINVAL, "n_chunks out of range");
  for (const void* t : {x, cs, (const void*)out_bf16_asm, (const void*)out_bf16_builtin})
    if (((uintptr_t)t & 15) != 0) return fail(BDH_EINVAL, "chunk pointers must be 16-byte aligned");
  hipLaunchKernelGGL(rot8_selftest_kernel, dim3((unsigned)((n_chunks + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, (const uint4*)x, (const uint4*)cs, (uint4*)out_bf16_asm,
                     (uint4*)out_bf16_builtin, out_f32_asm, out_f32_builtin, n_chunks);
  BDH_HIP_TRY(hipGetLastError());
  return BDH_OK;
}
