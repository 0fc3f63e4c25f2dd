// RoPE rotation for the fp32 path, in the reference's exact f32 op order
// (attention.rs:540-550): raw = p * f, (raw - floor(raw)) * 2pi, cos/sin,
// then x*cos + rotated*sin.
#include "bdh_internal.h"

namespace bdh {

// One thread per (row, pair): out = [even*c - odd*s, odd*c + even*s], each op
// rounded separately like the reference's element-wise tensor ops.
__global__ __launch_bounds__(256) void rope_rotate_f32_kernel(const float* __restrict__ x,
                                                              const float* __restrict__ freqs,
                                                              float* __restrict__ out,
                                                              int64_t rows, int64_t T,
                                                              int64_t half, int64_t pos0,
                                                              int fixed) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= rows * half) return;
  const int64_t row = i / half;          // s * T + t
  const int64_t k = i - row * half;
  const int64_t t = row % T;
  const float p = (float)(fixed ? pos0 : pos0 + t);
  const float2 xv = reinterpret_cast<const float2*>(x)[i];
  const float ph = rope_phase(p, freqs[2 * k]);
  float s, c;
  sincosf(ph, &s, &c);
  float e, o;
  rope_pair_exact(xv.x, xv.y, c, s, e, o);
  reinterpret_cast<float2*>(out)[i] = make_float2(e, o);
}

hipError_t launch_rope_rotate_f32(const float* x, const float* freqs, float* out, int64_t S,
                                  int64_t T, int64_t N, int64_t pos0, int fixed,
                                  hipStream_t st) {
  const int64_t half = N / 2;
  const int64_t n = S * T * half;
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(rope_rotate_f32_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     st, x, freqs, out, S * T, T, half, pos0, fixed);
  return hipGetLastError();
}

}  // namespace bdh
