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

// The same rotation, two pairs a thread (16-byte loads and stores), rows
// taken by workgroups in a grid-stride loop over 4 workgroups a CU, each
// thread keeping RQ loads in flight.  Same per-pair arithmetic, so the same
// bits.  (The one-pair kernel above ran the fp32 C2 shape's 1.07 GB at
// 4.85 TB/s.)
constexpr int RQ = 4;
__global__ __launch_bounds__(256) void rope_rotate_f32_quad_kernel(const float4* __restrict__ x,
                                                                   const float4* __restrict__ freqs,
                                                                   float4* __restrict__ out, int64_t rows,
                                                                   int64_t T, int q, int64_t pos0, int fixed) {
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    const int64_t t = row % T;
    const float p = (float)(fixed ? pos0 : pos0 + t);
    const float4* xr = x + row * q;
    float4* orow = out + row * q;
    for (int k0 = (int)threadIdx.x; k0 < q; k0 += 256 * RQ) {
      floatx4 xv[RQ];
      float4 fv[RQ];
#pragma unroll
      for (int u = 0; u < RQ; ++u) {
        const int k = k0 + 256 * u;
        if (k < q) {
          xv[u] = __builtin_nontemporal_load(reinterpret_cast<const floatx4*>(xr) + k);
          fv[u] = freqs[k];
        }
      }
#pragma unroll
      for (int u = 0; u < RQ; ++u) {
        const int k = k0 + 256 * u;
        if (k >= q) continue;
        float s0, c0, s1, c1;
        sincosf(rope_phase(p, fv[u].x), &s0, &c0);
        sincosf(rope_phase(p, fv[u].z), &s1, &c1);
        float o0, o1, o2, o3;
        rope_pair_exact(xv[u][0], xv[u][1], c0, s0, o0, o1);
        rope_pair_exact(xv[u][2], xv[u][3], c1, s1, o2, o3);
        __builtin_nontemporal_store(floatx4{o0, o1, o2, o3}, reinterpret_cast<floatx4*>(orow) + k);
      }
    }
  }
}

hipError_t launch_rope_rotate_f32(const float* x, const float* freqs, float* out, int64_t S,
                                  int64_t T, int64_t N, int64_t pos0, int fixed,
                                  hipStream_t st) {
  const int64_t half = N / 2;
  const int64_t n = S * T * half;
  if (n == 0) return hipSuccess;
  const bool quad = N % 4 == 0 && N / 4 <= INT32_MAX && ((uintptr_t)x & 15) == 0 && ((uintptr_t)out & 15) == 0 &&
                    ((uintptr_t)freqs & 15) == 0;
  if (quad) {
    const int64_t rows = S * T;
    const int64_t wg = 4 * (int64_t)device_cus();
    hipLaunchKernelGGL(rope_rotate_f32_quad_kernel, dim3((unsigned)(rows < wg ? rows : wg)), dim3(256), 0, st,
                       (const float4*)x, (const float4*)freqs, (float4*)out, rows, T, (int)(N / 4), pos0, fixed);
  } else {
    hipLaunchKernelGGL(rope_rotate_f32_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                       st, x, freqs, out, S * T, T, half, pos0, fixed);
  }
  return hipGetLastError();
}

}  // namespace bdh
