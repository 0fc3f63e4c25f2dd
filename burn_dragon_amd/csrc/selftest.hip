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

// ---------------------------------------------------------------------------
// HBM calibration kernels: the ceilings a decode step is compared against.
// A decode step reads and rewrites scattered 1 KiB rows of rho (one row per
// active neuron), which is neither a read nor a copy; these measure plain
// streams and a row RMW of the same granularity on this device.
namespace bdh {
namespace {

constexpr int kCalibBlock = 256;

__global__ __launch_bounds__(kCalibBlock) void calib_read_kernel(const float4* __restrict__ a,
                                                                 float* __restrict__ sink, int64_t n) {
  float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int64_t i = (int64_t)blockIdx.x * kCalibBlock + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kCalibBlock) {
    const float4 v = a[i];
    s.x += v.x; s.y += v.y; s.z += v.z; s.w += v.w;
  }
  // Never true for finite data; keeps the loads live without a store per thread.
  if (s.x == 1.5e38f && s.y == -1.5e38f) sink[0] = s.z + s.w;
}

__global__ __launch_bounds__(kCalibBlock) void calib_copy_kernel(const float4* __restrict__ a,
                                                                 float4* __restrict__ b, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * kCalibBlock + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kCalibBlock)
    b[i] = a[i];
}

__global__ __launch_bounds__(kCalibBlock) void calib_rmw_kernel(float4* __restrict__ a, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * kCalibBlock + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kCalibBlock) {
    float4 v = a[i];
    v.x += 1.0f;
    a[i] = v;
  }
}

// One wavefront per listed 1 KiB row (64 lanes x 16 B), four rows in flight
// per wavefront, rows taken in list order, written back with non-temporal
// stores (the decode step's store); an index outside [0, total_rows) is
// skipped.  (Measured: nontemporal stores take a 10 % random-row RMW from
// 4.8 to 5.4 TB/s on this device; one row in flight per wave with plain
// stores reached 4.8.)
constexpr int kRowsInFlight = 4;
__global__ __launch_bounds__(kCalibBlock) void calib_rmw_rows_kernel(float4* __restrict__ a,
                                                                     const int32_t* __restrict__ rows,
                                                                     int64_t n_rows, int64_t total_rows) {
  const int lane = threadIdx.x & 63;
  const int64_t waves = (int64_t)gridDim.x * (kCalibBlock / 64);
  for (int64_t r = ((int64_t)blockIdx.x * (kCalibBlock / 64) + (threadIdx.x >> 6)) * kRowsInFlight; r < n_rows;
       r += waves * kRowsInFlight) {
    int64_t row[kRowsInFlight];
    float4 v[kRowsInFlight];
#pragma unroll
    for (int j = 0; j < kRowsInFlight; ++j) {
      row[j] = r + j < n_rows ? rows[r + j] : -1;
      if (row[j] >= total_rows) row[j] = -1;
    }
#pragma unroll
    for (int j = 0; j < kRowsInFlight; ++j)
      if (row[j] >= 0) v[j] = a[row[j] * 64 + lane];
#pragma unroll
    for (int j = 0; j < kRowsInFlight; ++j)
      if (row[j] >= 0) {
        v[j].x += 1.0f;
        __builtin_nontemporal_store(floatx4{v[j].x, v[j].y, v[j].z, v[j].w},
                                    reinterpret_cast<floatx4*>(a + row[j] * 64 + lane));
      }
  }
}

// MFMA rate with register operands: each wave keeps 8 independent
// accumulator chains of one MFMA shape and issues `iters` rounds of 8; the
// operands never leave registers, so the launch measures the matrix cores
// alone.  Two 4-wave workgroups per CU (two waves per SIMD).
template <bool K32>
__global__ __launch_bounds__(kCalibBlock, 2) void calib_mfma_kernel(float* __restrict__ sink, int64_t iters) {
  const int lane = threadIdx.x & 63;
  bf16x8 a, b;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    a[e] = (bf16_t)(0.001f * (float)((lane + e) & 7));
    b[e] = (bf16_t)(0.002f * (float)((lane * 3 + e) & 7));
  }
  float tot = 0.0f;
  if (K32) {
    floatx4 acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = zero4();
    for (int64_t i = 0; i < iters; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] = mfma16(a, b, acc[j]);
#pragma unroll
    for (int j = 0; j < 8; ++j) tot += acc[j][0] + acc[j][3];
  } else {
    floatx16 acc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[j][r] = 0.0f;
    for (int64_t i = 0; i < iters; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[j] = mfma32(a, b, acc[j]);
#pragma unroll
    for (int j = 0; j < 4; ++j) tot += acc[j][0] + acc[j][15];
  }
  if (tot == -1.5e38f) sink[0] = tot;  // never true; keeps the chains live
}

// The fp32 matrix rate (v_mfma_f32_32x32x2f32, the fp32 path's GEMMs): 4
// independent accumulator chains per wave.
__global__ __launch_bounds__(kCalibBlock, 2) void calib_mfma_f32_kernel(float* __restrict__ sink, int64_t iters) {
  const int lane = threadIdx.x & 63;
  const float a = 0.001f * (float)(lane & 7), b = 0.002f * (float)((lane * 3) & 7);
  floatx16 acc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[j][r] = 0.0f;
  for (int64_t i = 0; i < iters; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc[j], 0, 0, 0);
  float tot = 0.0f;
#pragma unroll
  for (int j = 0; j < 4; ++j) tot += acc[j][0] + acc[j][15];
  if (tot == -1.5e38f) sink[0] = tot;  // never true; keeps the chains live
}

}  // namespace
}  // namespace bdh

extern "C" bdh_status bdh_calib_hbm(int32_t kind, void* buf, void* buf2, int64_t bytes,
                                    const int32_t* rows, int64_t n_rows, void* stream) {
  if (!buf || bytes <= 0 || (bytes & 1023) != 0) return fail(BDH_EINVAL, "bytes must be a positive multiple of 1024");
  if (((uintptr_t)buf & 15) != 0 || (buf2 && ((uintptr_t)buf2 & 15) != 0))
    return fail(BDH_EINVAL, "buffers must be 16-byte aligned");
  const int64_t n = bytes / 16;
  const hipStream_t st = (hipStream_t)stream;
  // Streams: 4 workgroups of 256 per CU, grid-stride loops cover the rest
  // (8 per CU read and copied 5-15 % slower here); rows: 16 per CU.
  const dim3 grid((unsigned)(4 * device_cus())), block(kCalibBlock);
  const dim3 grid_rows((unsigned)(16 * device_cus()));
  switch (kind) {
    case BDH_CALIB_READ:
      if (!buf2) return fail(BDH_EINVAL, "read needs a 16-byte sink in buf2");
      hipLaunchKernelGGL(calib_read_kernel, grid, block, 0, st, (const float4*)buf, (float*)buf2, n);
      break;
    case BDH_CALIB_COPY:
      if (!buf2) return fail(BDH_EINVAL, "copy needs a destination in buf2");
      hipLaunchKernelGGL(calib_copy_kernel, grid, block, 0, st, (const float4*)buf, (float4*)buf2, n);
      break;
    case BDH_CALIB_RMW:
      hipLaunchKernelGGL(calib_rmw_kernel, grid, block, 0, st, (float4*)buf, n);
      break;
    case BDH_CALIB_RMW_ROWS:
      if (!rows || n_rows <= 0) return fail(BDH_EINVAL, "rmw_rows needs row indices");
      hipLaunchKernelGGL(calib_rmw_rows_kernel, grid_rows, block, 0, st, (float4*)buf, rows, n_rows,
                         bytes / 1024);
      break;
    default:
      return fail(BDH_EINVAL, "unknown calibration kind");
  }
  BDH_HIP_TRY(hipGetLastError());
  return BDH_OK;
}

extern "C" bdh_status bdh_calib_mfma(int32_t kind, int64_t iters, float* sink, double* flop_out, void* stream) {
  if (!sink || !flop_out) return fail(BDH_EINVAL, "null pointer");
  if (iters <= 0 || iters > ((int64_t)1 << 24)) return fail(BDH_EINVAL, "iters out of range");
  const dim3 grid((unsigned)(2 * device_cus())), block(kCalibBlock);
  const double waves = (double)grid.x * (kCalibBlock / 64);
  switch (kind) {
    case BDH_CALIB_MFMA_16X16X32_BF16:
      hipLaunchKernelGGL(calib_mfma_kernel<true>, grid, block, 0, (hipStream_t)stream, sink, iters);
      *flop_out = waves * (double)iters * 8.0 * (2.0 * 16 * 16 * 32);
      break;
    case BDH_CALIB_MFMA_32X32X16_BF16:
      hipLaunchKernelGGL(calib_mfma_kernel<false>, grid, block, 0, (hipStream_t)stream, sink, iters);
      *flop_out = waves * (double)iters * 4.0 * (2.0 * 32 * 32 * 16);
      break;
    case BDH_CALIB_MFMA_32X32X2_F32:
      hipLaunchKernelGGL(calib_mfma_f32_kernel, grid, block, 0, (hipStream_t)stream, sink, iters);
      *flop_out = waves * (double)iters * 4.0 * (2.0 * 32 * 32 * 2);
      break;
    default:
      return fail(BDH_EINVAL, "unknown MFMA calibration kind");
  }
  BDH_HIP_TRY(hipGetLastError());
  return BDH_OK;
}
