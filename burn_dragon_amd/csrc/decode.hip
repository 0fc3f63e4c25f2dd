// Sparse decode step on gfx950 (fp32).  One launch per token:
//   A = active rows of rot(x)   (x_i != 0, or x_{i^1} != 0 and frac(p f_i) != 0)
//   a = rot(x)[A] . rho[A, :]   (read before the update)
//   rho[A, :] += rot(x)[A]^T v
// G 1024-thread workgroups per (batch, head) stream, each owning a range of
// N / G rows (G grows while the grid stays within one workgroup per CU).
// A workgroup compacts its range's active rows (8 rows per thread, wavefront
// prefix scan with DPP shuffles, workgroup offsets through LDS) into an LDS
// list (ascending), then its 16 waves stream exactly those rho rows: a whole
// 1 KiB row per wave per load at D = 256 (float4 per lane), 8 rows in flight
// per wave.  The readout is reduced across waves in LDS in a fixed order;
// with G > 1 the range partials (and range lists) go to scratch and a
// finalize kernel sums them (and concatenates the lists) in range order, so
// results are deterministic and no atomics or cross-workgroup fences are
// needed.  Rows outside A are never read or written.
#include "bdh_internal.h"

namespace bdh {
namespace {

constexpr int DR_THREADS = 1024;
constexpr int DR_WAVES = DR_THREADS / 64;
constexpr int DR_SEG = 8192;       // rows compacted per pass (LDS list capacity)
constexpr int DR_ROWS_PER_THREAD = DR_SEG / DR_THREADS;
constexpr int DR_UNROLL = 8;

struct DecodeKernelArgs {
  const float* x;
  const float* v;
  float* rho;
  const float* freqs;
  float* a_out;       // G == 1: [S, D]; else range partials [S, G, D]
  int32_t* idx_out;   // G == 1: [S, N]; else range lists at their first row [S, N]
  int32_t* cnt_out;   // G == 1: [S];    else range counts [S, G]
  int H, Hv, N, D;
  int G, rows;        // ranges per stream, rows per range (a multiple of 8)
  float pos;
};

template <bool VEC4>
struct ColBlock;
template <>
struct ColBlock<true> {
  static constexpr int W = 256;
};
template <>
struct ColBlock<false> {
  static constexpr int W = 64;
};

template <bool ROPE, bool VEC4>
__global__ __launch_bounds__(DR_THREADS) void decode_kernel(DecodeKernelArgs p) {
  constexpr int CB = ColBlock<VEC4>::W;
  __shared__ int32_t lidx[DR_SEG];
  __shared__ float lval[DR_SEG];
  __shared__ __attribute__((aligned(16))) float red[DR_WAVES * CB];
  __shared__ int32_t wtot[DR_WAVES];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t s = blockIdx.x / p.G;
  const int g = (int)(blockIdx.x - s * p.G);
  const int r0 = g * p.rows, r1 = min(p.N, r0 + p.rows);
  const int64_t b = s / p.H, h = s - b * p.H;
  const float* xs = p.x + s * p.N;
  const float* vs = p.v + (b * p.Hv + (p.Hv == 1 ? 0 : h)) * p.D;
  float* rho_s = p.rho + s * (int64_t)p.N * p.D;
  int done = 0;  // active rows listed so far (first column block only)
  int32_t* idx_s = p.idx_out ? p.idx_out + s * p.N + (p.G > 1 ? r0 : 0) : nullptr;
  float* a_s = p.a_out + (s * p.G + g) * p.D;

  for (int cb = 0; cb < p.D; cb += CB) {
    const bool first = cb == 0;
    const int c = VEC4 ? cb + lane * 4 : cb + lane;
    const bool cv = c < p.D;
    float4 vv = make_float4(0, 0, 0, 0), acc = make_float4(0, 0, 0, 0);
    if (cv) {
      if (VEC4) vv = *reinterpret_cast<const float4*>(vs + c);
      else vv.x = vs[c];
    }

    for (int seg0 = r0; seg0 < r1; seg0 += DR_SEG) {
      const int seg_end = min(r1, seg0 + DR_SEG);
      // ---- compaction of rows [seg0, seg_end) ----
      const int base = seg0 + tid * DR_ROWS_PER_THREAD;
      float r[DR_ROWS_PER_THREAD];
      unsigned m = 0;
      // A thread's 8 rows hold 4 whole (even, odd) pairs.  With N a multiple
      // of 8 they are one aligned 32-byte block of x (and of the
      // frequencies): two 16-byte loads each instead of 24 scalar loads.
      float xv[DR_ROWS_PER_THREAD], fv[DR_ROWS_PER_THREAD];
      const bool blk = (p.N & 7) == 0 && base < seg_end &&
                       ((reinterpret_cast<uintptr_t>(p.x) | reinterpret_cast<uintptr_t>(p.freqs)) & 15) == 0;
      if (blk) {
        *reinterpret_cast<float4*>(&xv[0]) = *reinterpret_cast<const float4*>(xs + base);
        *reinterpret_cast<float4*>(&xv[4]) = *reinterpret_cast<const float4*>(xs + base + 4);
        if (ROPE) {
          *reinterpret_cast<float4*>(&fv[0]) = *reinterpret_cast<const float4*>(p.freqs + base);
          *reinterpret_cast<float4*>(&fv[4]) = *reinterpret_cast<const float4*>(p.freqs + base + 4);
        }
      }
#pragma unroll
      for (int e = 0; e < DR_ROWS_PER_THREAD; ++e) {
        const int i = base + e;
        r[e] = 0.0f;
        if (i < seg_end) {
          const float xi = blk ? xv[e] : xs[i];
          bool on;
          if (ROPE) {
            const float xp = blk ? xv[e ^ 1] : xs[i ^ 1];
            const float fi = blk ? fv[e] : p.freqs[i];
            on = xi != 0.0f || (xp != 0.0f && rope_frac(p.pos, fi) != 0.0f);
            if (on) {
              float sn, cs, ev, od;
              sincosf(rope_phase(p.pos, fi), &sn, &cs);
              if ((i & 1) == 0) rope_pair_exact(xi, xp, cs, sn, ev, od), r[e] = ev;
              else rope_pair_exact(xp, xi, cs, sn, ev, od), r[e] = od;
            }
          } else {
            on = xi != 0.0f;
            r[e] = xi;
          }
          if (on) m |= 1u << e;
        }
      }
      const int cnt = __popc(m);
      int incl = cnt;
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const int y = __shfl_up(incl, d, 64);
        if (lane >= d) incl += y;
      }
      if (lane == 63) wtot[wave] = incl;
      __syncthreads();
      int off = 0, seg_total = 0;
#pragma unroll
      for (int w = 0; w < DR_WAVES; ++w) {
        const int t = wtot[w];
        off += w < wave ? t : 0;
        seg_total += t;
      }
      int pos = off + incl - cnt;
#pragma unroll
      for (int e = 0; e < DR_ROWS_PER_THREAD; ++e)
        if ((m >> e) & 1u) {
          lidx[pos] = base + e;
          lval[pos] = r[e];
          ++pos;
        }
      __syncthreads();
      if (first) {
        if (idx_s)
          for (int k = tid; k < seg_total; k += DR_THREADS) idx_s[done + k] = lidx[k];
        done += seg_total;
      }

      // ---- stream the active rows: a += r rho_row ; rho_row += r v ----
      for (int k0 = wave; k0 < seg_total; k0 += DR_WAVES * DR_UNROLL) {
        float4 row[DR_UNROLL];
        float rv[DR_UNROLL];
        float* ptr[DR_UNROLL];
#pragma unroll
        for (int u = 0; u < DR_UNROLL; ++u) {
          const int k = k0 + u * DR_WAVES;
          const bool ok = k < seg_total && cv;
          rv[u] = k < seg_total ? lval[k] : 0.0f;
          ptr[u] = rho_s + (int64_t)(k < seg_total ? lidx[k] : 0) * p.D + c;
          if (VEC4) row[u] = ok ? *reinterpret_cast<const float4*>(ptr[u]) : make_float4(0, 0, 0, 0);
          else row[u] = make_float4(ok ? *ptr[u] : 0.0f, 0, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < DR_UNROLL; ++u) {
          const int k = k0 + u * DR_WAVES;
          acc.x = fmaf(row[u].x, rv[u], acc.x);
          float4 nr;
          nr.x = fmaf(rv[u], vv.x, row[u].x);
          if (VEC4) {
            acc.y = fmaf(row[u].y, rv[u], acc.y);
            acc.z = fmaf(row[u].z, rv[u], acc.z);
            acc.w = fmaf(row[u].w, rv[u], acc.w);
            nr.y = fmaf(rv[u], vv.y, row[u].y);
            nr.z = fmaf(rv[u], vv.z, row[u].z);
            nr.w = fmaf(rv[u], vv.w, row[u].w);
          }
          if (k < seg_total && cv) {
            if (VEC4)  // streaming: a step does not read its rows again
              __builtin_nontemporal_store(floatx4{nr.x, nr.y, nr.z, nr.w}, reinterpret_cast<floatx4*>(ptr[u]));
            else *ptr[u] = nr.x;
          }
        }
      }
      __syncthreads();  // the next pass overwrites the list
    }

    // ---- readout: fixed-order sum of the 16 wave partials ----
    if (VEC4) *reinterpret_cast<float4*>(&red[wave * CB + lane * 4]) = acc;
    else red[wave * CB + lane] = acc.x;
    __syncthreads();
    for (int cc = tid; cc < CB; cc += DR_THREADS) {
      float sum = red[cc];
#pragma unroll
      for (int w = 1; w < DR_WAVES; ++w) sum += red[w * CB + cc];
      if (cb + cc < p.D) a_s[cb + cc] = sum;
    }
    __syncthreads();
  }
  if (p.G == 1 && idx_s)
    for (int k = done + tid; k < p.N; k += DR_THREADS) idx_s[k] = -1;
  if (p.cnt_out && tid == 0) p.cnt_out[s * p.G + g] = done;
}

// G > 1: a[s] = sum of the G range partials in range order; the range lists
// concatenated (ascending overall), padded with -1, and their total count.
__global__ __launch_bounds__(256) void decode_finalize_kernel(
    const float* __restrict__ a_part, const int32_t* __restrict__ idx_part,
    const int32_t* __restrict__ cnt_part, float* __restrict__ a_out, int32_t* __restrict__ idx_out,
    int32_t* __restrict__ cnt_out, int G, int rows, int N, int D) {
  const int64_t s = blockIdx.x;
  const int tid = threadIdx.x;
  for (int d = tid; d < D; d += 256) {
    float sum = a_part[s * G * D + d];
    for (int g = 1; g < G; ++g) sum += a_part[(s * G + g) * D + d];
    a_out[s * D + d] = sum;
  }
  if (!cnt_part) return;
  int off = 0;
  for (int g = 0; g < G; ++g) {
    const int c = cnt_part[s * G + g];
    if (idx_out)
      for (int k = tid; k < c; k += 256) idx_out[s * N + off + k] = idx_part[s * N + g * rows + k];
    off += c;
  }
  if (idx_out)
    for (int k = off + tid; k < N; k += 256) idx_out[s * N + k] = -1;
  if (cnt_out && tid == 0) cnt_out[s] = off;
}

}  // namespace

bdh_status run_decode(const DecodeArgs& a, hipStream_t st, uint64_t* launches) {
  const int64_t S = a.B * a.H;
  // Ranges per stream: double while the grid stays within one workgroup per
  // CU and a range keeps at least 256 rows.  (Measured: with a stream per CU
  // already, splitting further costs more in partials than it gains.)
  int G = 1;
  while (G < 16 && S * 2 * G <= (int64_t)device_cus() && a.N / (2 * G) >= 256) G *= 2;
  const int rows = (int)(((a.N + G - 1) / G + 7) / 8 * 8);
  DecodeKernelArgs p;
  p.x = a.x;
  p.v = a.v;
  p.rho = a.rho;
  p.freqs = a.freqs;
  p.a_out = a.a_out;
  p.idx_out = a.idx_out;
  p.cnt_out = a.cnt_out;
  p.H = (int)a.H;
  p.Hv = (int)a.Hv;
  p.N = (int)a.N;
  p.D = (int)a.D;
  p.G = G;
  p.rows = rows;
  p.pos = a.pos;
  if (G > 1) {
    void *ap = nullptr, *ip = nullptr, *cp = nullptr;
    bdh_status s = scratch(SLOT_DECODE_PART, (size_t)(S * G * a.D) * sizeof(float), &ap);
    if (s != BDH_OK) return s;
    p.a_out = (float*)ap;
    if (a.idx_out) {
      s = scratch(SLOT_DECODE_IDX, (size_t)(S * a.N) * sizeof(int32_t), &ip);
      if (s != BDH_OK) return s;
      p.idx_out = (int32_t*)ip;
    }
    if (a.idx_out || a.cnt_out) {
      s = scratch(SLOT_DECODE_CNT, (size_t)(S * G) * sizeof(int32_t), &cp);
      if (s != BDH_OK) return s;
      p.cnt_out = (int32_t*)cp;
    }
  }
  const dim3 grid((unsigned)(S * G));
  const bool vec4 = (a.D % 4) == 0;
  const int kt = ktime_begin(BDH_KERNEL_DECODE, st);
  if (a.freqs) {
    if (vec4) hipLaunchKernelGGL((decode_kernel<true, true>), grid, dim3(DR_THREADS), 0, st, p);
    else hipLaunchKernelGGL((decode_kernel<true, false>), grid, dim3(DR_THREADS), 0, st, p);
  } else {
    if (vec4) hipLaunchKernelGGL((decode_kernel<false, true>), grid, dim3(DR_THREADS), 0, st, p);
    else hipLaunchKernelGGL((decode_kernel<false, false>), grid, dim3(DR_THREADS), 0, st, p);
  }
  ktime_end(kt, st);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "decode_kernel launch");
  if (launches) *launches += 1;
  if (G > 1) {
    hipLaunchKernelGGL(decode_finalize_kernel, dim3((unsigned)S), dim3(256), 0, st, p.a_out,
                       p.idx_out, p.cnt_out, a.a_out, a.idx_out, a.cnt_out, G, rows, p.N, p.D);
    e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, "decode_finalize_kernel launch");
    if (launches) *launches += 1;
  }
  return BDH_OK;
}

}  // namespace bdh
