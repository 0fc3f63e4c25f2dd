// One-token (T = 1) steps of the recurrence on gfx950 (fp32), one launch per
// token (plus a finalize launch when streams are split into row ranges):
//   A = active rows of rot(x)   (x_i != 0, or x_{i^1} != 0 and frac(p f_i) != 0)
//   a = rot(x)[A] . rho[A, :]   (read before the update)
//   rho' = (rho + rot(x)^T v) * d
//
// Sparse step (rho updated in place, no decay): only the rows in A change,
// so only they are read and written.  G 1024-thread workgroups per (batch,
// head) stream each own a range of N / G rows (G grows while the grid stays
// within one workgroup per CU).  A workgroup compacts its range's active rows
// (8 rows per thread, wavefront prefix scan, workgroup offsets through LDS)
// into an LDS list (ascending), then its 16 waves stream exactly those rho
// rows: a whole 1 KiB row per wave per load at D = 256 (float4 per lane), 8
// rows in flight per wave.
//
// Dense step (rho' written to another buffer, a state of zeros, or a decay
// != 1): every row changes or must be copied, so every row is streamed once:
// read from rho_in (zeros when absent), written to rho_out.  256-thread
// workgroups each own 2048 rows of one stream; the rotated values of their
// rows go to LDS first.  This is the reference's private copy of rho
// (recurrent.rs:259) and its per-row update (recurrent.rs:415) in one pass.
//
// Readouts are reduced across waves in LDS in a fixed order; with G > 1 the
// range partials (and range lists) go to a range buffer and a finalize kernel
// sums them (and concatenates the lists) in range order, so results are
// deterministic and no atomics or cross-workgroup fences are needed.
#include "bdh_internal.h"

namespace bdh {
namespace {

constexpr int DR_THREADS = 1024;
constexpr int DR_WAVES = DR_THREADS / 64;
constexpr int DR_SEG = 8192;       // rows compacted per pass (LDS list capacity)
constexpr int DR_UNROLL = 8;
constexpr int ROWS_PER_THREAD = 8;  // 4 whole (even, odd) RoPE pairs
constexpr int DD_THREADS = 256;     // dense step
constexpr int DD_WAVES = DD_THREADS / 64;
constexpr int DD_ROWS = DD_THREADS * ROWS_PER_THREAD;
constexpr int DD_UNROLL = 8;

struct DecodeKernelArgs {
  const float* x;
  const float* v;
  const float* rho_in;  // dense step: source rows (null: zeros); sparse: == rho
  float* rho;
  const float* decay;   // dense step only; null: ones
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

// Rotated values r[e] of rows base + e (e < 8, rows < end) of one stream's x
// and the mask of the active ones.  blk: the 8 rows are one aligned 32-byte
// block of x and of the frequencies (two 16-byte loads each instead of 24
// scalar loads).  The phase frac(p f) is computed in the reference's f32 op
// order so that the active test agrees with it bit for bit.
template <bool ROPE>
__device__ __forceinline__ unsigned rows8(const float* xs, const float* freqs, float pos, int base,
                                          int end, bool blk, float (&r)[ROWS_PER_THREAD]) {
  float xv[ROWS_PER_THREAD], fv[ROWS_PER_THREAD];
  if (blk) {
    *reinterpret_cast<float4*>(&xv[0]) = *reinterpret_cast<const float4*>(xs + base);
    *reinterpret_cast<float4*>(&xv[4]) = *reinterpret_cast<const float4*>(xs + base + 4);
    if (ROPE) {
      *reinterpret_cast<float4*>(&fv[0]) = *reinterpret_cast<const float4*>(freqs + base);
      *reinterpret_cast<float4*>(&fv[4]) = *reinterpret_cast<const float4*>(freqs + base + 4);
    }
  }
  unsigned m = 0;
#pragma unroll
  for (int e = 0; e < ROWS_PER_THREAD; ++e) {
    const int i = base + e;
    r[e] = 0.0f;
    if (i < end) {
      const float xi = blk ? xv[e] : xs[i];
      bool on;
      if (ROPE) {
        const float xp = blk ? xv[e ^ 1] : xs[i ^ 1];
        const float fi = blk ? fv[e] : freqs[i];
        on = xi != 0.0f || (xp != 0.0f && rope_frac(pos, fi) != 0.0f);
        if (on) {
          float sn, cs, ev, od;
          sincosf(rope_phase(pos, fi), &sn, &cs);
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
  return m;
}

// Workgroup-wide exclusive prefix of cnt (thread order) and the total:
// wavefront scan, per-wave totals through LDS (wtot[NW]).  Holds one
// barrier; wtot may be rewritten after the caller's next barrier.
template <int NW>
__device__ __forceinline__ int block_prefix(int cnt, int lane, int wave, int32_t* wtot, int& total) {
  int incl = cnt;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int y = __shfl_up(incl, d, 64);
    if (lane >= d) incl += y;
  }
  if (lane == 63) wtot[wave] = incl;
  __syncthreads();
  int off = 0;
  total = 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const int t = wtot[w];
    off += w < wave ? t : 0;
    total += t;
  }
  return off + incl - cnt;
}

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
  const bool aligned =
      (p.N & 7) == 0 && ((reinterpret_cast<uintptr_t>(p.x) | reinterpret_cast<uintptr_t>(p.freqs)) & 15) == 0;

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
      const int base = seg0 + tid * ROWS_PER_THREAD;
      float r[ROWS_PER_THREAD];
      const unsigned m = rows8<ROPE>(xs, p.freqs, p.pos, base, seg_end, aligned && base < seg_end, r);
      int seg_total = 0;
      int pos = block_prefix<DR_WAVES>(__popc(m), lane, wave, wtot, seg_total);
#pragma unroll
      for (int e = 0; e < ROWS_PER_THREAD; ++e)
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

// Dense step over rows [g * rows, g * rows + rows) of stream s (rows =
// DD_ROWS): every row is read from rho_in (SRC) or taken as zeros, and
// written to rho.  Rows outside A keep their value (times the decay) bit for
// bit: no add is made for them.
template <bool ROPE, bool VEC4, bool DECAY, bool SRC>
__global__ __launch_bounds__(DD_THREADS) void decode_dense_kernel(DecodeKernelArgs p) {
  constexpr int CB = ColBlock<VEC4>::W;
  __shared__ float lval[DD_ROWS];
  __shared__ __attribute__((aligned(16))) float red[DD_WAVES * CB];
  __shared__ int32_t wtot[DD_WAVES];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t s = blockIdx.x / p.G;
  const int g = (int)(blockIdx.x - s * p.G);
  const int r0 = g * p.rows, r1 = min(p.N, r0 + p.rows);
  const int64_t b = s / p.H, h = s - b * p.H;
  const float* xs = p.x + s * p.N;
  const float* vs = p.v + (b * p.Hv + (p.Hv == 1 ? 0 : h)) * p.D;
  const float* src_s = SRC ? p.rho_in + s * (int64_t)p.N * p.D : nullptr;
  float* dst_s = p.rho + s * (int64_t)p.N * p.D;
  float* a_s = p.a_out + (s * p.G + g) * p.D;
  const float dk = DECAY ? p.decay[h] : 1.0f;
  const bool aligned =
      (p.N & 7) == 0 && ((reinterpret_cast<uintptr_t>(p.x) | reinterpret_cast<uintptr_t>(p.freqs)) & 15) == 0;

  // ---- rotated values of the range's rows (0 for inactive rows) ----
  const int base = r0 + tid * ROWS_PER_THREAD;
  float r[ROWS_PER_THREAD];
  const unsigned m = rows8<ROPE>(xs, p.freqs, p.pos, base, r1, aligned && base < r1, r);
#pragma unroll
  for (int e = 0; e < ROWS_PER_THREAD; ++e) lval[tid * ROWS_PER_THREAD + e] = r[e];
  if (p.idx_out || p.cnt_out) {
    // Range list (ascending) and count, as the sparse step writes them.
    int total = 0;
    int pos = block_prefix<DD_WAVES>(__popc(m), lane, wave, wtot, total);
    int32_t* idx_s = p.idx_out ? p.idx_out + s * p.N + (p.G > 1 ? r0 : 0) : nullptr;
    if (idx_s) {
#pragma unroll
      for (int e = 0; e < ROWS_PER_THREAD; ++e)
        if ((m >> e) & 1u) idx_s[pos++] = base + e;
      if (p.G == 1)
        for (int k = total + tid; k < p.N; k += DD_THREADS) idx_s[k] = -1;
    }
    if (p.cnt_out && tid == 0) p.cnt_out[s * p.G + g] = total;
  }
  __syncthreads();

  const int n = r1 - r0;
  for (int cb = 0; cb < p.D; cb += CB) {
    const int c = VEC4 ? cb + lane * 4 : cb + lane;
    const bool cv = c < p.D;
    float4 vv = make_float4(0, 0, 0, 0), acc = make_float4(0, 0, 0, 0);
    if (cv) {
      if (VEC4) vv = *reinterpret_cast<const float4*>(vs + c);
      else vv.x = vs[c];
    }
    for (int k0 = wave; k0 < n; k0 += DD_WAVES * DD_UNROLL) {
      float4 row[DD_UNROLL];
#pragma unroll
      for (int u = 0; u < DD_UNROLL; ++u) {
        const int k = k0 + u * DD_WAVES;
        const bool ok = SRC && k < n && cv;
        const float* sp = src_s + (int64_t)(r0 + k) * p.D + c;
        if (VEC4) row[u] = ok ? *reinterpret_cast<const float4*>(sp) : make_float4(0, 0, 0, 0);
        else row[u] = make_float4(ok ? *sp : 0.0f, 0, 0, 0);
      }
#pragma unroll
      for (int u = 0; u < DD_UNROLL; ++u) {
        const int k = k0 + u * DD_WAVES;
        if (k >= n || !cv) continue;
        const float rv = lval[k];
        float4 nr = row[u];
        if (rv != 0.0f) {
          acc.x = fmaf(row[u].x, rv, acc.x);
          nr.x = fmaf(rv, vv.x, row[u].x);
          if (VEC4) {
            acc.y = fmaf(row[u].y, rv, acc.y);
            acc.z = fmaf(row[u].z, rv, acc.z);
            acc.w = fmaf(row[u].w, rv, acc.w);
            nr.y = fmaf(rv, vv.y, row[u].y);
            nr.z = fmaf(rv, vv.z, row[u].z);
            nr.w = fmaf(rv, vv.w, row[u].w);
          }
        }
        if (DECAY) {
          nr.x *= dk;
          nr.y *= dk;
          nr.z *= dk;
          nr.w *= dk;
        }
        float* dp = dst_s + (int64_t)(r0 + k) * p.D + c;
        if (VEC4) __builtin_nontemporal_store(floatx4{nr.x, nr.y, nr.z, nr.w}, reinterpret_cast<floatx4*>(dp));
        else *dp = nr.x;
      }
    }
    if (VEC4) *reinterpret_cast<float4*>(&red[wave * CB + lane * 4]) = acc;
    else red[wave * CB + lane] = acc.x;
    __syncthreads();
    for (int cc = tid; cc < CB; cc += DD_THREADS) {
      float sum = red[cc];
#pragma unroll
      for (int w = 1; w < DD_WAVES; ++w) sum += red[w * CB + cc];
      if (cb + cc < p.D) a_s[cb + cc] = sum;
    }
    __syncthreads();
  }
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

bool sparse_step(const DecodeArgs& a) { return a.decay == nullptr && a.rho_in != nullptr && a.rho_in == a.rho; }

// Ranges per stream and rows per range.
void decode_ranges(const DecodeArgs& a, int* G, int* rows) {
  if (sparse_step(a)) {
    // Double while the grid stays within one workgroup per CU and a range
    // keeps at least 256 rows.  (Measured: with a stream per CU already,
    // splitting further costs more in partials than it gains.)
    int g = 1;
    const int64_t S = a.B * a.H;
    while (g < 16 && S * 2 * g <= (int64_t)device_cus() && a.N / (2 * g) >= 256) g *= 2;
    *G = g;
    *rows = (int)(((a.N + g - 1) / g + 7) / 8 * 8);
  } else {
    *G = (int)((a.N + DD_ROWS - 1) / DD_ROWS);
    *rows = DD_ROWS;
  }
}

// Range buffer layout: partial readouts [S, G, D] f32, then (lists asked
// for) range lists [S, N] int32 and range counts [S, G] int32, each
// 256-byte aligned.
size_t align256(size_t n) { return (n + 255) / 256 * 256; }

}  // namespace

size_t decode_part_bytes(const DecodeArgs& a) {
  int G = 1, rows = 0;
  decode_ranges(a, &G, &rows);
  if (G == 1) return 0;
  const int64_t S = a.B * a.H;
  size_t n = align256((size_t)(S * G * a.D) * sizeof(float));
  if (a.idx_out) n += align256((size_t)(S * a.N) * sizeof(int32_t));
  if (a.idx_out || a.cnt_out) n += align256((size_t)(S * G) * sizeof(int32_t));
  return n;
}

bdh_status run_decode(const DecodeArgs& a, hipStream_t st, uint64_t* launches) {
  const int64_t S = a.B * a.H;
  int G = 1, rows = 0;
  decode_ranges(a, &G, &rows);
  const bool sparse = sparse_step(a);
  DecodeKernelArgs p;
  p.x = a.x;
  p.v = a.v;
  p.rho_in = a.rho_in;
  p.rho = a.rho;
  p.decay = a.decay;
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
    const size_t need = decode_part_bytes(a);
    char* buf = (char*)a.part_buf;
    if (buf) {
      if (a.part_bytes < need) return fail(BDH_EINVAL, "decode range buffer too small");
    } else {
      void* sp = nullptr;
      bdh_status s = scratch(st, SLOT_DECODE_PART, need, &sp);
      if (s != BDH_OK) return s;
      buf = (char*)sp;
    }
    p.a_out = (float*)buf;
    buf += align256((size_t)(S * G * a.D) * sizeof(float));
    if (a.idx_out) {
      p.idx_out = (int32_t*)buf;
      buf += align256((size_t)(S * a.N) * sizeof(int32_t));
    }
    if (a.idx_out || a.cnt_out) p.cnt_out = (int32_t*)buf;
  }
  // Float4 columns need D % 4 == 0 and 16-byte aligned rows.
  const bool vec4 = (a.D % 4) == 0 &&
                    ((reinterpret_cast<uintptr_t>(a.v) | reinterpret_cast<uintptr_t>(a.rho) |
                      reinterpret_cast<uintptr_t>(a.rho_in) | reinterpret_cast<uintptr_t>(p.a_out)) & 15) == 0;
  const bool rope = a.freqs != nullptr;
  const int kt = ktime_begin(BDH_KERNEL_DECODE, st);
  if (sparse) {
    const dim3 grid((unsigned)(S * G)), blk(DR_THREADS);
    if (rope) {
      if (vec4) hipLaunchKernelGGL((decode_kernel<true, true>), grid, blk, 0, st, p);
      else hipLaunchKernelGGL((decode_kernel<true, false>), grid, blk, 0, st, p);
    } else {
      if (vec4) hipLaunchKernelGGL((decode_kernel<false, true>), grid, blk, 0, st, p);
      else hipLaunchKernelGGL((decode_kernel<false, false>), grid, blk, 0, st, p);
    }
  } else {
    const dim3 grid((unsigned)(S * G)), blk(DD_THREADS);
    const int key = (rope ? 8 : 0) | (vec4 ? 4 : 0) | (a.decay ? 2 : 0) | (a.rho_in ? 1 : 0);
#define BDH_DENSE(K, R, V, DC, SR) \
  case K: hipLaunchKernelGGL((decode_dense_kernel<R, V, DC, SR>), grid, blk, 0, st, p); break;
    switch (key) {
      BDH_DENSE(0, false, false, false, false)
      BDH_DENSE(1, false, false, false, true)
      BDH_DENSE(2, false, false, true, false)
      BDH_DENSE(3, false, false, true, true)
      BDH_DENSE(4, false, true, false, false)
      BDH_DENSE(5, false, true, false, true)
      BDH_DENSE(6, false, true, true, false)
      BDH_DENSE(7, false, true, true, true)
      BDH_DENSE(8, true, false, false, false)
      BDH_DENSE(9, true, false, false, true)
      BDH_DENSE(10, true, false, true, false)
      BDH_DENSE(11, true, false, true, true)
      BDH_DENSE(12, true, true, false, false)
      BDH_DENSE(13, true, true, false, true)
      BDH_DENSE(14, true, true, true, false)
      BDH_DENSE(15, true, true, true, true)
    }
#undef BDH_DENSE
  }
  ktime_end(kt, st);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "decode step launch");
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
