// Sparse decode step on gfx950 (fp32).  One launch per token:
//   A = active rows of rot(x)   (x_i != 0, or x_{i^1} != 0 and frac(p f_i) != 0)
//   a = rot(x)[A] . rho[A, :]   (read before the update)
//   rho[A, :] += rot(x)[A]^T v
// Grid (splits, streams).  Workgroup j of a stream owns rows
// [j*R, (j+1)*R): it compacts its active rows with a wavefront ballot and a
// workgroup prefix scan into LDS, then streams exactly those rho rows
// (coalesced float4 per lane, a whole 1 KiB row per wave at D = 256).  The
// per-workgroup partial readouts are summed in a fixed order by the last
// workgroup of the stream to arrive (deterministic), which also stitches
// the per-segment active lists.  Inactive rows are never read or written.
#include "bdh_internal.h"

namespace bdh {
namespace {

constexpr int DEC_THREADS = 256;
constexpr int DEC_WAVES = DEC_THREADS / 64;
constexpr int DEC_UNROLL = 4;

struct DecodeKernelArgs {
  const float* x;
  const float* v;
  float* rho;
  const float* freqs;
  float* a_out;
  int32_t* idx_out;
  int32_t* cnt_out;
  float* partial;     // [S, splits, D]
  int32_t* seg_cnt;   // [S, splits]
  int32_t* seg_idx;   // [S, N]
  uint32_t* counters; // [S]
  int H, Hv, N, D, rows_per, splits;
  float pos;
};

template <bool ROPE, bool VEC4>
__global__ __launch_bounds__(DEC_THREADS) void decode_kernel(DecodeKernelArgs p) {
  extern __shared__ float smem[];
  // layout: lval[rows_per] f32 | lidx[rows_per] i32 | red[DEC_WAVES * D] f32
  float* lval = smem;
  int32_t* lidx = reinterpret_cast<int32_t*>(smem + p.rows_per);
  float* red = smem + 2 * p.rows_per;
  __shared__ int32_t wave_cnt[DEC_WAVES];
  __shared__ int32_t total_cnt;
  __shared__ int32_t is_last;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int j = blockIdx.x;
  const int64_t s = blockIdx.y;
  const int r0 = j * p.rows_per;
  const int r1 = min(p.N, r0 + p.rows_per);
  const float* xs = p.x + s * p.N;

  // ---- 1. compaction of this segment's active rows (ascending order) ----
  if (tid == 0) total_cnt = 0;
  __syncthreads();
  for (int base = r0; base < r1; base += DEC_THREADS) {
    const int i = base + tid;
    bool on = false;
    float r = 0.0f;
    if (i < r1) {
      const float xi = xs[i];
      if (ROPE) {
        const float xp = xs[i ^ 1];
        on = xi != 0.0f || (xp != 0.0f && rope_frac(p.pos, p.freqs[i]) != 0.0f);
        if (on) {
          float sn, cs;
          sincosf(rope_phase(p.pos, p.freqs[i]), &sn, &cs);
          float e, o;
          if ((i & 1) == 0) rope_pair_exact(xi, xp, cs, sn, e, o), r = e;
          else rope_pair_exact(xp, xi, cs, sn, e, o), r = o;
        }
      } else {
        on = xi != 0.0f;
        r = xi;
      }
    }
    const uint64_t mask = __ballot(on);
    const int before = __popcll(mask & ((1ull << lane) - 1ull));
    if (lane == 0) wave_cnt[wave] = __popcll(mask);
    __syncthreads();
    int off = total_cnt;
    for (int w = 0; w < wave; ++w) off += wave_cnt[w];
    if (on) {
      lidx[off + before] = i;
      lval[off + before] = r;
    }
    __syncthreads();
    if (tid == 0) {
      int t = total_cnt;
      for (int w = 0; w < DEC_WAVES; ++w) t += wave_cnt[w];
      total_cnt = t;
    }
    __syncthreads();
  }
  const int cnt = total_cnt;

  // ---- 2. stream the active rows: a += r * rho_row ; rho_row += r * v ----
  const int64_t b = s / p.H, h = s - b * p.H;
  const float* vs = p.v + (b * p.Hv + (p.Hv == 1 ? 0 : h)) * p.D;
  float* rho_s = p.rho + s * (int64_t)p.N * p.D;
  for (int cb = 0; cb < p.D; cb += (VEC4 ? 256 : 64)) {
    if (VEC4) {
      const int c = cb + lane * 4;
      const bool cv = c < p.D;
      float4 vv = cv ? *reinterpret_cast<const float4*>(vs + c) : make_float4(0, 0, 0, 0);
      float4 acc = make_float4(0, 0, 0, 0);
      int k = wave;
      for (; k + (DEC_UNROLL - 1) * DEC_WAVES < cnt; k += DEC_UNROLL * DEC_WAVES) {
        float4 row[DEC_UNROLL];
        float rv[DEC_UNROLL];
        float* ptr[DEC_UNROLL];
#pragma unroll
        for (int u = 0; u < DEC_UNROLL; ++u) {
          const int kk = k + u * DEC_WAVES;
          rv[u] = lval[kk];
          ptr[u] = rho_s + (int64_t)lidx[kk] * p.D + c;
          row[u] = cv ? *reinterpret_cast<const float4*>(ptr[u]) : make_float4(0, 0, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < DEC_UNROLL; ++u) {
          acc.x = fmaf(row[u].x, rv[u], acc.x);
          acc.y = fmaf(row[u].y, rv[u], acc.y);
          acc.z = fmaf(row[u].z, rv[u], acc.z);
          acc.w = fmaf(row[u].w, rv[u], acc.w);
          float4 nr;
          nr.x = fmaf(rv[u], vv.x, row[u].x);
          nr.y = fmaf(rv[u], vv.y, row[u].y);
          nr.z = fmaf(rv[u], vv.z, row[u].z);
          nr.w = fmaf(rv[u], vv.w, row[u].w);
          if (cv) *reinterpret_cast<float4*>(ptr[u]) = nr;
        }
      }
      for (; k < cnt; k += DEC_WAVES) {
        const float rv = lval[k];
        float* ptr = rho_s + (int64_t)lidx[k] * p.D + c;
        if (cv) {
          float4 row = *reinterpret_cast<const float4*>(ptr);
          acc.x = fmaf(row.x, rv, acc.x);
          acc.y = fmaf(row.y, rv, acc.y);
          acc.z = fmaf(row.z, rv, acc.z);
          acc.w = fmaf(row.w, rv, acc.w);
          row.x = fmaf(rv, vv.x, row.x);
          row.y = fmaf(rv, vv.y, row.y);
          row.z = fmaf(rv, vv.z, row.z);
          row.w = fmaf(rv, vv.w, row.w);
          *reinterpret_cast<float4*>(ptr) = row;
        }
      }
      if (cv) *reinterpret_cast<float4*>(red + wave * p.D + c) = acc;
    } else {
      const int c = cb + lane;
      const bool cv = c < p.D;
      const float vv = cv ? vs[c] : 0.0f;
      float acc = 0.0f;
      for (int k = wave; k < cnt; k += DEC_WAVES) {
        const float rv = lval[k];
        if (cv) {
          float* ptr = rho_s + (int64_t)lidx[k] * p.D + c;
          const float row = *ptr;
          acc = fmaf(row, rv, acc);
          *ptr = fmaf(rv, vv, row);
        }
      }
      if (cv) red[wave * p.D + c] = acc;
    }
  }
  __syncthreads();

  // ---- 3. workgroup partial of a, fixed wave order ----
  float* dst = p.splits == 1 ? p.a_out + s * p.D : p.partial + (s * p.splits + j) * p.D;
  for (int c = tid; c < p.D; c += DEC_THREADS) {
    float sum = red[c];
    for (int w = 1; w < DEC_WAVES; ++w) sum += red[w * p.D + c];
    dst[c] = sum;
  }
  if (p.splits == 1) {
    if (p.idx_out)
      for (int k = tid; k < p.N; k += DEC_THREADS) p.idx_out[s * p.N + k] = k < cnt ? lidx[k] : -1;
    if (p.cnt_out && tid == 0) p.cnt_out[s] = cnt;
    return;
  }
  if (p.idx_out)
    for (int k = tid; k < cnt; k += DEC_THREADS) p.seg_idx[s * p.N + r0 + k] = lidx[k];
  if (tid == 0) p.seg_cnt[s * p.splits + j] = cnt;

  // ---- 4. the last workgroup of the stream reduces the partials ----
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const uint32_t old = atomicAdd(p.counters + s, 1u);
    is_last = (old == (uint32_t)(p.splits - 1)) ? 1 : 0;
  }
  __syncthreads();
  if (!is_last) return;
  __threadfence();
  const float* part = p.partial + s * p.splits * p.D;
  for (int c = tid; c < p.D; c += DEC_THREADS) {
    float sum = part[c];
    for (int jj = 1; jj < p.splits; ++jj) sum += part[jj * p.D + c];
    p.a_out[s * p.D + c] = sum;
  }
  if (p.idx_out || p.cnt_out) {
    int total = 0;
    for (int jj = 0; jj < p.splits; ++jj) {
      const int sc = p.seg_cnt[s * p.splits + jj];
      if (p.idx_out)
        for (int k = tid; k < sc; k += DEC_THREADS)
          p.idx_out[s * p.N + total + k] = p.seg_idx[s * p.N + jj * p.rows_per + k];
      total += sc;
    }
    if (p.idx_out)
      for (int k = total + tid; k < p.N; k += DEC_THREADS) p.idx_out[s * p.N + k] = -1;
    if (p.cnt_out && tid == 0) p.cnt_out[s] = total;
  }
  if (tid == 0) p.counters[s] = 0u;  // ready for the next launch on this stream
}

}  // namespace

bdh_status run_decode(const DecodeArgs& a, hipStream_t st, uint64_t* launches) {
  const int64_t S = a.B * a.H;
  // Segments of 1024 rows: ~100 active rows per workgroup at 9.75 % density,
  // 8 workgroups per stream at N = 8192.
  const int rows_per = (int)(a.N < 1024 ? ((a.N + 63) / 64) * 64 : 1024);
  const int splits = (int)((a.N + rows_per - 1) / rows_per);
  void* ws = nullptr;
  const size_t part_bytes = (size_t)S * splits * a.D * sizeof(float);
  const size_t segc_bytes = (size_t)S * splits * sizeof(int32_t);
  const size_t segi_bytes = (size_t)S * a.N * sizeof(int32_t);
  bdh_status stt = BDH_OK;
  if (splits > 1) {
    stt = scratch(SLOT_DECODE, part_bytes + segc_bytes + segi_bytes, &ws);
    if (stt != BDH_OK) return stt;
  }
  void* ctr = nullptr;
  if (splits > 1) {
    stt = scratch(SLOT_COUNTERS, (size_t)S * sizeof(uint32_t), &ctr, /*zero_on_alloc=*/true);
    if (stt != BDH_OK) return stt;
  }
  DecodeKernelArgs p;
  p.x = a.x;
  p.v = a.v;
  p.rho = a.rho;
  p.freqs = a.freqs;
  p.a_out = a.a_out;
  p.idx_out = a.idx_out;
  p.cnt_out = a.cnt_out;
  char* w = (char*)ws;
  p.partial = (float*)w;
  p.seg_cnt = (int32_t*)(w ? w + part_bytes : nullptr);
  p.seg_idx = (int32_t*)(w ? w + part_bytes + segc_bytes : nullptr);
  p.counters = (uint32_t*)ctr;
  p.H = (int)a.H;
  p.Hv = (int)a.Hv;
  p.N = (int)a.N;
  p.D = (int)a.D;
  p.rows_per = rows_per;
  p.splits = splits;
  p.pos = a.pos;
  const size_t lds = (size_t)(2 * rows_per + DEC_WAVES * a.D) * sizeof(float);
  const dim3 grid((unsigned)splits, (unsigned)S);
  const bool vec4 = (a.D % 4) == 0;
  if (a.freqs) {
    if (vec4) hipLaunchKernelGGL((decode_kernel<true, true>), grid, dim3(DEC_THREADS), lds, st, p);
    else hipLaunchKernelGGL((decode_kernel<true, false>), grid, dim3(DEC_THREADS), lds, st, p);
  } else {
    if (vec4) hipLaunchKernelGGL((decode_kernel<false, true>), grid, dim3(DEC_THREADS), lds, st, p);
    else hipLaunchKernelGGL((decode_kernel<false, false>), grid, dim3(DEC_THREADS), lds, st, p);
  }
  if (launches) *launches += 1;
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "decode_kernel launch");
  return BDH_OK;
}

}  // namespace bdh
