// bf16 MFMA tile machinery shared by the prefill units (mfma_prefill.hip)
// and the layer GEMMs (layer_bf16.hip): 256-thread workgroups whose 4 waves
// each own a 64x128 block of v_mfma_f32_16x16x32_bf16 accumulators, operands
// staged through LDS in 32-deep k steps (double-buffered), and an epilogue
// that writes the accumulators back as rows through LDS.
#pragma once

#include <type_traits>
#include <utility>

#include "bdh_bf16.h"

namespace bdh {
namespace mfma {

constexpr int NT = 256;               // 4 waves
constexpr int BK = 32;                // k step: 64-byte LDS rows of four 16-byte chunks
constexpr int ROWS = T256 + T256 / 2; // operand rows per step (256 + 128)
constexpr int BUF = ROWS * BK;        // bf16 elements of one step's operands

// Element offset of 16-byte chunk c (0..3) of LDS row r.  Chunks are XOR
// swizzled with bits 1..2 of the row: measured on gfx950 (LDS bank-conflict
// counter), this makes both the MFMA fragment reads (16 rows x 4 chunks per
// wave) and the row-segment writes (4 lanes per row) conflict-free, where a
// padded 80-byte pitch has 2x conflicts on each.
__device__ __forceinline__ int lds_off(int r, int c) { return r * BK + ((c ^ ((r >> 1) & 3)) << 3); }

__device__ __forceinline__ bf16x8 frag(const bf16_t* base, int row, int lane) {
  return *reinterpret_cast<const bf16x8*>(&base[lds_off(row + (lane & 15), lane >> 4)]);
}

// acc[mi][ni] += A[arow + 16 mi] x B[brow + 16 ni]^T over one 32-deep step
// (rows of both operands k-contiguous): 4 x 8 MFMAs.  All 12 fragments are
// requested up front, in the order the MFMAs consume them, so the first
// MFMAs wait only for the first reads and one LDS round trip covers the step.
__device__ __forceinline__ void mma_64x128(const bf16_t* A, const bf16_t* B, int lane, int arow,
                                           int brow, floatx4 (&acc)[4][8]) {
  bf16x8 af[4], bfr[8];
  af[0] = frag(A, arow, lane);
#pragma unroll
  for (int ni = 0; ni < 4; ++ni) bfr[ni] = frag(B, brow + ni * 16, lane);
#pragma unroll
  for (int mi = 1; mi < 4; ++mi) af[mi] = frag(A, arow + mi * 16, lane);
#pragma unroll
  for (int ni = 4; ni < 8; ++ni) bfr[ni] = frag(B, brow + ni * 16, lane);
#pragma unroll
  for (int nh = 0; nh < 2; ++nh)
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
      for (int ni = 0; ni < 4; ++ni)
        acc[mi][nh * 4 + ni] = mfma16(af[mi], bfr[nh * 4 + ni], acc[mi][nh * 4 + ni]);
}

__device__ __forceinline__ void zero_acc(floatx4 (&acc)[4][8]) {
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
#pragma unroll
    for (int ni = 0; ni < 8; ++ni) acc[mi][ni] = zero4();
}

// Epilogue of a wave's 64 x 128 fp32 accumulator block, through LDS (free
// once the step loop's last barrier has passed): per 16-row slice mi the
// wave writes its block to its own region (row pitch 132 floats, so the four
// 4-row groups of one store land in distinct banks) and reads it back as
// rows, two per instruction, 16 bytes per lane; emit(row, col, v) receives
// row 0..63 and column 0..124 (a multiple of 4) of the block.  Every wave
// of the workgroup must call it (it holds barriers).
template <class Emit>
__device__ __forceinline__ void epilogue_64x128(const floatx4 (&acc)[4][8], bf16_t* lds, int w,
                                                int lane, Emit&& emit) {
  constexpr int EP = 132;
  float* E = reinterpret_cast<float*>(lds) + w * 16 * EP;
#pragma unroll
  for (int mi = 0; mi < 4; ++mi) {
#pragma unroll
    for (int ni = 0; ni < 8; ++ni)
#pragma unroll
      for (int r = 0; r < 4; ++r) E[acc16_row(lane, r) * EP + ni * 16 + acc16_col(lane)] = acc[mi][ni][r];
    __syncthreads();
#pragma unroll
    for (int rr = 0; rr < 16; rr += 2) {
      // A lane's columns are the same in every call (GEMM X relies on it).
      const int row = rr + (lane >> 5), col = 4 * (lane & 31);
      emit(mi * 16 + row, col, *reinterpret_cast<const float4*>(&E[row * EP + col]));
    }
    __syncthreads();
  }
}

// As epilogue_64x128 with 8 columns per call: emit(row, col, lo, hi) gets
// columns col .. col + 3 (lo) and col + 4 .. col + 7 (hi) of one row, with
// col = 8 (lane & 15) the same in every call and 4 rows per wave call, so a
// caller writing bf16 issues one 16-byte store per lane and call.
template <class Emit>
__device__ __forceinline__ void epilogue8_64x128(const floatx4 (&acc)[4][8], bf16_t* lds, int w,
                                                 int lane, Emit&& emit) {
  constexpr int EP = 132;
  float* E = reinterpret_cast<float*>(lds) + w * 16 * EP;
#pragma unroll
  for (int mi = 0; mi < 4; ++mi) {
#pragma unroll
    for (int ni = 0; ni < 8; ++ni)
#pragma unroll
      for (int r = 0; r < 4; ++r) E[acc16_row(lane, r) * EP + ni * 16 + acc16_col(lane)] = acc[mi][ni][r];
    __syncthreads();
#pragma unroll
    for (int rr = 0; rr < 16; rr += 4) {
      const int row = rr + (lane >> 4), col = 8 * (lane & 15);
      emit(mi * 16 + row, col, *reinterpret_cast<const float4*>(&E[row * EP + col]),
           *reinterpret_cast<const float4*>(&E[row * EP + col + 4]));
    }
    __syncthreads();
  }
}

// Steps [kb, ke), an even count: LDS buffer (kt - kb) & 1 holds step kt; the
// loads of step kt+1 are issued before step kt's MFMAs and written to the
// other buffer after them.
template <class Load, class Store, class Compute>
__device__ __forceinline__ void run_steps(int kb, int ke, Load&& load, Store&& store,
                                          Compute&& compute) {
  load(kb);
  store(0);
  __syncthreads();
  for (int kt = kb; kt < ke; kt += 2) {
    load(kt + 1);
    compute(0);
    store(1);
    __syncthreads();
    if (kt + 2 < ke) load(kt + 2);
    compute(1);
    if (kt + 2 < ke) store(0);
    __syncthreads();
  }
}

// --- direct global -> LDS loads (gfx950 global_load_lds_dwordx4) -----------
// Byte address of an LDS location (the value M0 takes for an LDS DMA).
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)p;
}
// Each lane fetches 16 bytes from gbase + voff and the hardware writes them
// to LDS at m0 + 16 * lane: one instruction fills 1 KiB (16 rows of 64
// bytes).  Written in assembly so that the compiler, which does not know
// which LDS bytes a DMA writes, does not wait for every DMA in flight before
// each LDS read; the pipeline's own waits (dma_wait_barrier) order them.
// gbase is wave-uniform at every call; it is read from the first lane so
// that it is an SGPR pair even where the compiler kept it in VGPRs.  The
// builtin returns a signed int: each half goes through uint32_t, or the low
// half would be sign-extended into the high one.  The compiler does not see
// the load inside the assembly, so the block waits 5 states itself (an SGPR
// written by a VALU instruction, such as v_readfirstlane, needs 5 before a
// vector memory instruction reads it; M0 needs 1 before an LDS DMA).
__device__ __forceinline__ void dma16(const void* gbase, uint32_t voff, uint32_t m0) {
  const uint64_t b = reinterpret_cast<uint64_t>(gbase);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(b >> 32));
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)b);
  const uint64_t bu = ((uint64_t)hi << 32) | (uint64_t)lo;
  asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(reinterpret_cast<const void*>(bu)),
               "{m0}"(m0)
               : "memory");
}
// As dma16 with the non-temporal hint: for data read once, so that it does
// not evict the L2 lines of operands that are read again.
__device__ __forceinline__ void dma16_nt(const void* gbase, uint32_t voff, uint32_t m0) {
  const uint64_t b = reinterpret_cast<uint64_t>(gbase);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(b >> 32));
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)b);
  const uint64_t bu = ((uint64_t)hi << 32) | (uint64_t)lo;
  asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %0, %1 nt" ::"v"(voff), "s"(reinterpret_cast<const void*>(bu)),
               "{m0}"(m0)
               : "memory");
}
// As dma16 with 4 bytes per lane, written to LDS at m0 + 4 * lane.
__device__ __forceinline__ void dma4(const void* gbase, uint32_t voff, uint32_t m0) {
  const uint64_t b = reinterpret_cast<uint64_t>(gbase);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(b >> 32));
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)b);
  const uint64_t bu = ((uint64_t)hi << 32) | (uint64_t)lo;
  asm volatile("s_nop 4\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(reinterpret_cast<const void*>(bu)),
               "{m0}"(m0)
               : "memory");
}
// Wait until at most N of this wave's vector memory operations are in
// flight (the oldest complete first), then a workgroup barrier: every wave's
// DMAs issued before its last N have landed in LDS, and every wave has
// finished the LDS reads it issued before the barrier.
template <int N>
__device__ __forceinline__ void dma_wait_barrier() {
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(N) : "memory");
}


// acc += A x B^T over one 32-deep step, as mma_64x128, with the fragment LDS
// reads in assembly: used where the LDS holds direct-load stages, so that
// the compiler (which cannot tell them apart from the DMAs in flight) does
// not make them wait for those.  The reads are issued in the order the
// MFMAs consume them (a0 b0..b3, a1..a3, b4..b7) and waited for with
// lgkmcnt counts (LDS reads complete in order) tied to the fragment
// registers, so no MFMA can be scheduled before its wait.
__device__ __forceinline__ void mma_64x128_dsasm(const bf16_t* A, const bf16_t* B, int lane, int arow,
                                                 int brow, floatx4 (&acc)[4][8]) {
  typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
  const uint32_t a = lds_addr(A) + (uint32_t)(2 * lds_off(arow + (lane & 15), lane >> 4));
  const uint32_t b = lds_addr(B) + (uint32_t)(2 * lds_off(brow + (lane & 15), lane >> 4));
  u32x4_t af[4], bf[8];
#define BDH_DSR(dst, addr, off) asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(dst) : "v"(addr), "n"(off))
  BDH_DSR(af[0], a, 0);
  BDH_DSR(bf[0], b, 0);
  BDH_DSR(bf[1], b, 1024);
  BDH_DSR(bf[2], b, 2048);
  BDH_DSR(bf[3], b, 3072);
  BDH_DSR(af[1], a, 1024);
  BDH_DSR(af[2], a, 2048);
  BDH_DSR(af[3], a, 3072);
  BDH_DSR(bf[4], b, 4096);
  BDH_DSR(bf[5], b, 5120);
  BDH_DSR(bf[6], b, 6144);
  BDH_DSR(bf[7], b, 7168);
#undef BDH_DSR
  auto mm = [&](int mi, int ni) {
    acc[mi][ni] = mfma16(__builtin_bit_cast(bf16x8, af[mi]), __builtin_bit_cast(bf16x8, bf[ni]), acc[mi][ni]);
  };
  asm volatile("s_waitcnt lgkmcnt(7)" : "+v"(af[0]), "+v"(bf[0]), "+v"(bf[1]), "+v"(bf[2]), "+v"(bf[3]));
#pragma unroll
  for (int ni = 0; ni < 4; ++ni) mm(0, ni);
  asm volatile("s_waitcnt lgkmcnt(4)" : "+v"(af[1]), "+v"(af[2]), "+v"(af[3]));
#pragma unroll
  for (int mi = 1; mi < 4; ++mi)
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) mm(mi, ni);
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(bf[4]), "+v"(bf[5]), "+v"(bf[6]), "+v"(bf[7]));
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
#pragma unroll
    for (int ni = 4; ni < 8; ++ni) mm(mi, ni);
}

// The same for a 64 x 64 block: 4 A and 4 B fragments, 16 MFMAs;
// acc[mi][ni] += A[arow + 16 mi] x B[brow + 16 ni]^T.
__device__ __forceinline__ void mma_64x64_dsasm(const bf16_t* A, const bf16_t* B, int lane, int arow,
                                                int brow, floatx4 (&acc)[4][4]) {
  typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
  const uint32_t a = lds_addr(A) + (uint32_t)(2 * lds_off(arow + (lane & 15), lane >> 4));
  const uint32_t b = lds_addr(B) + (uint32_t)(2 * lds_off(brow + (lane & 15), lane >> 4));
  u32x4_t af[4], bf[4];
#define BDH_DSR(dst, addr, off) asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(dst) : "v"(addr), "n"(off))
  BDH_DSR(af[0], a, 0);
  BDH_DSR(bf[0], b, 0);
  BDH_DSR(bf[1], b, 1024);
  BDH_DSR(bf[2], b, 2048);
  BDH_DSR(bf[3], b, 3072);
  BDH_DSR(af[1], a, 1024);
  BDH_DSR(af[2], a, 2048);
  BDH_DSR(af[3], a, 3072);
#undef BDH_DSR
  auto mm = [&](int mi, int ni) {
    acc[mi][ni] = mfma16(__builtin_bit_cast(bf16x8, af[mi]), __builtin_bit_cast(bf16x8, bf[ni]), acc[mi][ni]);
  };
  asm volatile("s_waitcnt lgkmcnt(3)" : "+v"(af[0]), "+v"(bf[0]), "+v"(bf[1]), "+v"(bf[2]), "+v"(bf[3]));
#pragma unroll
  for (int ni = 0; ni < 4; ++ni) mm(0, ni);
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(af[1]), "+v"(af[2]), "+v"(af[3]));
#pragma unroll
  for (int mi = 1; mi < 4; ++mi)
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) mm(mi, ni);
}

// Cross-step form of mma_64x128_dsasm for rings whose next stage is known to
// have landed while the current one is multiplied:
//   frags_64x128_wait(f)        f (read one step earlier) has arrived: all of
//                               the wave's LDS reads are waited for, so no
//                               more than 12 are ever in flight;
//   frag_64x128_read<I>(a, b, g)  starts fragment read I (0..3: A rows
//                               16 I.., 4..11: B rows 16 (I - 4)..) of the
//                               next step, a and b from frag_64x128_base;
//   mma_64x128_frags(f, acc, between)
//                               the step's 32 MFMAs in 8 groups of 4 (one B
//                               fragment each); between(integral_constant<G>)
//                               runs after group G, fenced so that the
//                               scheduler keeps it there.
// A caller spreads the next step's fragment reads (and its DMAs) over the
// groups: issued together after a barrier, 8 waves' reads (96 KiB) queue in
// the LDS for hundreds of cycles, and each wave's MFMAs wait behind its own
// reads' issue.
__device__ __forceinline__ uint32_t frag_64x128_base(const bf16_t* M, int lane, int row) {
  return lds_addr(M) + (uint32_t)(2 * lds_off(row + (lane & 15), lane >> 4));
}
template <int I>
__device__ __forceinline__ void frag_64x128_read(uint32_t a, uint32_t b, u32x4 (&af)[4], u32x4 (&bf)[8]) {
  if constexpr (I < 4)
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(af[I]) : "v"(a), "n"(I * 1024));
  else
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(bf[I - 4]) : "v"(b), "n"((I - 4) * 1024));
}
__device__ __forceinline__ void frags_64x128_wait(u32x4 (&af)[4], u32x4 (&bf)[8]) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(af[0]), "+v"(af[1]), "+v"(af[2]), "+v"(af[3]), "+v"(bf[0]), "+v"(bf[1]), "+v"(bf[2]),
                 "+v"(bf[3]), "+v"(bf[4]), "+v"(bf[5]), "+v"(bf[6]), "+v"(bf[7]));
}
template <int G, class Between>
__device__ __forceinline__ void mma_64x128_group(const u32x4 (&af)[4], const u32x4 (&bf)[8], floatx4 (&acc)[4][8],
                                                 Between& between) {
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
    acc[mi][G] = mfma16(__builtin_bit_cast(bf16x8, af[mi]), __builtin_bit_cast(bf16x8, bf[G]), acc[mi][G]);
  __builtin_amdgcn_sched_barrier(0);
  between(std::integral_constant<int, G>{});
  __builtin_amdgcn_sched_barrier(0);
}
template <class Between, int... G>
__device__ __forceinline__ void mma_64x128_groups(const u32x4 (&af)[4], const u32x4 (&bf)[8], floatx4 (&acc)[4][8],
                                                  Between& between, std::integer_sequence<int, G...>) {
  (mma_64x128_group<G>(af, bf, acc, between), ...);
}
template <class Between>
__device__ __forceinline__ void mma_64x128_frags(u32x4 (&af)[4], u32x4 (&bf)[8], floatx4 (&acc)[4][8],
                                                 Between&& between) {
  __builtin_amdgcn_sched_barrier(0);
  mma_64x128_groups(af, bf, acc, between, std::make_integer_sequence<int, 8>{});
}

// Per-wave progress counters in LDS, each written by its one wave: a wave
// waits until the least of a group's 4 counters (one 16-byte read at byte
// address a) reaches target.  A poll, then a short sleep; bounded (about
// 2^20 polls, tens of milliseconds), so it ends whatever happens; the
// protocols that use it wait a few K steps at most.
// seen: the least value this wave last read (counters only grow), so a wait
// that an earlier poll already satisfied reads nothing.  N = 4 or 8
// counters, 16-byte aligned.
template <int N>
__device__ __forceinline__ void wave_wait_min(uint32_t a, uint32_t target, uint32_t& seen) {
  typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
  for (int poll = 0; poll < (1 << 20) && seen < target; ++poll) {
    if (poll > 0) __builtin_amdgcn_s_sleep(1);
    u32x4_t v, u = u32x4_t{0xffffffffu, 0xffffffffu, 0xffffffffu, 0xffffffffu};
    if (N == 8) {
      asm volatile("ds_read_b128 %0, %2\n\tds_read_b128 %1, %2 offset:16\n\ts_waitcnt lgkmcnt(0)"
                   : "=&v"(v), "=&v"(u) : "v"(a) : "memory");
    } else {
      asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(a) : "memory");
    }
    const uint32_t m = min(min(min(v.x, v.y), min(v.z, v.w)), min(min(u.x, u.y), min(u.z, u.w)));
    seen = (uint32_t)__builtin_amdgcn_readfirstlane((int)m);
  }
}
__device__ __forceinline__ void wave_count_set(uint32_t a, uint32_t value, int lane) {
  if (lane == 0) asm volatile("ds_write_b32 %0, %1" ::"v"(a), "v"(value) : "memory");
}

}  // namespace mfma
}  // namespace bdh
