// bdh_decode_step_noalloc: the decode step of bdh_decode_step without any
// device allocation, for callers that cannot allocate (code under HIP graph
// capture, tight serving loops).  Its buffers live in one file-scope device
// array of NOALLOC_BYTES, one copy per GPU, shared by every call on that GPU
// (calls that overlap on one GPU race on its range region):
//   [0, TABLE_BYTES)  RoPE frequency tables, one slot per (latent, theta)
//                     used on the device, assigned in order of first use and
//                     never overwritten: a graph captured with one key keeps
//                     valid frequencies whatever keys later calls use.  A key
//                     that no longer fits is refused (BDH_UNSUPPORTED);
//   [TABLE_BYTES, ..) range readouts, range lists and counts of a stream
//                     split into row ranges (decode_part_bytes), every
//                     element written by the decode kernel before the
//                     finalize kernel reads it, so nothing needs clearing.
// Host code never uses the array's name as an address: the address of each
// device's copy comes from hipGetSymbolAddress at the first call on that
// device and is kept per device.
#include <string.h>

#include <memory>
#include <mutex>
#include <vector>

#include "bdh_internal.h"

namespace {

constexpr size_t NOALLOC_BYTES = (size_t)16 << 20;
constexpr size_t TABLE_BYTES = (size_t)8 << 20;
constexpr size_t RANGE_BYTES = NOALLOC_BYTES - TABLE_BYTES;
constexpr int64_t NOALLOC_MAX_LATENT = (int64_t)1 << 20;  // one table of 4 MiB

static __device__ __align__(256) unsigned char noalloc_scratch[NOALLOC_BYTES];

struct TableSlot {
  int64_t latent;
  uint32_t theta_bits;
  size_t offset;                     // from the start of the array
  std::unique_ptr<float[]> host;     // host copy; outlives its upload
};

constexpr int kMaxDevices = 64;
struct DeviceSlot {
  bool ready = false;
  unsigned char* ptr = nullptr;  // this device's copy of noalloc_scratch
  size_t table_used = 0;         // bytes of the table region assigned
  std::vector<TableSlot> tables;
};
std::mutex g_mu;
DeviceSlot g_dev[kMaxDevices];

size_t round256(size_t n) { return (n + 255) / 256 * 256; }

}  // namespace

using namespace bdh;

extern "C" bdh_status bdh_decode_step_noalloc(int64_t batch, int64_t heads, int64_t value_heads,
                                              int64_t latent, int64_t embd, const float* x,
                                              const float* value, float* rho, const float* decay,
                                              const bdh_rope* rope, float* a_out,
                                              int32_t* active_idx_out, int32_t* active_cnt_out,
                                              void* stream) {
  if (batch <= 0 || heads <= 0 || latent <= 0 || embd <= 0)
    return fail(BDH_UNSUPPORTED, "zero-sized dimension");
  if (value_heads != 1 && value_heads != heads) return fail(BDH_UNSUPPORTED, "value_heads must be 1 or heads");
  if (batch * heads > 65535) return fail(BDH_UNSUPPORTED, "batch * heads exceeds 65535");
  if (!x || !value || !rho || !a_out) return fail(BDH_EINVAL, "null tensor pointer");
  for (const void* t : {(const void*)x, (const void*)value, (const void*)rho, (const void*)decay,
                        (const void*)a_out, (const void*)active_idx_out, (const void*)active_cnt_out})
    if (((uintptr_t)t & 3) != 0) return fail(BDH_EINVAL, "tensor pointers must be 4-byte aligned");
  if (rope && rope->mode != BDH_ROPE_SEQUENTIAL && rope->mode != BDH_ROPE_FIXED)
    return fail(BDH_EINVAL, "unknown rope mode");
  if (rope && latent % 2 != 0) return fail(BDH_UNSUPPORTED, "RoPE needs an even latent");
  if (rope && (rope->pos0 < 0 || rope->pos0 >= (int64_t)1 << 24))
    return fail(BDH_UNSUPPORTED, "position must lie in [0, 2^24)");
  if (rope && !(rope->theta > 0.0f)) return fail(BDH_EINVAL, "rope theta must be > 0");
  if (latent > NOALLOC_MAX_LATENT)
    return fail(BDH_UNSUPPORTED, "bdh_decode_step_noalloc: latent exceeds 1048576 (one frequency table slot)");

  hipStream_t st = (hipStream_t)stream;
  DecodeArgs a;
  a.x = x;
  a.v = value;
  a.rho_in = rho;
  a.rho = rho;
  a.decay = decay;
  a.freqs = nullptr;
  a.pos = rope ? (float)rope->pos0 : 0.0f;
  a.a_out = a_out;
  a.idx_out = active_idx_out;
  a.cnt_out = active_cnt_out;
  a.B = batch;
  a.H = heads;
  a.Hv = value_heads;
  a.N = latent;
  a.D = embd;
  const size_t part = decode_part_bytes(a);
  if (part > RANGE_BYTES)
    return fail(BDH_UNSUPPORTED, "bdh_decode_step_noalloc: the range buffers of this shape exceed its " +
                                     std::to_string(RANGE_BYTES >> 20) +
                                     " MiB range region; use bdh_decode_step");

  int dev = 0;
  BDH_HIP_TRY(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) return fail(BDH_UNSUPPORTED, "device ordinal out of range");
  std::lock_guard<std::mutex> lock(g_mu);
  DeviceSlot& ds = g_dev[dev];
  if (!ds.ready) {
    // This device's copy of the array (the current device is `dev`).
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(noalloc_scratch));
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(noalloc_scratch)");
    ds.ptr = (unsigned char*)p;
    ds.ready = true;
  }
  if (rope) {
    uint32_t tb;
    memcpy(&tb, &rope->theta, 4);
    const TableSlot* slot = nullptr;
    for (const TableSlot& t : ds.tables)
      if (t.latent == latent && t.theta_bits == tb) slot = &t;
    if (!slot) {
      // A new key gets the next free slot, computed on the host
      // (attention.rs:552-576, the same f32 arithmetic as every other entry
      // point) and copied in.  Slots already assigned are never touched.
      const size_t bytes = round256((size_t)latent * sizeof(float));
      if (ds.table_used + bytes > TABLE_BYTES)
        return fail(BDH_UNSUPPORTED,
                    "bdh_decode_step_noalloc: its " + std::to_string(TABLE_BYTES >> 20) +
                        " MiB frequency-table region holds " + std::to_string(ds.tables.size()) +
                        " (latent, theta) keys and has no room for another; use bdh_decode_step");
      bool capturing = false;
      stream_capturing(st, &capturing);
      if (capturing)
        return fail(BDH_UNSUPPORTED,
                    "bdh_decode_step_noalloc: the RoPE table of this (latent, theta) is uploaded on "
                    "its first call on the device, which cannot happen during graph capture: call "
                    "it once eagerly first");
      TableSlot t;
      t.latent = latent;
      t.theta_bits = tb;
      t.offset = ds.table_used;
      t.host.reset(new float[(size_t)latent]);
      rope_freqs_host(latent, rope->theta, t.host.get());
      BDH_HIP_TRY(hipMemcpyAsync(ds.ptr + t.offset, t.host.get(), (size_t)latent * sizeof(float),
                                 hipMemcpyHostToDevice, st));
      // Later calls may run on other streams: the table is complete before
      // this call returns.
      BDH_HIP_TRY(hipStreamSynchronize(st));
      ds.table_used += bytes;
      ds.tables.push_back(std::move(t));
      slot = &ds.tables.back();
    }
    a.freqs = (const float*)(ds.ptr + slot->offset);
  }
  a.part_buf = ds.ptr + TABLE_BYTES;
  a.part_bytes = RANGE_BYTES;
  return run_decode(a, st, nullptr);
}
