// C ABI of libbdh_hip (declared in include/bdh_hip.h): argument validation
// with the reference's None semantics, path selection, per-device scratch,
// the RoPE frequency table and the profiling counters.
#include <math.h>

#include <cmath>
#include <string.h>

#include <atomic>
#include <chrono>
#include <map>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "bdh_internal.h"

namespace bdh {

// ---------------------------------------------------------------- errors ----
static thread_local std::string g_last_error;

bdh_status fail(bdh_status st, const std::string& msg) {
  g_last_error = msg;
  return st;
}

bdh_status hip_fail(hipError_t e, const char* what) {
  return fail(BDH_EHIP, std::string(what) + ": " + hipGetErrorString(e));
}

// --------------------------------------------------------------- scratch ----
// Scratch is kept per (device, stream): calls on different streams never
// share a buffer, so they may run concurrently.  A slot grows (by 1.25x) on
// the first call that needs more.  Growth is refused while the stream is
// being captured into a graph (a graph must only hold buffers that outlive
// it: run the largest shape once eagerly on the capturing stream first).
// A replaced buffer is freed once this stream's queued work is done, unless
// a graph was ever captured on the stream with this set: a graph keeps its
// buffer pointers, so the buffer then stays until bdh_scratch_release.
namespace {
struct ScratchSet {
  void* ptr[SLOT_COUNT] = {};
  size_t bytes[SLOT_COUNT] = {};
  bool captured = false;
  std::vector<void*> retired;
};
std::mutex g_scratch_mu;
std::map<std::pair<int, hipStream_t>, ScratchSet> g_sets;
std::map<int, std::map<std::pair<int64_t, uint32_t>, float*>> g_freqs;

// Counters of the entry point running on this thread (profile snapshot).
struct CallCounters {
  uint64_t allocations = 0, upload_bytes = 0, reuse_hits = 0, reuse_bytes = 0;
};
thread_local CallCounters t_call;
}  // namespace

bdh_status stream_capturing(hipStream_t st, bool* capturing) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  const hipError_t e = hipStreamIsCapturing(st, &cs);
  // An implicit capture error (the legacy stream queried while another
  // stream captures) counts as capturing.
  *capturing = e != hipSuccess || cs != hipStreamCaptureStatusNone;
  if (e != hipSuccess) (void)hipGetLastError();
  return BDH_OK;
}

bdh_status scratch(hipStream_t st, int slot, size_t bytes, void** out, bool zero_on_alloc) {
  int dev = 0;
  BDH_HIP_TRY(hipGetDevice(&dev));
  bool capturing = false;
  stream_capturing(st, &capturing);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  ScratchSet& ss = g_sets[{dev, st}];
  if (capturing) {
    ss.captured = true;
  } else if (ss.captured) {
    // The first eager call after a capture leaves the set's buffers to the
    // captured graphs (retired: kept until bdh_scratch_release) and takes
    // fresh ones, so a replay on another stream never shares a buffer with
    // eager work on the capturing stream.
    for (int i = 0; i < SLOT_COUNT; ++i) {
      if (ss.ptr[i]) ss.retired.push_back(ss.ptr[i]);
      ss.ptr[i] = nullptr;
      ss.bytes[i] = 0;
    }
    ss.captured = false;
  }
  if (bytes == 0) bytes = 256;
  if (ss.bytes[slot] < bytes) {
    if (capturing)
      return fail(BDH_UNSUPPORTED,
                  "scratch must grow, which cannot happen during graph capture: run this shape "
                  "once eagerly on the capturing stream before capturing");
    if (ss.ptr[slot]) {
      if (ss.captured) {
        ss.retired.push_back(ss.ptr[slot]);
      } else {
        // Work queued on this stream may still use the old buffer.
        BDH_HIP_TRY(hipStreamSynchronize(st));
        BDH_HIP_TRY(hipFree(ss.ptr[slot]));
      }
      ss.ptr[slot] = nullptr;
      ss.bytes[slot] = 0;
    }
    const size_t grow = bytes + bytes / 4;
    void* p = nullptr;
    BDH_HIP_TRY(hipMalloc(&p, grow));
    ++t_call.allocations;
    if (zero_on_alloc) BDH_HIP_TRY(hipMemsetAsync(p, 0, grow, st));
    ss.ptr[slot] = p;
    ss.bytes[slot] = grow;
  }
  *out = ss.ptr[slot];
  return BDH_OK;
}

bdh_status scratch_release(hipStream_t st) {
  int dev = 0;
  BDH_HIP_TRY(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  auto it = g_sets.find({dev, st});
  if (it == g_sets.end()) return BDH_OK;
  BDH_HIP_TRY(hipStreamSynchronize(st));
  for (int i = 0; i < SLOT_COUNT; ++i)
    if (it->second.ptr[i]) BDH_HIP_TRY(hipFree(it->second.ptr[i]));
  for (void* p : it->second.retired) BDH_HIP_TRY(hipFree(p));
  g_sets.erase(it);
  return BDH_OK;
}


// ------------------------------------------------------------------ RoPE ----
// Attention::build_freqs, Rope arm (attention.rs:559-563), in f32:
//   exponent = (floor(idx / 2) * 2) / latent ; f = 1 / theta^exponent / (2 pi)
void rope_freqs_host(int64_t latent, float theta, float* out) {
  const float two_pi = 2.0f * 3.14159265358979323846f;
  for (int64_t idx = 0; idx < latent; ++idx) {
    volatile float exponent = (floorf((float)idx / 2.0f) * 2.0f) / (float)latent;
    volatile float inv = 1.0f / powf(theta, exponent);
    out[idx] = inv / two_pi;
  }
}

// Device copy of the table, one per (device, latent, theta), shared by all
// streams (read-only once written).  The upload is synchronous and happens
// once per key; it is refused during graph capture.
bdh_status rope_freqs_device(int64_t latent, float theta, hipStream_t st, const float** out) {
  int dev = 0;
  BDH_HIP_TRY(hipGetDevice(&dev));
  uint32_t tbits;
  memcpy(&tbits, &theta, 4);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  auto& m = g_freqs[dev];
  auto it = m.find({latent, tbits});
  if (it != m.end()) {
    ++t_call.reuse_hits;
    t_call.reuse_bytes += sizeof(float) * (uint64_t)latent;
    *out = it->second;
    return BDH_OK;
  }
  bool capturing = false;
  stream_capturing(st, &capturing);
  if (capturing)
    return fail(BDH_UNSUPPORTED,
                "the RoPE frequency table of this (latent, theta) is uploaded on first use, which "
                "cannot happen during graph capture: run one eager call first");
  std::vector<float> host((size_t)latent);
  rope_freqs_host(latent, theta, host.data());
  float* d = nullptr;
  BDH_HIP_TRY(hipMalloc(&d, sizeof(float) * (size_t)latent));
  ++t_call.allocations;
  BDH_HIP_TRY(hipMemcpy(d, host.data(), sizeof(float) * (size_t)latent, hipMemcpyHostToDevice));
  t_call.upload_bytes += sizeof(float) * (uint64_t)latent;
  m[{latent, tbits}] = d;
  *out = d;
  return BDH_OK;
}

// ------------------------------------------------------------- profiling ----
namespace {
std::mutex g_prof_mu;
bdh_profile_snapshot g_prof = {};
bool prof_env() {
  const char* a = getenv("DragonModel_STAGE_PROFILE");
  const char* b = getenv("BDH_STAGE_PROFILE");
  return (a && *a) || (b && *b);
}
bool g_prof_on = prof_env();

// One entry-point call.  The fields follow KernelProfileSnapshot
// (profiling.rs:3-16) as recurrent.rs:206-215, 344-356 fills them, with this
// library's meaning of each:
//   setup_ns      validation, plan and table lookup before the first launch;
//   copy_ns       host time of separate rho copies (none: the private copy of
//                 the reference, recurrent.rs:259, is fused into the kernel
//                 that writes rho_out), so it stays 0;
//   transient_allocations  device buffers allocated by the call (scratch
//                 growth, a first-use table); 0 once a shape is warm, where
//                 the reference allocates 5 per call;
//   metadata_upload_bytes  host-to-device bytes of shape tables (the RoPE
//                 frequencies on first use; plans upload nothing);
//   metadata_reuse_hits / _bytes  calls that found their table resident;
//   resident_rollout_steps  T = 1 steps that updated rho in place through
//                 the sparse decode (the state never left HBM).
struct ProfScope {
  std::chrono::steady_clock::time_point t0 = std::chrono::steady_clock::now();
  uint64_t launches = 0;
  uint64_t setup_ns = 0;
  uint64_t rollout_steps = 0;
  ProfScope() { t_call = CallCounters{}; }
  void done(bool ok) {
    if (!g_prof_on) return;
    const auto ns = (uint64_t)std::chrono::duration_cast<std::chrono::nanoseconds>(
                        std::chrono::steady_clock::now() - t0).count();
    std::lock_guard<std::mutex> lock(g_prof_mu);
    g_prof.calls += ok ? 1 : 0;
    g_prof.launches += launches;
    g_prof.total_ns += ns;
    g_prof.setup_ns += setup_ns;
    g_prof.dispatch_ns += ns > setup_ns ? ns - setup_ns : 0;
    g_prof.transient_allocations += t_call.allocations;
    g_prof.metadata_upload_bytes += t_call.upload_bytes;
    g_prof.metadata_reuse_hits += t_call.reuse_hits;
    g_prof.metadata_reuse_bytes += t_call.reuse_bytes;
    g_prof.resident_rollout_steps += rollout_steps;
  }
};
}  // namespace

// ----------------------------------------------------------- kernel timing --
namespace {
struct KTimeRec {
  hipEvent_t start, stop;
  int kind;
};
std::mutex g_kt_mu;
std::atomic<bool> g_kt_on{false};
std::vector<KTimeRec> g_kt_recs;
std::vector<hipEvent_t> g_kt_pool;

hipEvent_t kt_event() {
  if (!g_kt_pool.empty()) {
    hipEvent_t e = g_kt_pool.back();
    g_kt_pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

void kt_clear() {
  for (auto& r : g_kt_recs) {
    g_kt_pool.push_back(r.start);
    g_kt_pool.push_back(r.stop);
  }
  g_kt_recs.clear();
}
}  // namespace

int ktime_begin(int kind, hipStream_t st) {
  if (!g_kt_on) return -1;
  std::lock_guard<std::mutex> lock(g_kt_mu);
  KTimeRec r{kt_event(), kt_event(), kind};
  if (!r.start || !r.stop || hipEventRecord(r.start, st) != hipSuccess) {
    if (r.start) g_kt_pool.push_back(r.start);
    if (r.stop) g_kt_pool.push_back(r.stop);
    return -1;
  }
  g_kt_recs.push_back(r);
  return (int)g_kt_recs.size() - 1;
}

void ktime_end(int handle, hipStream_t st) {
  if (handle < 0) return;
  std::lock_guard<std::mutex> lock(g_kt_mu);
  if (handle < (int)g_kt_recs.size()) (void)hipEventRecord(g_kt_recs[handle].stop, st);
}

}  // namespace bdh

using namespace bdh;

namespace {

constexpr int64_t kMaxGrid = 65535;

bdh_status check_plan(const bdh_recurrent_plan* p) {
  if (!p) return fail(BDH_EINVAL, "plan is null");
  if (p->batch <= 0 || p->heads <= 0 || p->time <= 0 || p->latent <= 0 || p->embd <= 0)
    return fail(BDH_UNSUPPORTED, "zero-sized dimension");
  if (p->value_heads != 1 && p->value_heads != p->heads)
    return fail(BDH_UNSUPPORTED, "value_heads must be 1 or heads");
  if (p->batch * p->heads > kMaxGrid) return fail(BDH_UNSUPPORTED, "batch * heads exceeds 65535");
  return BDH_OK;
}

// State-carry interval of the MFMA path: rho is materialised every L tokens
// and the carries in between go through the chunk-pair score blocks.  L is
// the call's row chunk (the reference's dense_score_row_chunk, config.rs:46,
// default 512 at config.rs:10, used as linear.rs:117-118 uses it), shortened
// to the call's length rounded up to 128.
constexpr int64_t kMaxRowChunk = 4096;
// Row chunk 0 = auto: 512, the reference's default, which is also the
// fastest of the state-carry form (with or without decay): the gram work
// grows with the chunk, the snapshots shrink with it (C4: 0.74 ms at 512,
// 0.77 at 768, 0.81 at 1024).
int64_t state_interval(int64_t T, int32_t chunk, bool decay) {
  (void)decay;
  const int64_t L = chunk > 0 ? chunk : 512;
  return T < L ? ((T + 127) / 128) * 128 : L;
}

bdh_status forward_common(const bdh_recurrent_plan* plan, int32_t dtype, const void* q,
                          const void* v, const float* rho_in, const float* decay,
                          const bdh_rope* rope, float* ctx, float* rho_out, int32_t chunk,
                          void* stream, bool want_rho) {
  ProfScope prof;
  bdh_status st = check_plan(plan);
  if (st != BDH_OK) return st;
  if (!q || !v || !ctx || (want_rho && !rho_out)) return fail(BDH_EINVAL, "null tensor pointer");
  // The kernels move 16 bytes per lane.
  for (const void* t : {q, v, (const void*)rho_in, (const void*)ctx, (const void*)rho_out})
    if (((uintptr_t)t & 15) != 0) return fail(BDH_EINVAL, "tensor pointers must be 16-byte aligned");
  if (dtype != BDH_F32 && dtype != BDH_BF16) return fail(BDH_EINVAL, "unknown dtype");
  if (chunk < 0 || (chunk > 0 && (chunk % 128 != 0 || chunk > kMaxRowChunk)))
    return fail(BDH_UNSUPPORTED, "chunk must be 0 (auto) or a multiple of 128 up to 4096");
  if (rope && (rope->mode != BDH_ROPE_SEQUENTIAL && rope->mode != BDH_ROPE_FIXED))
    return fail(BDH_EINVAL, "unknown rope mode");
  if (rope && plan->latent % 2 != 0) return fail(BDH_UNSUPPORTED, "RoPE needs an even latent");
  if (rope && !(rope->theta > 0.0f)) return fail(BDH_EINVAL, "rope theta must be > 0");
  if (rope && (rope->pos0 < 0 || rope->pos0 + plan->time > (int64_t)1 << 24))
    return fail(BDH_UNSUPPORTED, "positions must lie in [0, 2^24) to be exact in f32");
  hipStream_t hs = (hipStream_t)stream;
  const int64_t B = plan->batch, H = plan->heads, Hv = plan->value_heads, T = plan->time,
                N = plan->latent, D = plan->embd;

  const float* freqs = nullptr;
  if (rope) {
    st = rope_freqs_device(N, rope->theta, hs, &freqs);
    if (st != BDH_OK) return st;
  }
  prof.setup_ns = (uint64_t)std::chrono::duration_cast<std::chrono::nanoseconds>(
                      std::chrono::steady_clock::now() - prof.t0).count();

  // One token: the reference picks its kernel by T (forward_runtime.rs:
  // 235-256) and decodes through this same op (sequence_dispatch.rs:109-124).
  // fp32 runs the one-token step: the sparse row gather when rho is updated
  // in place without decay, otherwise one dense pass that writes every row
  // of rho_out (the private copy fused with the update).
  if (T == 1 && dtype == BDH_F32 && want_rho) {
    DecodeArgs d;
    d.x = (const float*)q;
    d.v = (const float*)v;
    d.rho_in = rho_in;
    d.rho = rho_out;
    d.decay = decay;
    d.freqs = freqs;
    d.pos = rope ? (float)rope->pos0 : 0.0f;
    d.a_out = ctx;
    d.idx_out = nullptr;
    d.cnt_out = nullptr;
    d.B = B; d.H = H; d.Hv = Hv; d.N = N; d.D = D;
    if (N > (int64_t)1 << 24) return fail(BDH_UNSUPPORTED, "latent too large for the one-token step");
    st = run_decode(d, hs, &prof.launches);
    if (st != BDH_OK) return st;
    if (rho_in && rho_in == rho_out && !decay) prof.rollout_steps = 1;
    prof.done(true);
    return BDH_OK;
  }

  if (dtype == BDH_F32) {
    const float* qr = (const float*)q;
    if (rope) {
      void* rot = nullptr;
      st = scratch(hs, SLOT_ROTATED, (size_t)(B * H * T * N) * sizeof(float), &rot);
      if (st != BDH_OK) return st;
      BDH_HIP_TRY(launch_rope_rotate_f32((const float*)q, freqs, (float*)rot, B * H, T, N,
                                         rope->pos0, rope->mode == BDH_ROPE_FIXED, hs));
      ++prof.launches;
      qr = (const float*)rot;
    }
    const int64_t Lmax = want_rho ? (T < 256 ? T : 256) : T;
    void* scores = nullptr;
    st = scratch(hs, SLOT_SCORES, (size_t)(B * H * Lmax * Lmax) * sizeof(float), &scores);
    if (st != BDH_OK) return st;
    F32Args a{qr, (const float*)v, want_rho ? rho_in : nullptr, decay, ctx, rho_out,
              (float*)scores, nullptr, B, H, Hv, T, N, D, Lmax, want_rho};
    const size_t pe = f32_path_part_elems(a);
    if (pe) {
      void* part = nullptr;
      st = scratch(hs, SLOT_GEMM_PART, pe * sizeof(float), &part);
      if (st != BDH_OK) return st;
      a.part = (float*)part;
    }
    hipError_t e = run_f32_path(a, hs, &prof.launches);
    if (e != hipSuccess) return hip_fail(e, "fp32 path launch");
    prof.done(true);
    return BDH_OK;
  }

  const char* why = nullptr;
  if (!bf16_shape_supported(N, D, &why)) return fail(BDH_UNSUPPORTED, why);
  Bf16Args a;
  a.x = (const bf16_t*)q;
  a.v = (const bf16_t*)v;
  a.rho_in = want_rho ? rho_in : nullptr;
  a.decay = decay;
  a.freqs = freqs;
  a.pos0 = rope ? rope->pos0 : 0;
  a.fixed = rope ? rope->mode == BDH_ROPE_FIXED : 0;
  a.ctx = ctx;
  a.rho_out = rho_out;
  a.B = B;
  a.H = H;
  a.Hv = Hv;
  a.T = T;
  a.N = N;
  a.D = D;
  a.L = want_rho ? state_interval(T, chunk, decay != nullptr) : ((T + 127) / 128) * 128;
  a.state = want_rho;
  st = run_bf16_path(a, hs, &prof.launches);
  if (st != BDH_OK) return st;
  prof.done(true);
  return BDH_OK;
}

}  // namespace

extern "C" {

bdh_status bdh_rope_freqs(int64_t latent, float theta, float* freqs_out) {
  if (!freqs_out) return fail(BDH_EINVAL, "freqs_out is null");
  if (latent <= 0) return fail(BDH_UNSUPPORTED, "latent must be > 0");
  rope_freqs_host(latent, theta, freqs_out);
  return BDH_OK;
}

bdh_status bdh_recurrent_plan_new(int64_t batch, int64_t heads, int64_t value_heads, int64_t time,
                                  int64_t latent, int64_t embd, bdh_recurrent_plan* out) {
  if (!out) return fail(BDH_EINVAL, "out is null");
  bdh_recurrent_plan p{batch, heads, value_heads, time, latent, embd};
  bdh_status st = check_plan(&p);
  if (st != BDH_OK) return st;
  *out = p;
  return BDH_OK;
}

int32_t bdh_supports_backend(void) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return 0;
  return strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
}

bdh_status bdh_recurrent_attention_fwd(const bdh_recurrent_plan* plan, int32_t dtype,
                                       const void* query, const void* value, const float* rho_in,
                                       const float* decay, float* context_out, float* rho_out,
                                       int32_t chunk, void* stream) {
  return forward_common(plan, dtype, query, value, rho_in, decay, nullptr, context_out, rho_out,
                        chunk, stream, true);
}

bdh_status bdh_recurrent_attention_rope_fwd(const bdh_recurrent_plan* plan, int32_t dtype,
                                            const void* x, const void* value, const float* rho_in,
                                            const float* decay, const bdh_rope* rope,
                                            float* context_out, float* rho_out, int32_t chunk,
                                            void* stream) {
  if (!rope) return fail(BDH_EINVAL, "rope is null");
  return forward_common(plan, dtype, x, value, rho_in, decay, rope, context_out, rho_out, chunk,
                        stream, true);
}

bdh_status bdh_dense_causal_attention_fwd(const bdh_recurrent_plan* plan, int32_t dtype,
                                          const void* query, const void* value, const float* decay,
                                          float* context_out, void* stream) {
  bdh_status st = check_plan(plan);
  if (st != BDH_OK) return st;
  if (plan->time > 1024) return fail(BDH_UNSUPPORTED, "dense causal attention needs time <= 1024");
  return forward_common(plan, dtype, query, value, nullptr, decay, nullptr, context_out, nullptr,
                        0, stream, false);
}

bdh_status bdh_decode_step(int64_t batch, int64_t heads, int64_t value_heads, int64_t latent,
                           int64_t embd, const float* x, const float* value, float* rho,
                           const float* decay, const bdh_rope* rope, float* a_out,
                           int32_t* active_idx_out, int32_t* active_cnt_out, void* stream) {
  ProfScope prof;
  bdh_recurrent_plan p{batch, heads, value_heads, 1, latent, embd};
  bdh_status st = check_plan(&p);
  if (st != BDH_OK) return st;
  if (!x || !value || !rho || !a_out) return fail(BDH_EINVAL, "null tensor pointer");
  for (const void* t : {(const void*)x, (const void*)value, (const void*)rho, (const void*)decay,
                        (const void*)a_out, (const void*)active_idx_out, (const void*)active_cnt_out})
    if (((uintptr_t)t & 3) != 0) return fail(BDH_EINVAL, "tensor pointers must be 4-byte aligned");
  if (latent > (int64_t)1 << 24) return fail(BDH_UNSUPPORTED, "latent too large");
  if (rope && rope->mode != BDH_ROPE_SEQUENTIAL && rope->mode != BDH_ROPE_FIXED)
    return fail(BDH_EINVAL, "unknown rope mode");
  if (rope && latent % 2 != 0) return fail(BDH_UNSUPPORTED, "RoPE needs an even latent");
  if (rope && (rope->pos0 < 0 || rope->pos0 >= (int64_t)1 << 24))
    return fail(BDH_UNSUPPORTED, "position must lie in [0, 2^24)");
  if (rope && !(rope->theta > 0.0f)) return fail(BDH_EINVAL, "rope theta must be > 0");
  const float* freqs = nullptr;
  if (rope) {
    st = rope_freqs_device(latent, rope->theta, (hipStream_t)stream, &freqs);
    if (st != BDH_OK) return st;
  }
  DecodeArgs a;
  a.x = x;
  a.v = value;
  a.rho_in = rho;
  a.rho = rho;
  a.decay = decay;
  a.freqs = freqs;
  a.pos = rope ? (float)rope->pos0 : 0.0f;
  a.a_out = a_out;
  a.idx_out = active_idx_out;
  a.cnt_out = active_cnt_out;
  a.B = batch;
  a.H = heads;
  a.Hv = value_heads;
  a.N = latent;
  a.D = embd;
  st = run_decode(a, (hipStream_t)stream, &prof.launches);
  if (st != BDH_OK) return st;
  if (!decay) prof.rollout_steps = 1;
  prof.done(true);
  return BDH_OK;
}

bdh_status bdh_scratch_release(void* stream) { return scratch_release((hipStream_t)stream); }

static bdh_status vjp_common(const bdh_recurrent_plan* plan, const float* query, const float* value,
                             const float* decay, const float* rho0, const float* grad_out,
                             float* grad_query, float* grad_value, float* grad_decay, float* grad_rho0,
                             void* stream, bool recurrent) {
  ProfScope prof;
  bdh_status st = check_plan(plan);
  if (st != BDH_OK) return st;
  if (!query || !value || !grad_out || !grad_query || !grad_value)
    return fail(BDH_EINVAL, "null tensor pointer");
  if (grad_rho0 && !rho0) return fail(BDH_EINVAL, "grad_rho0 needs the initial state rho0");
  for (const void* t : {(const void*)query, (const void*)value, (const void*)decay, (const void*)rho0,
                        (const void*)grad_out, (const void*)grad_query, (const void*)grad_value,
                        (const void*)grad_decay, (const void*)grad_rho0})
    if (((uintptr_t)t & 3) != 0) return fail(BDH_EINVAL, "tensor pointers must be 4-byte aligned");
  if (plan->latent > ((int64_t)1 << 24) || plan->embd > ((int64_t)1 << 24))
    return fail(BDH_UNSUPPORTED, "latent and embd must be below 2^24");
  VjpArgs a;
  a.q = query;
  a.v = value;
  a.decay = decay;
  a.rho0 = rho0;
  a.g = grad_out;
  a.grad_q = grad_query;
  a.grad_v = grad_value;
  a.grad_decay = grad_decay;
  a.grad_rho0 = grad_rho0;
  a.B = plan->batch;
  a.H = plan->heads;
  a.Hv = plan->value_heads;
  a.T = plan->time;
  a.N = plan->latent;
  a.D = plan->embd;
  a.recurrent_eps = recurrent;
  st = run_attention_vjp(a, (hipStream_t)stream, &prof.launches);
  if (st != BDH_OK) return st;
  prof.done(true);
  return BDH_OK;
}

bdh_status bdh_dense_causal_attention_vjp(const bdh_recurrent_plan* plan, const float* query,
                                          const float* value, const float* decay, const float* rho0,
                                          const float* grad_output, float* grad_query, float* grad_value,
                                          float* grad_decay, float* grad_rho0, void* stream) {
  return vjp_common(plan, query, value, decay, rho0, grad_output, grad_query, grad_value, grad_decay,
                    grad_rho0, stream, false);
}

bdh_status bdh_recurrent_attention_vjp(const bdh_recurrent_plan* plan, const float* query,
                                       const float* value, const float* rho_in, const float* decay,
                                       const float* grad_context, float* grad_query, float* grad_value,
                                       float* grad_rho, float* grad_decay, void* stream) {
  return vjp_common(plan, query, value, decay, rho_in, grad_context, grad_query, grad_value, grad_decay,
                    grad_rho, stream, true);
}

bdh_status bdh_lowrank_pack_weights(int64_t heads, int64_t latent, int64_t embd,
                                    const float* encoder, const float* encoder_v,
                                    const float* decoder, void* encoder_packed,
                                    void* encoder_v_packed, void* decoder_packed,
                                    void* stream) {
  ProfScope prof;
  if (heads <= 0 || latent <= 0 || embd <= 0) return fail(BDH_UNSUPPORTED, "zero-sized dimension");
  if (!encoder || !encoder_v || !decoder || !encoder_packed || !encoder_v_packed || !decoder_packed)
    return fail(BDH_EINVAL, "null tensor pointer");
  if (heads * latent > (int64_t)32 * kMaxGrid) return fail(BDH_UNSUPPORTED, "heads * latent too large");
  if (heads > kMaxGrid) return fail(BDH_UNSUPPORTED, "heads exceeds 65535");
  if ((heads * latent) % 128 != 0) return fail(BDH_UNSUPPORTED, "heads * latent must be a multiple of 128");
  bdh_status st = pack_lowrank_weights(heads, latent, embd, encoder, encoder_v, decoder,
                                       (bf16_t*)encoder_packed, (bf16_t*)encoder_v_packed,
                                       (bf16_t*)decoder_packed, (hipStream_t)stream);
  if (st != BDH_OK) return st;
  prof.launches = 3;
  prof.done(true);
  return BDH_OK;
}

bdh_status bdh_lowrank_layer_fwd(const bdh_layer_plan* plan, const float* current,
                                 const void* encoder_packed, const void* encoder_v_packed,
                                 const void* decoder_packed, const bdh_rope* rope,
                                 const float* rho_in, float* next_out, float* rho_out,
                                 void* stream) {
  return bdh_lowrank_layer_fwd_ex(plan, current, encoder_packed, encoder_v_packed, decoder_packed, rope,
                                  rho_in, next_out, rho_out, nullptr, stream);
}

bdh_status bdh_lowrank_layer_fwd_ex(const bdh_layer_plan* plan, const float* current,
                                    const void* encoder_packed, const void* encoder_v_packed,
                                    const void* decoder_packed, const bdh_rope* rope,
                                    const float* rho_in, float* next_out, float* rho_out,
                                    const bdh_layer_options* options, void* stream) {
  ProfScope prof;
  if (options && !std::isfinite(options->relu_threshold))
    return fail(BDH_EINVAL, "relu_threshold must be finite");
  if (options && options->latent_mask && ((uintptr_t)options->latent_mask & 15) != 0)
    return fail(BDH_EINVAL, "latent_mask must be 16-byte aligned");
  if (!plan) return fail(BDH_EINVAL, "null plan");
  bdh_recurrent_plan p{plan->batch, plan->heads, 1, plan->time, plan->latent, plan->embd};
  bdh_status st = check_plan(&p);
  if (st != BDH_OK) return st;
  if (!current || !encoder_packed || !encoder_v_packed || !decoder_packed || !next_out)
    return fail(BDH_EINVAL, "null tensor pointer");
  if ((const float*)next_out == current) return fail(BDH_EINVAL, "next_out must not alias current");
  for (const void* t : {(const void*)current, encoder_packed, encoder_v_packed, decoder_packed,
                        (const void*)rho_in, (const void*)next_out, (const void*)rho_out})
    if (((uintptr_t)t & 15) != 0) return fail(BDH_EINVAL, "tensor pointers must be 16-byte aligned");
  const char* why = nullptr;
  if (!layer_shape_supported(p.latent, p.embd, &why)) return fail(BDH_UNSUPPORTED, why);
  if (rope && (rope->mode != BDH_ROPE_SEQUENTIAL && rope->mode != BDH_ROPE_FIXED))
    return fail(BDH_EINVAL, "unknown rope mode");
  if (rope && !(rope->theta > 0.0f)) return fail(BDH_EINVAL, "rope theta must be > 0");
  if (rope && (rope->pos0 < 0 || rope->pos0 + p.time > (int64_t)1 << 24))
    return fail(BDH_UNSUPPORTED, "positions must lie in [0, 2^24) to be exact in f32");
  if ((p.batch * p.time + 255) / 256 * (p.heads * p.latent / 128) > ((int64_t)1 << 31) - 1)
    return fail(BDH_UNSUPPORTED, "layer too large for one launch");
  const float* freqs = nullptr;
  if (rope) {
    st = rope_freqs_device(p.latent, rope->theta, (hipStream_t)stream, &freqs);
    if (st != BDH_OK) return st;
  }
  LayerArgs a;
  a.cur = current;
  a.enc = (const bf16_t*)encoder_packed;
  a.encv = (const bf16_t*)encoder_v_packed;
  a.dec = (const bf16_t*)decoder_packed;
  a.freqs = freqs;
  a.pos0 = rope ? rope->pos0 : 0;
  a.fixed = rope ? rope->mode == BDH_ROPE_FIXED : 0;
  a.next = next_out;
  a.rho_in = rho_in;
  a.rho_out = rho_out;
  a.B = p.batch;
  a.H = p.heads;
  a.T = p.time;
  a.N = p.latent;
  a.D = p.embd;
  a.state_interval = state_interval(p.time, 0, false);  // layer attention has no decay
  a.relu_th = options ? options->relu_threshold : 0.0f;
  a.mask = options ? options->latent_mask : nullptr;
  st = run_layer(a, (hipStream_t)stream, &prof.launches);
  if (st == BDH_OK) prof.done(true);
  return st;
}

bdh_status bdh_embed_norm(const int32_t* tokens, int64_t n_tokens, const float* embed,
                          int64_t vocab, int64_t embd, float* out, void* stream) {
  ProfScope prof;
  if (n_tokens <= 0 || vocab <= 0 || embd <= 0) return fail(BDH_UNSUPPORTED, "zero-sized dimension");
  if (!tokens || !embed || !out) return fail(BDH_EINVAL, "null tensor pointer");
  if (embd % 64 != 0 || embd > 2048) return fail(BDH_UNSUPPORTED, "embd % 64 == 0 and embd <= 2048 needed");
  if ((n_tokens + 3) / 4 > ((int64_t)1 << 31) - 1) return fail(BDH_UNSUPPORTED, "too many tokens");
  bdh_status st = embed_norm(tokens, n_tokens, embed, vocab, embd, out, (hipStream_t)stream);
  if (st != BDH_OK) return st;
  prof.launches = 1;
  prof.done(true);
  return BDH_OK;
}

bdh_status bdh_lm_head_pack(int64_t embd, int64_t vocab, const float* lm_head, void* packed,
                            void* stream) {
  ProfScope prof;
  if (vocab <= 0 || embd <= 0) return fail(BDH_UNSUPPORTED, "zero-sized dimension");
  if (!lm_head || !packed) return fail(BDH_EINVAL, "null tensor pointer");
  if ((embd + 31) / 32 > kMaxGrid) return fail(BDH_UNSUPPORTED, "embd too large");
  bdh_status st = pack_lm_head(embd, vocab, lm_head, (bf16_t*)packed, (hipStream_t)stream);
  if (st != BDH_OK) return st;
  prof.launches = 1;
  prof.done(true);
  return BDH_OK;
}

bdh_status bdh_lm_logits(const float* hidden, int64_t rows, int64_t embd,
                         const void* lm_head_packed, int64_t vocab, float* logits,
                         void* stream) {
  ProfScope prof;
  if (rows <= 0 || vocab <= 0 || embd <= 0) return fail(BDH_UNSUPPORTED, "zero-sized dimension");
  if (!hidden || !lm_head_packed || !logits) return fail(BDH_EINVAL, "null tensor pointer");
  if (embd % 64 != 0) return fail(BDH_UNSUPPORTED, "embd % 64 == 0 needed");
  if ((rows + 255) / 256 * ((vocab + 127) / 128) > ((int64_t)1 << 31) - 1)
    return fail(BDH_UNSUPPORTED, "too large for one launch");
  bdh_status st = lm_logits(hidden, rows, embd, (const bf16_t*)lm_head_packed, vocab, logits,
                            (hipStream_t)stream);
  if (st != BDH_OK) return st;
  prof.launches = 2;
  prof.done(true);
  return BDH_OK;
}

void bdh_profile_enable(int32_t enabled) { g_prof_on = enabled != 0; }

void bdh_profile_reset(void) {
  std::lock_guard<std::mutex> lock(g_prof_mu);
  g_prof = bdh_profile_snapshot{};
}

void bdh_profile_get(bdh_profile_snapshot* out) {
  if (!out) return;
  std::lock_guard<std::mutex> lock(g_prof_mu);
  *out = g_prof;
}

bdh_status bdh_profile_kernel_timing(int32_t enabled) {
  std::lock_guard<std::mutex> lock(g_kt_mu);
  for (auto& r : g_kt_recs) BDH_HIP_TRY(hipEventSynchronize(r.stop));
  kt_clear();
  g_kt_on = enabled != 0;
  return BDH_OK;
}

bdh_status bdh_profile_kernel_get(int32_t kind, double* total_ms, int64_t* launches) {
  if (!total_ms || !launches) return fail(BDH_EINVAL, "null output pointer");
  std::lock_guard<std::mutex> lock(g_kt_mu);
  double sum = 0.0;
  int64_t n = 0;
  for (auto& r : g_kt_recs) {
    if (r.kind != kind) continue;
    BDH_HIP_TRY(hipEventSynchronize(r.stop));
    float ms = 0.0f;
    BDH_HIP_TRY(hipEventElapsedTime(&ms, r.start, r.stop));
    sum += ms;
    ++n;
  }
  *total_ms = sum;
  *launches = n;
  return BDH_OK;
}

const char* bdh_last_error(void) { return g_last_error.c_str(); }

const char* bdh_version(void) { return "bdh_hip 0.1.0 (gfx950)"; }

}  // extern "C"
