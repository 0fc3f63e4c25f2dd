// Streaming-state record of the recurrent attention: the model position and
// each layer's carried rho with its sequence-state flags, saved from and
// loaded into device memory.  This path's counterpart of the reference's
// StreamingRuntimeStateRecord / LayerRuntimeStateRecord
// (crates/burn_dragon_language/src/train/runtime_checkpoint.rs:16-112) and
// of LayerState / ModelState (crates/burn_dragon_core/src/model/state.rs:7-30):
// the fields this path carries (rho, persist_sequence_state,
// retain_terminal_sequence_state, position); the state of other model
// variants (rho_norm, mamba, slow and y-neuron states) is recorded as absent.
//
// File layout (little endian):
//   "BDHRHO01"                                   8 bytes
//   u32 version (1), u32 n_layers, i64 position  16 bytes
//   n_layers x 64-byte layer entries:
//     i64 batch, heads, latent, embd             (all 0: the layer has no rho)
//     i32 persist_sequence_state, retain_terminal_sequence_state
//     u64 data offset (from the file start, a multiple of 4096)
//     u64 data bytes (batch * heads * latent * embd * 4)
//     u32 CRC32C of the data, u32 reserved (0)
//   the rho blocks, f32 row-major [batch, heads, latent, embd], zero padded
//   to 4096-byte offsets.
// Copies go through two pinned staging buffers, so the device-to-host copy
// of one chunk overlaps the file write and checksum of the previous one (and
// the reverse on load).
#include <nmmintrin.h>
#include <stdio.h>
#include <string.h>

#include <string>
#include <vector>

#include "bdh_internal.h"

namespace bdh {
namespace {

constexpr char kMagic[8] = {'B', 'D', 'H', 'R', 'H', 'O', '0', '1'};
constexpr uint32_t kVersion = 1;
constexpr size_t kHeader = 24;
constexpr size_t kEntry = 64;
constexpr size_t kAlign = 4096;
constexpr size_t kChunk = (size_t)32 << 20;

struct Entry {
  int64_t b, h, n, d;
  int32_t persist, retain;
  uint64_t offset, bytes;
  uint32_t crc, reserved;
};
static_assert(sizeof(Entry) == kEntry, "layer entry is 64 bytes");

// CRC-32C (Castagnoli) register update with the SSE4.2 instruction.  The
// standard checksum starts the register at ~0 and inverts it at the end
// (crc32c_final), so that "123456789" gives 0xE3069283.
constexpr uint32_t kCrcInit = 0xFFFFFFFFu;
uint32_t crc32c_final(uint32_t reg) { return reg ^ 0xFFFFFFFFu; }
__attribute__((target("sse4.2"))) uint32_t crc32c_update(uint32_t crc, const unsigned char* p, size_t n) {
  uint64_t c = crc;
  while (n >= 8) {
    uint64_t w;
    memcpy(&w, p, 8);
    c = _mm_crc32_u64(c, w);
    p += 8;
    n -= 8;
  }
  uint32_t c32 = (uint32_t)c;
  while (n--) c32 = _mm_crc32_u8(c32, *p++);
  return c32;
}

struct File {
  FILE* f = nullptr;
  ~File() {
    if (f) fclose(f);
  }
};

struct Pinned {
  void* p[2] = {nullptr, nullptr};
  hipEvent_t ev[2] = {nullptr, nullptr};
  ~Pinned() {
    for (int i = 0; i < 2; ++i) {
      if (ev[i]) (void)hipEventDestroy(ev[i]);
      if (p[i]) (void)hipHostFree(p[i]);
    }
  }
  bdh_status init() {
    for (int i = 0; i < 2; ++i) {
      BDH_HIP_TRY(hipHostMalloc(&p[i], kChunk, hipHostMallocDefault));
      BDH_HIP_TRY(hipEventCreateWithFlags(&ev[i], hipEventDisableTiming));
    }
    return BDH_OK;
  }
};

size_t align_up(size_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

bdh_status check_desc(const bdh_layer_state_desc& d) {
  const bool none = d.batch == 0 && d.heads == 0 && d.latent == 0 && d.embd == 0;
  if (!none && (d.batch <= 0 || d.heads <= 0 || d.latent <= 0 || d.embd <= 0))
    return fail(BDH_EINVAL, "a layer's rho dims must all be > 0, or all 0 (no rho)");
  return BDH_OK;
}

uint64_t desc_bytes(const bdh_layer_state_desc& d) {
  return (uint64_t)d.batch * (uint64_t)d.heads * (uint64_t)d.latent * (uint64_t)d.embd * 4u;
}

bdh_status read_header(FILE* f, int64_t* position, std::vector<Entry>* entries) {
  char magic[8];
  uint32_t version = 0, n = 0;
  int64_t pos = 0;
  if (fread(magic, 1, 8, f) != 8 || memcmp(magic, kMagic, 8) != 0)
    return fail(BDH_EINVAL, "not a bdh state record (bad magic)");
  if (fread(&version, 4, 1, f) != 1 || fread(&n, 4, 1, f) != 1 || fread(&pos, 8, 1, f) != 1)
    return fail(BDH_EINVAL, "truncated state record header");
  if (version != kVersion) return fail(BDH_EINVAL, "unsupported state record version");
  if (n > (1u << 20)) return fail(BDH_EINVAL, "implausible layer count in state record");
  entries->resize(n);
  if (n && fread(entries->data(), kEntry, n, f) != n) return fail(BDH_EINVAL, "truncated layer table");
  *position = pos;
  return BDH_OK;
}

}  // namespace
}  // namespace bdh

using namespace bdh;

extern "C" {

bdh_status bdh_state_record_save(const char* path, int64_t position, int32_t n_layers,
                                 const bdh_layer_state_desc* layers, const float* const* rho,
                                 void* stream) {
  if (!path || n_layers < 0 || (n_layers > 0 && (!layers || !rho)))
    return fail(BDH_EINVAL, "null path or layer arrays");
  hipStream_t st = (hipStream_t)stream;
  std::vector<Entry> ent((size_t)n_layers);
  size_t off = align_up(kHeader + kEntry * (size_t)n_layers);
  for (int32_t i = 0; i < n_layers; ++i) {
    bdh_status s = check_desc(layers[i]);
    if (s != BDH_OK) return s;
    Entry& e = ent[i];
    memset(&e, 0, sizeof(e));
    e.b = layers[i].batch;
    e.h = layers[i].heads;
    e.n = layers[i].latent;
    e.d = layers[i].embd;
    e.persist = layers[i].persist_sequence_state;
    e.retain = layers[i].retain_terminal_sequence_state;
    e.bytes = desc_bytes(layers[i]);
    if (e.bytes && !rho[i]) return fail(BDH_EINVAL, "a layer with rho dims has a null rho pointer");
    e.offset = e.bytes ? off : 0;
    off = align_up(off + e.bytes);
  }
  File file;
  file.f = fopen(path, "wb");
  if (!file.f) return fail(BDH_EINVAL, std::string("cannot open ") + path + " for writing");
  Pinned pin;
  bdh_status s = pin.init();
  if (s != BDH_OK) return s;
  // Blocks first (their checksums fill the table), the header last.
  for (int32_t i = 0; i < n_layers; ++i) {
    Entry& e = ent[i];
    if (!e.bytes) continue;
    if (fseek(file.f, (long)e.offset, SEEK_SET) != 0) return fail(BDH_EINVAL, "seek failed");
    const char* src = (const char*)rho[i];
    uint32_t crc = kCrcInit;
    const size_t nchunks = (size_t)((e.bytes + kChunk - 1) / kChunk);
    auto issue = [&](size_t c) -> bdh_status {
      const size_t lo = c * kChunk, len = (size_t)e.bytes - lo < kChunk ? (size_t)e.bytes - lo : kChunk;
      BDH_HIP_TRY(hipMemcpyAsync(pin.p[c & 1], src + lo, len, hipMemcpyDeviceToHost, st));
      BDH_HIP_TRY(hipEventRecord(pin.ev[c & 1], st));
      return BDH_OK;
    };
    s = issue(0);
    if (s != BDH_OK) return s;
    for (size_t c = 0; c < nchunks; ++c) {
      if (c + 1 < nchunks) {
        s = issue(c + 1);
        if (s != BDH_OK) return s;
      }
      BDH_HIP_TRY(hipEventSynchronize(pin.ev[c & 1]));
      const size_t lo = c * kChunk, len = (size_t)e.bytes - lo < kChunk ? (size_t)e.bytes - lo : kChunk;
      crc = crc32c_update(crc, (const unsigned char*)pin.p[c & 1], len);
      if (fwrite(pin.p[c & 1], 1, len, file.f) != len) return fail(BDH_EINVAL, "write failed");
    }
    e.crc = crc32c_final(crc);
  }
  // Zero padding up to the end of the last block keeps every offset valid.
  if (fseek(file.f, 0, SEEK_SET) != 0) return fail(BDH_EINVAL, "seek failed");
  const uint32_t ver = kVersion, nl = (uint32_t)n_layers;
  if (fwrite(kMagic, 1, 8, file.f) != 8 || fwrite(&ver, 4, 1, file.f) != 1 ||
      fwrite(&nl, 4, 1, file.f) != 1 || fwrite(&position, 8, 1, file.f) != 1 ||
      (n_layers && fwrite(ent.data(), kEntry, (size_t)n_layers, file.f) != (size_t)n_layers))
    return fail(BDH_EINVAL, "write failed");
  if (fclose(file.f) != 0) {
    file.f = nullptr;
    return fail(BDH_EINVAL, "close failed");
  }
  file.f = nullptr;
  return BDH_OK;
}

bdh_status bdh_state_record_info(const char* path, int64_t* position, int32_t* n_layers,
                                 bdh_layer_state_desc* layers, int32_t max_layers) {
  if (!path || !position || !n_layers) return fail(BDH_EINVAL, "null argument");
  File file;
  file.f = fopen(path, "rb");
  if (!file.f) return fail(BDH_EINVAL, std::string("cannot open ") + path);
  std::vector<Entry> ent;
  bdh_status s = read_header(file.f, position, &ent);
  if (s != BDH_OK) return s;
  *n_layers = (int32_t)ent.size();
  if (layers) {
    if (max_layers < (int32_t)ent.size()) return fail(BDH_EINVAL, "layers array too short");
    for (size_t i = 0; i < ent.size(); ++i) {
      layers[i].batch = ent[i].b;
      layers[i].heads = ent[i].h;
      layers[i].latent = ent[i].n;
      layers[i].embd = ent[i].d;
      layers[i].persist_sequence_state = ent[i].persist;
      layers[i].retain_terminal_sequence_state = ent[i].retain;
    }
  }
  return BDH_OK;
}

bdh_status bdh_state_record_load(const char* path, int32_t n_layers, const bdh_layer_state_desc* layers,
                                 float* const* rho, void* stream) {
  if (!path || n_layers < 0 || (n_layers > 0 && (!layers || !rho)))
    return fail(BDH_EINVAL, "null path or layer arrays");
  hipStream_t st = (hipStream_t)stream;
  File file;
  file.f = fopen(path, "rb");
  if (!file.f) return fail(BDH_EINVAL, std::string("cannot open ") + path);
  int64_t position = 0;
  std::vector<Entry> ent;
  bdh_status s = read_header(file.f, &position, &ent);
  if (s != BDH_OK) return s;
  if ((int32_t)ent.size() != n_layers) return fail(BDH_EINVAL, "layer count differs from the record");
  for (int32_t i = 0; i < n_layers; ++i) {
    const Entry& e = ent[i];
    if (e.b != layers[i].batch || e.h != layers[i].heads || e.n != layers[i].latent || e.d != layers[i].embd)
      return fail(BDH_EINVAL, "layer " + std::to_string(i) + ": rho shape differs from the record");
    if (e.bytes != desc_bytes(layers[i])) return fail(BDH_EINVAL, "corrupt layer entry");
    if (e.bytes && !rho[i]) return fail(BDH_EINVAL, "a layer with rho dims has a null rho pointer");
  }
  Pinned pin;
  s = pin.init();
  if (s != BDH_OK) return s;
  // First pass, host only: every layer's block is read and its checksum
  // checked before any device memory is written, so a corrupt or truncated
  // record leaves the caller's state as it was (as a failed restore of the
  // reference leaves the model untouched, runtime_checkpoint.rs:163-200).
  for (int32_t i = 0; i < n_layers; ++i) {
    const Entry& e = ent[i];
    if (!e.bytes) continue;
    if (fseek(file.f, (long)e.offset, SEEK_SET) != 0) return fail(BDH_EINVAL, "seek failed");
    uint32_t crc = kCrcInit;
    for (int64_t lo = 0; lo < e.bytes; lo += (int64_t)kChunk) {
      const size_t len = (size_t)(e.bytes - lo) < kChunk ? (size_t)(e.bytes - lo) : kChunk;
      if (fread(pin.p[0], 1, len, file.f) != len) return fail(BDH_EINVAL, "truncated rho block");
      crc = crc32c_update(crc, (const unsigned char*)pin.p[0], len);
    }
    if (crc32c_final(crc) != e.crc)
      return fail(BDH_EINVAL, "layer " + std::to_string(i) + ": rho checksum mismatch (corrupt record)");
  }
  // Second pass: the copies, checked again (a file changed between the two
  // passes is still reported, but then after its copy).
  for (int32_t i = 0; i < n_layers; ++i) {
    const Entry& e = ent[i];
    if (!e.bytes) continue;
    if (fseek(file.f, (long)e.offset, SEEK_SET) != 0) return fail(BDH_EINVAL, "seek failed");
    char* dst = (char*)rho[i];
    uint32_t crc = kCrcInit;
    const size_t nchunks = (size_t)((e.bytes + kChunk - 1) / kChunk);
    for (size_t c = 0; c < nchunks; ++c) {
      const size_t lo = c * kChunk, len = (size_t)e.bytes - lo < kChunk ? (size_t)e.bytes - lo : kChunk;
      // The staging buffer is free once the copy issued from it two chunks
      // ago has completed.
      if (c >= 2) BDH_HIP_TRY(hipEventSynchronize(pin.ev[c & 1]));
      if (fread(pin.p[c & 1], 1, len, file.f) != len) return fail(BDH_EINVAL, "truncated rho block");
      crc = crc32c_update(crc, (const unsigned char*)pin.p[c & 1], len);
      BDH_HIP_TRY(hipMemcpyAsync(dst + lo, pin.p[c & 1], len, hipMemcpyHostToDevice, st));
      BDH_HIP_TRY(hipEventRecord(pin.ev[c & 1], st));
    }
    BDH_HIP_TRY(hipStreamSynchronize(st));
    if (crc32c_final(crc) != e.crc)
      return fail(BDH_EINVAL, "layer " + std::to_string(i) +
                                  ": rho checksum mismatch (the record changed during the load)");
  }
  return BDH_OK;
}

}  // extern "C"
