// rf_runtime.hip — context, device-memory ledger and the op entry points of
// the C ABI (include/ramforge_hip.h).  Host code; kernels live in the other
// translation units.
#include "rf_runtime.h"

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <functional>
#include <thread>
#include <vector>

#include <cerrno>
#include <fcntl.h>
#include <unistd.h>

namespace rf {

static thread_local std::string g_err;

int32_t set_error(int32_t code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

thread_local bool g_plan_only = false;

hipError_t setup_outside_capture(hipStream_t st) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (st && hipStreamIsCapturing(st, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
    return hipErrorStreamCaptureUnsupported;
  return hipSuccess;
}

int32_t hip_error(hipError_t e, const char* what) {
  if (e == hipErrorStreamCaptureUnsupported)
    return set_error(RF_ERR_INVALID,
                     "%s: first launch of this kernel shape inside a stream capture; its one-time setup (dynamic "
                     "LDS, occupancy) runs outside captures only: launch the same shape once before capturing",
                     what);
  return set_error(RF_ERR_HIP, "%s failed: %s (%d)", what, hipGetErrorString(e), (int)e);
}

const char* type_name(uint32_t t) {
  switch (t) {
    case T_F32: return "F32"; case T_F16: return "F16"; case T_BF16: return "BF16";
    case T_Q4_0: return "Q4_0"; case T_Q5_0: return "Q5_0"; case T_Q8_0: return "Q8_0";
    case T_Q2_K: return "Q2_K"; case T_Q3_K: return "Q3_K"; case T_Q4_K: return "Q4_K";
    case T_Q5_K: return "Q5_K"; case T_Q6_K: return "Q6_K"; case T_Q8_K: return "Q8_K";
    default: return "unknown";
  }
}

// ------------------------------------------------------------------ Ledger
// Messages follow MemoryError (core/src/error.rs:62-90).
int32_t Ledger::allocate(const std::string& name, uint64_t bytes) {
  if (bytes == 0) return set_error(RF_ERR_BUDGET, "invalid allocation size: 0 (must be > 0)");
  if (allocs_.count(name)) return set_error(RF_ERR_BUDGET, "allocation '%s' already exists", name.c_str());
  const uint64_t avail = total_ - used_;
  if (bytes > avail)
    return set_error(RF_ERR_BUDGET,
                     "insufficient memory: requested %llu bytes for '%s', but only %llu bytes available (total %llu, used %llu)",
                     (unsigned long long)bytes, name.c_str(), (unsigned long long)avail, (unsigned long long)total_,
                     (unsigned long long)used_);
  allocs_[name] = bytes;
  used_ += bytes;
  if (used_ > peak_) peak_ = used_;
  return RF_OK;
}

int32_t Ledger::release(const std::string& name, uint64_t* released) {
  auto it = allocs_.find(name);
  if (it == allocs_.end()) return set_error(RF_ERR_BUDGET, "allocation '%s' not found", name.c_str());
  if (it->second > used_)
    return set_error(RF_ERR_BUDGET, "memory accounting underflow while releasing %llu bytes for '%s' (used %llu)",
                     (unsigned long long)it->second, name.c_str(), (unsigned long long)used_);
  used_ -= it->second;
  if (released) *released = it->second;
  allocs_.erase(it);
  return RF_OK;
}

int32_t Ledger::resize(const std::string& name, uint64_t bytes) {
  if (bytes == 0) return set_error(RF_ERR_BUDGET, "invalid allocation size: 0 (must be > 0)");
  auto it = allocs_.find(name);
  if (it == allocs_.end()) return set_error(RF_ERR_BUDGET, "allocation '%s' not found", name.c_str());
  const uint64_t old = it->second;
  if (bytes > old) {
    const uint64_t add = bytes - old, avail = total_ - used_;
    if (add > avail)
      return set_error(RF_ERR_BUDGET,
                       "insufficient memory: requested %llu bytes for '%s', but only %llu bytes available (total %llu, used %llu)",
                       (unsigned long long)add, name.c_str(), (unsigned long long)avail,
                       (unsigned long long)total_, (unsigned long long)used_);
    used_ += add;
  } else {
    used_ -= old - bytes;
  }
  it->second = bytes;
  if (used_ > peak_) peak_ = used_;
  return RF_OK;
}

// Keys that start with a prefix form one contiguous range of an ordered map,
// from lower_bound(prefix) on; renames walk that range only and re-key the
// nodes in place (the streaming tier renames a layer's charges twice a step).
template <class M>
static void prefix_keys(const M& m, const std::string& op, std::vector<std::string>* out) {
  for (auto it = m.lower_bound(op); it != m.end() && it->first.compare(0, op.size(), op) == 0; ++it)
    out->push_back(it->first);
}
template <class M>
static void rekey(M& m, const std::vector<std::string>& keys, const std::string& op, const std::string& np) {
  for (const std::string& k : keys) {
    auto nh = m.extract(k);
    nh.key() = np + k.substr(op.size());
    m.insert(std::move(nh));
  }
}

int32_t Ledger::rename_prefix(const std::string& op, const std::string& np) {
  std::vector<std::string> keys;
  prefix_keys(allocs_, op, &keys);
  if (keys.empty()) return set_error(RF_ERR_BUDGET, "allocation '%s' not found", op.c_str());
  for (const std::string& k : keys) {
    const std::string n = np + k.substr(op.size());
    if (allocs_.count(n)) return set_error(RF_ERR_BUDGET, "allocation '%s' already exists", n.c_str());
  }
  rekey(allocs_, keys, op, np);
  return RF_OK;
}

bool Ledger::get(const std::string& name, uint64_t* bytes) const {
  auto it = allocs_.find(name);
  if (it == allocs_.end()) return false;
  if (bytes) *bytes = it->second;
  return true;
}

// ------------------------------------------------------------ buffers
int32_t vram_alloc(rf_ctx* ctx, const std::string& charge, uint64_t bytes, void** out) {
  std::lock_guard<std::mutex> lk(ctx->mu);
  int32_t rc = ctx->ledger.allocate(charge, bytes);
  if (rc) return rc;
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, bytes);
  if (e != hipSuccess) {
    ctx->ledger.release(charge);  // roll back the reservation
    return hip_error(e, "hipMalloc");
  }
  ctx->buffers[charge] = p;
  *out = p;
  return RF_OK;
}

int32_t vram_release(rf_ctx* ctx, const std::string& charge) {
  std::lock_guard<std::mutex> lk(ctx->mu);
  auto it = ctx->buffers.find(charge);
  if (it == ctx->buffers.end()) return set_error(RF_ERR_BUDGET, "allocation '%s' not found", charge.c_str());
  hipError_t e = hipFree(it->second);  // physical free first (memory.rs:9-15)
  ctx->buffers.erase(it);
  const int32_t rc = ctx->ledger.release(charge);
  if (e != hipSuccess) return hip_error(e, "hipFree");
  return rc;
}

int32_t vram_rename_prefix(rf_ctx* ctx, const std::string& o, const std::string& n) {
  std::lock_guard<std::mutex> lk(ctx->mu);
  int32_t rc = ctx->ledger.rename_prefix(o, n);
  if (rc) return rc;
  std::vector<std::string> keys;
  prefix_keys(ctx->buffers, o, &keys);
  rekey(ctx->buffers, keys, o, n);
  return RF_OK;
}

bool vram_can_allocate(rf_ctx* ctx, uint64_t bytes) {
  std::lock_guard<std::mutex> lk(ctx->mu);
  return ctx->ledger.used() + bytes >= ctx->ledger.used() && ctx->ledger.used() + bytes <= ctx->ledger.total();
}

int32_t ensure_workspace(rf_ctx* ctx, Workspace& ws, const char* charge, uint64_t bytes, hipStream_t st) {
  if (ws.bytes >= bytes) return RF_OK;
  if (ctx->ws_fixed)
    return set_error(RF_ERR_INVALID, "%s needs %llu bytes but %llu are reserved and the workspaces are fixed", charge,
                     (unsigned long long)bytes, (unsigned long long)ws.bytes);
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (st && hipStreamIsCapturing(st, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
    return set_error(RF_ERR_INVALID,
                     "%s needs %llu bytes during graph capture; reserve it first (rf_ctx_reserve) or run the call "
                     "once before capturing",
                     charge, (unsigned long long)bytes);
  uint64_t want = bytes < 65536 ? 65536 : bytes;
  if (ws.ptr) {
    hipError_t e = hipDeviceSynchronize();  // the old buffer may still be read by queued kernels
    if (e != hipSuccess) return hip_error(e, "hipDeviceSynchronize");
    int32_t rc = vram_release(ctx, charge);
    ws.ptr = nullptr;
    ws.bytes = 0;
    ++ctx->ws_generation;  // graphs holding the old address are stale from here on
    if (rc) return rc;
  }
  void* p = nullptr;
  int32_t rc = vram_alloc(ctx, charge, want, &p);
  if (rc) return rc;
  ws.ptr = p;
  ws.bytes = want;
  return RF_OK;
}

// The no-allocation variant's scratch: one array per device, held until the
// process ends.  Host code never passes `scratch` itself to a kernel: its
// device address on the current device comes from hipGetSymbolAddress
// (resolved once per device in rf_ctx_create and kept in rf_ctx).
constexpr uint64_t NOALLOC_SCRATCH_BYTES = RF_ATTENTION_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[NOALLOC_SCRATCH_BYTES];
constexpr int MAX_DEVICES = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[MAX_DEVICES] = {};

// Called with `device` current.
int32_t resolve_scratch(int device, void** out) {
  if (device < 0 || device >= MAX_DEVICES)
    return set_error(RF_ERR_UNSUPPORTED, "HIP device %d beyond the %d the library tracks", device, MAX_DEVICES);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[device]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_error(e, "hipGetSymbolAddress(scratch)");
    if (!p) return set_error(RF_ERR_HIP, "hipGetSymbolAddress(scratch) returned a null address");
    g_scratch_ptr[device] = p;
  }
  *out = g_scratch_ptr[device];
  return RF_OK;
}

int32_t staged_upload(rf_ctx* ctx, void* dst, const void* src, uint64_t bytes) {
  constexpr uint64_t kStage = 64ull << 20;
  // one upload at a time: the two pinned buffers are the context's
  std::lock_guard<std::mutex> lk(ctx->stage_mu);
  if (!ctx->stage_bytes) {
    // all four objects or none: a later call never finds half a set
    void* pb[2] = {nullptr, nullptr};
    hipEvent_t ev[2] = {nullptr, nullptr};
    hipError_t e = hipSuccess;
    for (int i = 0; i < 2 && e == hipSuccess; ++i) {
      e = hipHostMalloc(&pb[i], kStage, hipHostMallocDefault);
      if (e == hipSuccess) e = hipEventCreateWithFlags(&ev[i], hipEventDisableTiming);
    }
    if (e != hipSuccess) {
      for (int i = 0; i < 2; ++i) {
        if (pb[i]) hipHostFree(pb[i]);
        if (ev[i]) hipEventDestroy(ev[i]);
      }
      return hip_error(e, "pinned staging setup");
    }
    for (int i = 0; i < 2; ++i) {
      ctx->pinned_stage[i] = pb[i];
      ctx->stage_ev[i] = ev[i];
    }
    ctx->stage_bytes = kStage;
  }
  const uint8_t* s = static_cast<const uint8_t*>(src);
  uint8_t* d = static_cast<uint8_t*>(dst);
  int buf = 0;
  bool used[2] = {false, false};
  hipError_t e = hipSuccess;
  const char* what = "";
  for (uint64_t off = 0; off < bytes && e == hipSuccess; off += kStage) {
    const uint64_t n = bytes - off < kStage ? bytes - off : kStage;
    if (used[buf]) {
      e = hipEventSynchronize(ctx->stage_ev[buf]);
      what = "hipEventSynchronize";
      if (e != hipSuccess) break;
    }
    std::memcpy(ctx->pinned_stage[buf], s + off, n);
    e = hipMemcpyAsync(d + off, ctx->pinned_stage[buf], n, hipMemcpyHostToDevice, ctx->copy);
    what = "hipMemcpyAsync";
    if (e == hipSuccess) {
      e = hipEventRecord(ctx->stage_ev[buf], ctx->copy);
      what = "hipEventRecord";
    }
    used[buf] = true;
    buf ^= 1;
  }
  // also on failure: no copy may still read a staging buffer when the next
  // upload refills it
  const hipError_t es = hipStreamSynchronize(ctx->copy);
  if (e != hipSuccess) return hip_error(e, what);
  if (es != hipSuccess) return hip_error(es, "hipStreamSynchronize");
  return RF_OK;
}

// RoPE angle table with the reference's expression: angle =
// theta.powf(-2.0 * i / hd) * pos in f32, then cos / sin (compute.rs:446-456).
void rope_table_host(float* out, uint64_t p0, uint64_t np, uint32_t hd, float theta) {
  const uint32_t half = hd / 2;
  for (uint64_t p = 0; p < np; ++p) {
    const float pos = (float)(p0 + p);
    for (uint32_t i = 0; i < half; ++i) {
      const float angle = powf(theta, -2.0f * (float)i / (float)hd) * pos;
      out[(p * half + i) * 2] = cosf(angle);
      out[(p * half + i) * 2 + 1] = sinf(angle);
    }
  }
}

}  // namespace rf

using namespace rf;

#define RF_CHECK_CTX(ctx) \
  if (!(ctx)) return set_error(RF_ERR_INVALID, "null context")
#define RF_HIP(call, what)                          \
  do {                                              \
    hipError_t _e = (call);                         \
    if (_e != hipSuccess) return hip_error(_e, what); \
  } while (0)

extern "C" {

size_t rf_last_error(char* buf, size_t cap) {
  if (buf && cap) {
    const size_t n = g_err.size() < cap - 1 ? g_err.size() : cap - 1;
    std::memcpy(buf, g_err.data(), n);
    buf[n] = 0;
  }
  return g_err.size();
}

const char* rf_version(void) { return "ramforge_hip 0.1.0 (gfx950)"; }

int32_t rf_ctx_create(int32_t device, uint64_t budget, rf_ctx** out) {
  if (!out) return set_error(RF_ERR_INVALID, "null output pointer");
  int n = 0;
  RF_HIP(hipGetDeviceCount(&n), "hipGetDeviceCount");
  if (device < 0 || device >= n) return set_error(RF_ERR_INVALID, "HIP device %d out of range (%d devices)", device, n);
  RF_HIP(hipSetDevice(device), "hipSetDevice");
  size_t free_b = 0, total_b = 0;
  RF_HIP(hipMemGetInfo(&free_b, &total_b), "hipMemGetInfo");
  rf_ctx* c = new rf_ctx();
  c->device = device;
  c->ledger = Ledger(budget ? budget : (uint64_t)total_b);
  hipError_t e = hipStreamCreateWithFlags(&c->compute, hipStreamNonBlocking);
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&c->copy, hipStreamNonBlocking);
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&c->copy2, hipStreamNonBlocking);
  if (e != hipSuccess) {
    const int32_t rc = hip_error(e, "hipStreamCreate");
    rf_ctx_destroy(c);  // the stream that was created, if any
    return rc;
  }
  // this device's address of the no-allocation scratch array (device current)
  int32_t rc = resolve_scratch(device, &c->noalloc_scratch);
  if (rc) {
    rf_ctx_destroy(c);
    return rc;
  }
  // Load every kernel file's code object now.  HIP loads one on the first use
  // of any of its kernels, and a decode step's first use can be inside a
  // stream capture (rf_model_decode_steps, rf_capture_begin), where the
  // load's own device allocation and copies are not capturable work.
  for (hipError_t (*load)() : {load_module_attention, load_module_elementwise, load_module_matvec,
                               load_module_packed, load_module_prefill}) {
    e = load();
    if (e != hipSuccess) {
      rc = hip_error(e, "loading the kernel code objects");
      rf_ctx_destroy(c);
      return rc;
    }
  }
  void* p = nullptr;
  rc = vram_alloc(c, "workspace:argmax", 256 * 8 + 64, &p);
  if (rc) {
    rf_ctx_destroy(c);
    return rc;
  }
  c->amax_val = static_cast<float*>(p);
  c->amax_idx = reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(p) + 256 * 4);
  *out = c;
  return RF_OK;
}

void rf_ctx_destroy(rf_ctx* ctx) {
  if (!ctx) return;
  hipSetDevice(ctx->device);
  hipDeviceSynchronize();
  for (auto& kv : ctx->buffers) hipFree(kv.second);  // includes the repack cache's buffers
  ctx->buffers.clear();
  for (auto& en : ctx->repack.entries)
    if (en.ready) hipEventDestroy(en.ready);
  for (int i = 0; i < 2; ++i) {
    if (ctx->pinned_stage[i]) hipHostFree(ctx->pinned_stage[i]);
    if (ctx->stage_ev[i]) hipEventDestroy(ctx->stage_ev[i]);
  }
  if (ctx->compute) hipStreamDestroy(ctx->compute);
  if (ctx->copy) hipStreamDestroy(ctx->copy);
  if (ctx->copy2) hipStreamDestroy(ctx->copy2);
  delete ctx;
}

int32_t rf_ctx_reserve(rf_ctx* ctx, uint64_t attention_bytes, uint64_t matmul_bytes, uint64_t staging_bytes,
                       int32_t fixed) {
  RF_CHECK_CTX(ctx);
  ctx->ws_fixed = false;  // growing is what reserving does
  int32_t rc = RF_OK;
  if (attention_bytes) rc = ensure_workspace(ctx, ctx->attn_ws, "workspace:attention", attention_bytes, ctx->compute);
  if (!rc && matmul_bytes) rc = ensure_workspace(ctx, ctx->mm_ws, "workspace:matmul", matmul_bytes, ctx->compute);
  if (!rc && staging_bytes) rc = ensure_workspace(ctx, ctx->scratch_ws, "workspace:scratch", staging_bytes, ctx->compute);
  if (!rc) ctx->ws_fixed = fixed != 0;
  return rc;
}

int32_t rf_ctx_synchronize(rf_ctx* ctx) {
  RF_CHECK_CTX(ctx);
  RF_HIP(hipStreamSynchronize(ctx->compute), "hipStreamSynchronize");
  RF_HIP(hipStreamSynchronize(ctx->copy), "hipStreamSynchronize");
  RF_HIP(hipStreamSynchronize(ctx->copy2), "hipStreamSynchronize");
  return RF_OK;
}

rf_stream_t rf_ctx_compute_stream(rf_ctx* ctx) { return ctx ? ctx->compute : nullptr; }
rf_stream_t rf_ctx_copy_stream(rf_ctx* ctx) { return ctx ? ctx->copy : nullptr; }

int32_t rf_ctx_device_info(rf_ctx* ctx, char* name, size_t cap, int32_t* cus) {
  RF_CHECK_CTX(ctx);
  hipDeviceProp_t prop;
  RF_HIP(hipGetDeviceProperties(&prop, ctx->device), "hipGetDeviceProperties");
  if (name && cap) {
    snprintf(name, cap, "%s (%s)", prop.name, prop.gcnArchName);
  }
  if (cus) *cus = prop.multiProcessorCount;
  return RF_OK;
}

int32_t rf_vram_alloc(rf_ctx* ctx, const char* charge, uint64_t bytes, void** out) {
  RF_CHECK_CTX(ctx);
  if (!charge || !out) return set_error(RF_ERR_INVALID, "null charge name or output pointer");
  return vram_alloc(ctx, charge, bytes, out);
}

int32_t rf_vram_release(rf_ctx* ctx, const char* charge) {
  RF_CHECK_CTX(ctx);
  if (!charge) return set_error(RF_ERR_INVALID, "null charge name");
  return vram_release(ctx, charge);
}

int32_t rf_vram_rename_prefix(rf_ctx* ctx, const char* op, const char* np) {
  RF_CHECK_CTX(ctx);
  if (!op || !np) return set_error(RF_ERR_INVALID, "null prefix");
  return vram_rename_prefix(ctx, op, np);
}

int32_t rf_vram_charge(rf_ctx* ctx, const char* charge, uint64_t* bytes) {
  RF_CHECK_CTX(ctx);
  std::lock_guard<std::mutex> lk(ctx->mu);
  if (!charge || !ctx->ledger.get(charge, bytes))
    return set_error(RF_ERR_INVALID, "allocation '%s' not found", charge ? charge : "(null)");
  return RF_OK;
}

uint64_t rf_vram_used(rf_ctx* ctx) {
  if (!ctx) return 0;
  std::lock_guard<std::mutex> lk(ctx->mu);
  return ctx->ledger.used();
}
uint64_t rf_vram_total(rf_ctx* ctx) {
  if (!ctx) return 0;
  std::lock_guard<std::mutex> lk(ctx->mu);
  return ctx->ledger.total();
}
uint64_t rf_vram_peak(rf_ctx* ctx) {
  if (!ctx) return 0;
  std::lock_guard<std::mutex> lk(ctx->mu);
  return ctx->ledger.peak();
}

int32_t rf_pinned_alloc(rf_ctx* ctx, uint64_t bytes, void** out) {
  RF_CHECK_CTX(ctx);
  if (!out || bytes == 0) return set_error(RF_ERR_INVALID, "invalid pinned allocation");
  RF_HIP(hipHostMalloc(out, bytes, hipHostMallocDefault), "hipHostMalloc");
  return RF_OK;
}

int32_t rf_pinned_free(rf_ctx* ctx, void* p) {
  RF_CHECK_CTX(ctx);
  if (p) RF_HIP(hipHostFree(p), "hipHostFree");
  return RF_OK;
}

}  // extern "C"

struct rf_file_source {
  int fd = -1;
  uint32_t threads = 1;
};

extern "C" {

int32_t rf_file_source_open(const char* path, uint32_t threads, rf_file_source** out) {
  if (!path || !out) return set_error(RF_ERR_INVALID, "null argument to rf_file_source_open");
  *out = nullptr;
  const int fd = open(path, O_RDONLY | O_CLOEXEC);
  if (fd < 0) return set_error(RF_ERR_IO, "cannot open '%s': %s", path, strerror(errno));
  rf_file_source* f = new rf_file_source();
  f->fd = fd;
  f->threads = threads < 1 ? 1u : (threads > 64 ? 64u : threads);
  *out = f;
  return RF_OK;
}

void rf_file_source_close(rf_file_source* f) {
  if (!f) return;
  if (f->fd >= 0) close(f->fd);
  delete f;
}

int32_t rf_file_source_read(void* user, uint64_t offset, uint64_t length, void* dst) {
  rf_file_source* f = static_cast<rf_file_source*>(user);
  if (!f || f->fd < 0 || (length && !dst)) return EINVAL;
  auto piece = [f, dst, offset](uint64_t a, uint64_t b) -> int32_t {  // [a, b) of the request
    uint8_t* d = static_cast<uint8_t*>(dst);
    while (a < b) {
      const uint64_t want = std::min<uint64_t>(b - a, 1ull << 30);
      const ssize_t n = pread(f->fd, d + a, (size_t)want, (off_t)(offset + a));
      if (n < 0) {
        if (errno == EINTR) continue;
        return errno ? errno : EIO;
      }
      if (n == 0) return EIO;  // past the end of the file
      a += (uint64_t)n;
    }
    return 0;
  };
  constexpr uint64_t kPiece = 4ull << 20;
  uint64_t np = std::min<uint64_t>(f->threads, (length + kPiece - 1) / kPiece);
  if (np <= 1) return piece(0, length);
  const uint64_t per = (length + np - 1) / np;
  std::vector<int32_t> rc(np, 0);
  std::vector<std::thread> th;
  th.reserve(np - 1);
  for (uint64_t i = 1; i < np; ++i)
    th.emplace_back([&, i] { rc[i] = piece(i * per, std::min(length, (i + 1) * per)); });
  rc[0] = piece(0, std::min(length, per));
  for (std::thread& t : th) t.join();
  for (int32_t r : rc)
    if (r) return r;
  return 0;
}

int32_t rf_upload_async(rf_ctx* ctx, void* dst, const void* src, uint64_t bytes, rf_stream_t s) {
  RF_CHECK_CTX(ctx);
  if (bytes == 0) return RF_OK;
  if (!dst || !src) return set_error(RF_ERR_INVALID, "null copy pointer");
  RF_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, pick_stream(ctx, s)), "hipMemcpyAsync");
  return RF_OK;
}

int32_t rf_upload(rf_ctx* ctx, void* dst, const void* src, uint64_t bytes) {
  RF_CHECK_CTX(ctx);
  if (bytes == 0) return RF_OK;
  if (!dst || !src) return set_error(RF_ERR_INVALID, "null copy pointer");
  RF_HIP(hipStreamSynchronize(ctx->compute), "hipStreamSynchronize");
  RF_HIP(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice), "hipMemcpy");
  return RF_OK;
}

int32_t rf_download(rf_ctx* ctx, void* dst, const void* src, uint64_t bytes) {
  RF_CHECK_CTX(ctx);
  if (bytes == 0) return RF_OK;
  if (!dst || !src) return set_error(RF_ERR_INVALID, "null copy pointer");
  RF_HIP(hipStreamSynchronize(ctx->compute), "hipStreamSynchronize");
  RF_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost), "hipMemcpy");
  return RF_OK;
}

int32_t rf_memset(rf_ctx* ctx, void* dst, int32_t value, uint64_t bytes) {
  RF_CHECK_CTX(ctx);
  if (bytes == 0) return RF_OK;
  RF_HIP(hipMemsetAsync(dst, value, bytes, ctx->compute), "hipMemsetAsync");
  RF_HIP(hipStreamSynchronize(ctx->compute), "hipStreamSynchronize");
  return RF_OK;
}

int32_t rf_copy_async(rf_ctx* ctx, void* dst, const void* src, uint64_t bytes, rf_stream_t s) {
  RF_CHECK_CTX(ctx);
  if (bytes == 0) return RF_OK;
  if (!dst || !src) return set_error(RF_ERR_INVALID, "null copy pointer");
  RF_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, pick_stream(ctx, s)), "hipMemcpyAsync");
  return RF_OK;
}

int32_t rf_event_create(rf_ctx* ctx, void** ev) {
  RF_CHECK_CTX(ctx);
  if (!ev) return set_error(RF_ERR_INVALID, "null event output");
  hipEvent_t e;
  RF_HIP(hipEventCreate(&e), "hipEventCreate");
  *ev = e;
  return RF_OK;
}

int32_t rf_event_destroy(rf_ctx* ctx, void* ev) {
  RF_CHECK_CTX(ctx);
  if (ev) RF_HIP(hipEventDestroy(static_cast<hipEvent_t>(ev)), "hipEventDestroy");
  return RF_OK;
}

int32_t rf_event_record(rf_ctx* ctx, void* ev, rf_stream_t s) {
  RF_CHECK_CTX(ctx);
  RF_HIP(hipEventRecord(static_cast<hipEvent_t>(ev), pick_stream(ctx, s)), "hipEventRecord");
  return RF_OK;
}

int32_t rf_stream_wait_event(rf_ctx* ctx, rf_stream_t s, void* ev) {
  RF_CHECK_CTX(ctx);
  RF_HIP(hipStreamWaitEvent(pick_stream(ctx, s), static_cast<hipEvent_t>(ev), 0), "hipStreamWaitEvent");
  return RF_OK;
}

int32_t rf_event_elapsed_ms(rf_ctx* ctx, void* a, void* b, float* ms) {
  RF_CHECK_CTX(ctx);
  RF_HIP(hipEventElapsedTime(ms, static_cast<hipEvent_t>(a), static_cast<hipEvent_t>(b)), "hipEventElapsedTime");
  return RF_OK;
}

int32_t rf_event_synchronize(rf_ctx* ctx, void* ev) {
  RF_CHECK_CTX(ctx);
  RF_HIP(hipEventSynchronize(static_cast<hipEvent_t>(ev)), "hipEventSynchronize");
  return RF_OK;
}

// ------------------------------------------------------------------ matvec
// a * b into *r; false when the product does not fit in 64 bits (a size
// computed from caller shapes must not wrap past the bounds checks).
static bool mul_u64(uint64_t a, uint64_t b, uint64_t* r) { return !__builtin_mul_overflow(a, b, r); }

// Shared argument validation of the matvec entry points, in the reference's
// order and wording (quant.rs:907-975, backend.rs:173-199).  On success
// *count is the number of rows to compute and *rb the bytes per row; a zero
// count or in_dim has already been handled (*done = true).
static int32_t validate_matvec(rf_ctx* ctx, uint32_t t, const void* w, uint64_t w_bytes, uint64_t out_dim,
                               uint64_t in_dim, const float* x, float* y, uint64_t row_start, uint64_t row_count,
                               rf_stream_t s, uint64_t* count_out, uint64_t* rb_out, bool* done) {
  *done = false;
  uint64_t qk = 0, bs = 0;
  if (!type_geometry(t, &qk, &bs))
    return set_error(RF_ERR_UNSUPPORTED, "matvec does not support tensor type %s (%u)", type_name(t), t);
  const char* nm = type_name(t);
  if (!w || !x || !y) return set_error(RF_ERR_INVALID, "%s matvec received a null pointer", nm);
  if (in_dim % qk != 0)
    return set_error(RF_ERR_INVALID, "%s in_dim %llu not divisible by %llu", nm, (unsigned long long)in_dim,
                     (unsigned long long)qk);
  if (row_start > out_dim)
    return set_error(RF_ERR_INVALID, "%s row start %llu exceeds out_dim %llu", nm, (unsigned long long)row_start,
                     (unsigned long long)out_dim);
  const uint64_t count = row_count == RF_ALL_ROWS ? out_dim - row_start : row_count;
  if (row_start + count < row_start) return set_error(RF_ERR_INVALID, "%s row range overflow", nm);
  if (row_start + count > out_dim)
    return set_error(RF_ERR_INVALID, "%s row range %llu..%llu exceeds out_dim %llu", nm,
                     (unsigned long long)row_start, (unsigned long long)(row_start + count),
                     (unsigned long long)out_dim);
  const uint64_t rb = in_dim / qk * bs;
  uint64_t need = 0;
  if (!mul_u64(out_dim, rb, &need))
    return set_error(RF_ERR_INVALID, "%s weight size of %llu rows of %llu overflows 64 bits", nm,
                     (unsigned long long)out_dim, (unsigned long long)in_dim);
  if (w_bytes < need) {
    if (t == T_F32)
      return set_error(RF_ERR_INVALID,
                       "backend matvec arity mismatch (ggml layout [in, out]): shape [%llu, %llu] requires %llu weight bytes, got %llu",
                       (unsigned long long)in_dim, (unsigned long long)out_dim, (unsigned long long)need,
                       (unsigned long long)w_bytes);
    return set_error(RF_ERR_INVALID, "%s weight truncated: expected %llu bytes, got %llu", nm,
                     (unsigned long long)need, (unsigned long long)w_bytes);
  }
  *count_out = count;
  *rb_out = rb;
  if (count == 0) {
    *done = true;
    return RF_OK;
  }
  if (in_dim == 0) {
    *done = true;
    hipError_t e = launch_fill(y, 0.f, count, pick_stream(ctx, s));
    return e == hipSuccess ? RF_OK : hip_error(e, "fill");
  }
  if (count > 0xFFFFFFFFull || rb > 0xFFFFFFFFull)
    return set_error(RF_ERR_UNSUPPORTED, "%s matvec shape exceeds 32-bit row indexing", nm);
  return RF_OK;
}

// Rows [row_start, row_start + count) of a validated packed tensor into y.
static int32_t launch_packed_rows(rf_ctx* ctx, uint32_t t, const void* packed, uint64_t out_dim, uint64_t in_dim,
                                  const float* x, float* y, uint64_t row_start, uint64_t count, hipStream_t st) {
  const float* xa = x;
  if ((reinterpret_cast<uintptr_t>(x) & 15u) != 0) {
    // the kernel reads x with 16-byte loads: stage a misaligned x in the context scratch
    int32_t rc = ensure_workspace(ctx, ctx->scratch_ws, "workspace:scratch", in_dim * 4, st);
    if (rc) return rc;
    RF_HIP(hipMemcpyAsync(ctx->scratch_ws.ptr, x, in_dim * 4, hipMemcpyDeviceToDevice, st), "hipMemcpyAsync");
    xa = static_cast<const float*>(ctx->scratch_ws.ptr);
  }
  PkSegDesc seg{packed, nullptr, out_dim, row_start, count, y, nullptr};
  hipError_t e = launch_matvec_packed(t, &seg, 1, xa, nullptr, 0.f, in_dim, EPI_STORE, st);
  if (e != hipSuccess) return hip_error(e, "packed matvec launch");
  return RF_OK;
}

// ------------------------------------------------------ repack cache
// rf_matvec's opt-in cache of packed copies of the GGUF tensors it is handed.
// Callers of the reference's matvec seam pass the same immutable tensor bytes
// token after token (TensorData of a loaded model, compute_dispatch.rs:40-58);
// the first call packs them once, later calls run the packed kernel.

// Drop entries [i] for which drop(entry) holds.  Buffers may still be read by
// queued work on any stream, so the device is synchronised before any free.
static int32_t repack_drop(rf_ctx* ctx, const std::function<bool(const RepackEntry&)>& drop) {
  RepackCache& c = ctx->repack;
  bool any = false;
  for (auto& en : c.entries) any = any || drop(en);
  if (!any) return RF_OK;
  RF_HIP(hipDeviceSynchronize(), "hipDeviceSynchronize");
  ++c.generation;  // graphs that captured a hit on the cache are stale from here on
  int32_t rc = RF_OK;
  std::vector<RepackEntry> keep;
  for (auto& en : c.entries) {
    if (!drop(en)) {
      keep.push_back(std::move(en));
      continue;
    }
    if (en.ready) hipEventDestroy(en.ready);
    const int32_t r = vram_release(ctx, en.charge);
    if (!rc) rc = r;
    c.bytes -= en.bytes;
  }
  c.entries.swap(keep);
  return rc;
}

// Evict least-recently-used entries until `need` more bytes fit both under
// the cache limit and in the device ledger.  False when they cannot.
static bool repack_make_room(rf_ctx* ctx, uint64_t need, int32_t* rc) {
  RepackCache& c = ctx->repack;
  *rc = RF_OK;
  if (need > c.limit) return false;
  uint64_t freed = 0;
  std::vector<const RepackEntry*> order;
  for (auto& en : c.entries) order.push_back(&en);
  std::sort(order.begin(), order.end(),
            [](const RepackEntry* a, const RepackEntry* b) { return a->last_use < b->last_use; });
  size_t n = 0;
  const auto fits = [&] {
    return c.bytes - freed + need <= c.limit && vram_can_allocate(ctx, need > freed ? need - freed : 0);
  };
  while (!fits() && n < order.size()) freed += order[n++]->bytes;
  if (!fits()) return false;
  if (n == 0) return true;
  const uint64_t evict = order[n - 1]->last_use;
  *rc = repack_drop(ctx, [evict](const RepackEntry& en) { return en.last_use <= evict; });
  return *rc == RF_OK;
}

// Marks entries whose pack has completed (host query of its event; not
// called inside a capture).
static void repack_settle(RepackCache& c) {
  for (auto& en : c.entries)
    if (!en.settled && hipEventQuery(en.ready) == hipSuccess) en.settled = true;
}

// The packed copy of w for this call, or nullptr when rf_matvec is to run the
// GGUF-layout kernel: the type has no packed layout, the shape is beyond the
// packed kernel, or the tensor does not fit.  Inside a stream capture only a
// hit on an entry whose pack has completed is served (nothing is allocated or
// waited for there); rf_capture_end notes that the graph holds cached
// buffers, and rf_graph_replay refuses it once an entry has been dropped.
// Once the context's workspaces are fixed (rf_ctx_reserve), no entry is
// added: a miss would allocate.
static int32_t repack_lookup(rf_ctx* ctx, uint32_t t, const void* w, uint64_t rows, uint64_t in_dim, uint64_t rb,
                             hipStream_t st, const void** out) {
  *out = nullptr;
  if (!packed_type(t) || !plan_packed(t, in_dim).ok) return RF_OK;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  RF_HIP(hipStreamIsCapturing(st, &cs), "hipStreamIsCapturing");
  const bool capturing = cs != hipStreamCaptureStatusNone;
  RepackCache& c = ctx->repack;
  std::lock_guard<std::mutex> lk(c.mu);
  const uint8_t* src = static_cast<const uint8_t*>(w);
  for (auto& en : c.entries) {
    if (en.src != src || en.type != t || en.rows != rows || en.in_dim != in_dim) continue;
    if (capturing) {
      if (!en.settled) return RF_OK;
      ++c.captured_hits;
    } else {
      if (!en.settled && hipEventQuery(en.ready) == hipSuccess) en.settled = true;
      if (!en.settled && en.packed_on != st) RF_HIP(hipStreamWaitEvent(st, en.ready, 0), "hipStreamWaitEvent");
    }
    en.last_use = ++c.clock;
    ++c.hits;
    *out = en.packed;
    return RF_OK;
  }
  if (capturing || ctx->ws_fixed) return RF_OK;
  const uint64_t bytes = rows * rb;
  int32_t rc = RF_OK;
  if (!repack_make_room(ctx, bytes, &rc)) return rc;
  RepackEntry en;
  en.src = src;
  en.type = t;
  en.rows = rows;
  en.in_dim = in_dim;
  en.bytes = bytes;
  en.charge = "workspace:repack:" + std::to_string(++c.seq);
  if (vram_alloc(ctx, en.charge, bytes, &en.packed) != RF_OK) return RF_OK;  // the GGUF kernel instead
  hipError_t e = launch_pack(t, w, en.packed, rows, in_dim, st);
  if (e == hipSuccess) e = hipEventCreateWithFlags(&en.ready, hipEventDisableTiming);
  if (e == hipSuccess) e = hipEventRecord(en.ready, st);
  if (e != hipSuccess) {
    if (en.ready) hipEventDestroy(en.ready);
    hipStreamSynchronize(st);  // the pack may be queued on the buffer
    vram_release(ctx, en.charge);
    return hip_error(e, "repack");
  }
  en.packed_on = st;
  en.last_use = ++c.clock;
  ++c.misses;
  c.bytes += bytes;
  *out = en.packed;
  c.entries.push_back(std::move(en));
  return RF_OK;
}

int32_t rf_matvec_cache(rf_ctx* ctx, uint64_t max_bytes) {
  RF_CHECK_CTX(ctx);
  RepackCache& c = ctx->repack;
  std::lock_guard<std::mutex> lk(c.mu);
  c.limit = max_bytes;
  if (c.bytes <= max_bytes) return RF_OK;
  // drop least-recently-used entries down to the new limit
  std::vector<uint64_t> uses;
  for (auto& en : c.entries) uses.push_back(en.last_use);
  std::sort(uses.begin(), uses.end());
  uint64_t left = c.bytes, cut = 0;
  for (uint64_t u : uses) {
    if (left <= max_bytes) break;
    for (auto& en : c.entries)
      if (en.last_use == u) left -= en.bytes;
    cut = u;
  }
  return repack_drop(ctx, [cut](const RepackEntry& en) { return en.last_use <= cut; });
}

int32_t rf_matvec_cache_forget(rf_ctx* ctx, const void* base, uint64_t bytes) {
  RF_CHECK_CTX(ctx);
  RepackCache& c = ctx->repack;
  std::lock_guard<std::mutex> lk(c.mu);
  const uint8_t* lo = static_cast<const uint8_t*>(base);
  const uint8_t* hi = lo + bytes;
  return repack_drop(ctx, [lo, hi](const RepackEntry& en) { return en.src < hi && lo < en.src + en.bytes; });
}

int32_t rf_matvec_cache_stats(rf_ctx* ctx, uint64_t* entries, uint64_t* bytes, uint64_t* hits, uint64_t* misses) {
  RF_CHECK_CTX(ctx);
  RepackCache& c = ctx->repack;
  std::lock_guard<std::mutex> lk(c.mu);
  if (entries) *entries = c.entries.size();
  if (bytes) *bytes = c.bytes;
  if (hits) *hits = c.hits;
  if (misses) *misses = c.misses;
  return RF_OK;
}

int32_t rf_matvec(rf_ctx* ctx, uint32_t t, const void* w, uint64_t w_bytes, uint64_t out_dim, uint64_t in_dim,
                  const float* x, float* y, uint64_t row_start, uint64_t row_count, rf_stream_t s) {
  RF_CHECK_CTX(ctx);
  uint64_t count = 0, rb = 0;
  bool done = false;
  int32_t rc = validate_matvec(ctx, t, w, w_bytes, out_dim, in_dim, x, y, row_start, row_count, s, &count, &rb,
                               &done);
  if (rc || done) return rc;
  hipStream_t st = pick_stream(ctx, s);
  if (ctx->repack.limit) {
    const void* packed = nullptr;
    rc = repack_lookup(ctx, t, w, out_dim, in_dim, rb, st, &packed);
    if (rc) return rc;
    if (packed) return launch_packed_rows(ctx, t, packed, out_dim, in_dim, x, y, row_start, count, st);
  }
  MvSegDesc seg{static_cast<const uint8_t*>(w) + row_start * rb, nullptr, y, nullptr, count};
  hipError_t e = launch_matvec_segments(t, &seg, 1, x, nullptr, 0.f, in_dim, EPI_STORE, st);
  if (e != hipSuccess) return hip_error(e, "matvec launch");
  return RF_OK;
}

int32_t rf_packed_supported(uint32_t t, uint64_t in_dim) { return plan_packed(t, in_dim).ok ? 1 : 0; }

int32_t rf_pack_weights(rf_ctx* ctx, uint32_t t, const void* raw, uint64_t raw_bytes, uint64_t rows, uint64_t in_dim,
                        void* packed, uint64_t packed_bytes, rf_stream_t s) {
  RF_CHECK_CTX(ctx);
  if (!packed_type(t))
    return set_error(RF_ERR_UNSUPPORTED, "packed layout does not support tensor type %s (%u)", type_name(t), t);
  const char* nm = type_name(t);
  if (!raw || !packed) return set_error(RF_ERR_INVALID, "%s pack received a null pointer", nm);
  uint64_t qk = 0, bs = 0;
  type_geometry(t, &qk, &bs);
  if (in_dim % qk != 0)
    return set_error(RF_ERR_INVALID, "%s in_dim %llu not divisible by %llu", nm, (unsigned long long)in_dim,
                     (unsigned long long)qk);
  uint64_t need = 0;
  if (!mul_u64(rows, in_dim / qk * bs, &need))
    return set_error(RF_ERR_INVALID, "%s weight size of %llu rows of %llu overflows 64 bits", nm,
                     (unsigned long long)rows, (unsigned long long)in_dim);
  if (raw_bytes < need)
    return set_error(RF_ERR_INVALID, "%s weight truncated: expected %llu bytes, got %llu", nm,
                     (unsigned long long)need, (unsigned long long)raw_bytes);
  if (packed_bytes < need)
    return set_error(RF_ERR_INVALID, "%s packed buffer holds %llu bytes, %llu needed", nm,
                     (unsigned long long)packed_bytes, (unsigned long long)need);
  const uint8_t* r8 = static_cast<const uint8_t*>(raw);
  const uint8_t* p8 = static_cast<const uint8_t*>(packed);
  if (p8 < r8 + need && r8 < p8 + need) return set_error(RF_ERR_INVALID, "%s pack buffers overlap", nm);
  hipError_t e = launch_pack(t, raw, packed, rows, in_dim, pick_stream(ctx, s));
  if (e != hipSuccess) return hip_error(e, "pack launch");
  return RF_OK;
}

int32_t rf_matvec_packed(rf_ctx* ctx, uint32_t t, const void* packed, uint64_t packed_bytes, uint64_t out_dim,
                         uint64_t in_dim, const float* x, float* y, uint64_t row_start, uint64_t row_count,
                         rf_stream_t s) {
  RF_CHECK_CTX(ctx);
  if (!packed_type(t))
    return set_error(RF_ERR_UNSUPPORTED, "packed matvec does not support tensor type %s (%u)", type_name(t), t);
  uint64_t count = 0, rb = 0;
  bool done = false;
  int32_t rc = validate_matvec(ctx, t, packed, packed_bytes, out_dim, in_dim, x, y, row_start, row_count, s, &count,
                               &rb, &done);
  if (rc || done) return rc;
  if (!plan_packed(t, in_dim).ok)
    return set_error(RF_ERR_UNSUPPORTED,
                     "packed %s matvec stages x in LDS: in_dim %llu exceeds this device's workgroup LDS",
                     type_name(t), (unsigned long long)in_dim);
  return launch_packed_rows(ctx, t, packed, out_dim, in_dim, x, y, row_start, count, pick_stream(ctx, s));
}

uint64_t rf_matmul_workspace_bytes(uint64_t out_dim, uint64_t in_dim, uint64_t n_tokens) {
  if (out_dim == 0 || in_dim == 0 || n_tokens == 0) return 0;
  const uint64_t chunk = n_tokens < MM_MAX_TOKENS ? n_tokens : MM_MAX_TOKENS;
  // the launches are chunk tokens each, the last one the remainder
  uint64_t part = mm_part_floats_at(&out_dim, 1, in_dim, chunk);
  if (n_tokens % chunk) part = std::max(part, mm_part_floats_at(&out_dim, 1, in_dim, n_tokens % chunk));
  return part * 4;
}

int32_t rf_matmul_packed(rf_ctx* ctx, uint32_t t, const void* packed, uint64_t packed_bytes, uint64_t out_dim,
                         uint64_t in_dim, const float* x, uint64_t n_tokens, float* y, rf_stream_t s) {
  RF_CHECK_CTX(ctx);
  if (!packed_type(t))
    return set_error(RF_ERR_UNSUPPORTED, "packed matmul does not support tensor type %s (%u)", type_name(t), t);
  const char* nm = type_name(t);
  if (!packed || !x || !y) return set_error(RF_ERR_INVALID, "%s matmul received a null pointer", nm);
  uint64_t qk = 0, bs = 0;
  type_geometry(t, &qk, &bs);
  if (in_dim == 0 || in_dim % qk != 0)
    return set_error(RF_ERR_INVALID, "%s row size %llu not divisible by block size %llu", nm,
                     (unsigned long long)in_dim, (unsigned long long)qk);
  if (out_dim == 0 || n_tokens == 0) return RF_OK;
  uint64_t need = 0, xn = 0, yn = 0;
  if (!mul_u64(out_dim, in_dim / qk * bs, &need) || !mul_u64(n_tokens, in_dim, &xn) || !mul_u64(xn, 4, &xn) ||
      !mul_u64(n_tokens, out_dim, &yn) || !mul_u64(yn, 4, &yn))
    return set_error(RF_ERR_INVALID, "%s matmul of %llu tokens x %llu rows of %llu overflows 64 bits", nm,
                     (unsigned long long)n_tokens, (unsigned long long)out_dim, (unsigned long long)in_dim);
  if (packed_bytes < need)
    return set_error(RF_ERR_INVALID, "%s tensor truncated: %llu bytes for %llu rows of %llu (need %llu)", nm,
                     (unsigned long long)packed_bytes, (unsigned long long)out_dim, (unsigned long long)in_dim,
                     (unsigned long long)need);
  if (!mm_supported(t, in_dim) || out_dim > 0xFFFFFFFFull)
    return set_error(RF_ERR_UNSUPPORTED, "packed %s matmul does not cover %llu x %llu", nm,
                     (unsigned long long)out_dim, (unsigned long long)in_dim);
  hipStream_t st = pick_stream(ctx, s);
  const uint64_t chunk = n_tokens < MM_MAX_TOKENS ? n_tokens : MM_MAX_TOKENS;
  int32_t rc = ensure_workspace(ctx, ctx->mm_ws, "workspace:matmul", rf_matmul_workspace_bytes(out_dim, in_dim, n_tokens),
                                st);
  if (rc) return rc;
  const bool aligned = (reinterpret_cast<uintptr_t>(x) & 15u) == 0 && in_dim % 4 == 0;
  if (!aligned) {  // the kernel stages x with 16-byte loads
    rc = ensure_workspace(ctx, ctx->scratch_ws, "workspace:scratch", chunk * in_dim * 4, st);
    if (rc) return rc;
  }
  for (uint64_t off = 0; off < n_tokens; off += MM_MAX_TOKENS) {
    const uint64_t nt = n_tokens - off < MM_MAX_TOKENS ? n_tokens - off : MM_MAX_TOKENS;
    const float* xc = x + off * in_dim;
    if (!aligned) {
      RF_HIP(hipMemcpyAsync(ctx->scratch_ws.ptr, xc, nt * in_dim * 4, hipMemcpyDeviceToDevice, st), "hipMemcpyAsync");
      xc = static_cast<const float*>(ctx->scratch_ws.ptr);
    }
    MmSegDesc seg{packed, out_dim, 0, out_dim, y + off * out_dim, nullptr, nullptr, out_dim};
    hipError_t e = launch_matmul_packed(t, &seg, 1, xc, in_dim, nt, in_dim, EPI_STORE,
                                        static_cast<float*>(ctx->mm_ws.ptr), ctx->mm_ws.bytes / 4, st);
    if (e != hipSuccess) return hip_error(e, "packed matmul launch");
  }
  return RF_OK;
}

int32_t rf_dequantize_rows(rf_ctx* ctx, uint32_t t, const void* w, uint64_t w_bytes, uint64_t in_dim,
                           uint64_t row_start, uint64_t row_count, float* out, rf_stream_t s) {
  RF_CHECK_CTX(ctx);
  uint64_t qk = 1, bs = 0;
  if (t == T_F32) bs = 4;
  else if (t == T_F16 || t == T_BF16) bs = 2;
  else if (!type_geometry(t, &qk, &bs))
    return set_error(RF_ERR_UNSUPPORTED, "decode_row_to_f32: unsupported tensor type %s", type_name(t));
  const char* nm = type_name(t);
  if (!w || !out) return set_error(RF_ERR_INVALID, "%s row decode received a null pointer", nm);
  if (in_dim % qk != 0)
    return set_error(RF_ERR_INVALID, "%s row size %llu not divisible by block size %llu", nm,
                     (unsigned long long)in_dim, (unsigned long long)qk);
  const uint64_t rb = in_dim / qk * bs;
  uint64_t need = 0;
  if (row_start + row_count < row_start || !mul_u64(row_start + row_count, rb, &need))
    return set_error(RF_ERR_INVALID, "%s row range %llu + %llu overflows 64 bits", nm,
                     (unsigned long long)row_start, (unsigned long long)row_count);
  if (w_bytes < need)
    return set_error(RF_ERR_INVALID, "%s row truncated: expected %llu bytes, got %llu", nm,
                     (unsigned long long)need, (unsigned long long)w_bytes);
  hipError_t e = launch_dequant_rows(t, static_cast<const uint8_t*>(w) + row_start * rb, in_dim, row_count, out,
                                     nullptr, 0, pick_stream(ctx, s));
  if (e != hipSuccess) return hip_error(e, "dequant launch");
  return RF_OK;
}

// --------------------------------------------------------------- attention
namespace {

// Validated launch arguments of one single-query attention call and the
// workspace bytes its kernels need (the split kernel's chunk records, or the
// any-shape kernel's score rows).
int32_t attention_setup(const float* q, const float* kh, const float* vh, const float* kc, const float* vc,
                        uint32_t hist, uint32_t qh, uint32_t kvh, uint32_t hd, float* out, AttnArgs* a, bool* fast,
                        uint64_t* ws_bytes) {
  if (qh == 0 || kvh == 0 || hd == 0)
    return set_error(RF_ERR_INVALID, "attention requires non-zero query heads, KV heads, and head dimension");
  if (qh % kvh != 0)
    return set_error(RF_ERR_INVALID, "GQA requires query_heads %u to be divisible by kv_heads %u", qh, kvh);
  if (!q || !kc || !vc || !out || (hist > 0 && (!kh || !vh)))
    return set_error(RF_ERR_INVALID, "attention tensor shape mismatch");
  if (hist == UINT32_MAX) return set_error(RF_ERR_UNSUPPORTED, "attention over more than 2^32 - 1 positions");
  const uint32_t total = hist + 1;
  *a = AttnArgs{};
  a->q = q; a->k_hist = kh; a->v_hist = vh; a->k_cur = kc; a->v_cur = vc; a->out = out;
  a->hist = hist; a->qh = qh; a->kvh = kvh; a->hd = hd;
  a->denom = sqrtf((float)hd);
  auto aligned = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
  *fast = attention_supported(qh, kvh, hd, total) && aligned(q) && (hist == 0 || (aligned(kh) && aligned(vh))) &&
          aligned(kc) && aligned(vc);
  if (*fast) {  // the context is known here: its own regime, sized to itself
    const AttnShape sh = attention_regime_shape(attention_regime(total, qh, kvh, total), qh, kvh, total);
    a->per_q = sh.per_q; a->nsplit = sh.nsplit; a->waves = sh.waves;
    *ws_bytes = attention_ws_floats(a->nsplit, qh, hd) * 4;
  } else {
    a->nsplit = 1;
    *ws_bytes = (uint64_t)qh * total * 4;
  }
  return RF_OK;
}

int32_t attention_launch(const AttnArgs& a, bool fast, hipStream_t st) {
  const hipError_t e = fast ? launch_attention(a, st) : launch_attention_naive(a, st);
  if (e != hipSuccess) return hip_error(e, "attention launch");
  return RF_OK;
}

}  // namespace

int32_t rf_attention_decode(rf_ctx* ctx, const float* q, const float* kh, const float* vh, const float* kc,
                            const float* vc, uint32_t hist, uint32_t qh, uint32_t kvh, uint32_t hd, float* out,
                            rf_stream_t s) {
  RF_CHECK_CTX(ctx);
  AttnArgs a;
  bool fast = false;
  uint64_t ws_bytes = 0;
  int32_t rc = attention_setup(q, kh, vh, kc, vc, hist, qh, kvh, hd, out, &a, &fast, &ws_bytes);
  if (rc) return rc;
  hipStream_t st = pick_stream(ctx, s);
  rc = ensure_workspace(ctx, ctx->attn_ws, "workspace:attention", ws_bytes, st);
  if (rc) return rc;
  a.ws = static_cast<float*>(ctx->attn_ws.ptr);
  return attention_launch(a, fast, st);
}

int32_t rf_attention_decode_noalloc(rf_ctx* ctx, const float* q, const float* kh, const float* vh, const float* kc,
                                    const float* vc, uint32_t hist, uint32_t qh, uint32_t kvh, uint32_t hd,
                                    float* out, rf_stream_t s) {
  RF_CHECK_CTX(ctx);
  AttnArgs a;
  bool fast = false;
  uint64_t ws_bytes = 0;
  int32_t rc = attention_setup(q, kh, vh, kc, vc, hist, qh, kvh, hd, out, &a, &fast, &ws_bytes);
  if (rc) return rc;
  if (ws_bytes > NOALLOC_SCRATCH_BYTES)
    return set_error(RF_ERR_INVALID,
                     "attention over %u positions with %u query heads of %u needs %llu bytes of scratch; the "
                     "no-allocation entry point holds %llu",
                     hist + 1, qh, hd, (unsigned long long)ws_bytes, (unsigned long long)NOALLOC_SCRATCH_BYTES);
  if (!ctx->noalloc_scratch) return set_error(RF_ERR_HIP, "no-allocation scratch was not resolved for this context");
  a.ws = static_cast<float*>(ctx->noalloc_scratch);
  return attention_launch(a, fast, pick_stream(ctx, s));
}

uint64_t rf_attention_workspace_bytes(uint64_t max_positions, uint32_t qh, uint32_t kvh, uint32_t hd) {
  if (max_positions == 0 || qh == 0 || kvh == 0 || hd == 0 || max_positions > 0xFFFFFFFFull) return 0;
  // The split kernel's record count grows with the context: 8 chunks per
  // query head at most below 1024 positions, then the per-KV-head split
  // count, which never decreases with the context.
  const uint32_t total = (uint32_t)max_positions;
  uint32_t nsplit = 1;
  for (int r = 0; r < ATT_REGIMES; ++r)
    nsplit = std::max(nsplit, attention_regime_shape(r, qh, kvh, total).nsplit);
  const uint64_t split = attention_ws_floats(nsplit, qh, hd) * 4;
  const uint64_t naive = (uint64_t)qh * max_positions * 4;
  return std::max(split, naive);
}

// --------------------------------------------------------------- elementwise
int32_t rf_rope(rf_ctx* ctx, float* q, float* k, uint64_t pos, uint32_t hd, uint32_t qh, uint32_t kvh, float theta,
                rf_stream_t s) {
  RF_CHECK_CTX(ctx);
  if (hd == 0 || hd % 2 != 0) return set_error(RF_ERR_INVALID, "RoPE head dimension must be non-zero and even");
  if (qh == 0 || kvh == 0) return set_error(RF_ERR_INVALID, "RoPE requires non-zero query and KV head counts");
  if (!std::isfinite(theta) || theta <= 0.f)
    return set_error(RF_ERR_INVALID, "RoPE frequency base must be finite and positive");
  if (hd > 512) return set_error(RF_ERR_UNSUPPORTED, "RoPE head dimension %u exceeds 512", hd);
  if (!q || !k) return set_error(RF_ERR_INVALID, "RoPE shape mismatch: null q or k");
  RopeCS cs{};
  rope_table_host(cs.cs, pos, 1, hd, theta);
  hipError_t e = launch_rope_pair(q, k, cs, hd, qh, kvh, pick_stream(ctx, s));
  if (e != hipSuccess) return hip_error(e, "rope launch");
  return RF_OK;
}

int32_t rf_rmsnorm(rf_ctx* ctx, const float* x, const float* w, uint64_t n, float eps, float* y, rf_stream_t s) {
  RF_CHECK_CTX(ctx);
  if (n == 0 || !x || !w || !y)
    return set_error(RF_ERR_INVALID, "RMSNorm shape mismatch: input %llu, weight %llu, output %llu",
                     (unsigned long long)n, (unsigned long long)n, (unsigned long long)n);
  if (!std::isfinite(eps) || eps < 0.f)
    return set_error(RF_ERR_INVALID, "RMSNorm epsilon must be finite and non-negative");
  hipError_t e = launch_rmsnorm(x, w, n, eps, y, pick_stream(ctx, s));
  return e == hipSuccess ? RF_OK : hip_error(e, "rmsnorm launch");
}

static int32_t binop(rf_ctx* ctx, int op, const float* a, const float* b, uint64_t n, float* out, rf_stream_t s) {
  RF_CHECK_CTX(ctx);
  if (n && (!a || !b || !out)) return set_error(RF_ERR_INVALID, "elementwise shape mismatch: null operand");
  hipError_t e = launch_binary(op, a, b, n, out, pick_stream(ctx, s));
  return e == hipSuccess ? RF_OK : hip_error(e, "elementwise launch");
}

int32_t rf_add(rf_ctx* ctx, const float* a, const float* b, uint64_t n, float* out, rf_stream_t s) {
  return binop(ctx, BIN_ADD, a, b, n, out, s);
}
int32_t rf_bias_add(rf_ctx* ctx, float* v, const float* bias, uint64_t n, rf_stream_t s) {
  RF_CHECK_CTX(ctx);
  if (n == 0) return RF_OK;
  if (!v || !bias) return set_error(RF_ERR_INVALID, "bias add shape mismatch: null operand");
  hipError_t e = launch_bias_add(v, bias, n, pick_stream(ctx, s));
  return e == hipSuccess ? RF_OK : hip_error(e, "bias add launch");
}
int32_t rf_mul(rf_ctx* ctx, const float* a, const float* b, uint64_t n, float* out, rf_stream_t s) {
  return binop(ctx, BIN_MUL, a, b, n, out, s);
}
int32_t rf_swiglu(rf_ctx* ctx, const float* g, const float* u, uint64_t n, float* out, rf_stream_t s) {
  return binop(ctx, BIN_SWIGLU, g, u, n, out, s);
}

int32_t rf_silu(rf_ctx* ctx, const float* x, uint64_t n, float* out, rf_stream_t s) {
  RF_CHECK_CTX(ctx);
  if (n && (!x || !out)) return set_error(RF_ERR_INVALID, "SiLU shape mismatch: null operand");
  hipError_t e = launch_silu(x, n, out, pick_stream(ctx, s));
  return e == hipSuccess ? RF_OK : hip_error(e, "silu launch");
}

int32_t rf_softmax(rf_ctx* ctx, float* v, uint64_t n, rf_stream_t s) {
  RF_CHECK_CTX(ctx);
  if (n == 0 || !v) return set_error(RF_ERR_INVALID, "softmax requires a non-empty vector");
  hipError_t e = launch_softmax(v, n, pick_stream(ctx, s));
  return e == hipSuccess ? RF_OK : hip_error(e, "softmax launch");
}

int32_t rf_argmax(rf_ctx* ctx, const float* logits, uint64_t n, uint32_t* out, rf_stream_t s) {
  RF_CHECK_CTX(ctx);
  if (!out) return set_error(RF_ERR_INVALID, "argmax output is null");
  if (n == 0) {
    hipError_t e = launch_set_u32(out, 0, pick_stream(ctx, s));  // sampling.rs:41-43
    return e == hipSuccess ? RF_OK : hip_error(e, "argmax launch");
  }
  if (!logits) return set_error(RF_ERR_INVALID, "argmax logits are null");
  if (n > 0xFFFFFFFFull) return set_error(RF_ERR_UNSUPPORTED, "argmax over more than 2^32 logits");
  hipError_t e = launch_argmax(logits, n, out, ctx->amax_val, ctx->amax_idx, nullptr, nullptr, pick_stream(ctx, s));
  return e == hipSuccess ? RF_OK : hip_error(e, "argmax launch");
}

int32_t rf_synth_blocks(rf_ctx* ctx, uint32_t t, uint64_t seed, uint64_t first, uint64_t n, double mul, void* dst,
                        uint64_t dst_bytes, rf_stream_t s) {
  RF_CHECK_CTX(ctx);
  uint64_t qk = 0, bs = 0;
  if (!type_geometry(t, &qk, &bs))
    return set_error(RF_ERR_UNSUPPORTED, "synthetic generator does not emit %s", type_name(t));
  if (n && !dst) return set_error(RF_ERR_INVALID, "null synthetic destination");
  if (n > dst_bytes / bs)
    return set_error(RF_ERR_INVALID, "%llu %s blocks need %llu bytes, destination holds %llu", (unsigned long long)n,
                     type_name(t), (unsigned long long)(n * bs), (unsigned long long)dst_bytes);
  hipError_t e = launch_synth(t, seed, first, n, mul, dst, pick_stream(ctx, s));
  return e == hipSuccess ? RF_OK : hip_error(e, "synth launch");
}

struct rf_graph_h {
  hipGraph_t g = nullptr;
  hipGraphExec_t x = nullptr;
  uint64_t ws_generation = 0;  // the context's workspace generation at capture
  bool repack = false;         // holds rf_matvec calls served by the repack cache
  uint64_t repack_generation = 0;
};

static thread_local uint64_t t_capture_hits = 0;  // repack hits before this thread's capture began

int32_t rf_capture_begin(rf_ctx* ctx) {
  RF_CHECK_CTX(ctx);
  {
    // completed packs become usable inside the capture
    std::lock_guard<std::mutex> lk(ctx->repack.mu);
    repack_settle(ctx->repack);
    t_capture_hits = ctx->repack.captured_hits;
  }
  RF_HIP(hipStreamBeginCapture(ctx->compute, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
  return RF_OK;
}

int32_t rf_capture_end(rf_ctx* ctx, void** graph) {
  RF_CHECK_CTX(ctx);
  if (!graph) return set_error(RF_ERR_INVALID, "null graph output");
  hipGraph_t g = nullptr;
  RF_HIP(hipStreamEndCapture(ctx->compute, &g), "hipStreamEndCapture");
  hipGraphExec_t x = nullptr;
  const hipError_t e = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
  if (e != hipSuccess) {
    hipGraphDestroy(g);
    return hip_error(e, "hipGraphInstantiate");
  }
  rf_graph_h* h = new rf_graph_h;
  h->g = g;
  h->x = x;
  h->ws_generation = ctx->ws_generation;
  {
    std::lock_guard<std::mutex> lk(ctx->repack.mu);
    h->repack = ctx->repack.captured_hits != t_capture_hits;
    h->repack_generation = ctx->repack.generation;
  }
  *graph = h;
  return RF_OK;
}

int32_t rf_graph_replay(rf_ctx* ctx, void* graph, uint32_t reps, float* ms_per_replay) {
  RF_CHECK_CTX(ctx);
  if (!graph || reps == 0) return set_error(RF_ERR_INVALID, "null graph or zero repetitions");
  rf_graph_h* h = static_cast<rf_graph_h*>(graph);
  if (h->ws_generation != ctx->ws_generation)
    return set_error(RF_ERR_INVALID,
                     "graph captured before a context workspace was reallocated (it holds the freed buffer); "
                     "capture it again");
  if (h->repack) {
    std::lock_guard<std::mutex> lk(ctx->repack.mu);
    if (h->repack_generation != ctx->repack.generation)
      return set_error(RF_ERR_INVALID,
                       "graph holds rf_matvec calls served by the repack cache, which has dropped entries since "
                       "(the graph may hold a freed copy); capture it again");
  }
  hipEvent_t a = nullptr, b = nullptr;
  RF_HIP(hipEventCreate(&a), "hipEventCreate");
  hipError_t e = hipEventCreate(&b);
  if (e == hipSuccess) e = hipEventRecord(a, ctx->compute);
  for (uint32_t i = 0; i < reps && e == hipSuccess; ++i) e = hipGraphLaunch(h->x, ctx->compute);
  if (e == hipSuccess) e = hipEventRecord(b, ctx->compute);
  if (e == hipSuccess) e = hipEventSynchronize(b);
  float ms = 0.f;
  if (e == hipSuccess) e = hipEventElapsedTime(&ms, a, b);
  hipEventDestroy(a);
  if (b) hipEventDestroy(b);
  if (e != hipSuccess) return hip_error(e, "graph replay");
  if (ms_per_replay) *ms_per_replay = ms / (float)reps;
  return RF_OK;
}

int32_t rf_graph_destroy(rf_ctx* ctx, void* graph) {
  RF_CHECK_CTX(ctx);
  if (!graph) return RF_OK;
  rf_graph_h* h = static_cast<rf_graph_h*>(graph);
  hipError_t e = hipStreamSynchronize(ctx->compute);
  if (h->x) hipGraphExecDestroy(h->x);
  if (h->g) hipGraphDestroy(h->g);
  delete h;
  return e == hipSuccess ? RF_OK : hip_error(e, "hipStreamSynchronize");
}

uint32_t rf_tune_matvec_tile_bytes(uint32_t bytes) {
  if (bytes) set_matvec_tile_bytes(bytes);
  return matvec_tile_bytes();
}

int32_t rf_tune_matvec_kernel(int32_t mode) {
  if (mode >= 0 && mode <= 2) {
    set_matvec_stream(mode >= 1);
    set_matvec_wave(mode == 2);
  }
  return matvec_wave_on() ? 2 : (matvec_stream() ? 1 : 0);
}

int32_t rf_tune_packed_inflight(int32_t mode) {
  if (mode == 0 || mode == 1) set_packed_inflight(mode);
  return packed_inflight();
}

int32_t rf_tune_matvec_digits(int32_t mode) {
  if (mode >= 0 && mode <= 2) set_matvec_digits(mode);
  return matvec_digits();
}

}  // extern "C"
