// rf_runtime.h — host-side runtime internals (context, ledger, errors).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/ramforge_hip.h"
#include "rf_kernels.h"

namespace rf {

// Thread-local last-error message; returns `code` for tail calls.
int32_t set_error(int32_t code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int32_t hip_error(hipError_t e, const char* what);

// Device-domain MemoryBudget (core/src/memory.rs:30-384): named charges,
// reserve before allocating, release after the physical free.
class Ledger {
 public:
  explicit Ledger(uint64_t total) : total_(total) {}
  int32_t allocate(const std::string& name, uint64_t bytes);
  int32_t release(const std::string& name, uint64_t* released = nullptr);
  int32_t resize(const std::string& name, uint64_t bytes);
  int32_t rename_prefix(const std::string& old_prefix, const std::string& new_prefix);
  bool get(const std::string& name, uint64_t* bytes) const;
  uint64_t used() const { return used_; }
  uint64_t total() const { return total_; }
  uint64_t peak() const { return peak_; }

 private:
  uint64_t total_;
  uint64_t used_ = 0;
  uint64_t peak_ = 0;
  std::map<std::string, uint64_t> allocs_;
};

struct Workspace {
  void* ptr = nullptr;
  uint64_t bytes = 0;
};

// One GGUF tensor held in the packed layout by rf_matvec's repack cache.
// Keyed by the caller's pointer, type and shape; the caller's bytes are
// assumed unchanged while the entry lives (rf_matvec_cache_forget drops it).
struct RepackEntry {
  const uint8_t* src = nullptr;
  uint32_t type = 0;
  uint64_t rows = 0, in_dim = 0, bytes = 0;
  void* packed = nullptr;
  std::string charge;
  hipEvent_t ready = nullptr;  // recorded on `packed_on` after the pack
  hipStream_t packed_on = nullptr;
  bool settled = false;  // the pack is known to have completed
  uint64_t last_use = 0;
};

struct RepackCache {
  std::mutex mu;
  uint64_t limit = 0;  // bytes; 0 = off
  uint64_t bytes = 0, hits = 0, misses = 0, clock = 0, seq = 0;
  uint64_t generation = 0;     // incremented whenever an entry is dropped
  uint64_t captured_hits = 0;  // hits served inside a stream capture
  std::vector<RepackEntry> entries;
};

}  // namespace rf

struct rf_ctx {
  int device = 0;
  hipStream_t compute = nullptr;
  hipStream_t copy = nullptr;
  hipStream_t copy2 = nullptr;  // second upload stream: a streamed layer's copies are split over both
  rf::Ledger ledger{0};
  std::mutex mu;
  std::map<std::string, void*> buffers;  // charge name -> device pointer
  rf::Workspace attn_ws, scratch_ws, mm_ws;
  // Incremented whenever a workspace buffer is replaced: graphs captured
  // before hold the old address and are refused by rf_graph_replay.
  uint64_t ws_generation = 0;
  // rf_ctx_reserve(..., fixed = 1): workspaces never grow after reservation.
  bool ws_fixed = false;
  void* noalloc_scratch = nullptr;  // this device's address of the no-allocation scratch array
  float* amax_val = nullptr;
  uint32_t* amax_idx = nullptr;
  std::mutex stage_mu;  // guards the staging buffers below (one upload at a time)
  void* pinned_stage[2] = {nullptr, nullptr};
  hipEvent_t stage_ev[2] = {nullptr, nullptr};
  uint64_t stage_bytes = 0;  // 0 until both buffers and events exist
  rf::RepackCache repack;    // rf_matvec_cache
};

namespace rf {
// Grow a context-owned workspace (charged as `charge`); synchronises the
// device before releasing a smaller previous buffer.  Refused (RF_ERR_INVALID)
// when the workspaces are fixed by rf_ctx_reserve or while `st` is being
// captured into a graph.
int32_t ensure_workspace(rf_ctx* ctx, Workspace& ws, const char* charge, uint64_t bytes, hipStream_t st);
// Allocate / free a ledger-charged device buffer.
int32_t vram_alloc(rf_ctx* ctx, const std::string& charge, uint64_t bytes, void** out);
int32_t vram_release(rf_ctx* ctx, const std::string& charge);
// Rename every charge (and its buffer record) that starts with old_prefix.
int32_t vram_rename_prefix(rf_ctx* ctx, const std::string& old_prefix, const std::string& new_prefix);
// MemoryBudget::can_allocate: whether `bytes` more fit under the budget.
bool vram_can_allocate(rf_ctx* ctx, uint64_t bytes);
// Upload host bytes through the pinned staging buffers on the copy stream.
int32_t staged_upload(rf_ctx* ctx, void* dst, const void* src, uint64_t bytes);
inline hipStream_t pick_stream(rf_ctx* ctx, rf_stream_t s) {
  return s ? static_cast<hipStream_t>(s) : ctx->compute;
}
const char* type_name(uint32_t t);
// Host cos/sin table for RoPE: out[p][i][2] for positions [p0, p0 + np),
// i < hd/2, with the reference's f32 expression (compute.rs:446-456).
void rope_table_host(float* out, uint64_t p0, uint64_t np, uint32_t hd, float theta);
}  // namespace rf
