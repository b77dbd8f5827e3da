// rf_model.hip — device-resident dense llama/qwen2 decode (host executor).
//
// Mirrors the reference's composition with the device kernels:
//   forward  = StreamingLlamaModel::forward_single_streaming
//              (runtime/src/streaming_model.rs:909-1305)
//   layer    = ModelExecutor::execute_layer (runtime/src/model_executor.rs:102-236)
//   logits   = compute_logits (streaming_model.rs:1334-1370)
//   generate = InferenceEngine::generate_impl's greedy loop (inference.rs:580-707)
//
// Per layer the op order is the reference's (RMSNorm -> Q/K/V -> bias -> RoPE
// -> attention -> o-proj -> residual -> RMSNorm -> gate/up -> SiLU*up -> down
// -> residual) with these launch-level fusions:
//   1. attn RMSNorm + Q/K/V projections: one matvec launch over three segments
//   2. RoPE + attention + K/V cache commit: the split-K attention kernel
//   3. o-proj + residual add: matvec epilogue
//   4. ffn RMSNorm + gate/up + SiLU(gate)*up: dual-tile matvec
//   5. down + residual add: matvec epilogue
// K/V of the token is written to slot `pos` of each layer's own cache while
// that layer runs; every layer reads only slots < pos, so this is equivalent
// to the reference's stage-then-commit after the last layer
// (streaming_model.rs:1049-1070, 1288-1295).
//
// Device state (current position, current token, generated-token ring) lives
// in VRAM so a decode step needs no host round-trip and can be captured once
// into a hipGraph and replayed.
#include <algorithm>
#include <condition_variable>
#include <list>
#include <mutex>
#include <thread>
#include <utility>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "rf_runtime.h"

namespace rf {

struct DevTensor {
  uint32_t type = 0;
  uint64_t ne0 = 0, ne1 = 0, nbytes = 0;
  void* d = nullptr;
  std::string charge;
  bool packed = false;  // device-native layout (rf_matvec_packed.hip), else GGUF bytes
  void* host = nullptr;  // streamed layers: pinned host copy in device layout (d set while resident)
  // Streamed layers read from the model's byte source (rf_model_set_tensor_source):
  // the GGUF type and byte range of the tensor, converted on the device at each load.
  bool src = false;
  uint32_t src_type = 0;
  uint64_t src_off = 0, src_bytes = 0;
  bool streamed() const { return host != nullptr || src; }
  bool present() const { return d != nullptr || streamed(); }
};

// Residency of one streamed layer (device side of load_layer / LayerCache,
// streaming_model.rs:581-873, layer_cache.rs:74-268).
enum { LAYER_HOST = 0, LAYER_ACTIVE = 1, LAYER_CACHED = 2, LAYER_RETIRED = 3 };
struct LayerRes {
  int state = LAYER_HOST;         // ACTIVE: charged "layer:{i}:*"; CACHED: "cache:layer:{i}:*";
                                  // RETIRED: computed, not cacheable, released once its kernels end
  uint64_t bytes = 0;             // device bytes of the layer (sum of its tensors)
  hipEvent_t uploaded = nullptr;  // copy stream: the layer's uploads finished
  hipEvent_t used = nullptr;      // compute stream: the last kernel reading the layer finished
};

// Projection weights in Q8_0 / Q4_0 / Q4_K / Q6_K are repacked at install
// unless disabled (rf_tune_packed_weights); the embedding stays in GGUF
// layout for its row gather.
static int g_pack_weights = 1;

struct Layer {
  DevTensor attn_norm, q, k, v, o, ffn_norm, gate, up, down, bq, bk, bv;
};

}  // namespace rf

using namespace rf;

struct rf_model {
  rf_ctx* ctx = nullptr;
  rf_model_config cfg{};
  uint64_t kv_cap = 0;    // positions the K/V buffers hold now (their layer stride)
  uint64_t kv_max = 0;    // capacity the model was created for: bounds growth, sizes workspaces and regimes
  bool kv_grow = false;   // rf_model_kv_growth: the cache grows in 256-position chunks
  uint64_t kv_limit = 0;  // growth bound of the running rf_model_generate (prompt + max_tokens); 0: kv_max
  DevTensor token_embd, output_norm, output;
  std::vector<Layer> layers;
  float* k_cache = nullptr;  // [layer][cap][kvh][hd]
  float* v_cache = nullptr;
  float* rope = nullptr;     // [cap][hd/2][2]
  float *hidden = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *attn_out = nullptr, *act = nullptr;
  float *logits = nullptr, *final_hidden = nullptr, *attn_ws = nullptr, *up_tmp = nullptr;
  bool attn_fast = false;  // split kernel (else the any-shape kernel)
  // set by enqueue_attention when it left the chunk records for the
  // o-projection to merge; enqueue_oproj follows it (one decision per layer)
  bool oproj_merge = false;
  float *xnorm = nullptr, *mvtmp = nullptr;  // scratch of the unfused fallback
  float* amax_val = nullptr;
  uint32_t* amax_idx = nullptr;
  int32_t* d_pos = nullptr;
  uint32_t* d_token = nullptr;
  uint32_t* d_ring = nullptr;  // token chosen for position p is stored at ring[p]
  uint32_t attn_chunks = 1;  // largest chunk count of the attention regimes (workspace records per head)
  uint64_t seq_len = 0;
  bool use_graph = false;
  // Persistent weights of a streaming model (persistent.rs:1-6, 466-470):
  // 0 = resident when at most 25% of the budget, else streamed (the
  // reference's rule); 1 = always streamed; 2 = always resident.  A streamed
  // embedding / output projection stays in mapped pinned host memory that the
  // kernels read in place (a row for the embedding, every row for logits).
  int persistent_policy = 0;
  // Profiler of the real forward (rf_model_profile): an event pair around
  // every launch group, collected when the pool is reused or read.
  bool prof = false;
  std::vector<hipEvent_t> prof_ev;  // pairs: [2k] before, [2k + 1] after
  std::vector<int> prof_kind;       // group of pair k (0..5 = RF_KERNEL_QKV - 1 ..)
  size_t prof_used = 0;             // pairs recorded and not collected
  double prof_ms[6] = {0, 0, 0, 0, 0, 0};
  uint64_t prof_n[6] = {0, 0, 0, 0, 0, 0};
  // one decode-step graph per attention regime (attn_regime)
  hipGraph_t graph[ATT_REGIMES] = {};
  hipGraphExec_t graph_exec[ATT_REGIMES] = {};
  std::vector<std::string> charges;
  // Layer streaming: every block tensor lives in pinned host memory and is
  // uploaded on demand; an LRU cache of at most cache_cap device bytes keeps
  // layers between tokens.
  bool streaming = false;
  uint64_t cache_cap = 0, cache_used = 0;
  std::vector<LayerRes> res;
  // Batched prefill (rf_model_prefill): activations of one chunk of prompt
  // tokens and its workspaces, charged "tmp:prefill" at the first use.
  bool prefill_batched = false;  // rf_model_generate forwards its prompt batched
  float *p_h = nullptr, *p_xn = nullptr, *p_q = nullptr, *p_k = nullptr, *p_v = nullptr, *p_qr = nullptr;
  float *p_a = nullptr, *p_act = nullptr, *p_up = nullptr, *p_part = nullptr, *p_att = nullptr;
  uint32_t* p_tok = nullptr;
  uint64_t p_part_floats = 0;
  std::list<uint32_t> lru;  // cached layers, most recently used first
  uint64_t st_hits = 0, st_misses = 0, st_evictions = 0, st_uploaded = 0;
  int cache_policy = 0;    // 0: LRU (LayerCache); 1: next use within the layer cycle
  // Streaming units per layer (rf_model_set_stream_units): 1, the whole
  // layer (the reference's LayerCache entry); 2 or 3, parts of it
  // (unit_slots).  res, lru and cur_layer count units.
  uint32_t upl = 1;
  uint32_t cur_layer = 0;  // streaming unit the forward pass is at (policy 1)
  // Byte source of streamed layers (rf_model_set_reader): ranges are read into
  // two pinned staging buffers of stage_bytes each and converted on the device
  // through a raw buffer charged "workspace:layer_read" (grown on demand).
  rf_read_fn reader = nullptr;
  void* reader_user = nullptr;
  void* rstage[2] = {nullptr, nullptr};
  hipEvent_t rstage_ev[2] = {nullptr, nullptr};
  hipEvent_t up2 = nullptr;  // a streamed layer's copies on the second upload stream ended
  uint64_t rstage_bytes = 0;
  void* rraw = nullptr;
  uint64_t rraw_bytes = 0;
  uint64_t st_read_calls = 0, st_read_bytes = 0;
  // Read-ahead (rf_model_set_read_ahead; on by default with the library's
  // own rf_file_source_read, whose reads are thread-safe): a worker thread
  // reads the next host-only layer's ranges into one of two pinned buffers
  // of a layer's source bytes while this thread queues the layers before it
  // (two, so that one layer's upload and the next one's read overlap).
  struct ReadAhead {
    std::thread th;
    std::mutex mu;
    std::condition_variable cv;
    bool on = false, stop = false;
    int state = 0;       // 0 idle, 1 requested (being read), 2 read, 3 the read failed
    int64_t layer = -1;  // layer of the request
    std::vector<std::pair<uint64_t, uint64_t>> ranges;  // (offset, length) of its reads, in buffer order
    int32_t err = 0;     // a failed read: the reader's code and range
    uint64_t err_off = 0, err_len = 0;
    void* buf[2] = {nullptr, nullptr};
    uint64_t bytes = 0;                     // of each buffer
    hipEvent_t done[2] = {nullptr, nullptr};  // the copies out of buf[i] ended
    int slot = 0;                           // buffer of the request
    uint64_t used = 0;                      // layers served from the buffers
  } ra;
};

namespace {

int32_t charge_alloc(rf_model* m, const std::string& name, uint64_t bytes, void** out) {
  int32_t rc = vram_alloc(m->ctx, name, bytes, out);
  if (rc == RF_OK) m->charges.push_back(name);
  return rc;
}

// Free a buffer made by charge_alloc and forget its charge.
int32_t release_charge(rf_model* m, const std::string& name) {
  const int32_t rc = vram_release(m->ctx, name);
  for (size_t i = 0; i < m->charges.size(); ++i)
    if (m->charges[i] == name) { m->charges.erase(m->charges.begin() + i); break; }
  return rc;
}

int32_t drop_tensor(rf_model* m, DevTensor& t) {
  if (!t.present()) return RF_OK;
  if (t.charge.empty() && t.host) {  // a streamed persistent weight: pinned host memory, no charge
    hipError_t e = hipStreamSynchronize(m->ctx->compute);
    hipHostFree(t.host);
    t = DevTensor{};
    return e == hipSuccess ? RF_OK : hip_error(e, "hipStreamSynchronize");
  }
  const int32_t rc = release_charge(m, t.charge);
  t = DevTensor{};
  return rc;
}

void reset_graph(rf_model* m) {
  for (int r = 0; r < ATT_REGIMES; ++r) {
    if (m->graph_exec[r]) hipGraphExecDestroy(m->graph_exec[r]);
    if (m->graph[r]) hipGraphDestroy(m->graph[r]);
    m->graph_exec[r] = nullptr;
    m->graph[r] = nullptr;
  }
}

// ------------------------------------------------------- layer streaming

// Host copies of the decode rules the device uses at install (F16/BF16 are
// widened to F32; quant.rs:40-65 incl. its subnormal rule, tensor.rs:1044-1047).
float host_half_to_float(uint32_t h) {
  const uint32_t sign = (h & 0x8000u) << 16, exp = (h >> 10) & 0x1Fu, frac = h & 0x3FFu;
  uint32_t bits;
  if (exp == 0u) {
    float v = (float)frac * 0x1p-25f;
    memcpy(&bits, &v, 4);
    bits |= sign;
  } else {
    bits = sign | (((exp == 0x1Fu) ? 0xFFu : exp + 112u) << 23) | (frac << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

// GGUF payload -> packed layout on the host (same rules as pack_blocks): the
// bytes of block i go to offset i * (region bytes per block) of each region.
void host_pack(uint32_t t, const uint8_t* raw, uint64_t rows, uint64_t in, uint8_t* out) {
  if (t == T_Q8_0 || t == T_Q4_0) {
    const uint64_t n = rows * (in / 32), bs = t == T_Q8_0 ? 34 : 18, cb = bs - 2;
    uint8_t* scales = out + n * cb;
    for (uint64_t i = 0; i < n; ++i) {
      const uint8_t* b = raw + i * bs;
      memcpy(scales + 2 * i, b, 2);
      memcpy(out + i * cb, b + 2, cb);
    }
  } else if (t == T_Q4_K) {
    const uint64_t n = rows * (in / 256);
    for (uint64_t i = 0; i < n; ++i) {
      const uint8_t* b = raw + i * 144;
      memcpy(out + n * 128 + 16 * i, b, 16);  // d, dmin, scales[12]
      memcpy(out + 128 * i, b + 16, 128);     // qs
    }
  } else {  // Q6_K
    const uint64_t n = rows * (in / 256);
    uint8_t *qh = out + n * 128, *sc = qh + n * 64, *d = sc + n * 16;
    for (uint64_t i = 0; i < n; ++i) {
      const uint8_t* b = raw + i * 210;
      memcpy(out + 128 * i, b, 128);  // ql
      memcpy(qh + 64 * i, b + 128, 64);
      memcpy(sc + 16 * i, b + 192, 16);
      memcpy(d + 2 * i, b + 208, 2);
    }
  }
}

void layer_slots(Layer& L, DevTensor* out[12]) {
  DevTensor* t[12] = {&L.attn_norm, &L.q, &L.k, &L.v, &L.o, &L.ffn_norm, &L.gate, &L.up, &L.down, &L.bq, &L.bk, &L.bv};
  for (int i = 0; i < 12; ++i) out[i] = t[i];
}

const char* slot_name(int i) {
  static const char* n[12] = {"attn_norm.weight", "attn_q.weight", "attn_k.weight", "attn_v.weight",
                              "attn_output.weight", "ffn_norm.weight", "ffn_gate.weight", "ffn_up.weight",
                              "ffn_down.weight", "attn_q.bias", "attn_k.bias", "attn_v.bias"};
  return n[i];
}

// Streaming units.  With upl units per layer, unit upl i + p is part p of
// layer i: upl 1, the whole layer; upl 2, the attention tensors with both
// norms (the prefill's o-projection applies the feed-forward norm), then
// the feed-forward matrices (gate, up, down); upl 3, the attention part,
// then gate and up, then down.  The pass acquires each part while the
// previous part's kernels run.
uint32_t slot_part(uint32_t upl, int i) {
  if (upl == 1 || i < 6 || i > 8) return 0;  // norms, attention, biases
  return upl == 2 ? 1 : (i == 8 ? 2 : 1);     // gate, up | down
}

uint32_t unit_count(const rf_model* m) { return (uint32_t)m->layers.size() * m->upl; }

uint32_t unit_layer(const rf_model* m, uint32_t u) { return u / m->upl; }

// The 12 tensor slots of unit u; the slots of the layer's other parts are an
// empty tensor (not streamed, no buffer), which every streaming loop skips.
void unit_slots(rf_model* m, uint32_t u, DevTensor* out[12]) {
  layer_slots(m->layers[unit_layer(m, u)], out);
  if (m->upl == 1) return;
  static DevTensor none;
  const uint32_t part = u % m->upl;
  for (int i = 0; i < 12; ++i)
    if (slot_part(m->upl, i) != part) out[i] = &none;
}

// Charge of slot i of unit u while the unit is active ("layer:{layer}:{tensor}").
std::string unit_charge(const rf_model* m, uint32_t u, int i) {
  return "layer:" + std::to_string(unit_layer(m, u)) + ":" + slot_name(i);
}

// Renames the charges of unit u's device tensors from prefix `from` + their
// active names to `to` + them ("" or "cache:"), tensor by tensor, so that the
// other half of a split layer keeps its names.
int32_t rename_unit(rf_model* m, uint32_t u, const std::string& from, const std::string& to) {
  DevTensor* t[12];
  unit_slots(m, u, t);
  for (int i = 0; i < 12; ++i) {
    if (!t[i]->d) continue;
    const std::string name = unit_charge(m, u, i);
    const int32_t rc = vram_rename_prefix(m->ctx, from + name, to + name);
    if (rc) return rc;
    t[i]->charge = to + name;
  }
  return RF_OK;
}

// Device bytes of each streaming unit of layer li.
void update_layer_bytes(rf_model* m, uint32_t li) {
  const uint32_t per = m->upl;
  for (uint32_t u = li * per; u < (li + 1) * per && u < m->res.size(); ++u) {
    DevTensor* t[12];
    unit_slots(m, u, t);
    uint64_t b = 0;
    for (DevTensor* x : t)
      if (x->streamed()) b += x->nbytes;
    m->res[u].bytes = b;
  }
}

// Physical free of a resident layer's buffers, then release of its charges
// (memory.rs:9-15): waits until the last kernel that read the layer ended.
int32_t layer_free(rf_model* m, uint32_t li) {
  LayerRes& R = m->res[li];
  if (R.state == LAYER_HOST) return RF_OK;
  hipError_t e = hipEventSynchronize(R.used);
  if (e == hipSuccess) e = hipEventSynchronize(R.uploaded);
  if (e != hipSuccess) return hip_error(e, "layer release");
  DevTensor* t[12];
  unit_slots(m, li, t);
  int32_t rc = RF_OK;
  for (DevTensor* x : t) {
    if (!x->d) continue;
    const int32_t r = vram_release(m->ctx, x->charge);
    if (r && !rc) rc = r;
    x->d = nullptr;
    x->charge.clear();
  }
  if (R.state == LAYER_CACHED) {
    m->lru.remove(li);
    m->cache_used -= R.bytes;
  }
  R.state = LAYER_HOST;
  return rc;
}

// Steps until layer j is needed again by the pass that is at cur_layer
// (every pass visits the layers in order; the current layer counts as a
// full cycle away once computed).
uint32_t next_use(const rf_model* m, uint32_t j) {
  const uint32_t n = unit_count(m);
  const uint32_t d = (j + n - m->cur_layer) % n;
  return d == 0 ? n : d;
}

// The cached layer to drop: LayerCache::evict_lru's least recently used one
// (policy 0), or the one needed furthest in the future (policy 1, the
// optimal choice for the cyclic layer scan of decoding).
uint32_t pick_victim(const rf_model* m) {
  if (m->cache_policy == 0) return m->lru.back();
  uint32_t best = m->lru.back(), bd = 0;
  for (uint32_t j : m->lru)
    if (next_use(m, j) > bd) { bd = next_use(m, j); best = j; }
  return best;
}

bool evict_lru(rf_model* m, int32_t* rc) {
  if (m->lru.empty()) return false;
  const uint32_t victim = pick_victim(m);
  *rc = layer_free(m, victim);
  m->st_evictions += 1;
  return true;
}

// Release every layer that was computed but is not cacheable.
int32_t release_retired(rf_model* m) {
  for (uint32_t li = 0; li < m->res.size(); ++li)
    if (m->res[li].state == LAYER_RETIRED) {
      const int32_t rc = layer_free(m, li);
      if (rc) return rc;
    }
  return RF_OK;
}

// Make room for `bytes`: retired layers first, then LRU cached layers
// (ensure_layer_cache_headroom, streaming_model.rs:555-572).
int32_t make_headroom(rf_model* m, uint64_t bytes) {
  if (vram_can_allocate(m->ctx, bytes)) return RF_OK;
  int32_t rc = release_retired(m);
  if (rc) return rc;
  while (!vram_can_allocate(m->ctx, bytes)) {
    if (!evict_lru(m, &rc)) return RF_ERR_BUDGET;
    if (rc) return rc;
  }
  return RF_OK;
}

constexpr uint64_t KV_GROW_CHUNK = 256;  // KvCache::GROW_CHUNK_TOKENS (kv_cache.rs:49)

// Reallocate the K/V caches for `target` positions, keeping the committed
// ones (KvCache::grow_to_with_budget, kv_cache.rs:297-356): the replacement
// is charged "kv_cache:{k,v}:growth" while the old buffers stay charged (the
// real peak of the copy), after streamed layers have been evicted to make
// room for it (ensure_layer_cache_headroom); then the old buffers are freed
// and the new charges take the old names.  On any failure the cache, its
// charges and the captured graphs are unchanged.
int32_t kv_resize(rf_model* m, uint64_t target) {
  const rf_model_config& c = m->cfg;
  const uint64_t kvd = c.head_count_kv * c.head_dim, nl = c.block_count;
  const uint64_t nb = nl * target * kvd * 4;
  if (m->streaming) {
    const int32_t rc = make_headroom(m, 2 * nb);
    if (rc && rc != RF_ERR_BUDGET) return rc;  // a short budget is reported by the allocation below
  }
  void *nk = nullptr, *nv = nullptr;
  int32_t rc = vram_alloc(m->ctx, "kv_cache:k:growth", nb, &nk);
  if (rc) return rc;
  rc = vram_alloc(m->ctx, "kv_cache:v:growth", nb, &nv);
  if (rc) {
    vram_release(m->ctx, "kv_cache:k:growth");
    return rc;
  }
  hipStream_t st = m->ctx->compute;
  const uint64_t keep = std::min(m->seq_len, target) * kvd * 4;
  hipError_t e = hipSuccess;
  for (uint64_t li = 0; li < nl && keep && e == hipSuccess; ++li) {
    e = hipMemcpyAsync(static_cast<float*>(nk) + li * target * kvd, m->k_cache + li * m->kv_cap * kvd, keep,
                       hipMemcpyDeviceToDevice, st);
    if (e == hipSuccess)
      e = hipMemcpyAsync(static_cast<float*>(nv) + li * target * kvd, m->v_cache + li * m->kv_cap * kvd, keep,
                         hipMemcpyDeviceToDevice, st);
  }
  if (e == hipSuccess) e = hipStreamSynchronize(st);
  if (e != hipSuccess) {
    vram_release(m->ctx, "kv_cache:k:growth");
    vram_release(m->ctx, "kv_cache:v:growth");
    return hip_error(e, "KV cache growth copy");
  }
  reset_graph(m);  // the graphs hold the old buffers and layer stride
  vram_release(m->ctx, "kv_cache:k");
  vram_release(m->ctx, "kv_cache:v");
  vram_rename_prefix(m->ctx, "kv_cache:k:growth", "kv_cache:k");
  vram_rename_prefix(m->ctx, "kv_cache:v:growth", "kv_cache:v");
  m->k_cache = static_cast<float*>(nk);
  m->v_cache = static_cast<float*>(nv);
  m->kv_cap = target;
  return RF_OK;
}

// Room for `need` positions before they are written: a fixed cache refuses
// past its capacity; a growing one takes the next multiple of 256 positions,
// at most the growth bound (inference.rs:666-687).
int32_t ensure_kv(rf_model* m, uint64_t need) {
  if (need <= m->kv_cap) return RF_OK;
  const uint64_t bound = m->kv_limit ? std::min(m->kv_limit, m->kv_max) : m->kv_max;
  if (!m->kv_grow || need > bound) return set_error(RF_ERR_INVALID, "KV cache full");
  uint64_t target = (need + KV_GROW_CHUNK - 1) / KV_GROW_CHUNK * KV_GROW_CHUNK;
  if (target > bound) target = bound;
  const int32_t rc = kv_resize(m, target);
  if (rc) {
    char why[512];
    rf_last_error(why, sizeof why);
    return set_error(rc, "failed to grow KV cache from %llu to %llu tokens: %s", (unsigned long long)m->kv_cap,
                     (unsigned long long)target, why);
  }
  return RF_OK;
}

constexpr uint64_t READ_GAP_BYTES = 4096;  // MAX_COALESCED_GAP_BYTES (layer_read.rs:6)

// The layer's source tensors as read ranges (build_layer_read_plan,
// layer_read.rs:51-160): sorted by offset and merged while the gap to the
// next tensor is at most 4 KiB and the merged span fits one staging buffer
// (the reference's bound is 64 MiB); a tensor larger than a buffer is a range
// of its own, read in buffer-sized pieces.
struct ReadRange {
  uint64_t off = 0, len = 0;
  std::vector<int> slots;
};
int32_t plan_layer_reads(rf_model* m, DevTensor* t[12], std::vector<ReadRange>* out) {
  std::vector<int> idx;
  for (int i = 0; i < 12; ++i)
    if (t[i]->src) idx.push_back(i);
  std::stable_sort(idx.begin(), idx.end(), [&](int a, int b) { return t[a]->src_off < t[b]->src_off; });
  std::vector<ReadRange>& r = *out;
  for (int i : idx) {
    const uint64_t off = t[i]->src_off, end = off + t[i]->src_bytes;
    if (!r.empty()) {
      ReadRange& c = r.back();
      const uint64_t cend = c.off + c.len;
      if (off < cend) return set_error(RF_ERR_INVALID, "tensor ranges overlap at '%s'", slot_name(i));
      if (off - cend <= READ_GAP_BYTES && end - c.off <= m->rstage_bytes) {
        c.len = end - c.off;
        c.slots.push_back(i);
        continue;
      }
    }
    ReadRange n;
    n.off = off;
    n.len = end - off;
    n.slots.push_back(i);
    r.push_back(n);
  }
  return RF_OK;
}

// Read-ahead worker: waits for a request, for the copies out of the buffer
// to end, then reads the request's ranges into it.
void ra_worker(rf_model* m) {
  rf_model::ReadAhead& ra = m->ra;
  (void)hipSetDevice(m->ctx->device);
  std::unique_lock<std::mutex> lk(ra.mu);
  for (;;) {
    ra.cv.wait(lk, [&] { return ra.stop || ra.state == 1; });
    if (ra.stop) return;
    const std::vector<std::pair<uint64_t, uint64_t>> ranges = ra.ranges;
    const int slot = ra.slot;
    lk.unlock();
    (void)hipEventSynchronize(ra.done[slot]);
    int32_t err = 0;
    uint64_t eo = 0, el = 0, pos = 0;
    for (const auto& r : ranges) {
      const int32_t rc = m->reader(m->reader_user, r.first, r.second, static_cast<uint8_t*>(ra.buf[slot]) + pos);
      if (rc != 0) {
        err = rc;
        eo = r.first;
        el = r.second;
        break;
      }
      pos += r.second;
    }
    lk.lock();
    ra.err = err;
    ra.err_off = eo;
    ra.err_len = el;
    ra.state = err ? 3 : 2;
    ra.cv.notify_all();
  }
}

void ra_stop(rf_model* m) {
  rf_model::ReadAhead& ra = m->ra;
  if (ra.th.joinable()) {
    {
      std::lock_guard<std::mutex> g(ra.mu);
      ra.stop = true;
    }
    ra.cv.notify_all();
    ra.th.join();
  }
  ra.stop = false;
  ra.state = 0;
  ra.layer = -1;
  for (int i = 0; i < 2; ++i) {
    if (ra.done[i]) (void)hipEventSynchronize(ra.done[i]);
    if (ra.buf[i]) hipHostFree(ra.buf[i]);
    ra.buf[i] = nullptr;
  }
  ra.bytes = 0;
}

int32_t plan_layer_reads(rf_model* m, DevTensor* t[12], std::vector<ReadRange>* out);

// Bytes a layer's reads fill (0 when it has no source tensors).
uint64_t layer_read_bytes(rf_model* m, uint32_t li) {
  DevTensor* t[12];
  unit_slots(m, li, t);
  std::vector<ReadRange> plan;
  if (plan_layer_reads(m, t, &plan) != RF_OK) return 0;
  uint64_t n = 0;
  for (const ReadRange& r : plan) n += r.len;
  return n;
}

// Requests layer li's bytes from the worker (started, with its buffer sized
// for the largest layer, at the first request).  A request while the worker
// reads is dropped; the layer is then read by the pass itself.
void ra_post(rf_model* m, uint32_t li) {
  rf_model::ReadAhead& ra = m->ra;
  if (!ra.on || !m->reader) return;
  if (!ra.buf[0]) {
    uint64_t most = 0;
    for (uint32_t j = 0; j < unit_count(m); ++j) most = std::max(most, layer_read_bytes(m, j));
    if (most == 0) return;
    for (int i = 0; i < 2; ++i) {
      if (!ra.done[i] && hipEventCreateWithFlags(&ra.done[i], hipEventDisableTiming) != hipSuccess) ra.done[i] = nullptr;
      if (ra.done[i] && hipHostMalloc(&ra.buf[i], most, hipHostMallocDefault) != hipSuccess) ra.buf[i] = nullptr;
    }
    if (!ra.buf[0] || !ra.buf[1]) {  // no room for them: the pass reads as without
      for (int i = 0; i < 2; ++i) {
        if (ra.buf[i]) hipHostFree(ra.buf[i]);
        ra.buf[i] = nullptr;
      }
      ra.on = false;
      return;
    }
    ra.bytes = most;
  }
  if (!ra.th.joinable()) ra.th = std::thread(ra_worker, m);
  DevTensor* t[12];
  unit_slots(m, li, t);
  std::vector<ReadRange> plan;
  if (plan_layer_reads(m, t, &plan) != RF_OK) return;
  uint64_t total = 0;
  for (const ReadRange& r : plan) total += r.len;
  if (total == 0 || total > ra.bytes) return;
  std::lock_guard<std::mutex> g(ra.mu);
  if (ra.state == 1 || (ra.state == 2 && ra.layer == (int64_t)li)) return;
  ra.ranges.clear();
  for (const ReadRange& r : plan) ra.ranges.emplace_back(r.off, r.len);
  // the last read's buffer may still be uploading from: read into the other
  // one (a read nobody took keeps its buffer)
  if (ra.state == 0) ra.slot ^= 1;
  ra.layer = li;
  ra.state = 1;
  ra.cv.notify_all();
}

// The next layer the pass will load from the byte source, in the layer cycle
// from `from` on: a host-only layer of this pass, else of the next one (a
// retired layer is released at the end of this pass); -1 when none.
int64_t next_read_layer(rf_model* m, uint32_t from) {
  const uint32_t nl = unit_count(m);
  for (uint32_t j = from; j < nl; ++j)
    if (m->res[j].state == LAYER_HOST) return j;
  for (uint32_t j = 0; j < std::min(from, nl); ++j)
    if (m->res[j].state == LAYER_HOST || m->res[j].state == LAYER_RETIRED) return j;
  return -1;
}

// Reads the layer's source tensors range by range into the pinned staging
// buffers (alternating, each reused once the copy out of it has finished),
// copies every tensor to its device buffer, or to the raw buffer and then
// packs or widens it into its device buffer, all on the copy stream.
int32_t read_layer_sources(rf_model* m, uint32_t li, DevTensor* t[12], hipStream_t cs) {
  std::vector<ReadRange> plan;
  int32_t rc = plan_layer_reads(m, t, &plan);
  if (rc) return rc;
  auto convert = [&](DevTensor* x) -> hipError_t {  // raw buffer -> device layout
    if (x->type == T_F32 && x->src_type != T_F32)
      return launch_dequant_rows(x->src_type, m->rraw, x->ne0, x->ne1, static_cast<float*>(x->d), nullptr, 0, cs);
    return launch_pack(x->src_type, m->rraw, x->d, x->ne1, x->ne0, cs);
  };
  auto needs_convert = [](const DevTensor* x) { return x->packed || (x->type == T_F32 && x->src_type != T_F32); };
  // read ahead by the worker: the layer's ranges are in its buffer, in plan order
  if (m->ra.on) {
    rf_model::ReadAhead& ra = m->ra;
    std::unique_lock<std::mutex> lk(ra.mu);
    if (ra.layer == (int64_t)li && ra.state != 0) {
      ra.cv.wait(lk, [&] { return ra.state != 1; });
      const bool failed = ra.state == 3;
      const int32_t err = ra.err;
      const uint64_t eo = ra.err_off, el = ra.err_len;
      uint64_t calls = 0, bytes = 0;
      for (const auto& r : ra.ranges) {
        calls += 1;
        bytes += r.second;
      }
      ra.state = 0;
      ra.layer = -1;
      if (failed)
        return set_error(RF_ERR_IO, "byte source read of %llu bytes at offset %llu failed (%d) for layer %u",
                         (unsigned long long)el, (unsigned long long)eo, (int)err, unit_layer(m, li));
      m->st_read_calls += calls;
      m->st_read_bytes += bytes;
      uint64_t pos = 0;
      for (const ReadRange& r : plan) {
        for (int i : r.slots) {
          DevTensor* x = t[i];
          const bool cv = needs_convert(x);
          hipError_t e = hipMemcpyAsync(cv ? m->rraw : x->d,
                                        static_cast<uint8_t*>(ra.buf[ra.slot]) + pos + (x->src_off - r.off),
                                        x->src_bytes, hipMemcpyHostToDevice, cs);
          if (e == hipSuccess && cv) e = convert(x);
          if (e != hipSuccess) return hip_error(e, "layer upload");
          m->st_uploaded += x->src_bytes;
        }
        pos += r.len;
      }
      ra.used += 1;
      const hipError_t e = hipEventRecord(ra.done[ra.slot], cs);
      return e == hipSuccess ? RF_OK : hip_error(e, "hipEventRecord");
    }
  }
  int buf = 0;
  auto fill = [&](uint64_t off, uint64_t len) -> int32_t {  // one reader call into the next staging buffer
    hipError_t e = hipEventSynchronize(m->rstage_ev[buf]);
    if (e != hipSuccess) return hip_error(e, "staging buffer wait");
    const int32_t r = m->reader(m->reader_user, off, len, m->rstage[buf]);
    m->st_read_calls += 1;
    if (r != 0)
      return set_error(RF_ERR_IO, "byte source read of %llu bytes at offset %llu failed (%d) for layer %u",
                       (unsigned long long)len, (unsigned long long)off, (int)r, unit_layer(m, li));
    m->st_read_bytes += len;
    return RF_OK;
  };
  for (const ReadRange& r : plan) {
    if (r.len <= m->rstage_bytes) {
      if ((rc = fill(r.off, r.len))) return rc;
      for (int i : r.slots) {
        DevTensor* x = t[i];
        const bool cv = needs_convert(x);
        hipError_t e = hipMemcpyAsync(cv ? m->rraw : x->d, static_cast<uint8_t*>(m->rstage[buf]) + (x->src_off - r.off),
                                      x->src_bytes, hipMemcpyHostToDevice, cs);
        if (e == hipSuccess && cv) e = convert(x);
        if (e != hipSuccess) return hip_error(e, "layer upload");
        m->st_uploaded += x->src_bytes;
      }
      hipError_t e = hipEventRecord(m->rstage_ev[buf], cs);
      if (e != hipSuccess) return hip_error(e, "hipEventRecord");
      buf ^= 1;
      continue;
    }
    DevTensor* x = t[r.slots[0]];  // one tensor larger than a staging buffer
    const bool cv = needs_convert(x);
    uint8_t* dst = static_cast<uint8_t*>(cv ? m->rraw : x->d);
    for (uint64_t p = 0; p < r.len; p += m->rstage_bytes) {
      const uint64_t n = std::min(m->rstage_bytes, r.len - p);
      if ((rc = fill(r.off + p, n))) return rc;
      hipError_t e = hipMemcpyAsync(dst + p, m->rstage[buf], n, hipMemcpyHostToDevice, cs);
      if (e == hipSuccess) e = hipEventRecord(m->rstage_ev[buf], cs);
      if (e != hipSuccess) return hip_error(e, "layer upload");
      buf ^= 1;
    }
    if (cv) {
      const hipError_t e = convert(x);
      if (e != hipSuccess) return hip_error(e, "layer conversion");
    }
    m->st_uploaded += x->src_bytes;
  }
  return RF_OK;
}

// A streamed pass that fails part-way releases every layer it loaded and did
// not cache (the reference releases each computed layer before the next, so
// its budget is back where it was), leaving cached layers cached.  Returns rc.
int32_t abort_pass(rf_model* m, int32_t rc) {
  for (uint32_t li = 0; li < m->res.size(); ++li)
    if (m->res[li].state == LAYER_ACTIVE || m->res[li].state == LAYER_RETIRED) (void)layer_free(m, li);
  return rc;
}

// load_layer (streaming_model.rs:581-847) on the device: every tensor is
// charged "layer:{i}:{name}" before its buffer is allocated, then uploaded
// from the pinned host copy on the copy stream.  On failure every charge made
// for the layer is released and the layer stays host-only.
// Whether layer v's resident buffers can hold layer li: the same tensors
// streamed, with the same sizes (all blocks of one model, in practice).
bool same_layout(rf_model* m, uint32_t v, uint32_t li) {
  DevTensor *a[12], *b[12];
  unit_slots(m, v, a);
  unit_slots(m, li, b);
  for (int i = 0; i < 12; ++i) {
    if (a[i]->streamed() != b[i]->streamed()) return false;
    if (a[i]->streamed() && (a[i]->nbytes != b[i]->nbytes || !a[i]->d)) return false;
  }
  return true;
}

// The layer whose buffers load_layer takes over instead of freeing them and
// allocating new ones: a retired layer first, then the cache's victim (the
// order make_headroom frees in).  -1 when none has li's layout.
int64_t recycle_candidate(rf_model* m, uint32_t li) {
  for (uint32_t v = 0; v < m->res.size(); ++v)
    if (v != li && m->res[v].state == LAYER_RETIRED && same_layout(m, v, li)) return v;
  if (m->lru.empty()) return -1;
  const uint32_t v = pick_victim(m);
  return same_layout(m, v, li) ? (int64_t)v : -1;
}

// Layer v's buffers become layer li's: its charges are renamed "layer:{li}:*"
// (the ledger's release of v and charge of li in one step, the same bytes),
// and the copy stream waits on the GPU for v's last kernel before writing
// them.  An eviction (release_layer + load) with no hipFree, hipMalloc or
// host wait in between.
int32_t adopt_buffers(rf_model* m, uint32_t v, uint32_t li) {
  LayerRes& V = m->res[v];
  hipError_t e = hipStreamWaitEvent(m->ctx->copy, V.used, 0);
  if (e == hipSuccess) e = hipStreamWaitEvent(m->ctx->copy2, V.used, 0);
  if (e != hipSuccess) return hip_error(e, "wait for the recycled layer's kernels");
  const bool cached = V.state == LAYER_CACHED;
  DevTensor *a[12], *b[12];
  unit_slots(m, v, a);
  unit_slots(m, li, b);
  for (int i = 0; i < 12; ++i) {
    if (!a[i]->streamed()) continue;
    const std::string to = unit_charge(m, li, i);
    const int32_t rc = vram_rename_prefix(m->ctx, (cached ? "cache:" : "") + unit_charge(m, v, i), to);
    if (rc) return rc;
    b[i]->d = a[i]->d;
    b[i]->charge = to;
    a[i]->d = nullptr;
    a[i]->charge.clear();
  }
  if (cached) {
    m->lru.remove(v);
    m->cache_used -= V.bytes;
    m->st_evictions += 1;
  }
  V.state = LAYER_HOST;
  return RF_OK;
}

int32_t load_layer(rf_model* m, uint32_t li) {
  LayerRes& R = m->res[li];
  DevTensor* t[12];
  unit_slots(m, li, t);
  hipStream_t cs = m->ctx->copy, cs2 = m->ctx->copy2;
  auto rollback = [&](int32_t code) {  // release every charge of this layer
    hipStreamSynchronize(cs);
    hipStreamSynchronize(cs2);
    for (DevTensor* y : t)
      if (y->d) {
        vram_release(m->ctx, y->charge);
        y->d = nullptr;
        y->charge.clear();
      }
    return code;
  };
  int32_t rc = RF_OK;
  const int64_t v = vram_can_allocate(m->ctx, R.bytes) ? -1 : recycle_candidate(m, li);
  if (v >= 0) {
    if ((rc = adopt_buffers(m, (uint32_t)v, li))) return rc;
  } else {
    rc = make_headroom(m, R.bytes);
    if (rc == RF_ERR_BUDGET)
      return set_error(RF_ERR_BUDGET,
                       "insufficient memory: layer %u needs %llu bytes, %llu of %llu in use after evicting every "
                       "cached layer",
                       li, (unsigned long long)R.bytes, (unsigned long long)m->ctx->ledger.used(),
                       (unsigned long long)m->ctx->ledger.total());
    if (rc) return rc;
    for (int i = 0; i < 12; ++i) {
      DevTensor* x = t[i];
      if (!x->streamed()) continue;
      const std::string charge = unit_charge(m, li, i);
      void* d = nullptr;
      rc = vram_alloc(m->ctx, charge, x->nbytes, &d);
      if (rc) return rollback(rc);
      x->d = d;
      x->charge = charge;
    }
  }
  // The copies go to whichever of the two upload streams has been given
  // fewer of this layer's bytes: each copy carries a fixed setup cost
  // (about 40 us between back-to-back copies on one stream, measured), which
  // the other stream's transfer hides.
  bool sourced = false;
  uint64_t given[2] = {0, 0};
  for (int i = 0; i < 12; ++i) {
    DevTensor* x = t[i];
    if (!x->streamed()) continue;
    if (x->src) {
      sourced = true;
      continue;
    }
    const int k = given[1] < given[0] ? 1 : 0;
    given[k] += x->nbytes;
    const hipError_t e = hipMemcpyAsync(x->d, x->host, x->nbytes, hipMemcpyHostToDevice, k ? cs2 : cs);
    if (e != hipSuccess) return rollback(hip_error(e, "layer upload"));
    m->st_uploaded += x->nbytes;
  }
  if (sourced && (rc = read_layer_sources(m, li, t, cs))) return rollback(rc);
  hipError_t e = hipSuccess;
  if (given[1]) {  // the second stream's copies join the first before the layer counts as uploaded
    e = hipEventRecord(m->up2, cs2);
    if (e == hipSuccess) e = hipStreamWaitEvent(cs, m->up2, 0);
  }
  if (e == hipSuccess) e = hipEventRecord(R.uploaded, cs);
  if (e == hipSuccess) e = hipEventRecord(R.used, m->ctx->compute);  // not in use yet
  if (e != hipSuccess) return hip_error(e, "hipEventRecord");
  R.state = LAYER_ACTIVE;
  return RF_OK;
}

// A layer about to be computed: a cached one returns to "layer:{i}:" (hit),
// a host-only one is loaded (miss).  With `prefetch` a miss that does not fit
// is skipped instead of failing.
int32_t acquire_layer(rf_model* m, uint32_t li, bool prefetch) {
  LayerRes& R = m->res[li];
  if (R.state == LAYER_ACTIVE || R.state == LAYER_RETIRED) {
    R.state = LAYER_ACTIVE;
    return RF_OK;
  }
  if (R.state == LAYER_CACHED) {
    const int32_t rc = rename_unit(m, li, "cache:", "");
    if (rc) return rc;
    m->lru.remove(li);
    m->cache_used -= R.bytes;
    R.state = LAYER_ACTIVE;
    m->st_hits += 1;
    return RF_OK;
  }
  if (prefetch && !vram_can_allocate(m->ctx, R.bytes) && m->lru.empty() && recycle_candidate(m, li) < 0)
    return RF_OK;
  int32_t rc = load_layer(m, li);
  if (prefetch && rc == RF_ERR_BUDGET) return RF_OK;
  if (rc == RF_OK) m->st_misses += 1;
  return rc;
}

// After the layer's kernels: LayerCache::insert_loaded (rename "layer:{i}:"
// -> "cache:layer:{i}:", evicting LRU layers while over capacity), or, when
// the layer cannot be cached, retire it for release once its kernels end.
int32_t settle_layer(rf_model* m, uint32_t li) {
  LayerRes& R = m->res[li];
  hipError_t e = hipEventRecord(R.used, m->ctx->compute);
  if (e != hipSuccess) return hip_error(e, "hipEventRecord");
  if (R.bytes == 0 || R.bytes > m->cache_cap) {
    R.state = LAYER_RETIRED;
    return RF_OK;
  }
  if (m->cache_policy == 1 && m->cache_used + R.bytes > m->cache_cap && !m->lru.empty() &&
      next_use(m, li) >= next_use(m, pick_victim(m))) {
    R.state = LAYER_RETIRED;  // needed later than every cached layer: not worth an eviction
    return RF_OK;
  }
  int32_t rc = RF_OK;
  while (m->cache_used + R.bytes > m->cache_cap)
    if (!evict_lru(m, &rc) || rc) return rc;
  if ((rc = rename_unit(m, li, "", "cache:"))) return rc;
  R.state = LAYER_CACHED;
  m->lru.push_front(li);
  m->cache_used += R.bytes;
  return RF_OK;
}

// Resolve a GGUF tensor name to its slot and expected shape [ne0, ne1].
int32_t resolve(rf_model* m, const std::string& name, DevTensor** slot, uint64_t* e0, uint64_t* e1,
                std::string* charge) {
  const rf_model_config& c = m->cfg;
  const uint64_t d = c.embedding_length, qd = c.head_count * c.head_dim, kvd = c.head_count_kv * c.head_dim;
  const uint64_t f = c.feed_forward_length;
  if (name == "token_embd.weight") { *slot = &m->token_embd; *e0 = d; *e1 = c.vocab_size; *charge = "persistent:" + name; return RF_OK; }
  if (name == "output_norm.weight") { *slot = &m->output_norm; *e0 = d; *e1 = 1; *charge = "persistent:" + name; return RF_OK; }
  if (name == "output.weight") { *slot = &m->output; *e0 = d; *e1 = c.vocab_size; *charge = "persistent:" + name; return RF_OK; }
  unsigned li = 0;
  char rest[128];
  if (sscanf(name.c_str(), "blk.%u.%127s", &li, rest) == 2 && li < m->layers.size()) {
    Layer& L = m->layers[li];
    const std::string r(rest);
    *charge = "layer:" + std::to_string(li) + ":" + r;
    struct E { const char* n; DevTensor* t; uint64_t a, b; } tab[] = {
        {"attn_norm.weight", &L.attn_norm, d, 1}, {"attn_q.weight", &L.q, d, qd},
        {"attn_k.weight", &L.k, d, kvd},          {"attn_v.weight", &L.v, d, kvd},
        {"attn_output.weight", &L.o, qd, d},      {"ffn_norm.weight", &L.ffn_norm, d, 1},
        {"ffn_gate.weight", &L.gate, d, f},       {"ffn_up.weight", &L.up, d, f},
        {"ffn_down.weight", &L.down, f, d},       {"attn_q.bias", &L.bq, qd, 1},
        {"attn_k.bias", &L.bk, kvd, 1},           {"attn_v.bias", &L.bv, kvd, 1}};
    for (auto& e : tab)
      if (r == e.n) { *slot = e.t; *e0 = e.a; *e1 = e.b; return RF_OK; }
  }
  return set_error(RF_ERR_INVALID, "unknown tensor '%s' for a %llu-layer llama model", name.c_str(),
                   (unsigned long long)c.block_count);
}

bool is_vector_slot(const std::string& name) {
  return name.find("_norm.weight") != std::string::npos || name.find(".bias") != std::string::npos;
}

int32_t check_tensor_shape(rf_model* m, const std::string& name, uint32_t t, uint64_t ne0, uint64_t ne1,
                           uint64_t e0, uint64_t e1, uint64_t* bytes) {
  if (ne0 != e0 || ne1 != e1)
    return set_error(RF_ERR_INVALID, "tensor '%s' has shape [%llu, %llu], expected [%llu, %llu]", name.c_str(),
                     (unsigned long long)ne0, (unsigned long long)ne1, (unsigned long long)e0,
                     (unsigned long long)e1);
  uint64_t qk = 1, bs = 0;
  if (t == T_F32) bs = 4;
  else if (t == T_F16 || t == T_BF16) bs = 2;
  else if (!type_geometry(t, &qk, &bs))
    return set_error(RF_ERR_UNSUPPORTED, "tensor '%s' has unsupported type %s", name.c_str(), type_name(t));
  if (ne0 % qk != 0)
    return set_error(RF_ERR_INVALID, "%s row size %llu not divisible by block size %llu", type_name(t),
                     (unsigned long long)ne0, (unsigned long long)qk);
  if (is_vector_slot(name) && t != T_F32 && t != T_F16 && t != T_BF16)
    return set_error(RF_ERR_UNSUPPORTED, "tensor '%s' must be F32/F16/BF16, got %s", name.c_str(), type_name(t));
  *bytes = ne0 / qk * bs * ne1;
  (void)m;
  return RF_OK;
}

// Upload (or synthesize) one tensor.  F16/BF16 payloads are decoded to F32 on
// the device, as TensorData decodes them at load (core/src/tensor.rs:460-521).
// The matrices the decode step multiplies (everything but the embedding, the
// norms and the biases).
bool is_projection(const std::string& name) {
  if (name == "output.weight") return true;
  static const char* sfx[] = {".attn_q.weight", ".attn_k.weight", ".attn_v.weight", ".attn_output.weight",
                              ".ffn_gate.weight", ".ffn_up.weight", ".ffn_down.weight"};
  if (name.rfind("blk.", 0) != 0) return false;
  for (const char* x : sfx) {
    const size_t n = strlen(x);
    if (name.size() > n && name.compare(name.size() - n, n, x) == 0) return true;
  }
  return false;
}

int32_t fill_pinned(rf_model* m, const std::string& name, uint32_t t, uint64_t ne0, uint64_t ne1, uint64_t bytes,
                    const void* host, bool synth, uint64_t seed, double mul, float constant, bool pack,
                    unsigned flags, void** out);

// A block tensor of a streaming model: its device-layout bytes go to pinned
// host memory (packed / widened as on the device path); the layer is uploaded
// when a forward pass needs it.
int32_t install_streamed(rf_model* m, const std::string& name, DevTensor* slot, uint32_t t, uint64_t ne0,
                         uint64_t ne1, uint64_t bytes, const void* host, bool synth, uint64_t seed, double mul,
                         float constant) {
  unsigned li = 0;
  if (sscanf(name.c_str(), "blk.%u.", &li) != 1 || li >= m->layers.size())
    return set_error(RF_ERR_INVALID, "unknown tensor '%s'", name.c_str());
  reset_graph(m);
  int32_t rc = layer_free(m, li);  // a resident copy of the layer is stale now
  if (rc) return rc;
  const bool widen = (t == T_F16 || t == T_BF16);
  const bool pack = g_pack_weights && is_projection(name) && plan_packed(t, ne0).ok;
  const uint64_t fbytes = widen ? ne0 * ne1 * 4 : bytes;
  void* pin = nullptr;
  rc = fill_pinned(m, name, t, ne0, ne1, bytes, host, synth, seed, mul, constant, pack, hipHostMallocDefault, &pin);
  if (rc) return rc;
  if (slot->host) hipHostFree(slot->host);
  slot->src = false;
  slot->type = widen ? T_F32 : t;
  slot->ne0 = ne0;
  slot->ne1 = ne1;
  slot->nbytes = fbytes;
  slot->d = nullptr;
  slot->charge.clear();
  slot->packed = pack;
  slot->host = pin;
  update_layer_bytes(m, li);
  return RF_OK;
}

// The device-layout bytes of a tensor (packed, widened, or as given) in new
// pinned host memory allocated with `flags`: synthesized on the device and
// copied back, widened or packed on the host, or copied.
int32_t fill_pinned(rf_model* m, const std::string& name, uint32_t t, uint64_t ne0, uint64_t ne1, uint64_t bytes,
                    const void* host, bool synth, uint64_t seed, double mul, float constant, bool pack,
                    unsigned flags, void** out) {
  rf_ctx* ctx = m->ctx;
  const bool widen = (t == T_F16 || t == T_BF16);
  const uint64_t fbytes = widen ? ne0 * ne1 * 4 : bytes;
  int32_t rc = RF_OK;
  void* pin = nullptr;
  hipError_t e = hipHostMalloc(&pin, fbytes, flags);
  if (e != hipSuccess) return hip_error(e, "hipHostMalloc");
  if (synth) {
    void *tmp = nullptr, *tmp2 = nullptr;
    rc = vram_alloc(ctx, "tmp:synth:" + name, bytes, &tmp);
    if (rc == RF_OK && pack) rc = vram_alloc(ctx, "tmp:pack:" + name, bytes, &tmp2);
    if (rc == RF_OK) {
      uint64_t qk = 1, bs = 4;
      type_geometry(t, &qk, &bs);
      const uint64_t nblk = t == T_F32 ? ne0 * ne1 : ne0 / qk * ne1;
      if (t == T_F32 && !std::isnan(constant)) e = launch_fill(static_cast<float*>(tmp), constant, ne0 * ne1, ctx->compute);
      else e = launch_synth(t, seed, 0, nblk, mul, tmp, ctx->compute);
      if (e == hipSuccess && pack) e = launch_pack(t, tmp, tmp2, ne1, ne0, ctx->compute);
      if (e == hipSuccess) e = hipMemcpyAsync(pin, pack ? tmp2 : tmp, fbytes, hipMemcpyDeviceToHost, ctx->compute);
      if (e == hipSuccess) e = hipStreamSynchronize(ctx->compute);
      if (e != hipSuccess) rc = hip_error(e, "tensor synthesis");
    }
    if (tmp2) vram_release(ctx, "tmp:pack:" + name);
    if (tmp) vram_release(ctx, "tmp:synth:" + name);
  } else if (widen) {
    const uint16_t* h = static_cast<const uint16_t*>(host);
    float* o = static_cast<float*>(pin);
    for (uint64_t i = 0; i < ne0 * ne1; ++i) {
      if (t == T_F16) {
        o[i] = host_half_to_float(h[i]);
      } else {
        const uint32_t b = (uint32_t)h[i] << 16;
        memcpy(&o[i], &b, 4);
      }
    }
  } else if (pack) {
    host_pack(t, static_cast<const uint8_t*>(host), ne1, ne0, static_cast<uint8_t*>(pin));
  } else {
    memcpy(pin, host, bytes);
  }
  if (rc) {
    hipHostFree(pin);
    return rc;
  }
  *out = pin;
  return RF_OK;
}

// An embedding or output projection of a streaming model that the policy
// streams (streamed_matvec_into / get_embedding_into, persistent.rs:60-463):
// its device-layout bytes stay in mapped pinned host memory and the kernels
// read them there, one row per token for the embedding and every row for the
// logits, so no device memory is charged for it.
int32_t install_persistent_streamed(rf_model* m, const std::string& name, DevTensor* slot, uint32_t t,
                                    uint64_t ne0, uint64_t ne1, uint64_t bytes, const void* host, bool synth,
                                    uint64_t seed, double mul, float constant) {
  const bool widen = (t == T_F16 || t == T_BF16);
  const bool pack = g_pack_weights && is_projection(name) && plan_packed(t, ne0).ok;
  void* pin = nullptr;
  int32_t rc = fill_pinned(m, name, t, ne0, ne1, bytes, host, synth, seed, mul, constant, pack, hipHostMallocMapped,
                           &pin);
  if (rc) return rc;
  void* dptr = nullptr;
  const hipError_t e = hipHostGetDevicePointer(&dptr, pin, 0);
  if (e != hipSuccess) {
    hipHostFree(pin);
    return hip_error(e, "hipHostGetDevicePointer");
  }
  rc = drop_tensor(m, *slot);
  if (rc) {
    hipHostFree(pin);
    return rc;
  }
  slot->src = false;
  slot->type = widen ? T_F32 : t;
  slot->ne0 = ne0;
  slot->ne1 = ne1;
  slot->nbytes = widen ? ne0 * ne1 * 4 : bytes;
  slot->d = dptr;
  slot->charge.clear();
  slot->packed = pack;
  slot->host = pin;
  return RF_OK;
}

int32_t install(rf_model* m, const char* cname, uint32_t t, uint64_t ne0, uint64_t ne1, const void* host,
                uint64_t nbytes, bool synth, uint64_t seed, double mul, float constant) {
  if (!m || !cname) return set_error(RF_ERR_INVALID, "null model or tensor name");
  const std::string name(cname);
  DevTensor* slot = nullptr;
  uint64_t e0 = 0, e1 = 0, bytes = 0;
  std::string charge;
  int32_t rc = resolve(m, name, &slot, &e0, &e1, &charge);
  if (rc) return rc;
  rc = check_tensor_shape(m, name, t, ne0, ne1, e0, e1, &bytes);
  if (rc) return rc;
  if (!synth && nbytes < bytes)
    return set_error(RF_ERR_INVALID, "tensor '%s' truncated: expected %llu bytes, got %llu", name.c_str(),
                     (unsigned long long)bytes, (unsigned long long)nbytes);
  if (synth && (t == T_F16 || t == T_BF16))
    return set_error(RF_ERR_UNSUPPORTED, "synthetic generator does not emit %s", type_name(t));
  if (m->streaming && name.rfind("blk.", 0) == 0)
    return install_streamed(m, name, slot, t, ne0, ne1, bytes, host, synth, seed, mul, constant);
  if (m->streaming && (name == "token_embd.weight" || name == "output.weight")) {
    // should_keep_resident (persistent.rs:466-470): resident when its device
    // bytes are at most a quarter of the budget; policy 3 streams the
    // embedding table regardless (its gather reads one row per token) and
    // applies that rule to the output projection
    const uint64_t resident = (t == T_F16 || t == T_BF16) ? ne0 * ne1 * 4 : bytes;
    const bool embd = name == "token_embd.weight";
    const int pol = m->persistent_policy;
    const bool by_rule = pol == 0 || (pol == 3 && !embd);
    const bool stream = pol == 1 || (pol == 3 && embd) || (by_rule && resident > m->ctx->ledger.total() / 4);
    if (stream) {
      reset_graph(m);
      return install_persistent_streamed(m, name, slot, t, ne0, ne1, bytes, host, synth, seed, mul, constant);
    }
  }
  rf_ctx* ctx = m->ctx;
  reset_graph(m);
  hipError_t e = hipStreamSynchronize(ctx->compute);
  if (e != hipSuccess) return hip_error(e, "hipStreamSynchronize");
  rc = drop_tensor(m, *slot);
  if (rc) return rc;
  const bool widen = (t == T_F16 || t == T_BF16);
  const uint64_t final_bytes = widen ? ne0 * ne1 * 4 : bytes;
  void* d = nullptr;
  rc = charge_alloc(m, charge, final_bytes, &d);
  if (rc) return rc;
  // Any failure from here on releases the new buffer and its charge (the slot
  // is already empty): the model is left as if the call had not been made
  // but for the dropped old tensor, and the same call can be retried.
  auto fail = [&](int32_t code) {
    hipStreamSynchronize(ctx->compute);  // nothing may still write into d
    release_charge(m, charge);
    return code;
  };
  if (synth) {
    uint64_t qk = 1, bs = 4;
    type_geometry(t, &qk, &bs);
    const uint64_t nblk = t == T_F32 ? ne0 * ne1 : ne0 / qk * ne1;
    if (t == T_F32 && !std::isnan(constant)) e = launch_fill(static_cast<float*>(d), constant, ne0 * ne1, ctx->compute);
    else e = launch_synth(t, seed, 0, nblk, mul, d, ctx->compute);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->compute);
    if (e != hipSuccess) return fail(hip_error(e, "tensor synthesis"));
  } else if (widen) {
    void* tmp = nullptr;
    rc = vram_alloc(ctx, "tmp:load:" + name, bytes, &tmp);
    if (rc) return fail(rc);
    rc = staged_upload(ctx, tmp, host, bytes);
    if (rc == RF_OK) {
      e = launch_dequant_rows(t, tmp, ne0, ne1, static_cast<float*>(d), nullptr, 0, ctx->compute);
      if (e == hipSuccess) e = hipStreamSynchronize(ctx->compute);
      if (e != hipSuccess) rc = hip_error(e, "F16/BF16 widen");
    }
    const int32_t rc2 = vram_release(ctx, "tmp:load:" + name);
    if (rc) return fail(rc);
    if (rc2) return fail(rc2);
  } else {
    rc = staged_upload(ctx, d, host, bytes);
    if (rc) return fail(rc);
  }
  bool packed = false;
  if (g_pack_weights && is_projection(name) && plan_packed(t, ne0).ok) {
    // GGUF -> packed through a temporary copy (install time only)
    void* tmp = nullptr;
    rc = vram_alloc(ctx, "tmp:pack:" + name, bytes, &tmp);
    if (rc) return fail(rc);
    e = launch_pack(t, d, tmp, ne1, ne0, ctx->compute);
    if (e == hipSuccess) e = hipMemcpyAsync(d, tmp, bytes, hipMemcpyDeviceToDevice, ctx->compute);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->compute);
    const int32_t rc2 = vram_release(ctx, "tmp:pack:" + name);
    if (e != hipSuccess) return fail(hip_error(e, "weight packing"));
    if (rc2) return fail(rc2);
    packed = true;
  }
  slot->type = widen ? T_F32 : t;
  slot->ne0 = ne0;
  slot->ne1 = ne1;
  slot->nbytes = final_bytes;
  slot->d = d;
  slot->charge = charge;
  slot->packed = packed;
  return RF_OK;
}

int32_t check_ready(rf_model* m) {
  if (!m->token_embd.present()) return set_error(RF_ERR_INVALID, "model tensor 'token_embd.weight' not loaded");
  if (!m->output_norm.present()) return set_error(RF_ERR_INVALID, "model tensor 'output_norm.weight' not loaded");
  for (size_t i = 0; i < m->layers.size(); ++i) {
    Layer& L = m->layers[i];
    const DevTensor* req[] = {&L.attn_norm, &L.q, &L.k, &L.v, &L.o, &L.ffn_norm, &L.gate, &L.up, &L.down};
    for (const DevTensor* t : req)
      if (!t->present()) return set_error(RF_ERR_INVALID, "layer %zu is missing a required tensor", i);
    const int nb = L.bq.present() + L.bk.present() + L.bv.present();
    if (nb != 0 && nb != 3)
      return set_error(RF_ERR_INVALID, "internal error: incomplete Q/K/V bias set survived load of layer %zu", i);
  }
  return RF_OK;
}

#define RF_LAUNCH(expr, what)                               \
  do {                                                      \
    hipError_t _e = (expr);                                 \
    if (_e != hipSuccess) return hip_error(_e, what);       \
  } while (0)

// One output segment of a model matvec: a weight tensor (and its "up" pair
// for SiLU(gate)*up), the output and the residual input.
struct MSeg {
  const DevTensor* w;
  const DevTensor* w_up;
  float* y;
  const float* res;
  uint64_t rows;
};

// A fused matvec launch over segments of one type and layout: the packed
// kernel for packed tensors; else the GGUF-layout kernels, or — when a row
// does not fit the LDS tile (very wide F32 rows) — the same computation as
// separate kernels: RMSNorm into xnorm, rowwise matvec, then the residual /
// SiLU*up epilogue.
hipError_t fused_matvec_impl(rf_model* m, const MSeg* ms, int nseg, const float* x, const float* norm_w,
                             uint64_t in_dim, int epi);

// advance: the device position, incremented once by the launch (the packed
// kernel does it; the GGUF-layout path adds the one-thread kernel).
hipError_t fused_matvec(rf_model* m, const MSeg* ms, int nseg, const float* x, const float* norm_w, uint64_t in_dim,
                        int epi, int32_t* advance = nullptr) {
  hipStream_t st = m->ctx->compute;
  const uint32_t t = ms[0].w->type;
  if (ms[0].w->packed) {
    PkSegDesc ps[3];
    for (int i = 0; i < nseg; ++i)
      ps[i] = PkSegDesc{ms[i].w->d, ms[i].w_up ? ms[i].w_up->d : nullptr, ms[i].w->ne1, 0, ms[i].rows, ms[i].y,
                        ms[i].res};
    return launch_matvec_packed(t, ps, nseg, x, norm_w, m->cfg.rms_eps, in_dim, epi, st, advance);
  }
  hipError_t e = fused_matvec_impl(m, ms, nseg, x, norm_w, in_dim, epi);
  if (e == hipSuccess && advance) e = launch_advance_pos(advance, st);
  return e;
}

hipError_t fused_matvec_impl(rf_model* m, const MSeg* ms, int nseg, const float* x, const float* norm_w,
                             uint64_t in_dim, int epi) {
  hipStream_t st = m->ctx->compute;
  const uint32_t t = ms[0].w->type;
  MvSegDesc segs[3];
  for (int i = 0; i < nseg; ++i)
    segs[i] = MvSegDesc{ms[i].w->d, ms[i].w_up ? ms[i].w_up->d : nullptr, ms[i].y, ms[i].res, ms[i].rows};
  const bool x_vec = (reinterpret_cast<uintptr_t>(x) & 15u) == 0 && (reinterpret_cast<uintptr_t>(norm_w) & 15u) == 0;
  if (plan_matvec(t, in_dim, epi == EPI_SWIGLU).tiled && x_vec)
    return launch_matvec_segments(t, segs, nseg, x, norm_w, m->cfg.rms_eps, in_dim, epi, st);
  hipError_t e = hipSuccess;
  const float* xe = x;
  if (norm_w) {
    e = launch_rmsnorm(x, norm_w, in_dim, m->cfg.rms_eps, m->xnorm, st);
    if (e != hipSuccess) return e;
    xe = m->xnorm;
  }
  for (int i = 0; i < nseg && e == hipSuccess; ++i) {
    const MvSegDesc& s = segs[i];
    if (epi == EPI_STORE) {
      e = launch_matvec_segments(t, &s, 1, xe, nullptr, 0.f, in_dim, EPI_STORE, st);
    } else if (epi == EPI_RESIDUAL) {
      MvSegDesc tmp{s.w, nullptr, m->mvtmp, nullptr, s.rows};
      e = launch_matvec_segments(t, &tmp, 1, xe, nullptr, 0.f, in_dim, EPI_STORE, st);
      if (e == hipSuccess) e = launch_binary(BIN_ADD, s.res, m->mvtmp, s.rows, s.y, st);
    } else {
      MvSegDesc g{s.w, nullptr, s.y, nullptr, s.rows}, u{s.w_up, nullptr, m->mvtmp, nullptr, s.rows};
      e = launch_matvec_segments(t, &g, 1, xe, nullptr, 0.f, in_dim, EPI_STORE, st);
      if (e == hipSuccess) e = launch_matvec_segments(t, &u, 1, xe, nullptr, 0.f, in_dim, EPI_STORE, st);
      if (e == hipSuccess) e = launch_binary(BIN_SWIGLU, s.y, m->mvtmp, s.rows, s.y, st);
    }
  }
  return e;
}

// The five launch groups of one transformer block (model_executor.rs:102-236).
// 1. attention RMSNorm + Q/K/V projections (+ bias), segments grouped by type.
int32_t enqueue_qkv(rf_model* m, size_t li) {
  const rf_model_config& c = m->cfg;
  Layer& L = m->layers[li];
  hipStream_t st = m->ctx->compute;
  const uint64_t d = c.embedding_length, hd = c.head_dim, qd = c.head_count * hd, kvd = c.head_count_kv * hd;
  const float* attn_norm = static_cast<const float*>(L.attn_norm.d);
  const DevTensor* qkv[3] = {&L.q, &L.k, &L.v};
  float* outs[3] = {m->q, m->k, m->v};
  const uint64_t rows[3] = {qd, kvd, kvd};
  int i = 0;
  while (i < 3) {  // consecutive projections of one type and layout share a launch
    MSeg segs[3];
    int n = 0;
    const uint32_t t = qkv[i]->type;
    const bool pk = qkv[i]->packed;
    while (i < 3 && qkv[i]->type == t && qkv[i]->packed == pk) {
      segs[n++] = MSeg{qkv[i], nullptr, outs[i], nullptr, rows[i]};
      ++i;
    }
    RF_LAUNCH(fused_matvec(m, segs, n, m->hidden, attn_norm, d, EPI_STORE), "qkv matvec");
  }
  if (L.bq.present()) {
    RF_LAUNCH(launch_bias_add(m->q, static_cast<const float*>(L.bq.d), qd, st), "bias");
    RF_LAUNCH(launch_bias_add(m->k, static_cast<const float*>(L.bk.d), kvd, st), "bias");
    RF_LAUNCH(launch_bias_add(m->v, static_cast<const float*>(L.bv.d), kvd, st), "bias");
  }
  return RF_OK;
}

// Attention launch regime of the step at position pos (attention_regime with
// the KV capacity as the longest context): each regime is a decode graph of
// its own, so the launch shape is fixed within one.  The any-shape kernel has
// a single shape.
int attn_regime(const rf_model* m, uint64_t pos) {
  if (!m->attn_fast) return 0;
  return attention_regime(pos + 1, (uint32_t)m->cfg.head_count, (uint32_t)m->cfg.head_count_kv, m->kv_max);
}

// Whether layer li's o-projection merges the attention's chunk records
// itself (matvec_packed's merged-x launch), which saves the merge launch:
// the regimes that split per query head (at most 8 chunks) and packed
// Q8_0 / Q4_0 / Q4_K o-projections whose rows take the single-step launch
// (q_heads * head_dim up to 4096).  rf_tune_attention_merge switches it off.
static int g_oproj_merge = 1;
static hipError_t oproj_merges(const rf_model* m, size_t li, const AttnShape& sh, bool* merge) {
  *merge = false;
  if (!g_oproj_merge || !m->attn_fast || !sh.per_q || sh.nsplit < 2) return hipSuccess;
  const rf_model_config& c = m->cfg;
  const Layer& L = m->layers[li];
  if (!L.o.packed) return hipSuccess;
  const hipError_t e = pk_merge_supported(L.o.type, c.head_count * c.head_dim, c.embedding_length, sh.nsplit,
                                          (uint32_t)c.head_count, (uint32_t)c.head_dim, m->ctx->compute);
  if (e == hipErrorNotSupported) return hipSuccess;
  *merge = e == hipSuccess;
  return e;
}

// 2. RoPE + attention + K/V cache write.
int32_t enqueue_attention(rf_model* m, size_t li) {
  const rf_model_config& c = m->cfg;
  hipStream_t st = m->ctx->compute;
  const uint64_t hd = c.head_dim, kvd = c.head_count_kv * hd;
  float* kc = m->k_cache + li * m->kv_cap * kvd;
  float* vc = m->v_cache + li * m->kv_cap * kvd;
  AttnArgs a{};
  a.q = m->q; a.k_hist = kc; a.v_hist = vc; a.k_cur = m->k; a.v_cur = m->v; a.out = m->attn_out;
  a.ws = m->attn_ws; a.rope = m->rope; a.k_store = kc; a.v_store = vc; a.d_pos = m->d_pos;
  a.qh = (uint32_t)c.head_count; a.kvh = (uint32_t)c.head_count_kv; a.hd = (uint32_t)hd;
  // the position this step processes picks the shape
  const AttnShape sh = attention_regime_shape(attn_regime(m, m->seq_len), a.qh, a.kvh, m->kv_max);
  a.per_q = sh.per_q; a.nsplit = sh.nsplit; a.waves = sh.waves;
  m->oproj_merge = false;
  bool merge = false;
  RF_LAUNCH(oproj_merges(m, li, sh, &merge), "attention (o-projection merge plan)");
  a.defer_merge = merge ? 1u : 0u;
  a.denom = sqrtf((float)hd);
  RF_LAUNCH(m->attn_fast ? launch_attention(a, st) : launch_attention_naive(a, st), "attention");
  m->oproj_merge = merge;  // only once the launch that leaves the chunk records succeeded
  return RF_OK;
}

// 3. o-proj + residual (merging the attention's chunk records into its x
// when oproj_merges).
int32_t enqueue_oproj(rf_model* m, size_t li) {
  const rf_model_config& c = m->cfg;
  Layer& L = m->layers[li];
  const uint64_t d = c.embedding_length, qd = c.head_count * c.head_dim;
  if (m->oproj_merge) {  // the attention just enqueued left its chunk records
    m->oproj_merge = false;
    const AttnShape sh = attention_regime_shape(attn_regime(m, m->seq_len), (uint32_t)c.head_count,
                                                (uint32_t)c.head_count_kv, m->kv_max);
    const PkMerge mg{m->attn_ws, m->d_pos, sh.nsplit, (uint32_t)c.head_count, (uint32_t)c.head_dim};
    PkSegDesc ps{L.o.d, nullptr, L.o.ne1, 0, d, m->hidden, m->hidden};
    RF_LAUNCH(launch_matvec_packed(L.o.type, &ps, 1, m->attn_out, nullptr, 0.f, qd, EPI_RESIDUAL, m->ctx->compute,
                                   nullptr, &mg),
              "o-proj (merging attention chunks)");
    return RF_OK;
  }
  MSeg s{&L.o, nullptr, m->hidden, m->hidden, d};
  RF_LAUNCH(fused_matvec(m, &s, 1, m->attn_out, nullptr, qd, EPI_RESIDUAL), "o-proj");
  return RF_OK;
}

// 4. ffn RMSNorm + gate/up + SiLU(gate) * up.
int32_t enqueue_gateup(rf_model* m, size_t li) {
  const rf_model_config& c = m->cfg;
  Layer& L = m->layers[li];
  hipStream_t st = m->ctx->compute;
  const uint64_t d = c.embedding_length, f = c.feed_forward_length;
  const float* ffn_norm = static_cast<const float*>(L.ffn_norm.d);
  if (L.gate.type == L.up.type && L.gate.packed == L.up.packed) {
    MSeg s{&L.gate, &L.up, m->act, nullptr, f};
    RF_LAUNCH(fused_matvec(m, &s, 1, m->hidden, ffn_norm, d, EPI_SWIGLU), "gate/up");
  } else {
    float* up_tmp = m->up_tmp;
    MSeg sg{&L.gate, nullptr, m->act, nullptr, f};
    MSeg su{&L.up, nullptr, up_tmp, nullptr, f};
    RF_LAUNCH(fused_matvec(m, &sg, 1, m->hidden, ffn_norm, d, EPI_STORE), "gate");
    RF_LAUNCH(fused_matvec(m, &su, 1, m->hidden, ffn_norm, d, EPI_STORE), "up");
    RF_LAUNCH(launch_binary(BIN_SWIGLU, m->act, up_tmp, f, m->act, st), "swiglu");
  }
  return RF_OK;
}

// 5. down + residual (advance: the position step that ends a forward pass).
int32_t enqueue_down(rf_model* m, size_t li, int32_t* advance = nullptr) {
  const rf_model_config& c = m->cfg;
  Layer& L = m->layers[li];
  const uint64_t d = c.embedding_length, f = c.feed_forward_length;
  MSeg s{&L.down, nullptr, m->hidden, m->hidden, d};
  RF_LAUNCH(fused_matvec(m, &s, 1, m->act, nullptr, f, EPI_RESIDUAL, advance), "down");
  return RF_OK;
}

// Adds the recorded event pairs to the per-group totals (waits for the
// last one) and frees the pool for reuse.
int32_t prof_collect(rf_model* m) {
  if (m->prof_used == 0) return RF_OK;
  hipError_t e = hipEventSynchronize(m->prof_ev[2 * m->prof_used - 1]);
  for (size_t k = 0; k < m->prof_used && e == hipSuccess; ++k) {
    float ms = 0.f;
    e = hipEventElapsedTime(&ms, m->prof_ev[2 * k], m->prof_ev[2 * k + 1]);
    m->prof_ms[m->prof_kind[k]] += ms;
    m->prof_n[m->prof_kind[k]] += 1;
  }
  m->prof_used = 0;
  return e == hipSuccess ? RF_OK : hip_error(e, "profiler events");
}

// One launch group, bracketed by profiler events when profiling is on
// (ProfileEvent::QuantizedMatvec around each matvec, compute_dispatch.rs:48-56;
// LayerCompute for attention, profile.rs:8-23).
template <typename F>
int32_t prof_group(rf_model* m, int kind, F&& body) {
  if (!m->prof) return body();
  if (m->prof_used * 2 + 2 > m->prof_ev.size()) {
    int32_t rc = prof_collect(m);
    if (rc) return rc;
  }
  const size_t k = m->prof_used;
  hipStream_t st = m->ctx->compute;
  RF_LAUNCH(hipEventRecord(m->prof_ev[2 * k], st), "profiler event");
  const int32_t rc = body();
  if (rc) return rc;
  RF_LAUNCH(hipEventRecord(m->prof_ev[2 * k + 1], st), "profiler event");
  m->prof_kind[k] = kind;
  m->prof_used = k + 1;
  return RF_OK;
}

// The launch groups of part p of a layer split into upl streaming units
// (slot_part): group 0 Q/K/V, attention, o-projection; 1 gate/up; 2 down.
void part_groups(uint32_t upl, uint32_t p, int* g0, int* g1) {
  if (upl == 1) { *g0 = 0; *g1 = 2; }
  else if (upl == 2) { *g0 = p == 0 ? 0 : 1; *g1 = p == 0 ? 0 : 2; }
  else { *g0 = *g1 = (int)p; }
}

int32_t enqueue_layer_groups(rf_model* m, size_t li, int g0, int g1, int32_t* advance = nullptr) {
  int32_t rc;
  for (int g = g0; g <= g1; ++g) {
    if (g == 0) {
      m->oproj_merge = false;
      if ((rc = prof_group(m, 0, [&] { return enqueue_qkv(m, li); }))) return rc;
      if ((rc = prof_group(m, 1, [&] { return enqueue_attention(m, li); }))) return rc;
      if ((rc = prof_group(m, 2, [&] { return enqueue_oproj(m, li); }))) return rc;
    } else if (g == 1) {
      if ((rc = prof_group(m, 3, [&] { return enqueue_gateup(m, li); }))) return rc;
    } else {
      if ((rc = prof_group(m, 4, [&] { return enqueue_down(m, li, advance); }))) return rc;
    }
  }
  return RF_OK;
}

int32_t enqueue_layer(rf_model* m, size_t li, int32_t* advance = nullptr) {
  return enqueue_layer_groups(m, li, 0, 2, advance);
}

// Algorithmic HBM bytes of one launch group of layer li (weights + vectors read
// + vectors written); attention counts the K/V history it reads at `hist`.
uint64_t part_bytes(rf_model* m, int kind, size_t li, uint64_t hist) {
  const rf_model_config& c = m->cfg;
  const uint64_t d = c.embedding_length, hd = c.head_dim, qd = c.head_count * hd, kvd = c.head_count_kv * hd;
  const uint64_t f = c.feed_forward_length, V = c.vocab_size;
  if (kind == RF_KERNEL_LOGITS) {
    const DevTensor& w = m->output.present() ? m->output : m->token_embd;
    return w.nbytes + 4 * (d + d + V);
  }
  Layer& L = m->layers[li];
  switch (kind) {
    case RF_KERNEL_QKV: return L.q.nbytes + L.k.nbytes + L.v.nbytes + 4 * (d + d + qd + 2 * kvd);
    case RF_KERNEL_ATTENTION: return 4 * (2 * hist * kvd + 2 * qd + 2 * kvd) + 2 * 4 * kvd;
    case RF_KERNEL_OPROJ: return L.o.nbytes + 4 * (qd + 2 * d);
    case RF_KERNEL_GATEUP: return L.gate.nbytes + L.up.nbytes + 4 * (2 * d + f);
    case RF_KERNEL_DOWN: return L.down.nbytes + 4 * (f + 2 * d);
    default: return 0;
  }
}

// Layer li of a streamed pass split into upl units (unit upl li + p is part
// p).  Each unit is acquired (a hit, or loaded if its upload was not started
// yet), the next unit's upload started, and part p's kernels wait for unit p
// only.  All the layer's units are settled after its last part (the
// feed-forward kernels read the feed-forward norm, which the first unit
// holds).  With a byte source, reads run on this thread between the parts,
// and the worker reads the next host-only unit meanwhile.  `part(p)` enqueues
// part p's kernels.
template <class Part>
int32_t forward_layer_units(rf_model* m, uint32_t li, Part part) {
  hipStream_t st = m->ctx->compute;
  const uint32_t k = m->upl, first = k * li, nu = unit_count(m);
  const bool read_after = m->reader != nullptr;
  int32_t rc;
  for (uint32_t p = 0; p < k; ++p) {
    const uint32_t u = first + p;
    m->cur_layer = u;
    if ((rc = acquire_layer(m, u, false))) return abort_pass(m, rc);
    if (!read_after && u + 1 < nu && (rc = acquire_layer(m, u + 1, true))) return abort_pass(m, rc);
    RF_LAUNCH(hipStreamWaitEvent(st, m->res[u].uploaded, 0), "wait for layer upload");
    if ((rc = part(p))) return abort_pass(m, rc);
  }
  for (uint32_t p = 0; p < k; ++p)
    if ((rc = settle_layer(m, first + p))) return abort_pass(m, rc);
  const uint32_t next = first + k;
  if (read_after && next < nu && (rc = acquire_layer(m, next, true))) return abort_pass(m, rc);
  if (read_after && m->ra.on) {
    const int64_t nx = next_read_layer(m, next + 1);
    if (nx >= 0) ra_post(m, (uint32_t)nx);
  }
  return RF_OK;
}

// Embedding of *d_token (unless the caller's argmax already decoded it into
// the hidden state), all layers, position advance (inside the last layer's
// down projection).
int32_t enqueue_forward(rf_model* m, bool embed = true) {
  hipStream_t st = m->ctx->compute;
  const rf_model_config& c = m->cfg;
  if (embed)
    RF_LAUNCH(launch_dequant_rows(m->token_embd.type, m->token_embd.d, c.embedding_length, 1, m->hidden, m->d_token,
                                  c.vocab_size, st),
              "embedding");
  const uint32_t nl = (uint32_t)m->layers.size();
  if (m->streaming && m->upl > 1) {
    for (uint32_t li = 0; li < nl; ++li) {
      const int32_t rc = forward_layer_units(m, li, [&](uint32_t p) {
        int g0, g1;
        part_groups(m->upl, p, &g0, &g1);
        return enqueue_layer_groups(m, li, g0, g1, g1 == 2 && li + 1 == nl ? m->d_pos : nullptr);
      });
      if (rc) return rc;
    }
    const int32_t rc = release_retired(m);
    if (rc) return rc;
    if (nl == 0) RF_LAUNCH(launch_advance_pos(m->d_pos, st), "advance position");
    return RF_OK;
  }
  for (uint32_t li = 0; li < nl; ++li) {
    int32_t rc;
    m->cur_layer = li;
    // A byte source's reads run on this thread: the next layer is read once
    // this layer's kernels are queued, so the device computes meanwhile.
    const bool read_after = m->streaming && m->reader != nullptr;
    if (m->streaming) {
      // this layer resident (hit or load), the next one's upload started so it
      // overlaps this layer's kernels, then the kernels wait for the upload
      if ((rc = acquire_layer(m, li, false))) return abort_pass(m, rc);
      if (!read_after && li + 1 < nl && (rc = acquire_layer(m, li + 1, true))) return abort_pass(m, rc);
      RF_LAUNCH(hipStreamWaitEvent(st, m->res[li].uploaded, 0), "wait for layer upload");
    }
    if ((rc = enqueue_layer(m, li, li + 1 == nl ? m->d_pos : nullptr))) return m->streaming ? abort_pass(m, rc) : rc;
    if (m->streaming && (rc = settle_layer(m, li))) return abort_pass(m, rc);
    if (read_after && li + 1 < nl && (rc = acquire_layer(m, li + 1, true))) return abort_pass(m, rc);
    if (read_after && m->ra.on) {  // the worker reads the next host-only layer meanwhile
      const int64_t nx = next_read_layer(m, li + 2);
      if (nx >= 0) ra_post(m, (uint32_t)nx);
    }
  }
  if (m->streaming) {
    int32_t rc = release_retired(m);  // release_layer for layers the cache did not take
    if (rc) return rc;
  }
  if (nl == 0) RF_LAUNCH(launch_advance_pos(m->d_pos, st), "advance position");
  return RF_OK;
}

// Output norm + output projection (or tied embedding) into m->logits.
int32_t enqueue_logits(rf_model* m) {
  const rf_model_config& c = m->cfg;
  const DevTensor& w = m->output.present() ? m->output : m->token_embd;
  MSeg s{&w, nullptr, m->logits, nullptr, c.vocab_size};
  return prof_group(m, 5, [&]() -> int32_t {
    RF_LAUNCH(fused_matvec(m, &s, 1, m->hidden, static_cast<const float*>(m->output_norm.d), c.embedding_length,
                           EPI_STORE),
              "logits");
    return RF_OK;
  });
}

// One decode step: logits -> argmax (token stored at ring[pos]) with the
// chosen token's embedding row decoded by the same kernel -> layers.
int32_t enqueue_decode_step(rf_model* m);

// The host side of one decode step with no launch (g_plan_only): every
// launcher's one-time kernel setup for this step's shapes (dynamic LDS,
// occupancy) runs here, before the step is captured; inside the capture
// such setup is refused (setup_outside_capture).
int32_t plan_decode_step(rf_model* m) {
  g_plan_only = true;
  const int32_t rc = enqueue_decode_step(m);
  g_plan_only = false;
  m->oproj_merge = false;
  return rc;
}

int32_t enqueue_decode_step(rf_model* m) {
  int32_t rc = enqueue_logits(m);
  if (rc) return rc;
  RF_LAUNCH(launch_argmax_embed(m->logits, m->cfg.vocab_size, m->d_token, m->amax_val, m->amax_idx, m->d_ring,
                                m->d_pos, m->token_embd.type, m->token_embd.d, m->cfg.embedding_length, m->hidden,
                                m->ctx->compute),
            "argmax");
  return enqueue_forward(m, false);
}

int32_t sync(rf_model* m) {
  hipError_t e = hipStreamSynchronize(m->ctx->compute);
  return e == hipSuccess ? RF_OK : hip_error(e, "hipStreamSynchronize");
}

int32_t forward_token(rf_model* m, uint32_t token, uint64_t pos) {
  if (pos != m->seq_len)
    return set_error(RF_ERR_INVALID, "KV position/history mismatch: position %llu requires cache history %llu, got %llu",
                     (unsigned long long)pos, (unsigned long long)pos, (unsigned long long)m->seq_len);
  if (token >= m->cfg.vocab_size)
    return set_error(RF_ERR_INVALID, "token_id %u out of bounds for embedding with %llu rows", token,
                     (unsigned long long)m->cfg.vocab_size);
  int32_t rc = check_ready(m);
  if (rc) return rc;
  if ((rc = ensure_kv(m, m->seq_len + 1))) return rc;
  RF_LAUNCH(launch_set_u32(m->d_token, token, m->ctx->compute), "set token");
  rc = enqueue_forward(m);
  if (rc) return rc;
  m->seq_len += 1;
  return RF_OK;
}

// ---------------------------------------------------------------- prefill
// A chunk of up to MM_MAX_TOKENS prompt tokens through one layer
// (model_executor.rs:102-236 for each token): the projections as GEMMs over
// the chunk (rf_prefill.hip), RMSNorm per token, RoPE + K/V cache rows, then
// causal attention of each token over the cache up to its own position.

uint32_t prefill_attn_splits(uint64_t total) {
  const uint64_t n = (total + ATT_PREFILL_CHUNK - 1) / ATT_PREFILL_CHUNK;
  return (uint32_t)(n < 1 ? 1 : n);
}

bool prefill_supported(const rf_model* m) {
  if (!m->attn_fast) return false;
  const uint64_t d = m->cfg.embedding_length, qd = m->cfg.head_count * m->cfg.head_dim, f = m->cfg.feed_forward_length;
  for (const Layer& L : m->layers) {
    const DevTensor* w[] = {&L.q, &L.k, &L.v, &L.o, &L.gate, &L.up, &L.down};
    const uint64_t in[] = {d, d, d, qd, d, d, f};
    for (int i = 0; i < 7; ++i)
      if (!w[i]->packed || !mm_supported(w[i]->type, in[i])) return false;
  }
  return true;
}

int32_t ensure_prefill_ws(rf_model* m) {
  if (m->p_h) return RF_OK;
  const rf_model_config& c = m->cfg;
  const uint64_t T = MM_MAX_TOKENS, d = c.embedding_length, hd = c.head_dim, qd = c.head_count * hd;
  const uint64_t kvd = c.head_count_kv * hd, f = c.feed_forward_length;
  // split-K partials: the largest of the launches a layer makes
  uint64_t part = 0;
  auto take_max = [&](std::initializer_list<uint64_t> rows, uint64_t in) {
    uint64_t r[3] = {0, 0, 0};
    int n = 0;
    for (uint64_t x : rows) r[n++] = x;
    const uint64_t v = mm_part_floats(r, n, in, T);
    if (v > part) part = v;
  };
  take_max({qd, kvd, kvd}, d);
  take_max({qd, kvd}, d);
  take_max({kvd, kvd}, d);
  take_max({qd}, d);
  take_max({kvd}, d);
  take_max({d}, qd);
  take_max({f, f}, d);
  take_max({f}, d);
  take_max({d}, f);
  // chunk records of either prefill attention kernel: tokens x splits of
  // the largest launch (the matrix-core kernel takes more splits for fewer
  // tokens)
  uint64_t recs = 0;
  for (uint64_t nt = 1; nt <= T; ++nt)
    recs = std::max<uint64_t>(recs, nt * std::max<uint64_t>(prefill_attn_splits(m->kv_max),
                                                            prefill_attention_mfma_splits(
                                                                m->kv_max, nt, (uint32_t)c.head_count_kv)));
  const uint64_t att = recs * c.head_count * att_rec((uint32_t)hd);
  const uint64_t sizes[] = {T * d, T * d, T * qd, T * kvd, T * kvd, T * qd, T * qd, T * f, T * f, part, att};
  uint64_t total = 0;
  for (uint64_t n : sizes) total += (n + 63) / 64 * 64;
  const uint64_t bytes = total * 4 + T * 4;
  int32_t rc = RF_OK;
  // a streaming model evicts cached layers to make room, as a KV growth does
  // (ensure_layer_cache_headroom, streaming_model.rs:555-572); when that is
  // not enough, the charge below reports the budget
  if (m->streaming && (rc = make_headroom(m, bytes)) && rc != RF_ERR_BUDGET) return rc;
  void* p = nullptr;
  rc = charge_alloc(m, "tmp:prefill", bytes, &p);
  if (rc) return rc;
  float* base = static_cast<float*>(p);
  float** dst[] = {&m->p_h,  &m->p_xn,  &m->p_q,  &m->p_k,    &m->p_v,  &m->p_qr,
                   &m->p_a,  &m->p_act, &m->p_up, &m->p_part, &m->p_att};
  for (int i = 0; i < 11; ++i) {
    *dst[i] = base;
    base += (sizes[i] + 63) / 64 * 64;
  }
  m->p_tok = reinterpret_cast<uint32_t*>(base);
  m->p_part_floats = part;
  return RF_OK;
}

// A streaming model gives the prefill workspace back after the prompt: its
// charge would otherwise hold VRAM the layer cache fills while decoding.
int32_t release_prefill_ws(rf_model* m) {
  if (!m->p_h) return RF_OK;
  int32_t rc = sync(m);
  if (rc) return rc;
  m->p_h = m->p_xn = m->p_q = m->p_k = m->p_v = m->p_qr = m->p_a = m->p_act = m->p_up = m->p_part = m->p_att = nullptr;
  m->p_tok = nullptr;
  m->p_part_floats = 0;
  return release_charge(m, "tmp:prefill");
}

// normed: p_xn already holds this layer's attention RMSNorm (the previous
// layer's down projection produced it).  next_norm: the next layer's
// attention norm weights, produced with this layer's down projection (null
// for the last layer, and when streaming: the next layer may still be
// uploading).
// Launch groups g0..g1: 0 norm, Q/K/V, RoPE and K/V rows, attention,
// o-projection (with the feed-forward norm); 1 gate/up; 2 down.
int32_t enqueue_prefill_layer(rf_model* m, size_t li, uint64_t pos0, uint64_t nt, bool normed,
                              const float* next_norm, int g0 = 0, int g1 = 2) {
  const rf_model_config& c = m->cfg;
  Layer& L = m->layers[li];
  hipStream_t st = m->ctx->compute;
  const uint64_t d = c.embedding_length, hd = c.head_dim, qd = c.head_count * hd, kvd = c.head_count_kv * hd;
  const uint64_t f = c.feed_forward_length;
  const float eps = c.rms_eps;
  auto mm = [&](const MmSegDesc* segs, int n, uint32_t t, const float* x, uint64_t in, int epi,
                const float* norm_w = nullptr, const MmRope* rope = nullptr) {
    return launch_matmul_packed(t, segs, n, x, in, nt, in, epi, m->p_part, m->p_part_floats, st, norm_w, eps,
                                norm_w ? m->p_xn : nullptr, rope);
  };
  if (g0 <= 0) {
    // 1. attention RMSNorm, Q/K/V (+ bias), consecutive projections of one type per launch
    if (!normed)
      RF_LAUNCH(launch_rmsnorm_rows(m->p_h, static_cast<const float*>(L.attn_norm.d), d, nt, d, eps, m->p_xn, st),
                "prefill attn norm");
    const DevTensor* qkv[3] = {&L.q, &L.k, &L.v};
    const DevTensor* bias[3] = {&L.bq, &L.bk, &L.bv};
    float* outs[3] = {m->p_q, m->p_k, m->p_v};
    const uint64_t rows[3] = {qd, kvd, kvd};
    float* kc = m->k_cache + li * m->kv_cap * kvd;
    float* vc = m->v_cache + li * m->kv_cap * kvd;
    // 2. RoPE of q and k, K/V cache rows pos0 .. pos0 + nt - 1: in the split-K
    // reduce when Q, K and V are one launch (one weight type), else a launch
    // of its own
    const MmRope rope{m->rope, (uint32_t)pos0, (uint32_t)c.head_count, (uint32_t)c.head_count_kv, (uint32_t)hd,
                      m->p_qr, kc, vc};
    const bool fused = L.q.type == L.k.type && L.k.type == L.v.type && hd % 8 == 0;
    for (int i = 0; i < 3;) {
      MmSegDesc segs[3];
      int n = 0;
      const uint32_t t = qkv[i]->type;
      while (i < 3 && qkv[i]->type == t) {
        const float* b = bias[i]->present() ? static_cast<const float*>(bias[i]->d) : nullptr;
        segs[n++] = MmSegDesc{qkv[i]->d, qkv[i]->ne1, 0, rows[i], outs[i], nullptr, b, rows[i]};
        ++i;
      }
      RF_LAUNCH(mm(segs, n, t, m->p_xn, d, EPI_STORE, nullptr, fused ? &rope : nullptr), "prefill qkv");
    }
    if (!fused)
      RF_LAUNCH(launch_rope_kv_rows(m->p_q, m->p_k, m->p_v, m->rope, pos0, nt, (uint32_t)c.head_count,
                                    (uint32_t)c.head_count_kv, (uint32_t)hd, m->p_qr, kc, vc, st),
                "prefill rope");
    // 3. attention of every token over positions 0 .. its own
    AttnArgs a{};
    a.q = m->p_qr; a.k_hist = kc; a.v_hist = vc; a.out = m->p_a; a.ws = m->p_att;
    a.hist = (uint32_t)pos0; a.ntok = (uint32_t)nt;
    a.qh = (uint32_t)c.head_count; a.kvh = (uint32_t)c.head_count_kv; a.hd = (uint32_t)hd;
    // The matrix-core kernel: 16-token tiles x KV heads x position splits.
    // Otherwise the decode split kernel with a token dimension: nt x kvh
    // workgroups, one per KV head (its query heads share each K/V row read)
    // and chunks of up to ATT_MAX_CHUNK positions, so up to 1024 positions
    // need no merge.
    a.per_q = 0;
    a.nsplit = prefill_attention_mfma_supported(a.qh, a.kvh, a.hd, pos0 + nt)
                   ? prefill_attention_mfma_splits(pos0 + nt, nt, a.kvh)
                   : prefill_attn_splits(pos0 + nt);
    a.waves = attention_waves(att_chunk_positions(pos0 + nt, a.nsplit), 0);
    a.denom = sqrtf((float)hd);
    RF_LAUNCH(launch_attention(a, st), "prefill attention");
    // 4. o-proj + residual, with the ffn RMSNorm
    MmSegDesc so{L.o.d, L.o.ne1, 0, d, m->p_h, m->p_h, nullptr, d};
    RF_LAUNCH(mm(&so, 1, L.o.type, m->p_a, qd, EPI_RESIDUAL, static_cast<const float*>(L.ffn_norm.d)),
              "prefill o-proj + ffn norm");
  }
  if (g0 <= 1 && g1 >= 1) {
    // 5. gate/up, SiLU(gate) * up
    MmSegDesc sg[2] = {MmSegDesc{L.gate.d, L.gate.ne1, 0, f, m->p_act, nullptr, nullptr, f},
                       MmSegDesc{L.up.d, L.up.ne1, 0, f, m->p_up, nullptr, nullptr, f}};
    if (L.gate.type == L.up.type) {
      RF_LAUNCH(mm(sg, 2, L.gate.type, m->p_xn, d, EPI_SWIGLU), "prefill gate/up");
    } else {
      RF_LAUNCH(mm(&sg[0], 1, L.gate.type, m->p_xn, d, EPI_STORE), "prefill gate");
      RF_LAUNCH(mm(&sg[1], 1, L.up.type, m->p_xn, d, EPI_STORE), "prefill up");
      RF_LAUNCH(launch_binary(BIN_SWIGLU, m->p_act, m->p_up, nt * f, m->p_act, st), "prefill swiglu");
    }
  }
  if (g1 >= 2) {
    // 6. down + residual (with the next layer's attention RMSNorm)
    MmSegDesc sd{L.down.d, L.down.ne1, 0, d, m->p_h, m->p_h, nullptr, d};
    RF_LAUNCH(mm(&sd, 1, L.down.type, m->p_act, f, EPI_RESIDUAL, next_norm), "prefill down");
  }
  return RF_OK;
}

int32_t prefill_tokens(rf_model* m, const uint32_t* tokens, uint64_t n) {
  if (n == 0) return RF_OK;
  if (n > m->kv_max - m->seq_len) return set_error(RF_ERR_INVALID, "KV cache full");  // seq_len <= kv_cap <= kv_max
  for (uint64_t i = 0; i < n; ++i)
    if (tokens[i] >= m->cfg.vocab_size)
      return set_error(RF_ERR_INVALID, "token_id %u out of bounds for embedding with %llu rows", tokens[i],
                       (unsigned long long)m->cfg.vocab_size);
  int32_t rc = check_ready(m);
  if (rc) return rc;
  if ((rc = ensure_kv(m, m->seq_len + n))) return rc;
  if (!prefill_supported(m)) {
    for (uint64_t i = 0; i < n; ++i)
      if ((rc = forward_token(m, tokens[i], m->seq_len))) return rc;
    return RF_OK;
  }
  if ((rc = ensure_prefill_ws(m))) return rc;
  const rf_model_config& c = m->cfg;
  hipStream_t st = m->ctx->compute;
  const uint64_t d = c.embedding_length;
  const uint32_t nl = (uint32_t)m->layers.size();
  uint64_t nt = 0;
  for (uint64_t off = 0; off < n; off += nt) {
    nt = n - off < MM_MAX_TOKENS ? n - off : MM_MAX_TOKENS;
    const uint64_t pos0 = m->seq_len;
    RF_LAUNCH(hipMemcpyAsync(m->p_tok, tokens + off, nt * 4, hipMemcpyHostToDevice, st), "upload prompt tokens");
    RF_LAUNCH(launch_dequant_rows(m->token_embd.type, m->token_embd.d, d, nt, m->p_h, m->p_tok, c.vocab_size, st),
              "prefill embedding");
    for (uint32_t li = 0; li < nl; ++li) {
      if (m->streaming && m->upl > 1) {
        rc = forward_layer_units(m, li, [&](uint32_t p) {
          int g0, g1;
          part_groups(m->upl, p, &g0, &g1);
          return enqueue_prefill_layer(m, li, pos0, nt, false, nullptr, g0, g1);
        });
        if (rc) return rc;
        continue;
      }
      m->cur_layer = li;
      if (m->streaming) {  // as enqueue_forward: this layer resident, the next one's upload started
        if ((rc = acquire_layer(m, li, false))) return abort_pass(m, rc);
        if (li + 1 < nl && (rc = acquire_layer(m, li + 1, true))) return abort_pass(m, rc);
        RF_LAUNCH(hipStreamWaitEvent(st, m->res[li].uploaded, 0), "wait for layer upload");
      }
      const float* next_norm =
          !m->streaming && li + 1 < nl ? static_cast<const float*>(m->layers[li + 1].attn_norm.d) : nullptr;
      const bool normed = li > 0 && !m->streaming;
      if ((rc = enqueue_prefill_layer(m, li, pos0, nt, normed, next_norm)))
        return m->streaming ? abort_pass(m, rc) : rc;
      if (m->streaming && (rc = settle_layer(m, li))) return abort_pass(m, rc);
    }
    if (m->streaming && (rc = release_retired(m))) return rc;
    m->seq_len += nt;
  }
  // the decode path continues from the last token's hidden state and position
  RF_LAUNCH(hipMemcpyAsync(m->hidden, m->p_h + (nt - 1) * d, d * 4, hipMemcpyDeviceToDevice, st), "prefill hidden");
  RF_LAUNCH(launch_set_i32(m->d_pos, (int32_t)m->seq_len, st), "prefill position");
  return m->streaming ? release_prefill_ws(m) : RF_OK;
}

}  // namespace

extern "C" {

namespace {
int32_t model_create(rf_ctx* ctx, const rf_model_config* cfg, uint64_t kv_cap, uint64_t kv_initial, bool grow,
                     rf_model** out);
}

int32_t rf_model_create(rf_ctx* ctx, const rf_model_config* cfg, uint64_t kv_cap, rf_model** out) {
  return model_create(ctx, cfg, kv_cap, kv_cap, false, out);
}

int32_t rf_model_create_growing(rf_ctx* ctx, const rf_model_config* cfg, uint64_t kv_capacity, uint64_t initial_tokens,
                                rf_model** out) {
  if (initial_tokens == 0 || initial_tokens > kv_capacity)
    return set_error(RF_ERR_INVALID, "initial KV capacity %llu must be in 1..=%llu", (unsigned long long)initial_tokens,
                     (unsigned long long)kv_capacity);
  return model_create(ctx, cfg, kv_capacity, initial_tokens, true, out);
}

}  // extern "C"

namespace {
int32_t model_create(rf_ctx* ctx, const rf_model_config* cfg, uint64_t kv_cap, uint64_t kv_initial, bool grow,
                     rf_model** out) {
  if (!ctx || !cfg || !out) return set_error(RF_ERR_INVALID, "null argument to rf_model_create");
  const rf_model_config& c = *cfg;
  if (c.embedding_length == 0 || c.head_count == 0 || c.head_count_kv == 0 || c.head_dim == 0 || c.vocab_size == 0 ||
      c.block_count == 0 || c.feed_forward_length == 0)
    return set_error(RF_ERR_INVALID, "model dimensions must be non-zero");
  if (c.head_count % c.head_count_kv != 0)
    return set_error(RF_ERR_INVALID, "GQA requires query_heads %llu to be divisible by kv_heads %llu",
                     (unsigned long long)c.head_count, (unsigned long long)c.head_count_kv);
  if (c.head_dim % 2 != 0 || c.head_dim > 512)
    return set_error(RF_ERR_INVALID, "RoPE head dimension must be non-zero and even (<= 512)");
  if (kv_cap == 0 || kv_cap > c.context_length)
    return set_error(RF_ERR_INVALID, "KV capacity %llu must be in 1..=context_length %llu",
                     (unsigned long long)kv_cap, (unsigned long long)c.context_length);
  if (c.vocab_size > 0xFFFFFFFFull) return set_error(RF_ERR_UNSUPPORTED, "vocabulary exceeds 2^32 entries");
  // The kernels index rows, heads and positions with 32 bits, and every size
  // below is then far from wrapping: widths and positions below 2^24, at
  // most 2^16 heads and layers, and KV caches within 64 bits.
  constexpr uint64_t kDim = 1ull << 24, kCount = 1ull << 16;
  uint64_t kv_bytes = 0;
  if (c.embedding_length > kDim || c.feed_forward_length > kDim || c.vocab_size > kDim ||
      c.head_count * c.head_dim > kDim || c.head_count > kCount || c.block_count > kCount || kv_cap > kDim ||
      __builtin_mul_overflow(c.block_count * kv_cap, c.head_count_kv * c.head_dim * 4, &kv_bytes))
    return set_error(RF_ERR_UNSUPPORTED,
                     "model dimensions out of range: widths, vocabulary and KV capacity must be below 2^24, heads "
                     "and layers at most 2^16");
  rf_model* m = new rf_model();
  m->ctx = ctx;
  m->cfg = c;
  m->kv_cap = kv_initial;
  m->kv_max = kv_cap;
  m->kv_grow = grow;
  kv_bytes = kv_bytes / kv_cap * kv_initial;  // c.block_count * kv_initial * kvd * 4
  m->layers.resize(c.block_count);
  const uint64_t d = c.embedding_length, qd = c.head_count * c.head_dim, kvd = c.head_count_kv * c.head_dim;
  const uint64_t f = c.feed_forward_length;
  void* p = nullptr;
  int32_t rc = charge_alloc(m, "kv_cache:k", kv_bytes, &p);
  if (rc) { rf_model_destroy(m); return rc; }
  m->k_cache = static_cast<float*>(p);
  rc = charge_alloc(m, "kv_cache:v", kv_bytes, &p);
  if (rc) { rf_model_destroy(m); return rc; }
  m->v_cache = static_cast<float*>(p);
  // activations: hidden, q, k, v, attn_out, act, up scratch, logits, final hidden
  const uint64_t wide = std::max(std::max(d, qd), f), widest = std::max(wide, (uint64_t)c.vocab_size);
  const uint64_t act_floats = d + qd + kvd + kvd + qd + f + f + c.vocab_size + d + wide + widest + 11 * 16;
  rc = charge_alloc(m, "tmp:forward", act_floats * 4 + 64 * 8, &p);
  if (rc) { rf_model_destroy(m); return rc; }
  float* base = static_cast<float*>(p);
  auto take = [&](uint64_t n) { float* r = base; base += (n + 15) / 16 * 16; return r; };
  m->hidden = take(d); m->q = take(qd); m->k = take(kvd); m->v = take(kvd); m->attn_out = take(qd);
  m->act = take(f); m->up_tmp = take(f); m->logits = take(c.vocab_size); m->final_hidden = take(d);
  m->xnorm = take(wide); m->mvtmp = take(widest);
  // attention workspace: fixed split count for the capacity (graph-friendly)
  const bool fast = attention_supported((uint32_t)c.head_count, (uint32_t)c.head_count_kv, (uint32_t)c.head_dim,
                                        kv_cap);
  m->attn_fast = fast;
  m->attn_chunks = 1;
  for (int r = 0; fast && r < ATT_REGIMES; ++r) {
    const AttnShape sh = attention_regime_shape(r, (uint32_t)c.head_count, (uint32_t)c.head_count_kv, kv_cap);
    if (sh.nsplit > m->attn_chunks) m->attn_chunks = sh.nsplit;
  }
  const uint64_t ws_floats = fast ? attention_ws_floats(m->attn_chunks, (uint32_t)c.head_count, (uint32_t)c.head_dim)
                                  : c.head_count * kv_cap;
  rc = charge_alloc(m, "workspace:model_attention", ws_floats * 4, &p);
  if (rc) { rf_model_destroy(m); return rc; }
  m->attn_ws = static_cast<float*>(p);
  rc = charge_alloc(m, "workspace:model_state", 256 * 8 + 64 + kv_cap * 4 + 64, &p);
  if (rc) { rf_model_destroy(m); return rc; }
  m->amax_val = static_cast<float*>(p);
  m->amax_idx = reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(p) + 256 * 4);
  m->d_pos = reinterpret_cast<int32_t*>(static_cast<uint8_t*>(p) + 256 * 8);
  m->d_token = reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(p) + 256 * 8 + 16);
  m->d_ring = reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(p) + 256 * 8 + 64);
  // RoPE table for every position of the cache (host libm, reference expression)
  const uint64_t rope_floats = kv_cap * c.head_dim;
  rc = charge_alloc(m, "persistent:rope_table", rope_floats * 4, &p);
  if (rc) { rf_model_destroy(m); return rc; }
  m->rope = static_cast<float*>(p);
  std::vector<float> tab(rope_floats);
  rope_table_host(tab.data(), 0, kv_cap, (uint32_t)c.head_dim, c.rope_freq_base);
  rc = staged_upload(ctx, m->rope, tab.data(), rope_floats * 4);
  if (rc) { rf_model_destroy(m); return rc; }
  hipError_t e = launch_set_i32(m->d_pos, 0, ctx->compute);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->compute);
  if (e != hipSuccess) { rf_model_destroy(m); return hip_error(e, "model init"); }
  *out = m;
  return RF_OK;
}
}  // namespace

extern "C" {

void rf_model_destroy(rf_model* m) {
  if (!m) return;
  ra_stop(m);
  for (hipEvent_t e : m->ra.done)
    if (e) hipEventDestroy(e);
  reset_graph(m);
  hipStreamSynchronize(m->ctx->compute);
  hipStreamSynchronize(m->ctx->copy);
  hipStreamSynchronize(m->ctx->copy2);
  for (uint32_t u = 0; u < m->res.size(); ++u) {
    layer_free(m, u);
    if (m->res[u].uploaded) hipEventDestroy(m->res[u].uploaded);
    if (m->res[u].used) hipEventDestroy(m->res[u].used);
  }
  for (Layer& L : m->layers) {
    DevTensor* t[12];
    layer_slots(L, t);
    for (DevTensor* x : t)
      if (x->host) hipHostFree(x->host);
  }
  if (m->up2) hipEventDestroy(m->up2);
  for (auto it = m->charges.rbegin(); it != m->charges.rend(); ++it) vram_release(m->ctx, *it);
  for (DevTensor* x : {&m->token_embd, &m->output, &m->output_norm})
    if (x->host) hipHostFree(x->host);
  for (hipEvent_t e : m->prof_ev)
    if (e) hipEventDestroy(e);
  for (int i = 0; i < 2; ++i) {
    if (m->rstage[i]) hipHostFree(m->rstage[i]);
    if (m->rstage_ev[i]) hipEventDestroy(m->rstage_ev[i]);
  }
  delete m;
}

int32_t rf_model_set_tensor(rf_model* m, const char* name, uint32_t t, uint64_t ne0, uint64_t ne1, const void* host,
                            uint64_t nbytes) {
  if (!host) return set_error(RF_ERR_INVALID, "null tensor data");
  return install(m, name, t, ne0, ne1, host, nbytes, false, 0, 0.0, NAN);
}

int32_t rf_model_synth_tensor(rf_model* m, const char* name, uint32_t t, uint64_t ne0, uint64_t ne1, uint64_t seed,
                              double mul, float constant) {
  return install(m, name, t, ne0, ne1, nullptr, 0, true, seed, mul, constant);
}

int32_t rf_model_reset(rf_model* m) {
  if (!m) return set_error(RF_ERR_INVALID, "null model");
  m->seq_len = 0;
  hipError_t e = launch_set_i32(m->d_pos, 0, m->ctx->compute);
  if (e != hipSuccess) return hip_error(e, "reset");
  return sync(m);
}

uint64_t rf_model_seq_len(rf_model* m) { return m ? m->seq_len : 0; }

int32_t rf_model_forward(rf_model* m, uint32_t token, uint64_t pos, float* final_hidden) {
  if (!m) return set_error(RF_ERR_INVALID, "null model");
  int32_t rc = forward_token(m, token, pos);
  if (rc) return rc;
  if (final_hidden) {
    // output_norm of the last hidden state (streaming_model.rs:1297-1301)
    RF_LAUNCH(launch_rmsnorm(m->hidden, static_cast<const float*>(m->output_norm.d), m->cfg.embedding_length,
                             m->cfg.rms_eps, m->final_hidden, m->ctx->compute),
              "output norm");
    RF_LAUNCH(hipMemcpyAsync(final_hidden, m->final_hidden, m->cfg.embedding_length * 4, hipMemcpyDeviceToHost,
                             m->ctx->compute),
              "download hidden");
  }
  return sync(m);
}

int32_t rf_model_prefill(rf_model* m, const uint32_t* tokens, uint64_t n, float* final_hidden) {
  if (!m || (n && !tokens)) return set_error(RF_ERR_INVALID, "null argument to rf_model_prefill");
  int32_t rc = prefill_tokens(m, tokens, n);
  if (rc) return rc;
  if (final_hidden && m->seq_len > 0) {
    RF_LAUNCH(launch_rmsnorm(m->hidden, static_cast<const float*>(m->output_norm.d), m->cfg.embedding_length,
                             m->cfg.rms_eps, m->final_hidden, m->ctx->compute),
              "output norm");
    RF_LAUNCH(hipMemcpyAsync(final_hidden, m->final_hidden, m->cfg.embedding_length * 4, hipMemcpyDeviceToHost,
                             m->ctx->compute),
              "download hidden");
  }
  return sync(m);
}

int32_t rf_model_set_prefill(rf_model* m, int32_t batched) {
  if (!m) return set_error(RF_ERR_INVALID, "null model");
  m->prefill_batched = batched != 0;
  return RF_OK;
}

int32_t rf_model_logits(rf_model* m, float* logits) {
  if (!m || !logits) return set_error(RF_ERR_INVALID, "null argument");
  if (m->seq_len == 0) return set_error(RF_ERR_INVALID, "logits requested before any forward pass");
  int32_t rc = enqueue_logits(m);
  if (rc) return rc;
  RF_LAUNCH(hipMemcpyAsync(logits, m->logits, m->cfg.vocab_size * 4, hipMemcpyDeviceToHost, m->ctx->compute),
            "download logits");
  return sync(m);
}

int32_t rf_model_generate(rf_model* m, const uint32_t* prompt, uint64_t plen, uint64_t max_tokens, int64_t eos,
                          uint32_t* out, uint64_t* n_out) {
  if (!m || (plen && !prompt) || (max_tokens && !out) || !n_out) return set_error(RF_ERR_INVALID, "null argument");
  *n_out = 0;
  const uint64_t ctx_len = m->cfg.context_length;
  // inference.rs:465-476: the request must fit the context.
  if (plen > ctx_len || max_tokens > ctx_len - plen)
    return set_error(RF_ERR_INVALID, "prompt (%llu tokens) plus max_tokens (%llu) exceeds context length %llu",
                     (unsigned long long)plen, (unsigned long long)max_tokens, (unsigned long long)ctx_len);
  // A growing cache starts at the prompt's length and grows by 256-position
  // chunks up to prompt + max_tokens (inference.rs:478-496, 666-687).
  struct LimitGuard {
    rf_model* m;
    ~LimitGuard() { m->kv_limit = 0; }
  } guard{m};
  if (m->kv_grow) {
    const uint64_t need = m->seq_len + plen;
    m->kv_limit = std::min(need + max_tokens, m->kv_max);
    if (need > m->kv_cap && need <= m->kv_limit) {
      const int32_t rc = kv_resize(m, need);
      if (rc) return rc;
    }
  }
  if (m->prefill_batched) {
    int32_t rc = prefill_tokens(m, prompt, plen);
    if (rc) return rc;
  } else {
    for (uint64_t p = 0; p < plen; ++p) {
      int32_t rc = forward_token(m, prompt[p], m->seq_len);
      if (rc) return rc;
    }
  }
  uint64_t cur = m->seq_len;
  uint64_t n = 0;
  for (uint64_t gi = 0; gi < max_tokens; ++gi) {
    if (m->seq_len == 0) return set_error(RF_ERR_INVALID, "generation requires a non-empty prompt");
    int32_t rc = enqueue_logits(m);
    if (rc) return rc;
    RF_LAUNCH(launch_argmax(m->logits, m->cfg.vocab_size, m->d_token, m->amax_val, m->amax_idx, nullptr, nullptr,
                            m->ctx->compute),
              "argmax");
    uint32_t next = 0;
    RF_LAUNCH(hipMemcpyAsync(&next, m->d_token, 4, hipMemcpyDeviceToHost, m->ctx->compute), "download token");
    rc = sync(m);
    if (rc) return rc;
    if (eos >= 0 && (int64_t)next == eos) break;
    out[n++] = next;
    *n_out = n;
    const uint64_t next_pos = cur + 1;
    if (gi + 1 >= max_tokens) break;        // terminal forward skipped (inference.rs:643-653)
    if (next_pos >= ctx_len) break;
    rc = forward_token(m, next, cur);
    if (rc) return rc;
    cur = next_pos;
    if (cur >= ctx_len) break;
  }
  return sync(m);
}

int32_t rf_model_kv_growth(rf_model* m, uint64_t initial_tokens) {
  if (!m) return set_error(RF_ERR_INVALID, "null model");
  if (m->seq_len != 0) return set_error(RF_ERR_INVALID, "KV growth must be enabled on an empty cache (reset first)");
  if (initial_tokens == 0 || initial_tokens > m->kv_max)
    return set_error(RF_ERR_INVALID, "initial KV capacity %llu must be in 1..=%llu", (unsigned long long)initial_tokens,
                     (unsigned long long)m->kv_max);
  if (initial_tokens != m->kv_cap) {
    const int32_t rc = kv_resize(m, initial_tokens);
    if (rc) return rc;
  }
  m->kv_grow = true;
  return RF_OK;
}

int32_t rf_model_kv_capacity(rf_model* m, uint64_t* tokens) {
  if (!m || !tokens) return set_error(RF_ERR_INVALID, "null argument");
  *tokens = m->kv_cap;
  return RF_OK;
}

int32_t rf_model_paths(rf_model* m, uint64_t pos, int32_t* split_attention, int32_t* regime,
                       int32_t* batched_prefill) {
  if (!m || !split_attention || !regime || !batched_prefill) return set_error(RF_ERR_INVALID, "null argument");
  *split_attention = m->attn_fast ? 1 : 0;
  *regime = attn_regime(m, pos);
  *batched_prefill = prefill_supported(m) ? 1 : 0;
  return RF_OK;
}

int32_t rf_model_use_graph(rf_model* m, int32_t enable) {
  if (!m) return set_error(RF_ERR_INVALID, "null model");
  if (enable && m->prof)
    return set_error(RF_ERR_INVALID, "graph replay is unavailable while the forward profiler is on");
  if (enable && m->streaming)
    return set_error(RF_ERR_UNSUPPORTED, "graph replay needs every layer resident; this model streams its layers");
  m->use_graph = enable != 0;
  if (!m->use_graph) reset_graph(m);
  return RF_OK;
}

int32_t rf_model_decode_steps(rf_model* m, uint64_t steps) {
  if (!m) return set_error(RF_ERR_INVALID, "null model");
  if (m->seq_len == 0) return set_error(RF_ERR_INVALID, "decode requires a forwarded prompt");
  if (steps > m->kv_max - m->seq_len) return set_error(RF_ERR_INVALID, "KV cache full");  // seq_len <= kv_cap <= kv_max
  int32_t rc = check_ready(m);
  if (rc) return rc;
  if ((rc = ensure_kv(m, m->seq_len + steps))) return rc;  // before any graph is captured or replayed
  hipStream_t st = m->ctx->compute;
  for (uint64_t s = 0; s < steps; ++s) {
    const int r = attn_regime(m, m->seq_len);
    if (m->use_graph && !m->graph_exec[r]) {
      // captured at the first step of its regime; replays read the position from d_pos
      if ((rc = plan_decode_step(m))) return rc;
      RF_LAUNCH(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal), "begin capture");
      rc = enqueue_decode_step(m);
      hipGraph_t g = nullptr;
      hipError_t e = hipStreamEndCapture(st, &g);
      if (rc) { if (g) hipGraphDestroy(g); return rc; }
      if (e != hipSuccess) return hip_error(e, "end capture");
      m->graph[r] = g;
      e = hipGraphInstantiate(&m->graph_exec[r], g, nullptr, nullptr, 0);
      if (e != hipSuccess) { reset_graph(m); return hip_error(e, "graph instantiate"); }
    }
    if (m->use_graph) {
      RF_LAUNCH(hipGraphLaunch(m->graph_exec[r], st), "graph launch");
    } else {
      rc = enqueue_decode_step(m);
      if (rc) return rc;
    }
    m->seq_len += 1;
  }
  return RF_OK;
}

int32_t rf_model_kernel_name(rf_model* m, uint32_t kind, char* buf, uint64_t cap) {
  if (!m || !buf || cap == 0) return set_error(RF_ERR_INVALID, "null argument");
  if (kind < RF_KERNEL_QKV || kind > RF_KERNEL_LOGITS)
    return set_error(RF_ERR_INVALID, "unknown kernel group %u", kind);
  int32_t rc = check_ready(m);
  if (rc) return rc;
  if (m->streaming) return set_error(RF_ERR_UNSUPPORTED, "kernel naming needs every layer resident");
  // a planning pass of the group on layer 0 (the o-projection after its
  // attention, whose regime decides whether it merges chunk records)
  clear_last_packed_kernel();
  g_plan_only = true;
  m->oproj_merge = false;
  switch (kind) {
    case RF_KERNEL_QKV: rc = enqueue_qkv(m, 0); break;
    case RF_KERNEL_ATTENTION: rc = enqueue_attention(m, 0); break;
    case RF_KERNEL_OPROJ:
      rc = enqueue_attention(m, 0);
      if (!rc) {
        clear_last_packed_kernel();
        rc = enqueue_oproj(m, 0);
      }
      break;
    case RF_KERNEL_GATEUP: rc = enqueue_gateup(m, 0); break;
    case RF_KERNEL_DOWN: rc = enqueue_down(m, 0); break;
    default: rc = enqueue_logits(m); break;
  }
  g_plan_only = false;
  m->oproj_merge = false;
  if (rc) return rc;
  snprintf(buf, cap, "%s", last_packed_kernel());
  return RF_OK;
}

int32_t rf_model_time_kernel(rf_model* m, uint32_t kind, uint32_t reps, float* avg_ms, uint64_t* bytes_per_launch,
                             uint64_t* launches) {
  if (!m || !avg_ms || !bytes_per_launch || !launches || reps == 0) return set_error(RF_ERR_INVALID, "null argument");
  if (kind < RF_KERNEL_QKV || kind > RF_KERNEL_LOGITS)
    return set_error(RF_ERR_INVALID, "unknown kernel group %u", kind);
  int32_t rc = check_ready(m);
  if (rc) return rc;
  if (m->streaming) return set_error(RF_ERR_UNSUPPORTED, "kernel timing needs every layer resident");
  if (kind == RF_KERNEL_ATTENTION && m->seq_len == 0)
    return set_error(RF_ERR_INVALID, "attention timing needs a forwarded prompt");
  if (kind == RF_KERNEL_ATTENTION && m->seq_len >= m->kv_cap)
    return set_error(RF_ERR_INVALID, "attention timing writes K/V slot %llu but the cache holds %llu",
                     (unsigned long long)m->seq_len, (unsigned long long)m->kv_cap);
  hipStream_t st = m->ctx->compute;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  RF_LAUNCH(hipEventCreate(&e0), "hipEventCreate");
  if (hipError_t ec = hipEventCreate(&e1); ec != hipSuccess) {
    hipEventDestroy(e0);
    return hip_error(ec, "hipEventCreate");
  }
  // Attention is timed at the current position (the kernel only reads d_pos).
  const uint64_t hist = m->seq_len;
  uint64_t n = 0, bytes = 0;
  m->oproj_merge = false;
  hipError_t e = hipEventRecord(e0, st);
  for (uint32_t r = 0; r < reps && e == hipSuccess && rc == RF_OK; ++r) {
    if (kind == RF_KERNEL_LOGITS) {
      rc = enqueue_logits(m);
      bytes += part_bytes(m, kind, 0, hist);
      ++n;
      continue;
    }
    for (size_t li = 0; li < m->layers.size() && rc == RF_OK; ++li) {
      switch (kind) {
        case RF_KERNEL_QKV: rc = enqueue_qkv(m, li); break;
        case RF_KERNEL_ATTENTION: rc = enqueue_attention(m, li); break;
        case RF_KERNEL_OPROJ: rc = enqueue_oproj(m, li); break;
        case RF_KERNEL_GATEUP: rc = enqueue_gateup(m, li); break;
        case RF_KERNEL_DOWN: rc = enqueue_down(m, li); break;
      }
      bytes += part_bytes(m, kind, li, hist);
      ++n;
    }
  }
  m->oproj_merge = false;  // a timed attention's deferred merge is not the next o-projection's
  if (e == hipSuccess) e = hipEventRecord(e1, st);
  if (e == hipSuccess) e = hipEventSynchronize(e1);
  float ms = 0.f;
  if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
  hipEventDestroy(e0);
  hipEventDestroy(e1);
  if (rc) return rc;
  if (e != hipSuccess) return hip_error(e, "kernel timing");
  // The attention kernel wrote K/V into slot `hist` of every layer; that slot is
  // rewritten by the next forward, so the cache contents stay consistent.
  *avg_ms = ms / (float)n;
  *bytes_per_launch = bytes / n;
  *launches = n;
  return RF_OK;
}

int32_t rf_model_enable_streaming(rf_model* m, uint64_t layer_cache_bytes) {
  if (!m) return set_error(RF_ERR_INVALID, "null model");
  if (m->streaming) {
    m->cache_cap = layer_cache_bytes;
    return RF_OK;
  }
  for (Layer& L : m->layers) {
    DevTensor* t[12];
    layer_slots(L, t);
    for (DevTensor* x : t)
      if (x->present()) return set_error(RF_ERR_INVALID, "layer streaming must be enabled before block tensors load");
  }
  m->res.resize(unit_count(m));
  for (LayerRes& R : m->res) {
    hipError_t e = hipEventCreateWithFlags(&R.uploaded, hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&R.used, hipEventDisableTiming);
    if (e != hipSuccess) return hip_error(e, "hipEventCreate");
  }
  if (!m->up2) {
    const hipError_t e = hipEventCreateWithFlags(&m->up2, hipEventDisableTiming);
    if (e != hipSuccess) return hip_error(e, "hipEventCreate");
  }
  m->streaming = true;
  m->cache_cap = layer_cache_bytes;
  m->use_graph = false;
  reset_graph(m);
  return RF_OK;
}

int32_t rf_model_set_reader(rf_model* m, rf_read_fn read, void* user, uint64_t staging_bytes) {
  if (!m || !read) return set_error(RF_ERR_INVALID, "null model or reader");
  if (!m->streaming) return set_error(RF_ERR_INVALID, "a byte source needs layer streaming (rf_model_enable_streaming)");
  if (staging_bytes < 4096) return set_error(RF_ERR_INVALID, "staging buffers of %llu bytes (at least 4096)",
                                             (unsigned long long)staging_bytes);
  for (Layer& L : m->layers) {
    DevTensor* t[12];
    layer_slots(L, t);
    for (DevTensor* x : t)
      if (x->src) return set_error(RF_ERR_INVALID, "the byte source must be set before source tensors are declared");
  }
  void* b[2] = {nullptr, nullptr};
  hipEvent_t ev[2] = {nullptr, nullptr};
  hipError_t e = hipSuccess;
  for (int i = 0; i < 2 && e == hipSuccess; ++i) {
    e = hipHostMalloc(&b[i], staging_bytes, hipHostMallocDefault);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&ev[i], hipEventDisableTiming);
  }
  if (e != hipSuccess) {
    for (int i = 0; i < 2; ++i) {
      if (b[i]) hipHostFree(b[i]);
      if (ev[i]) hipEventDestroy(ev[i]);
    }
    return hip_error(e, "staging buffers");
  }
  for (int i = 0; i < 2; ++i) {
    if (m->rstage[i]) hipHostFree(m->rstage[i]);
    if (m->rstage_ev[i]) hipEventDestroy(m->rstage_ev[i]);
    m->rstage[i] = b[i];
    m->rstage_ev[i] = ev[i];
  }
  ra_stop(m);
  m->rstage_bytes = staging_bytes;
  m->reader = read;
  m->reader_user = user;
  m->ra.on = read == rf_file_source_read;  // thread-safe: read ahead by default
  return RF_OK;
}

int32_t rf_model_set_read_ahead(rf_model* m, int32_t on) {
  if (!m) return set_error(RF_ERR_INVALID, "null model");
  if (on != 0 && on != 1) return set_error(RF_ERR_INVALID, "read-ahead is 0 or 1, got %d", (int)on);
  if (on && !m->reader) return set_error(RF_ERR_INVALID, "no byte source (rf_model_set_reader)");
  if (!on) ra_stop(m);
  m->ra.on = on == 1;
  return RF_OK;
}

int32_t rf_model_set_tensor_source(rf_model* m, const char* cname, uint32_t t, uint64_t ne0, uint64_t ne1,
                                   uint64_t offset, uint64_t nbytes) {
  if (!m || !cname) return set_error(RF_ERR_INVALID, "null model or tensor name");
  if (!m->reader) return set_error(RF_ERR_INVALID, "no byte source (rf_model_set_reader)");
  const std::string name(cname);
  unsigned li = 0;
  if (name.rfind("blk.", 0) != 0 || sscanf(name.c_str(), "blk.%u.", &li) != 1 || li >= m->layers.size())
    return set_error(RF_ERR_INVALID, "only block tensors stream from the byte source, got '%s'", name.c_str());
  DevTensor* slot = nullptr;
  uint64_t e0 = 0, e1 = 0, bytes = 0;
  std::string charge;
  int32_t rc = resolve(m, name, &slot, &e0, &e1, &charge);
  if (rc) return rc;
  rc = check_tensor_shape(m, name, t, ne0, ne1, e0, e1, &bytes);
  if (rc) return rc;
  if (nbytes != bytes)
    return set_error(RF_ERR_INVALID, "tensor '%s' spans %llu bytes, its shape needs %llu", name.c_str(),
                     (unsigned long long)nbytes, (unsigned long long)bytes);
  if (offset + nbytes < offset) return set_error(RF_ERR_INVALID, "tensor '%s' range overflows", name.c_str());
  const bool widen = (t == T_F16 || t == T_BF16);
  const bool pack = g_pack_weights && is_projection(name) && plan_packed(t, ne0).ok;
  if ((widen || pack) && bytes > m->rraw_bytes) {  // the raw buffer holds the largest converted tensor
    hipError_t e = hipStreamSynchronize(m->ctx->copy);
    if (e != hipSuccess) return hip_error(e, "hipStreamSynchronize");
    void* d = nullptr;
    rc = vram_alloc(m->ctx, "workspace:layer_read:new", bytes, &d);
    if (rc) return rc;
    if (m->rraw) release_charge(m, "workspace:layer_read");
    vram_rename_prefix(m->ctx, "workspace:layer_read:new", "workspace:layer_read");
    m->charges.push_back("workspace:layer_read");
    m->rraw = d;
    m->rraw_bytes = bytes;
  }
  reset_graph(m);
  rc = layer_free(m, li);  // a resident copy of the layer is stale now
  if (rc) return rc;
  if (slot->host) hipHostFree(slot->host);
  slot->host = nullptr;
  slot->d = nullptr;
  slot->charge.clear();
  slot->type = widen ? T_F32 : t;
  slot->ne0 = ne0;
  slot->ne1 = ne1;
  slot->nbytes = widen ? ne0 * ne1 * 4 : bytes;
  slot->packed = pack;
  slot->src = true;
  slot->src_type = t;
  slot->src_off = offset;
  slot->src_bytes = bytes;
  update_layer_bytes(m, li);
  return RF_OK;
}

int32_t rf_model_profile(rf_model* m, int32_t enable) {
  if (!m) return set_error(RF_ERR_INVALID, "null model");
  if (enable && m->use_graph)
    return set_error(RF_ERR_INVALID, "the forward profiler needs eager launches (rf_model_use_graph(model, 0))");
  int32_t rc = prof_collect(m);
  if (rc) return rc;
  if (enable && m->prof_ev.empty()) {
    const size_t pairs = 5 * m->layers.size() + 2;
    std::vector<hipEvent_t> ev(2 * pairs, nullptr);
    for (hipEvent_t& e : ev) {
      const hipError_t he = hipEventCreate(&e);
      if (he != hipSuccess) {
        for (hipEvent_t x : ev)
          if (x) hipEventDestroy(x);
        return hip_error(he, "hipEventCreate");
      }
    }
    m->prof_ev.swap(ev);
    m->prof_kind.assign(pairs, 0);
  }
  m->prof = enable != 0;
  return RF_OK;
}

int32_t rf_model_profile_read(rf_model* m, double* ms, uint64_t* counts, int32_t reset) {
  if (!m || !ms || !counts) return set_error(RF_ERR_INVALID, "null argument");
  int32_t rc = prof_collect(m);
  if (rc) return rc;
  for (int i = 0; i < 6; ++i) {
    ms[i] = m->prof_ms[i];
    counts[i] = m->prof_n[i];
    if (reset) { m->prof_ms[i] = 0; m->prof_n[i] = 0; }
  }
  return RF_OK;
}

int32_t rf_model_set_persistent_policy(rf_model* m, int32_t policy) {
  if (!m) return set_error(RF_ERR_INVALID, "null model");
  if (policy < 0 || policy > 3) return set_error(RF_ERR_INVALID, "unknown persistent-weight policy %d", policy);
  if (m->token_embd.present() || m->output.present())
    return set_error(RF_ERR_INVALID, "the persistent-weight policy must be set before token_embd / output load");
  m->persistent_policy = policy;
  return RF_OK;
}

int32_t rf_model_persistent_streamed(rf_model* m, uint32_t* mask) {
  if (!m || !mask) return set_error(RF_ERR_INVALID, "null argument");
  *mask = (m->token_embd.present() && m->token_embd.charge.empty() && m->token_embd.host ? 1u : 0u) |
          (m->output.present() && m->output.charge.empty() && m->output.host ? 2u : 0u);
  return RF_OK;
}

int32_t rf_model_read_stats(rf_model* m, uint64_t* out) {
  if (!m || !out) return set_error(RF_ERR_INVALID, "null argument");
  out[0] = m->st_read_calls;
  out[1] = m->st_read_bytes;
  return RF_OK;
}

int32_t rf_model_set_cache_policy(rf_model* m, int32_t policy) {
  if (!m) return set_error(RF_ERR_INVALID, "null model");
  if (policy != 0 && policy != 1) return set_error(RF_ERR_INVALID, "unknown layer cache policy %d", policy);
  m->cache_policy = policy;
  return RF_OK;
}

int32_t rf_model_set_stream_units(rf_model* m, int32_t per_layer) {
  if (!m) return set_error(RF_ERR_INVALID, "null model");
  if (per_layer < 1 || per_layer > 3)
    return set_error(RF_ERR_INVALID, "streaming units per layer must be 1, 2 or 3, got %d", per_layer);
  if (!m->streaming) return set_error(RF_ERR_INVALID, "streaming units need layer streaming (rf_model_enable_streaming)");
  if ((uint32_t)per_layer == m->upl) return RF_OK;
  // every resident unit is released (waiting for its kernels), then the
  // residency records are rebuilt for the new units
  ra_stop(m);
  const hipError_t se = hipStreamSynchronize(m->ctx->compute);
  if (se != hipSuccess) return hip_error(se, "hipStreamSynchronize");
  for (uint32_t u = 0; u < m->res.size(); ++u) {
    const int32_t rc = layer_free(m, u);
    if (rc) return rc;
  }
  const size_t n = m->layers.size() * (size_t)per_layer;
  while (m->res.size() > n) {
    LayerRes& R = m->res.back();
    if (R.uploaded) hipEventDestroy(R.uploaded);
    if (R.used) hipEventDestroy(R.used);
    m->res.pop_back();
  }
  while (m->res.size() < n) {
    m->res.emplace_back();
    LayerRes& R = m->res.back();
    hipError_t e = hipEventCreateWithFlags(&R.uploaded, hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&R.used, hipEventDisableTiming);
    if (e != hipSuccess) return hip_error(e, "hipEventCreate");
  }
  for (LayerRes& R : m->res) R.state = LAYER_HOST;
  m->lru.clear();
  m->cache_used = 0;
  m->upl = (uint32_t)per_layer;
  m->cur_layer = 0;
  for (uint32_t li = 0; li < m->layers.size(); ++li) update_layer_bytes(m, li);
  return RF_OK;
}

int32_t rf_model_host_bytes(rf_model* m, uint64_t* pinned) {
  if (!m || !pinned) return set_error(RF_ERR_INVALID, "null argument");
  uint64_t n = 0;
  for (Layer& L : m->layers) {
    DevTensor* t[12];
    layer_slots(L, t);
    for (DevTensor* x : t)
      if (x->host) n += x->nbytes;
  }
  for (DevTensor* x : {&m->token_embd, &m->output, &m->output_norm})
    if (x->host) n += x->nbytes;
  for (int i = 0; i < 2; ++i)
    if (m->rstage[i]) n += m->rstage_bytes;
  n += 2 * m->ra.bytes;
  *pinned = n;
  return RF_OK;
}

int32_t rf_model_residency_stats(rf_model* m, uint64_t* out) {
  if (!m || !out) return set_error(RF_ERR_INVALID, "null argument");
  out[0] = m->st_hits;
  out[1] = m->st_misses;
  out[2] = m->st_evictions;
  out[3] = m->st_uploaded;
  out[4] = m->cache_used;
  out[5] = m->lru.size();
  return RF_OK;
}

int32_t rf_tune_attention_single(int32_t positions) {
  if (positions == 64 || positions == 128 || positions == 256) set_attention_single((uint32_t)positions);
  return (int32_t)attention_single();
}

int32_t rf_tune_prefill_attention(int32_t mode) {
  if (mode >= 0 && mode <= 2) set_prefill_attention_mfma(mode);
  return prefill_attention_mfma();
}

int32_t rf_tune_attention_kernel(int32_t mode) {
  if (mode >= 0 && mode <= 2) set_attention_kernel(mode);
  return attention_kernel();
}

int32_t rf_tune_attention_merge(int32_t mode) {
  if (mode == 0 || mode == 1) g_oproj_merge = mode;
  return g_oproj_merge;
}

int32_t rf_tune_packed_weights(int32_t mode) {
  if (mode == 0 || mode == 1) g_pack_weights = mode;
  return g_pack_weights;
}

int32_t rf_model_read_tokens(rf_model* m, uint32_t* out, uint64_t n) {
  if (!m || (n && !out)) return set_error(RF_ERR_INVALID, "null argument");
  if (n > m->seq_len) return set_error(RF_ERR_INVALID, "only %llu positions exist", (unsigned long long)m->seq_len);
  int32_t rc = sync(m);
  if (rc) return rc;
  // the token forwarded at position p was chosen from position p-1's logits
  RF_LAUNCH(hipMemcpy(out, m->d_ring + (m->seq_len - n), n * 4, hipMemcpyDeviceToHost), "download tokens");
  return RF_OK;
}

}  // extern "C"
