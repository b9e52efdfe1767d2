// Host side of the resident decode epoch: engine lifecycle, weight arena,
// device-resident state, per-K epoch graphs and the C-ABI of
// include/resident_epoch.h.
//
// One epoch = one hipGraph launch that contains exactly one host-to-device
// copy (the feed), the controller kernels, K decoder steps whose kernels all
// return at once when the device "done" flag is set (no active rows left or a
// fallback status), and exactly one device-to-host copy (the fetch).
#include <time.h>

#include <algorithm>
#include <array>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <map>
#include <memory>
#include <mutex>
#include <sstream>
#include <string>
#include <vector>

#include "../../include/resident_epoch.h"
#include "re_json.h"
#include "re_layout.h"

namespace re {
// Scratch of resident_epoch_prefill_batch_noalloc: the batched prefill's
// activations and token tables for callers that cannot allocate device
// memory.  One copy per GPU, held until the process ends; every call on a
// GPU shares it (calls are serialized by g_noalloc_mutex, and a call leaves
// its contents behind: nothing in it needs to start at zero, every byte a
// pass reads is written earlier in the same pass).
constexpr size_t kNoAllocScratchBytes = 64ull << 20;
}  // namespace re

static __device__ __align__(256) uint8_t scratch[re::kNoAllocScratchBytes];

namespace re {
namespace {

constexpr int kBridgeRows = 4;  // rows of the bridge call's host arrays
constexpr int kCreateOk = 0, kCreateArgs = 1, kCreateTiling = 2, kCreateConfig = 3, kCreateGraph = 4,
              kCreateWeights = 5, kCreateRuntime = 6, kCreateDevice = 7;

std::mutex g_lifecycle_mutex;
bool g_engine_active = false;

// Device addresses of `scratch`, per device: host code never names the array
// itself (its host-side name is not a device address).
constexpr int kMaxDevices = 64;
std::mutex g_noalloc_mutex;
uint8_t* g_noalloc_ptr[kMaxDevices] = {};

// Resolves the array's address on `device`, which must be current; once per
// device (on the no-allocation entry point's first call there).  False on a
// HIP error.
bool noalloc_setup(int device) {
  if (device < 0 || device >= kMaxDevices) return false;
  std::lock_guard<std::mutex> lock(g_noalloc_mutex);
  if (g_noalloc_ptr[device] != nullptr) return true;
  void* ptr = nullptr;
  if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || ptr == nullptr) {
    (void)hipGetLastError();
    return false;
  }
  g_noalloc_ptr[device] = static_cast<uint8_t*>(ptr);
  return true;
}

uint8_t* noalloc_scratch(int device) {
  if (device < 0 || device >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_noalloc_mutex);
  return g_noalloc_ptr[device];
}

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

int64_t process_cpu_us() {
  timespec value{};
  if (clock_gettime(CLOCK_PROCESS_CPUTIME_ID, &value) != 0) return -1;
  return static_cast<int64_t>(value.tv_sec) * 1000000LL + static_cast<int64_t>(value.tv_nsec) / 1000LL;
}

bool read_file(const std::string& path, std::string& out) {
  std::ifstream f(path, std::ios::binary);
  if (!f) return false;
  std::stringstream ss;
  ss << f.rdbuf();
  out = ss.str();
  return static_cast<bool>(f) || f.eof();
}

struct WeightSlot {
  size_t offset;
  size_t bytes;
  long long elems;
};

struct Engine {
  Dims dims{};
  LaunchPlan plan{};
  int device = 0;
  int cus = 256;
  hipStream_t stream = nullptr;
  std::array<uint8_t, kTilingBytes> tiling{};

  // weights
  uint8_t* weights = nullptr;
  size_t weight_bytes = 0;
  size_t streamed_weight_bytes = 0;
  std::vector<LayerOffsets> layer_off;
  size_t embedding_off = 0, final_norm_off = 0, lm_head_off = 0;
  std::map<std::string, WeightSlot> weight_slots;
  std::vector<std::string> weight_order;
  // the matrix-core copy (plan.mfma): the matrices packed into 1 KB tiles
  uint8_t* packed = nullptr;
  std::vector<PackedOffsets> packed_off;
  size_t packed_lm_off = 0;

  // resident caches and state
  void* key_cache = nullptr;
  void* value_cache = nullptr;
  size_t cache_bytes = 0;
  uint8_t* state_mem = nullptr;
  StatePtrs st{};
  Scratch scratch{};
  uint8_t* scratch_mem = nullptr;
  float* logits = nullptr;

  // decoder-step ABI buffers
  uint8_t* step_mem = nullptr;
  StepPtrs step_io{};
  void* dec_key = nullptr;
  void* dec_value = nullptr;

  // host staging (pinned)
  uint8_t* h_feed = nullptr;
  uint8_t* h_fetch = nullptr;
  size_t feed_bytes = 0, import_feed_bytes = 0, fetch_bytes = 0, payload_bytes = 0;
  // Batched prefill scratch (grown on demand, freed with the engine).
  uint8_t* pf_mem = nullptr;
  size_t pf_bytes = 0;
  bool pf_ready = false;
  // Device-IPC import: mapped source allocations, keyed by the 64-byte
  // handle, with their mapped sizes; closed when the engine is destroyed.
  struct IpcMapping {
    void* ptr;
    size_t bytes;
  };
  std::map<std::string, IpcMapping> ipc_maps;
  unsigned long long* checksum_dev = nullptr;  // import Adler-32 partial sums [2]

  // graphs keyed by (K * 3 + feed mode) * 4 + part (0 whole epoch; 1 and 2
  // the halves around the timed launch)
  std::map<int, hipGraphExec_t> graphs;
  std::map<int, hipGraph_t> graph_defs;
  // Nodes each captured graph holds, read back from the graph: {memory
  // copies, memsets, kernels}; and the sums over the last epoch launched.
  std::map<int, std::array<int, 3>> graph_copies;
  std::array<int, 3> last_epoch_copies{{-1, -1, -1}};
  // Kernel timing: the gate/up launch of layer timing_layer in an epoch's last
  // step runs between two HIP events on the engine stream, outside the graphs.
  bool timing = false;
  int timing_layer = 0;
  hipEvent_t ev_start = nullptr, ev_stop = nullptr;
  std::vector<float> timing_ms;

  std::mutex execute_mutex;

  KernelEnv env() const {
    KernelEnv e{};
    e.dims = dims;
    e.plan = plan;
    e.weights = weights;
    e.layer_off = layer_off.data();
    e.embedding_off = embedding_off;
    e.final_norm_off = final_norm_off;
    e.lm_head_off = lm_head_off;
    e.scratch = scratch;
    e.packed = packed;
    e.packed_off = packed_off.data();
    e.packed_lm_off = packed_lm_off;
    return e;
  }
};

bool parse_dims(const Json& cfg, Dims& d) {
  // Defaults: Qwen2.5-7B (batched_decoder_step.py:19-33) at the reference B=4
  // geometry with the reference logical capacity of 8.
  d.layers = 28;
  d.hidden = 3584;
  d.heads = 28;
  d.kv_heads = 4;
  d.head_dim = 128;
  d.intermediate = 18944;
  d.vocab = 152064;
  d.rope_theta = 1000000.0f;
  d.rms_eps = 1e-6f;
  d.dtype_bytes = 2;
  d.batch = 4;
  d.physical_blocks = 8;
  d.block_size = 128;
  d.blocks_per_row = 2;
  d.capacity = 8;
  d.configured_eos = 151645;
  // The reference graph_config.json: decoder input descriptors (token [B,1],
  // ..., key_cache [L, P, bs, KVH, d], ..., block_table [B, BPR]).
  if (const Json* descs = cfg.get("inputs_tensor_desc")) {
    if (descs->kind != Json::kArray || descs->arr.size() != 9) return false;
    auto shape = [&](int i) -> std::vector<int> {
      std::vector<int> s;
      const Json* sh = descs->arr[i].get("shape");
      if (sh && sh->kind == Json::kArray)
        for (const Json& v : sh->arr) s.push_back(static_cast<int>(v.num));
      return s;
    };
    std::vector<int> tok = shape(0), kc = shape(3), table = shape(6);
    if (tok.size() < 1 || kc.size() != 5 || table.size() != 2) return false;
    d.batch = tok[0];
    d.layers = kc[0];
    d.physical_blocks = kc[1];
    d.block_size = kc[2];
    d.kv_heads = kc[3];
    d.head_dim = kc[4];
    d.blocks_per_row = table[1];
    const std::string dt = descs->arr[3].string_or("data_type", "DT_BFLOAT16");
    d.dtype_bytes = dt == "DT_FLOAT" ? 4 : 2;
  }
  if (const Json* m = cfg.get("model")) {
    d.layers = static_cast<int>(m->number_or("num_layers", d.layers));
    d.hidden = static_cast<int>(m->number_or("hidden", d.hidden));
    d.heads = static_cast<int>(m->number_or("num_heads", d.heads));
    d.kv_heads = static_cast<int>(m->number_or("num_kv_heads", d.kv_heads));
    d.head_dim = static_cast<int>(m->number_or("head_dim", d.head_dim));
    d.intermediate = static_cast<int>(m->number_or("intermediate", d.intermediate));
    d.vocab = static_cast<int>(m->number_or("vocab", d.vocab));
    d.rope_theta = static_cast<float>(m->number_or("rope_theta", d.rope_theta));
    d.rms_eps = static_cast<float>(m->number_or("rms_eps", d.rms_eps));
    const std::string dt = m->string_or("dtype", d.dtype_bytes == 4 ? "fp32" : "bf16");
    if (dt != "bf16" && dt != "fp32") return false;
    d.dtype_bytes = dt == "fp32" ? 4 : 2;
  }
  if (const Json* e = cfg.get("engine")) {
    d.batch = static_cast<int>(e->number_or("batch", d.batch));
    d.physical_blocks = static_cast<int>(e->number_or("physical_blocks", d.physical_blocks));
    d.block_size = static_cast<int>(e->number_or("block_size", d.block_size));
    d.blocks_per_row = static_cast<int>(e->number_or("blocks_per_row", d.blocks_per_row));
    d.capacity = static_cast<int>(e->number_or("logical_capacity", d.capacity));
    d.configured_eos = static_cast<int>(e->number_or("configured_eos", d.configured_eos));
  }
  const int G = d.kv_heads > 0 ? d.heads / d.kv_heads : 0;
  return d.layers > 0 && d.hidden > 0 && d.heads > 0 && d.kv_heads > 0 && d.heads % d.kv_heads == 0 &&
         G <= 8 && (d.head_dim == 64 || d.head_dim == 128 || d.head_dim == 256) && d.hidden % 8 == 0 &&
         d.intermediate % 8 == 0 && (d.heads * d.head_dim) % 8 == 0 && d.vocab > 0 && d.vocab % 2 == 0 &&
         d.hidden % 2 == 0 && d.batch >= 1 && d.batch <= 256 && d.physical_blocks >= 1 &&
         d.block_size >= 1 && d.blocks_per_row >= 1 && d.capacity >= 1 &&
         d.capacity <= d.blocks_per_row * d.block_size && d.capacity <= 8192 &&
         (static_cast<long long>(d.block_size) * d.kv_heads * d.head_dim * d.dtype_bytes) % 16 == 0;
}

int balance(int groups, int resident) {
  if (groups <= resident) return groups;
  const int iters = (groups + resident - 1) / resident;
  return (groups + iters - 1) / iters;
}

bool make_plan(Engine& e, const Json& cfg) {
  const Dims& d = e.dims;
  LaunchPlan& p = e.plan;
  p.mb = d.batch <= 4 ? 4 : 8;
  p.row_tiles = (d.batch + p.mb - 1) / p.mb;
  p.waves = 4;
  // Normed projections hold the whole hidden row in one K-segment; the row
  // kernels hold it as one 8-element vector per thread.
  if (d.hidden > k_segment_elems() || d.hidden > row_kernel_max_hidden() || d.hidden % 8 != 0) return false;
  if (d.head_dim % 2 != 0) return false;
  const size_t normed_lds = normed_lds_bytes(p.mb, d.hidden, d.dtype_bytes, p.waves);
  if (normed_lds > 64 * 1024 || resid_lds_bytes(p.mb, d.dtype_bytes, p.waves) > 64 * 1024) return false;
  // attention: scores of the window + P.V partials + block table, plus 16 bytes of static LDS
  if (attention_lds_bytes(d) > 160 * 1024 - 64 || prepare_attention(d) != hipSuccess) return false;
  // cache offsets of one layer are 32-bit in the attention kernel
  if ((long long)d.slots() * d.kv_dim() >= (1LL << 31)) return false;
  plan_grids(p, d, e.cus);
  // "tuning": {"qkv_ksplit": 0} runs qkv as one row pair per wave over the
  // whole K (the general path) where the K-split kernel applies: a
  // cross-check of the two, whose fp32 sums run in different orders.
  if (const Json* t = cfg.get("tuning"))
    if (t->number_or("qkv_ksplit", 1) == 0) p.qkv_ksplit = 0;
  const Json* tune = cfg.get("tuning");
  // 64 bf16 rows of Qwen2.5-7B's shape: projections on the matrix cores,
  // gate/up and the LM head one workgroup per CU, qkv, o and down split over
  // (strip group, K range) (re_mfma.hip); "tuning": {"mfma": 0} keeps the
  // row-tiled kernels
  p.mfma = 0;
  p.gu_cu = 0;
  if (mfma_step_supported(d) && mfma_lm_cu_fits(d, e.cus) && mfma_gu_cu_fits(d, e.cus) && mfma_qkv_split_fits(d) &&
      (tune == nullptr || tune->number_or("mfma", 1) != 0) && prepare_mfma() == hipSuccess) {
    p.mfma = 1;
    p.gu_cu = e.cus;
    p.lm_wg = e.cus;  // k_mf_lm_cu's workgroups
  }
  // the matrix-core LM head leaves one argmax partial per (row, CU), row-major
  p.argmax_parts = p.mfma ? e.cus : p.lm_wg;
  p.argmax_row_major = p.mfma;
  // grouped decode attention: by default for many rows; "tuning":
  // {"grouped_attention": 0 or 1} forces it where the shape allows it
  p.grouped_attn = group_attention_default(d) ? 1 : 0;
  if (tune != nullptr && group_attention_fits(d))
    p.grouped_attn = static_cast<int>(tune->number_or("grouped_attention", p.grouped_attn)) != 0 ? 1 : 0;
  // the grouped attention's products on the matrix cores ("tuning":
  // {"attention_mfma": 0} keeps the vector-unit version)
  if (p.grouped_attn && group_attention_mfma_fits(d) &&
      (tune == nullptr || tune->number_or("attention_mfma", 1) != 0))
    p.grouped_attn = 2;
  // Decode attention split over the window in 256-position tiles (three
  // launches of one tile per workgroup; "tuning": {"attention_split": 0 or
  // 1} forces it off or on):
  // - per (row, head): by default past 768 positions, where it beats walking
  //   the tiles in a row;
  // - on the matrix cores per (row, KV head): by default only for many rows
  //   whose window is past the single-launch grouped kernels' LDS (at 1,024
  //   positions the single launch is faster: 40.4 against 49.8 us at 64
  //   rows); "grouped_attention": 0 or "attention_mfma": 0 keep the
  //   per-head split there.
  p.attn_split = 0;
  const int split_tiles = (d.capacity + 255) / 256;
  if (p.grouped_attn == 0) {
    const bool many_rows = d.batch * d.kv_heads >= 64;
    if (many_rows && !group_attention_fits(d) && group_attention_msplit_fits(d) &&
        (tune == nullptr ||
         (tune->number_or("grouped_attention", 1) != 0 && tune->number_or("attention_mfma", 1) != 0 &&
          tune->number_or("attention_split", 1) != 0))) {
      p.grouped_attn = 2;
      p.attn_split = split_tiles;
    } else {
      bool split = d.capacity > 768;
      if (tune != nullptr) split = tune->number_or("attention_split", split ? 1 : 0) != 0;
      if (split) p.attn_split = split_tiles;
    }
  } else if (p.grouped_attn == 2 && group_attention_msplit_fits(d) && tune != nullptr &&
             tune->number_or("attention_split", 0) != 0) {
    p.attn_split = split_tiles;
  }
  p.o_grid = (d.hidden / 2 + p.waves - 1) / p.waves;
  p.down_grid = p.o_grid;
  p.o_segments = (d.q_dim() + k_segment_elems() - 1) / k_segment_elems();
  p.down_segments = (d.intermediate + k_segment_elems() - 1) / k_segment_elems();
  // o-proj with exactly seven row pairs per CU (Qwen2.5-7B: 1,792 on 256
  // CUs): one 7-wave workgroup per CU; otherwise 4-wave workgroups
  p.o_waves = p.waves;
  if (d.dtype_bytes == 2 && p.mb == 4 && p.o_segments == 1 && d.hidden / 2 == 7 * e.cus) p.o_waves = 7;
  p.o_grid = (d.hidden / 2 + p.o_waves - 1) / p.o_waves;
  return true;
}

void layout_weights(Engine& e) {
  const Dims& d = e.dims;
  const size_t T = d.dtype_bytes;
  size_t off = 0;
  auto add = [&](const std::string& name, long long elems, bool streamed) -> size_t {
    const size_t at = off;
    e.weight_slots[name] = WeightSlot{at, (size_t)elems * T, elems};
    e.weight_order.push_back(name);
    off = align_up(off + (size_t)elems * T, 256);
    if (streamed) e.streamed_weight_bytes += (size_t)elems * T;
    return at;
  };
  e.embedding_off = add("embedding", (long long)d.vocab * d.hidden, false);
  e.layer_off.resize(d.layers);
  for (int l = 0; l < d.layers; ++l) {
    const std::string p = "layers_" + std::to_string(l) + "_";
    LayerOffsets& lo = e.layer_off[l];
    lo.input_norm = add(p + "input_norm", d.hidden, true);
    lo.post_norm = add(p + "post_norm", d.hidden, true);
    // q, k, v rows stacked into one matrix (and biases into one vector).
    const size_t qkv_bytes = (size_t)d.qkv_rows() * d.hidden * T;
    lo.qkv_w = off;
    e.weight_slots[p + "q_weight"] = WeightSlot{off, (size_t)d.q_dim() * d.hidden * T, (long long)d.q_dim() * d.hidden};
    e.weight_slots[p + "k_weight"] = WeightSlot{off + (size_t)d.q_dim() * d.hidden * T, (size_t)d.kv_dim() * d.hidden * T,
                                                (long long)d.kv_dim() * d.hidden};
    e.weight_slots[p + "v_weight"] = WeightSlot{off + (size_t)(d.q_dim() + d.kv_dim()) * d.hidden * T,
                                                (size_t)d.kv_dim() * d.hidden * T, (long long)d.kv_dim() * d.hidden};
    e.weight_order.push_back(p + "q_weight");
    e.weight_order.push_back(p + "k_weight");
    e.weight_order.push_back(p + "v_weight");
    off = align_up(off + qkv_bytes, 256);
    e.streamed_weight_bytes += qkv_bytes;
    lo.qkv_b = off;
    e.weight_slots[p + "q_bias"] = WeightSlot{off, (size_t)d.q_dim() * T, d.q_dim()};
    e.weight_slots[p + "k_bias"] = WeightSlot{off + (size_t)d.q_dim() * T, (size_t)d.kv_dim() * T, d.kv_dim()};
    e.weight_slots[p + "v_bias"] = WeightSlot{off + (size_t)(d.q_dim() + d.kv_dim()) * T, (size_t)d.kv_dim() * T, d.kv_dim()};
    e.weight_order.push_back(p + "q_bias");
    e.weight_order.push_back(p + "k_bias");
    e.weight_order.push_back(p + "v_bias");
    off = align_up(off + (size_t)d.qkv_rows() * T, 256);
    e.streamed_weight_bytes += (size_t)d.qkv_rows() * T;
    lo.o_w = add(p + "o_weight", (long long)d.hidden * d.q_dim(), true);
    lo.gate_w = add(p + "gate_weight", (long long)d.intermediate * d.hidden, true);
    lo.up_w = add(p + "up_weight", (long long)d.intermediate * d.hidden, true);
    lo.down_w = add(p + "down_weight", (long long)d.hidden * d.intermediate, true);
  }
  e.final_norm_off = add("final_norm", d.hidden, true);
  e.lm_head_off = add("lm_head", (long long)d.vocab * d.hidden, true);
  e.weight_bytes = off;
}

// The packed copy of the matrix a weight slot belongs to, refreshed after the
// slot is written (matrix-core plan only; other slots have no copy).
hipError_t repack_slot(Engine& e, const std::string& name) {
  if (!e.plan.mfma) return hipSuccess;
  const Dims& d = e.dims;
  if (name == "lm_head")
    return mfma_pack_matrix(e.weights + e.lm_head_off, e.packed + e.packed_lm_off, d.vocab, d.hidden, 0, e.stream);
  if (name.rfind("layers_", 0) != 0) return hipSuccess;
  const size_t us = name.find('_', 7);
  if (us == std::string::npos) return hipSuccess;
  const int l = std::atoi(name.substr(7, us - 7).c_str());
  if (l < 0 || l >= d.layers) return hipSuccess;
  const std::string what = name.substr(us + 1);
  const LayerOffsets& lo = e.layer_off[l];
  const PackedOffsets& po = e.packed_off[l];
  if (what == "q_weight" || what == "k_weight" || what == "v_weight")
    return mfma_pack_matrix(e.weights + lo.qkv_w, e.packed + po.qkv, d.qkv_rows(), d.hidden, d.head_dim, e.stream);
  if (what == "o_weight")
    return mfma_pack_matrix(e.weights + lo.o_w, e.packed + po.o, d.hidden, d.q_dim(), 0, e.stream);
  if (what == "gate_weight")
    return mfma_pack_matrix(e.weights + lo.gate_w, e.packed + po.gate, d.intermediate, d.hidden, 0, e.stream);
  if (what == "up_weight")
    return mfma_pack_matrix(e.weights + lo.up_w, e.packed + po.up, d.intermediate, d.hidden, 0, e.stream);
  if (what == "down_weight")
    return mfma_pack_matrix(e.weights + lo.down_w, e.packed + po.down, d.hidden, d.intermediate, 0, e.stream);
  return hipSuccess;
}

bool repack_all(Engine& e) {
  if (!e.plan.mfma) return true;
  for (int l = 0; l < e.dims.layers; ++l) {
    const std::string p = "layers_" + std::to_string(l) + "_";
    for (const char* w : {"q_weight", "o_weight", "gate_weight", "up_weight", "down_weight"})
      if (repack_slot(e, p + w) != hipSuccess) return false;
  }
  return repack_slot(e, "lm_head") == hipSuccess && hipStreamSynchronize(e.stream) == hipSuccess;
}

bool alloc_state(Engine& e) {
  const Dims& d = e.dims;
  const int B = d.batch;
  e.feed_bytes = 8 * B + 8 * B + 4 * B + 4 * B + 4 * B + 4 * (size_t)B * d.blocks_per_row + kTilingBytes + 4 * (3 + 2 * B);
  e.payload_bytes = 2ULL * d.layers * B * d.block_size * d.kv_dim() * d.dtype_bytes;
  e.import_feed_bytes = e.payload_bytes + e.feed_bytes - 4 * B;
  e.fetch_bytes = 8 * kMaxEpochSteps * B + 4 * (6 + 4 * B + 2 + B);

  // state buffer
  size_t off = 0;
  std::vector<std::pair<void**, size_t>> parts;
  auto part = [&](void** p, size_t bytes) { parts.push_back({p, bytes}); };
  part(reinterpret_cast<void**>(&e.st.feed), align_up(e.import_feed_bytes, 256));
  part(reinterpret_cast<void**>(&e.st.cur_token), 8 * B);
  part(reinterpret_cast<void**>(&e.st.cur_pos), 8 * B);
  part(reinterpret_cast<void**>(&e.st.cur_len), 4 * B);
  part(reinterpret_cast<void**>(&e.st.cur_slot), 4 * B);
  part(reinterpret_cast<void**>(&e.st.cur_active), 4 * B);
  part(reinterpret_cast<void**>(&e.st.table), 4 * (size_t)B * d.blocks_per_row);
  part(reinterpret_cast<void**>(&e.st.done), 4);
  part(reinterpret_cast<void**>(&e.st.status), 4);
  part(reinterpret_cast<void**>(&e.st.model_calls), 4);
  part(reinterpret_cast<void**>(&e.st.executed), 4 * B);
  part(reinterpret_cast<void**>(&e.st.reason), 4 * B);
  part(reinterpret_cast<void**>(&e.st.clear_row), 4 * B);
  part(reinterpret_cast<void**>(&e.st.eos), 4 * B);
  part(reinterpret_cast<void**>(&e.st.initial_active), 4 * B);
  part(reinterpret_cast<void**>(&e.st.generation), 4 * B);
  part(reinterpret_cast<void**>(&e.st.misc), 4 * 8);
  part(reinterpret_cast<void**>(&e.st.res_gen), 4 * B);
  part(reinterpret_cast<void**>(&e.st.res_token), 8 * B);
  part(reinterpret_cast<void**>(&e.st.res_pos), 8 * B);
  part(reinterpret_cast<void**>(&e.st.res_len), 4 * B);
  part(reinterpret_cast<void**>(&e.st.res_valid), 4 * B);
  part(reinterpret_cast<void**>(&e.st.fetch), e.fetch_bytes);
  std::vector<size_t> offs;
  for (auto& pr : parts) {
    offs.push_back(off);
    off = align_up(off + pr.second, 256);
  }
  if (hipMalloc(&e.state_mem, off) != hipSuccess) return false;
  if (hipMemset(e.state_mem, 0, off) != hipSuccess) return false;
  for (size_t i = 0; i < parts.size(); ++i) *parts[i].first = e.state_mem + offs[i];

  // scratch
  const LaunchPlan& p = e.plan;
  const size_t T = d.dtype_bytes;
  struct Part {
    void** p;
    size_t bytes;
  };
  std::vector<Part> sp = {
      {&e.scratch.hidden, (size_t)B * d.hidden * T},
      {&e.scratch.q, (size_t)B * d.q_dim() * T},
      {&e.scratch.attn, (size_t)B * d.q_dim() * T},
      {&e.scratch.mlp, (size_t)B * d.intermediate * T},
      {reinterpret_cast<void**>(&e.scratch.partial),
       (size_t)std::max(p.down_segments, p.o_segments) * B * d.hidden * sizeof(float)},
      {reinterpret_cast<void**>(&e.scratch.am_val), (size_t)p.lm_wg * B * sizeof(float)},
      {reinterpret_cast<void**>(&e.scratch.am_idx), (size_t)p.lm_wg * B * sizeof(int32_t)},
      {reinterpret_cast<void**>(&e.scratch.am_bad), (size_t)p.lm_wg * B * sizeof(int32_t)},
      {reinterpret_cast<void**>(&e.scratch.inv_freq), (size_t)d.head_dim / 2 * sizeof(float)},
      {reinterpret_cast<void**>(&e.scratch.rope), (size_t)B * d.head_dim * sizeof(float)},
      {&e.scratch.xn, p.mfma ? (size_t)B * d.hidden * T : 0},
      {reinterpret_cast<void**>(&e.scratch.mf_part), p.mfma ? mfma_split_partial_bytes(d) : 0},
      {reinterpret_cast<void**>(&e.scratch.sp_scores), (size_t)p.attn_split * 256 * B * d.heads * sizeof(float)},
      {reinterpret_cast<void**>(&e.scratch.sp_stats), (size_t)p.attn_split * 2 * B * d.heads * sizeof(float)},
      {reinterpret_cast<void**>(&e.scratch.sp_part),
       (size_t)p.attn_split * d.head_dim * B * d.heads * sizeof(float)},
      {reinterpret_cast<void**>(&e.logits), (size_t)B * d.vocab * sizeof(float)},
      {reinterpret_cast<void**>(&e.checksum_dev), 64},
  };
  off = 0;
  offs.clear();
  for (auto& pr : sp) {
    offs.push_back(off);
    off = align_up(off + pr.bytes, 256);
  }
  if (hipMalloc(&e.scratch_mem, off) != hipSuccess) return false;
  if (hipMemset(e.scratch_mem, 0, off) != hipSuccess) return false;
  for (size_t i = 0; i < sp.size(); ++i) *sp[i].p = e.scratch_mem + offs[i];
  e.st.import_sum = e.checksum_dev;

  // decoder-step ABI inputs
  std::vector<Part> io = {
      {reinterpret_cast<void**>(const_cast<int64_t**>(&e.step_io.token)), 8 * (size_t)B},
      {reinterpret_cast<void**>(const_cast<int64_t**>(&e.step_io.pos)), 8 * (size_t)B},
      {reinterpret_cast<void**>(const_cast<int32_t**>(&e.step_io.len)), 4 * (size_t)B},
      {reinterpret_cast<void**>(const_cast<int32_t**>(&e.step_io.slot)), 4 * (size_t)B},
      {reinterpret_cast<void**>(const_cast<int32_t**>(&e.step_io.active)), 4 * (size_t)B},
      {reinterpret_cast<void**>(const_cast<int32_t**>(&e.step_io.table)), 4 * (size_t)B * d.blocks_per_row},
      {reinterpret_cast<void**>(&e.step_io.next_pos), 8 * (size_t)B},
  };
  off = 0;
  offs.clear();
  for (auto& pr : io) {
    offs.push_back(off);
    off = align_up(off + pr.bytes, 256);
  }
  if (hipMalloc(&e.step_mem, off) != hipSuccess) return false;
  if (hipMemset(e.step_mem, 0, off) != hipSuccess) return false;
  for (size_t i = 0; i < io.size(); ++i) *io[i].p = e.step_mem + offs[i];

  // inv_freq = 1 / theta^(2i/d) (batched_decoder_step.py:213-216), fp32
  std::vector<float> inv(d.head_dim / 2);
  for (int i = 0; i < d.head_dim / 2; ++i)
    inv[i] = static_cast<float>(1.0 / std::pow(static_cast<double>(d.rope_theta),
                                               static_cast<double>(static_cast<float>(2 * i) / d.head_dim)));
  if (hipMemcpy(e.scratch.inv_freq, inv.data(), inv.size() * sizeof(float), hipMemcpyHostToDevice) != hipSuccess)
    return false;

  // caches
  e.cache_bytes = (size_t)d.cache_elems() * T;
  if (hipMalloc(&e.key_cache, e.cache_bytes) != hipSuccess) return false;
  if (hipMalloc(&e.value_cache, e.cache_bytes) != hipSuccess) return false;
  if (hipMemset(e.key_cache, 0, e.cache_bytes) != hipSuccess) return false;  // CTRL:258-261
  if (hipMemset(e.value_cache, 0, e.cache_bytes) != hipSuccess) return false;

  // pinned host staging
  if (hipHostMalloc(reinterpret_cast<void**>(&e.h_feed), align_up(e.import_feed_bytes, 4096), 0) != hipSuccess)
    return false;
  if (hipHostMalloc(reinterpret_cast<void**>(&e.h_fetch), align_up(e.fetch_bytes, 4096), 0) != hipSuccess)
    return false;
  std::memset(e.h_feed, 0, e.import_feed_bytes);
  std::memset(e.h_fetch, 0, e.fetch_bytes);
  return true;
}

bool load_bundle(Engine& e, const std::string& dir) {
  const size_t chunk = 64u << 20;
  uint8_t* staging = nullptr;
  if (hipHostMalloc(reinterpret_cast<void**>(&staging), chunk, 0) != hipSuccess) return false;
  bool ok = true;
  for (const std::string& name : e.weight_order) {
    const WeightSlot& ws = e.weight_slots[name];
    std::ifstream f(dir + "/" + name, std::ios::binary | std::ios::ate);
    if (!f || static_cast<size_t>(f.tellg()) != ws.bytes) {
      ok = false;
      break;
    }
    f.seekg(0);
    size_t done = 0;
    while (done < ws.bytes) {
      const size_t n = std::min(chunk, ws.bytes - done);
      f.read(reinterpret_cast<char*>(staging), n);
      if (!f || hipMemcpy(e.weights + ws.offset + done, staging, n, hipMemcpyHostToDevice) != hipSuccess) {
        ok = false;
        break;
      }
      done += n;
    }
    if (!ok) break;
  }
  if (ok) {  // optional derived inv_freq (materialize_runtime_weights.py:341-353)
    std::ifstream f(dir + "/inv_freq", std::ios::binary | std::ios::ate);
    if (f && static_cast<size_t>(f.tellg()) == (size_t)e.dims.head_dim / 2 * sizeof(float)) {
      std::vector<float> inv(e.dims.head_dim / 2);
      f.seekg(0);
      f.read(reinterpret_cast<char*>(inv.data()), inv.size() * sizeof(float));
      // a present but unreadable file fails the load rather than leaving the
      // computed frequencies in place silently
      if (!f || hipMemcpy(e.scratch.inv_freq, inv.data(), inv.size() * sizeof(float), hipMemcpyHostToDevice) !=
                    hipSuccess)
        ok = false;
    }
  }
  (void)hipHostFree(staging);
  return ok;
}

bool load_synthetic(Engine& e, unsigned long long seed, float std_dev) {
  unsigned long long stream_id = 0;
  for (const std::string& name : e.weight_order) {
    const WeightSlot& ws = e.weight_slots[name];
    if (launch_fill_synthetic(e.weights + ws.offset, ws.elems, e.dims.dtype_bytes, seed, stream_id++, std_dev,
                              e.stream) != hipSuccess)
      return false;
  }
  return hipStreamSynchronize(e.stream) == hipSuccess;
}

StepPtrs epoch_step_ptrs(const Engine& e) {
  StepPtrs s{};
  s.token = e.st.cur_token;
  s.pos = e.st.cur_pos;
  s.len = e.st.cur_len;
  s.slot = e.st.cur_slot;
  s.active = e.st.cur_active;
  s.table = e.st.table;
  s.key_cache = e.key_cache;
  s.value_cache = e.value_cache;
  s.logits = e.logits;
  s.next_pos = nullptr;
  s.done = e.st.done;
  return s;
}

// part 0: the whole epoch -- feed copy, init, row clear, K x (step, ctrl_step),
// finish, fetch copy.  part 1: everything before the timed launch (the
// gate/up projection of timing_layer in the last step); part 2: everything
// after it.
// How the epoch's inputs reach the device feed: the plain feed, an import
// feed with its payload copied from the host (transfer file or the 8-input
// ABI), or an import feed whose payload the device-IPC gather has already
// written (only the part after the payload is copied).
enum FeedMode : int { kFeedPlain = 0, kFeedHostImport = 1, kFeedDeviceImport = 2 };

hipError_t record_epoch(Engine& e, int K, FeedMode mode, int part) {
  const bool importing = mode != kFeedPlain;
  const KernelEnv env = e.env();
  const int nops = step_op_count(env);
  const int split = timed_op_index(env, e.timing_layer);
  hipError_t err = hipSuccess;
  if (part != 2) {
    const size_t skip = mode == kFeedDeviceImport ? e.payload_bytes : 0;
    const size_t feed = (importing ? e.import_feed_bytes : e.feed_bytes) - skip;
    if ((err = hipMemcpyAsync(e.st.feed + skip, e.h_feed + skip, feed, hipMemcpyHostToDevice, e.stream)) !=
        hipSuccess)
      return err;
    if ((err = launch_ctrl_init(env, e.st, importing ? 1 : 0, e.stream)) != hipSuccess) return err;
    if ((err = launch_clear_rows(env, e.st, e.key_cache, e.value_cache, e.stream)) != hipSuccess) return err;
    if (importing &&
        (err = launch_import_checksum(env, e.st, e.key_cache, e.value_cache, e.stream)) != hipSuccess)
      return err;
  }
  const StepPtrs sp = epoch_step_ptrs(e);
  for (int k = 0; k < K; ++k) {
    const bool last = k == K - 1;
    if (part == 2 && !last) continue;
    int begin = 0, end = nops;
    if (last && part == 1) end = split;
    if (last && part == 2) begin = split + 1;
    if ((err = launch_step_ops(env, sp, e.stream, begin, end)) != hipSuccess) return err;
    if (!(last && part == 1) && (err = launch_ctrl_step(env, e.st, e.stream)) != hipSuccess) return err;
  }
  if (part == 1) return hipSuccess;
  if ((err = launch_ctrl_finish(env, e.st, e.stream)) != hipSuccess) return err;
  return hipMemcpyAsync(e.h_fetch, e.st.fetch, e.fetch_bytes, hipMemcpyDeviceToHost, e.stream);
}

int graph_key(int K, FeedMode mode, int part) { return (K * 3 + mode) * 4 + part; }

// The nodes of a captured graph by kind, read from the graph: {memory copies,
// memsets, kernels}.  (The direction of a captured copy is not reported by
// every HIP runtime's node query, so only copies are counted here; the
// kernel trace shows each copy's transfer.)
std::array<int, 3> count_nodes(hipGraph_t graph) {
  std::array<int, 3> c{{0, 0, 0}};
  size_t n = 0;
  if (hipGraphGetNodes(graph, nullptr, &n) != hipSuccess) return {{-1, -1, -1}};
  std::vector<hipGraphNode_t> nodes(n);
  if (n > 0 && hipGraphGetNodes(graph, nodes.data(), &n) != hipSuccess) return {{-1, -1, -1}};
  for (hipGraphNode_t node : nodes) {
    hipGraphNodeType type{};
    if (hipGraphNodeGetType(node, &type) != hipSuccess) return {{-1, -1, -1}};
    if (type == hipGraphNodeTypeMemcpy) ++c[0];
    else if (type == hipGraphNodeTypeMemset) ++c[1];
    else if (type == hipGraphNodeTypeKernel) ++c[2];
  }
  return c;
}

hipGraphExec_t epoch_graph(Engine& e, int K, FeedMode mode, int part) {
  const int key = graph_key(K, mode, part);
  auto it = e.graphs.find(key);
  if (it != e.graphs.end()) return it->second;
  hipGraph_t graph = nullptr;
  if (hipStreamBeginCapture(e.stream, hipStreamCaptureModeThreadLocal) != hipSuccess) return nullptr;
  hipError_t rec = record_epoch(e, K, mode, part);
  hipError_t end = hipStreamEndCapture(e.stream, &graph);
  if (rec != hipSuccess || end != hipSuccess || graph == nullptr) {
    if (graph) (void)hipGraphDestroy(graph);
    return nullptr;
  }
  hipGraphExec_t exec = nullptr;
  if (hipGraphInstantiateWithFlags(&exec, graph, 0) != hipSuccess) {
    (void)hipGraphDestroy(graph);
    return nullptr;
  }
  e.graphs[key] = exec;
  e.graph_defs[key] = graph;
  e.graph_copies[key] = count_nodes(graph);
  return exec;
}

void drop_graphs(Engine& e) {
  for (auto& kv : e.graphs) (void)hipGraphExecDestroy(kv.second);
  for (auto& kv : e.graph_defs) (void)hipGraphDestroy(kv.second);
  e.graphs.clear();
  e.graph_defs.clear();
}

void free_engine(Engine* e) {
  if (!e) return;
  drop_graphs(*e);
  if (e->ev_start) (void)hipEventDestroy(e->ev_start);
  if (e->ev_stop) (void)hipEventDestroy(e->ev_stop);
  if (e->weights) (void)hipFree(e->weights);
  if (e->packed) (void)hipFree(e->packed);
  if (e->key_cache) (void)hipFree(e->key_cache);
  if (e->value_cache) (void)hipFree(e->value_cache);
  if (e->state_mem) (void)hipFree(e->state_mem);
  if (e->scratch_mem) (void)hipFree(e->scratch_mem);
  if (e->step_mem) (void)hipFree(e->step_mem);
  if (e->dec_key) (void)hipFree(e->dec_key);
  if (e->dec_value) (void)hipFree(e->dec_value);
  if (e->h_feed) (void)hipHostFree(e->h_feed);
  if (e->h_fetch) (void)hipHostFree(e->h_fetch);
  for (auto& kv : e->ipc_maps) (void)hipIpcCloseMemHandle(kv.second.ptr);
  if (e->pf_mem) (void)hipFree(e->pf_mem);
  if (e->stream) (void)hipStreamDestroy(e->stream);
  delete e;
}

// Identity block table and slot of the bridge (resident_epoch_bridge.cpp:350-357, 524-532).
int32_t bridge_slot(const Dims& d, int row, int64_t position) {
  if (row < 0 || row >= d.batch || position < 0 || position >= d.capacity) return -1;
  return row * d.blocks_per_row * d.block_size + static_cast<int32_t>(position);
}

uint8_t* put(uint8_t* p, const void* src, size_t n) {
  std::memcpy(p, src, n);
  return p + n;
}

#pragma pack(push, 1)
struct TransferHeader {  // resident_epoch_bridge.cpp:72-89
  uint64_t magic;
  uint32_t version;
  uint32_t header_bytes;
  uint64_t transfer_id;
  uint64_t payload_bytes;
  uint32_t import_mask;
  int32_t row_generations[4];
  uint32_t layers;
  uint32_t batch_size;
  uint32_t block_size;
  uint32_t kv_heads;
  uint32_t head_size;
  uint32_t element_bytes;
  uint32_t checksum;
};
#pragma pack(pop)
static_assert(sizeof(TransferHeader) == CRUISE_RESIDENT_TRANSFER_HEADER_BYTES, "transfer header ABI");
static_assert(sizeof(ResidentEpochIpcMetadata) == CRUISE_RESIDENT_IPC_METADATA_BYTES, "IPC metadata ABI");

// ReadTransfer (resident_epoch_bridge.cpp:108-154): header checks, then the
// payload straight into the pinned import feed.
bool read_transfer(Engine& e, const char* path, uint64_t transfer_id, const int32_t* gens, int32_t& import_mask,
                   uint32_t& expected_checksum) {
  const Dims& d = e.dims;
  if (path == nullptr || gens == nullptr || transfer_id == 0 || std::strncmp(path, "/dev/shm/", 9) != 0 ||
      d.batch != 4)
    return false;
  std::ifstream f(path, std::ios::binary | std::ios::ate);
  if (!f || static_cast<size_t>(f.tellg()) != sizeof(TransferHeader) + e.payload_bytes) return false;
  f.seekg(0);
  TransferHeader h{};
  f.read(reinterpret_cast<char*>(&h), sizeof(h));
  if (!f || h.magic != CRUISE_RESIDENT_TRANSFER_MAGIC || h.version != CRUISE_RESIDENT_TRANSFER_VERSION ||
      h.header_bytes != CRUISE_RESIDENT_TRANSFER_HEADER_BYTES || h.transfer_id != transfer_id ||
      h.payload_bytes != e.payload_bytes || h.import_mask == 0 || h.import_mask >= (1u << d.batch) ||
      h.layers != (uint32_t)d.layers || h.batch_size != (uint32_t)d.batch ||
      h.block_size != (uint32_t)d.block_size || h.kv_heads != (uint32_t)d.kv_heads ||
      h.head_size != (uint32_t)d.head_dim || h.element_bytes != (uint32_t)d.dtype_bytes || h.checksum == 0)
    return false;
  for (int r = 0; r < d.batch; ++r) {
    const bool selected = (h.import_mask & (1u << r)) != 0;
    if (selected) {
      if (h.row_generations[r] <= 0 || h.row_generations[r] != gens[r]) return false;
    } else if (h.row_generations[r] != 0) {
      return false;
    }
  }
  f.read(reinterpret_cast<char*>(e.h_feed), e.payload_bytes);
  if (!f) return false;
  import_mask = static_cast<int32_t>(h.import_mask);
  expected_checksum = h.checksum;
  return true;
}

// Exported allocations of 2 GiB or more are refused: opening such a handle
// has been seen not to return on the ROCm 7 dmabuf IPC path.
constexpr uint64_t kIpcMaxSourceBytes = 2ULL << 30;

// The mapping of one exported allocation, opened once per engine.
const Engine::IpcMapping* ipc_mapping(Engine& e, const char (&key)[CRUISE_RESIDENT_IPC_KEY_BYTES],
                                      uint64_t source_bytes) {
  const std::string id(key, CRUISE_RESIDENT_IPC_KEY_BYTES);
  auto it = e.ipc_maps.find(id);
  if (it == e.ipc_maps.end()) {
    hipIpcMemHandle_t handle;
    static_assert(sizeof(handle) == CRUISE_RESIDENT_IPC_KEY_BYTES, "HIP IPC handle size");
    std::memcpy(&handle, key, sizeof(handle));
    void* ptr = nullptr;
    if (hipIpcOpenMemHandle(&ptr, handle, hipIpcMemLazyEnablePeerAccess) != hipSuccess || ptr == nullptr) {
      (void)hipGetLastError();
      return nullptr;
    }
    hipDeviceptr_t base = nullptr;
    size_t bytes = 0;
    if (hipMemGetAddressRange(&base, &bytes, ptr) != hipSuccess || base != ptr) {
      (void)hipGetLastError();
      (void)hipIpcCloseMemHandle(ptr);
      return nullptr;
    }
    it = e.ipc_maps.emplace(id, Engine::IpcMapping{ptr, bytes}).first;
  }
  // every source range was checked against source_bytes; the mapping must hold them
  return it->second.bytes >= source_bytes ? &it->second : nullptr;
}

// ValidateIpcMetadata + PrepareDeviceIpcPayload (resident_epoch_bridge.cpp:
// 156-243): check the record against the engine's geometry and the rows'
// generations, map the exported allocations, and gather the imported blocks
// into the device feed's payload region on the engine stream.  Cache slots
// past 2 x layers (models with fewer than 28 layers) must be all zero.
bool prepare_device_import(Engine& e, const ResidentEpochIpcMetadata* m, const int32_t* gens, int32_t& import_mask) {
  const Dims& d = e.dims;
  constexpr int kRows = 4;
  const int caches = 2 * d.layers;
  const uint64_t block_bytes = (uint64_t)d.block_size * d.kv_dim() * d.dtype_bytes;
  if (d.batch != kRows || caches > CRUISE_RESIDENT_IPC_KEY_COUNT || caches > kImportMaxCaches || block_bytes % 16 != 0)
    return false;
  if (m->magic != CRUISE_RESIDENT_IPC_METADATA_MAGIC || m->version != CRUISE_RESIDENT_IPC_METADATA_VERSION ||
      m->import_mask == 0 || m->import_mask >= (1u << kRows) || m->source_bytes >= kIpcMaxSourceBytes ||
      m->source_bytes < (uint64_t)d.physical_blocks * block_bytes)
    return false;
  ImportGatherArgs g{};
  for (int r = 0; r < kRows; ++r) {
    const bool selected = (m->import_mask >> r) & 1u;
    if (selected) {
      if (m->row_generations[r] <= 0 || m->row_generations[r] != gens[r] || m->block_ids[r] < 0) return false;
      g.rows[g.nrows++] = r;
    } else if (m->row_generations[r] != 0 || m->block_ids[r] != 0) {
      return false;
    }
    g.block_ids[r] = m->block_ids[r];
  }
  for (int c = 0; c < CRUISE_RESIDENT_IPC_KEY_COUNT; ++c) {
    const char* key = m->keys[c];
    const bool key_set = std::any_of(key, key + CRUISE_RESIDENT_IPC_KEY_BYTES, [](char v) { return v != 0; });
    const uint64_t off = m->source_offsets[c];
    if (c >= caches) {
      if (key_set || off != 0) return false;
      continue;
    }
    if (!key_set || off % 16 != 0 || off > m->source_bytes) return false;
    for (int k = 0; k < g.nrows; ++k) {
      const uint64_t end = ((uint64_t)m->block_ids[g.rows[k]] + 1) * block_bytes;
      if (end > m->source_bytes - off) return false;
    }
  }
  for (int c = 0; c < caches; ++c) {
    const Engine::IpcMapping* map = ipc_mapping(e, m->keys[c], m->source_bytes);
    if (map == nullptr) return false;
    g.src[c] = static_cast<const uint8_t*>(map->ptr) + m->source_offsets[c];
  }
  g.dst = e.st.feed;
  g.layers = d.layers;
  g.batch = d.batch;
  g.block_bytes = static_cast<long long>(block_bytes);
  if (launch_import_gather(g, e.stream) != hipSuccess) return false;
  import_mask = static_cast<int32_t>(m->import_mask);
  return true;
}

// Launch one epoch.  Without timing it is one graph; with timing it is graph
// part 1, the timed gate/up launch between two events, graph part 2 -- all on
// the engine stream, still one feed copy and one fetch copy.
bool run_graph(Engine& e, int K, FeedMode mode) {
  if (!e.timing) {
    hipGraphExec_t g = epoch_graph(e, K, mode, 0);
    if (g == nullptr) return false;
    e.last_epoch_copies = e.graph_copies[graph_key(K, mode, 0)];
    return hipGraphLaunch(g, e.stream) == hipSuccess;
  }
  hipGraphExec_t pre = epoch_graph(e, K, mode, 1);
  hipGraphExec_t post = epoch_graph(e, K, mode, 2);
  if (pre == nullptr || post == nullptr) return false;
  const std::array<int, 3>& c1 = e.graph_copies[graph_key(K, mode, 1)];
  const std::array<int, 3>& c2 = e.graph_copies[graph_key(K, mode, 2)];
  for (int i = 0; i < 3; ++i) e.last_epoch_copies[i] = c1[i] + c2[i];
  const int op = timed_op_index(e.env(), e.timing_layer);
  return hipGraphLaunch(pre, e.stream) == hipSuccess && hipEventRecord(e.ev_start, e.stream) == hipSuccess &&
         launch_step_ops(e.env(), epoch_step_ptrs(e), e.stream, op, op + 1) == hipSuccess &&
         hipEventRecord(e.ev_stop, e.stream) == hipSuccess && hipGraphLaunch(post, e.stream) == hipSuccess;
}

// After the epoch has completed: keep the timed launch's duration when every
// step of the epoch ran (an early-finished epoch skips its kernels).
void collect_timing(Engine& e, int K) {
  if (!e.timing) return;
  const int32_t* control = reinterpret_cast<const int32_t*>(e.h_fetch + 8 * kMaxEpochSteps * e.dims.batch);
  float ms = 0.f;
  if (control[3] == 0 && control[4] == K && hipEventElapsedTime(&ms, e.ev_start, e.ev_stop) == hipSuccess)
    e.timing_ms.push_back(ms);
}

}  // namespace
}  // namespace re

using re::Engine;

extern "C" void* resident_epoch_create(const char* air_path, const char* graph_config, const char* func_config,
                                       const char* external_weight_dir, const char* tiling_path, int32_t* status) {
  using namespace re;
  if (status == nullptr) return nullptr;
  *status = kCreateArgs;
  std::lock_guard<std::mutex> lifecycle(g_lifecycle_mutex);
  if (g_engine_active || air_path == nullptr || graph_config == nullptr || func_config == nullptr ||
      external_weight_dir == nullptr)
    return nullptr;
  // Check order of resident_epoch_bridge.cpp:364-375: arguments and the
  // /dev/shm weight directory (1), then the tiling file (2), then the graph
  // configuration (3).  The configuration may lift the /dev/shm rule
  // ("engine": {"require_dev_shm": false}); an unreadable one keeps it.
  std::string cfg_text;
  Json cfg;
  const bool cfg_ok =
      read_file(graph_config, cfg_text) && JsonParser(cfg_text).parse(cfg) && cfg.kind == Json::kObject;
  const Json* eng = cfg_ok ? cfg.get("engine") : nullptr;
  const bool require_shm = eng ? eng->bool_or("require_dev_shm", true) : true;
  if (require_shm && std::strncmp(external_weight_dir, "/dev/shm/", 9) != 0) return nullptr;  // bridge.cpp:369
  std::unique_ptr<Engine, void (*)(Engine*)> e(new Engine(), free_engine);
  {
    std::ifstream t(tiling_path ? tiling_path : "", std::ios::binary | std::ios::ate);
    if (!t || static_cast<size_t>(t.tellg()) != e->tiling.size()) {
      *status = kCreateTiling;
      return nullptr;
    }
    t.seekg(0);
    t.read(reinterpret_cast<char*>(e->tiling.data()), e->tiling.size());
  }
  if (!cfg_ok) {
    *status = kCreateConfig;
    return nullptr;
  }
  if (!parse_dims(cfg, e->dims)) {
    *status = kCreateConfig;
    return nullptr;
  }
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess) {
    *status = kCreateRuntime;
    return nullptr;
  }
  if (count < 1 || hipSetDevice(0) != hipSuccess) {
    *status = kCreateDevice;
    return nullptr;
  }
  e->device = 0;
  hipDeviceProp_t prop{};
  if (hipGetDeviceProperties(&prop, 0) == hipSuccess && prop.multiProcessorCount > 0)
    e->cus = prop.multiProcessorCount;
  if (hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking) != hipSuccess) {
    *status = kCreateRuntime;
    return nullptr;
  }
  if (!make_plan(*e, cfg)) {
    *status = kCreateGraph;
    return nullptr;
  }
  layout_weights(*e);
  if (hipMalloc(&e->weights, e->weight_bytes) != hipSuccess || !alloc_state(*e)) {
    *status = kCreateDevice;
    return nullptr;
  }
  if (hipMemset(e->weights, 0, e->weight_bytes) != hipSuccess) {
    *status = kCreateDevice;
    return nullptr;
  }
  if (e->plan.mfma) {
    e->packed_off.resize(e->dims.layers);
    const size_t packed_bytes = mfma_packed_layout(e->dims, e->packed_off.data(), &e->packed_lm_off);
    if (hipMalloc(&e->packed, packed_bytes) != hipSuccess) {
      *status = kCreateDevice;
      return nullptr;
    }
  }
  const Json* w = cfg.get("weights");
  const std::string source = w ? w->string_or("source", "bundle") : "bundle";
  bool loaded = false;
  if (source == "bundle") {
    loaded = load_bundle(*e, external_weight_dir);
  } else if (source == "synthetic") {
    loaded = load_synthetic(*e, static_cast<unsigned long long>(w->number_or("seed", 0)),
                            static_cast<float>(w->number_or("std", 0.02)));
  } else if (source == "upload") {
    loaded = true;
  }
  if (!loaded || !repack_all(*e)) {
    *status = kCreateWeights;
    return nullptr;
  }
  e->timing_layer = e->dims.layers / 2;
  if (hipEventCreate(&e->ev_start) != hipSuccess || hipEventCreate(&e->ev_stop) != hipSuccess) {
    *status = kCreateRuntime;
    return nullptr;
  }
  if (re::epoch_graph(*e, 1, re::kFeedPlain, 0) == nullptr) {
    *status = kCreateGraph;
    return nullptr;
  }
  g_engine_active = true;
  *status = kCreateOk;
  return e.release();
}

extern "C" int32_t resident_epoch_execute(
    void* opaque, int32_t request_count, int32_t max_steps, const int64_t* input_token_ids,
    const int64_t* input_positions, const int32_t* input_sequence_lengths, const int32_t* input_eos_token_ids,
    const int32_t* input_row_generations, int64_t* output_token_ids, int32_t* output_executed,
    int32_t* output_row_generations, int32_t* output_model_calls, int32_t* output_device_status,
    int32_t* output_feed_calls, int32_t* output_fetch_calls, int32_t* output_commit_state,
    int32_t* output_kv_import_checksum, int64_t* output_wall_us, int64_t* output_native_cpu_us,
    int64_t* output_declared_input_bytes, int64_t* output_declared_output_bytes, const char* transfer_path,
    uint64_t transfer_id, const ResidentEpochIpcMetadata* ipc_metadata) {
  using namespace re;
  if (output_commit_state == nullptr) return 10;
  *output_commit_state = CRUISE_EPOCH_PREPARED;
  const bool direct_device_import = ipc_metadata != nullptr;
  const bool importing = transfer_path != nullptr || direct_device_import;
  Engine* e = static_cast<Engine*>(opaque);
  // The bridge's row arrays are four rows wide (resident_epoch_bridge.h:29-43):
  // an engine of another batch is served through resident_epoch_proc only.
  const int B = e ? e->dims.batch : 0;
  if (e == nullptr || B != kBridgeRows || request_count < 1 || request_count > B || max_steps < 1 ||
      max_steps > kMaxEpochSteps ||
      input_token_ids == nullptr || input_positions == nullptr || input_sequence_lengths == nullptr ||
      input_eos_token_ids == nullptr || input_row_generations == nullptr || output_token_ids == nullptr ||
      output_executed == nullptr || output_row_generations == nullptr || output_model_calls == nullptr ||
      output_device_status == nullptr || output_feed_calls == nullptr || output_fetch_calls == nullptr ||
      output_kv_import_checksum == nullptr || output_wall_us == nullptr || output_native_cpu_us == nullptr ||
      output_declared_input_bytes == nullptr || output_declared_output_bytes == nullptr ||
      (importing && transfer_id == 0) || (!importing && transfer_id != 0) ||
      (transfer_path != nullptr && direct_device_import)) {
    return 10;
  }
  std::lock_guard<std::mutex> lock(e->execute_mutex);
  const Dims& d = e->dims;
  int32_t import_mask = 0;
  uint32_t expected_checksum = 0;
  if (importing && !direct_device_import &&
      !read_transfer(*e, transfer_path, transfer_id, input_row_generations, import_mask, expected_checksum)) {
    return 13;
  }
  if (direct_device_import && !prepare_device_import(*e, ipc_metadata, input_row_generations, import_mask)) return 35;
  *output_model_calls = 0;
  *output_device_status = -1;
  *output_feed_calls = 0;
  *output_fetch_calls = 0;
  *output_kv_import_checksum = 0;
  *output_wall_us = 0;
  *output_native_cpu_us = 0;
  // a device-IPC epoch declares what crossed the host boundary: the request
  // and the metadata record (resident_epoch_bridge.cpp:42-43)
  *output_declared_input_bytes =
      direct_device_import ? static_cast<int64_t>(CRUISE_SIDECAR_REQUEST_BYTES + CRUISE_RESIDENT_IPC_METADATA_BYTES)
      : importing          ? static_cast<int64_t>(e->import_feed_bytes)
                           : static_cast<int64_t>(e->feed_bytes);
  *output_declared_output_bytes = static_cast<int64_t>(e->fetch_bytes);
  const int64_t cpu_start = process_cpu_us();
  std::fill(output_token_ids, output_token_ids + B * kMaxEpochSteps, -1);
  std::fill(output_executed, output_executed + B, 0);
  std::fill(output_row_generations, output_row_generations + B, 0);

  std::vector<int64_t> tok(B, 0), pos(B, 0);
  std::vector<int32_t> len(B, 0), slot(B, 0), active(B, 0), table((size_t)B * d.blocks_per_row);
  for (int r = 0; r < B; ++r) {
    for (int j = 0; j < d.blocks_per_row; ++j) table[r * d.blocks_per_row + j] = r * d.blocks_per_row + j;
    slot[r] = bridge_slot(d, r, 0);
  }
  int active_count = 0;
  for (int r = 0; r < B; ++r) {  // bridge.cpp:533-552
    if (input_row_generations[r] == 0) continue;
    ++active_count;
    if (input_row_generations[r] < 0 || input_token_ids[r] < 0 || input_token_ids[r] >= d.vocab ||
        input_positions[r] < 0 || input_positions[r] + max_steps > d.capacity ||
        input_sequence_lengths[r] != input_positions[r] + 1 || input_eos_token_ids[r] < 0 ||
        input_eos_token_ids[r] >= d.vocab) {
      return 11;
    }
    tok[r] = input_token_ids[r];
    pos[r] = input_positions[r];
    len[r] = input_sequence_lengths[r];
    slot[r] = bridge_slot(d, r, input_positions[r]);
    active[r] = 1;
  }
  if (active_count != request_count) return 12;
  std::vector<int32_t> control(3 + 2 * B, 0);  // bridge.cpp:555-567
  control[0] = max_steps;
  for (int r = 0; r < B; ++r) {
    control[1 + r] = input_row_generations[r] != 0 ? input_eos_token_ids[r] : d.configured_eos;
    control[3 + B + r] = input_row_generations[r];
  }
  control[2 + B] = importing ? (kImportGraphFlag | import_mask) : 0;
  uint8_t* p = e->h_feed + (importing ? e->payload_bytes : 0);
  p = put(p, tok.data(), 8 * B);
  p = put(p, pos.data(), 8 * B);
  p = put(p, len.data(), 4 * B);
  if (!importing) p = put(p, slot.data(), 4 * B);
  p = put(p, active.data(), 4 * B);
  p = put(p, table.data(), 4 * table.size());
  p = put(p, e->tiling.data(), e->tiling.size());
  p = put(p, control.data(), 4 * control.size());

  const auto wall_start = std::chrono::steady_clock::now();
  *output_commit_state = CRUISE_EPOCH_EXECUTING;
  const bool launched =
      run_graph(*e, max_steps, direct_device_import ? kFeedDeviceImport : importing ? kFeedHostImport : kFeedPlain);
  *output_feed_calls = 1;
  if (!launched) return 30;
  const hipError_t synced = hipStreamSynchronize(e->stream);
  *output_fetch_calls = 1;
  const auto wall_end = std::chrono::steady_clock::now();
  *output_wall_us = std::chrono::duration_cast<std::chrono::microseconds>(wall_end - wall_start).count();
  if (synced != hipSuccess) return 31;
  collect_timing(*e, max_steps);
  const int64_t* history = reinterpret_cast<const int64_t*>(e->h_fetch);
  int32_t* result_control = reinterpret_cast<int32_t*>(e->h_fetch + 8 * kMaxEpochSteps * B);
  *output_device_status = result_control[3];
  *output_model_calls = result_control[4];
  *output_kv_import_checksum = result_control[5];
  if (*output_device_status == 0) {
    // a device-IPC import must prove itself with a checksum; a file import
    // with the one its header carries
    if (direct_device_import && *output_kv_import_checksum == 0) return 34;
    if (importing && !direct_device_import && static_cast<uint32_t>(*output_kv_import_checksum) != expected_checksum)
      return 34;
  }
  for (int r = 0; r < B; ++r) {  // bridge.cpp:632-642
    const int32_t executed = result_control[6 + 2 * B + r];
    if (executed < 0 || executed > max_steps) return 33;
    output_executed[r] = executed;
    output_row_generations[r] = result_control[6 + 4 * B + 2 + r];
    for (int s = 0; s < executed; ++s) output_token_ids[r * kMaxEpochSteps + s] = history[s * B + r];
  }
  const int64_t cpu_end = process_cpu_us();
  if (cpu_start >= 0 && cpu_end >= cpu_start) *output_native_cpu_us = cpu_end - cpu_start;
  *output_commit_state = CRUISE_EPOCH_COMMITTED;
  return 0;
}

extern "C" void resident_epoch_destroy(void* opaque) {
  using namespace re;
  if (opaque == nullptr) return;
  std::lock_guard<std::mutex> lifecycle(g_lifecycle_mutex);
  Engine* e = static_cast<Engine*>(opaque);
  {
    std::lock_guard<std::mutex> lock(e->execute_mutex);
    (void)hipStreamSynchronize(e->stream);  // teardown proceeds whatever a failed launch left
  }
  free_engine(e);
  g_engine_active = false;
}

extern "C" int32_t resident_epoch_proc(void* engine, const void* feed, int64_t feed_bytes, void* fetch,
                                       int64_t fetch_bytes) {
  using namespace re;
  Engine* e = static_cast<Engine*>(engine);
  if (e == nullptr || feed == nullptr || fetch == nullptr || fetch_bytes != static_cast<int64_t>(e->fetch_bytes))
    return -1;
  const bool importing = feed_bytes == static_cast<int64_t>(e->import_feed_bytes);
  if (!importing && feed_bytes != static_cast<int64_t>(e->feed_bytes)) return -1;
  std::lock_guard<std::mutex> lock(e->execute_mutex);
  std::memcpy(e->h_feed, feed, feed_bytes);
  const int B = e->dims.batch;
  const size_t ctl_off = (importing ? e->payload_bytes : 0) + 8 * B + 8 * B + 4 * B + (importing ? 0 : 4 * B) +
                         4 * B + 4 * (size_t)B * e->dims.blocks_per_row + kTilingBytes;
  int32_t K = 0;
  std::memcpy(&K, e->h_feed + ctl_off, 4);
  // An out-of-range K still runs a one-step graph: the device rejects it (201).
  const int graph_k = (K >= 1 && K <= kMaxEpochSteps) ? K : 1;
  if (!run_graph(*e, graph_k, importing ? kFeedHostImport : kFeedPlain)) return -2;
  if (hipStreamSynchronize(e->stream) != hipSuccess) return -2;
  collect_timing(*e, graph_k);
  std::memcpy(fetch, e->h_fetch, e->fetch_bytes);
  return 0;
}

namespace {
bool copy_in(void* dst, const void* src, size_t bytes, hipStream_t s) {
  return hipMemcpyAsync(dst, src, bytes, hipMemcpyDefault, s) == hipSuccess;
}
}  // namespace

extern "C" int32_t resident_decoder_step(void* engine, const int64_t* token_id, const int64_t* position,
                                         const int32_t* sequence_length, void* key_cache,
                                         const int32_t* slot_mapping, const int32_t* active_mask,
                                         const int32_t* block_table, void* value_cache,
                                         const uint8_t* explicit_tiling, float* logits, int64_t* next_position) {
  using namespace re;
  Engine* e = static_cast<Engine*>(engine);
  if (e == nullptr || token_id == nullptr || position == nullptr || sequence_length == nullptr ||
      key_cache == nullptr || slot_mapping == nullptr || active_mask == nullptr || block_table == nullptr ||
      value_cache == nullptr || explicit_tiling == nullptr || logits == nullptr || next_position == nullptr)
    return -1;
  std::lock_guard<std::mutex> lock(e->execute_mutex);
  const Dims& d = e->dims;
  const int B = d.batch;
  hipStream_t s = e->stream;
  if (e->dec_key == nullptr) {
    if (hipMalloc(&e->dec_key, e->cache_bytes) != hipSuccess) return -2;
    if (hipMalloc(&e->dec_value, e->cache_bytes) != hipSuccess) return -2;
  }
  StepPtrs sp = e->step_io;
  bool ok = copy_in(const_cast<int64_t*>(sp.token), token_id, 8 * B, s) &&
            copy_in(const_cast<int64_t*>(sp.pos), position, 8 * B, s) &&
            copy_in(const_cast<int32_t*>(sp.len), sequence_length, 4 * B, s) &&
            copy_in(const_cast<int32_t*>(sp.slot), slot_mapping, 4 * B, s) &&
            copy_in(const_cast<int32_t*>(sp.active), active_mask, 4 * B, s) &&
            copy_in(const_cast<int32_t*>(sp.table), block_table, 4 * (size_t)B * d.blocks_per_row, s) &&
            copy_in(e->dec_key, key_cache, e->cache_bytes, s) && copy_in(e->dec_value, value_cache, e->cache_bytes, s);
  if (!ok) return -2;
  sp.key_cache = e->dec_key;
  sp.value_cache = e->dec_value;
  sp.logits = e->logits;
  sp.done = nullptr;
  if (launch_decoder_step(e->env(), sp, s) != hipSuccess) return -2;
  std::vector<int64_t> pos(B), npos(B);
  std::vector<int32_t> act(B);
  ok = hipMemcpyAsync(pos.data(), sp.pos, 8 * B, hipMemcpyDeviceToHost, s) == hipSuccess &&
       hipMemcpyAsync(act.data(), sp.active, 4 * B, hipMemcpyDeviceToHost, s) == hipSuccess &&
       hipMemcpyAsync(logits, e->logits, (size_t)B * d.vocab * sizeof(float), hipMemcpyDefault, s) == hipSuccess &&
       hipMemcpyAsync(key_cache, e->dec_key, e->cache_bytes, hipMemcpyDefault, s) == hipSuccess &&
       hipMemcpyAsync(value_cache, e->dec_value, e->cache_bytes, hipMemcpyDefault, s) == hipSuccess &&
       hipStreamSynchronize(s) == hipSuccess;
  if (!ok) return -2;
  // next_position = where(active, pos + 1, pos) (batched_decoder_step.py:409-411)
  for (int b = 0; b < B; ++b) npos[b] = act[b] != 0 ? pos[b] + 1 : pos[b];
  if (hipMemcpy(next_position, npos.data(), 8 * B, hipMemcpyDefault) != hipSuccess) return -2;
  return 0;
}

extern "C" int32_t resident_epoch_prefill(void* engine, int32_t row, int32_t generation, const int64_t* prompt,
                                          int32_t prompt_len, const int32_t* block_table_row) {
  using namespace re;
  Engine* e = static_cast<Engine*>(engine);
  if (e == nullptr || prompt == nullptr || block_table_row == nullptr) return -1;
  const Dims& d = e->dims;
  const int B = d.batch;
  if (row < 0 || row >= B || generation <= 0 || prompt_len < 1 || prompt_len > d.capacity) return -1;
  std::vector<int64_t> toks(prompt, prompt + prompt_len);
  for (int64_t t : toks)
    if (t < 0 || t >= d.vocab) return -1;
  std::vector<int32_t> trow(block_table_row, block_table_row + d.blocks_per_row);
  for (int32_t blk : trow)
    if (blk < 0 || blk >= d.physical_blocks) return -1;
  std::lock_guard<std::mutex> lock(e->execute_mutex);
  hipStream_t s = e->stream;
  StepPtrs sp = e->step_io;
  if (!copy_in(const_cast<int32_t*>(sp.table) + row * d.blocks_per_row, trow.data(), 4 * trow.size(), s)) return -2;
  if (launch_clear_blocks(e->env(), e->key_cache, e->value_cache, sp.table + row * d.blocks_per_row,
                          d.blocks_per_row, s) != hipSuccess)
    return -2;
  std::vector<int32_t> table((size_t)B * d.blocks_per_row, 0);
  for (int j = 0; j < d.blocks_per_row; ++j) table[row * d.blocks_per_row + j] = trow[j];
  std::vector<int64_t> tok(B, 0), pos(B, 0);
  std::vector<int32_t> len(B, 0), slot(B, -1), act(B, 0);
  sp.key_cache = e->key_cache;
  sp.value_cache = e->value_cache;
  sp.logits = e->logits;
  sp.done = nullptr;
  for (int p = 0; p + 1 < prompt_len; ++p) {
    tok[row] = toks[p];
    pos[row] = p;
    len[row] = p + 1;
    act[row] = 1;
    const int lb = p / d.block_size;
    slot[row] = trow[lb] * d.block_size + p % d.block_size;
    // each step's inputs are staged synchronously: the host vectors change next iteration
    bool ok = hipMemcpy(const_cast<int64_t*>(sp.token), tok.data(), 8 * B, hipMemcpyHostToDevice) == hipSuccess &&
              hipMemcpy(const_cast<int64_t*>(sp.pos), pos.data(), 8 * B, hipMemcpyHostToDevice) == hipSuccess &&
              hipMemcpy(const_cast<int32_t*>(sp.len), len.data(), 4 * B, hipMemcpyHostToDevice) == hipSuccess &&
              hipMemcpy(const_cast<int32_t*>(sp.slot), slot.data(), 4 * B, hipMemcpyHostToDevice) == hipSuccess &&
              hipMemcpy(const_cast<int32_t*>(sp.active), act.data(), 4 * B, hipMemcpyHostToDevice) == hipSuccess &&
              hipMemcpy(const_cast<int32_t*>(sp.table), table.data(), 4 * table.size(), hipMemcpyHostToDevice) ==
                  hipSuccess;
    if (!ok) return -2;
    if (launch_decoder_step(e->env(), sp, s) != hipSuccess) return -2;
    if (hipStreamSynchronize(s) != hipSuccess) return -2;
  }
  const int32_t gen = generation, len_v = prompt_len, valid = 1;
  const int64_t last_tok = toks[prompt_len - 1], last_pos = prompt_len - 1;
  bool ok = hipMemcpy(e->st.res_gen + row, &gen, 4, hipMemcpyHostToDevice) == hipSuccess &&
            hipMemcpy(e->st.res_token + row, &last_tok, 8, hipMemcpyHostToDevice) == hipSuccess &&
            hipMemcpy(e->st.res_pos + row, &last_pos, 8, hipMemcpyHostToDevice) == hipSuccess &&
            hipMemcpy(e->st.res_len + row, &len_v, 4, hipMemcpyHostToDevice) == hipSuccess &&
            hipMemcpy(e->st.res_valid + row, &valid, 4, hipMemcpyHostToDevice) == hipSuccess &&
            hipStreamSynchronize(s) == hipSuccess;
  return ok ? 0 : -2;
}

namespace {

// One pass of the decoder over the prompt tokens of several rows (see
// resident_epoch_prefill_batch).  Token i of the pass is (row, position);
// a row's tokens are consecutive and start at position 0.
// Scratch: the engine's own buffer, grown on demand, or (fixed != nullptr)
// the caller's fixed buffer of fixed_bytes, in which case nothing is
// allocated and a pass that does not fit returns -3.
int32_t prefill_batch(Engine& e, const std::vector<int>& rows, const std::vector<int32_t>& gens,
                      const std::vector<std::vector<int64_t>>& prompts, const std::vector<int32_t>& tables,
                      uint8_t* fixed = nullptr, size_t fixed_bytes = 0) {
  using namespace re;
  const Dims& d = e.dims;
  const int nr = static_cast<int>(rows.size());
  const int bpr = d.blocks_per_row;
  hipStream_t s = e.stream;
  if (!e.pf_ready) {
    if (prepare_prefill(d) != hipSuccess) return -2;
    e.pf_ready = true;
  }
  // token table and attention tiles
  std::vector<int64_t> tok;
  std::vector<int32_t> pos, slot;
  std::vector<int4> tiles;
  for (int i = 0; i < nr; ++i) {
    const int base = static_cast<int>(tok.size());
    const int n = static_cast<int>(prompts[i].size()) - 1;  // positions 0 .. len-2 are prefilled
    for (int p = 0; p < n; ++p) {
      tok.push_back(prompts[i][p]);
      pos.push_back(p);
      slot.push_back(tables[i * bpr + p / d.block_size] * d.block_size + p % d.block_size);
    }
    for (int q = 0; q < n; q += 64) tiles.push_back(make_int4(base + q, base, std::min(64, n - q), q));
  }
  const int M = static_cast<int>(tok.size());
  const size_t T = d.dtype_bytes;
  const size_t I = d.intermediate, H = d.hidden;
  // scratch layout
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off = align_up(off + bytes, 256);
    return at;
  };
  const size_t o_hidden = take(M * H * T), o_xn = take(M * H * T), o_qkv = take((size_t)M * d.qkv_rows() * T);
  // bf16: gate, up and SwiGLU in one GEMM (no gate/up buffers); fp32: two
  // GEMMs and the elementwise SwiGLU
  const bool fused_mlp = d.dtype_bytes == 2;
  const size_t o_attn = take((size_t)M * d.q_dim() * T), o_gate = fused_mlp ? 0 : take(M * I * T);
  const size_t o_up = fused_mlp ? 0 : take(M * I * T);
  const size_t o_mlp = take(M * I * T), o_rope = take((size_t)M * d.head_dim * sizeof(float));
  const size_t o_tok = take(8 * (size_t)M), o_pos = take(4 * (size_t)M), o_slot = take(4 * (size_t)M);
  const size_t o_tiles = take(sizeof(int4) * tiles.size()), o_blocks = take(4 * tables.size());
  if (fixed != nullptr) {
    if (off > fixed_bytes) return -3;
  } else if (off > e.pf_bytes) {
    if (e.pf_mem) (void)hipFree(e.pf_mem);
    e.pf_mem = nullptr;
    e.pf_bytes = 0;
    if (hipMalloc(&e.pf_mem, off) != hipSuccess) return -2;
    e.pf_bytes = off;
  }
  uint8_t* b = fixed != nullptr ? fixed : e.pf_mem;
  const bool ok = (M == 0 || (hipMemcpy(b + o_tok, tok.data(), 8 * M, hipMemcpyHostToDevice) == hipSuccess &&
                              hipMemcpy(b + o_pos, pos.data(), 4 * M, hipMemcpyHostToDevice) == hipSuccess &&
                              hipMemcpy(b + o_slot, slot.data(), 4 * M, hipMemcpyHostToDevice) == hipSuccess &&
                              hipMemcpy(b + o_tiles, tiles.data(), sizeof(int4) * tiles.size(),
                                        hipMemcpyHostToDevice) == hipSuccess)) &&
                  hipMemcpy(b + o_blocks, tables.data(), 4 * tables.size(), hipMemcpyHostToDevice) == hipSuccess;
  if (!ok) return -2;
  const KernelEnv env = e.env();
  if (launch_clear_blocks(env, e.key_cache, e.value_cache, reinterpret_cast<const int32_t*>(b + o_blocks),
                          static_cast<int>(tables.size()), s) != hipSuccess)
    return -2;
  if (M > 0) {
    hipError_t err = hipSuccess;
    auto run = [&](hipError_t r) {
      if (err == hipSuccess) err = r;
    };
    PrefillRows er{};
    er.token = reinterpret_cast<const int64_t*>(b + o_tok);
    er.pos = reinterpret_cast<const int32_t*>(b + o_pos);
    er.embedding = e.weights + e.embedding_off;
    er.inv_freq = e.scratch.inv_freq;
    er.hidden = b + o_hidden;
    er.rope = reinterpret_cast<float*>(b + o_rope);
    er.M = M;
    er.H = d.hidden;
    er.V = d.vocab;
    er.head_dim = d.head_dim;
    run(launch_prefill_embed(er, d.dtype_bytes, s));
    const long long cache_layer_elems = d.slots() * d.kv_dim();
    for (int l = 0; l < d.layers && err == hipSuccess; ++l) {
      const LayerOffsets& lo = e.layer_off[l];
      auto gemm = [&](size_t a_off, long long lda, size_t w_off, size_t bias_off, size_t out_off, long long ldo, int N,
                      int K, int epi) {
        GemmArgs g{};
        g.A = b + a_off;
        g.W = e.weights + w_off;
        g.bias = bias_off == SIZE_MAX ? nullptr : e.weights + bias_off;
        g.out = b + out_off;
        g.M = M;
        g.N = N;
        g.K = K;
        g.lda = lda;
        g.ldw = K;
        g.ldo = ldo;
        run(launch_gemm(g, epi, d.dtype_bytes, s));
      };
      run(launch_prefill_rmsnorm(b + o_hidden, e.weights + lo.input_norm, b + o_xn, M, d.hidden, d.rms_eps,
                                 d.dtype_bytes, s));
      gemm(o_xn, d.hidden, lo.qkv_w, lo.qkv_b, o_qkv, d.qkv_rows(), d.qkv_rows(), d.hidden, kGemmStore);
      PrefillQkv qp{};
      qp.qkv = b + o_qkv;
      qp.rope = er.rope;
      qp.slot = reinterpret_cast<const int32_t*>(b + o_slot);
      qp.key_cache = static_cast<uint8_t*>(e.key_cache) + l * cache_layer_elems * T;
      qp.value_cache = static_cast<uint8_t*>(e.value_cache) + l * cache_layer_elems * T;
      qp.slots = d.slots();
      qp.M = M;
      qp.ld = d.qkv_rows();
      qp.heads = d.heads;
      qp.kv_heads = d.kv_heads;
      qp.head_dim = d.head_dim;
      run(launch_prefill_qkv_post(qp, d.dtype_bytes, s));
      PrefillAttn at{};
      at.qkv = b + o_qkv;
      at.out = b + o_attn;
      at.pos = er.pos;
      at.tiles = reinterpret_cast<const int4*>(b + o_tiles);
      at.M = M;
      at.ld = d.qkv_rows();
      at.heads = d.heads;
      at.kv_heads = d.kv_heads;
      at.head_dim = d.head_dim;
      run(launch_prefill_attention(at, d, static_cast<int>(tiles.size()), s));
      gemm(o_attn, d.q_dim(), lo.o_w, SIZE_MAX, o_hidden, d.hidden, d.hidden, d.q_dim(), kGemmResidual);
      run(launch_prefill_rmsnorm(b + o_hidden, e.weights + lo.post_norm, b + o_xn, M, d.hidden, d.rms_eps,
                                 d.dtype_bytes, s));
      if (fused_mlp) {
        GemmArgs g{};
        g.A = b + o_xn;
        g.W = e.weights + lo.gate_w;
        g.W2 = e.weights + lo.up_w;
        g.out = b + o_mlp;
        g.M = M;
        g.N = d.intermediate;
        g.K = d.hidden;
        g.lda = d.hidden;
        g.ldw = d.hidden;
        g.ldo = d.intermediate;
        run(launch_gemm(g, kGemmSwiGlu, d.dtype_bytes, s));
      } else {
        gemm(o_xn, d.hidden, lo.gate_w, SIZE_MAX, o_gate, d.intermediate, d.intermediate, d.hidden, kGemmStore);
        gemm(o_xn, d.hidden, lo.up_w, SIZE_MAX, o_up, d.intermediate, d.intermediate, d.hidden, kGemmStore);
        run(launch_prefill_swiglu(b + o_gate, b + o_up, b + o_mlp, (long long)M * d.intermediate, d.dtype_bytes, s));
      }
      gemm(o_mlp, d.intermediate, lo.down_w, SIZE_MAX, o_hidden, d.hidden, d.hidden, d.intermediate, kGemmResidual);
    }
    if (err != hipSuccess) return -2;
  }
  if (hipStreamSynchronize(s) != hipSuccess) return -2;
  for (int i = 0; i < nr; ++i) {
    const int r = rows[i];
    const int32_t len = static_cast<int32_t>(prompts[i].size()), valid = 1;
    const int64_t last_tok = prompts[i].back(), last_pos = len - 1;
    const bool stored = hipMemcpy(e.st.res_gen + r, &gens[i], 4, hipMemcpyHostToDevice) == hipSuccess &&
                        hipMemcpy(e.st.res_token + r, &last_tok, 8, hipMemcpyHostToDevice) == hipSuccess &&
                        hipMemcpy(e.st.res_pos + r, &last_pos, 8, hipMemcpyHostToDevice) == hipSuccess &&
                        hipMemcpy(e.st.res_len + r, &len, 4, hipMemcpyHostToDevice) == hipSuccess &&
                        hipMemcpy(e.st.res_valid + r, &valid, 4, hipMemcpyHostToDevice) == hipSuccess;
    if (!stored) return -2;
  }
  return 0;
}

}  // namespace

namespace {

// The arguments of a batched prefill, checked and copied (false: -1).
struct PrefillRequest {
  std::vector<int> rows;
  std::vector<int32_t> gens;
  std::vector<std::vector<int64_t>> prompts;
  std::vector<int32_t> tables;
};

bool parse_prefill(const re::Dims& d, int32_t n_rows, const int32_t* rows, const int32_t* generations,
                   const int64_t* prompts, const int32_t* prompt_lens, const int32_t* block_tables,
                   PrefillRequest& req) {
  if (rows == nullptr || generations == nullptr || prompts == nullptr || prompt_lens == nullptr ||
      block_tables == nullptr || n_rows < 1 || n_rows > d.batch)
    return false;
  req.rows.assign(n_rows, 0);
  req.gens.assign(generations, generations + n_rows);
  req.prompts.assign(n_rows, {});
  req.tables.assign(block_tables, block_tables + (size_t)n_rows * d.blocks_per_row);
  std::vector<bool> seen(d.batch, false);
  size_t at = 0;
  for (int i = 0; i < n_rows; ++i) {
    const int r = rows[i];
    if (r < 0 || r >= d.batch || seen[r] || req.gens[i] <= 0) return false;
    seen[r] = true;
    req.rows[i] = r;
    const int len = prompt_lens[i];
    if (len < 1 || len > d.capacity || (len > 1 && (len - 2) / d.block_size >= d.blocks_per_row)) return false;
    req.prompts[i].assign(prompts + at, prompts + at + len);
    at += len;
    for (int64_t t : req.prompts[i])
      if (t < 0 || t >= d.vocab) return false;
  }
  for (int32_t blk : req.tables)
    if (blk < 0 || blk >= d.physical_blocks) return false;
  return true;
}

}  // namespace

extern "C" int32_t resident_epoch_prefill_batch(void* engine, int32_t n_rows, const int32_t* rows,
                                                const int32_t* generations, const int64_t* prompts,
                                                const int32_t* prompt_lens, const int32_t* block_tables) {
  using namespace re;
  Engine* e = static_cast<Engine*>(engine);
  PrefillRequest req;
  if (e == nullptr || !parse_prefill(e->dims, n_rows, rows, generations, prompts, prompt_lens, block_tables, req))
    return -1;
  std::lock_guard<std::mutex> lock(e->execute_mutex);
  return prefill_batch(*e, req.rows, req.gens, req.prompts, req.tables);
}

extern "C" int32_t resident_epoch_prefill_batch_noalloc(void* engine, int32_t n_rows, const int32_t* rows,
                                                        const int32_t* generations, const int64_t* prompts,
                                                        const int32_t* prompt_lens, const int32_t* block_tables) {
  using namespace re;
  Engine* e = static_cast<Engine*>(engine);
  PrefillRequest req;
  if (e == nullptr || !parse_prefill(e->dims, n_rows, rows, generations, prompts, prompt_lens, block_tables, req))
    return -1;
  // The array's address on the engine's device, resolved on this entry
  // point's first call there (resolving allocates nothing).
  if (hipSetDevice(e->device) != hipSuccess || !noalloc_setup(e->device)) return -2;
  uint8_t* scratch_ptr = noalloc_scratch(e->device);
  if (scratch_ptr == nullptr) return -2;
  std::lock_guard<std::mutex> lock(e->execute_mutex);
  std::lock_guard<std::mutex> shared(g_noalloc_mutex);
  return prefill_batch(*e, req.rows, req.gens, req.prompts, req.tables, scratch_ptr, kNoAllocScratchBytes);
}

namespace {
enum class Access { kRead, kWrite };

int32_t state_access(Engine* e, const char* name, void* buf, int64_t bytes, Access mode) {
  using namespace re;
  if (e == nullptr || name == nullptr || buf == nullptr || bytes < 0) return -1;
  std::lock_guard<std::mutex> lock(e->execute_mutex);
  const Dims& d = e->dims;
  const std::string n(name);
  void* dev = nullptr;
  size_t size = 0;
  if (n == "key_cache") {
    dev = e->key_cache;
    size = e->cache_bytes;
  } else if (n == "value_cache") {
    dev = e->value_cache;
    size = e->cache_bytes;
  } else if (n == "logits") {
    dev = e->logits;
    size = (size_t)d.batch * d.vocab * sizeof(float);
  } else if (n == "inv_freq") {
    dev = e->scratch.inv_freq;
    size = (size_t)d.head_dim / 2 * sizeof(float);
  } else if (n == "resident_rows") {
    const int B = d.batch;
    if (static_cast<size_t>(bytes) != 5 * 8 * (size_t)B) return -1;
    std::vector<int32_t> gen(B), len(B), valid(B);
    std::vector<int64_t> tok(B), pos(B), rows(5 * B);
    if (hipStreamSynchronize(e->stream) != hipSuccess) return -2;
    if (mode == Access::kRead) {
      bool ok = hipMemcpy(gen.data(), e->st.res_gen, 4 * B, hipMemcpyDeviceToHost) == hipSuccess &&
                hipMemcpy(tok.data(), e->st.res_token, 8 * B, hipMemcpyDeviceToHost) == hipSuccess &&
                hipMemcpy(pos.data(), e->st.res_pos, 8 * B, hipMemcpyDeviceToHost) == hipSuccess &&
                hipMemcpy(len.data(), e->st.res_len, 4 * B, hipMemcpyDeviceToHost) == hipSuccess &&
                hipMemcpy(valid.data(), e->st.res_valid, 4 * B, hipMemcpyDeviceToHost) == hipSuccess;
      if (!ok) return -2;
      for (int r = 0; r < B; ++r) {
        rows[r] = gen[r];
        rows[B + r] = tok[r];
        rows[2 * B + r] = pos[r];
        rows[3 * B + r] = len[r];
        rows[4 * B + r] = valid[r];
      }
      return hipMemcpy(buf, rows.data(), bytes, hipMemcpyDefault) == hipSuccess ? 0 : -2;
    }
    if (hipMemcpy(rows.data(), buf, bytes, hipMemcpyDefault) != hipSuccess) return -2;
    for (int r = 0; r < B; ++r) {
      gen[r] = static_cast<int32_t>(rows[r]);
      tok[r] = rows[B + r];
      pos[r] = rows[2 * B + r];
      len[r] = static_cast<int32_t>(rows[3 * B + r]);
      valid[r] = static_cast<int32_t>(rows[4 * B + r]);
    }
    bool ok = hipMemcpy(e->st.res_gen, gen.data(), 4 * B, hipMemcpyHostToDevice) == hipSuccess &&
              hipMemcpy(e->st.res_token, tok.data(), 8 * B, hipMemcpyHostToDevice) == hipSuccess &&
              hipMemcpy(e->st.res_pos, pos.data(), 8 * B, hipMemcpyHostToDevice) == hipSuccess &&
              hipMemcpy(e->st.res_len, len.data(), 4 * B, hipMemcpyHostToDevice) == hipSuccess &&
              hipMemcpy(e->st.res_valid, valid.data(), 4 * B, hipMemcpyHostToDevice) == hipSuccess;
    return ok ? 0 : -2;
  } else {
    auto it = e->weight_slots.find(n);
    if (it == e->weight_slots.end()) return -1;
    dev = e->weights + it->second.offset;
    size = it->second.bytes;
  }
  if (static_cast<size_t>(bytes) != size) return -1;
  if (hipStreamSynchronize(e->stream) != hipSuccess) return -2;
  // On the engine's stream (which does not wait for the null stream), so the
  // repack of a written matrix sees the new values, and complete on return
  // (a device-to-device hipMemcpy may return before the copy has finished).
  const hipError_t err = mode == Access::kRead ? hipMemcpyAsync(buf, dev, size, hipMemcpyDefault, e->stream)
                                               : hipMemcpyAsync(dev, buf, size, hipMemcpyDefault, e->stream);
  if (err != hipSuccess) return -2;
  if (mode == Access::kWrite && repack_slot(*e, n) != hipSuccess) return -2;
  return hipStreamSynchronize(e->stream) == hipSuccess ? 0 : -2;
}
}  // namespace

extern "C" int32_t resident_epoch_read_state(void* engine, const char* name, void* dst, int64_t bytes) {
  return state_access(static_cast<Engine*>(engine), name, dst, bytes, Access::kRead);
}

extern "C" int32_t resident_epoch_write_state(void* engine, const char* name, const void* src, int64_t bytes) {
  return state_access(static_cast<Engine*>(engine), name, const_cast<void*>(src), bytes, Access::kWrite);
}

extern "C" int32_t resident_epoch_info(void* engine, const char* key, int64_t* value) {
  Engine* e = static_cast<Engine*>(engine);
  if (e == nullptr || key == nullptr || value == nullptr) return -1;
  const re::Dims& d = e->dims;
  const std::string k(key);
  const std::map<std::string, int64_t> facts = {
      {"batch", d.batch},
      {"layers", d.layers},
      {"hidden", d.hidden},
      {"heads", d.heads},
      {"kv_heads", d.kv_heads},
      {"head_dim", d.head_dim},
      {"intermediate", d.intermediate},
      {"vocab", d.vocab},
      {"physical_blocks", d.physical_blocks},
      {"block_size", d.block_size},
      {"blocks_per_row", d.blocks_per_row},
      {"capacity", d.capacity},
      {"dtype_bytes", d.dtype_bytes},
      {"feed_bytes", static_cast<int64_t>(e->feed_bytes)},
      {"import_feed_bytes", static_cast<int64_t>(e->import_feed_bytes)},
      {"fetch_bytes", static_cast<int64_t>(e->fetch_bytes)},
      {"cache_bytes", static_cast<int64_t>(e->cache_bytes)},
      {"weight_bytes", static_cast<int64_t>(e->weight_bytes)},
      {"streamed_weight_bytes", static_cast<int64_t>(e->streamed_weight_bytes)},
      {"configured_eos", d.configured_eos},
      {"step_ops", re::step_op_count(e->env())},
      {"ops_per_layer", 7},
      {"timing_layer", e->timing_layer},
      {"qkv_grid", e->plan.qkv_grid},
      {"o_segments", e->plan.o_segments},
      {"gemv_rows_per_pass", e->plan.mb},
      {"gateup_grid", e->plan.gu_grid},
      {"down_segments", e->plan.down_segments},
      {"down_whole_grid", e->plan.down_whole_grid},
      {"qkv_waves", e->plan.qkv_waves},
      {"qkv_ksplit", e->plan.qkv_ksplit},
      {"o_waves", e->plan.o_waves},
      {"mfma", e->plan.mfma},
      {"gu_cu", e->plan.gu_cu},
      {"grouped_attention", e->plan.grouped_attn},
      {"attention_split", e->plan.attn_split},
      {"argmax_parts", e->plan.argmax_parts},
      {"o_grid", e->plan.o_grid},
      {"lm_grid", e->plan.lm_grid},
      {"compute_units", e->cus},
      {"epoch_memcpy_nodes", e->last_epoch_copies[0]},
      {"epoch_memset_nodes", e->last_epoch_copies[1]},
      {"epoch_kernel_nodes", e->last_epoch_copies[2]},
  };
  auto it = facts.find(k);
  if (it == facts.end()) return -1;
  *value = it->second;
  return 0;
}

extern "C" int32_t resident_epoch_time_ops(void* engine, int32_t begin, int32_t end, int32_t iters,
                                           float* avg_ms) {
  using namespace re;
  Engine* e = static_cast<Engine*>(engine);
  if (e == nullptr || avg_ms == nullptr || iters < 1) return -1;
  std::lock_guard<std::mutex> lock(e->execute_mutex);
  const KernelEnv env = e->env();
  if (begin < 0 || end > step_op_count(env) || begin >= end) return -1;
  if (e->dec_key == nullptr) {
    if (hipMalloc(&e->dec_key, e->cache_bytes) != hipSuccess) return -2;
    if (hipMalloc(&e->dec_value, e->cache_bytes) != hipSuccess) return -2;
    if (hipMemset(e->dec_key, 0, e->cache_bytes) != hipSuccess) return -2;
    if (hipMemset(e->dec_value, 0, e->cache_bytes) != hipSuccess) return -2;
  }
  // Inputs: the decoder-step staging buffers (rows inactive unless a
  // resident_decoder_step call left others); caches: the decoder-step scratch
  // caches, so the resident epoch state is untouched.
  StepPtrs sp = e->step_io;
  sp.key_cache = e->dec_key;
  sp.value_cache = e->dec_value;
  sp.logits = e->logits;
  sp.done = nullptr;
  if (launch_step_ops(env, sp, e->stream, begin, end) != hipSuccess) return -2;  // warm
  if (hipEventRecord(e->ev_start, e->stream) != hipSuccess) return -2;
  for (int i = 0; i < iters; ++i)
    if (launch_step_ops(env, sp, e->stream, begin, end) != hipSuccess) return -2;
  if (hipEventRecord(e->ev_stop, e->stream) != hipSuccess || hipEventSynchronize(e->ev_stop) != hipSuccess) return -2;
  float ms = 0.f;
  if (hipEventElapsedTime(&ms, e->ev_start, e->ev_stop) != hipSuccess) return -2;
  *avg_ms = ms / iters;
  return 0;
}

extern "C" int32_t resident_epoch_time_layer_op(void* engine, int32_t which, int32_t passes, float* avg_ms) {
  using namespace re;
  Engine* e = static_cast<Engine*>(engine);
  if (e == nullptr || avg_ms == nullptr || passes < 1) return -1;
  std::lock_guard<std::mutex> lock(e->execute_mutex);
  const KernelEnv env = e->env();
  const int per_layer = (step_op_count(env) - 2) / e->dims.layers;
  if (which < 0 || which >= per_layer || !layer_op_launches(env, which)) return -1;
  if (e->dec_key == nullptr) {
    if (hipMalloc(&e->dec_key, e->cache_bytes) != hipSuccess) return -2;
    if (hipMalloc(&e->dec_value, e->cache_bytes) != hipSuccess) return -2;
    if (hipMemset(e->dec_key, 0, e->cache_bytes) != hipSuccess) return -2;
    if (hipMemset(e->dec_value, 0, e->cache_bytes) != hipSuccess) return -2;
  }
  StepPtrs sp = e->step_io;
  sp.key_cache = e->dec_key;
  sp.value_cache = e->dec_value;
  sp.logits = e->logits;
  sp.done = nullptr;
  auto op = [&](int l) { return 1 + per_layer * l + which; };
  if (launch_step_ops(env, sp, e->stream, op(0), op(0) + 1) != hipSuccess) return -2;  // warm
  if (hipEventRecord(e->ev_start, e->stream) != hipSuccess) return -2;
  for (int i = 0; i < passes; ++i)
    for (int l = 0; l < e->dims.layers; ++l)
      if (launch_step_ops(env, sp, e->stream, op(l), op(l) + 1) != hipSuccess) return -2;
  if (hipEventRecord(e->ev_stop, e->stream) != hipSuccess || hipEventSynchronize(e->ev_stop) != hipSuccess) return -2;
  float ms = 0.f;
  if (hipEventElapsedTime(&ms, e->ev_start, e->ev_stop) != hipSuccess) return -2;
  *avg_ms = ms / (passes * e->dims.layers);
  return 0;
}

extern "C" int32_t resident_epoch_gemm(const void* A, const void* W, const void* W2, const void* bias, void* out,
                                       int32_t M, int32_t N, int32_t K, int32_t epilogue, int32_t dtype_bytes) {
  using namespace re;
  if (A == nullptr || W == nullptr || out == nullptr || M < 0 || N <= 0 || K <= 0 || epilogue < kGemmStore ||
      epilogue > kGemmSwiGlu || (dtype_bytes != 2 && dtype_bytes != 4) || (epilogue == kGemmSwiGlu && W2 == nullptr))
    return -1;
  // the bf16 kernel reads the bias four elements at a time
  if (dtype_bytes == 2 && epilogue == kGemmStore && bias != nullptr && (reinterpret_cast<uintptr_t>(bias) & 7) != 0)
    return -1;
  GemmArgs g{};
  g.A = A;
  g.W = W;
  g.W2 = W2;
  g.out = out;
  g.bias = epilogue == kGemmStore ? bias : nullptr;
  g.M = M;
  g.N = N;
  g.K = K;
  g.lda = K;
  g.ldw = K;
  g.ldo = N;
  const hipError_t e = launch_gemm(g, epilogue, dtype_bytes, nullptr);
  if (e == hipErrorInvalidValue) {
    (void)hipGetLastError();
    return -1;
  }
  if (e != hipSuccess || hipStreamSynchronize(nullptr) != hipSuccess) return -2;
  return 0;
}

extern "C" int32_t resident_epoch_kernel_timing(void* engine, int32_t enable) {
  Engine* e = static_cast<Engine*>(engine);
  if (e == nullptr) return -1;
  std::lock_guard<std::mutex> lock(e->execute_mutex);
  e->timing = enable != 0;
  e->timing_ms.clear();
  return 0;
}

extern "C" int32_t resident_epoch_read_kernel_timing(void* engine, float* ms, int32_t n) {
  Engine* e = static_cast<Engine*>(engine);
  if (e == nullptr || ms == nullptr || n < 0) return -1;
  std::lock_guard<std::mutex> lock(e->execute_mutex);
  const int count = std::min<int>(n, static_cast<int>(e->timing_ms.size()));
  for (int i = 0; i < count; ++i) ms[i] = e->timing_ms[i];
  e->timing_ms.erase(e->timing_ms.begin(), e->timing_ms.begin() + count);
  return count;
}
