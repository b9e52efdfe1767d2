// Host/device shared layout of the resident-epoch engine: model dims, the
// weight arena offsets, device state pointers and the kernel launchers.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace re {

constexpr int kMaxEpochSteps = 8;       // controller/g4c_b4_resident_epoch.cpp:17
constexpr int kImportGraphFlag = 0x100;  // controller/g4c_b4_resident_epoch.cpp:27
constexpr int kTilingBytes = 72;        // native/resident_epoch_bridge.cpp:61

// Device statuses (controller/g4c_b4_resident_epoch.cpp:60-74) and finish
// reasons (51-58).
enum Status : int32_t {
  kStatusOk = 0,
  kStatusInvalidMetadata = 201,
  kStatusCapacityExceeded = 202,
  kStatusInvalidBlockTable = 203,
  kStatusSlotMismatch = 204,
  kStatusUnsupportedSampling = 205,
  kStatusUnsupportedGraph = 206,
  kStatusModelError = 207,
  kStatusInvalidModelOutput = 208,
  kStatusNonFiniteLogits = 209,
  kStatusPositionProgress = 210,
  kStatusAllocationFailure = 211,
  kStatusResidentContinuity = 212,
};
enum Finish : int32_t {
  kFinishNone = 0,
  kFinishEos = 1,
  kFinishMaxSteps = 2,
  kFinishFallback = 3,
  kFinishEmpty = 4,
  kFinishAlreadyFinished = 5,
};

struct Dims {
  int layers, hidden, heads, kv_heads, head_dim, intermediate, vocab;
  float rope_theta, rms_eps;
  int dtype_bytes;  // 2 = bf16, 4 = fp32
  // paged geometry
  int batch, physical_blocks, block_size, blocks_per_row, capacity;
  int configured_eos;

  int groups() const { return heads / kv_heads; }
  int q_dim() const { return heads * head_dim; }
  int kv_dim() const { return kv_heads * head_dim; }
  int qkv_rows() const { return q_dim() + 2 * kv_dim(); }
  long long slots() const { return (long long)physical_blocks * block_size; }
  long long cache_elems() const { return (long long)layers * slots() * kv_dim(); }
};

// Byte offsets of one layer's tensors inside the weight arena (each 256-byte
// aligned).  q, k and v rows are stacked into one [qkv_rows, hidden] matrix.
struct LayerOffsets {
  size_t input_norm, post_norm, qkv_w, qkv_b, o_w, gate_w, up_w, down_w;
};

// Byte offsets of one layer's matrices in the packed copy the matrix-core
// projections stream (re_mfma.hip): each matrix as 16-row strips of 32-wide k
// steps, one 1 KB tile per (strip, step) in the order the wave's lanes read it.
struct PackedOffsets {
  size_t qkv, o, gate, up, down;
};

// The epoch's device state.  Feed and fetch are contiguous byte buffers in
// the ABI order so one copy moves each; the rest persists across epochs.
struct StatePtrs {
  // feed (H2D once per epoch)
  uint8_t* feed;
  // working rows of the current step (CTRL:473-483)
  int64_t* cur_token;
  int64_t* cur_pos;
  int32_t* cur_len;
  int32_t* cur_slot;
  int32_t* cur_active;
  int32_t* table;  // [B * BPR]
  // epoch bookkeeping
  int32_t* done;        // 1 = remaining steps are skipped
  int32_t* status;      // device status
  int32_t* model_calls;
  int32_t* executed;    // [B]
  int32_t* reason;      // [B]
  int32_t* clear_row;   // [B] new generation -> clear the row's blocks
  int32_t* eos;         // [B]
  int32_t* initial_active;  // [B]
  int32_t* generation;  // [B] from control
  int32_t* misc;        // [0] K, [1] sampling, [2] variant, [3] importing, [4] import mask,
                        // [5] import complete, [6] some import row adopted
  // resident state (CTRL:624-631)
  int32_t* res_gen;
  int64_t* res_token;
  int64_t* res_pos;
  int32_t* res_len;
  int32_t* res_valid;
  // fetch (D2H once per epoch): history i64[8,B] then control i32[6+4B+2+B]
  uint8_t* fetch;
  // import mode: Adler-32 partial sums (sum of bytes, sum of weighted bytes)
  unsigned long long* import_sum;
};

// Inputs of one decoder step (the 9-input decoder ABI, resolved to device
// pointers) plus the step's outputs.
struct StepPtrs {
  const int64_t* token;
  const int64_t* pos;
  const int32_t* len;
  const int32_t* slot;
  const int32_t* active;
  const int32_t* table;
  void* key_cache;
  void* value_cache;
  float* logits;          // [B, V]
  int64_t* next_pos;      // [B] (nullptr: not written)
  const int32_t* done;    // early-exit flag (nullptr: always run)
};

// Activation and scratch buffers of one engine.
struct Scratch {
  void* hidden;       // T [B, H] residual stream
  void* q;            // T [B, NH*d] post-RoPE queries
  void* attn;         // T [B, NH*d]
  void* mlp;          // T [B, I]
  float* partial;     // K-segment partial sums [segments, B, H]
  float* am_val;      // argmax partial values [nwg, B]
  int32_t* am_idx;    // argmax partial indices [nwg, B]
  int32_t* am_bad;    // non-finite flags [nwg, B]
  float* inv_freq;    // fp32 [d/2]
  float* rope;        // [B, d/2, 2] the step's RoPE cos, sin (rounded to T)
  void* xn;           // T [B, H] normalized rows (matrix-core projections)
  float* mf_part;     // matrix-core o / down partial sums [8][B][H] (split plan)
  float* sp_scores;   // window-split attention: scores, tile statistics, tile P.V (AttnArgs)
  float* sp_stats;
  float* sp_part;
};

struct LaunchPlan {
  int mb;          // batch rows per GEMV pass (4 or 8)
  int row_tiles;   // ceil(B / mb)
  int waves;       // waves per GEMV workgroup
  int qkv_grid, o_grid, gu_grid, down_grid, lm_grid;
  int qkv_waves;          // waves per qkv workgroup of the row-pair kernel (one RoPE row pair each)
  int qkv_ksplit;         // > 0: qkv as k_qkv_ksplit, K split over 7 waves (the grid); 0: k_proj
  int o_waves;            // waves per o-proj workgroup (one row pair each): 4, or 7
  int o_segments, down_segments;  // K-segments of 3584 elements
  int lm_wg;       // workgroups of the LM head (= argmax partial count)
  int argmax_parts;  // partials per row k_ctrl_step reduces: lm_wg, or one per CU (matrix-core LM head)
  int argmax_row_major;  // 1: the partials of a row are contiguous (per-CU LM head)
  int slot_cus;    // > 0: gate/up and LM head use slot-weighted unit ranges (re_step.hip)
  int slot_w[4];   // their per-slot weights
  // Down projection with the whole K in one workgroup (re_step.hip
  // k_down_whole): 0 = split-K segments + reduce launch; else its grid.
  int down_whole_grid;
  // 1: the projections run on the matrix cores (re_mfma.hip, 64 rows)
  int mfma;
  // > 0 (with mfma): gate/up runs one workgroup per CU (k_mf_gu_cu), this grid
  int gu_cu;
  // 1: decode attention per (row, KV head) for all query heads of the group
  int grouped_attn;
  int attn_split;  // > 0: decode attention split over the window in this many 256-position tiles
};

// Arguments of the paged decode attention (re_attn.hip).
struct AttnArgs {
  const int32_t* done;
  const void* q;           // T [B, NH*d]
  const void* key_cache;   // this layer [slots, KVH, d]
  const void* value_cache;
  const int32_t* len;
  const int32_t* table;    // [B, BPR]
  void* out;               // T [B, NH*d]
  int B, heads, kv_heads, head_dim, block_size, blocks_per_row, window;
  long long slots;
  int bs_shift;            // log2(block_size) when it is a power of two, else -1
  int grouped;             // 1: one workgroup per (row, KV head) (re_attn.hip k_attn_group); 2: the same on
                           // the matrix cores (k_attn_mgroup)
  int packed_out;          // out in the matrix-core path's packed layout (xpack_index, K = NH*d)
  // > 0: the window split into split_tiles tiles of 256 positions over three
  // launches: one workgroup per (row, head, tile) with grouped == 0
  // (re_attn.hip k_attn_split_*), per (row, KV head, tile) with grouped == 2
  // (k_attn_msplit_*); not with grouped == 1
  int split_tiles;
  float* sp_scores;        // [B*NH][window] scaled scores
  float* sp_stats;         // [B*NH][split_tiles][2] each tile's max and sum of exp(s - max)
  float* sp_part;          // [B*NH][split_tiles][d] each tile's P.V
};
size_t attention_lds_bytes(const Dims& d);
// The grouped attention's default: many rows (B x KV heads >= 64); whether the
// shape allows it at all.
bool group_attention_default(const Dims& d);
bool group_attention_fits(const Dims& d);
bool group_attention_mfma_fits(const Dims& d);
bool group_attention_msplit_fits(const Dims& d);
hipError_t prepare_attention(const Dims& d);
hipError_t launch_attention(const AttnArgs& a, const Dims& d, hipStream_t stream);

// LDS bytes of the projection kernels and their K-segment length (re_step.hip).
size_t normed_lds_bytes(int mb, int hidden, int dtype_bytes, int waves);
size_t resid_lds_bytes(int mb, int dtype_bytes, int waves);
int k_segment_elems();
// Largest hidden size of the row kernels (embed+norm, residual reduce+norm).
int row_kernel_max_hidden();

// ---- kernel launchers (re_kernels.hip) ----
struct KernelEnv {
  Dims dims;
  LaunchPlan plan;
  const uint8_t* weights;  // arena base
  const LayerOffsets* layer_off;  // host array [layers]
  size_t embedding_off, final_norm_off, lm_head_off;
  Scratch scratch;
  const uint8_t* packed;               // matrix-core copy of the matrices (plan.mfma)
  const PackedOffsets* packed_off;     // host array [layers]
  size_t packed_lm_off;
};

// One decoder step: embedding, L layers, final norm + LM head with argmax
// partials.  The step is an indexed list of launches; launch_step_ops runs the
// range [begin, end) of it (re_step.hip).
hipError_t launch_decoder_step(const KernelEnv& env, const StepPtrs& step, hipStream_t stream);
hipError_t launch_step_ops(const KernelEnv& env, const StepPtrs& step, hipStream_t stream, int begin, int end);
int step_op_count(const KernelEnv& env);
bool layer_op_launches(const KernelEnv& env, int which);
// The op whose launch the epoch timing brackets: layer's gate/up projection.
int timed_op_index(const KernelEnv& env, int layer);
// Grid sizes of the grid-stride projections from the kernels' occupancy.
void plan_grids(LaunchPlan& p, const Dims& d, int cus);
// Decode projections on the matrix cores at 64 batch rows (re_mfma.hip):
// the RMSNorm (where the projection has one) and the projection of one op.
enum class MfmaOp { kQkv, kO, kGateUp, kDown, kLmHead };
bool mfma_step_supported(const Dims& d);
int mfma_lm_partials(const Dims& d);
bool mfma_lm_cu_fits(const Dims& d, int cus);
bool mfma_split_fits(const Dims& d);
bool mfma_gu_cu_fits(const Dims& d, int cus);
size_t mfma_split_partial_bytes(const Dims& d);
bool mfma_qkv_split_fits(const Dims& d);
hipError_t prepare_mfma();
// Layout of the packed copy; returns its bytes.
size_t mfma_packed_layout(const Dims& d, PackedOffsets* layers, size_t* lm_off);
// Pack one [rows, K] matrix (qkv_head_dim > 0: the stacked qkv matrix, whose
// strips hold RoPE pairs of heads of that size).
hipError_t mfma_pack_matrix(const void* src, void* dst, int rows, int K, int qkv_head_dim, hipStream_t stream);
hipError_t launch_mfma_op(MfmaOp op, const KernelEnv& env, const StepPtrs& st, int layer, hipStream_t stream);
// Controller kernels.
hipError_t launch_ctrl_init(const KernelEnv& env, const StatePtrs& st, int has_payload,
                            hipStream_t stream);
hipError_t launch_clear_rows(const KernelEnv& env, const StatePtrs& st, void* key_cache,
                             void* value_cache, hipStream_t stream);
hipError_t launch_ctrl_step(const KernelEnv& env, const StatePtrs& st, hipStream_t stream);
hipError_t launch_ctrl_finish(const KernelEnv& env, const StatePtrs& st, hipStream_t stream);
// Import mode: Adler-32 of the imported blocks as they sit in the caches.
hipError_t launch_import_checksum(const KernelEnv& env, const StatePtrs& st, const void* key_cache,
                                  const void* value_cache, hipStream_t stream);
// Device-IPC import: gather each imported row's source block of every cache
// (2 x layers caches, mapped from another process) into the payload region
// [K|V][layer][row][block] of the device feed, so the import epoch runs as a
// host-file import would without the payload crossing the host.
constexpr int kImportMaxCaches = 56;  // 2 x 28 layers: the IPC record's slots
struct ImportGatherArgs {
  const uint8_t* src[kImportMaxCaches];  // cache c's first byte (allocation base + offset)
  uint8_t* dst;                          // the payload region of the device feed
  long long block_ids[4];                // source block of each row
  int rows[4];                           // imported rows, ascending
  int nrows, layers, batch;
  long long block_bytes;                 // a multiple of 16
};
hipError_t launch_import_gather(const ImportGatherArgs& a, hipStream_t stream);
// Batched prefill (re_prefill.hip): M prompt tokens of several rows at once.
struct PrefillRows {           // embedding + per-token RoPE table
  const int64_t* token;        // [M]
  const int32_t* pos;          // [M] position of each token in its row
  const void* embedding;
  const float* inv_freq;       // [d/2]
  void* hidden;                // T [M, H]
  float* rope;                 // [M, d/2, 2] cos, sin (rounded to T)
  int M, H, V, head_dim;
};
struct PrefillQkv {            // RoPE in place + paged KV write
  void* qkv;                   // T [M, ld]: q | k | v rows, bias included
  const float* rope;
  const int32_t* slot;         // [M] paged slot of each token
  void* key_cache;             // this layer [slots, KVH, d]
  void* value_cache;
  long long slots;
  int M, ld, heads, kv_heads, head_dim;
};
struct PrefillAttn {           // causal attention within each row's prompt
  const void* qkv;             // T [M, ld] after RoPE
  void* out;                   // T [M, heads * d]
  const int32_t* pos;          // [M]
  const int4* tiles;           // MFMA path: {first query token, row's first token, queries, first position}
  int M, ld, heads, kv_heads, head_dim;
};
// Store: out = T(acc + bias); Residual: out = T(out + T(acc)); SwiGlu (bf16
// only): W holds the gate rows and W2 the up rows, and out[m, n] =
// T(T(silu(T(gate))) * T(up)) over N output columns.
enum GemmEpilogue : int { kGemmStore = 0, kGemmResidual = 1, kGemmSwiGlu = 2 };
struct GemmArgs {              // out[M,N] (epilogue) A[M,K] W[N,K]^T
  const void* A;
  const void* W;
  void* out;
  const void* bias;            // [N] or null (store epilogue)
  int M, N, K;
  long long lda, ldw, ldo;
  const void* W2;              // [N,K] up rows of the SwiGLU epilogue (W: the gate rows)
};
hipError_t launch_prefill_embed(const PrefillRows& a, int dtype_bytes, hipStream_t stream);
hipError_t launch_prefill_rmsnorm(const void* x, const void* w, void* y, int M, int H, float eps, int dtype_bytes,
                                  hipStream_t stream);
hipError_t launch_prefill_swiglu(const void* gate, const void* up, void* out, long long n, int dtype_bytes,
                                 hipStream_t stream);
hipError_t launch_prefill_qkv_post(const PrefillQkv& a, int dtype_bytes, hipStream_t stream);
hipError_t launch_gemm(const GemmArgs& a, int epi, int dtype_bytes, hipStream_t stream);
// The MFMA attention serves bf16 models with head_dim 128 (64-query tiles).
bool prefill_attention_mfma(const Dims& d);
size_t prefill_attention_lds(const Dims& d, int max_keys);
hipError_t prepare_prefill(const Dims& d);
hipError_t launch_prefill_attention(const PrefillAttn& a, const Dims& d, int ntiles, hipStream_t stream);
// Helpers for prefill / state management.
hipError_t launch_clear_blocks(const KernelEnv& env, void* key_cache, void* value_cache,
                               const int32_t* blocks, int nblocks, hipStream_t stream);
hipError_t launch_fill_synthetic(void* dst, long long elems, int dtype_bytes, unsigned long long seed,
                                 unsigned long long stream_id, float std_dev, hipStream_t stream);

}  // namespace re
