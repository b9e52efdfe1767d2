/* C-ABI of the MI355X resident decode epoch library (libresident_epoch.so).
 *
 * Plain C: pointers and sizes only.  Host pointers and device pointers are
 * both accepted wherever an argument is marked "host or device" (the library
 * copies with hipMemcpyDefault).
 *
 * The first three entry points keep the reference's signatures, argument
 * meaning, status codes and commit-state ordering so existing callers
 * (the sidecar server and the ctypes engine) bind them unchanged.  The
 * remaining entry points expose the reference's two internal ABIs (the
 * 8-input/2-output epoch and the 9-input/4-output decoder step) plus the
 * state access a caller of those ABIs needs.
 */
#ifndef CRUISE_RESIDENT_EPOCH_H
#define CRUISE_RESIDENT_EPOCH_H

#include <stdint.h>

#include "resident_epoch_protocol.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Device-IPC KV metadata, 4,088 bytes packed.
 * Same layout as native/resident_epoch_bridge.h:7-22.  On MI355X each key
 * slot holds the 64-byte hipIpcMemHandle_t of the allocation containing
 * cache c (c = 2 * layer + 0 for K, 1 for V); source_offsets[c] is that
 * cache's byte offset in the allocation (a multiple of 16), source_bytes the
 * common allocation size (below 2 GiB), block_ids[r] the source block of
 * imported row r.  Slots past 2 x layers are all zero. */
#pragma pack(push, 1)
typedef struct ResidentEpochIpcMetadata {
  uint64_t magic;
  uint32_t version;
  uint32_t import_mask;
  uint64_t source_bytes;
  int32_t row_generations[4];
  int32_t block_ids[4];
  uint64_t source_offsets[56];
  char keys[56][64];
} ResidentEpochIpcMetadata;
#pragma pack(pop)

/* Replaces native/resident_epoch_bridge.h:24-27 (resident_epoch_bridge.cpp:360-422).
 *
 * graph_config: JSON.  The reference's config/graph_config.json is accepted
 *   as is (its "inputs_tensor_desc" fixes B, layers, blocks, block size, KV
 *   heads and head dim; the model defaults to Qwen2.5-7B and the logical
 *   capacity to 8).  Optional "model", "engine" and "weights" objects set the
 *   dims, dtype, paged geometry, capacity and weight source.
 * external_weight_dir: directory of raw tensor files in the reference bundle
 *   naming (materialize_runtime_weights.py:53-80: embedding, final_norm,
 *   lm_head, layers_<i>_<name>), read when "weights.source" is "bundle".
 * air_path, func_config: must be non-null (kept for call compatibility; the
 *   HIP library has no AIR graph or DataFlow function to load).
 * tiling_path: must name a file of exactly 72 bytes (bridge.cpp:97-106).
 * *status, checked in the reference's order: 0 ok; 1 bad arguments, an
 *   engine already active or a weight directory outside /dev/shm/ (unless
 *   the configuration sets "engine": {"require_dev_shm": false}); 2 tiling;
 *   3 graph_config unreadable or invalid; 4 graph build failed; 5 weight
 *   load failed; 6 HIP runtime init failed; 7 no usable HIP device or device
 *   memory exhausted. */
void *resident_epoch_create(const char *air_path, const char *graph_config,
                            const char *func_config,
                            const char *external_weight_dir,
                            const char *tiling_path, int32_t *status);

/* Replaces native/resident_epoch_bridge.h:29-43 (resident_epoch_bridge.cpp:424-649).
 * Host arrays of 4 rows, as in the reference; an engine whose batch is not 4
 * returns 10 (it is driven through resident_epoch_proc instead).
 * output_token_ids is row-major [row * 8 + step].
 * Return: 0 ok; 10 arguments; 11 row metadata;
 * 12 active rows != request_count; 13 transfer file; 30 epoch launch failed;
 * 31 epoch completion failed; 33 executed count out of range; 34 import
 * checksum mismatch; 35 IPC metadata invalid or not mappable (the engine maps
 * each exported allocation once and gathers the imported blocks device to
 * device; handles from the calling process itself cannot be opened).
 * A device fallback (201-212) returns 0
 * with *output_device_status set.  *output_commit_state goes PREPARED ->
 * EXECUTING (just before the one host-to-device copy) -> COMMITTED (after the
 * one device-to-host copy and the unpacking). */
int32_t resident_epoch_execute(
    void *opaque, int32_t request_count, int32_t max_steps,
    const int64_t *input_token_ids, const int64_t *input_positions,
    const int32_t *input_sequence_lengths, const int32_t *input_eos_token_ids,
    const int32_t *input_row_generations, int64_t *output_token_ids,
    int32_t *output_executed, int32_t *output_row_generations,
    int32_t *output_model_calls, int32_t *output_device_status,
    int32_t *output_feed_calls, int32_t *output_fetch_calls,
    int32_t *output_commit_state, int32_t *output_kv_import_checksum,
    int64_t *output_wall_us, int64_t *output_native_cpu_us,
    int64_t *output_declared_input_bytes,
    int64_t *output_declared_output_bytes, const char *transfer_path,
    uint64_t transfer_id, const ResidentEpochIpcMetadata *ipc_metadata);

/* Replaces native/resident_epoch_bridge.h:45 (resident_epoch_bridge.cpp:651-670). */
void resident_epoch_destroy(void *opaque);

/* The 8-input/2-output epoch ABI (config/resident_epoch_func.json; the UDF
 * G4cB4ResidentEpoch::Proc, controller/g4c_b4_resident_epoch.cpp:177-622).
 * feed: host buffer holding token i64[B], position i64[B], sequence_length
 *   i32[B], slot_mapping i32[B], active_mask i32[B], block_table i32[B*BPR],
 *   tiling u8[72], control i32[3+2B] back to back (260 bytes at B=4, BPR=2).
 *   With the import flag (control[2+B] & 0x100) the feed instead starts with
 *   the KV payload and omits slot_mapping (bridge.cpp:499-507, 573-593).
 * fetch: host buffer receiving token_history i64[8,B] then control
 *   i32[6+4B+2+B] (368 bytes at B=4).
 * One host-to-device copy, one epoch, one device-to-host copy.
 * Return: 0 (device status is in the fetched control[3]); -1 bad arguments
 * or sizes; -2 HIP failure. */
int32_t resident_epoch_proc(void *engine, const void *feed, int64_t feed_bytes,
                            void *fetch, int64_t fetch_bytes);

/* The 9-input/4-output decoder step (config/graph_config.json input order;
 * PagedQwenDecoderStep.forward, batched_decoder_step.py:277-417).
 * key_cache/value_cache (host or device) are read and updated in place; the
 * other inputs are host or device arrays of B rows; logits (fp32 [B,V]) and
 * next_position (i64[B]) are written (host or device).  The engine's resident
 * epoch state is not touched.  Return 0, -1 bad arguments, -2 HIP failure. */
int32_t resident_decoder_step(void *engine, const int64_t *token_id,
                              const int64_t *position,
                              const int32_t *sequence_length, void *key_cache,
                              const int32_t *slot_mapping,
                              const int32_t *active_mask,
                              const int32_t *block_table, void *value_cache,
                              const uint8_t *explicit_tiling, float *logits,
                              int64_t *next_position);

/* Teacher-forced prefill of one row for a new generation: clears the row's
 * blocks (block_table_row, BPR entries), runs decoder steps at positions
 * 0..prompt_len-2 with only this row active, and records the row as resident
 * with token prompt[len-1], position len-1, length len.  This stands in for
 * stock-vLLM prefill plus the KV import the reference uses to hand prefilled
 * rows to the device (controller/g4c_b4_resident_epoch.cpp:387-446).
 * Return 0, -1 bad arguments, -2 HIP failure. */
int32_t resident_epoch_prefill(void *engine, int32_t row, int32_t generation,
                               const int64_t *prompt, int32_t prompt_len,
                               const int32_t *block_table_row);

/* Batched prefill of new generations (no reference counterpart: the
 * reference prefills on the host with stock vLLM and imports the KV).  For
 * each of n_rows rows: clear the row's blocks (block_tables row i, BPR
 * entries), write the K/V of prompt positions 0..len-2 to their paged slots,
 * and record the row as resident with token prompt[len-1], position len-1,
 * length len -- the state resident_epoch_prefill leaves, computed in one pass
 * over all the rows' tokens per layer: GEMMs with M = tokens (MFMA for bf16),
 * causal attention within each prompt.
 * rows[n_rows] distinct, generations[n_rows] > 0, prompt_lens[n_rows] in
 * [1, capacity], prompts: the prompts back to back (sum of lengths).
 * Return 0, -1 bad arguments, -2 HIP failure. */
int32_t resident_epoch_prefill_batch(void *engine, int32_t n_rows,
                                     const int32_t *rows,
                                     const int32_t *generations,
                                     const int64_t *prompts,
                                     const int32_t *prompt_lens,
                                     const int32_t *block_tables);

/* resident_epoch_prefill_batch without device allocation.  No counterpart in
 * the reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, serving loops, harnesses that forbid hipMalloc).
 * Same arguments, checks and resulting state as resident_epoch_prefill_batch,
 * but the pass's activations and token tables live in a fixed 64 MiB device
 * array of the library (one per GPU, held until the process ends) instead of
 * the engine's grown-on-demand buffer.  Calls on
 * one GPU share the array and are serialized; a call leaves its contents
 * behind.  The array's device address is resolved on the first call on a
 * device (no allocation).  Return 0, -1 bad arguments, -2 HIP failure
 * (including an unresolvable array address), -3 the pass does not
 * fit the array (about 69 KB per prompt token at Qwen2.5-7B's shape, so
 * some 970 tokens at most; prompts of one token need none). */
int32_t resident_epoch_prefill_batch_noalloc(void *engine, int32_t n_rows,
                                             const int32_t *rows,
                                             const int32_t *generations,
                                             const int64_t *prompts,
                                             const int32_t *prompt_lens,
                                             const int32_t *block_tables);

/* Named state access (host or device buffers of exactly the named size).
 * Names: any weight of the bundle ("embedding", "layers_3_q_weight", ...),
 * "key_cache", "value_cache" (resident caches [L,P,bs,KVH,d]), "logits"
 * (fp32 [B,V] of the last step run), "resident_rows" (i64[5,B]: generation,
 * token, position, length, valid).  Writing a weight is how weights arrive
 * when "weights.source" is "upload".  Return 0, -1 unknown name or size,
 * -2 HIP failure. */
int32_t resident_epoch_read_state(void *engine, const char *name, void *dst,
                                  int64_t bytes);
int32_t resident_epoch_write_state(void *engine, const char *name,
                                   const void *src, int64_t bytes);

/* Integer facts about an engine: "batch", "layers", "hidden", "heads",
 * "kv_heads", "head_dim", "intermediate", "vocab", "physical_blocks",
 * "block_size", "blocks_per_row", "capacity", "dtype_bytes",
 * "feed_bytes", "fetch_bytes", "cache_bytes", "weight_bytes",
 * "streamed_weight_bytes", "configured_eos", "import_feed_bytes",
 * "step_ops" (entries of a decoder step's launch list), "ops_per_layer",
 * "timing_layer", launch-plan sizes ("qkv_grid", "gateup_grid", "lm_grid",
 * "o_segments", "down_segments", "gemv_rows_per_pass"), "compute_units",
 * and the nodes of the last epoch launched, counted from its captured
 * graph(s): "epoch_memcpy_nodes", "epoch_memset_nodes", "epoch_kernel_nodes"
 * (-1 before the first epoch).  Return 0 or -1 for an unknown key. */
int32_t resident_epoch_info(void *engine, const char *key, int64_t *value);

/* Kernel timing in the epoch: when enabled, each epoch runs as graph part 1,
 * then the gate/up projection of the middle layer of its last step launched
 * between two HIP events on the engine stream, then graph part 2 (still one
 * feed copy and one fetch copy).  read returns, in milliseconds, the timed
 * launches of the epochs completed since the previous read (only epochs in
 * which every step ran), up to n values, and their count. */
int32_t resident_epoch_kernel_timing(void *engine, int32_t enable);
int32_t resident_epoch_read_kernel_timing(void *engine, float *ms, int32_t n);

/* Microbenchmark: launches the range [begin, end) of one decoder step's
 * launch list ("step_ops" entries: embed, then per layer qkv, attention,
 * o-proj, o-reduce, gate/up, down, down-reduce, then the LM head) iters
 * times back to back on the engine stream between two HIP events, on the
 * decoder-step staging inputs and scratch caches (the resident epoch state is
 * not touched).  *avg_ms receives the mean time per repetition.
 * Return 0, -1 bad arguments, -2 HIP failure. */
int32_t resident_epoch_time_ops(void *engine, int32_t begin, int32_t end, int32_t iters, float *avg_ms);

/* Microbenchmark with cold weights: launches op `which` of the per-layer
 * launch list (0 qkv, 1 attention, 2 o-proj, 3 o-reduce, 4 gate/up, 5 down,
 * 6 down-reduce) for layer 0, 1, ..., L-1 in turn, `passes` times, back to
 * back on the engine stream between two HIP events, on the same inputs as
 * resident_epoch_time_ops.  Each launch streams another layer's weights, so
 * none of them is left in the memory-side cache by the launch before (at
 * Qwen2.5-7B's shape a layer's gate/up weights are 272 MB, the cache 256 MB).
 * *avg_ms receives the mean time per launch.  Return 0, -1 bad arguments
 * or an op that launches nothing under the engine's plan (the o- and
 * down-reduce entries unless that projection runs split-K on the row-tiled
 * path), -2 HIP failure. */
int32_t resident_epoch_time_layer_op(void *engine, int32_t which, int32_t passes, float *avg_ms);

/* The batched-prefill GEMM on caller buffers, for checking it against a plain
 * matrix product (no reference counterpart: the reference's prompts are
 * prefilled by stock vLLM).  out[M,N] from A[M,K] and W[N,K], both operands
 * K-contiguous, leading dimensions K, K and N:
 *   epilogue 0: out = T(A W^T + bias)           (bias [N], or null)
 *   epilogue 1: out = T(out + T(A W^T))         (the residual add)
 *   epilogue 2: out = T(T(silu(T(A W^T))) T(A W2^T))  (W gate rows, W2 up rows)
 * T is the rounding to the element type.  dtype_bytes 2: bf16 on the matrix
 * cores (K % 64 == 0, N % 8 == 0, 16-byte aligned buffers, an 8-byte
 * aligned bias); 4: fp32
 * (epilogues 0 and 1).  Device pointers; runs on the null stream and waits
 * for it.  Return 0, -1 bad arguments or a shape the kernel refuses, -2 HIP
 * failure. */
int32_t resident_epoch_gemm(const void *A, const void *W, const void *W2, const void *bias, void *out,
                            int32_t M, int32_t N, int32_t K, int32_t epilogue, int32_t dtype_bytes);

#ifdef __cplusplus
}
#endif

#endif
