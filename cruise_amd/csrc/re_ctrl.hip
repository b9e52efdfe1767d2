// Epoch controller kernels of the resident decode epoch (gfx950): validation,
// generation continuity, row clear / KV import, per-step argmax and row update,
// finish and emit (controller/g4c_b4_resident_epoch.cpp:177-622), plus the
// synthetic weight fill.  Integer state, bit-exact with the reference.
#include <algorithm>

#include "re_device.h"
#include "re_layout.h"

namespace re {
namespace {

// ---------------------------------------------------------------------------
// Epoch controller (controller/g4c_b4_resident_epoch.cpp).
// ---------------------------------------------------------------------------
struct CtrlArgs {
  StatePtrs st;
  int B, bpr, physical_blocks, block_size, capacity, vocab;
  int lm_wg;          // argmax partials per batch row
  int am_row_major;   // partial p of row b at [b * lm_wg + p] (else [p * B + b])
  int layers, kv_dim, elem_bytes;  // cache geometry (import checksum length)
  const float* am_val;
  const int32_t* am_idx;
  const int32_t* am_bad;
  int has_payload;
};

__device__ __forceinline__ int compute_slot(const int32_t* table, const CtrlArgs& a, int request,
                                            long long position) {
  // ComputeSlot, CTRL:84-97, with the capacity / blocks-per-row parameters.
  if (request < 0 || request >= a.B || position < 0 || position >= a.capacity) return -1;
  const int logical = static_cast<int>(position / a.block_size);
  const int offset = static_cast<int>(position % a.block_size);
  if (logical >= a.bpr) return -1;
  const int physical = table[request * a.bpr + logical];
  if (physical < 0 || physical >= a.physical_blocks) return -1;
  return physical * a.block_size + offset;
}

// compute_slot with the block-table entry already read (physical: the entry
// of the position's logical block, clamped into the row).
__device__ __forceinline__ int slot_of_physical(int physical, const CtrlArgs& a, int request, long long position) {
  if (request < 0 || request >= a.B || position < 0 || position >= a.capacity) return -1;
  const int logical = static_cast<int>(position / a.block_size);
  const int offset = static_cast<int>(position % a.block_size);
  if (logical >= a.bpr) return -1;
  if (physical < 0 || physical >= a.physical_blocks) return -1;
  return physical * a.block_size + offset;
}

struct FeedView {
  const int64_t* token;
  const int64_t* pos;
  const int32_t* len;
  const int32_t* slot;  // nullptr in import mode
  const int32_t* active;
  const int32_t* table;
  const int32_t* control;
};

__device__ FeedView feed_view(const uint8_t* feed, int B, int bpr, bool importing, long long payload_bytes) {
  FeedView f;
  const uint8_t* p = feed + (importing ? payload_bytes : 0);
  f.token = reinterpret_cast<const int64_t*>(p);
  p += 8 * B;
  f.pos = reinterpret_cast<const int64_t*>(p);
  p += 8 * B;
  f.len = reinterpret_cast<const int32_t*>(p);
  p += 4 * B;
  if (importing) {
    f.slot = nullptr;
  } else {
    f.slot = reinterpret_cast<const int32_t*>(p);
    p += 4 * B;
  }
  f.active = reinterpret_cast<const int32_t*>(p);
  p += 4 * B;
  f.table = reinterpret_cast<const int32_t*>(p);
  p += 4 * B * bpr;
  p += kTilingBytes;
  f.control = reinterpret_cast<const int32_t*>(p);
  return f;
}

// Row-parallel controller kernels: one workgroup, thread r owns batch row r
// (rows strided by the block size).  A check the reference runs row by row
// and stops at the first failing row becomes a per-row code plus the lowest
// failing row, found with an LDS atomicMin over the key (row << 8) | (status -
// 200); the row's code is the status, and the side effects of the rows before
// it are applied exactly as the sequential loop applies them.
constexpr int kCtrlThreads = 1024;
constexpr int kNoFailure = 0x7fffffff;
// Block-uniqueness bitmap: pools up to 32 x 15360 = 491,520 blocks are checked
// in LDS; larger pools compare pairs in global memory.
constexpr int kBitmapWords = 15360;

__device__ __forceinline__ int fail_key(int row, int32_t status) { return (row << 8) | (status - 200); }
__device__ __forceinline__ int fail_row(int key) { return key == kNoFailure ? 0x7fffffff : key >> 8; }
__device__ __forceinline__ int32_t fail_status(int key) { return (key & 0xff) + 200; }

// Validation, import bookkeeping, generation continuity (CTRL:204-471) and the
// loop's initial state (CTRL:473-483), in the reference's order of checks:
// feed form, K / sampling / variant (335-340), EOS ids (341-345), block table
// range and uniqueness (346-353), per-row metadata and slots (354-385), import
// mask and rows (387-429), generation continuity (448-464).
__global__ void __launch_bounds__(kCtrlThreads) k_ctrl_init(CtrlArgs a, long long payload_bytes) {
  __shared__ unsigned seen[kBitmapWords];
  __shared__ int eos_bad, block_bad, meta_key, import_key, cont_key, active_count, any_adopted;
  StatePtrs& s = a.st;
  const int B = a.B, tid = threadIdx.x, T = blockDim.x;
  // In import mode the payload precedes everything and the slot input is
  // absent, so the control offset differs; the host tells us the form.
  const bool importing = a.has_payload != 0;
  const FeedView f = feed_view(s.feed, B, a.bpr, importing, payload_bytes);
  const int32_t* ctl = f.control;
  const int32_t encoded_variant = ctl[2 + B];
  const bool flagged = (encoded_variant & kImportGraphFlag) != 0;
  const int32_t import_mask = flagged ? (encoded_variant & (kImportGraphFlag - 1)) : 0;
  const int32_t graph_variant = flagged ? (encoded_variant & ~(kImportGraphFlag | 0xF)) : encoded_variant;
  const int32_t max_steps = ctl[0];
  const int32_t sampling = ctl[1 + B];
  const int nent = B * a.bpr;
  const bool bitmap = a.physical_blocks <= kBitmapWords * 32;
  if (tid == 0) {
    eos_bad = 0;
    block_bad = 0;
    meta_key = kNoFailure;
    import_key = kNoFailure;
    cont_key = kNoFailure;
    active_count = 0;
    any_adopted = 0;
  }
  if (bitmap)
    for (int i = tid; i < (a.physical_blocks + 31) / 32; i += T) seen[i] = 0u;
  int64_t* history = reinterpret_cast<int64_t*>(s.fetch);
  for (int i = tid; i < kMaxEpochSteps * B; i += T) history[i] = -1;
  for (int i = tid; i < nent; i += T) s.table[i] = f.table[i];
  for (int r = tid; r < B; r += T) {
    s.executed[r] = 0;
    s.eos[r] = ctl[1 + r];
    s.initial_active[r] = f.active[r];
    s.generation[r] = ctl[3 + B + r];
    s.cur_token[r] = f.token[r];
    s.cur_pos[r] = f.pos[r];
    s.cur_len[r] = f.len[r];
    s.cur_active[r] = f.active[r];
    s.cur_slot[r] = f.slot ? f.slot[r] : compute_slot(f.table, a, r, f.pos[r]);
  }
  __syncthreads();

  // Every check evaluated in parallel; which one decides is settled below.
  for (int r = tid; r < B; r += T)
    if (ctl[1 + r] < 0 || ctl[1 + r] >= a.vocab) atomicOr(&eos_bad, 1);
  for (int i = tid; i < nent; i += T) {
    const int blk = f.table[i];
    bool bad = blk < 0 || blk >= a.physical_blocks;
    if (!bad && bitmap) {
      bad = (atomicOr(&seen[blk >> 5], 1u << (blk & 31)) >> (blk & 31)) & 1u;
    } else if (!bad) {
      for (int j = 0; j < i && !bad; ++j) bad = f.table[j] == blk;
    }
    if (bad) atomicOr(&block_bad, 1);
  }
  for (int r = tid; r < B; r += T) {
    const int32_t act = f.active[r], len = f.len[r], gen = ctl[3 + B + r];
    const int64_t tok = f.token[r], pos = f.pos[r];
    int32_t code = kStatusOk;
    if ((act != 0 && act != 1) || tok < 0 || tok >= a.vocab || pos < 0 || pos >= a.capacity) {
      code = kStatusInvalidMetadata;
    } else if (act == 1) {
      if (gen <= 0 || len != pos + 1) code = kStatusInvalidMetadata;
      else if (pos + max_steps > a.capacity) code = kStatusCapacityExceeded;
    } else if (len == 0) {
      if (gen != 0) code = kStatusInvalidMetadata;
    } else if (len != pos + 1) {
      code = kStatusInvalidMetadata;
    }
    if (code == kStatusOk && compute_slot(f.table, a, r, pos) != (f.slot ? f.slot[r] : compute_slot(f.table, a, r, pos)))
      code = kStatusSlotMismatch;
    if (code != kStatusOk) atomicMin(&meta_key, fail_key(r, code));
    if (importing && r < 31 && ((import_mask >> r) & 1) != 0 && (act != 1 || gen <= 0))
      atomicMin(&import_key, fail_key(r, kStatusInvalidMetadata));
    const bool imported = importing && r < 31 && ((import_mask >> r) & 1) != 0;
    if (act == 1 && !imported) {
      // A row adopted by the import matches its resident record by construction.
      const bool same_gen = s.res_gen[r] == gen;
      const bool ok = same_gen ? (s.res_valid[r] != 0 && s.res_token[r] == tok && s.res_pos[r] == pos &&
                                  s.res_len[r] == len)
                               : (pos == 0 && len == 1);
      if (!ok) atomicMin(&cont_key, fail_key(r, kStatusResidentContinuity));
    }
  }
  __syncthreads();

  int32_t status = kStatusOk;
  bool import_reached = false;  // every earlier check passed: the import loop runs
  if (flagged != importing) {
    status = kStatusInvalidMetadata;  // feed form and flag disagree
  } else if (max_steps < 1 || max_steps > kMaxEpochSteps || sampling != 0 || graph_variant != 0) {
    status = sampling != 0 ? kStatusUnsupportedSampling
             : graph_variant != 0 ? kStatusUnsupportedGraph
                                  : kStatusInvalidMetadata;
  } else if (eos_bad) {
    status = kStatusInvalidMetadata;
  } else if (block_bad) {
    status = kStatusInvalidBlockTable;
  } else if (meta_key != kNoFailure) {
    status = fail_status(meta_key);
  } else if (importing && (import_mask <= 0 || (B < 31 && import_mask >= (1 << B)))) {
    status = kStatusInvalidMetadata;
  } else {
    import_reached = importing;
    if (importing && import_key != kNoFailure) status = kStatusInvalidMetadata;
    else if (cont_key != kNoFailure) status = kStatusResidentContinuity;
  }
  // The import loop adopts rows in order up to its first failing row; they
  // keep their copied blocks even when the epoch then falls back.
  const int adopt_below = import_reached ? (import_key == kNoFailure ? B : fail_row(import_key)) : 0;
  for (int r = tid; r < B; r += T) {
    const bool adopted = r < adopt_below && r < 31 && ((import_mask >> r) & 1) != 0;
    if (adopted) {
      atomicOr(&any_adopted, 1);
      s.res_gen[r] = ctl[3 + B + r];
      s.res_token[r] = f.token[r];
      s.res_pos[r] = f.pos[r];
      s.res_len[r] = f.len[r];
      s.res_valid[r] = 1;
    }
    int32_t reason = kFinishFallback, clear = adopted ? 2 : 0;
    if (status == kStatusOk) {
      const int32_t act = f.active[r];
      reason = act == 1 ? kFinishNone : (f.len[r] == 0 ? kFinishEmpty : kFinishAlreadyFinished);
      if (act == 1 && !adopted && s.res_gen[r] != ctl[3 + B + r]) clear = 1;  // a new generation
      if (act != 0) atomicAdd(&active_count, 1);
    }
    s.reason[r] = reason;
    s.clear_row[r] = clear;
  }
  __syncthreads();
  if (tid == 0) {
    s.import_sum[0] = 0;  // accumulators of k_import_checksum
    s.import_sum[1] = 0;
    s.misc[0] = max_steps;
    s.misc[1] = sampling;
    s.misc[2] = graph_variant;
    s.misc[3] = flagged ? 1 : 0;
    s.misc[4] = import_mask;
    // the whole mask adopted: the checksum is emitted even when the
    // continuity check after the import then falls back (CTRL:430-464)
    s.misc[5] = import_reached && import_key == kNoFailure ? 1 : 0;
    s.misc[6] = any_adopted;  // some masked row adopted: its copy runs
    *s.model_calls = 0;
    *s.status = status;
    // the loop runs no step after a fallback or with no active row (CTRL:488)
    *s.done = (status != kStatusOk || active_count == 0) ? 1 : 0;
  }
}

// Row clear (ClearCacheRow, CTRL:129-147, following the row's table entries)
// and, in import mode, the copy of one block per layer from the payload
// (CTRL:411-423).  Grid-stride over 16-byte words of all flagged blocks.
struct ClearArgs {
  const int32_t* clear_row;
  const int32_t* table;
  const uint8_t* payload;  // nullptr unless importing
  uint8_t* key_cache;
  uint8_t* value_cache;
  int B, bpr, layers;
  long long block_bytes, layer_bytes;  // bytes of one block / one layer of a cache
};

__global__ void k_clear_rows(ClearArgs a) {
  const long long words_per_block = a.block_bytes / 16;
  const long long per_row = (long long)a.layers * a.bpr * words_per_block;
  const long long total = 2LL * a.B * per_row;  // key and value
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (long long)gridDim.x * blockDim.x) {
    const int cache = static_cast<int>(i / (a.B * per_row));
    long long rem = i - (long long)cache * a.B * per_row;
    const int r = static_cast<int>(rem / per_row);
    const int flag = a.clear_row[r];
    if (flag == 0) continue;
    rem -= (long long)r * per_row;
    const int layer = static_cast<int>(rem / (a.bpr * words_per_block));
    rem -= (long long)layer * a.bpr * words_per_block;
    const int local = static_cast<int>(rem / words_per_block);
    const long long w = rem - (long long)local * words_per_block;
    const int blk = a.table[r * a.bpr + local];
    uint8_t* base = cache == 0 ? a.key_cache : a.value_cache;
    uint4* dst = reinterpret_cast<uint4*>(base + layer * a.layer_bytes + blk * a.block_bytes) + w;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (flag == 2 && local == 0 && a.payload != nullptr) {
      // payload [K|V][layers][B][block]
      const uint8_t* src = a.payload + ((size_t)cache * a.layers * a.B + (size_t)layer * a.B + r) * a.block_bytes;
      v = reinterpret_cast<const uint4*>(src)[w];
    }
    *dst = v;
  }
}

// One step of the loop body after the model call (CTRL:496-589): argmax over
// the LM-head partials, position progress, history, EOS, slot and length.
__global__ void __launch_bounds__(1024) k_ctrl_step(CtrlArgs a) {
  StatePtrs& s = a.st;
  if (*s.done != 0) return;
  const int B = a.B;
  __shared__ int tok_s[256];
  __shared__ int bad_s[256];
  __shared__ int fail_at, active_count;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nwaves = blockDim.x >> 6;
  // The state of row r = tid the update below reads, requested first so it
  // arrives while the partials are merged (clamped: threads past B ignore it).
  const int rq = min(tid, B - 1);
  const int32_t act_r = s.cur_active[rq];
  const int64_t pos_r = s.cur_pos[rq];
  const int64_t eos_r = s.eos[rq];
  const int32_t exec_r = s.executed[rq];
  // the block-table entry of the next position (compute_slot's lookup)
  const int64_t np_r = pos_r + 1;
  const int lg_r = static_cast<int>(min(max(np_r, (int64_t)0), (int64_t)a.capacity) / a.block_size);
  const int32_t phys_r = s.table[rq * a.bpr + min(lg_r, a.bpr - 1)];
  // Final argmax over the LM head's workgroup partials (CTRL:99-119): one wave
  // per batch row; each lane requests its strided share of the partials at
  // once (clamped, ignored past the count), then a shuffle reduction keeps the
  // first index of the maximum; any non-finite logit flags the row.  Up to 256
  // partials per row (one per CU): a wave takes four rows at once, four
  // partials per lane each, so every request of the pass is in flight
  // together.
  auto better = [](float ov, int oi, float bv, int bi) {
    return oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi < bi));
  };
  constexpr int kRows = 4, kPer = 4;
  if (a.lm_wg <= 64 * kPer) {
    for (int b0 = wave; b0 < B; b0 += nwaves * kRows) {
      float v[kRows][kPer];
      int ix[kRows][kPer], fl[kRows][kPer];
#pragma unroll
      for (int i = 0; i < kRows; ++i)
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
          const int b = min(b0 + i * nwaves, B - 1);
          const int p = min(lane + 64 * j, a.lm_wg - 1);
          const size_t o = a.am_row_major ? (size_t)b * a.lm_wg + p : (size_t)p * B + b;
          v[i][j] = a.am_val[o];
          ix[i][j] = a.am_idx[o];
          fl[i][j] = a.am_bad[o];
        }
      float bv[kRows];
      int bi[kRows], bb[kRows];
#pragma unroll
      for (int i = 0; i < kRows; ++i) {
        bv[i] = 0.f;
        bi[i] = -1;
        bb[i] = 0;
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
          if (lane + 64 * j >= a.lm_wg) continue;
          bb[i] |= fl[i][j];
          if (better(v[i][j], ix[i][j], bv[i], bi[i])) {
            bv[i] = v[i][j];
            bi[i] = ix[i][j];
          }
        }
      }
#pragma unroll
      for (int m = 32; m >= 1; m >>= 1)
#pragma unroll
        for (int i = 0; i < kRows; ++i) {
          const float ov = __shfl_xor(bv[i], m, 64);
          const int oi = __shfl_xor(bi[i], m, 64);
          bb[i] |= __shfl_xor(bb[i], m, 64);
          if (better(ov, oi, bv[i], bi[i])) {
            bv[i] = ov;
            bi[i] = oi;
          }
        }
      if (lane == 0)
#pragma unroll
        for (int i = 0; i < kRows; ++i)
          if (b0 + i * nwaves < B) {
            tok_s[b0 + i * nwaves] = bi[i];
            bad_s[b0 + i * nwaves] = bb[i];
          }
    }
  } else {
    constexpr int kUnroll = 16;
    for (int b = wave; b < B; b += nwaves) {
      float bv = 0.f;
      int bi = -1, bb = 0;
      for (int w0 = 0; w0 < a.lm_wg; w0 += 64 * kUnroll) {
        float v[kUnroll];
        int ix[kUnroll], fl[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
          const int p = min(w0 + lane + 64 * u, a.lm_wg - 1);
          const size_t o = a.am_row_major ? (size_t)b * a.lm_wg + p : (size_t)p * B + b;
          v[u] = a.am_val[o];
          ix[u] = a.am_idx[o];
          fl[u] = a.am_bad[o];
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
          if (w0 + lane + 64 * u >= a.lm_wg) continue;
          bb |= fl[u];
          if (better(v[u], ix[u], bv, bi)) {
            bv = v[u];
            bi = ix[u];
          }
        }
      }
#pragma unroll
      for (int m = 32; m >= 1; m >>= 1) {
        const float ov = __shfl_xor(bv, m, 64);
        const int oi = __shfl_xor(bi, m, 64);
        bb |= __shfl_xor(bb, m, 64);
        if (better(ov, oi, bv, bi)) {
          bv = ov;
          bi = oi;
        }
      }
      if (lane == 0) {
        tok_s[b] = bi;
        bad_s[b] = bb;
      }
    }
  }
  if (tid == 0) {
    fail_at = kNoFailure;
    active_count = 0;
  }
  const int call = *s.model_calls + 1;  // read by every thread before thread 0 stores it
  __syncthreads();
  int64_t* history = reinterpret_cast<int64_t*>(s.fetch);
  // The row update (CTRL:546-581).  Row r fails with NonFinite (bad logits),
  // PositionProgress (never, with next_position = where(active, pos + 1,
  // pos), batched_decoder_step.py:409-411) or CapacityExceeded (no slot for
  // the next position: checked after the row's history, count, position,
  // token and length are updated).  The rows before the first failing row are
  // updated in full, as the sequential loop does before it stops.
  // B <= 256 < blockDim.x: thread r owns row r.
  const int r = tid;
  const bool live = r < B && act_r != 0;
  int32_t code = kStatusOk;
  int slot_next = -1;
  if (live) {
    const int64_t next_pos = np_r;
    if (bad_s[r] != 0 || tok_s[r] < 0) {
      code = kStatusNonFiniteLogits;
    } else if (next_pos != a.capacity) {
      slot_next = slot_of_physical(phys_r, a, r, next_pos);  // compute_slot with the entry requested above
      if (slot_next < 0) code = kStatusCapacityExceeded;
    }
    if (code != kStatusOk) atomicMin(&fail_at, fail_key(r, code));
  }
  __syncthreads();
  const int first = fail_row(fail_at);  // uniform
  if (live && (r < first || (r == first && code == kStatusCapacityExceeded))) {
    const int64_t tok = tok_s[r];
    const int64_t next_pos = np_r;
    history[(call - 1) * B + r] = tok;
    s.executed[r] = exec_r + 1;
    s.cur_pos[r] = next_pos;
    s.cur_token[r] = tok;
    s.cur_len[r] = static_cast<int32_t>(next_pos + 1);
    if (r < first) {
      s.cur_slot[r] = slot_next;  // -1 at the capacity
      if (tok == eos_r) {
        s.cur_active[r] = 0;
        s.reason[r] = kFinishEos;
      } else {
        atomicAdd(&active_count, 1);
      }
    }
  }
  const bool failed = first != 0x7fffffff;
  if (failed && r < B) s.reason[r] = kFinishFallback;  // the same thread wrote any EOS reason above
  __syncthreads();
  if (tid == 0) {
    *s.model_calls = call;
    if (failed) {
      *s.status = fail_status(fail_at);
      *s.done = 1;
    } else if (active_count == 0) {
      *s.done = 1;
    }
  }
}

// Adler-32 of the imported blocks as they sit in the resident caches, in the
// order of CTRL:430-445 (key cache then value cache, layer-major, rows
// ascending), computed in parallel: over bytes d_0..d_{N-1} with a = 1, b = 0
// at the start, a = 1 + sum d_i and b = N + sum (N - i) d_i (mod 65521).  Each
// thread reduces its 16-byte words, each workgroup adds its two residues
// into s.import_sum with one 64-bit atomic (integer sums: the order does not
// matter); k_ctrl_finish forms the checksum.
struct ImportSumArgs {
  const int32_t* misc;    // [4] import mask, [5] import applied
  const int32_t* table;
  const uint8_t* key_cache;
  const uint8_t* value_cache;
  unsigned long long* sum;
  int B, bpr, layers;
  long long block_bytes, layer_bytes;
};

constexpr unsigned kAdlerModulus = 65521;

__global__ void __launch_bounds__(256) k_import_checksum(ImportSumArgs a) {
  __shared__ unsigned long long red[2][4];
  if (a.misc[5] == 0) return;  // no import applied this epoch
  const int mask = a.misc[4];
  int rows[32];
  int nsel = 0;
  for (int r = 0; r < a.B && r < 32; ++r)
    if (mask & (1 << r)) rows[nsel++] = r;
  const long long words_per_block = a.block_bytes / 16;
  const long long total_words = 2LL * a.layers * nsel * words_per_block;
  const unsigned long long n = (unsigned long long)total_words * 16;
  unsigned long long s1 = 0, s2 = 0;
  for (long long w = (long long)blockIdx.x * blockDim.x + threadIdx.x; w < total_words;
       w += (long long)gridDim.x * blockDim.x) {
    const long long piece = w / words_per_block;  // (cache, layer, k-th selected row)
    const long long off = w - piece * words_per_block;
    const int k = static_cast<int>(piece % nsel);
    const int layer = static_cast<int>((piece / nsel) % a.layers);
    const int cache = static_cast<int>(piece / ((long long)nsel * a.layers));
    const int blk = a.table[rows[k] * a.bpr];
    const uint8_t* base = cache == 0 ? a.key_cache : a.value_cache;
    const uint4 v = reinterpret_cast<const uint4*>(base + layer * a.layer_bytes + blk * a.block_bytes)[off];
    const unsigned words[4] = {v.x, v.y, v.z, v.w};
    const unsigned long long i0 = (unsigned long long)w * 16;  // stream index of the word's first byte
#pragma unroll
    for (int q = 0; q < 4; ++q) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const unsigned long long d = (words[q] >> (8 * e)) & 0xFFu;
        s1 += d;
        s2 += d * (n - (i0 + 4 * q + e));
      }
    }
    s1 %= kAdlerModulus;
    s2 %= kAdlerModulus;
  }
  // workgroup sum of the residues (each < 65521), one atomic per workgroup
  for (int m = 32; m >= 1; m >>= 1) {
    s1 += __shfl_xor(s1, m, 64);
    s2 += __shfl_xor(s2, m, 64);
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    red[0][wave] = s1;
    red[1][wave] = s2;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long t1 = 0, t2 = 0;
    for (int i = 0; i < 4; ++i) {
      t1 += red[0][i];
      t2 += red[1][i];
    }
    atomicAdd(&a.sum[0], t1 % kAdlerModulus);
    atomicAdd(&a.sum[1], t2 % kAdlerModulus);
  }
}

// Finish reasons, resident save and emit (CTRL:296-324, 592-621), one thread
// per row.
__global__ void __launch_bounds__(256) k_ctrl_finish(CtrlArgs a, uint32_t import_checksum_unused) {
  (void)import_checksum_unused;
  __shared__ int initial, final_count, nsel;
  StatePtrs& s = a.st;
  const int B = a.B, tid = threadIdx.x;
  const int32_t status = *s.status;
  const bool fallback = status != kStatusOk;
  const bool importing = s.misc[3] != 0;
  const int32_t mask = s.misc[4];
  int32_t* control = reinterpret_cast<int32_t*>(s.fetch + 8 * kMaxEpochSteps * B);
  if (tid == 0) {
    initial = 0;
    final_count = 0;
    nsel = 0;
  }
  __syncthreads();
  for (int r = tid; r < B; r += blockDim.x) {
    const int32_t init = s.initial_active[r];
    int32_t reason = s.reason[r];
    if (!fallback && init == 1 && reason == kFinishNone) reason = kFinishMaxSteps;
    if (!fallback && init != 0) {
      s.reason[r] = reason;
      s.res_gen[r] = s.generation[r];
      s.res_token[r] = s.cur_token[r];
      s.res_pos[r] = s.cur_pos[r];
      s.res_len[r] = s.cur_len[r];
      s.res_valid[r] = 1;
    }
    control[6 + r] = s.eos[r];
    control[6 + B + r] = init;
    control[6 + 2 * B + r] = s.executed[r];
    control[6 + 3 * B + r] = reason;
    control[6 + 4 * B + 2 + r] = init == 1 ? s.generation[r] : 0;
    if (init != 0) atomicAdd(&initial, 1);
    if ((fallback ? init : s.cur_active[r]) != 0) atomicAdd(&final_count, 1);
    if (r < 31 && ((mask >> r) & 1) != 0) atomicAdd(&nsel, 1);
  }
  __syncthreads();
  if (tid != 0) return;
  control[0] = s.misc[0];
  control[1] = s.misc[1];
  control[2] = s.misc[2];
  control[3] = status;
  control[4] = *s.model_calls;
  if (importing && s.misc[5] != 0) {
    // CTRL:301-303: the import checksum; see k_import_checksum for the sums
    const unsigned long long n =
        2ULL * a.layers * nsel * (unsigned long long)a.block_size * a.kv_dim * a.elem_bytes;
    const unsigned first = static_cast<unsigned>((1 + s.import_sum[0]) % kAdlerModulus);
    const unsigned second = static_cast<unsigned>((n % kAdlerModulus + s.import_sum[1]) % kAdlerModulus);
    control[5] = static_cast<int32_t>((second << 16) | first);
  } else {
    control[5] = importing ? 0 : (fallback ? 1 : 0);  // import rejected before the copy: 0
  }
  control[6 + 4 * B] = initial;
  control[6 + 4 * B + 1] = final_count;
}

// Counter-based N(0, std) fill for synthetic weights: a 64-bit mix of
// (seed, stream, index) gives two uniforms, Box-Muller in fp32.
__device__ __forceinline__ unsigned long long mix64(unsigned long long x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

__global__ void k_fill_normal(void* dst, long long elems, int dtype_bytes, unsigned long long seed,
                              unsigned long long stream_id, float std_dev) {
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < elems;
       i += (long long)gridDim.x * blockDim.x) {
    const unsigned long long h = mix64(mix64(seed ^ (stream_id * 0xD1B54A32D192ED03ull)) + (unsigned long long)i);
    const float u1 = (static_cast<float>(h >> 40) + 1.0f) * (1.0f / 16777216.0f);          // (0, 1]
    const float u2 = static_cast<float>((h >> 16) & 0xFFFFFFull) * (1.0f / 16777216.0f);    // [0, 1)
    const float z = sqrtf(-2.0f * logf(u1)) * cosf(6.283185307179586f * u2);
    const float v = z * std_dev;
    if (dtype_bytes == 2)
      static_cast<bf16_t*>(dst)[i] = f_to_bf16(v);
    else
      static_cast<float*>(dst)[i] = v;
  }
}

}  // namespace

static CtrlArgs ctrl_args(const KernelEnv& env, const StatePtrs& st) {
  CtrlArgs a{};
  a.st = st;
  a.B = env.dims.batch;
  a.bpr = env.dims.blocks_per_row;
  a.physical_blocks = env.dims.physical_blocks;
  a.block_size = env.dims.block_size;
  a.capacity = env.dims.capacity;
  a.vocab = env.dims.vocab;
  a.lm_wg = env.plan.argmax_parts;
  a.am_row_major = env.plan.argmax_row_major;
  a.layers = env.dims.layers;
  a.kv_dim = env.dims.kv_dim();
  a.elem_bytes = env.dims.dtype_bytes;
  a.am_val = env.scratch.am_val;
  a.am_idx = env.scratch.am_idx;
  a.am_bad = env.scratch.am_bad;
  return a;
}

static long long payload_bytes_of(const Dims& d) {
  return 2LL * d.layers * d.batch * d.block_size * d.kv_dim() * d.dtype_bytes;
}

hipError_t launch_ctrl_init(const KernelEnv& env, const StatePtrs& st, int has_payload, hipStream_t stream) {
  CtrlArgs a = ctrl_args(env, st);
  a.has_payload = has_payload;
  k_ctrl_init<<<1, kCtrlThreads, 0, stream>>>(a, has_payload ? payload_bytes_of(env.dims) : 0);
  return hipGetLastError();
}

hipError_t launch_clear_rows(const KernelEnv& env, const StatePtrs& st, void* key_cache, void* value_cache,
                             hipStream_t stream) {
  const Dims& d = env.dims;
  ClearArgs c{};
  c.clear_row = st.clear_row;
  c.table = st.table;
  c.payload = st.feed;  // payload leads the feed in import mode; rows flagged 2 only then
  c.key_cache = static_cast<uint8_t*>(key_cache);
  c.value_cache = static_cast<uint8_t*>(value_cache);
  c.B = d.batch;
  c.bpr = d.blocks_per_row;
  c.layers = d.layers;
  c.block_bytes = (long long)d.block_size * d.kv_dim() * d.dtype_bytes;
  c.layer_bytes = (long long)d.slots() * d.kv_dim() * d.dtype_bytes;
  k_clear_rows<<<1024, 256, 0, stream>>>(c);
  return hipGetLastError();
}

hipError_t launch_import_checksum(const KernelEnv& env, const StatePtrs& st, const void* key_cache,
                                  const void* value_cache, hipStream_t stream) {
  const Dims& d = env.dims;
  ImportSumArgs c{};
  c.misc = st.misc;
  c.table = st.table;
  c.key_cache = static_cast<const uint8_t*>(key_cache);
  c.value_cache = static_cast<const uint8_t*>(value_cache);
  c.sum = st.import_sum;
  c.B = d.batch;
  c.bpr = d.blocks_per_row;
  c.layers = d.layers;
  c.block_bytes = (long long)d.block_size * d.kv_dim() * d.dtype_bytes;
  c.layer_bytes = (long long)d.slots() * d.kv_dim() * d.dtype_bytes;
  k_import_checksum<<<256, 256, 0, stream>>>(c);
  return hipGetLastError();
}

// One workgroup column per (imported row, cache); 16-byte copies, coalesced.
// The host has checked every source range against the mapped allocation.
__global__ void __launch_bounds__(256) k_import_gather(ImportGatherArgs a) {
  const int cache = blockIdx.z;  // 2 * layer + (0 for K, 1 for V)
  const int layer = cache >> 1, kv = cache & 1;
  const int row = a.rows[blockIdx.y];
  const re_u32x4* src = reinterpret_cast<const re_u32x4*>(a.src[cache] + a.block_ids[row] * a.block_bytes);
  re_u32x4* dst = reinterpret_cast<re_u32x4*>(
      a.dst + (((long long)kv * a.layers + layer) * a.batch + row) * a.block_bytes);
  const long long n = a.block_bytes / 16;
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long long)gridDim.x * blockDim.x)
    dst[i] = __builtin_nontemporal_load(src + i);
}

hipError_t launch_import_gather(const ImportGatherArgs& a, hipStream_t stream) {
  if (a.nrows < 1 || a.nrows > 4 || a.layers < 1 || 2 * a.layers > kImportMaxCaches || a.block_bytes % 16 != 0)
    return hipErrorInvalidValue;
  const long long words = a.block_bytes / 16;
  const int chunks = static_cast<int>(std::min<long long>((words + 255) / 256, 64));
  k_import_gather<<<dim3(chunks, a.nrows, 2 * a.layers), 256, 0, stream>>>(a);
  return hipGetLastError();
}

hipError_t launch_ctrl_step(const KernelEnv& env, const StatePtrs& st, hipStream_t stream) {
  k_ctrl_step<<<1, 1024, 0, stream>>>(ctrl_args(env, st));
  return hipGetLastError();
}

hipError_t launch_ctrl_finish(const KernelEnv& env, const StatePtrs& st, hipStream_t stream) {
  k_ctrl_finish<<<1, 256, 0, stream>>>(ctrl_args(env, st), 0u);
  return hipGetLastError();
}

namespace {
__global__ void k_clear_blocks(uint8_t* kc, uint8_t* vc, const int32_t* blocks, int nblocks, int layers,
                               long long block_bytes, long long layer_bytes) {
  const long long words = block_bytes / 16;
  const long long total = 2LL * layers * nblocks * words;
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (long long)gridDim.x * blockDim.x) {
    const int cache = static_cast<int>(i / ((long long)layers * nblocks * words));
    long long rem = i - (long long)cache * layers * nblocks * words;
    const int layer = static_cast<int>(rem / (nblocks * words));
    rem -= (long long)layer * nblocks * words;
    const int bi = static_cast<int>(rem / words);
    const long long w = rem - (long long)bi * words;
    uint8_t* base = cache == 0 ? kc : vc;
    reinterpret_cast<uint4*>(base + layer * layer_bytes + (long long)blocks[bi] * block_bytes)[w] =
        make_uint4(0, 0, 0, 0);
  }
}
}  // namespace

hipError_t launch_clear_blocks(const KernelEnv& env, void* key_cache, void* value_cache, const int32_t* blocks,
                               int nblocks, hipStream_t stream) {
  const Dims& d = env.dims;
  k_clear_blocks<<<512, 256, 0, stream>>>(static_cast<uint8_t*>(key_cache), static_cast<uint8_t*>(value_cache),
                                          blocks, nblocks, d.layers,
                                          (long long)d.block_size * d.kv_dim() * d.dtype_bytes,
                                          (long long)d.slots() * d.kv_dim() * d.dtype_bytes);
  return hipGetLastError();
}

hipError_t launch_fill_synthetic(void* dst, long long elems, int dtype_bytes, unsigned long long seed,
                                 unsigned long long stream_id, float std_dev, hipStream_t stream) {
  k_fill_normal<<<4096, 256, 0, stream>>>(dst, elems, dtype_bytes, seed, stream_id, std_dev);
  return hipGetLastError();
}

}  // namespace re
