// Persistent decoder-step kernel of the resident decode epoch (gfx950, bf16,
// up to four batch rows, hidden = q_dim = 3584, head_dim 128).
//
// One launch runs the L layers and the LM head of a decoder step
// (batched_decoder_step.py:301-408).  The per-op path (re_step.hip) launches
// six kernels per layer; each launch drains the chip before the next one
// fills it, and at B=4 every op is a weight stream that is too short to hide
// that ramp.  Here the grid is exactly the resident capacity of the chip
// (occupancy x CUs) and every workgroup walks the same phase sequence
//
//   for each layer: QKV -> ATTN -> OPROJ -> GATEUP -> DOWN;   then LM head
//
// doing its static share of each phase.  A phase's weights do not depend on
// the activations, so a workgroup issues the loads of its next weight rows
// *before* it waits for the phase's inputs: while the dependency chain
// (qkv -> attention -> o-proj) runs on a few hundred workgroups, the rest of
// the chip already has its next rows in flight and HBM stays busy.
//
// Hand-off between workgroups: one counter per (layer, phase) in `sync`
// (128 bytes apart).  A producer makes its outputs with device-coherent (sc1)
// stores, waits for them to be acknowledged (s_waitcnt vmcnt(0)), passes a
// workgroup barrier, and one thread adds 1 to the counter (relaxed,
// agent-scope atomic).  A consumer's thread 0 polls the counter (sc1 load)
// until it reaches the number of producer workgroups; the workgroup passes an
// LDS-only barrier (weight loads stay in flight) and reads the inputs with
// sc1 loads whose offsets carry a zero read back from LDS after the barrier,
// so they cannot be issued before the wait.  No agent-scope cache write-back
// or invalidate is needed (those cost ~30 ns each, serialized per XCD).
//
// Progress: the grid never exceeds the resident capacity, so every
// workgroup is running; a workgroup only waits for phases that come earlier
// in the sequence, and the earliest unfinished phase always has its inputs.
// A wait that exceeds its deadline sets the abort flag (sync[0]); every
// later wait sees it and the kernel drains, and the controller turns the flag
// into device status 207.
//
// The arithmetic of every phase is the per-op path's (same dot order, same
// wave reductions, same rounding points, down's K-segments summed in segment
// order), so both paths give bit-identical results.
#include <algorithm>
#include <vector>

#include "re_attn.h"
#include "re_device.h"
#include "re_gemv.h"
#include "re_layout.h"

namespace re {
namespace {

#ifndef FUSED_POLL_SLEEP
#define FUSED_POLL_SLEEP 1  // s_sleep units (64 clocks) between polls of a counter
#endif

using FT = bf16_t;
constexpr int kFWaves = 4;
constexpr int kFThreads = kFWaves * 64;
constexpr int kFMB = 4;          // batch rows per pass (B <= 4)
constexpr int kFHeadDim = 128;
constexpr int kCtrStride = 32;   // ints between counters: one 128-byte line each
constexpr int kRedFloats = 128;  // wave totals [0, 32), norm scratch [96, 112), LM combine [0, 48)
constexpr int kNormRedOff = 3 * kFWaves * kRowsPerWave * kFMB;

enum FusedPhase : int { kPhQkv = 0, kPhAttn = 1, kPhO = 2, kPhGu = 3, kPhDown = 4, kPhRed = 5, kPhases = 6 };
constexpr int kRedWgs = 56;  // workgroups that sum DOWN's partials (one value per thread each)
__host__ __device__ constexpr int ctr_index(int layer, int phase) { return 1 + layer * kPhases + phase; }

struct FusedLayerW {
  const FT* in_norm;
  const FT* post_norm;
  const FT* qkv_w;
  const FT* qkv_b;
  const FT* o_w;
  const FT* gate_w;
  const FT* up_w;
  const FT* down_w;
};

struct FusedArgs {
  const int32_t* done;
  const FusedLayerW* lw;  // [L], device memory
  const FT* final_norm;
  const FT* lm_w;
  const FT* hidden;       // [B, H] the step's embedding rows (layer 0's input)
  // Per-layer activations, each written once per launch: layer l's block at
  // act + l * act_stride holds q [B, heads*d], attn [B, heads*d], mlp [B, I],
  // h_mid [B, H] (residual after attention), h_out [B, H] (the layer's
  // output, layer l+1's input) and DOWN's fp32 segment partials
  // [row group][segment][B][8 rows] (a row group's in whole 128-byte lines).
  uint8_t* act;
  long long act_stride;
  int off_q, off_attn, off_mlp, off_hmid, off_hout, off_part;
  const float* rope;      // [B, d/2, 2]
  const int32_t* slot;
  const int32_t* active;
  const int32_t* len;
  const int32_t* table;
  FT* key_cache;          // layer 0; layer l at + l * layer_elems
  FT* value_cache;
  long long layer_elems;
  float* logits;          // [B, V]
  float* am_val;          // [grid, B]
  int32_t* am_idx;
  int32_t* am_bad;
  int32_t* sync;          // [0] abort, then kPhases counters per layer
  unsigned long long* trace;  // optional [grid][L*kPhases+1][3] wall-clock ticks, nullptr: off
  long long slots;
  long long timeout_ticks;  // wall-clock ticks (100 MHz) a wait may last
  int B, H, heads, kv_heads, head_dim, I, V, L;
  int block_size, blocks_per_row, window;
  float eps;
};

// Per-launch schedule, derived from the grid size: the small phases' items
// go to disjoint ranges of workgroups where the grid allows (QKV and DOWN on
// different workgroups, so the next layer's QKV rows can be requested while
// DOWN still runs), GATEUP and the LM head spread over every workgroup.
struct Sched {
  int G;
  int qkv_pairs, qkv_items, attn_items, o_items, dn_items;
  int dn_groups, dn_segs;  // DOWN: row groups (4 row pairs) x K-segments
  int base_o, base_dn;
  int gu_items;
  int t_qkv, t_attn, t_o, t_gu, t_dn, t_red;  // producer workgroups of each phase
};

__device__ __forceinline__ Sched make_sched(const FusedArgs& a) {
  Sched s;
  s.G = gridDim.x;
  s.qkv_pairs = (a.heads + 2 * a.kv_heads) * a.head_dim / 2;
  s.qkv_items = (s.qkv_pairs + kFWaves - 1) / kFWaves;
  s.attn_items = a.B * a.heads;
  s.o_items = (a.H / 2 + kFWaves - 1) / kFWaves;
  s.dn_groups = (a.H / 2 + kFWaves - 1) / kFWaves;
  s.dn_segs = (a.I + kSeg - 1) / kSeg;
  s.dn_items = s.dn_groups * s.dn_segs;
  s.base_o = s.attn_items % s.G;
  s.base_dn = s.qkv_items % s.G;
  s.t_qkv = min(s.G, s.qkv_items);
  s.t_attn = min(s.G, s.attn_items);
  s.t_o = min(s.G, s.o_items);
  s.gu_items = (a.I + kFWaves - 1) / kFWaves;
  s.t_gu = min(s.G, s.gu_items);
  s.t_red = min(s.G, kRedWgs);
  s.t_dn = min(s.G, s.dn_items);  // workgroups with DOWN items (a static first one each)
  return s;
}

// The kernel's loop over layers would otherwise let the compiler hoist every
// per-lane address and every argument-derived value out of it and keep them
// live across all phases, which spills at the 128-register budget.  Each
// phase therefore re-reads its arguments through an opaque copy of the
// kernarg pointer (scalar loads) and re-derives its lane values from an
// opaque copy of the thread id, so its live ranges stay inside the phase.
template <typename V>
__device__ __forceinline__ V opaque_v(V x) {
  asm volatile("" : "+v"(x));
  return x;
}
// The pointers of the arguments are marked global again (the opaque copy
// hides that they came from the kernel arguments).
__device__ __forceinline__ FusedArgs fargs() {
  typedef const __attribute__((address_space(4))) FusedArgs* ConstArgs;  // scalar loads
  ConstArgs p = (ConstArgs)__builtin_amdgcn_kernarg_segment_ptr();
  asm volatile("" : "+s"(p));
  // word by word through the constant address space (scalar loads); unused
  // words are dropped by the compiler
  static_assert(sizeof(FusedArgs) % 4 == 0, "argument block is whole words");
  uint32_t words[sizeof(FusedArgs) / 4];
  const __attribute__((address_space(4))) uint32_t* src = (const __attribute__((address_space(4))) uint32_t*)p;
#pragma unroll
  for (size_t i = 0; i < sizeof(FusedArgs) / 4; ++i) words[i] = src[i];
  FusedArgs a;
  __builtin_memcpy(&a, words, sizeof(FusedArgs));
  a.done = as_global(a.done);
  a.final_norm = as_global(a.final_norm);
  a.lm_w = as_global(a.lm_w);
  a.hidden = as_global(a.hidden);
  a.act = as_global(a.act);
  a.rope = as_global(a.rope);
  a.slot = as_global(a.slot);
  a.active = as_global(a.active);
  a.len = as_global(a.len);
  a.table = as_global(a.table);
  a.key_cache = as_global(a.key_cache);
  a.value_cache = as_global(a.value_cache);
  a.logits = as_global(a.logits);
  a.am_val = as_global(a.am_val);
  a.am_idx = as_global(a.am_idx);
  a.am_bad = as_global(a.am_bad);
  a.sync = as_global(a.sync);
  a.trace = as_global(a.trace);
  return a;
}

__device__ __forceinline__ FusedLayerW layer_w(const FusedArgs& a, int l) {
  typedef const __attribute__((address_space(4))) FusedLayerW* ConstTable;  // scalar loads (read-only table)
  const ConstTable t = (ConstTable)a.lw + l;
  FusedLayerW w;
  w.in_norm = t->in_norm;
  w.post_norm = t->post_norm;
  w.qkv_w = t->qkv_w;
  w.qkv_b = t->qkv_b;
  w.o_w = t->o_w;
  w.gate_w = t->gate_w;
  w.up_w = t->up_w;
  w.down_w = t->down_w;
  w.in_norm = as_global(w.in_norm);
  w.post_norm = as_global(w.post_norm);
  w.qkv_w = as_global(w.qkv_w);
  w.qkv_b = as_global(w.qkv_b);
  w.o_w = as_global(w.o_w);
  w.gate_w = as_global(w.gate_w);
  w.up_w = as_global(w.up_w);
  w.down_w = as_global(w.down_w);
  return w;
}
__device__ __forceinline__ int phase_tid() { return opaque_v(static_cast<int>(threadIdx.x)); }

// Phase trace (diagnostics): thread 0 of each workgroup records the 100 MHz
// wall clock when the phase starts (its first weights requested), when its
// inputs are ready (the wait returned) and when it ends.
enum TraceMark : int { kTrStart = 0, kTrReady = 1, kTrEnd = 2 };
__device__ __forceinline__ void trace_mark(const FusedArgs& a, int slot, int mark);

// Progress-based wave priority for the streaming phases.  The SIMD arbiter
// favours older waves, so with equal static shares the youngest workgroups
// would finish last while the older ones already idle, and the phase would
// end with a fraction of the chip streaming.  A wave that has done `done` of
// its `total` units drops from priority 3 towards 0, which lets the waves
// that are behind catch up.
__device__ __forceinline__ void progress_prio(int done, int total) {
  const int p = total > 0 ? 3 - min(3, (4 * done) / total) : 0;
  switch (p) {
    case 3: __builtin_amdgcn_s_setprio(3); break;
    case 2: __builtin_amdgcn_s_setprio(2); break;
    case 1: __builtin_amdgcn_s_setprio(1); break;
    default: __builtin_amdgcn_s_setprio(0); break;
  }
}

// First item of a phase whose item i runs on workgroup (base + i) mod G.
__device__ __forceinline__ int first_item(int base, int G) { return ((int)blockIdx.x - base + G) % G; }

struct Lds {
  FT* xs;        // [MB][3584] normalized rows or staged activations
  float* red;    // kRedFloats
  int* bcast;    // wait result
  unsigned char* attn;  // attention scratch (aliases xs)
};

// Thread 0 polls counter `idx` (idx < 0: no dependency) until it reaches
// `target`, the abort flag is set, or the deadline passes (which sets the
// flag); then the workgroup passes an LDS-only barrier.  Returns the zero
// read back from LDS, or -1 when the kernel is aborting.
__device__ __forceinline__ int wait_for(const FusedArgs& a, int idx, int target, const Lds& s) {
  if (threadIdx.x == 0) {
    int r = 0;
    if (idx >= 0) {
      const int32_t* c = a.sync + idx * kCtrStride;
      if (__hip_atomic_load(c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
        const uint64_t t0 = wall_clock64();
        // Bounded twice: by the wall-clock deadline and by a poll count
        // (about a second of sleeps) should the clock not advance.
        for (int polls = 0;; ++polls) {
          __builtin_amdgcn_s_sleep(FUSED_POLL_SLEEP);
          if (__hip_atomic_load(c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= target) break;
          if (__hip_atomic_load(a.sync, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) {
            r = -1;
            break;
          }
          if (static_cast<long long>(wall_clock64() - t0) > a.timeout_ticks || polls > (1 << 22)) {
            __hip_atomic_store(a.sync, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            r = -1;
            break;
          }
        }
      }
    }
    *s.bcast = r;
  }
  lds_barrier();
  return *s.bcast;
}

__device__ __forceinline__ void trace_mark(const FusedArgs& a, int slot, int mark) {
  if (a.trace != nullptr && threadIdx.x == 0)
    a.trace[((size_t)blockIdx.x * (a.L * kPhases + 1) + slot) * 3 + mark] = wall_clock64();
}

// The workgroup's coherent stores are acknowledged, then one increment.
__device__ __forceinline__ void signal(const FusedArgs& a, int idx) {
  wait_vmem();
  __syncthreads();
  if (threadIdx.x == 0)
    __hip_atomic_fetch_add(a.sync + idx * kCtrStride, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ CoBuf cobuf(const void* p, long long bytes) {
  return CoBuf::make(p, static_cast<uint32_t>(bytes));
}

// Layer l's activation buffer at byte offset `off` of its block.  Producers
// write them through CoBuf (write-through, acknowledged before the signal);
// consumers read them with ordinary loads after the wait: no L2 can hold a
// stale copy, because every buffer is written once per launch and only read
// after that write (lines cached before the launch were invalidated at its
// start).  Buffers are never reused within a launch for the same reason.
__device__ __forceinline__ FT* act_buf(const FusedArgs& a, int l, int off) {
  return as_global(reinterpret_cast<FT*>(a.act + (size_t)l * a.act_stride + off));
}
__device__ __forceinline__ const FT* layer_input(const FusedArgs& a, int l) {
  return l == 0 ? a.hidden : act_buf(a, l - 1, a.off_hout);
}

// RMSNorm prologue of QKV, GATEUP and the LM head: the rows come straight
// into LDS (global->LDS loads, no registers), the norm weight into
// registers, then the in-place norm (norm_to_lds's arithmetic).  rows must
// already carry the ordering zero.
__device__ __forceinline__ void norm_prologue(const FusedArgs& a, const FT* rows, const FT* norm_w, const Lds& s,
                                              int tid) {
  Vec8<FT> wn[kNormChunks];
  const int per_row = a.H / 8;
#pragma unroll
  for (int j = 0; j < kNormChunks; ++j) wn[j] = Vec8<FT>::load_cached(norm_w + min(tid + 256 * j, per_row - 1) * 8);
  lds_barrier();  // every earlier reader of xs is done
  dma_rows<kFMB>(s.xs, a.H, rows, a.H, a.B, 0, a.H, tid);
  wait_vmem();
  lds_barrier();
  norm_in_lds<kFMB>(s.xs, wn, a.H, a.eps, s.red + kNormRedOff, tid);
}

// Activation rows of a projection into xs [MB][kSeg] (columns [k0, k0+len)
// of X), after every earlier reader of xs is done.
__device__ __forceinline__ void stage_rows(const FusedArgs& a, const FT* X, int ldg, int k0, int len, const Lds& s,
                                           int tid) {
  lds_barrier();
  dma_rows<kFMB>(s.xs, kSeg, X, ldg, a.B, k0, len, tid);
  wait_vmem();
  lds_barrier();
}

// ---------------------------------------------------------------------------
// QKV: RMSNorm prologue, q/k/v rows j and j + d/2 of one head per wave (the
// RoPE pair), bias, RoPE, q store or paged KV slot write -- k_proj<kQkv>'s
// arithmetic (batched_decoder_step.py:224-229, 305-324, 250-264).
// ---------------------------------------------------------------------------
__device__ __forceinline__ bool ph_qkv(int l, const Lds& s) {
  const FusedArgs a = fargs();
  const Sched sc = make_sched(a);
  int i = first_item(0, sc.G);
  if (i >= sc.qkv_items) return true;
  trace_mark(a, l * kPhases + kPhQkv, kTrStart);
  const FusedLayerW w = layer_w(a, l);
  FT* kc = a.key_cache + (size_t)l * a.layer_elems;
  FT* vc = a.value_cache + (size_t)l * a.layer_elems;
  const int tid = phase_tid(), lane = tid & 63, wave = wave_index(tid);
  const int half = a.head_dim >> 1;
  const int nq = a.heads, nkv = a.kv_heads;
  float* wred = s.red + wave * (kRowsPerWave * kFMB);
  const CoBuf qb = cobuf(act_buf(a, l, a.off_q), (long long)a.B * nq * a.head_dim * 2);
  const long long cache_bytes = a.layer_elems * 2;
  const CoBuf kb = cobuf(kc, cache_bytes), vb = cobuf(vc, cache_bytes);
  // The item's q/k/v rows j and j + d/2 of head hg, their biases and the
  // rows' RoPE cos/sin, requested together (before the wait on the first).
  Vec8<FT> wv[kSegChunks][kRowsPerWave];
  int u = 0, hg = 0, j = 0;
  float bias0 = 0.f, bias1 = 0.f, cs = 1.f, sn = 0.f;
  auto issue = [&](int item) {
    u = item * kFWaves + wave;
    const int uc = min(u, sc.qkv_pairs - 1);
    hg = uc / half;
    j = uc - hg * half;
    const int row0 = hg * a.head_dim + j, row1 = row0 + half;
    const FT* wr[kRowsPerWave] = {w.qkv_w + (size_t)row0 * a.H, w.qkv_w + (size_t)row1 * a.H};
    load_rows<FT, kRowsPerWave, true>(wv, wr, 0, a.H, lane);
    bias0 = bf16_to_f(w.qkv_b[row0]);
    bias1 = bf16_to_f(w.qkv_b[row1]);
    const int bc = min(lane, a.B - 1);
    cs = a.rope[((size_t)bc * half + j) * 2];
    sn = a.rope[((size_t)bc * half + j) * 2 + 1];
  };
  issue(i);
  __builtin_amdgcn_sched_barrier(0);
  {
    const int z = wait_for(a, l == 0 ? -1 : ctr_index(l - 1, kPhRed), sc.t_red, s);
    if (z < 0) return false;
    trace_mark(a, l * kPhases + kPhQkv, kTrReady);
    norm_prologue(a, layer_input(a, l) + z, w.in_norm, s, tid);
  }
  for (;;) {
    __builtin_amdgcn_sched_barrier(0);
    float acc[kRowsPerWave][kFMB];
#pragma unroll
    for (int r = 0; r < kRowsPerWave; ++r)
#pragma unroll
      for (int m = 0; m < kFMB; ++m) acc[r][m] = 0.f;
    dot_rows<FT, kFMB, kRowsPerWave, true>(wv, s.xs, a.H, 0, a.H, lane, acc);
    wave_totals<kFMB, kRowsPerWave>(acc, lane, wred);
    if (u < sc.qkv_pairs && lane < a.B) {
      const int b = lane;
      const float qa = round_bf16(wred[0 * kFMB + b] + bias0);
      const float qb_ = round_bf16(wred[1 * kFMB + b] + bias1);
      float oa = qa, ob = qb_;
      if (hg < nq + nkv) {
        oa = round_bf16(round_bf16(qa * cs) + round_bf16(-qb_ * sn));
        ob = round_bf16(round_bf16(qb_ * cs) + round_bf16(qa * sn));
      }
      if (hg < nq) {
        const uint32_t o = static_cast<uint32_t>(((size_t)b * nq * a.head_dim + (size_t)hg * a.head_dim + j) * 2);
        qb.store2(o, f_to_bf16(oa));
        qb.store2(o + half * 2, f_to_bf16(ob));
      } else {
        const int sl = a.slot[b];
        if (a.active[b] != 0 && sl >= 0 && sl < a.slots) {
          const bool is_key = hg < nq + nkv;
          const int kvh = is_key ? hg - nq : hg - nq - nkv;
          const uint32_t o = static_cast<uint32_t>((((size_t)sl * nkv + kvh) * a.head_dim + j) * 2);
          const CoBuf& cb = is_key ? kb : vb;
          cb.store2(o, f_to_bf16(oa));
          cb.store2(o + half * 2, f_to_bf16(ob));
        }
      }
    }
    i += sc.G;
    if (i >= sc.qkv_items) break;
    issue(i);
  }
  signal(a, ctr_index(l, kPhQkv));
  trace_mark(a, l * kPhases + kPhQkv, kTrEnd);
  return true;
}

// ---------------------------------------------------------------------------
// ATTN: one (batch row, query head) per item, the paged decode attention.
// ---------------------------------------------------------------------------
__device__ __forceinline__ bool ph_attn(int l, const Lds& s) {
  const FusedArgs a = fargs();
  const Sched sc = make_sched(a);
  int i = first_item(0, sc.G);
  if (i >= sc.attn_items) return true;
  trace_mark(a, l * kPhases + kPhAttn, kTrStart);
  FT* kc = a.key_cache + (size_t)l * a.layer_elems;
  FT* vc = a.value_cache + (size_t)l * a.layer_elems;
  const int tid = phase_tid();
  const int z = wait_for(a, ctr_index(l, kPhQkv), sc.t_qkv, s);
  if (z < 0) return false;
  trace_mark(a, l * kPhases + kPhAttn, kTrReady);
  AttnArgs at{};
  at.done = nullptr;
  at.q = act_buf(a, l, a.off_q);
  at.key_cache = kc;
  at.value_cache = vc;
  at.len = a.len;
  at.table = a.table;
  at.out = act_buf(a, l, a.off_attn);
  at.B = a.B;
  at.heads = a.heads;
  at.kv_heads = a.kv_heads;
  at.head_dim = a.head_dim;
  at.block_size = a.block_size;
  at.blocks_per_row = a.blocks_per_row;
  at.window = a.window;
  at.slots = a.slots;
  for (; i < sc.attn_items; i += sc.G) {
    attn_body_lean<FT, kFHeadDim>(at, i, s.attn, s.red, static_cast<uint32_t>(z), tid);
    __syncthreads();  // the next item rewrites the scratch
  }
  signal(a, ctr_index(l, kPhAttn));
  trace_mark(a, l * kPhases + kPhAttn, kTrEnd);
  return true;
}

// ---------------------------------------------------------------------------
// OPROJ: rows 2u, 2u+1 of Wo per wave over the one K-segment, residual add
// h = T(h + T(attn Wo^T)) -- k_resid's single-segment arithmetic
// (batched_decoder_step.py:380-386).
// ---------------------------------------------------------------------------
__device__ __forceinline__ bool ph_oproj(int l, const Lds& s) {
  const FusedArgs a = fargs();
  const Sched sc = make_sched(a);
  int i = first_item(sc.base_o, sc.G);
  if (i >= sc.o_items) return true;
  trace_mark(a, l * kPhases + kPhO, kTrStart);
  const FusedLayerW w = layer_w(a, l);
  const int tid = phase_tid(), lane = tid & 63, wave = wave_index(tid);
  const int units = a.H / 2;
  const int K = a.heads * a.head_dim;  // == kSeg
  float* wred = s.red + wave * (kRowsPerWave * kFMB);
  const FT* hin = layer_input(a, l);
  const FT* attn = act_buf(a, l, a.off_attn);
  const CoBuf hmid = cobuf(act_buf(a, l, a.off_hmid), (long long)a.B * a.H * 2);
  uint32_t z = 0;
  bool first = true;
  for (; i < sc.o_items; i += sc.G) {
    const int u = i * kFWaves + wave;
    const int uc = min(u, units - 1);
    const FT* wr[kRowsPerWave] = {w.o_w + (size_t)(2 * uc) * K, w.o_w + (size_t)(2 * uc + 1) * K};
    Vec8<FT> wv[kSegChunks][kRowsPerWave];
    load_rows<FT, kRowsPerWave, true>(wv, wr, 0, K, lane);
    __builtin_amdgcn_sched_barrier(0);
    if (first) {
      const int zz = wait_for(a, ctr_index(l, kPhAttn), sc.t_attn, s);
      if (zz < 0) return false;
      trace_mark(a, l * kPhases + kPhO, kTrReady);
      z = static_cast<uint32_t>(zz);
      first = false;
    }
    const size_t hidx = (size_t)min(lane, a.B - 1) * a.H + 2 * uc;
    const uint32_t hp = *reinterpret_cast<const uint32_t*>(hin + hidx + z);
    stage_rows(a, attn + z, K, 0, K, s, tid);
    float acc[kRowsPerWave][kFMB];
#pragma unroll
    for (int r = 0; r < kRowsPerWave; ++r)
#pragma unroll
      for (int m = 0; m < kFMB; ++m) acc[r][m] = 0.f;
    dot_rows<FT, kFMB, kRowsPerWave, true>(wv, s.xs, kSeg, 0, K, lane, acc);
    wave_totals<kFMB, kRowsPerWave>(acc, lane, wred);
    if (u < units && lane < a.B) {
      const float h0 = __uint_as_float(hp << 16), h1 = __uint_as_float(hp & 0xffff0000u);
      const float n0 = h0 + round_bf16(wred[0 * kFMB + lane]);
      const float n1 = h1 + round_bf16(wred[1 * kFMB + lane]);
      hmid.store4(static_cast<uint32_t>(hidx * 2), f2_to_bf16x2(n0, n1));
    }
  }
  signal(a, ctr_index(l, kPhO));
  trace_mark(a, l * kPhases + kPhO, kTrEnd);
  return true;
}

// ---------------------------------------------------------------------------
// GATEUP: RMSNorm prologue, gate row u and up row u per wave, SiLU(gate)*up
// -- k_proj<kGateUp>'s arithmetic (batched_decoder_step.py:388-398).  Each
// workgroup owns a contiguous range of units, its waves taking every fourth.
// A unit's output is stored after the next unit's rows are requested, so the
// store's acknowledgement never delays those rows.
// ---------------------------------------------------------------------------
__device__ __forceinline__ bool ph_gateup(int l, const Lds& s) {
  const FusedArgs a = fargs();
  const Sched sc = make_sched(a);
  const int U = a.I;
  const int u0 = (int)((long long)blockIdx.x * U / sc.G), u1 = (int)((long long)(blockIdx.x + 1) * U / sc.G);
  if (u0 >= u1) return true;
  trace_mark(a, l * kPhases + kPhGu, kTrStart);
  const FusedLayerW w = layer_w(a, l);
  const int tid = phase_tid(), lane = tid & 63, wave = wave_index(tid);
  float* wred = s.red + wave * (kRowsPerWave * kFMB);
  const CoBuf mb = cobuf(act_buf(a, l, a.off_mlp), (long long)a.B * U * 2);
  Vec8<FT> wv[kSegChunks][kRowsPerWave];
  auto issue = [&](int u) {
    const int uc = min(u, u1 - 1);
    const FT* wr[kRowsPerWave] = {w.gate_w + (size_t)uc * a.H, w.up_w + (size_t)uc * a.H};
    load_rows<FT, kRowsPerWave, true>(wv, wr, 0, a.H, lane);
  };
  int u = u0 + wave;
  const int mine = (u1 - u0 - wave + kFWaves - 1) / kFWaves;  // this wave's units
  issue(u);
  __builtin_amdgcn_sched_barrier(0);
  const int z = wait_for(a, ctr_index(l, kPhO), sc.t_o, s);
  if (z < 0) return false;
  trace_mark(a, l * kPhases + kPhGu, kTrReady);
  norm_prologue(a, act_buf(a, l, a.off_hmid) + z, w.post_norm, s, tid);
  for (int done = 0; u < u1; ++done) {
    progress_prio(done, mine);
    __builtin_amdgcn_sched_barrier(0);
    float acc[kRowsPerWave][kFMB];
#pragma unroll
    for (int r = 0; r < kRowsPerWave; ++r)
#pragma unroll
      for (int m = 0; m < kFMB; ++m) acc[r][m] = 0.f;
    dot_rows<FT, kFMB, kRowsPerWave, true>(wv, s.xs, a.H, 0, a.H, lane, acc);
    wave_totals<kFMB, kRowsPerWave>(acc, lane, wred);
    bf16_t out = 0;
    if (lane < a.B) {
      const float g = round_bf16(wred[0 * kFMB + lane]);
      const float up = round_bf16(wred[1 * kFMB + lane]);
      const float sg = round_bf16(g / (1.0f + expf(-g)));
      out = f_to_bf16(round_bf16(sg * up));
    }
    const int cur = u;
    u += kFWaves;
    if (u < u1) issue(u);
    if (lane < a.B) mb.store2(static_cast<uint32_t>(((size_t)lane * U + cur) * 2), out);
  }
  __builtin_amdgcn_s_setprio(0);
  signal(a, ctr_index(l, kPhGu));
  trace_mark(a, l * kPhases + kPhGu, kTrEnd);
  return true;
}

// DOWN, split over every workgroup: an item is (K-segment, row group of 4
// row pairs); each wave computes its pair's totals over the segment and
// stores them as fp32 partials [segment][B][H].  Workgroup g takes items g,
// g + G, ...; it signals once, after its last item.
__device__ __forceinline__ bool ph_down(int l, const Lds& s) {
  const FusedArgs a = fargs();
  const Sched sc = make_sched(a);
  int item = blockIdx.x;
  if (item >= sc.dn_items) return true;
  trace_mark(a, l * kPhases + kPhDown, kTrStart);
  const FusedLayerW w = layer_w(a, l);
  const int tid = phase_tid(), lane = tid & 63, wave = wave_index(tid);
  const int units = a.H / 2;
  const int K = a.I;
  float* wred = s.red + wave * (kRowsPerWave * kFMB);
  const FT* mlp = act_buf(a, l, a.off_mlp);
  const CoBuf pb = cobuf(act_buf(a, l, a.off_part), (long long)sc.dn_segs * a.B * a.H * sizeof(float));
  const int mine = (sc.dn_items - item + sc.G - 1) / sc.G;  // this workgroup's items
  Vec8<FT> wv[kSegChunks][kRowsPerWave];
  int seg = 0, rg = 0, k0 = 0, len = 0;
  auto issue = [&](int it) {
    seg = it / sc.dn_groups;
    rg = it - seg * sc.dn_groups;
    k0 = seg * kSeg;
    len = min(K - k0, kSeg);
    const int pc = min(rg * kFWaves + wave, units - 1);
    const FT* wr[kRowsPerWave] = {w.down_w + (size_t)(2 * pc) * K, w.down_w + (size_t)(2 * pc + 1) * K};
    if (len == kSeg)
      load_rows<FT, kRowsPerWave, true>(wv, wr, k0, len, lane);
    else
      load_rows<FT, kRowsPerWave, false>(wv, wr, k0, len, lane);
  };
  issue(item);
  __builtin_amdgcn_sched_barrier(0);
  const int z = wait_for(a, ctr_index(l, kPhGu), sc.t_gu, s);
  if (z < 0) return false;
  trace_mark(a, l * kPhases + kPhDown, kTrReady);
  for (int done = 0;; ++done) {
    progress_prio(done, mine);
    stage_rows(a, mlp + z, K, k0, len, s, tid);
    float acc[kRowsPerWave][kFMB];
#pragma unroll
    for (int r = 0; r < kRowsPerWave; ++r)
#pragma unroll
      for (int m = 0; m < kFMB; ++m) acc[r][m] = 0.f;
    if (len == kSeg)
      dot_rows<FT, kFMB, kRowsPerWave, true>(wv, s.xs, kSeg, 0, len, lane, acc);
    else
      dot_rows<FT, kFMB, kRowsPerWave, false>(wv, s.xs, kSeg, 0, len, lane, acc);
    wave_totals<kFMB, kRowsPerWave>(acc, lane, wred);
    const int p = rg * kFWaves + wave;
    const bool have = p < units && lane < a.B;
    const uint32_t o = static_cast<uint32_t>((((size_t)seg * a.B + min(lane, a.B - 1)) * a.H + 2 * p) * 4);
    const float t0 = wred[0 * kFMB + lane], t1 = wred[1 * kFMB + lane];
    item += sc.G;
    if (item < sc.dn_items) issue(item);
    if (have) {
      pb.store4(o, __float_as_uint(t0));
      pb.store4(o + 4, __float_as_uint(t1));
    }
    if (item >= sc.dn_items) break;
  }
  __builtin_amdgcn_s_setprio(0);
  signal(a, ctr_index(l, kPhDown));
  trace_mark(a, l * kPhases + kPhDown, kTrEnd);
  return true;
}

// REDUCE: the partials of every segment summed in segment order, rounded,
// and added to the residual -- k_resid_reduce's arithmetic
// (batched_decoder_step.py:399-403) -- one value per thread on the first
// kRedWgs workgroups.
__device__ __forceinline__ bool ph_reduce(int l, const Lds& s) {
  const FusedArgs a = fargs();
  const Sched sc = make_sched(a);
  if ((int)blockIdx.x >= sc.t_red) return true;
  trace_mark(a, l * kPhases + kPhRed, kTrStart);
  const int tid = phase_tid();
  const int z = wait_for(a, ctr_index(l, kPhDown), sc.t_dn, s);
  if (z < 0) return false;
  trace_mark(a, l * kPhases + kPhRed, kTrReady);
  const float* part = reinterpret_cast<const float*>(act_buf(a, l, a.off_part)) + z;
  const FT* hmid = act_buf(a, l, a.off_hmid) + z;
  const CoBuf hout = cobuf(act_buf(a, l, a.off_hout), (long long)a.B * a.H * 2);
  const int n = a.B * a.H;
  for (int e = (int)blockIdx.x * kFThreads + tid; e < n; e += sc.t_red * kFThreads) {
    float run = 0.f;
    for (int sg = 0; sg < sc.dn_segs; ++sg) run += part[(size_t)sg * n + e];
    hout.store2(static_cast<uint32_t>(e * 2), f_to_bf16(bf16_to_f(hmid[e]) + round_bf16(run)));
  }
  signal(a, ctr_index(l, kPhRed));
  trace_mark(a, l * kPhases + kPhRed, kTrEnd);
  return true;
}

// ---------------------------------------------------------------------------
// LM head: final RMSNorm prologue, vocabulary rows 2u, 2u+1 per wave, logits
// in T then fp32, argmax partials of the workgroup -- k_proj<kLmHead>'s
// arithmetic (batched_decoder_step.py:405-408, CTRL:99-119).
// ---------------------------------------------------------------------------
__device__ __forceinline__ void ph_lmhead(const Lds& s) {
  const FusedArgs a = fargs();
  const Sched sc = make_sched(a);
  const int P = a.V / 2;  // vocabulary row pairs
  const int u0 = (int)((long long)blockIdx.x * P / sc.G), u1 = (int)((long long)(blockIdx.x + 1) * P / sc.G);
  const int tid = phase_tid(), lane = tid & 63, wave = wave_index(tid);
  float* wred = s.red + wave * (kRowsPerWave * kFMB);
  float best_v = 0.f;
  int best_i = -1;
  int bad = 0;
  trace_mark(a, a.L * kPhases, kTrStart);
  if (u0 < u1) {
    Vec8<FT> wv[kSegChunks][kRowsPerWave];
    auto issue = [&](int u) {
      const int uc = min(u, u1 - 1);
      const FT* wr[kRowsPerWave] = {a.lm_w + (size_t)(2 * uc) * a.H, a.lm_w + (size_t)(2 * uc + 1) * a.H};
      load_rows<FT, kRowsPerWave, true>(wv, wr, 0, a.H, lane);
    };
    int u = u0 + wave;
    const int mine = (u1 - u0 - wave + kFWaves - 1) / kFWaves;
    issue(u);
    __builtin_amdgcn_sched_barrier(0);
    const int z = wait_for(a, ctr_index(a.L - 1, kPhRed), sc.t_red, s);
    if (z < 0) return;
    trace_mark(a, a.L * kPhases, kTrReady);
    norm_prologue(a, layer_input(a, a.L) + z, a.final_norm, s, tid);
    for (int done = 0; u < u1; ++done) {
      progress_prio(done, mine);
      __builtin_amdgcn_sched_barrier(0);
      float acc[kRowsPerWave][kFMB];
#pragma unroll
      for (int r = 0; r < kRowsPerWave; ++r)
#pragma unroll
        for (int m = 0; m < kFMB; ++m) acc[r][m] = 0.f;
      dot_rows<FT, kFMB, kRowsPerWave, true>(wv, s.xs, a.H, 0, a.H, lane, acc);
      wave_totals<kFMB, kRowsPerWave>(acc, lane, wred);
      if (lane < a.B) {
        const int c0 = 2 * u, c1 = c0 + 1;
        const float l0 = round_bf16(wred[0 * kFMB + lane]);
        const float l1 = round_bf16(wred[1 * kFMB + lane]);
        a.logits[(size_t)lane * a.V + c0] = l0;
        a.logits[(size_t)lane * a.V + c1] = l1;
        if (!isfinite(l0) || !isfinite(l1)) bad = 1;
        if (best_i < 0 || l0 > best_v) {
          best_v = l0;
          best_i = c0;
        }
        if (l1 > best_v) {
          best_v = l1;
          best_i = c1;
        }
      }
      u += kFWaves;
      if (u < u1) issue(u);
    }
    __builtin_amdgcn_s_setprio(0);
  }
  // Combine the waves; ties go to the lowest index.  A workgroup without
  // vocabulary rows leaves index -1, which the merge ignores.
  __syncthreads();
  float* cv = s.red;
  int* ci = reinterpret_cast<int*>(s.red + kFWaves * kFMB);
  int* cb = ci + kFWaves * kFMB;
  if (lane < kFMB) {
    cv[wave * kFMB + lane] = best_v;
    ci[wave * kFMB + lane] = best_i;
    cb[wave * kFMB + lane] = bad;
  }
  __syncthreads();
  if (tid < a.B) {
    float bv = 0.f;
    int bi = -1, bb = 0;
    for (int wv = 0; wv < kFWaves; ++wv) {
      const int i = ci[wv * kFMB + tid];
      const float v = cv[wv * kFMB + tid];
      bb |= cb[wv * kFMB + tid];
      if (i < 0) continue;
      if (bi < 0 || v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
      }
    }
    const size_t o = (size_t)blockIdx.x * a.B + tid;
    a.am_val[o] = bv;
    a.am_idx[o] = bi;
    a.am_bad[o] = bb;
  }
  trace_mark(a, a.L * kPhases, kTrEnd);
}

__global__ void __launch_bounds__(kFThreads, 4) k_step_fused(FusedArgs args) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  if (args.done != nullptr && __builtin_nontemporal_load(args.done) != 0) return;
  const size_t xs_bytes = (size_t)kFMB * kSeg * sizeof(FT);
  Lds s;
  s.xs = reinterpret_cast<FT*>(smem_raw);
  s.attn = smem_raw;
  s.red = reinterpret_cast<float*>(smem_raw + xs_bytes);
  s.bcast = reinterpret_cast<int*>(s.red + kRedFloats);
  for (int l = 0; l < args.L; ++l) {
    // The dependency chain runs at a raised wave priority, so the streaming
    // waves sharing its SIMDs do not delay it.
    __builtin_amdgcn_s_setprio(2);
    if (!ph_qkv(l, s)) return;
    if (!ph_attn(l, s)) return;
    if (!ph_oproj(l, s)) return;
    __builtin_amdgcn_s_setprio(0);
    if (!ph_gateup(l, s)) return;
    if (!ph_down(l, s)) return;
    __builtin_amdgcn_s_setprio(2);
    if (!ph_reduce(l, s)) return;
    __builtin_amdgcn_s_setprio(0);
  }
  ph_lmhead(s);
}

// Embedding gather and the step's RoPE table (k_embed's arithmetic) plus the
// reset of the persistent kernel's counters; one workgroup per batch row.
struct EmbedSyncArgs {
  const int32_t* done;
  const int64_t* token;
  const FT* embedding;
  FT* hidden;
  const int64_t* pos;
  const float* inv_freq;
  float* rope;
  int32_t* sync;
  int sync_ints;
  int B, H, V, half;
};

__global__ void __launch_bounds__(256) k_embed_sync(EmbedSyncArgs a) {
  if (a.done != nullptr && __builtin_nontemporal_load(a.done) != 0) return;
  const int b = blockIdx.x, tid = threadIdx.x;
  for (int i = b * blockDim.x + tid; i < a.sync_ints; i += gridDim.x * blockDim.x) a.sync[i] = 0;
  if (a.token == nullptr) return;  // counter reset only
  long long t = a.token[b];
  if (t < 0 || t >= a.V) t = 0;  // the controller rejects such ids (CTRL:356); reads stay in bounds
  for (int j = tid; j < a.half; j += blockDim.x) {
    const float ang = static_cast<float>(a.pos[b]) * a.inv_freq[j];
    a.rope[((size_t)b * a.half + j) * 2] = round_bf16(cosf(ang));
    a.rope[((size_t)b * a.half + j) * 2 + 1] = round_bf16(sinf(ang));
  }
  const FT* src = a.embedding + (size_t)t * a.H;
  FT* dst = a.hidden + (size_t)b * a.H;
  for (int c = tid; c < a.H / 8; c += blockDim.x)
    *reinterpret_cast<Vec8<FT>*>(dst + c * 8) = Vec8<FT>::load_cached(src + c * 8);
}

size_t fused_lds_bytes_impl(const Dims& d) {
  const size_t xs = (size_t)kFMB * kSeg * sizeof(FT);
  const size_t attn = attention_lds_bytes(d);
  return std::max(xs, (attn + 15) / 16 * 16) + kRedFloats * sizeof(float) + 16;
}

}  // namespace

bool fused_step_eligible(const Dims& d) {
  return d.dtype_bytes == 2 && d.batch >= 1 && d.batch <= kFMB && d.hidden == kSeg && d.q_dim() == kSeg &&
         d.head_dim == kFHeadDim && d.vocab % 2 == 0 && d.intermediate % 8 == 0 &&
         attention_lds_bytes(d) <= (size_t)kFMB * kSeg * sizeof(FT) &&
         (long long)d.slots() * d.kv_dim() * 2 < (1LL << 31) && (long long)d.batch * d.intermediate * 2 < (1LL << 31);
}

size_t fused_lds_bytes(const Dims& d) { return fused_lds_bytes_impl(d); }

FusedActLayout fused_act_layout(const Dims& d) {
  auto up = [](size_t v) { return (v + 255) / 256 * 256; };
  FusedActLayout al{};
  const size_t T = sizeof(FT);
  al.q = 0;
  al.attn = al.q + up((size_t)d.batch * d.q_dim() * T);
  al.mlp = al.attn + up((size_t)d.batch * d.q_dim() * T);
  al.h_mid = al.mlp + up((size_t)d.batch * d.intermediate * T);
  al.h_out = al.h_mid + up((size_t)d.batch * d.hidden * T);
  al.part = al.h_out + up((size_t)d.batch * d.hidden * T);
  const size_t segs = (d.intermediate + kSeg - 1) / kSeg;
  al.stride = al.part + up(segs * d.batch * d.hidden * sizeof(float));
  return al;
}
size_t fused_act_bytes(const Dims& d) { return fused_act_layout(d).stride * d.layers; }
size_t fused_layer_table_bytes(const Dims& d) { return (size_t)d.layers * sizeof(FusedLayerW); }
// Phase counters, one 128-byte line each.
int fused_sync_ints(const Dims& d) { return (1 + d.layers * kPhases) * kCtrStride; }
size_t fused_trace_bytes(const Dims& d, int grid) {
  return (size_t)grid * (d.layers * kPhases + 1) * 3 * sizeof(unsigned long long);
}

int fused_grid_capacity(const Dims& d, int cus) {
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_step_fused, kFThreads, fused_lds_bytes_impl(d)) !=
          hipSuccess ||
      per_cu < 1)
    return 0;
  return per_cu * cus;
}

// Default grid: two workgroups per CU.  The waves of a CU's later-dispatched
// workgroups are served after the earlier ones', so with equal static shares
// the third and fourth workgroup of a CU finish a streaming phase 20-50%
// later than the first two; two per CU streamed the 28-layer Qwen2.5-7B step
// in 4.76 ms against 5.24 ms at three and 5.78 ms at four.
int fused_grid(const Dims& d, int cus) { return std::min(2 * cus, fused_grid_capacity(d, cus)); }

// A grid the kernel can run with: every workgroup resident at once.
bool fused_grid_valid(const Dims& d, int grid, int cus) {
  return grid >= 1 && grid <= fused_grid_capacity(d, cus);
}

hipError_t write_fused_layer_table(const Dims& d, const uint8_t* weights, const LayerOffsets* lo, void* dst) {
  std::vector<FusedLayerW> t(d.layers);
  for (int l = 0; l < d.layers; ++l) {
    t[l].in_norm = reinterpret_cast<const FT*>(weights + lo[l].input_norm);
    t[l].post_norm = reinterpret_cast<const FT*>(weights + lo[l].post_norm);
    t[l].qkv_w = reinterpret_cast<const FT*>(weights + lo[l].qkv_w);
    t[l].qkv_b = reinterpret_cast<const FT*>(weights + lo[l].qkv_b);
    t[l].o_w = reinterpret_cast<const FT*>(weights + lo[l].o_w);
    t[l].gate_w = reinterpret_cast<const FT*>(weights + lo[l].gate_w);
    t[l].up_w = reinterpret_cast<const FT*>(weights + lo[l].up_w);
    t[l].down_w = reinterpret_cast<const FT*>(weights + lo[l].down_w);
  }
  return hipMemcpy(dst, t.data(), t.size() * sizeof(FusedLayerW), hipMemcpyHostToDevice);
}

// ops: 0 = embedding + counter reset, 1 = the persistent step kernel.
hipError_t launch_fused_ops(const KernelEnv& env, const StepPtrs& st, hipStream_t stream, int begin, int end) {
  const Dims& d = env.dims;
  const Scratch& scr = env.scratch;
  if (begin < end && end > 0 && begin <= 1) {
    // Op 0 (embedding + counter reset); a range that starts at the kernel
    // itself still gets its counters reset.
    EmbedSyncArgs e{};
    e.done = st.done;
    e.token = st.token;
    e.embedding = reinterpret_cast<const FT*>(env.weights + env.embedding_off);
    e.hidden = static_cast<FT*>(scr.hidden);
    e.pos = st.pos;
    e.inv_freq = scr.inv_freq;
    e.rope = scr.rope;
    e.sync = scr.sync;
    e.sync_ints = fused_sync_ints(d);
    e.B = d.batch;
    e.H = d.hidden;
    e.V = d.vocab;
    e.half = d.head_dim / 2;
    if (begin == 1) e.token = nullptr;
    k_embed_sync<<<d.batch, 256, 0, stream>>>(e);
  }
  if (begin <= 1 && end > 1) {
    FusedArgs a{};
    a.done = st.done;
    a.lw = static_cast<const FusedLayerW*>(scr.fused_layers);
    a.final_norm = reinterpret_cast<const FT*>(env.weights + env.final_norm_off);
    a.lm_w = reinterpret_cast<const FT*>(env.weights + env.lm_head_off);
    a.hidden = static_cast<const FT*>(scr.hidden);
    const FusedActLayout al = fused_act_layout(d);
    a.act = static_cast<uint8_t*>(scr.fused_act);
    a.act_stride = static_cast<long long>(al.stride);
    a.off_q = static_cast<int>(al.q);
    a.off_attn = static_cast<int>(al.attn);
    a.off_mlp = static_cast<int>(al.mlp);
    a.off_hmid = static_cast<int>(al.h_mid);
    a.off_hout = static_cast<int>(al.h_out);
    a.off_part = static_cast<int>(al.part);
    a.rope = scr.rope;
    a.slot = st.slot;
    a.active = st.active;
    a.len = st.len;
    a.table = st.table;
    a.key_cache = static_cast<FT*>(st.key_cache);
    a.value_cache = static_cast<FT*>(st.value_cache);
    a.layer_elems = (long long)d.slots() * d.kv_dim();
    a.logits = st.logits;
    a.am_val = scr.am_val;
    a.am_idx = scr.am_idx;
    a.am_bad = scr.am_bad;
    a.sync = scr.sync;
    a.trace = scr.step_trace;
    a.slots = d.slots();
    a.timeout_ticks = 20000000LL;  // 200 ms of the 100 MHz wall clock; a step takes ~2 ms
    a.B = d.batch;
    a.H = d.hidden;
    a.heads = d.heads;
    a.kv_heads = d.kv_heads;
    a.head_dim = d.head_dim;
    a.I = d.intermediate;
    a.V = d.vocab;
    a.L = d.layers;
    a.block_size = d.block_size;
    a.blocks_per_row = d.blocks_per_row;
    a.window = d.capacity;
    a.eps = d.rms_eps;
    k_step_fused<<<env.plan.fused_grid, kFThreads, fused_lds_bytes_impl(d), stream>>>(a);
  }
  return hipGetLastError();
}

}  // namespace re
