// Decode projections of the resident epoch on the matrix cores (gfx950), for
// 64 batch rows (the scaled-batch configuration): Y[B, N] = X[B, K] W[N, K]^T
// with v_mfma_f32_16x16x32_bf16, the weights streamed from HBM once per step.
//
// Work layout.  Weights stream as 16-row column strips: lane l holds row
// l % 16 of the strip and elements 8 (l / 16) ..+8 of each 32-wide k step (a
// 64-byte run per row per load instruction; the packed copy makes a wave's
// step one 1 KB run), against the matching activation fragments of the four
// 16-row batch tiles, staged once per CU in LDS.  Weights are requested kRing
// (or more) steps ahead with every wait count known at compile time.
//   LM head, gate/up  one workgroup per CU, each wave a strip (two for
//                     gate/up) over the whole K (k_mf_lm_cu, k_mf_gu_cu);
//   o, down, qkv      split over (strip group, K range): each wave one strip
//                     over one of 8 K ranges, fp32 partials added in range
//                     order by the next launch (k_mf_part_cu; the next
//                     RMSNorm for o and down, k_mf_qkv_finish for qkv) -- a
//                     fixed order, so results do not depend on timing.
// The epilogues apply the same operations and roundings as the four-row
// kernels of re_step.hip:
//   qkv     + bias, RoPE of q and k (the partner element j + d/2 sits in lane
//           l ^ 8: a strip holds 8 pairs), q out, k and v to the paged slots
//   gate/up silu(gate) * up
//   resid   h + T(y) for the o and down projections
//   LM head logits (T(y) as fp32) and per-workgroup argmax partials
// MFMA result layout: value v of lane l is row 4 (l / 16) + v of the tile,
// column l % 16.
//
// The RMSNorm before qkv, gate/up and the LM head runs as its own kernel
// (one workgroup per row) into a normalized copy of the rows.
#include <type_traits>

#include "re_device.h"
#include "re_layout.h"

namespace re {
namespace {

typedef __bf16 mf_bf16x8 __attribute__((ext_vector_type(8)));
typedef float mf_f32x4 __attribute__((ext_vector_type(4)));

constexpr int kMfRows = 64;   // batch rows of the configuration
constexpr int kMfTiles = kMfRows / 16;
constexpr int kMfK = 32;      // k per MFMA step
constexpr int kRing = 8;      // weight steps in flight per wave
// Qwen2.5-7B's shape, the one these instantiations are compiled for
constexpr int kMfHidden = 3584;
constexpr int kMfInter = 18944;

struct MfArgs {
  const int32_t* done;
  const bf16_t* x;   // [B, K]
  const bf16_t* p0;  // packed weights (gate/up: gate)
  const bf16_t* p1;  // gate/up: packed up weights
  const bf16_t* w1;  // qkv: bias [rows]
  int B, K;
  // qkv
  bf16_t* q;
  bf16_t* key_cache;
  bf16_t* value_cache;
  const float* rope;
  const int32_t* slot;
  const int32_t* active;
  long long slots;
  int heads, kv_heads, head_dim;
  // gate/up output, residual stream
  bf16_t* out;
  bf16_t* hidden;
  int hidden_dim;
  // partial sums of the split launches: [gridDim.y][B][N] fp32, N = hidden_dim
  float* part;
  // LM head
  float* logits;
  float* am_val;
  int32_t* am_idx;
  int32_t* am_bad;
  int vocab;
};

// Row of column c (0..15) of qkv strip g: head g / (d / 16), pairs 8 t ..+8 of
// that head; columns 0..7 are elements j of the pairs, columns 8..15 their
// partners j + d/2.
__device__ __forceinline__ int qkv_strip_row(int head_dim, int g, int c) {
  const int half = head_dim >> 1, per_head = half >> 3;
  const int head = g / per_head, t = g - head * per_head;
  return head * head_dim + 8 * t + (c & 7) + (c >= 8 ? half : 0);
}

// Packed activations: xpack_index (re_device.h).

// LM head with one workgroup per CU.  Workgroups of a few waves would each
// fetch the whole 64 x K activation block (with 4-wave workgroups, 0.7 GB per
// step on top of the 1.09 GB of weights); here the 8 waves of a CU's one
// workgroup share one copy, staged through LDS in blocks of 16 k steps
// (64 KB, two buffers, filled by global -> LDS loads).  Workgroup g owns
// strips [g T / G, (g + 1) T / G) of the T = V / 16 column strips; wave w
// owns strips w, w + 8, ... of that range (NS = 4 or 5 of them) over the whole
// K, with kLcRing k steps of weights in flight.  Per step a wave reads the
// four batch tiles' fragments from LDS and runs NS x 4 products, every logit
// one chain of MFMA steps in k order; the argmax partial of (workgroup, row) is the first
// index of the maximum over the workgroup's columns (CTRL:99-119), combined
// over the waves in wave order, stored row-major ([row][G]).
constexpr int kLcWaves = 8;
constexpr int kLcBlock = 16;   // k steps per LDS activation block
constexpr int kLcRing = 4;     // weight steps in flight per wave
constexpr int kLcMaxNs = 5;    // strips per wave at most
constexpr int kLcBlockBytes = kMfTiles * kLcBlock * 1024;
constexpr size_t kLcLds = 2 * (size_t)kLcBlockBytes + (size_t)kLcWaves * kMfRows * 12;

typedef const __attribute__((address_space(1))) void* lc_gptr;
typedef __attribute__((address_space(3))) void* lc_lptr;

// s_waitcnt immediate: vmcnt <= vm, lgkmcnt 0, expcnt untouched.
constexpr int lc_wait(int vm) { return (vm & 15) | ((vm >> 4) << 14) | (7 << 4); }

// The K loop of a per-CU workgroup: the activations pass through LDS in
// blocks of kLcBlock steps (every wave issues its eighth of each block's
// global -> LDS loads), and this wave streams NS weight strips (wp: step 0 of
// each, packed) with RING steps in flight, accumulating acc[j][t] over the
// whole K in step order.  NS = 0: a wave with no strip only loads and joins
// the barriers (every wave runs the same 1 + K / (32 kLcBlock) barriers).
template <int NS, int RING>
__device__ __forceinline__ void cu_stream(const MfArgs& a, unsigned char* lds, const bf16_t* const* wp, int lane,
                                          int wave, mf_f32x4 (*acc)[kMfTiles]) {
  constexpr int NA = NS > 0 ? NS : 1;
  static_assert(RING * NS + 8 <= 63, "vmcnt holds at most 63");
  static_assert(kLcBlock % RING == 0, "ring slots are compile-time within a block");
  const int ksteps = a.K / kMfK, nblocks = ksteps / kLcBlock;
  // activation block b, tile t, steps 8 (w & 1) ..+8 go to LDS by wave w's 8
  // loads (load i: step s0 + i)
  auto issue_x1 = [&](int b, int i) {
    const int t = wave >> 1, s0 = (wave & 1) * 8;
    const bf16_t* src = a.x + ((size_t)t * ksteps + b * kLcBlock + s0 + i) * 512 + lane * 8;
    unsigned char* dst = lds + (b & 1) * kLcBlockBytes + (t * kLcBlock + s0 + i) * 1024;
    __builtin_amdgcn_global_load_lds((lc_gptr)src, (lc_lptr)dst, 16, 0, 0);
  };
  auto issue_x = [&](int b) {
#pragma unroll
    for (int i = 0; i < 8; ++i) issue_x1(b, i);
  };
  if constexpr (NS > 0) {
#pragma unroll
    for (int j = 0; j < NS; ++j)
#pragma unroll
      for (int t = 0; t < kMfTiles; ++t) acc[j][t] = mf_f32x4{0.f, 0.f, 0.f, 0.f};
  }
  re_u32x4 wr[RING][NA];
  issue_x(0);
  if constexpr (NS > 0) {
#pragma unroll
    for (int s = 0; s < RING; ++s)
#pragma unroll
      for (int j = 0; j < NS; ++j) wr[s][j] = __builtin_nontemporal_load(reinterpret_cast<const re_u32x4*>(wp[j] + s * 512));
  }
  // Block b + 1 goes to LDS during block b (its buffer was freed by the
  // barrier that ended block b - 1).  SPREAD (a ring no deeper than the
  // block's last 8 steps): one load per step over the block's first 8
  // steps, so no wave stalls on a burst of eight requests, and at least RING
  // steps of refills follow the last one, so the block-end wait (all but the
  // last RING * NS loads) covers it; a wave without strips issues them at
  // the block's start.  Otherwise (a deeper ring, whose block-end wait
  // leaves loads of the whole block in flight): block b + 2 in one burst
  // after the barrier that ends block b.
  constexpr bool SPREAD = RING <= kLcBlock - 8;
  if constexpr (!SPREAD) issue_x(1);
  // block 0 in LDS (the ring, and block 1 without SPREAD, may still be in flight)
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(lc_wait(RING * NS + (SPREAD ? 0 : 8)));
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  for (int b = 0; b < nblocks; ++b) {
    if constexpr (SPREAD && NS == 0) {
      if (b + 1 < nblocks) issue_x(b + 1);
    }
    if constexpr (NS > 0) {
      const unsigned char* xb = lds + (b & 1) * kLcBlockBytes + lane * 16;
#pragma unroll
      for (int s = 0; s < kLcBlock; ++s) {
        const int S = b * kLcBlock + s, rw = S % RING;
        mf_bf16x8 xf[kMfTiles];
#pragma unroll
        for (int t = 0; t < kMfTiles; ++t) xf[t] = *reinterpret_cast<const mf_bf16x8*>(xb + (t * kLcBlock + s) * 1024);
#pragma unroll
        for (int j = 0; j < NS; ++j)
#pragma unroll
          for (int t = 0; t < kMfTiles; ++t)
            acc[j][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xf[t], __builtin_bit_cast(mf_bf16x8, wr[rw][j]), acc[j][t], 0, 0, 0);
        // the refill past the last step re-reads the last one (unconditional,
        // so every wait counts exactly these loads)
        const int nxt = min(S + RING, ksteps - 1);
#pragma unroll
        for (int j = 0; j < NS; ++j) wr[rw][j] = __builtin_nontemporal_load(reinterpret_cast<const re_u32x4*>(wp[j] + nxt * 512));
        if (SPREAD && s < 8 && b + 1 < nblocks) issue_x1(b + 1, s);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    // Every wave is done with buffer b & 1, and block b + 1 has landed: only
    // the ring may still be in flight.
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(lc_wait(RING * NS));
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (!SPREAD && b + 2 < nblocks) issue_x(b + 2);
  }
  __builtin_amdgcn_s_waitcnt(lc_wait(0));
}

template <int NS>
__device__ __forceinline__ void lm_cu_body(const MfArgs& a, unsigned char* lds, int s_begin, int lane, int wave,
                                           float* cval, int* cidx, int* cbad) {
  const int ksteps = a.K / kMfK;
  const bf16_t* wp[NS];
#pragma unroll
  for (int j = 0; j < NS; ++j) wp[j] = a.p0 + (size_t)(s_begin + wave + kLcWaves * j) * ksteps * 512 + lane * 8;
  mf_f32x4 acc[NS][kMfTiles];
  cu_stream<NS, kLcRing>(a, lds, wp, lane, wave, acc);
  // Logits T(y) as fp32 (batched_decoder_step.py:405-408) and this wave's
  // first maximum per row over its strips.
  const int c = lane & 15, mrow = 4 * (lane >> 4);
#pragma unroll
  for (int t = 0; t < kMfTiles; ++t)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int m = t * 16 + mrow + v;
      float bv = 0.f;
      int bi = -1, bad = 0;
#pragma unroll
      for (int j = 0; j < NS; ++j) {
        const int n = (s_begin + wave + kLcWaves * j) * 16 + c;
        const float l = Elt<bf16_t>::r(acc[j][t][v]);
        if (m < a.B) a.logits[(size_t)m * a.vocab + n] = l;
        bad |= isfinite(l) ? 0 : 1;
        if (bi < 0 || l > bv) {  // strips in increasing order: ties keep the earlier
          bv = l;
          bi = n;
        }
      }
#pragma unroll
      for (int x = 1; x < 16; x <<= 1) {
        const float ov = __shfl_xor(bv, x, 64);
        const int oi = __shfl_xor(bi, x, 64);
        bad |= __shfl_xor(bad, x, 64);
        if (ov > bv || (ov == bv && oi < bi)) {
          bv = ov;
          bi = oi;
        }
      }
      if (c == 0) {
        cval[wave * kMfRows + m] = bv;
        cidx[wave * kMfRows + m] = bi;
        cbad[wave * kMfRows + m] = bad;
      }
    }
}

__global__ void __launch_bounds__(kLcWaves * 64, 1) k_mf_lm_cu(MfArgs a) {
  extern __shared__ __align__(16) unsigned char lc_smem[];
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_index(tid);
  const int32_t stop = a.done != nullptr ? request_flag(a.done) : 0;
  if (flag_set(stop)) return;  // uniform
  const int G = gridDim.x, g = blockIdx.x, T = a.vocab / 16;
  const int s_begin = (int)((long long)g * T / G), s_end = (int)((long long)(g + 1) * T / G);
  const int ns = (s_end - s_begin - wave + kLcWaves - 1) / kLcWaves;  // strips of this wave
  float* cval = reinterpret_cast<float*>(lc_smem + 2 * (size_t)kLcBlockBytes);
  int* cidx = reinterpret_cast<int*>(cval + kLcWaves * kMfRows);
  int* cbad = cidx + kLcWaves * kMfRows;
  // every wave runs the same barriers whatever its strip count
  switch (ns) {
    case 5: lm_cu_body<5>(a, lc_smem, s_begin, lane, wave, cval, cidx, cbad); break;
    case 4: lm_cu_body<4>(a, lc_smem, s_begin, lane, wave, cval, cidx, cbad); break;
    case 3: lm_cu_body<3>(a, lc_smem, s_begin, lane, wave, cval, cidx, cbad); break;
    case 2: lm_cu_body<2>(a, lc_smem, s_begin, lane, wave, cval, cidx, cbad); break;
    default: lm_cu_body<1>(a, lc_smem, s_begin, lane, wave, cval, cidx, cbad); break;  // ns >= 1 (launch check)
  }
  __syncthreads();
  if (tid < a.B) {
    float bv = 0.f;
    int bi = -1, bb = 0;
    for (int w = 0; w < kLcWaves; ++w) {
      const float v = cval[w * kMfRows + tid];
      const int i = cidx[w * kMfRows + tid];
      bb |= cbad[w * kMfRows + tid];
      if (i >= 0 && (bi < 0 || v > bv || (v == bv && i < bi))) {
        bv = v;
        bi = i;
      }
    }
    // row-major partials: a row's G partials are contiguous for the controller
    a.am_val[(size_t)tid * G + g] = bv;
    a.am_idx[(size_t)tid * G + g] = bi;
    a.am_bad[(size_t)tid * G + g] = bb;
  }
}

// gate/up with one workgroup per CU (64 rows): the I / 16 column strips are
// split over the CUs (4-5 each for Qwen2.5-7B), wave w < that count streams
// strip s_begin + w of the gate and of the up matrix over the whole K,
// sharing the LDS-staged activations with the other waves, then the SiLU *
// up epilogue.
constexpr int kGcRing = 8;  // weight steps in flight per wave (few waves stream)

__global__ void __launch_bounds__(kLcWaves * 64, 1) k_mf_gu_cu(MfArgs a) {
  extern __shared__ __align__(16) unsigned char lc_smem[];
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_index(tid);
  const int32_t stop = a.done != nullptr ? request_flag(a.done) : 0;
  if (flag_set(stop)) return;  // uniform
  const int G = gridDim.x, g = blockIdx.x, T = a.hidden_dim / 16;  // hidden_dim: I
  const int s_begin = (int)((long long)g * T / G), s_end = (int)((long long)(g + 1) * T / G);
  const int u = s_begin + wave;
  if (u >= s_end) {
    cu_stream<0, kGcRing>(a, lc_smem, nullptr, lane, wave, nullptr);
    return;
  }
  const int ksteps = a.K / kMfK;
  const bf16_t* wp[2] = {a.p0 + (size_t)u * ksteps * 512 + lane * 8, a.p1 + (size_t)u * ksteps * 512 + lane * 8};
  mf_f32x4 acc[2][kMfTiles];
  cu_stream<2, kGcRing>(a, lc_smem, wp, lane, wave, acc);
  const int c = lane & 15, mrow = 4 * (lane >> 4), n = u * 16 + c;
#pragma unroll
  for (int t = 0; t < kMfTiles; ++t)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int m = t * 16 + mrow + v;
      if (m >= a.B) continue;
      // silu(gate) * up, each result rounded (batched_decoder_step.py:391-398)
      const float gt = Elt<bf16_t>::r(acc[0][t][v]);
      const float up = Elt<bf16_t>::r(acc[1][t][v]);
      const float sg = Elt<bf16_t>::r(gt / (1.0f + expf(-gt)));
      a.out[xpack_index(m, n, a.hidden_dim)] = Elt<bf16_t>::t(Elt<bf16_t>::r(sg * up));
    }
}

// o, down and qkv split over (strip group, K range) with the range's
// activations staged in LDS: workgroup (x, y) runs strips x * WAVES + wave
// over the y-th of 8 K ranges, one strip per wave.  The waves copy the
// range's activation fragments (4 tiles x 1 KB per k step) to LDS together
// (global -> LDS, one 1 KB fragment per instruction), in blocks of BLK steps
// through two buffers, and each wave reads them from LDS while it streams its
// strip's weights with kRing steps in flight.  Every count is known at
// compile time, so each wait is exact.  A CU fetches one K range of the
// activations instead of all of them.  QKV: the partial of column c of strip g goes
// to qkv row qkv_strip_row(g, c) (N = the qkv rows, k_mf_qkv_finish adds
// them up); otherwise to column 16 g + c (N = hidden, the next norm adds them).
template <int STEPS, int BLK>
constexpr int part_block_steps(int b) {
  return STEPS - b * BLK < BLK ? STEPS - b * BLK : BLK;
}
template <int STEPS, int BLK, int WAVES>
constexpr int part_block_copies(int b) {  // per wave
  return (kMfTiles * part_block_steps<STEPS, BLK>(b) + WAVES - 1) / WAVES;
}
template <int STEPS, int BLK>
constexpr int part_block_refills(int b) {  // weight loads issued during block b
  int n = 0;
  for (int s = b * BLK; s < b * BLK + part_block_steps<STEPS, BLK>(b); ++s) n += s + kRing < STEPS ? 1 : 0;
  return n;
}
template <int STEPS, int BLK>
constexpr size_t part_cu_lds() {
  return (size_t)(STEPS > BLK ? 2 : 1) * kMfTiles * BLK * 1024;
}

template <int STEPS, int WAVES, int BLK, bool QKV>
__global__ void __launch_bounds__(WAVES * 64) k_mf_part_cu(MfArgs a) {
  extern __shared__ __align__(16) unsigned char pc_smem[];  // [2][kMfTiles][BLK] fragments of 1 KB
  constexpr int NB = (STEPS + BLK - 1) / BLK;
  constexpr int R = kRing < STEPS ? kRing : STEPS;
  constexpr int kBuf = kMfTiles * BLK * 1024;
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_index(tid);
  const int c = lane & 15;
  const int g = blockIdx.x * WAVES + wave;  // this wave's strip
  const int kstep0 = blockIdx.y * STEPS;
  const int ksteps = a.K / kMfK;
  const int32_t stop = a.done != nullptr ? request_flag(a.done) : 0;
  if (flag_set(stop)) return;  // uniform
  // block b's fragment f = t * steps + s (tile t, step s of the block) by
  // wave f % WAVES; a wave past the end copies the last one again
  auto stage = [&](auto bc) {
    constexpr int b = decltype(bc)::value;
    constexpr int ns = part_block_steps<STEPS, BLK>(b);
    constexpr int nf = kMfTiles * ns;
    unsigned char* dst = pc_smem + (b & 1) * kBuf;
#pragma unroll
    for (int i = 0; i < part_block_copies<STEPS, BLK, WAVES>(b); ++i) {
      const int f = min(wave + i * WAVES, nf - 1);
      const int t = f / ns, sl = f - t * ns;
      __builtin_amdgcn_global_load_lds((lc_gptr)(a.x + ((size_t)t * ksteps + kstep0 + b * BLK + sl) * 512 + lane * 8),
                                       (lc_lptr)(dst + (t * BLK + sl) * 1024), 16, 0, 0);
    }
  };
  const bf16_t* wp = a.p0 + ((size_t)g * ksteps + kstep0) * 512 + lane * 8;
  re_u32x4 wr[R];
  stage(std::integral_constant<int, 0>{});
#pragma unroll
  for (int s = 0; s < R; ++s) wr[s] = __builtin_nontemporal_load(reinterpret_cast<const re_u32x4*>(wp + s * 512));
  int pending = R;  // loads issued after the block now awaited (compile-time after unrolling)
  if constexpr (NB > 1) {
    stage(std::integral_constant<int, 1>{});
    pending += part_block_copies<STEPS, BLK, WAVES>(1);
  }
  // block 0 is in LDS: this wave's copies first, then everyone's
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(lc_wait(R + (NB > 1 ? part_block_copies<STEPS, BLK, WAVES>(1) : 0)));
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  (void)pending;
  mf_f32x4 acc[kMfTiles];
#pragma unroll
  for (int t = 0; t < kMfTiles; ++t) acc[t] = mf_f32x4{0.f, 0.f, 0.f, 0.f};
  auto block = [&](auto bc) {
    constexpr int b = decltype(bc)::value;
    constexpr int ns = part_block_steps<STEPS, BLK>(b);
    const unsigned char* xb = pc_smem + (b & 1) * kBuf + lane * 16;
#pragma unroll
    for (int sl = 0; sl < ns; ++sl) {
      const int s = b * BLK + sl;
      mf_bf16x8 xf[kMfTiles];
#pragma unroll
      for (int t = 0; t < kMfTiles; ++t) xf[t] = *reinterpret_cast<const mf_bf16x8*>(xb + (t * BLK + sl) * 1024);
#pragma unroll
      for (int t = 0; t < kMfTiles; ++t)
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xf[t], __builtin_bit_cast(mf_bf16x8, wr[s % R]), acc[t], 0, 0, 0);
      if (s + R < STEPS) wr[s % R] = __builtin_nontemporal_load(reinterpret_cast<const re_u32x4*>(wp + (s + R) * 512));
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (b + 1 < NB) {
      // block b + 1 landed (only this block's refills may still be in flight),
      // and every wave is done with buffer b & 1; then block b + 2 goes there
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_waitcnt(lc_wait(part_block_refills<STEPS, BLK>(b)));
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      if constexpr (b + 2 < NB) stage(std::integral_constant<int, b + 2>{});
    }
  };
  static_assert(NB <= 6, "at most six staged blocks");
  block(std::integral_constant<int, 0>{});
  if constexpr (NB > 1) block(std::integral_constant<int, 1>{});
  if constexpr (NB > 2) block(std::integral_constant<int, 2>{});
  if constexpr (NB > 3) block(std::integral_constant<int, 3>{});
  if constexpr (NB > 4) block(std::integral_constant<int, 4>{});
  if constexpr (NB > 5) block(std::integral_constant<int, 5>{});
  const int mrow = 4 * (lane >> 4);
  const int n = QKV ? qkv_strip_row(a.head_dim, g, c) : g * 16 + c;
  float* part = a.part + (size_t)blockIdx.y * a.B * a.hidden_dim;
#pragma unroll
  for (int t = 0; t < kMfTiles; ++t)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int m = t * 16 + mrow + v;
      if (m < a.B) part[(size_t)m * a.hidden_dim + n] = acc[t][v];
    }
}

// The qkv epilogue after k_mf_part_cu: the 8 K-range partials added in range
// order, then bias, RoPE and the q / paged K/V writes (the four-row qkv
// epilogue's roundings).
// Thread: one (row, head, pair j < d/2), both elements of the RoPE pair.
template <int RANGES>
__global__ void __launch_bounds__(256) k_mf_qkv_finish(MfArgs a) {
  const int half = a.head_dim >> 1;
  const int nheads = a.hidden_dim / a.head_dim;  // q, k and v heads
  const int idx = blockIdx.x * 256 + threadIdx.x;
  if (idx >= a.B * nheads * half) return;
  const int32_t stop = a.done != nullptr ? request_flag(a.done) : 0;
  if (flag_set(stop)) return;
  const int m = idx / (nheads * half), rem = idx - m * nheads * half;
  const int head = rem / half, j = rem - head * half;
  const int r0 = head * a.head_dim + j, r1 = r0 + half;
  const size_t plane = (size_t)a.B * a.hidden_dim;
  const float* p = a.part + (size_t)m * a.hidden_dim;
  float v0[RANGES], v1[RANGES];  // every partial requested before the first add
#pragma unroll
  for (int r = 0; r < RANGES; ++r) {
    v0[r] = p[r * plane + r0];
    v1[r] = p[r * plane + r1];
  }
  float s0 = v0[0], s1 = v1[0];
#pragma unroll
  for (int r = 1; r < RANGES; ++r) {
    s0 += v0[r];
    s1 += v1[r];
  }
  // F.linear with bias: fp32 sum + bias, one rounding (g4a_linear_t_bias.py:18-21)
  const float y0 = Elt<bf16_t>::r(s0 + Elt<bf16_t>::f(a.w1[r0]));
  const float y1 = Elt<bf16_t>::r(s1 + Elt<bf16_t>::f(a.w1[r1]));
  float o0 = y0, o1 = y1;
  if (head < a.heads + a.kv_heads) {
    // q' = q*cos + rotate_half(q)*sin, each product and the sum rounded
    // (batched_decoder_step.py:231-240, 323-324)
    const float cs = a.rope[((size_t)m * half + j) * 2], sn = a.rope[((size_t)m * half + j) * 2 + 1];
    o0 = Elt<bf16_t>::r(Elt<bf16_t>::r(y0 * cs) + Elt<bf16_t>::r(-y1 * sn));
    o1 = Elt<bf16_t>::r(Elt<bf16_t>::r(y1 * cs) + Elt<bf16_t>::r(y0 * sn));
  }
  if (head < a.heads) {
    bf16_t* q = a.q + ((size_t)m * a.heads + head) * a.head_dim;
    q[j] = Elt<bf16_t>::t(o0);
    q[j + half] = Elt<bf16_t>::t(o1);
  } else {
    // paged slot write, active rows only (batched_decoder_step.py:250-264)
    const int sl = a.slot[m];
    if (a.active[m] != 0 && sl >= 0 && sl < a.slots) {
      const bool is_key = head < a.heads + a.kv_heads;
      const int kvh = is_key ? head - a.heads : head - a.heads - a.kv_heads;
      bf16_t* cache = (is_key ? a.key_cache : a.value_cache) + ((size_t)sl * a.kv_heads + kvh) * a.head_dim;
      cache[j] = Elt<bf16_t>::t(o0);
      cache[j + half] = Elt<bf16_t>::t(o1);
    }
  }
}

// RMSNorm of each row into a normalized copy, packed like the activations the
// projections read: T(T(h * rs) * w) with rs = rsqrt(mean(h^2) + eps) in fp32
// (batched_decoder_step.py:224-229).  Eight consecutive elements stay
// contiguous in the packed layout.
//
// With parts > 0 the residual add of the preceding split projection happens
// first: h = T(h + T(p_0 + p_1 + ... )) over its fp32 partials in range order
// (batched_decoder_step.py:380-386, 399-403), written back to the residual
// stream, then normalized.
template <int PARTS>
__global__ void __launch_bounds__(256) k_mf_norm(const int32_t* done, bf16_t* h, const bf16_t* w, bf16_t* y,
                                               int H, float eps, const float* part, int B) {
  __shared__ float red[4];
  if (done != nullptr && __builtin_nontemporal_load(done) != 0) return;
  const int m = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = wave_index(tid);
  bf16_t* hr = h + (size_t)m * H;
  constexpr int kMaxChunks = 4;  // H <= 4 * 256 * 8
  Vec8<bf16_t> hv[kMaxChunks];
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < kMaxChunks; ++i) {
    const int ch = tid + 256 * i;
    hv[i] = ch * 8 < H ? Vec8<bf16_t>::load_cached(hr + ch * 8) : Vec8<bf16_t>{};
    if (PARTS > 0 && ch * 8 < H) {
      // all PARTS partials requested at once, then added in order
      re_f32x4 pv[PARTS > 0 ? PARTS : 1][2];
      const float* p0 = part + (size_t)m * H + ch * 8;
#pragma unroll
      for (int r = 0; r < PARTS; ++r) {
        pv[r][0] = *reinterpret_cast<const re_f32x4*>(p0 + (size_t)r * B * H);
        pv[r][1] = *reinterpret_cast<const re_f32x4*>(p0 + (size_t)r * B * H + 4);
      }
      float sum[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) sum[e] = pv[0][e >> 2][e & 3];
#pragma unroll
      for (int r = 1; r < PARTS; ++r)
#pragma unroll
        for (int e = 0; e < 8; ++e) sum[e] += pv[r][e >> 2][e & 3];
      float nh[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) nh[e] = bf16_to_f(f_to_bf16(hv[i].get(e) + round_bf16(sum[e])));
      hv[i] = Vec8<bf16_t>::from_floats(nh);
      *reinterpret_cast<Vec8<bf16_t>*>(hr + ch * 8) = hv[i];
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) s = fmaf(hv[i].get(e), hv[i].get(e), s);
  }
  s = wave_sum(s);
  if (lane == 0) red[wave] = s;
  __syncthreads();
  const float rs = rsqrtf((red[0] + red[1] + red[2] + red[3]) / static_cast<float>(H) + eps);
#pragma unroll
  for (int i = 0; i < kMaxChunks; ++i) {
    const int ch = tid + 256 * i;
    if (ch * 8 >= H) continue;
    const Vec8<bf16_t> wv = Vec8<bf16_t>::load_cached(w + ch * 8);
    float out[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = round_bf16(round_bf16(hv[i].get(e) * rs) * wv.get(e));
    *reinterpret_cast<Vec8<bf16_t>*>(y + xpack_index(m, ch * 8, H)) = Vec8<bf16_t>::from_floats(out);
  }
}

// The packed copy of one [rows, K] matrix: 16-byte unit u = (strip * K/32 +
// step) * 64 + lane holds row strip * 16 + lane % 16 (qkv: qkv_strip_row), elements
// step * 32 + 8 (lane / 16) ..+8.
__global__ void k_mf_pack(const bf16_t* src, bf16_t* dst, int rows, int K, int qkv_head_dim) {
  const long long units = (long long)rows / 16 * (K / kMfK) * 64;
  for (long long u = (long long)blockIdx.x * blockDim.x + threadIdx.x; u < units;
       u += (long long)gridDim.x * blockDim.x) {
    const int lane = static_cast<int>(u & 63);
    const long long tile = u >> 6;
    const int steps = K / kMfK;
    const int strip = static_cast<int>(tile / steps), step = static_cast<int>(tile - (long long)strip * steps);
    const int c = lane & 15;
    const int row = qkv_head_dim > 0 ? qkv_strip_row(qkv_head_dim, strip, c) : strip * 16 + c;
    const re_u32x4 v = *reinterpret_cast<const re_u32x4*>(src + (size_t)row * K + step * kMfK + (lane >> 4) * 8);
    *reinterpret_cast<re_u32x4*>(dst + u * 8) = v;
  }
}

// The split launches: K in 8 ranges of kHidSteps(8) (hidden) or kInterSteps
// (intermediate) k steps; o / down run 7 strips (one per wave) per workgroup.
constexpr int kPartRanges = 8;
constexpr int kHidSteps(int ranges) { return kMfHidden / kMfK / ranges; }
constexpr int kInterSteps = kMfInter / kMfK / kPartRanges;
constexpr int kPartWaves = 7;
// the staged split kernels: o and qkv stage their 14-step K range at once,
// down its 74 steps in blocks of 16
constexpr int kQkvPartWaves = 9;  // qkv strips per workgroup: 288 = 32 x 9
constexpr int kDownBlk = 16;

}  // namespace

bool mfma_step_supported(const Dims& d) {
  return d.dtype_bytes == 2 && d.batch == kMfRows && d.hidden == kMfHidden && d.q_dim() == kMfHidden &&
         d.intermediate == kMfInter && d.head_dim % 16 == 0 && d.qkv_rows() % 16 == 0 &&
         d.vocab % 32 == 0 && d.hidden % 16 == 0;
}

int mfma_lm_partials(const Dims& d) { return d.vocab / 32; }

// gate/up per CU: 1 to 8 strips per workgroup and whole LDS blocks.
bool mfma_gu_cu_fits(const Dims& d, int cus) {
  const int strips = d.intermediate / 16;
  return mfma_step_supported(d) && cus > 0 && strips >= cus && strips <= kLcWaves * cus &&
         d.hidden % (kMfK * kLcBlock) == 0 && d.hidden / (kMfK * kLcBlock) >= 2;
}

bool mfma_split_fits(const Dims& d) { return mfma_step_supported(d) && (d.hidden / 16) % kPartWaves == 0; }
bool mfma_qkv_split_fits(const Dims& d) {
  return mfma_split_fits(d) && (d.qkv_rows() / 16) % kQkvPartWaves == 0 && d.q_dim() == d.hidden;
}
size_t mfma_split_partial_bytes(const Dims& d) {
  return (size_t)kPartRanges * d.batch * std::max(d.hidden, d.qkv_rows()) * sizeof(float);
}

// The per-CU LM head needs 8 to 40 strips per workgroup and whole LDS blocks.
bool mfma_lm_cu_fits(const Dims& d, int cus) {
  const int strips = d.vocab / 16;
  return mfma_step_supported(d) && cus > 0 && strips >= kLcWaves * cus && strips <= kLcWaves * kLcMaxNs * cus &&
         d.hidden % (kMfK * kLcBlock) == 0 && d.hidden / (kMfK * kLcBlock) >= 2 && cus <= mfma_lm_partials(d);
}

size_t mfma_packed_layout(const Dims& d, PackedOffsets* layers, size_t* lm_off) {
  size_t off = 0;
  auto add = [&](long long rows, long long k) {
    const size_t at = off;
    off += (size_t)rows * k * sizeof(bf16_t);
    off = (off + 255) & ~size_t(255);
    return at;
  };
  for (int l = 0; l < d.layers; ++l) {
    layers[l].qkv = add(d.qkv_rows(), d.hidden);
    layers[l].o = add(d.hidden, d.q_dim());
    layers[l].gate = add(d.intermediate, d.hidden);
    layers[l].up = add(d.intermediate, d.hidden);
    layers[l].down = add(d.hidden, d.intermediate);
  }
  *lm_off = add(d.vocab, d.hidden);
  return off;
}

hipError_t mfma_pack_matrix(const void* src, void* dst, int rows, int K, int qkv_head_dim, hipStream_t stream) {
  if (rows % 16 != 0 || K % kMfK != 0 || (qkv_head_dim > 0 && qkv_head_dim % 16 != 0)) return hipErrorInvalidValue;
  k_mf_pack<<<2048, 256, 0, stream>>>(static_cast<const bf16_t*>(src), static_cast<bf16_t*>(dst), rows, K,
                                      qkv_head_dim);
  return hipGetLastError();
}

template <int STEPS, int WAVES, int BLK, bool QKV>
static hipError_t part_cu_prepare() {
  return hipFuncSetAttribute(reinterpret_cast<const void*>(k_mf_part_cu<STEPS, WAVES, BLK, QKV>),
                             hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(part_cu_lds<STEPS, BLK>()));
}
template <int STEPS, int WAVES, int BLK, bool QKV>
static void part_cu_launch(const MfArgs& a, int groups, hipStream_t stream) {
  k_mf_part_cu<STEPS, WAVES, BLK, QKV><<<dim3(groups, kPartRanges), WAVES * 64, part_cu_lds<STEPS, BLK>(), stream>>>(a);
}

hipError_t prepare_mfma() {
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(k_mf_lm_cu), hipFuncAttributeMaxDynamicSharedMemorySize,
                                     static_cast<int>(kLcLds));
  if (e == hipSuccess)
    e = hipFuncSetAttribute(reinterpret_cast<const void*>(k_mf_gu_cu), hipFuncAttributeMaxDynamicSharedMemorySize,
                            static_cast<int>(kLcLds));
  if (e == hipSuccess) e = part_cu_prepare<kHidSteps(kPartRanges), kPartWaves, kHidSteps(kPartRanges), false>();
  if (e == hipSuccess) e = part_cu_prepare<kInterSteps, kPartWaves, kDownBlk, false>();
  if (e == hipSuccess) e = part_cu_prepare<kHidSteps(kPartRanges), kQkvPartWaves, kHidSteps(kPartRanges), true>();
  return e;
}

// The RMSNorm launch; with pending (o or down split) partials it adds them first.
static void mf_norm(const KernelEnv& env, const StepPtrs& st, size_t w_off, bool pending, hipStream_t stream) {
  const Dims& d = env.dims;
  const Scratch& sc = env.scratch;
  bf16_t* h = static_cast<bf16_t*>(sc.hidden);
  const bf16_t* w = reinterpret_cast<const bf16_t*>(env.weights + w_off);
  bf16_t* y = static_cast<bf16_t*>(sc.xn);
  if (pending)
    k_mf_norm<kPartRanges><<<d.batch, 256, 0, stream>>>(st.done, h, w, y, d.hidden, d.rms_eps, sc.mf_part, d.batch);
  else
    k_mf_norm<0><<<d.batch, 256, 0, stream>>>(st.done, h, w, y, d.hidden, d.rms_eps, nullptr, d.batch);
}

hipError_t launch_mfma_op(MfmaOp op, const KernelEnv& env, const StepPtrs& st, int layer, hipStream_t stream) {
  const Dims& d = env.dims;
  const Scratch& sc = env.scratch;
  MfArgs a{};
  a.done = st.done;
  a.B = d.batch;
  a.hidden_dim = d.hidden;
  auto wt = [&](size_t off) { return reinterpret_cast<const bf16_t*>(env.weights + off); };
  auto pk = [&](size_t off) { return reinterpret_cast<const bf16_t*>(env.packed + off); };
  if (op == MfmaOp::kLmHead) {
    // the last layer's down projection is still in partials
    mf_norm(env, st, env.final_norm_off, true, stream);
    a.x = static_cast<const bf16_t*>(sc.xn);
    a.p0 = pk(env.packed_lm_off);
    a.K = d.hidden;
    a.logits = st.logits;
    a.am_val = sc.am_val;
    a.am_idx = sc.am_idx;
    a.am_bad = sc.am_bad;
    a.vocab = d.vocab;
    // one workgroup per CU; its argmax partials go straight to k_ctrl_step
    k_mf_lm_cu<<<env.plan.argmax_parts, kLcWaves * 64, kLcLds, stream>>>(a);
    return hipGetLastError();
  }
  const LayerOffsets& lo = env.layer_off[layer];
  const PackedOffsets& po = env.packed_off[layer];
  const size_t cache_layer_elems = (size_t)d.slots() * d.kv_dim();
  switch (op) {
    case MfmaOp::kQkv: {
      // layer > 0: the previous layer's down projection is still in partials
      mf_norm(env, st, lo.input_norm, layer > 0, stream);
      a.x = static_cast<const bf16_t*>(sc.xn);
      a.p0 = pk(po.qkv);
      a.w1 = wt(lo.qkv_b);
      a.K = d.hidden;
      a.q = static_cast<bf16_t*>(sc.q);
      a.key_cache = static_cast<bf16_t*>(st.key_cache) + layer * cache_layer_elems;
      a.value_cache = static_cast<bf16_t*>(st.value_cache) + layer * cache_layer_elems;
      a.rope = sc.rope;
      a.slot = st.slot;
      a.active = st.active;
      a.slots = d.slots();
      a.heads = d.heads;
      a.kv_heads = d.kv_heads;
      a.head_dim = d.head_dim;
      // 8 K-range partials per qkv row, then the epilogue in k_mf_qkv_finish
      a.part = sc.mf_part;
      a.hidden_dim = d.qkv_rows();
      part_cu_launch<kHidSteps(kPartRanges), kQkvPartWaves, kHidSteps(kPartRanges), true>(
          a, d.qkv_rows() / 16 / kQkvPartWaves, stream);
      const int threads = d.batch * (d.qkv_rows() / d.head_dim) * (d.head_dim / 2);
      k_mf_qkv_finish<kPartRanges><<<(threads + 255) / 256, 256, 0, stream>>>(a);
      break;
    }
    case MfmaOp::kO:
      // the attention writes its output packed on this path (AttnArgs::packed_out)
      a.x = static_cast<const bf16_t*>(sc.attn);
      a.p0 = pk(po.o);
      a.K = d.q_dim();
      a.hidden = static_cast<bf16_t*>(sc.hidden);
      a.part = sc.mf_part;
      part_cu_launch<kHidSteps(kPartRanges), kPartWaves, kHidSteps(kPartRanges), false>(a, d.hidden / 16 / kPartWaves,
                                                                                         stream);
      break;
    case MfmaOp::kGateUp:
      mf_norm(env, st, lo.post_norm, true, stream);
      a.x = static_cast<const bf16_t*>(sc.xn);
      a.p0 = pk(po.gate);
      a.p1 = pk(po.up);
      a.K = d.hidden;
      a.out = static_cast<bf16_t*>(sc.mlp);
      a.hidden_dim = d.intermediate;
      k_mf_gu_cu<<<env.plan.gu_cu, kLcWaves * 64, kLcLds, stream>>>(a);
      break;
    case MfmaOp::kDown:
      a.x = static_cast<const bf16_t*>(sc.mlp);
      a.p0 = pk(po.down);
      a.K = d.intermediate;
      a.hidden = static_cast<bf16_t*>(sc.hidden);
      a.part = sc.mf_part;
      part_cu_launch<kInterSteps, kPartWaves, kDownBlk, false>(a, d.hidden / 16 / kPartWaves, stream);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace re
