// GQA paged decode attention of the resident decode epoch (gfx950)
// (batched_decoder_step.py:265-279, 334-379), one workgroup per
// (batch row, query head):
//   window positions j < W gathered through the block table;
//   s_j = bf16(bf16(q.k_j) / sqrt(d)) -- ExactQk is bf16-out; fp32 models keep
//   the fp32 product, then the bf16 rounding of the scaled score;
//   masked (j >= seq_len) positions contribute exp(bf16_min - max) = 0, so the
//   softmax runs over j < min(seq_len, W); a row with seq_len <= 0 has every
//   position masked and averages the whole window uniformly, as the reference;
//   p = bf16(softmax_fp32(s)) over the whole window (global max and sum first,
//   then each probability rounded); o = T(sum_j p_j v_j), fp32 accumulation.
//
// Layout of the work: LPR = d/8 lanes share one key (or value) row, each
// holding 8 of its elements, so one wave-wide 16-byte load covers 64/LPR whole
// rows (contiguous 2d-byte runs of the cache).  A lane issues LPR such loads per
// tile of 256 positions (4 waves x 64), then a halving exchange over its LPR
// lanes leaves one complete score per lane.  The keys and values of the first
// tile are requested together with the query at launch: one memory round
// trip for contexts up to 256.  The 7 query heads that share a KV head are
// placed on one XCD (block id = group + groups * head_in_group), so their
// key/value reads hit the same L2.
#pragma once

#include "re_device.h"
#include "re_layout.h"

namespace re {
namespace {

constexpr int kAttnThreads = 256;
constexpr int kAttnTile = 256;  // positions per tile: 4 waves x 64

template <int D>
struct AttnShape {
  static constexpr int kLpr = D / 8;         // lanes per row
  static constexpr int kRg = 64 / kLpr;      // rows per wave-wide load
  static constexpr int kLoads = kLpr;        // loads per lane per tile (64 rows per wave)
};

// Halving exchange over the N lanes of a group (lane offset c = lane % N,
// N a power of two from 2 to 32): afterwards lane c holds the total over the
// group of value c.  The levels at masks N/2, ..., 1 are re_device.h's
// reduce_step (DPP moves inside 16-lane rows, a permlane16 swap across).
template <int N, int M>
__device__ __forceinline__ void group_levels(float (&v)[N], int c) {
  if constexpr (M >= 1) {
    reduce_step<M, 2 * M>(v, c);
    group_levels<N, M / 2>(v, c);
  }
}
template <int N>
__device__ __forceinline__ void group_reduce_transpose(float (&v)[N], int c) {
  static_assert(N >= 2 && N <= 32 && (N & (N - 1)) == 0, "N must be a power of two in [2, 32]");
  group_levels<N, N / 2>(v, c);
}

// Position of load i of lane group r in wave w of tile t.
template <int D>
__device__ __forceinline__ int tile_pos(int t, int w, int i, int r) {
  return t * kAttnTile + w * 64 + i * AttnShape<D>::kRg + r;
}

// Element offsets (within this layer's cache) of the rows of one tile this
// lane loads: row chunk c of positions tile_pos(t, w, i, r); -1 where the
// position is >= neff or its slot is outside the cache.  tabs: the row's
// block table in LDS.
// Block and position within the block of position j >= 0: by division, or
// (P2: a power-of-two block size, a.bs_shift its log2) by shift and mask.
template <bool P2>
__device__ __forceinline__ void block_of(int j, const AttnArgs& a, int& blk, int& in_blk) {
  if constexpr (P2) {
    blk = j >> a.bs_shift;
    in_blk = j & (a.block_size - 1);
  } else {
    blk = j / a.block_size;
    in_blk = j % a.block_size;
  }
}

template <int D, bool P2 = false>
__device__ __forceinline__ void tile_offsets(int (&off)[AttnShape<D>::kLoads], const int* tabs, int t, int w,
                                             int r, int c, int neff, const AttnArgs& a, int g) {
#pragma unroll
  for (int i = 0; i < AttnShape<D>::kLoads; ++i) {
    const int j = tile_pos<D>(t, w, i, r);
    int bq, jb;
    block_of<P2>(j, a, bq, jb);
    const int blk = min(bq, a.blocks_per_row - 1);
    const long long slot = (long long)tabs[blk] * a.block_size + jb;
    const bool ok = j < neff && slot >= 0 && slot < a.slots;
    off[i] = ok ? static_cast<int>((slot * a.kv_heads + g) * D + c * 8) : -1;
  }
}

// Issue the loads of one tile's rows (keys or values): unconditional (a
// missing row reads row 0 and is zeroed afterwards), so all of them are in
// flight before the first is used.
template <typename T, int D>
__device__ __forceinline__ void load_tile(Vec8<T> (&v)[AttnShape<D>::kLoads], const T* cache,
                                          const int (&off)[AttnShape<D>::kLoads], int c) {
#pragma unroll
  for (int i = 0; i < AttnShape<D>::kLoads; ++i) v[i] = Vec8<T>::load_cached(cache + (off[i] >= 0 ? off[i] : c * 8));
}

__device__ __forceinline__ float attn_block_max(float v, float* red, int tid) {
  const int lane = tid & 63, wave = wave_index(tid);
  v = wave_max_dpp(v);
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float m = red[0];
#pragma unroll
  for (int i = 1; i < kAttnThreads / 64; ++i) m = fmaxf(m, red[i]);
  return m;
}

__device__ __forceinline__ float attn_block_sum(float v, float* red, int tid) {
  const int lane = tid & 63, wave = wave_index(tid);
  v = wave_sum_dpp(v);
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < kAttnThreads / 64; ++i) s += red[i];
  return s;
}

// The attention of one (batch row, query head): block = group + groups *
// head_in_group.  smem: dynamic LDS (attention_lds_bytes), red: 4 floats.
// P2: the block size is a power of two (a.bs_shift).
template <typename T, int D, bool P2 = false>
__device__ __forceinline__ void attn_body(const AttnArgs& a, int block, unsigned char* smem_raw, float* red,
                                          int tid) {
  using S = AttnShape<D>;
  constexpr int L = S::kLpr;
  const int W = a.window;
  float* sc = reinterpret_cast<float*>(smem_raw);  // [W] scores, then probabilities
  float* part = sc + W;                            // [4 waves][64 lanes][8] P.V partials
  const int G = a.heads / a.kv_heads;
  const int groups = a.B * a.kv_heads;
  const int grp = block % groups, hi = block / groups;
  const int b = grp / a.kv_heads, g = grp - b * a.kv_heads;
  const int h = g * G + hi;
  const int lane = tid & 63, w = wave_index(tid);
  const int r = lane / L, c = lane % L;
  const int n = a.len[b];
  const bool uniform = n <= 0;
  const int neff = uniform ? W : min(n, W);
  const int ntiles = (neff + kAttnTile - 1) / kAttnTile;
  const T* KC = static_cast<const T*>(a.key_cache);
  const T* VC = static_cast<const T*>(a.value_cache);
  const int32_t* tab = a.table + (size_t)b * a.blocks_per_row;
  int* tabs = reinterpret_cast<int*>(part + kAttnThreads * 8);  // [blocks_per_row]

  // Round trip 1: the row's block table (into LDS) and the query chunk.
  // Round trip 2: the first tile of keys and values, all loads in flight.
  const int32_t stop = a.done != nullptr ? request_flag(a.done) : 0;
  for (int e = tid; e < a.blocks_per_row; e += kAttnThreads) tabs[e] = tab[e];
  const Vec8<T> qv = Vec8<T>::load_cached(static_cast<const T*>(a.q) + ((size_t)b * a.heads + h) * D + c * 8);
  lds_barrier();
  if (flag_set(stop)) return;  // uniform over the workgroup
  int off[S::kLoads];
  tile_offsets<D, P2>(off, tabs, 0, w, r, c, neff, a, g);
  Vec8<T> kr[S::kLoads], vr[S::kLoads];
  load_tile<T, D>(kr, KC, off, c);
  load_tile<T, D>(vr, VC, off, c);

  // Scores of every tile into sc.
  const float scale_div = sqrtf(static_cast<float>(D));
  float smax = -INFINITY;
  for (int t = 0; t < ntiles; ++t) {
    if (t > 0) {
      tile_offsets<D, P2>(off, tabs, t, w, r, c, neff, a, g);
      load_tile<T, D>(kr, KC, off, c);
    }
    // a missing row (slot outside the cache) is a zero key: score 0
    float part_dot[L];
#pragma unroll
    for (int i = 0; i < L; ++i) part_dot[i] = off[i] >= 0 ? dot8(kr[i], qv, 0.f) : 0.f;
    group_reduce_transpose<L>(part_dot, c);
    // lane (r, c) now holds the score of position tile_pos(t, w, c, r)
    const int j = tile_pos<D>(t, w, c, r);
    float s = part_dot[0];
    if constexpr (sizeof(T) == 2) s = round_bf16(s);  // ExactQk output is bf16
    s = round_bf16(s / scale_div);
    if (uniform) s = -3.38953139e38f;  // every position masked to bf16 min
    if (j < neff) {
      sc[j] = s;
      smax = fmaxf(smax, s);
    }
  }
  const float mx = attn_block_max(smax, red, tid);
  float esum = 0.f;
  for (int j = tid; j < neff; j += kAttnThreads) esum += expf(sc[j] - mx);
  const float inv = 1.0f / attn_block_sum(esum, red, tid);
  for (int j = tid; j < neff; j += kAttnThreads) sc[j] = round_bf16(expf(sc[j] - mx) * inv);
  __syncthreads();

  // P.V: lane (r, c) accumulates elements c*8..c*8+7 over its rows.
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.f;
  for (int t = 0; t < ntiles; ++t) {
    if (t > 0) {
      tile_offsets<D, P2>(off, tabs, t, w, r, c, neff, a, g);
      load_tile<T, D>(vr, VC, off, c);
    } else if (ntiles > 1) {
      tile_offsets<D, P2>(off, tabs, 0, w, r, c, neff, a, g);  // the score loop moved on
    }
#pragma unroll
    for (int i = 0; i < S::kLoads; ++i) {
      // positions >= neff have off < 0; a missing row is a zero value.  The
      // read is unconditional (index clamped into the window) so the tile's
      // reads do not wait one by one.
      const float pr = sc[min(tile_pos<D>(t, w, i, r), W - 1)];
      const float p = off[i] >= 0 ? pr : 0.f;
      const Vec8<T> v = off[i] >= 0 ? vr[i] : Vec8<T>{};
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = fmaf(p, v.get(e), acc[e]);
    }
  }
  // Combine the 64/L row groups of each wave and the 4 waves, in a fixed order.
#pragma unroll
  for (int e = 0; e < 8; ++e) part[(w * 64 + lane) * 8 + e] = acc[e];
  __syncthreads();
  if (tid < D) {
    const int cc = tid / 8, e = tid % 8;
    float o = 0.f;
    for (int ww = 0; ww < kAttnThreads / 64; ++ww)
      for (int rr = 0; rr < S::kRg; ++rr) o += part[(ww * 64 + rr * L + cc) * 8 + e];
    const int k = h * D + tid;
    static_cast<T*>(a.out)[a.packed_out ? xpack_index(b, k, a.heads * D) : (size_t)b * a.heads * D + k] = Elt<T>::t(o);
  }
}

}  // namespace
}  // namespace re
