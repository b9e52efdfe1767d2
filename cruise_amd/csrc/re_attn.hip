// Paged decode attention launches (the body lives in re_attn.h).
#include "re_attn.h"

namespace re {
namespace {

template <typename T, int D, bool P2>
__global__ void __launch_bounds__(kAttnThreads) k_attn(AttnArgs a) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  __shared__ float red[kAttnThreads / 64];
  attn_body<T, D, P2>(a, blockIdx.x, smem_raw, red, threadIdx.x);
}

// ---------------------------------------------------------------------------
// Decode attention split over the window (long contexts at few rows): one
// workgroup per (row, query head, tile of 256 positions), so a window of n
// tiles costs the round trips of one tile instead of n in a row.  Same
// arithmetic and rounding points as attn_body; the row's max and sum are
// exact before any probability is rounded:
//   k_attn_split_scores: s_j as attn_body, into sp_scores; the tile's max m_t
//     and e_t = sum of exp(s_j - m_t) over its positions into sp_stats;
//   k_attn_split_pv: M = max_t m_t, sum = sum_t e_t exp(m_t - M) (tiles
//     summed in a fixed order), p_j = bf16(exp(s_j - M) / sum), and the
//     tile's P.V (fp32) into sp_part;
//   k_attn_split_sum: o = T(sum of the tiles' P.V in tile order).
// Only the fp32 summation orders differ from attn_body.  Tiles past the
// row's context (neff) do nothing and are not read.  The 7 heads sharing a
// KV head sit 8 * k block ids apart (block = unit + units * head_in_group,
// unit = grp + groups * tile, units a multiple of 8 for 4 KV heads and an
// even row count) so their key and value reads share an XCD's L2.

struct SplitUnit {
  int b, g, h, t;
};

__device__ __forceinline__ SplitUnit split_unit(const AttnArgs& a, int block) {
  const int G = a.heads / a.kv_heads;
  const int groups = a.B * a.kv_heads;
  const int units = groups * a.split_tiles;
  const int hi = block / units, u = block - hi * units;
  const int t = u / groups, grp = u - t * groups;
  SplitUnit s;
  s.b = grp / a.kv_heads;
  s.g = grp - s.b * a.kv_heads;
  s.h = s.g * G + hi;
  s.t = t;
  return s;
}

__device__ __forceinline__ int split_neff(const AttnArgs& a, int b) {
  const int n = a.len[b];
  return n <= 0 ? a.window : min(n, a.window);
}

template <typename T, int D, bool P2>
__global__ void __launch_bounds__(kAttnThreads) k_attn_split_scores(AttnArgs a) {
  using S = AttnShape<D>;
  constexpr int L = S::kLpr;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  __shared__ float red[kAttnThreads / 64];
  int* tabs = reinterpret_cast<int*>(smem_raw);  // [blocks_per_row]
  const int tid = threadIdx.x;
  const SplitUnit u = split_unit(a, blockIdx.x);
  const int32_t stop = a.done != nullptr ? request_flag(a.done) : 0;
  const bool uniform = a.len[u.b] <= 0;
  const int neff = split_neff(a, u.b);
  if (flag_set(stop) || u.t * kAttnTile >= neff) return;  // uniform over the workgroup
  const int lane = tid & 63, w = wave_index(tid);
  const int r = lane / L, c = lane % L;
  const int32_t* tab = a.table + (size_t)u.b * a.blocks_per_row;
  for (int e = tid; e < a.blocks_per_row; e += kAttnThreads) tabs[e] = tab[e];
  const Vec8<T> qv = Vec8<T>::load_cached(static_cast<const T*>(a.q) + ((size_t)u.b * a.heads + u.h) * D + c * 8);
  lds_barrier();
  int off[S::kLoads];
  tile_offsets<D, P2>(off, tabs, u.t, w, r, c, neff, a, u.g);
  Vec8<T> kr[S::kLoads];
  load_tile<T, D>(kr, static_cast<const T*>(a.key_cache), off, c);
  // a missing row (slot outside the cache) is a zero key: score 0
  float part_dot[L];
#pragma unroll
  for (int i = 0; i < L; ++i) part_dot[i] = off[i] >= 0 ? dot8(kr[i], qv, 0.f) : 0.f;
  group_reduce_transpose<L>(part_dot, c);
  // lane (r, c) holds the score of position tile_pos(t, w, c, r)
  const int j = tile_pos<D>(u.t, w, c, r);
  float s = part_dot[0];
  if constexpr (sizeof(T) == 2) s = round_bf16(s);  // ExactQk output is bf16
  s = round_bf16(s / sqrtf(static_cast<float>(D)));
  if (uniform) s = -3.38953139e38f;  // every position masked to bf16 min
  const bool in = j < neff;
  const size_t row = (size_t)u.b * a.heads + u.h;
  if (in) a.sp_scores[row * a.window + j] = s;
  const float mt = attn_block_max(in ? s : -INFINITY, red, tid);
  const float et = attn_block_sum(in ? expf(s - mt) : 0.f, red, tid);
  if (tid == 0) {
    float* st = a.sp_stats + (row * a.split_tiles + u.t) * 2;
    st[0] = mt;
    st[1] = et;
  }
}

template <typename T, int D, bool P2>
__global__ void __launch_bounds__(kAttnThreads) k_attn_split_pv(AttnArgs a) {
  using S = AttnShape<D>;
  constexpr int L = S::kLpr;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  __shared__ float red[kAttnThreads / 64];
  __shared__ float pr[kAttnTile];               // the tile's probabilities
  __shared__ float part[kAttnThreads * 8];      // [4 waves][64 lanes][8] P.V partials
  int* tabs = reinterpret_cast<int*>(smem_raw);  // [blocks_per_row]
  const int tid = threadIdx.x;
  const SplitUnit u = split_unit(a, blockIdx.x);
  const int32_t stop = a.done != nullptr ? request_flag(a.done) : 0;
  const int neff = split_neff(a, u.b);
  if (flag_set(stop) || u.t * kAttnTile >= neff) return;  // uniform over the workgroup
  const int lane = tid & 63, w = wave_index(tid);
  const int r = lane / L, c = lane % L;
  // Round trip 1: the block table, this thread's score and the first tile
  // statistics it reduces (clamped reads; the masks below drop the extras).
  // Round trip 2: the tile's values.
  const size_t row = (size_t)u.b * a.heads + u.h;
  const int nt = (neff + kAttnTile - 1) / kAttnTile;
  const float* st = a.sp_stats + row * a.split_tiles * 2;
  const int j = u.t * kAttnTile + tid;
  const float sj = a.sp_scores[row * a.window + min(j, neff - 1)];
  const int i0 = min(tid, nt - 1);
  const float m0 = st[2 * i0], e0 = st[2 * i0 + 1];
  const int32_t* tab = a.table + (size_t)u.b * a.blocks_per_row;
  for (int e = tid; e < a.blocks_per_row; e += kAttnThreads) tabs[e] = tab[e];
  lds_barrier();
  int off[S::kLoads];
  tile_offsets<D, P2>(off, tabs, u.t, w, r, c, neff, a, u.g);
  Vec8<T> vr[S::kLoads];
  load_tile<T, D>(vr, static_cast<const T*>(a.value_cache), off, c);

  // The row's exact max and sum from the tiles' statistics.
  float m = tid < nt ? m0 : -INFINITY;
  for (int i = tid + kAttnThreads; i < nt; i += kAttnThreads) m = fmaxf(m, st[2 * i]);
  const float mx = attn_block_max(m, red, tid);
  float e = tid < nt ? e0 * expf(m0 - mx) : 0.f;
  for (int i = tid + kAttnThreads; i < nt; i += kAttnThreads) e += st[2 * i + 1] * expf(st[2 * i] - mx);
  const float inv = 1.0f / attn_block_sum(e, red, tid);
  pr[tid] = j < neff ? round_bf16(expf(sj - mx) * inv) : 0.f;
  __syncthreads();

  // P.V of the tile: lane (r, c) accumulates elements c*8..c*8+7 over its rows.
  float acc[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) acc[k] = 0.f;
#pragma unroll
  for (int i = 0; i < S::kLoads; ++i) {
    // positions >= neff have off < 0; a missing row is a zero value
    const float p = off[i] >= 0 ? pr[w * 64 + i * S::kRg + r] : 0.f;
    const Vec8<T> v = off[i] >= 0 ? vr[i] : Vec8<T>{};
#pragma unroll
    for (int k = 0; k < 8; ++k) acc[k] = fmaf(p, v.get(k), acc[k]);
  }
#pragma unroll
  for (int k = 0; k < 8; ++k) part[(w * 64 + lane) * 8 + k] = acc[k];
  __syncthreads();
  if (tid < D) {
    const int cc = tid / 8, k = tid % 8;
    float o = 0.f;
    for (int ww = 0; ww < kAttnThreads / 64; ++ww)
      for (int rr = 0; rr < S::kRg; ++rr) o += part[(ww * 64 + rr * L + cc) * 8 + k];
    a.sp_part[(row * a.split_tiles + u.t) * D + tid] = o;
  }
}

// One thread per output element (row, head, element): the tiles' P.V in
// tile order.
template <typename T>
__global__ void __launch_bounds__(256) k_attn_split_sum(AttnArgs a) {
  const int D = a.head_dim;
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= a.B * a.heads * D) return;
  if (a.done != nullptr && __builtin_nontemporal_load(a.done) != 0) return;
  const int row = i / D, k = i - row * D;
  const int b = row / a.heads;
  const int nt = (split_neff(a, b) + kAttnTile - 1) / kAttnTile;
  const float* p = a.sp_part + (size_t)row * a.split_tiles * D + k;
  // 8 tiles requested at a time (clamped reads, masked adds), added in order
  float o = 0.f;
  for (int t = 0; t < nt; t += 8) {
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = p[(size_t)min(t + i, nt - 1) * D];
#pragma unroll
    for (int i = 0; i < 8; ++i) o = t + i < nt ? o + v[i] : o;
  }
  const int hk = (row - b * a.heads) * D + k;
  static_cast<T*>(a.out)[a.packed_out ? xpack_index(b, hk, a.heads * D) : (size_t)b * a.heads * D + hk] =
      Elt<T>::t(o);
}

// ---------------------------------------------------------------------------
// Grouped decode attention for many rows (B x KV heads >= 64, bf16,
// head_dim 128): one workgroup per (row, KV head) computes the G <= 8 query
// heads that share the KV head, so every key and value row is read once for
// all of them (the per-(row, head) kernel reads it G times) and 256
// workgroups cover 64 rows x 4 KV heads.  Same arithmetic and rounding points
// as attn_body: s = bf16(bf16(q.k) / sqrt(d)); masked positions drop out of
// the softmax (a row with no context averages the whole window uniformly);
// p = bf16(exp(s - max) / sum) with the exact max and sum of the row; o =
// T(sum p v) in fp32.  Only the fp32 summation orders differ.
//
// Layout: thread t handles elements (t % 16) * 8 ..+8 of the head (16 lanes
// per 256-byte key or value row) and position slot t / 16 of each group of
// 32 positions; a tile is 256 positions, 8 rows per thread, all requested at
// once.  Scores go to LDS per head, then the softmax runs over LDS, then P.V
// accumulates per thread over its positions and the 32 position slots are
// added (shuffles within a wave, LDS across the eight waves, in order).
// ---------------------------------------------------------------------------
constexpr int kGrpThreads = 512;  // 8 waves: two per SIMD hide each other's latency
constexpr int kGrpMaxG = 8;
constexpr int kGrpD = 128;
constexpr int kGrpWaves = kGrpThreads / 64;
constexpr int kGrpTile = 256;                      // positions per tile
constexpr int kGrpSlots = kGrpThreads / 16;        // positions per wave-wide load of the block
constexpr int kGrpRows = kGrpTile / kGrpSlots;      // rows per thread per tile

size_t group_smem_bytes(int G, int window, int blocks_per_row) {
  return (size_t)G * window * sizeof(float) + (size_t)kGrpWaves * G * kGrpD * sizeof(float) +
         (size_t)blocks_per_row * sizeof(int);
}

template <bool P2>
__global__ void __launch_bounds__(kGrpThreads) k_attn_group(AttnArgs a) {
  extern __shared__ __align__(16) float gsm[];
  __shared__ float red[kGrpWaves][kGrpMaxG];
  const int G = a.heads / a.kv_heads, W = a.window;
  const int b = blockIdx.x / a.kv_heads, g = blockIdx.x - b * a.kv_heads;
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_index(tid);
  const int c = tid & 15, r = tid >> 4;
  float* sc = gsm;                   // [G][W] scores, then probabilities
  float* osum = sc + (size_t)G * W;  // [waves][G][D]
  int* tabs = reinterpret_cast<int*>(osum + kGrpWaves * G * kGrpD);
  const bf16_t* KC = static_cast<const bf16_t*>(a.key_cache);
  const bf16_t* VC = static_cast<const bf16_t*>(a.value_cache);
  const int n = a.len[b];
  const bool uniform = n <= 0;
  const int neff = uniform ? W : min(n, W);
  const int ntiles = (neff + kGrpTile - 1) / kGrpTile;

  const int32_t stop = a.done != nullptr ? request_flag(a.done) : 0;
  for (int e = tid; e < a.blocks_per_row; e += kGrpThreads) tabs[e] = a.table[(size_t)b * a.blocks_per_row + e];
  Vec8<bf16_t> qv[kGrpMaxG];
#pragma unroll
  for (int h = 0; h < kGrpMaxG; ++h)
    qv[h] = Vec8<bf16_t>::load_cached(static_cast<const bf16_t*>(a.q) +
                                      ((size_t)b * a.heads + g * G + min(h, G - 1)) * kGrpD + c * 8);
  lds_barrier();
  if (flag_set(stop)) return;  // uniform

  // element offset of position j's row chunk in this layer's cache, or -1
  auto row_off = [&](int j) -> int {
    if (j >= neff) return -1;
    int blk, in_blk;
    block_of<P2>(j, a, blk, in_blk);
    const long long slot = (long long)tabs[min(blk, a.blocks_per_row - 1)] * a.block_size + in_blk;
    return slot >= 0 && slot < a.slots ? static_cast<int>((slot * a.kv_heads + g) * kGrpD + c * 8) : -1;
  };
  auto load_tile = [&](Vec8<bf16_t>(&v)[kGrpRows], int (&off)[kGrpRows], const bf16_t* cache, int t) {
#pragma unroll
    for (int i = 0; i < kGrpRows; ++i) {
      off[i] = row_off(t * kGrpTile + i * kGrpSlots + r);
      v[i] = Vec8<bf16_t>::load_cached(cache + (off[i] >= 0 ? off[i] : c * 8));
    }
  };

  // Scores.  After the exchanges lane c < G holds head c's score.  Two
  // register sets: the next tile's rows are in flight while a tile is
  // computed (a tile past the context loads one valid line per lane and is
  // dropped).
  auto score_tile = [&](const Vec8<bf16_t>(&kr)[kGrpRows], const int (&off)[kGrpRows], int t) {
#pragma unroll
    for (int i = 0; i < kGrpRows; ++i) {
      float part[kGrpMaxG];
#pragma unroll
      for (int h = 0; h < kGrpMaxG; ++h) part[h] = off[i] >= 0 ? dot8(kr[i], qv[h], 0.f) : 0.f;  // missing row: zero key
#pragma unroll
      for (int h = 0; h < kGrpMaxG; ++h) part[h] = xor_add<8>(part[h], lane);
      group_reduce_transpose<kGrpMaxG>(part, c & 7);
      const int j = t * kGrpTile + i * kGrpSlots + r;
      // ExactQk output is bf16, then the bf16 quotient by sqrt(128)
      float s = round_bf16(div_sqrt128_bf16(round_bf16(part[0])));
      if (uniform) s = -3.38953139e38f;  // every position masked to bf16 min
      if (c < G && j < neff) sc[(size_t)c * W + j] = s;
    }
  };
  {
    Vec8<bf16_t> ka[kGrpRows], kb[kGrpRows];
    int oa[kGrpRows], ob[kGrpRows];
    load_tile(ka, oa, KC, 0);
    for (int t = 0; t < ntiles; t += 2) {
      load_tile(kb, ob, KC, t + 1);
      __builtin_amdgcn_sched_barrier(0);
      score_tile(ka, oa, t);
      if (t + 2 < ntiles) load_tile(ka, oa, KC, t + 2);
      __builtin_amdgcn_sched_barrier(0);
      score_tile(kb, ob, t + 1);
    }
  }
  lds_barrier();

  // Softmax per head over LDS: exact max and sum, then each probability rounded.
  float mx[kGrpMaxG], inv[kGrpMaxG];
#pragma unroll
  for (int h = 0; h < kGrpMaxG; ++h) {
    float m = -INFINITY;
    if (h < G)
      for (int j = tid; j < neff; j += kGrpThreads) m = fmaxf(m, sc[(size_t)h * W + j]);
    m = wave_max(m);
    if (lane == 0) red[wave][h] = m;
  }
  lds_barrier();
#pragma unroll
  for (int h = 0; h < kGrpMaxG; ++h) {
    mx[h] = red[0][h];
#pragma unroll
    for (int w = 1; w < kGrpWaves; ++w) mx[h] = fmaxf(mx[h], red[w][h]);
    float e = 0.f;
    if (h < G)
      for (int j = tid; j < neff; j += kGrpThreads) e += expf(sc[(size_t)h * W + j] - mx[h]);
    inv[h] = wave_sum(e);
  }
  lds_barrier();  // every max read before red is reused
  if (lane == 0) {
#pragma unroll
    for (int h = 0; h < kGrpMaxG; ++h) red[wave][h] = inv[h];
  }
  lds_barrier();
#pragma unroll
  for (int h = 0; h < kGrpMaxG; ++h) {
    float total = 0.f;
#pragma unroll
    for (int w = 0; w < kGrpWaves; ++w) total += red[w][h];
    inv[h] = 1.0f / total;
    if (h < G)
      for (int j = tid; j < neff; j += kGrpThreads)
        sc[(size_t)h * W + j] = round_bf16(expf(sc[(size_t)h * W + j] - mx[h]) * inv[h]);
  }
  lds_barrier();

  // P.V over this thread's positions, then the 16 position slots added.
  float acc[kGrpMaxG][8];
#pragma unroll
  for (int h = 0; h < kGrpMaxG; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[h][e] = 0.f;
  auto pv_tile = [&](const Vec8<bf16_t>(&vr)[kGrpRows], const int (&off)[kGrpRows], int t) {
#pragma unroll
    for (int i = 0; i < kGrpRows; ++i) {
      const int j = t * kGrpTile + i * kGrpSlots + r;
      if (off[i] < 0) continue;  // past the context, or a missing row (a zero value)
#pragma unroll
      for (int h = 0; h < kGrpMaxG; ++h) {
        if (h >= G) break;
        const float p = sc[(size_t)h * W + j];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[h][e] = fmaf(p, vr[i].get(e), acc[h][e]);
      }
    }
  };
  {
    Vec8<bf16_t> va[kGrpRows], vb[kGrpRows];
    int oa[kGrpRows], ob[kGrpRows];
    load_tile(va, oa, VC, 0);
    for (int t = 0; t < ntiles; t += 2) {
      load_tile(vb, ob, VC, t + 1);
      __builtin_amdgcn_sched_barrier(0);
      pv_tile(va, oa, t);
      if (t + 2 < ntiles) load_tile(va, oa, VC, t + 2);
      __builtin_amdgcn_sched_barrier(0);
      pv_tile(vb, ob, t + 1);
    }
  }
#pragma unroll
  for (int h = 0; h < kGrpMaxG; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      acc[h][e] = xor_add<16>(acc[h][e], lane);
      acc[h][e] = xor_add<32>(acc[h][e], lane);
    }
  if (lane < 16) {
#pragma unroll
    for (int h = 0; h < kGrpMaxG; ++h)
      if (h < G)
#pragma unroll
        for (int e = 0; e < 8; ++e) osum[((size_t)wave * G + h) * kGrpD + c * 8 + e] = acc[h][e];
  }
  lds_barrier();
  for (int o = tid; o < G * kGrpD; o += kGrpThreads) {
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < kGrpWaves; ++w) v += osum[w * G * kGrpD + o];
    const int h = o / kGrpD, d = o - h * kGrpD;
    const int k = (g * G + h) * kGrpD + d;
    static_cast<bf16_t*>(a.out)[a.packed_out ? xpack_index(b, k, a.heads * kGrpD) : (size_t)b * a.heads * kGrpD + k] =
        f_to_bf16(v);
  }
}

// ---------------------------------------------------------------------------
// Grouped decode attention on the matrix cores (bf16, head_dim 128, up to 8
// query heads per KV head): one workgroup of 8 waves per (row, KV head), as
// k_attn_group, with both products on v_mfma_f32_16x16x32_bf16.
//   requests  the keys of a chunk of up to four 256-position tiles go out
//             together (wave w: position groups 2w and 2w + 1 of each tile;
//             lane l: row l % 16, elements 8 (l / 16) + 32 kk ..+8, the MFMA
//             operand layout), and the first chunk's values follow as the
//             last chunk's key tiles are consumed, so they stream during the
//             softmax;
//   scores    Sᵀ tile of 16 positions x 16 head slots: A = 16 key rows, B =
//             the queries (head l % 16, zero past G), four k steps of 32;
//             s = bf16(bf16(q.k) / sqrt(d)) into LDS, position-major (the 8
//             head slots of a position in 32 bytes);
//   softmax   exact max and sum per head over LDS: a thread reads all heads
//             of a position in two 16-byte reads, the heads' wave reductions
//             are interleaved (one wait per exchange step); then
//             p = bf16(exp(s - max) / sum) into a bf16 array, zero past the
//             context;
//   P.V       wave w multiplies the value rows it loaded (its 32 positions
//             of each tile) from registers: A = p (head l % 16, the lane's 8
//             positions, one 16-byte LDS read), B = element e of the lane's
//             8 rows (8 products per tile, output columns permuted to dims
//             8 (l % 16) + e); the 8 waves' fp32 partials are added in wave
//             order through LDS at the end.
// Same rounding points as k_attn_group; only fp32 summation orders differ.
// Rows whose slot is outside the cache are zero keys (score 0) and zero
// values.  Every key and value request is unconditional (a row past the
// context or missing reads the cache's first row): a load under a per-lane
// condition would make the next use wait for every outstanding load.
// ---------------------------------------------------------------------------
typedef __bf16 mg_bf16x8 __attribute__((ext_vector_type(8)));
typedef float mg_f32x4 __attribute__((ext_vector_type(4)));
constexpr int kMgThreads = 512, kMgWaves = 8, kMgTile = 256, kMgD = 128, kMgMaxG = 8;
constexpr int kMgChunk = 4;           // tiles whose keys are requested together

// P.V of one wave's 32 positions of a tile, from the value rows the wave
// loaded: lane (l / 16, l % 16) holds elements 8 (l % 16) + e of rows
// 8 (l / 16) + i (bit i of mask: the row is present; absent rows enter as
// zeros).  Product e takes element e of the lane's 8 rows (4 v_perm) as the B
// operand -- k = the lane's 8 positions, column l % 16 = dim 8 (l % 16) + e --
// so its 16 output columns are dims e, 8 + e, ..., 120 + e and the 8
// products cover all 128 dims without a transpose.  pa: p of head l % 16 at
// the lane's 8 positions.  Value v of lane l in oacc[e]: head 4 (l / 16) + v,
// dim 8 (l % 16) + e.
__device__ __forceinline__ void mg_pv_rows(mg_f32x4 (&oacc)[8], const re_u32x4& pa, const Vec8<bf16_t> (&v)[8],
                                           int mask) {
  re_u32x4 w[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) w[i] = v[i].v;
  if (__builtin_amdgcn_ballot_w64(mask != 0xff) != 0) {  // some row of the wave absent
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (!((mask >> i) & 1)) w[i] = re_u32x4{0u, 0u, 0u, 0u};
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    // word i: element e of rows 2 i (low half) and 2 i + 1 (high half)
    const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
    re_u32x4 bw;
#pragma unroll
    for (int i = 0; i < 4; ++i) bw[i] = __builtin_amdgcn_perm(w[2 * i + 1][e >> 1], w[2 * i][e >> 1], sel);
    oacc[e] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(mg_bf16x8, pa), __builtin_bit_cast(mg_bf16x8, bw),
                                                      oacc[e], 0, 0, 0);
  }
}

// The waves' partial outputs in LDS: fp32 [8 waves][8 head slots][128].
constexpr size_t kMgPartBytes = (size_t)kMgWaves * kMgMaxG * kMgD * sizeof(float);
__device__ __forceinline__ void mg_put_partials(float* part, const mg_f32x4 (&oacc)[8], int wave, int lane) {
  const int lq = lane >> 4, l16 = lane & 15;
  if (lq < 2) {  // head slots 0..7
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      float* dst = part + ((size_t)wave * kMgMaxG + lq * 4 + v) * kMgD + l16 * 8;
      *reinterpret_cast<re_f32x4*>(dst) = re_f32x4{oacc[0][v], oacc[1][v], oacc[2][v], oacc[3][v]};
      *reinterpret_cast<re_f32x4*>(dst + 4) = re_f32x4{oacc[4][v], oacc[5][v], oacc[6][v], oacc[7][v]};
    }
  }
}
// Element e = h * 128 + d of the output: the 8 waves' partials in wave order.
__device__ __forceinline__ float mg_sum_partials(const float* part, int e) {
  float o = 0.f;
#pragma unroll
  for (int w = 0; w < kMgWaves; ++w) o += part[(size_t)w * kMgMaxG * kMgD + e];
  return o;
}

// The window's tiles rounded up to whole chunks.
__host__ __device__ int mgroup_tiles(int window) {
  const int t = (window + kMgTile - 1) / kMgTile;
  return (t + kMgChunk - 1) / kMgChunk * kMgChunk;
}
// LDS: scores [window][8] fp32, probabilities [8][tiles * 256] bf16, the
// waves' partial outputs [8][8][128] fp32, row offsets [tiles * 256] int,
// the block table.
struct MgLayout {
  size_t pb, part, roff, tabs, total;
};
__host__ __device__ MgLayout mgroup_layout(int G, int window, int blocks_per_row) {
  MgLayout l;
  const size_t span = (size_t)mgroup_tiles(window) * kMgTile;
  (void)G;
  l.pb = (size_t)window * kMgMaxG * sizeof(float);
  l.part = l.pb + (size_t)kMgMaxG * span * sizeof(bf16_t);
  l.roff = l.part + kMgPartBytes;
  l.tabs = l.roff + span * sizeof(int);
  l.total = l.tabs + (size_t)blocks_per_row * sizeof(int);
  return l;
}
size_t mgroup_smem_bytes(int G, int window, int blocks_per_row) { return mgroup_layout(G, window, blocks_per_row).total; }

// Wave-wide max / sum of N values at once: the N exchanges of a step are
// independent, so they wait together.
template <int S, int N>
__device__ __forceinline__ void wave_max_steps(float (&v)[N], int lane) {
  if constexpr (S >= 1) {
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = xor_max<S>(v[i], lane);
    wave_max_steps<S / 2>(v, lane);
  }
}
template <int S, int N>
__device__ __forceinline__ void wave_sum_steps(float (&v)[N], int lane) {
  if constexpr (S >= 1) {
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = xor_add<S>(v[i], lane);
    wave_sum_steps<S / 2>(v, lane);
  }
}
template <int N>
__device__ __forceinline__ void wave_max_n(float (&v)[N]) {
  wave_max_steps<32>(v, static_cast<int>(threadIdx.x & 63));
}
template <int N>
__device__ __forceinline__ void wave_sum_n(float (&v)[N]) {
  wave_sum_steps<32>(v, static_cast<int>(threadIdx.x & 63));
}

template <bool P2>
__global__ void __launch_bounds__(kMgThreads) k_attn_mgroup(AttnArgs a) {
  extern __shared__ __align__(16) unsigned char mg_smem[];
  __shared__ float red[kMgWaves][kMgMaxG], red_sum[kMgWaves][kMgMaxG];
  const int G = a.heads / a.kv_heads, W = a.window;
  const int b = blockIdx.x / a.kv_heads, g = blockIdx.x - b * a.kv_heads;
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_index(tid);
  const int l16 = lane & 15, lq = lane >> 4;
  const MgLayout L = mgroup_layout(G, W, a.blocks_per_row);
  const int span = mgroup_tiles(W) * kMgTile;
  float* sc = reinterpret_cast<float*>(mg_smem);            // [W][kMgMaxG]
  bf16_t* pb = reinterpret_cast<bf16_t*>(mg_smem + L.pb);   // [kMgMaxG][span]
  int* roff = reinterpret_cast<int*>(mg_smem + L.roff);     // [span]
  int* tabs = reinterpret_cast<int*>(mg_smem + L.tabs);
  const bf16_t* KC = static_cast<const bf16_t*>(a.key_cache);
  const bf16_t* VC = static_cast<const bf16_t*>(a.value_cache);
  const int n = a.len[b];
  const bool uniform = n <= 0;
  const int neff = uniform ? W : min(n, W);
  const int ntiles = (neff + kMgTile - 1) / kMgTile;
  const int nchunks = (ntiles + kMgChunk - 1) / kMgChunk;
  const int padded = nchunks * kMgChunk * kMgTile;  // positions the requests cover (<= span)

  const int32_t stop = a.done != nullptr ? request_flag(a.done) : 0;
  for (int e = tid; e < a.blocks_per_row; e += kMgThreads) tabs[e] = a.table[(size_t)b * a.blocks_per_row + e];
  // queries as the B operand: head l % 16 (zero past G), 4 k steps
  mg_bf16x8 qf[4];
  {
    const bf16_t* qrow = static_cast<const bf16_t*>(a.q) + ((size_t)b * a.heads + g * G + min(l16, G - 1)) * kMgD;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const re_u32x4 v = *reinterpret_cast<const re_u32x4*>(qrow + kk * 32 + lq * 8);
      qf[kk] = __builtin_bit_cast(mg_bf16x8, l16 < G ? v : re_u32x4{0u, 0u, 0u, 0u});
    }
  }
  lds_barrier();
  if (flag_set(stop)) return;  // uniform

  // Element offset of each position's row (this KV head) in the layer's
  // cache, or -1 past the context or for a slot outside the cache; one LDS
  // read per request afterwards (cache offsets of a layer fit 32 bits).
  for (int j = tid; j < padded; j += kMgThreads) {
    int o = -1;
    if (j < neff) {
      int blk, in_blk;
      block_of<P2>(j, a, blk, in_blk);
      const long long slot = (long long)tabs[min(blk, a.blocks_per_row - 1)] * a.block_size + in_blk;
      if (slot >= 0 && slot < a.slots) o = static_cast<int>((slot * a.kv_heads + g) * kMgD);
    }
    roff[j] = o;
  }
  lds_barrier();

  float smax = -INFINITY;
  // Keys of tile t: kvalid[q] bit r marks row r of position group 2 w + q
  // present (lanes r and r + 16 k hold the same row).
  auto load_k = [&](re_u32x4(&kf)[2][4], uint32_t(&kvalid)[2], int t) {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int off = roff[t * kMgTile + (2 * wave + q) * 16 + l16];
      kvalid[q] = static_cast<uint32_t>(__builtin_amdgcn_ballot_w64(off >= 0)) & 0xffffu;
      const bf16_t* row = KC + (off >= 0 ? off : 0);
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) kf[q][kk] = *reinterpret_cast<const re_u32x4*>(row + kk * 32 + lq * 8);
    }
  };
  auto score_k = [&](const re_u32x4(&kf)[2][4], const uint32_t(&kvalid)[2], int t) {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      mg_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(mg_bf16x8, kf[q][kk]), qf[kk], acc, 0, 0, 0);
      // value v of lane l: position 4 (l / 16) + v of the group, head l % 16
      const uint32_t present = kvalid[q] >> (lq * 4);
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int j = t * kMgTile + (2 * wave + q) * 16 + lq * 4 + v;
        // ExactQk output is bf16, then the bf16 quotient by sqrt(128)
        float s = round_bf16(div_sqrt128_bf16(round_bf16(acc[v])));
        if (uniform) s = -3.38953139e38f;  // every position masked to bf16 min
        // a missing row (slot outside the cache) is a zero key: score 0
        if (l16 < G && j < neff) {
          const float st = (present >> v) & 1 || uniform ? s : 0.f;
          sc[(size_t)j * kMgMaxG + l16] = st;
          smax = fmaxf(smax, st);
        }
      }
    }
  };
  // value rows p0 .. p0+7 of tile t, chunk l16 (elements 8 l16 ..+8); bit i
  // of the returned mask marks row i valid (invalid rows enter as zero)
  const int p0 = wave * 32 + lq * 8;
  auto load_v = [&](Vec8<bf16_t>(&vr)[8], int t) {
    int mask = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int off = roff[t * kMgTile + p0 + i];
      vr[i] = Vec8<bf16_t>::load_cached(VC + (off >= 0 ? off : 0) + l16 * 8);
      mask |= (off >= 0 ? 1 : 0) << i;
    }
    return mask;
  };

  // Scores, one chunk of key tiles at a time; the first chunk's values are
  // requested as the last chunk's key tiles are consumed.  smax: the lane's
  // running max of its head's stored scores.
  Vec8<bf16_t> vr[kMgChunk][8];
  int vmask[kMgChunk];
  for (int c = 0; c + 1 < nchunks; ++c) {
    re_u32x4 kf[kMgChunk][2][4];
    uint32_t kvalid[kMgChunk][2];
#pragma unroll
    for (int i = 0; i < kMgChunk; ++i) load_k(kf[i], kvalid[i], c * kMgChunk + i);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < kMgChunk; ++i) score_k(kf[i], kvalid[i], c * kMgChunk + i);
  }
  {
    const int c = nchunks - 1;
    re_u32x4 kf[kMgChunk][2][4];
    uint32_t kvalid[kMgChunk][2];
#pragma unroll
    for (int i = 0; i < kMgChunk; ++i) load_k(kf[i], kvalid[i], c * kMgChunk + i);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < kMgChunk; ++i) {
      score_k(kf[i], kvalid[i], c * kMgChunk + i);
      vmask[i] = load_v(vr[i], i);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // each head's max over the wave (lanes l % 16 == h), published with the scores
  smax = xor_max<16>(smax, lane);
  smax = xor_max<32>(smax, lane);
  if (lq == 0 && l16 < kMgMaxG) red[wave][l16] = smax;
  lds_barrier();

  // Softmax per head over LDS: the exact max (from the score pass) and sum,
  // then each probability rounded to bf16 (zero from the context's end to
  // the requests' end).  Head slots from G up hold no score: they are
  // masked, not branched on.
  auto head_scores = [&](int j, float (&v)[kMgMaxG]) {
    const re_f32x4 lo = *reinterpret_cast<const re_f32x4*>(sc + (size_t)j * kMgMaxG);
    const re_f32x4 hi = *reinterpret_cast<const re_f32x4*>(sc + (size_t)j * kMgMaxG + 4);
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      v[h] = lo[h];
      v[h + 4] = hi[h];
    }
  };
  float mx[kMgMaxG], inv[kMgMaxG];
#pragma unroll
  for (int h = 0; h < kMgMaxG; ++h) {
    mx[h] = red[0][h];
#pragma unroll
    for (int w = 1; w < kMgWaves; ++w) mx[h] = fmaxf(mx[h], red[w][h]);
  }
  // e = exp(s - max) replaces the score in LDS (the thread reads it back for
  // the probability), and the sums go to a second exchange array
  {
    float e[kMgMaxG];
#pragma unroll
    for (int h = 0; h < kMgMaxG; ++h) e[h] = 0.f;
    for (int j = tid; j < neff; j += kMgThreads) {
      float v[kMgMaxG];
      head_scores(j, v);
#pragma unroll
      for (int h = 0; h < kMgMaxG; ++h) {
        v[h] = h < G ? expf(v[h] - mx[h]) : 0.f;
        e[h] += v[h];
      }
      *reinterpret_cast<re_f32x4*>(sc + (size_t)j * kMgMaxG) = re_f32x4{v[0], v[1], v[2], v[3]};
      *reinterpret_cast<re_f32x4*>(sc + (size_t)j * kMgMaxG + 4) = re_f32x4{v[4], v[5], v[6], v[7]};
    }
    wave_sum_n<kMgMaxG>(e);
    if (lane == 0)
#pragma unroll
      for (int h = 0; h < kMgMaxG; ++h) red_sum[wave][h] = e[h];
  }
  lds_barrier();
#pragma unroll
  for (int h = 0; h < kMgMaxG; ++h) {
    float total = 0.f;
#pragma unroll
    for (int w = 0; w < kMgWaves; ++w) total += red_sum[w][h];
    inv[h] = 1.0f / total;
  }
  for (int j = tid; j < padded; j += kMgThreads) {
    float v[kMgMaxG];
    if (j < neff) {
      head_scores(j, v);
    } else {
#pragma unroll
      for (int h = 0; h < kMgMaxG; ++h) v[h] = 0.f;
    }
#pragma unroll
    for (int h = 0; h < kMgMaxG; ++h) {
      const float p = h < G && j < neff ? round_bf16(v[h] * inv[h]) : 0.f;
      pb[(size_t)h * span + j] = f_to_bf16(p);  // exact: p is bf16
    }
  }

  // P.V: wave w multiplies the value rows it loaded (its 32 positions of
  // each tile) from registers into partial outputs of every head (A rows
  // G..7 are zero; rows 8..15 repeat 0..7, and an output row depends on its
  // A row alone, so those rows land in output rows that are never read).
  mg_f32x4 oacc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) oacc[e] = mg_f32x4{0.f, 0.f, 0.f, 0.f};
  auto pv_tile = [&](const Vec8<bf16_t>(&v)[8], int mask, int t) {
    const re_u32x4 pa = *reinterpret_cast<const re_u32x4*>(pb + (size_t)(l16 & (kMgMaxG - 1)) * span + t * kMgTile +
                                                            wave * 32 + lq * 8);
    mg_pv_rows(oacc, pa, v, mask);
  };
  lds_barrier();  // the probabilities are written
#pragma unroll
  for (int i = 0; i < kMgChunk; ++i) pv_tile(vr[i], vmask[i], i);
  for (int c = 1; c < nchunks; ++c) {
#pragma unroll
    for (int i = 0; i < kMgChunk; ++i) vmask[i] = load_v(vr[i], c * kMgChunk + i);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < kMgChunk; ++i) pv_tile(vr[i], vmask[i], c * kMgChunk + i);
  }
  // the 8 waves' partials added in wave order
  float* part = reinterpret_cast<float*>(mg_smem + L.part);
  mg_put_partials(part, oacc, wave, lane);
  lds_barrier();
  for (int e = tid; e < G * kMgD; e += kMgThreads) {
    const int k = g * G * kMgD + e;
    static_cast<bf16_t*>(a.out)[a.packed_out ? xpack_index(b, k, a.heads * kMgD) : (size_t)b * a.heads * kMgD + k] =
        f_to_bf16(mg_sum_partials(part, e));
  }
}

// ---------------------------------------------------------------------------
// The matrix-core grouped attention split over the window: one workgroup per
// (row, KV head, tile of 256 positions), so a row's long window spreads over
// many CUs instead of one, with k_attn_mgroup's arithmetic and rounding
// points (only fp32 summation orders differ):
//   k_attn_msplit_scores: the tile's scores of the G heads on the matrix
//     cores (k_attn_mgroup's key loads and products), into sp_scores, with
//     each head's tile max m_t and e_t = sum of exp(s - m_t) into sp_stats;
//   k_attn_msplit_pv: each head's row max M = max_t m_t and sum
//     L = sum_t e_t exp(m_t - M) (tiles in order), p = bf16(exp(s - M) / L)
//     and the tile's P.V on the matrix cores into sp_part (fp32);
//   k_attn_split_sum: o = bf16(sum of the tiles' P.V in tile order).
// Block b = grp + groups * tile (grp = row * KV heads + KV head).
constexpr int kMsRows = kMgTile;  // positions per workgroup
struct MsLayout {
  size_t roff, sc, pb, part, stat, tabs, total;
};
// LDS of the two kernels: row offsets [256] int, then the scores kernel's
// scores [256][8] fp32, or the P.V kernel's probabilities [8][256] bf16, the
// waves' partial outputs [8][8][128] fp32 and head statistics [2][8] fp32;
// the block table last.
__host__ __device__ MsLayout msplit_layout(int blocks_per_row, bool pv) {
  MsLayout l;
  l.roff = 0;
  l.sc = l.roff + kMsRows * sizeof(int);
  l.pb = l.sc;
  l.part = l.pb + (size_t)kMgMaxG * kMsRows * sizeof(bf16_t);
  l.stat = l.part + kMgPartBytes;
  l.tabs = pv ? l.stat + 2 * kMgMaxG * sizeof(float) : l.sc + (size_t)kMsRows * kMgMaxG * sizeof(float);
  l.total = l.tabs + (size_t)blocks_per_row * sizeof(int);
  return l;
}
size_t msplit_smem_bytes(int blocks_per_row, bool pv) { return msplit_layout(blocks_per_row, pv).total; }

// Row offsets of the tile's positions (this KV head), -1 past the context or
// for a slot outside the cache.
template <bool P2>
__device__ __forceinline__ void msplit_offsets(const AttnArgs& a, const int* tabs, int* roff, int t, int g, int neff,
                                               int tid) {
  for (int jl = tid; jl < kMsRows; jl += kMgThreads) {
    const int j = t * kMsRows + jl;
    int o = -1;
    if (j < neff) {
      int blk, in_blk;
      block_of<P2>(j, a, blk, in_blk);
      const long long slot = (long long)tabs[min(blk, a.blocks_per_row - 1)] * a.block_size + in_blk;
      if (slot >= 0 && slot < a.slots) o = static_cast<int>((slot * a.kv_heads + g) * kMgD);
    }
    roff[jl] = o;
  }
}

template <bool P2>
__global__ void __launch_bounds__(kMgThreads) k_attn_msplit_scores(AttnArgs a) {
  extern __shared__ __align__(16) unsigned char ms_smem[];
  __shared__ float red[kMgWaves][kMgMaxG];
  const int G = a.heads / a.kv_heads, W = a.window;
  const int groups = a.B * a.kv_heads;
  const int t = blockIdx.x / groups, grp = blockIdx.x - t * groups;
  const int b = grp / a.kv_heads, g = grp - b * a.kv_heads;
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_index(tid);
  const int l16 = lane & 15, lq = lane >> 4;
  const MsLayout L = msplit_layout(a.blocks_per_row, false);
  int* roff = reinterpret_cast<int*>(ms_smem + L.roff);
  float* sc = reinterpret_cast<float*>(ms_smem + L.sc);  // [256][kMgMaxG]
  int* tabs = reinterpret_cast<int*>(ms_smem + L.tabs);
  const int32_t stop = a.done != nullptr ? request_flag(a.done) : 0;
  const int n = a.len[b];
  const bool uniform = n <= 0;
  const int neff = uniform ? W : min(n, W);
  if (flag_set(stop) || t * kMsRows >= neff) return;  // uniform over the workgroup
  for (int e = tid; e < a.blocks_per_row; e += kMgThreads) tabs[e] = a.table[(size_t)b * a.blocks_per_row + e];
  mg_bf16x8 qf[4];
  {
    const bf16_t* qrow = static_cast<const bf16_t*>(a.q) + ((size_t)b * a.heads + g * G + min(l16, G - 1)) * kMgD;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const re_u32x4 v = *reinterpret_cast<const re_u32x4*>(qrow + kk * 32 + lq * 8);
      qf[kk] = __builtin_bit_cast(mg_bf16x8, l16 < G ? v : re_u32x4{0u, 0u, 0u, 0u});
    }
  }
  lds_barrier();
  msplit_offsets<P2>(a, tabs, roff, t, g, neff, tid);
  lds_barrier();
  // keys: wave w, step q reads positions (2 w + q) * 16 + l % 16 of the tile
  const bf16_t* KC = static_cast<const bf16_t*>(a.key_cache);
  re_u32x4 kf[2][4];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int off = roff[(2 * wave + q) * 16 + l16];
    const bf16_t* row = KC + (off >= 0 ? off : 0);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) kf[q][kk] = *reinterpret_cast<const re_u32x4*>(row + kk * 32 + lq * 8);
  }
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    mg_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(mg_bf16x8, kf[q][kk]), qf[kk], acc, 0, 0, 0);
    // value v of lane l: position 4 (l / 16) + v of the group, head l % 16
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int jl = (2 * wave + q) * 16 + lq * 4 + v;
      // ExactQk output is bf16, then the bf16 quotient by sqrt(128)
      float s = round_bf16(div_sqrt128_bf16(round_bf16(acc[v])));
      if (uniform) s = -3.38953139e38f;  // every position masked to bf16 min
      // a missing row (slot outside the cache) is a zero key: score 0
      if (l16 < kMgMaxG) sc[(size_t)jl * kMgMaxG + l16] = roff[jl] >= 0 || uniform ? s : 0.f;
    }
  }
  lds_barrier();
  // Threads 0-255 own one position each (all heads); the rest hold nothing.
  const int jl = tid & (kMsRows - 1);
  const bool in = tid < kMsRows && t * kMsRows + jl < neff;
  float v[kMgMaxG];
  {
    const re_f32x4 lo = *reinterpret_cast<const re_f32x4*>(sc + (size_t)jl * kMgMaxG);
    const re_f32x4 hi = *reinterpret_cast<const re_f32x4*>(sc + (size_t)jl * kMgMaxG + 4);
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      v[h] = lo[h];
      v[h + 4] = hi[h];
    }
  }
  float m[kMgMaxG];
#pragma unroll
  for (int h = 0; h < kMgMaxG; ++h) m[h] = in ? v[h] : -INFINITY;
  wave_max_n<kMgMaxG>(m);
  if (lane == 0)
#pragma unroll
    for (int h = 0; h < kMgMaxG; ++h) red[wave][h] = m[h];
  lds_barrier();
  float mx[kMgMaxG];
#pragma unroll
  for (int h = 0; h < kMgMaxG; ++h) {
    mx[h] = red[0][h];
#pragma unroll
    for (int w = 1; w < kMgWaves; ++w) mx[h] = fmaxf(mx[h], red[w][h]);
  }
  lds_barrier();  // every max read before red is reused
  float e[kMgMaxG];
#pragma unroll
  for (int h = 0; h < kMgMaxG; ++h) e[h] = in ? expf(v[h] - mx[h]) : 0.f;
  wave_sum_n<kMgMaxG>(e);
  if (lane == 0)
#pragma unroll
    for (int h = 0; h < kMgMaxG; ++h) red[wave][h] = e[h];
  lds_barrier();
  const size_t row0 = (size_t)b * a.heads + g * G;  // (row, first head of the group)
  if (tid == 0) {
#pragma unroll
    for (int h = 0; h < kMgMaxG; ++h) {
      if (h < G) {
        float total = 0.f;
#pragma unroll
        for (int w = 0; w < kMgWaves; ++w) total += red[w][h];
        float* st = a.sp_stats + ((row0 + h) * a.split_tiles + t) * 2;
        st[0] = mx[h];
        st[1] = total;
      }
    }
  }
  if (in) {
#pragma unroll
    for (int h = 0; h < kMgMaxG; ++h)
      if (h < G) a.sp_scores[(row0 + h) * W + t * kMsRows + jl] = v[h];
  }
}

template <bool P2>
__global__ void __launch_bounds__(kMgThreads) k_attn_msplit_pv(AttnArgs a) {
  extern __shared__ __align__(16) unsigned char ms_smem[];
  const int G = a.heads / a.kv_heads, W = a.window;
  const int groups = a.B * a.kv_heads;
  const int t = blockIdx.x / groups, grp = blockIdx.x - t * groups;
  const int b = grp / a.kv_heads, g = grp - b * a.kv_heads;
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_index(tid);
  const int l16 = lane & 15, lq = lane >> 4;
  const MsLayout L = msplit_layout(a.blocks_per_row, true);
  int* roff = reinterpret_cast<int*>(ms_smem + L.roff);
  bf16_t* pb = reinterpret_cast<bf16_t*>(ms_smem + L.pb);  // [kMgMaxG][256]
  float* part = reinterpret_cast<float*>(ms_smem + L.part);  // [8 waves][8][128]
  float* stat = reinterpret_cast<float*>(ms_smem + L.stat);  // [max, 1 / sum][kMgMaxG]
  int* tabs = reinterpret_cast<int*>(ms_smem + L.tabs);
  const int32_t stop = a.done != nullptr ? request_flag(a.done) : 0;
  const int n = a.len[b];
  const int neff = n <= 0 ? W : min(n, W);
  if (flag_set(stop) || t * kMsRows >= neff) return;  // uniform over the workgroup
  const int nt = (neff + kMsRows - 1) / kMsRows;
  const size_t row0 = (size_t)b * a.heads + g * G;
  for (int e = tid; e < a.blocks_per_row; e += kMgThreads) tabs[e] = a.table[(size_t)b * a.blocks_per_row + e];
  // Each head's row max and sum from the tiles' statistics: wave h < G
  // reduces head h (tiles lane, lane + 64, ... then the wave in a fixed order).
  if (wave < G) {
    const float* st = a.sp_stats + (row0 + wave) * a.split_tiles * 2;
    float m = -INFINITY;
    for (int i = lane; i < nt; i += 64) m = fmaxf(m, st[2 * i]);
    m = wave_max_dpp(m);
    float e = 0.f;
    for (int i = lane; i < nt; i += 64) e += st[2 * i + 1] * expf(st[2 * i] - m);
    e = wave_sum_dpp(e);
    if (lane == 0) {
      stat[wave] = m;
      stat[kMgMaxG + wave] = 1.0f / e;
    }
  }
  lds_barrier();
  msplit_offsets<P2>(a, tabs, roff, t, g, neff, tid);
  lds_barrier();
  // value rows p0 .. p0+7 of the tile, chunk l16 (elements 8 l16 ..+8); bit i
  // of the mask marks row i valid (invalid rows enter as zero)
  const bf16_t* VC = static_cast<const bf16_t*>(a.value_cache);
  const int p0 = wave * 32 + lq * 8;
  Vec8<bf16_t> vr[8];
  int mask = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int off = roff[p0 + i];
    vr[i] = Vec8<bf16_t>::load_cached(VC + (off >= 0 ? off : 0) + l16 * 8);
    mask |= (off >= 0 ? 1 : 0) << i;
  }
  // probabilities of the tile: thread t covers position t % 256 of heads
  // t / 256, t / 256 + 2, ... (zero past the context and for head slots >= G)
  for (int i = tid; i < kMgMaxG * kMsRows; i += kMgThreads) {
    const int h = i / kMsRows, jl = i - h * kMsRows;
    const int j = t * kMsRows + jl;
    float p = 0.f;
    if (h < G && j < neff) p = round_bf16(expf(a.sp_scores[(row0 + h) * W + j] - stat[h]) * stat[kMgMaxG + h]);
    pb[(size_t)h * kMsRows + jl] = f_to_bf16(p);  // exact: p is bf16
  }
  // P.V from registers: wave w multiplies its own 32 positions (A rows G..7
  // zero, rows 8..15 reach only output rows that are never read), then the
  // 8 waves' partials are added in wave order.
  lds_barrier();  // the probabilities are written
  mg_f32x4 oacc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) oacc[e] = mg_f32x4{0.f, 0.f, 0.f, 0.f};
  const re_u32x4 pa = *reinterpret_cast<const re_u32x4*>(pb + (size_t)(l16 & (kMgMaxG - 1)) * kMsRows + wave * 32 + lq * 8);
  mg_pv_rows(oacc, pa, vr, mask);
  mg_put_partials(part, oacc, wave, lane);
  lds_barrier();
  for (int e = tid; e < G * kMgD; e += kMgThreads) {
    const int h = e / kMgD, d = e - h * kMgD;
    a.sp_part[((row0 + h) * a.split_tiles + t) * kMgD + d] = mg_sum_partials(part, e);
  }
}

}  // namespace

bool group_attention_fits(const Dims& d) {
  return d.dtype_bytes == 2 && d.head_dim == kGrpD && d.groups() <= kGrpMaxG &&
         group_smem_bytes(d.groups(), d.capacity, d.blocks_per_row) <= 96 * 1024;
}
bool group_attention_default(const Dims& d) { return group_attention_fits(d) && d.batch * d.kv_heads >= 64; }
bool group_attention_mfma_fits(const Dims& d) {
  return group_attention_fits(d) && d.groups() <= kMgMaxG && d.head_dim == kMgD &&
         mgroup_smem_bytes(d.groups(), d.capacity, d.blocks_per_row) <= 150 * 1024;
}
// The split matrix-core version: its LDS does not grow with the window.
bool group_attention_msplit_fits(const Dims& d) {
  return d.dtype_bytes == 2 && d.head_dim == kMgD && d.groups() <= kMgMaxG &&
         msplit_smem_bytes(d.blocks_per_row, true) <= 150 * 1024;
}

namespace {

size_t smem_bytes(int window, int blocks_per_row) {
  return (size_t)window * sizeof(float) + (size_t)kAttnThreads * 8 * sizeof(float) + (size_t)blocks_per_row * sizeof(int);
}

// The window-split attention's three launches.
template <typename T, int D>
hipError_t launch_split_t(const AttnArgs& a, hipStream_t stream) {
  const int grid = a.B * a.heads * a.split_tiles;
  const size_t smem = (size_t)a.blocks_per_row * sizeof(int);
  if (a.bs_shift >= 0 && (1 << a.bs_shift) == a.block_size) {
    k_attn_split_scores<T, D, true><<<grid, kAttnThreads, smem, stream>>>(a);
    k_attn_split_pv<T, D, true><<<grid, kAttnThreads, smem, stream>>>(a);
  } else {
    k_attn_split_scores<T, D, false><<<grid, kAttnThreads, smem, stream>>>(a);
    k_attn_split_pv<T, D, false><<<grid, kAttnThreads, smem, stream>>>(a);
  }
  k_attn_split_sum<T><<<(a.B * a.heads * D + 255) / 256, 256, 0, stream>>>(a);
  return hipGetLastError();
}

// Power-of-two block sizes take the shift-and-mask position arithmetic.
template <typename T, int D>
hipError_t launch_t(const AttnArgs& a, hipStream_t stream) {
  if (a.split_tiles > 0) {
    if (a.sp_scores == nullptr || a.sp_stats == nullptr || a.sp_part == nullptr ||
        a.split_tiles * kAttnTile < a.window)
      return hipErrorInvalidValue;
    return launch_split_t<T, D>(a, stream);
  }
  const size_t smem = smem_bytes(a.window, a.blocks_per_row);
  if (a.bs_shift >= 0 && (1 << a.bs_shift) == a.block_size)
    k_attn<T, D, true><<<a.B * a.heads, kAttnThreads, smem, stream>>>(a);
  else
    k_attn<T, D, false><<<a.B * a.heads, kAttnThreads, smem, stream>>>(a);
  return hipGetLastError();
}

// Dynamic LDS the launches of this engine need (the window's scores grow
// with the capacity); the static reduction scratch comes on top of it.
template <typename T, int D>
hipError_t allow_t(size_t bytes) {
  const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(k_attn<T, D, false>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes));
  if (e != hipSuccess) return e;
  return hipFuncSetAttribute(reinterpret_cast<const void*>(k_attn<T, D, true>),
                             hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes));
}

}  // namespace

size_t attention_lds_bytes(const Dims& d) { return smem_bytes(d.capacity, d.blocks_per_row); }

hipError_t prepare_attention(const Dims& d) {
  if (d.head_dim != 64 && d.head_dim != 128 && d.head_dim != 256) return hipErrorInvalidValue;
  if (group_attention_fits(d)) {
    const int bytes = static_cast<int>(group_smem_bytes(d.groups(), d.capacity, d.blocks_per_row));
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(k_attn_group<true>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e == hipSuccess)
      e = hipFuncSetAttribute(reinterpret_cast<const void*>(k_attn_group<false>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e != hipSuccess) return e;
  }
  if (group_attention_mfma_fits(d)) {
    const int bytes = static_cast<int>(mgroup_smem_bytes(d.groups(), d.capacity, d.blocks_per_row));
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(k_attn_mgroup<true>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e == hipSuccess)
      e = hipFuncSetAttribute(reinterpret_cast<const void*>(k_attn_mgroup<false>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e != hipSuccess) return e;
  }
  if (group_attention_msplit_fits(d)) {
    const int pv_bytes = static_cast<int>(msplit_smem_bytes(d.blocks_per_row, true));
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(k_attn_msplit_pv<true>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, pv_bytes);
    if (e == hipSuccess)
      e = hipFuncSetAttribute(reinterpret_cast<const void*>(k_attn_msplit_pv<false>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, pv_bytes);
    if (e != hipSuccess) return e;
  }
  const size_t bytes = attention_lds_bytes(d);
  if (d.dtype_bytes == 2) {
    if (d.head_dim == 64) return allow_t<bf16_t, 64>(bytes);
    if (d.head_dim == 128) return allow_t<bf16_t, 128>(bytes);
    return allow_t<bf16_t, 256>(bytes);
  }
  if (d.head_dim == 64) return allow_t<float, 64>(bytes);
  if (d.head_dim == 128) return allow_t<float, 128>(bytes);
  return allow_t<float, 256>(bytes);
}

hipError_t launch_attention(const AttnArgs& a, const Dims& d, hipStream_t stream) {
  if (a.grouped == 2 && a.split_tiles > 0 && group_attention_msplit_fits(d)) {
    if (a.sp_scores == nullptr || a.sp_stats == nullptr || a.sp_part == nullptr ||
        a.split_tiles * kMsRows < a.window)
      return hipErrorInvalidValue;
    const int grid = a.B * a.kv_heads * a.split_tiles;
    const size_t s_smem = msplit_smem_bytes(a.blocks_per_row, false), p_smem = msplit_smem_bytes(a.blocks_per_row, true);
    if (a.bs_shift >= 0 && (1 << a.bs_shift) == a.block_size) {
      k_attn_msplit_scores<true><<<grid, kMgThreads, s_smem, stream>>>(a);
      k_attn_msplit_pv<true><<<grid, kMgThreads, p_smem, stream>>>(a);
    } else {
      k_attn_msplit_scores<false><<<grid, kMgThreads, s_smem, stream>>>(a);
      k_attn_msplit_pv<false><<<grid, kMgThreads, p_smem, stream>>>(a);
    }
    k_attn_split_sum<bf16_t><<<(a.B * a.heads * kMgD + 255) / 256, 256, 0, stream>>>(a);
    return hipGetLastError();
  }
  if (a.grouped == 2 && group_attention_mfma_fits(d)) {
    const size_t smem = mgroup_smem_bytes(d.groups(), a.window, a.blocks_per_row);
    if (a.bs_shift >= 0 && (1 << a.bs_shift) == a.block_size)
      k_attn_mgroup<true><<<a.B * a.kv_heads, kMgThreads, smem, stream>>>(a);
    else
      k_attn_mgroup<false><<<a.B * a.kv_heads, kMgThreads, smem, stream>>>(a);
    return hipGetLastError();
  }
  if (a.grouped && group_attention_fits(d)) {
    const size_t smem = group_smem_bytes(d.groups(), a.window, a.blocks_per_row);
    if (a.bs_shift >= 0 && (1 << a.bs_shift) == a.block_size)
      k_attn_group<true><<<a.B * a.kv_heads, kGrpThreads, smem, stream>>>(a);
    else
      k_attn_group<false><<<a.B * a.kv_heads, kGrpThreads, smem, stream>>>(a);
    return hipGetLastError();
  }
  if (d.dtype_bytes == 2) {
    if (d.head_dim == 64) return launch_t<bf16_t, 64>(a, stream);
    if (d.head_dim == 128) return launch_t<bf16_t, 128>(a, stream);
    return launch_t<bf16_t, 256>(a, stream);
  }
  if (d.head_dim == 64) return launch_t<float, 64>(a, stream);
  if (d.head_dim == 128) return launch_t<float, 128>(a, stream);
  return launch_t<float, 256>(a, stream);
}

}  // namespace re
