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

  const int32_t stop = a.done != nullptr ? __builtin_nontemporal_load(a.done) : 0;
  for (int e = tid; e < a.blocks_per_row; e += kGrpThreads) tabs[e] = a.table[(size_t)b * a.blocks_per_row + e];
  Vec8<bf16_t> qv[kGrpMaxG];
#pragma unroll
  for (int h = 0; h < kGrpMaxG; ++h)
    qv[h] = Vec8<bf16_t>::load_cached(static_cast<const bf16_t*>(a.q) +
                                      ((size_t)b * a.heads + g * G + min(h, G - 1)) * kGrpD + c * 8);
  lds_barrier();
  if (stop != 0) return;  // uniform

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
  const float scale_div = sqrtf(static_cast<float>(kGrpD));
  auto score_tile = [&](const Vec8<bf16_t>(&kr)[kGrpRows], const int (&off)[kGrpRows], int t) {
#pragma unroll
    for (int i = 0; i < kGrpRows; ++i) {
      float part[kGrpMaxG];
#pragma unroll
      for (int h = 0; h < kGrpMaxG; ++h) part[h] = off[i] >= 0 ? dot8(kr[i], qv[h], 0.f) : 0.f;  // missing row: zero key
#pragma unroll
      for (int h = 0; h < kGrpMaxG; ++h) part[h] += __shfl_xor(part[h], 8, 64);
      group_reduce_transpose<kGrpMaxG>(part, c & 7);
      const int j = t * kGrpTile + i * kGrpSlots + r;
      float s = round_bf16(part[0]);  // ExactQk output is bf16
      s = round_bf16(s / scale_div);
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
      acc[h][e] += __shfl_xor(acc[h][e], 16, 64);
      acc[h][e] += __shfl_xor(acc[h][e], 32, 64);
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
    static_cast<bf16_t*>(a.out)[((size_t)b * a.heads + g * G + h) * kGrpD + d] = f_to_bf16(v);
  }
}

}  // namespace

bool group_attention_fits(const Dims& d) {
  return d.dtype_bytes == 2 && d.head_dim == kGrpD && d.groups() <= kGrpMaxG &&
         group_smem_bytes(d.groups(), d.capacity, d.blocks_per_row) <= 96 * 1024;
}
bool group_attention_default(const Dims& d) { return group_attention_fits(d) && d.batch * d.kv_heads >= 64; }

namespace {

size_t smem_bytes(int window, int blocks_per_row) {
  return (size_t)window * sizeof(float) + (size_t)kAttnThreads * 8 * sizeof(float) + (size_t)blocks_per_row * sizeof(int);
}

// Power-of-two block sizes take the shift-and-mask position arithmetic.
template <typename T, int D>
hipError_t launch_t(const AttnArgs& a, hipStream_t stream) {
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
