// GQA paged decode attention of the resident decode epoch (gfx950), one
// workgroup per (batch row, KV head) (batched_decoder_step.py:265-279, 334-379):
//   window positions j < W gathered through the block table;
//   s_j = bf16(bf16(q.k_j) / sqrt(d)) -- ExactQk is bf16-out; fp32 models keep
//   the fp32 product, then the bf16 rounding of the scaled score;
//   masked (j >= seq_len) positions contribute exp(bf16_min - max) = 0, so the
//   softmax runs over j < min(seq_len, W); a row with seq_len <= 0 has every
//   position masked and averages the whole window uniformly, as the reference;
//   p = bf16(softmax_fp32(s)); o = T(sum_j p_j v_j) with fp32 accumulation.
//
// Positions are processed in tiles of 64: the query heads and the first tile's
// keys and values are requested together (one memory round trip for the
// common short context), key rows are staged in LDS with a 16-byte pad so the
// per-lane row reads hit distinct banks, and the next tile's loads are issued
// before the current tile is consumed.
#include "re_device.h"
#include "re_layout.h"

namespace re {
namespace {

constexpr int kTile = 64;
constexpr int kThreads = 256;

template <typename T, int D>
struct AttnShape {
  static constexpr int kVecRow = D / 8;                       // Vec8 per key/value row
  static constexpr int kTileVecs = kTile * kVecRow;           // Vec8 per tile
  static constexpr int kPerThread = (kTileVecs + kThreads - 1) / kThreads;
  static constexpr int kPad = 16 / sizeof(T);                 // elements of padding per staged row
  static constexpr int kRow = D + kPad;                       // staged row stride (elements)
};

__device__ __forceinline__ long long window_slot(const int32_t* tab, int j, int block_size) {
  return (long long)tab[j / block_size] * block_size + (j % block_size);
}

// Issue the loads of positions [t0, t0 + kTile) of one KV head (rows past
// neff or outside the cache read as zero).
template <typename T, int D, int NPT>
__device__ __forceinline__ void load_tile(Vec8<T> (&v)[NPT], const T* cache, const int32_t* tab,
                                          int t0, int neff, const AttnArgs& a, int g) {
  using S = AttnShape<T, D>;
#pragma unroll
  for (int i = 0; i < S::kPerThread; ++i) {
    const int idx = threadIdx.x + kThreads * i;
    const int jj = idx / S::kVecRow, c = idx - jj * S::kVecRow;
    const int j = t0 + jj;
    v[i] = Vec8<T>{};
    if (idx < S::kTileVecs && j < neff) {
      const long long slot = window_slot(tab, j, a.block_size);
      if (slot >= 0 && slot < a.slots) v[i] = Vec8<T>::load_cached(cache + ((size_t)slot * a.kv_heads + g) * D + c * 8);
    }
  }
}

template <typename T, int D, int NPT>
__device__ __forceinline__ void store_tile(const Vec8<T> (&v)[NPT], T* tile) {
  using S = AttnShape<T, D>;
#pragma unroll
  for (int i = 0; i < S::kPerThread; ++i) {
    const int idx = threadIdx.x + kThreads * i;
    if (idx < S::kTileVecs) {
      const int jj = idx / S::kVecRow, c = idx - jj * S::kVecRow;
      *reinterpret_cast<Vec8<T>*>(tile + jj * S::kRow + c * 8) = v[i];
    }
  }
}

// Tiles gi*kGroupTiles .. +kGroupTiles-1 (those below ntiles) into registers.
constexpr int kGroupTiles = 4;

template <typename T, int D, int NPT>
__device__ __forceinline__ void load_group(Vec8<T> (&v)[kGroupTiles][NPT], const T* cache, const int32_t* tab, int gi,
                                           int ntiles, int neff, const AttnArgs& a, int g) {
#pragma unroll
  for (int tt = 0; tt < kGroupTiles; ++tt) {
    const int t = gi * kGroupTiles + tt;
    if (t < ntiles) load_tile<T, D>(v[tt], cache, tab, t * kTile, neff, a, g);
  }
}

template <typename T, int D>
__global__ void __launch_bounds__(kThreads) k_attn(AttnArgs a) {
  using S = AttnShape<T, D>;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const int G = a.heads / a.kv_heads, W = a.window;
  float* qs = reinterpret_cast<float*>(smem_raw);   // [G, D]
  float* sc = qs + G * D;                            // [G, W]
  T* kt = reinterpret_cast<T*>(sc + G * W);          // [kTile, kRow] keys, then values
  const int b = blockIdx.x, g = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nwaves = kThreads / 64;
  const int n = a.len[b];
  const bool uniform = n <= 0;
  const int neff = uniform ? W : min(n, W);
  const int ntiles = (neff + kTile - 1) / kTile;
  const T* Q = static_cast<const T*>(a.q) + (size_t)b * a.heads * D + (size_t)g * G * D;
  const T* KC = static_cast<const T*>(a.key_cache);
  const T* VC = static_cast<const T*>(a.value_cache);
  const int32_t* tab = a.table + (size_t)b * a.blocks_per_row;

  // One round trip: query heads and the keys and values of the first
  // kGroupTiles tiles (256 positions) are requested together.
  Vec8<T> qv = Vec8<T>{};
  const int qvecs = G * D / 8;
  if (tid < qvecs) qv = Vec8<T>::load_cached(Q + tid * 8);
  Vec8<T> kr[kGroupTiles][S::kPerThread], vr[kGroupTiles][S::kPerThread];
  load_group<T, D>(kr, KC, tab, 0, ntiles, neff, a, g);
  load_group<T, D>(vr, VC, tab, 0, ntiles, neff, a, g);
  if (a.done != nullptr && __builtin_nontemporal_load(a.done) != 0) return;  // read while loads fly
  if (tid < qvecs) {
#pragma unroll
    for (int e = 0; e < 8; ++e) qs[tid * 8 + e] = qv.get(e);
  }
  const float scale_div = sqrtf(static_cast<float>(D));
  const int ngroups = (ntiles + kGroupTiles - 1) / kGroupTiles;
  // Pass 1: scores of every tile.
  for (int gi = 0; gi < ngroups; ++gi) {
    if (gi > 0) load_group<T, D>(kr, KC, tab, gi, ntiles, neff, a, g);
#pragma unroll
    for (int tt = 0; tt < kGroupTiles; ++tt) {
      const int t = gi * kGroupTiles + tt;
      if (t < ntiles) {
        store_tile<T, D>(kr[tt], kt);
        __syncthreads();
        const int t0 = t * kTile;
        for (int p = tid; p < G * kTile; p += kThreads) {
          const int h = p / kTile, jj = p - h * kTile, j = t0 + jj;
          if (j < neff) {
            const T* krow = kt + jj * S::kRow;
            const float* qrow = qs + h * D;
            float s = 0.f;
#pragma unroll
            for (int c = 0; c < S::kVecRow; ++c) {
              const Vec8<T> k8 = Vec8<T>::load_cached(krow + c * 8);
#pragma unroll
              for (int e = 0; e < 8; ++e) s = fmaf(qrow[c * 8 + e], k8.get(e), s);
            }
            if constexpr (sizeof(T) == 2) s = round_bf16(s);  // ExactQk output is bf16
            s = round_bf16(s / scale_div);
            if (uniform) s = -3.38953139e38f;  // every position masked to bf16 min
            sc[h * W + j] = s;
          }
        }
        __syncthreads();
      }
    }
  }
  // Softmax per head (fp32), probabilities rounded to bf16.
  for (int h = wave; h < G; h += nwaves) {
    float mx = -INFINITY;
    for (int j = lane; j < neff; j += 64) mx = fmaxf(mx, sc[h * W + j]);
    mx = wave_max(mx);
    float sum = 0.f;
    for (int j = lane; j < neff; j += 64) sum += expf(sc[h * W + j] - mx);
    sum = wave_sum(sum);
    const float inv = 1.0f / sum;
    for (int j = lane; j < neff; j += 64) sc[h * W + j] = round_bf16(expf(sc[h * W + j] - mx) * inv);
  }
  // Pass 2: P.V.  Thread (dd, part) accumulates heads h = part, part + nsplit, ...
  constexpr int kSplit = kThreads / D;  // D divides 256
  const int dd = tid % D, part = tid / D;
  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.f;
  for (int gi = 0; gi < ngroups; ++gi) {
    if (gi > 0) load_group<T, D>(vr, VC, tab, gi, ntiles, neff, a, g);
#pragma unroll
    for (int tt = 0; tt < kGroupTiles; ++tt) {
      const int t = gi * kGroupTiles + tt;
      if (t < ntiles) {
        __syncthreads();  // scores final / previous tile consumed
        store_tile<T, D>(vr[tt], kt);
        __syncthreads();
        const int t0 = t * kTile;
        const int tn = min(kTile, neff - t0);
        for (int jj = 0; jj < tn; ++jj) {
          const float v = Elt<T>::f(kt[jj * S::kRow + dd]);
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const int h = part + i * kSplit;
            if (i * kSplit < 8 && h < G) acc[i] = fmaf(sc[h * W + t0 + jj], v, acc[i]);
          }
        }
      }
    }
  }
  T* O = static_cast<T*>(a.out) + (size_t)b * a.heads * D + (size_t)g * G * D;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int h = part + i * kSplit;
    if (i * kSplit < 8 && h < G) O[h * D + dd] = Elt<T>::t(acc[i]);
  }
}

template <typename T, int D>
hipError_t launch_t(const AttnArgs& a, int G, hipStream_t stream) {
  using S = AttnShape<T, D>;
  const size_t smem = (size_t)(G * D + G * a.window) * sizeof(float) + (size_t)kTile * S::kRow * sizeof(T);
  k_attn<T, D><<<dim3(a.B, a.kv_heads), kThreads, smem, stream>>>(a);
  return hipGetLastError();
}

template <typename T, int D>
hipError_t allow_t() {
  return hipFuncSetAttribute(reinterpret_cast<const void*>(k_attn<T, D>), hipFuncAttributeMaxDynamicSharedMemorySize,
                             160 * 1024);
}

}  // namespace

size_t attention_lds_bytes(const Dims& d) {
  const int row = d.head_dim + 16 / d.dtype_bytes;
  return (size_t)(d.groups() * d.head_dim + d.groups() * d.capacity) * sizeof(float) +
         (size_t)kTile * row * d.dtype_bytes;
}

hipError_t prepare_attention(const Dims& d) {
  if (d.dtype_bytes == 2) {
    if (d.head_dim == 64) return allow_t<bf16_t, 64>();
    if (d.head_dim == 128) return allow_t<bf16_t, 128>();
    return allow_t<bf16_t, 256>();
  }
  if (d.head_dim == 64) return allow_t<float, 64>();
  if (d.head_dim == 128) return allow_t<float, 128>();
  return allow_t<float, 256>();
}

hipError_t launch_attention(const AttnArgs& a, const Dims& d, hipStream_t stream) {
  const int G = d.groups();
  if (d.dtype_bytes == 2) {
    if (d.head_dim == 64) return launch_t<bf16_t, 64>(a, G, stream);
    if (d.head_dim == 128) return launch_t<bf16_t, 128>(a, G, stream);
    return launch_t<bf16_t, 256>(a, G, stream);
  }
  if (d.head_dim == 64) return launch_t<float, 64>(a, G, stream);
  if (d.head_dim == 128) return launch_t<float, 128>(a, G, stream);
  return launch_t<float, 256>(a, G, stream);
}

}  // namespace re
