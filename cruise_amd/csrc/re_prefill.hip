// Batched prefill kernels (gfx950): the decoder over all prompt tokens of
// several rows at once, M = tokens.  Same operations and rounding points as
// the decode step (batched_decoder_step.py:277-403), laid out for large M:
//
//   embed      token rows + per-token RoPE table
//   rmsnorm    one workgroup per token
//   GEMM       C[M,N] = A[M,K] W[N,K]^T, both operands K-contiguous.
//              bf16: MFMA v_mfma_f32_32x32x16_bf16, 128x128 workgroup tiles
//              (four waves of 64x64), K in steps of 32 through double-buffered
//              LDS, fp32 accumulation; epilogues "T(acc + bias)" and the
//              residual "T(h + T(acc))".  fp32 models: an LDS-tiled FMA GEMM.
//   qkv post   RoPE of q and k in place, K/V rows to their paged slots
//   attention  causal within each row's prompt.  bf16, head_dim 128: MFMA
//              for Q K^T and P V per (64-query tile, head), the bf16 scores of
//              the whole tile kept in LDS so the softmax is the exact
//              two-pass one of the decode step; otherwise one workgroup per
//              (token, head).
//   SwiGLU     elementwise on the gate and up products
#include <algorithm>

#include "re_device.h"
#include "re_layout.h"

namespace re {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

__device__ __forceinline__ bf16x8_t lds_frag(const bf16_t* p) {
  return __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const re_u32x4*>(p));
}

// ---------------------------------------------------------------------------
// Row kernels
// ---------------------------------------------------------------------------
template <typename T>
__global__ void __launch_bounds__(256) k_pf_embed(PrefillRows a) {
  const int m = blockIdx.x, tid = threadIdx.x;
  long long t = a.token[m];
  if (t < 0 || t >= a.V) t = 0;  // validated on the host; reads stay in bounds
  const int half = a.head_dim / 2;
  for (int j = tid; j < half; j += blockDim.x) {
    const float ang = static_cast<float>(a.pos[m]) * a.inv_freq[j];
    a.rope[((size_t)m * half + j) * 2] = Elt<T>::r(cosf(ang));
    a.rope[((size_t)m * half + j) * 2 + 1] = Elt<T>::r(sinf(ang));
  }
  const T* src = static_cast<const T*>(a.embedding) + (size_t)t * a.H;
  T* dst = static_cast<T*>(a.hidden) + (size_t)m * a.H;
  for (int c = tid; c < a.H / 8; c += blockDim.x)
    *reinterpret_cast<Vec8<T>*>(dst + c * 8) = Vec8<T>::load_cached(src + c * 8);
}

// RMSNorm (batched_decoder_step.py:224-229): fp32 mean of squares, rsqrt,
// cast to T, T x T product with the weight.
template <typename T>
__global__ void __launch_bounds__(256) k_pf_rmsnorm(const void* x, const void* w, void* y, int H, float eps) {
  __shared__ float red[4];
  const int m = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const T* xr = static_cast<const T*>(x) + (size_t)m * H;
  const T* wr = static_cast<const T*>(w);
  T* yr = static_cast<T*>(y) + (size_t)m * H;
  float s = 0.f;
  for (int c = tid; c < H / 8; c += 256) {
    const Vec8<T> v = Vec8<T>::load_cached(xr + c * 8);
#pragma unroll
    for (int e = 0; e < 8; ++e) s = fmaf(v.get(e), v.get(e), s);
  }
  s = wave_sum(s);
  if (lane == 0) red[wave] = s;
  __syncthreads();
  const float rs = rsqrtf((red[0] + red[1] + red[2] + red[3]) / static_cast<float>(H) + eps);
  for (int c = tid; c < H / 8; c += 256) {
    const Vec8<T> v = Vec8<T>::load_cached(xr + c * 8);
    const Vec8<T> g = Vec8<T>::load_cached(wr + c * 8);
    float out[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = Elt<T>::r(Elt<T>::r(v.get(e) * rs) * g.get(e));
    *reinterpret_cast<Vec8<T>*>(yr + c * 8) = Vec8<T>::from_floats(out);
  }
}

// gate = silu(g), product with up (batched_decoder_step.py:391-398); g and up
// arrive rounded to T by their GEMMs.
template <typename T>
__global__ void __launch_bounds__(256) k_pf_swiglu(const void* gate, const void* up, void* out, long long n) {
  const T* g = static_cast<const T*>(gate);
  const T* u = static_cast<const T*>(up);
  T* o = static_cast<T*>(out);
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long long)gridDim.x * blockDim.x) {
    const float gv = Elt<T>::f(g[i]);
    const float sg = Elt<T>::r(gv / (1.0f + expf(-gv)));
    o[i] = Elt<T>::t(Elt<T>::r(sg * Elt<T>::f(u[i])));
  }
}

// RoPE of q and k (rows already rounded with their bias) in place, and the
// paged slot write of k and v (batched_decoder_step.py:231-264, 323-324).
template <typename T>
__global__ void __launch_bounds__(256) k_pf_qkv_post(PrefillQkv a) {
  const int m = blockIdx.x;
  const int half = a.head_dim / 2;
  const int nq = a.heads, nkv = a.kv_heads;
  T* row = static_cast<T*>(a.qkv) + (size_t)m * a.ld;
  const int s = a.slot[m];
  for (int idx = threadIdx.x; idx < (nq + 2 * nkv) * half; idx += blockDim.x) {
    const int hg = idx / half, j = idx - hg * half;
    T* p = row + (size_t)hg * a.head_dim;
    float oa = Elt<T>::f(p[j]), ob = Elt<T>::f(p[j + half]);
    if (hg < nq + nkv) {
      const float c = a.rope[((size_t)m * half + j) * 2], sn = a.rope[((size_t)m * half + j) * 2 + 1];
      const float qa = oa, qb = ob;
      oa = Elt<T>::r(Elt<T>::r(qa * c) + Elt<T>::r(-qb * sn));
      ob = Elt<T>::r(Elt<T>::r(qb * c) + Elt<T>::r(qa * sn));
      p[j] = Elt<T>::t(oa);
      p[j + half] = Elt<T>::t(ob);
    }
    if (hg >= nq && s >= 0 && s < a.slots) {
      const bool is_key = hg < nq + nkv;
      const int kvh = is_key ? hg - nq : hg - nq - nkv;
      T* cache = static_cast<T*>(is_key ? a.key_cache : a.value_cache) + ((size_t)s * nkv + kvh) * a.head_dim;
      cache[j] = Elt<T>::t(oa);
      cache[j + half] = Elt<T>::t(ob);
    }
  }
}

// ---------------------------------------------------------------------------
// GEMMs
// ---------------------------------------------------------------------------
// Workgroup tile 128 x 256, K-steps of 32; wave (wm, wn) of the 2 x 2 waves
// owns a 64 x 128 block: 2 x 4 MFMA tiles of 32 x 32, so each fragment read
// from LDS feeds 2 (B) or 4 (A) products.
constexpr int kGbm = 128, kGbn = 256, kGbk = 32;
constexpr int kGld = kGbk + 8;                  // LDS row stride in elements (80 bytes)
constexpr int kGtm = 2, kGtn = 4;               // MFMA tiles per wave
constexpr int kGva = kGbm * kGbk / 8 / 256;     // 16-byte vectors per thread, A tile
constexpr int kGvb = kGbn * kGbk / 8 / 256;     // 16-byte vectors per thread, W tile

template <int EPI>
__device__ __forceinline__ void gemm_store(const GemmArgs& a, int m, int n, float y) {
  bf16_t* out = static_cast<bf16_t*>(a.out) + (size_t)m * a.ldo + n;
  if constexpr (EPI == kGemmStore) {
    if (a.bias != nullptr) y += bf16_to_f(static_cast<const bf16_t*>(a.bias)[n]);
    *out = f_to_bf16(y);
  } else {
    *out = f_to_bf16(bf16_to_f(*out) + round_bf16(y));
  }
}

// Software pipeline: while the waves multiply K-tile kt out of LDS, tile
// kt + 1 is in flight into registers, then goes to the other LDS buffer.
// The barrier orders LDS only (the next prefetch may already be in flight);
// the loads are unconditional (the last tile's addresses are clamped), so
// each wait counts exactly.
template <int EPI>
__global__ void __launch_bounds__(256, 2) k_gemm_bf16(GemmArgs a) {
  __shared__ __align__(16) bf16_t As[2][kGbm * kGld];
  __shared__ __align__(16) bf16_t Bs[2][kGbn * kGld];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int m0 = blockIdx.y * kGbm, n0 = blockIdx.x * kGbn;
  const bf16_t* A = static_cast<const bf16_t*>(a.A);
  const bf16_t* W = static_cast<const bf16_t*>(a.W);
  const int nk = (a.K + kGbk - 1) / kGbk;
  const re_u32x4 zero = {0u, 0u, 0u, 0u};
  struct Stage {
    re_u32x4 a[kGva], b[kGvb];
  };
  Stage st;
  // 16-byte vector v of a tile with 32 columns: row v / 4, columns
  // (v % 4) * 8 ..+8.  Rows past M or N read a valid row (clamped) whose
  // results are never stored; columns past K read as zeros.
  auto gload = [&](Stage& s, int kt) {
    const int k0 = min(kt, nk - 1) * kGbk;
#pragma unroll
    for (int i = 0; i < kGva; ++i) {
      const int v = tid + 256 * i, row = v >> 2, k = k0 + (v & 3) * 8;
      const bool kin = k < a.K;
      const re_u32x4 x = *reinterpret_cast<const re_u32x4*>(A + (size_t)min(m0 + row, a.M - 1) * a.lda + (kin ? k : 0));
      s.a[i] = kin ? x : zero;
    }
#pragma unroll
    for (int i = 0; i < kGvb; ++i) {
      const int v = tid + 256 * i, row = v >> 2, k = k0 + (v & 3) * 8;
      const bool kin = k < a.K;
      const re_u32x4 y = *reinterpret_cast<const re_u32x4*>(W + (size_t)min(n0 + row, a.N - 1) * a.ldw + (kin ? k : 0));
      s.b[i] = kin ? y : zero;
    }
  };
  auto sstore = [&](const Stage& s, int buf) {
#pragma unroll
    for (int i = 0; i < kGva; ++i) {
      const int v = tid + 256 * i;
      *reinterpret_cast<re_u32x4*>(&As[buf][(v >> 2) * kGld + (v & 3) * 8]) = s.a[i];
    }
#pragma unroll
    for (int i = 0; i < kGvb; ++i) {
      const int v = tid + 256 * i;
      *reinterpret_cast<re_u32x4*>(&Bs[buf][(v >> 2) * kGld + (v & 3) * 8]) = s.b[i];
    }
  };
  f32x16_t acc[kGtm][kGtn];
#pragma unroll
  for (int i = 0; i < kGtm; ++i)
#pragma unroll
    for (int j = 0; j < kGtn; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;
  auto mma_tile = [&](int buf) {
#pragma unroll
    for (int ks = 0; ks < kGbk / 16; ++ks) {
      // lane l supplies row l % 32 of its operand, elements (l / 32) * 8 ..+8
      const int kof = ks * 16 + (lane >> 5) * 8;
      bf16x8_t af[kGtm], bf[kGtn];
#pragma unroll
      for (int i = 0; i < kGtm; ++i) af[i] = lds_frag(&As[buf][(wm * 64 + i * 32 + (lane & 31)) * kGld + kof]);
#pragma unroll
      for (int j = 0; j < kGtn; ++j) bf[j] = lds_frag(&Bs[buf][(wn * 128 + j * 32 + (lane & 31)) * kGld + kof]);
#pragma unroll
      for (int i = 0; i < kGtm; ++i)
#pragma unroll
        for (int j = 0; j < kGtn; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
  };
  gload(st, 0);
  sstore(st, 0);
  lds_barrier();
  for (int kt = 0; kt < nk; ++kt) {
    gload(st, kt + 1);
    __builtin_amdgcn_sched_barrier(0);
    mma_tile(kt & 1);
    __builtin_amdgcn_sched_barrier(0);
    sstore(st, (kt + 1) & 1);
    lds_barrier();
  }
  // accumulator v of lane l: row 8 (v / 4) + 4 (l / 32) + v % 4, column l % 32
#pragma unroll
  for (int i = 0; i < kGtm; ++i)
#pragma unroll
    for (int j = 0; j < kGtn; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int m = m0 + wm * 64 + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        const int n = n0 + wn * 128 + j * 32 + (lane & 31);
        if (m < a.M && n < a.N) gemm_store<EPI>(a, m, n, acc[i][j][v]);
      }
}

// fp32 models: 64 x 64 tiles, 4 x 4 outputs per thread, K in steps of 16.
template <int EPI>
__global__ void __launch_bounds__(256) k_gemm_f32(GemmArgs a) {
  __shared__ float As[16][64 + 4];
  __shared__ float Ws[16][64 + 4];
  const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
  const int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
  const float* A = static_cast<const float*>(a.A);
  const float* W = static_cast<const float*>(a.W);
  float acc[4][4] = {};
  for (int k0 = 0; k0 < a.K; k0 += 16) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int idx = tid + 256 * i, row = idx >> 4, kk = idx & 15, k = k0 + kk;
      const bool kin = k < a.K;
      const float x = A[(size_t)min(m0 + row, a.M - 1) * a.lda + (kin ? k : 0)];
      const float y = W[(size_t)min(n0 + row, a.N - 1) * a.ldw + (kin ? k : 0)];
      As[kk][row] = kin ? x : 0.f;
      Ws[kk][row] = kin ? y : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) {
      float av[4], wv[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        av[r] = As[kk][ty * 4 + r];
        wv[r] = Ws[kk][tx * 4 + r];
      }
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[r][c] = fmaf(av[r], wv[c], acc[r][c]);
    }
    __syncthreads();
  }
  float* out = static_cast<float*>(a.out);
  const float* bias = static_cast<const float*>(a.bias);
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int m = m0 + ty * 4 + r, n = n0 + tx * 4 + c;
      if (m >= a.M || n >= a.N) continue;
      float* o = out + (size_t)m * a.ldo + n;
      if constexpr (EPI == kGemmStore)
        *o = acc[r][c] + (bias != nullptr ? bias[n] : 0.f);
      else
        *o = *o + acc[r][c];
    }
}

// ---------------------------------------------------------------------------
// Attention
// ---------------------------------------------------------------------------
// One workgroup per (token m, head h): keys 0..pos of m's row, which are the
// row's tokens m - pos .. m (a prefilled row starts at position 0).  Same
// steps as the decode attention: s = bf16(bf16(q.k) / sqrt(d)) (fp32 models
// keep the fp32 product), exact softmax, p rounded to bf16, o = T(sum p v).
template <typename T>
__global__ void __launch_bounds__(256) k_pf_attn_rows(PrefillAttn a) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  float* sc = reinterpret_cast<float*>(smem_raw);  // [capacity]
  __shared__ float red[8];
  __shared__ float part[256];
  const int m = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
  const int D = a.head_dim, nq = a.heads, g = a.heads / a.kv_heads;
  const int kvh = h / g;
  const int pos = a.pos[m];
  const int n = pos + 1;
  const T* qkv = static_cast<const T*>(a.qkv);
  const T* q = qkv + (size_t)m * a.ld + (size_t)h * D;
  const size_t koff = (size_t)nq * D + (size_t)kvh * D;
  const size_t voff = (size_t)(nq + a.kv_heads) * D + (size_t)kvh * D;
  const long long first = (long long)m - pos;
  const float scale_div = sqrtf(static_cast<float>(D));
  float lmax = -INFINITY;
  for (int j = tid; j < n; j += 256) {
    const T* k = qkv + (size_t)(first + j) * a.ld + koff;
    float s = 0.f;
    for (int c = 0; c < D; c += 8) s = dot8(Vec8<T>::load_cached(k + c), Vec8<T>::load_cached(q + c), s);
    if constexpr (sizeof(T) == 2) s = round_bf16(s);
    s = round_bf16(s / scale_div);
    sc[j] = s;
    lmax = fmaxf(lmax, s);
  }
  lmax = wave_max(lmax);
  if ((tid & 63) == 0) red[tid >> 6] = lmax;
  __syncthreads();
  const float mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  float es = 0.f;
  for (int j = tid; j < n; j += 256) es += expf(sc[j] - mx);
  es = wave_sum(es);
  __syncthreads();
  if ((tid & 63) == 0) red[4 + (tid >> 6)] = es;
  __syncthreads();
  const float inv = 1.0f / (red[4] + red[5] + red[6] + red[7]);
  for (int j = tid; j < n; j += 256) sc[j] = round_bf16(expf(sc[j] - mx) * inv);
  __syncthreads();
  // P.V: thread (c, grp) sums element c over keys grp, grp + G, ...
  const int G = 256 / D;  // D divides 256
  const int c = tid % D, grp = tid / D;
  float o = 0.f;
  for (int j = grp; j < n; j += G) o = fmaf(sc[j], Elt<T>::f(qkv[(size_t)(first + j) * a.ld + voff + c]), o);
  part[tid] = o;
  __syncthreads();
  if (tid < D) {
    float t = 0.f;
    for (int r = 0; r < G; ++r) t += part[r * D + tid];
    static_cast<T*>(a.out)[(size_t)m * nq * D + (size_t)h * D + tid] = Elt<T>::t(t);
  }
}

// bf16, head_dim 128: one workgroup per (tile of up to 64 queries of one row,
// head).  Wave w owns queries (w / 2) * 32 ..+32 and, per 64-key tile, keys
// (w % 2) * 32 ..+32 of Q K^T; for P V it owns output columns (w % 2) * 64
// ..+64.  The tile's bf16 scores, then probabilities, stay in LDS
// (64 x keys), so the softmax is exact: global max and sum, then each p
// rounded to bf16, as the decode step does.
constexpr int kAq = 64, kAk = 64, kAd = 128;
constexpr int kAkld = kAd + 8;  // K tile row stride (elements)
constexpr int kAvld = kAk + 8;  // transposed V tile row stride

__global__ void __launch_bounds__(256) k_pf_attn_mfma(PrefillAttn a) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  bf16_t* kv = reinterpret_cast<bf16_t*>(smem_raw);  // K tile [64][136] or V^T tile [128][72]
  bf16_t* S = kv + kAd * kAvld;                      // [64][sld]
  const int sld = a.score_ld;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int4 tile = a.tiles[blockIdx.x];  // first query token, first token of the row, queries, first query's position
  const int h = blockIdx.y;
  const int m_start = tile.x, r0 = tile.y, nqt = tile.z, p0 = tile.w;
  const int nq = a.heads, kvh = h / (a.heads / a.kv_heads);
  const bf16_t* qkv = static_cast<const bf16_t*>(a.qkv);
  const size_t koff = (size_t)nq * kAd + (size_t)kvh * kAd;
  const size_t voff = (size_t)(nq + a.kv_heads) * kAd + (size_t)kvh * kAd;
  const int nkeys = p0 + nqt;  // keys 0 .. p0 + nqt - 1 of the row
  const int nkt = (nkeys + kAk - 1) / kAk;
  const int sm = wave >> 1, sn = wave & 1;

  // Q fragments of this wave's 32 queries (rows past the tile read the last one)
  bf16x8_t qf[kAd / 16];
  {
    const int qi = min(sm * 32 + (lane & 31), nqt - 1);
    const bf16_t* qrow = qkv + (size_t)(m_start + qi) * a.ld + (size_t)h * kAd + (lane >> 5) * 8;
#pragma unroll
    for (int ks = 0; ks < kAd / 16; ++ks) qf[ks] = lds_frag(qrow + ks * 16);
  }
  const float scale_div = sqrtf(static_cast<float>(kAd));
  const bf16_t neg_inf = 0xFF80;

  // A 64-row tile of keys in registers: vector v = tid + 256 i is row v / 16,
  // elements (v % 16) * 8 ..+8; rows past the keys read the last.
  re_u32x4 pre[4];
  auto tile_load = [&](int kt, size_t col) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int v = tid + 256 * i;
      const int tok = r0 + min(min(kt, nkt - 1) * kAk + (v >> 4), nkeys - 1);
      pre[i] = *reinterpret_cast<const re_u32x4*>(qkv + (size_t)tok * a.ld + col + (v & 15) * 8);
    }
  };
  // A 64-row tile of values: vector v is row v % 64, elements (v / 64) * 8
  // ..+8, so the 64 lanes of a wave hold one 8-column slice of 64 keys and
  // the transposed LDS writes of one instruction cover 64 consecutive keys of
  // one row (128 contiguous bytes, no bank conflicts).
  auto tile_load_v = [&](int kt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int v = tid + 256 * i;
      const int tok = r0 + min(min(kt, nkt - 1) * kAk + (v & 63), nkeys - 1);
      pre[i] = *reinterpret_cast<const re_u32x4*>(qkv + (size_t)tok * a.ld + voff + (v >> 6) * 8);
    }
  };

  // Scores: S[q][j] = bf16(bf16(q.k_j) / sqrt(d)), causal mask as -inf.  The
  // next key tile is in flight while this one is multiplied.
  tile_load(0, koff);
  for (int kt = 0; kt < nkt; ++kt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int v = tid + 256 * i;
      *reinterpret_cast<re_u32x4*>(&kv[(v >> 4) * kAkld + (v & 15) * 8]) = pre[i];
    }
    tile_load(kt + 1, koff);
    lds_barrier();
    f32x16_t acc;
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[v] = 0.f;
#pragma unroll
    for (int ks = 0; ks < kAd / 16; ++ks) {
      const bf16x8_t bfr = lds_frag(&kv[(sn * 32 + (lane & 31)) * kAkld + ks * 16 + (lane >> 5) * 8]);
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qf[ks], bfr, acc, 0, 0, 0);
    }
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int qi = sm * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
      const int kj = kt * kAk + sn * 32 + (lane & 31);
      const float s = round_bf16(round_bf16(acc[v]) / scale_div);
      S[qi * sld + kj] = kj <= p0 + qi ? f_to_bf16(s) : neg_inf;
    }
    lds_barrier();
  }
  tile_load_v(0);  // the first value tile travels during the softmax
  // Softmax of each query row: four threads per row, eight scores per
  // 16-byte LDS access.  Exact global max and sum, then each p rounded to
  // bf16; exp(x) is the hardware 2^(x log2 e) (v_exp_f32), whose fp32 error
  // is far below the bf16 rounding of p.  Keys past the row's causal limit
  // hold -inf (p = 0); a padding query row (nvalid = 0) gets p = 0.
  {
    const int qi = tid >> 2, part = tid & 3;
    const int nvalid = qi < nqt ? p0 + qi + 1 : 0;
    const int nvec = (nvalid + 7) / 8, nall = nkt * kAk / 8;
    Vec8<bf16_t>* srow = reinterpret_cast<Vec8<bf16_t>*>(S + qi * sld);
    float mx = -INFINITY;
    for (int v = part; v < nvec; v += 4) {
      const Vec8<bf16_t> x = srow[v];
#pragma unroll
      for (int e = 0; e < 8; ++e) mx = fmaxf(mx, x.get(e));
    }
    mx = fmaxf(mx, __shfl_xor(mx, 1, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 2, 64));
    constexpr float kLog2e = 1.44269504088896340736f;
    const float base = mx * kLog2e;
    float es = 0.f;
    for (int v = part; v < nvec; v += 4) {
      const Vec8<bf16_t> x = srow[v];
#pragma unroll
      for (int e = 0; e < 8; ++e) es += __builtin_amdgcn_exp2f(fmaf(x.get(e), kLog2e, -base));
    }
    es += __shfl_xor(es, 1, 64);
    es += __shfl_xor(es, 2, 64);
    const float inv = nvalid > 0 ? 1.0f / es : 0.f;
    for (int v = part; v < nall; v += 4) {
      const Vec8<bf16_t> x = srow[v];
      float pv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e)
        pv[e] = v * 8 + e < nvalid ? __builtin_amdgcn_exp2f(fmaf(x.get(e), kLog2e, -base)) * inv : 0.f;
      srow[v] = Vec8<bf16_t>::from_floats(pv);
    }
  }
  lds_barrier();
  // O = P V, fp32 accumulation.
  f32x16_t o[2];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int v = 0; v < 16; ++v) o[t][v] = 0.f;
  for (int kt = 0; kt < nkt; ++kt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int v = tid + 256 * i, key = v & 63, c = (v >> 6) * 8;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t w = pre[i][e];
        kv[(c + 2 * e) * kAvld + key] = static_cast<bf16_t>(w & 0xffffu);
        kv[(c + 2 * e + 1) * kAvld + key] = static_cast<bf16_t>(w >> 16);
      }
    }
    tile_load_v(kt + 1);
    lds_barrier();
#pragma unroll
    for (int ks = 0; ks < kAk / 16; ++ks) {
      const bf16x8_t af = lds_frag(&S[(sm * 32 + (lane & 31)) * sld + kt * kAk + ks * 16 + (lane >> 5) * 8]);
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const bf16x8_t bfr = lds_frag(&kv[((sn * 2 + t) * 32 + (lane & 31)) * kAvld + ks * 16 + (lane >> 5) * 8]);
        o[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, bfr, o[t], 0, 0, 0);
      }
    }
    lds_barrier();
  }
  bf16_t* out = static_cast<bf16_t*>(a.out);
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int qi = sm * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
      const int col = (sn * 2 + t) * 32 + (lane & 31);
      if (qi < nqt) out[(size_t)(m_start + qi) * nq * kAd + (size_t)h * kAd + col] = f_to_bf16(o[t][v]);
    }
}

}  // namespace

// ---------------------------------------------------------------------------
// Launchers
// ---------------------------------------------------------------------------
hipError_t launch_prefill_embed(const PrefillRows& a, int dtype_bytes, hipStream_t stream) {
  if (a.M <= 0) return hipSuccess;
  if (dtype_bytes == 2)
    k_pf_embed<bf16_t><<<a.M, 256, 0, stream>>>(a);
  else
    k_pf_embed<float><<<a.M, 256, 0, stream>>>(a);
  return hipGetLastError();
}

hipError_t launch_prefill_rmsnorm(const void* x, const void* w, void* y, int M, int H, float eps, int dtype_bytes,
                                  hipStream_t stream) {
  if (M <= 0) return hipSuccess;
  if (dtype_bytes == 2)
    k_pf_rmsnorm<bf16_t><<<M, 256, 0, stream>>>(x, w, y, H, eps);
  else
    k_pf_rmsnorm<float><<<M, 256, 0, stream>>>(x, w, y, H, eps);
  return hipGetLastError();
}

hipError_t launch_prefill_swiglu(const void* gate, const void* up, void* out, long long n, int dtype_bytes,
                                 hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  const int blocks = static_cast<int>(std::min<long long>((n + 255) / 256, 8192));
  if (dtype_bytes == 2)
    k_pf_swiglu<bf16_t><<<blocks, 256, 0, stream>>>(gate, up, out, n);
  else
    k_pf_swiglu<float><<<blocks, 256, 0, stream>>>(gate, up, out, n);
  return hipGetLastError();
}

hipError_t launch_prefill_qkv_post(const PrefillQkv& a, int dtype_bytes, hipStream_t stream) {
  if (a.M <= 0) return hipSuccess;
  if (dtype_bytes == 2)
    k_pf_qkv_post<bf16_t><<<a.M, 256, 0, stream>>>(a);
  else
    k_pf_qkv_post<float><<<a.M, 256, 0, stream>>>(a);
  return hipGetLastError();
}

hipError_t launch_gemm(const GemmArgs& a, int epi, int dtype_bytes, hipStream_t stream) {
  if (a.M <= 0 || a.N <= 0) return hipSuccess;
  if (a.K <= 0 || a.K % 8 != 0 || a.lda % 8 != 0 || a.ldw % 8 != 0) return hipErrorInvalidValue;
  if (dtype_bytes == 2) {
    const dim3 grid((a.N + kGbn - 1) / kGbn, (a.M + kGbm - 1) / kGbm);
    if (epi == kGemmStore)
      k_gemm_bf16<kGemmStore><<<grid, 256, 0, stream>>>(a);
    else
      k_gemm_bf16<kGemmResidual><<<grid, 256, 0, stream>>>(a);
  } else {
    const dim3 grid((a.N + 63) / 64, (a.M + 63) / 64);
    if (epi == kGemmStore)
      k_gemm_f32<kGemmStore><<<grid, 256, 0, stream>>>(a);
    else
      k_gemm_f32<kGemmResidual><<<grid, 256, 0, stream>>>(a);
  }
  return hipGetLastError();
}

// The tile's scores for the whole window must fit the LDS (window <= 1024).
bool prefill_attention_mfma(const Dims& d) {
  const size_t bytes = (size_t)kAd * kAvld * 2 + (size_t)kAq * ((d.capacity + kAk - 1) / kAk * kAk + 8) * 2;
  return d.dtype_bytes == 2 && d.head_dim == kAd && bytes <= 160 * 1024;
}

size_t prefill_attention_lds(const Dims& d, int max_keys) {
  if (prefill_attention_mfma(d)) {
    const int nk = (max_keys + kAk - 1) / kAk * kAk;
    return (size_t)kAd * kAvld * 2 + (size_t)kAq * (nk + 8) * 2;
  }
  return (size_t)max_keys * sizeof(float);
}

hipError_t prepare_prefill(const Dims& d) {
  const int bytes = static_cast<int>(prefill_attention_lds(d, d.capacity));
  if (prefill_attention_mfma(d))
    return hipFuncSetAttribute(reinterpret_cast<const void*>(k_pf_attn_mfma),
                               hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (d.dtype_bytes == 2)
    return hipFuncSetAttribute(reinterpret_cast<const void*>(k_pf_attn_rows<bf16_t>),
                               hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  return hipFuncSetAttribute(reinterpret_cast<const void*>(k_pf_attn_rows<float>),
                             hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
}

hipError_t launch_prefill_attention(const PrefillAttn& a, const Dims& d, int ntiles, hipStream_t stream) {
  if (a.M <= 0) return hipSuccess;
  if (prefill_attention_mfma(d)) {
    if (ntiles <= 0 || a.score_ld % 8 != 0) return hipErrorInvalidValue;
    const size_t bytes = (size_t)kAd * kAvld * 2 + (size_t)kAq * a.score_ld * 2;
    k_pf_attn_mfma<<<dim3(ntiles, d.heads), 256, bytes, stream>>>(a);
  } else {
    if (256 % d.head_dim != 0 || d.head_dim % 8 != 0) return hipErrorInvalidValue;
    const size_t bytes = (size_t)d.capacity * sizeof(float);
    if (d.dtype_bytes == 2)
      k_pf_attn_rows<bf16_t><<<dim3(a.M, d.heads), 256, bytes, stream>>>(a);
    else
      k_pf_attn_rows<float><<<dim3(a.M, d.heads), 256, bytes, stream>>>(a);
  }
  return hipGetLastError();
}

}  // namespace re
