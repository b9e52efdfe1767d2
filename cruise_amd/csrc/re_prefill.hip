// Batched prefill kernels (gfx950): the decoder over all prompt tokens of
// several rows at once, M = tokens.  Same operations and rounding points as
// the decode step (batched_decoder_step.py:277-403), laid out for large M:
//
//   embed      token rows + per-token RoPE table
//   rmsnorm    one workgroup per token
//   GEMM       C[M,N] = A[M,K] W[N,K]^T, both operands K-contiguous.
//              bf16: MFMA v_mfma_f32_16x16x32_bf16, 256x256 workgroup tiles
//              (eight waves of 128x64), K in steps of 64 through two LDS
//              stages filled by direct global -> LDS loads, fp32
//              accumulation; epilogues "T(acc + bias)", the residual
//              "T(h + T(acc))", and gate/up with SwiGLU in one GEMM (the
//              tile's W rows half gate, half up).  fp32 models: an
//              LDS-tiled FMA GEMM.
//   qkv post   RoPE of q and k in place, K/V rows to their paged slots
//   attention  causal within each row's prompt.  bf16, head_dim 128: MFMA
//              for Q K^T and P V per (64-query tile, head), the bf16 scores of
//              the whole tile kept in LDS so the softmax is the exact
//              two-pass one of the decode step; otherwise one workgroup per
//              (token, head).
//   SwiGLU     elementwise on the gate and up products (fp32 models; bf16
//              models take it in the gate/up GEMM's epilogue)
#include <algorithm>
#include <type_traits>

#include "re_device.h"
#include "re_layout.h"

namespace re {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short lds_v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) lds_v4i16* lds_v4i16_ptr;
typedef float f32x4_t __attribute__((ext_vector_type(4)));
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
// Eight elements per thread and step (16-byte bf16 accesses); n % 8 == 0.
template <typename T>
__global__ void __launch_bounds__(256) k_pf_swiglu(const void* gate, const void* up, void* out, long long n) {
  const T* g = static_cast<const T*>(gate);
  const T* u = static_cast<const T*>(up);
  T* o = static_cast<T*>(out);
  const long long nv = n / 8;
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < nv; i += (long long)gridDim.x * blockDim.x) {
    const Vec8<T> gv = Vec8<T>::load(g + i * 8);
    const Vec8<T> uv = Vec8<T>::load(u + i * 8);
    float y[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float x = gv.get(e);
      const float sg = Elt<T>::r(x / (1.0f + expf(-x)));
      y[e] = Elt<T>::r(sg * uv.get(e));
    }
    *reinterpret_cast<Vec8<T>*>(o + i * 8) = Vec8<T>::from_floats(y);
  }
}

// RoPE of q and k (rows already rounded with their bias) in place, and the
// paged slot write of k and v (batched_decoder_step.py:231-264, 323-324).
template <typename T>
__device__ __forceinline__ void store8(T* p, const Vec8<T>& v);
template <>
__device__ __forceinline__ void store8<bf16_t>(bf16_t* p, const Vec8<bf16_t>& v) {
  *reinterpret_cast<re_u32x4*>(p) = v.v;
}
template <>
__device__ __forceinline__ void store8<float>(float* p, const Vec8<float>& v) {
  reinterpret_cast<re_f32x4*>(p)[0] = v.a;
  reinterpret_cast<re_f32x4*>(p)[1] = v.b;
}

// One workgroup per token; a thread takes 8 consecutive pair indices j of one
// head (16-byte accesses of both halves, the RoPE table's 8 cos/sin pairs),
// head_dim a multiple of 16.
template <typename T>
__global__ void __launch_bounds__(256) k_pf_qkv_post(PrefillQkv a) {
  const int m = blockIdx.x;
  const int half = a.head_dim / 2, hv = half / 8;
  const int nq = a.heads, nkv = a.kv_heads;
  T* row = static_cast<T*>(a.qkv) + (size_t)m * a.ld;
  const int s = a.slot[m];
  const bool to_cache = s >= 0 && s < a.slots;
  const float* rope = a.rope + (size_t)m * half * 2;
  for (int idx = threadIdx.x; idx < (nq + 2 * nkv) * hv; idx += blockDim.x) {
    const int hg = idx / hv, j = (idx - hg * hv) * 8;
    T* p = row + (size_t)hg * a.head_dim;
    Vec8<T> va = Vec8<T>::load_cached(p + j), vb = Vec8<T>::load_cached(p + j + half);
    if (hg < nq + nkv) {
      float oa[8], ob[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float c = rope[(j + e) * 2], sn = rope[(j + e) * 2 + 1];
        const float qa = va.get(e), qb = vb.get(e);
        oa[e] = Elt<T>::r(Elt<T>::r(qa * c) + Elt<T>::r(-qb * sn));
        ob[e] = Elt<T>::r(Elt<T>::r(qb * c) + Elt<T>::r(qa * sn));
      }
      va = Vec8<T>::from_floats(oa);
      vb = Vec8<T>::from_floats(ob);
      store8<T>(p + j, va);
      store8<T>(p + j + half, vb);
    }
    if (hg >= nq && to_cache) {
      const bool is_key = hg < nq + nkv;
      const int kvh = is_key ? hg - nq : hg - nq - nkv;
      T* cache = static_cast<T*>(is_key ? a.key_cache : a.value_cache) + ((size_t)s * nkv + kvh) * a.head_dim;
      store8<T>(cache + j, va);
      store8<T>(cache + j + half, vb);
    }
  }
}

// ---------------------------------------------------------------------------
// GEMMs
// ---------------------------------------------------------------------------
// bf16: one 256 x 256 output tile per workgroup of 8 waves, K in steps of 64.
//
// Operands reach LDS by direct global -> LDS loads (global_load_lds_dwordx4,
// 16 bytes per lane, no register staging) into two stages of 64 KB: W tile
// rows 0..255, then A tile rows 256..511, 128 bytes (one K step) per row.
// Chunk c (16 bytes) of row r sits in slot c ^ gemm_swz(r), so the fragment
// reads below hit distinct banks for 8 and for 16 consecutive rows.  The
// products run as C^T = W A^T on v_mfma_f32_16x16x32_bf16: wave (wn, wm) owns
// n 128 x m 64 (8 x 4 tiles of 16 x 16), and a lane's accumulator holds four
// consecutive output columns of one row.  A stage is two sub-steps of K = 32;
// each sub-step's 12 fragments are read under the previous sub-step's 32
// products, one read per two products.  The stage's one barrier sits between
// its sub-steps: before it each wave waits for its own loads of stage kt + 1
// and its reads of stage kt, so after it stage kt + 1 is complete in LDS and
// stage kt's buffer is free.  The loads of stage kt + 2 go out during the
// second sub-step (waves 0-3 at its start, waves 4-7 after 12 of their 32
// products, so the two waves of a SIMD do not stall on them together), and
// stage kt + 1's first fragments are read under the second sub-step's
// products, so no wave waits on LDS at a stage boundary.  The
// epilogue rounds the tile to bf16 in LDS (rows padded to 264 elements) and
// writes it as row-contiguous 16-byte vectors: "T(acc + bias)" (qkv), or the
// residual "T(h + T(acc))".
//
// Workgroups are dispatched round-robin over the 8 XCDs; workgroup b runs
// tile t = (b % 8) * ceil(T / 8) + b / 8 of a grouped order (4 M tiles by
// every N tile), so the 32 tiles an XCD runs at once share 4 A and 8 W row
// blocks in its L2.
//
// Requirements (checked by launch_gemm): K % 64 == 0, N % 8 == 0, lda, ldw
// and ldo multiples of 8 elements, 16-byte aligned operands.
constexpr int kGm = 256, kGn = 256, kGk = 64;
constexpr int kGrowBytes = kGk * 2;                   // one K step of one row
constexpr int kGstage = (kGm + kGn) * kGrowBytes;     // 64 KB
constexpr int kGwaves = 8, kGthreads = kGwaves * 64;
constexpr int kGdmaRows = (kGm + kGn) / kGwaves;      // rows each wave loads per stage
constexpr int kGdmaInsts = kGdmaRows / 8;             // 8 rows (1 KB) per instruction
constexpr int kGoutLd = kGn + 8;                      // epilogue row stride (elements)
constexpr int kGsmem = kGm * kGoutLd * 2 > 2 * kGstage ? kGm * kGoutLd * 2 : 2 * kGstage;
constexpr int kGgroupM = 4;

typedef const __attribute__((address_space(1))) void* gemm_gptr;
typedef __attribute__((address_space(3))) void* gemm_lptr;

__device__ __forceinline__ int gemm_swz(int r) { return (r & 7) ^ ((r >> 3) & 1); }

// s_waitcnt immediate: vmcnt <= vm (6 bits), lgkmcnt 0, expcnt untouched.
constexpr int gemm_wait_vm(int vm) { return (vm & 15) | ((vm >> 4) << 14) | (7 << 4); }

// End of a stage: this wave's loads and LDS reads are done, then the barrier.
// The empty asm statements keep the compiler from moving memory accesses
// across; the wait is a real instruction the wait-count pass accounts for.
__device__ __forceinline__ void gemm_stage_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_waitcnt(gemm_wait_vm(0));
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("" ::: "memory");
}

__device__ __forceinline__ void gemm_tile_of(int b, int nM, int nN, int& mt, int& nt) {
  const int total = nM * nN, x = b & 7, local = b >> 3, q = total >> 3, r = total & 7;
  const int t = x < r ? x * (q + 1) + local : r * (q + 1) + (x - r) * q + local;
  const int per_group = kGgroupM * nN, g = t / per_group, first = g * kGgroupM;
  const int gm = min(kGgroupM, nM - first), w = t - g * per_group;
  mt = first + w % gm;
  nt = w / gm;
}

template <int EPI>
__global__ void __launch_bounds__(kGthreads, 1) k_gemm_bf16(GemmArgs a, int nM, int nN) {
  extern __shared__ __align__(16) unsigned char gsm[];
  // wave-uniform, so the load base lives in SGPRs (32-bit per-lane offsets)
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_index(tid);
  int mt, nt;
  gemm_tile_of(blockIdx.x, nM, nN, mt, nt);
  // The SwiGLU epilogue's tile covers 128 output columns: W tile rows 0..127
  // are their gate rows, rows 128..255 their up rows.
  constexpr bool kSwiGlu = EPI == kGemmSwiGlu;
  constexpr int kTileN = kSwiGlu ? kGn / 2 : kGn;
  const int m0 = mt * kGm, n0 = nt * kTileN;
  // Loads: waves 0-3 bring W rows 0..255, waves 4-7 A rows 0..255.  Rows past
  // M or N read a valid row (clamped) whose results are never stored.
  const int row0 = wave * kGdmaRows;
  const bool loads_w = row0 < kGn;
  const void* wsrc = kSwiGlu && row0 >= kTileN ? a.W2 : a.W;
  const char* gbase = loads_w ? static_cast<const char*>(wsrc) + (size_t)n0 * a.ldw * 2
                              : static_cast<const char*>(a.A) + (size_t)m0 * a.lda * 2;
  const long long ld = loads_w ? a.ldw : a.lda;
  const int rows_left = loads_w ? a.N - n0 : a.M - m0;
  uint32_t goff[kGdmaInsts];
#pragma unroll
  for (int i = 0; i < kGdmaInsts; ++i) {
    // lane l of instruction i writes slot l % 8 of row row0 + 8 i + l / 8
    const int row = row0 + i * 8 + (lane >> 3);
    const int chunk = (lane & 7) ^ gemm_swz(row);
    const int local = loads_w ? row % kTileN : row & 255;  // the row within its source matrix
    goff[i] = static_cast<uint32_t>(min(local, rows_left - 1) * ld * 2 + chunk * 16);
  }
  const int nk = a.K / kGk;
  auto issue = [&](int kt) {  // stages past the end re-read the last one (clamped, never used)
    const char* g = gbase + (size_t)min(kt, nk - 1) * kGrowBytes;
    unsigned char* l = gsm + (kt & 1) * kGstage + row0 * kGrowBytes;
#pragma unroll
    for (int i = 0; i < kGdmaInsts; ++i)
      __builtin_amdgcn_global_load_lds((gemm_gptr)(g + goff[i]), (gemm_lptr)(l + i * 1024), 16, 0, 0);
  };
  const int wn = wave & 1, wm = wave >> 1;
  f32x4_t acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[i][j][v] = 0.f;
  // lane l supplies row l % 16 of a 16-row operand tile, K elements
  // 8 (l / 16) ..+8 of the 32-wide sub-step
  const int fr = lane & 15, fq = lane >> 4;
  auto frag = [&](int st, int row, int ks) -> bf16x8_t {
    const int c = (4 * ks + fq) ^ gemm_swz(row);
    return lds_frag(reinterpret_cast<const bf16_t*>(gsm + st * kGstage + row * kGrowBytes + c * 16));
  };
  // fragment sets: [set][0..7] W rows (n), [set][8..11] A rows (m)
  bf16x8_t f[2][12];
  auto read_set = [&](int set, int st, int ks) {
#pragma unroll
    for (int i = 0; i < 8; ++i) f[set][i] = frag(st, wn * 128 + i * 16 + fr, ks);
#pragma unroll
    for (int j = 0; j < 4; ++j) f[set][8 + j] = frag(st, kGn + wm * 64 + j * 16 + fr, ks);
  };
  auto products = [&](int set) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(f[set][i], f[set][8 + j], acc[i][j], 0, 0, 0);
#pragma unroll
    for (int r = 0; r < 12; ++r) {  // one fragment read per two products
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  issue(0);
  issue(1);
  __builtin_amdgcn_s_waitcnt(gemm_wait_vm(kGdmaInsts));  // this wave's stage 0
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  read_set(0, 0, 0);
  __builtin_amdgcn_sched_barrier(0);
  for (int kt = 0; kt < nk; ++kt) {
    const int st = kt & 1;
    read_set(1, st, 1);
    products(0);
    gemm_stage_barrier();  // stage kt + 1 complete, stage kt's buffer free
    // Second sub-step, in a fixed order: the 32 products row block by row
    // block, the next stage's 12 first fragments one per two products (past
    // the last stage: a buffer in flight, never used), and the loads of
    // stage kt + 2.  The two waves of a SIMD (w and w + 4) issue their loads
    // apart: an issuing wave waits while the memory pipeline takes its
    // eight 1 KB requests, and meanwhile the other wave's products run.
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (i == 0 && wave < 4) issue(kt + 2);
      if (i == 3 && wave >= 4) issue(kt + 2);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(f[1][i], f[1][8 + j], acc[i][j], 0, 0, 0);
        if (i < 6 && (j & 1)) {
          const int idx = 2 * i + (j >> 1);
          f[0][idx] = idx < 8 ? frag(st ^ 1, wn * 128 + idx * 16 + fr, 0)
                              : frag(st ^ 1, kGn + wm * 64 + (idx - 8) * 16 + fr, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
  gemm_stage_barrier();
  // acc[i][j] value v of lane l: n = 16 i + 4 (l / 16) + v, m = 16 j + l % 16
  // within the wave's block
  bf16_t* T = reinterpret_cast<bf16_t*>(gsm);
  const bf16_t* bias = static_cast<const bf16_t*>(a.bias);
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int ml = wm * 64 + j * 16 + fr, nl = wn * 128 + i * 16 + 4 * fq;
      float y[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) y[e] = acc[i][j][e];
      if (EPI == kGemmStore && bias != nullptr) {
        const uint2 b = *reinterpret_cast<const uint2*>(bias + min(n0 + nl, a.N - 4));
        y[0] += __uint_as_float(b.x << 16);
        y[1] += __uint_as_float(b.x & 0xffff0000u);
        y[2] += __uint_as_float(b.y << 16);
        y[3] += __uint_as_float(b.y & 0xffff0000u);
      }
      *reinterpret_cast<uint2*>(T + ml * kGoutLd + nl) =
          make_uint2(f_to_bf16(y[0]) | ((uint32_t)f_to_bf16(y[1]) << 16),
                     f_to_bf16(y[2]) | ((uint32_t)f_to_bf16(y[3]) << 16));
    }
  gemm_stage_barrier();
  bf16_t* out = static_cast<bf16_t*>(a.out);
  if constexpr (kSwiGlu) {
    // columns c of the gate half and 128 + c of the up half give output
    // column n0 + c: silu as the decode step computes it, rounded, then the
    // rounded product
#pragma unroll 4
    for (int idx = tid; idx < kGm * kTileN / 8; idx += kGthreads) {
      const int r = idx / (kTileN / 8), c = idx % (kTileN / 8);
      const int m = m0 + r, n = n0 + c * 8;
      if (m >= a.M || n >= a.N) continue;
      const Vec8<bf16_t> gv = Vec8<bf16_t>::load_cached(T + r * kGoutLd + c * 8);
      const Vec8<bf16_t> uv = Vec8<bf16_t>::load_cached(T + r * kGoutLd + kTileN + c * 8);
      float y[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = gv.get(e);
        const float sg = round_bf16(x / (1.0f + expf(-x)));
        y[e] = round_bf16(sg * uv.get(e));
      }
      *reinterpret_cast<Vec8<bf16_t>*>(out + (size_t)m * a.ldo + n) = Vec8<bf16_t>::from_floats(y);
    }
    return;
  }
#pragma unroll 4
  for (int idx = tid; idx < kGm * kGn / 8; idx += kGthreads) {
    const int r = idx / (kGn / 8), c = idx % (kGn / 8);
    const int m = m0 + r, n = n0 + c * 8;
    if (m >= a.M || n >= a.N) continue;
    re_u32x4 t = *reinterpret_cast<const re_u32x4*>(T + r * kGoutLd + c * 8);
    re_u32x4* p = reinterpret_cast<re_u32x4*>(out + (size_t)m * a.ldo + n);
    if constexpr (EPI == kGemmResidual) {
      const re_u32x4 h = *p;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float lo = __uint_as_float(h[e] << 16) + __uint_as_float(t[e] << 16);
        const float hi = __uint_as_float(h[e] & 0xffff0000u) + __uint_as_float(t[e] & 0xffff0000u);
        t[e] = f_to_bf16(lo) | ((uint32_t)f_to_bf16(hi) << 16);
      }
    }
    *p = t;
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

// Tile shapes of the MFMA attention below (keys per tile, head dim; the
// query tiles of up to 64 come from the launch's tile list).
constexpr int kAk = 64, kAd = 128;
constexpr int kAkld = kAd + 8;   // K tile row stride (elements)
constexpr int kAvld = kAd + 16;  // V tile row stride: 4 key rows of a transposing read cover 4 x 32 bytes of distinct banks

// bf16, head_dim 128: one workgroup per (tile of up to 64 queries of one row,
// head), two passes over the key tiles of 64, no score tile in LDS.
// Wave w owns queries (w / 2) * 32 ..+32 and, in every key tile, keys
// (w % 2) * 32 ..+32.  S^T = K Q^T on MFMA (keys are the A rows, queries the
// B columns), so a lane holds 16 scores of one query (its column).
//   pass 1: every score s = bf16(bf16(q.k) / sqrt(d)) (keys past the
//     query's causal limit are -inf); per lane a running max and the sum of
//     exp(s - max) rescaled as the max grows; lanes l and l ^ 32 and the two
//     key halves are then combined: the exact row max M and the sum L.
//   pass 2: the scores again, p = bf16(exp(s - M) / L) -- the reference's
//     rounding point -- and O += P V on MFMA straight from the score
//     registers: for each 16-key block the MFMA's k index runs over the keys
//     in the order the accumulator layout holds them (j 0-7 from lanes 0-31:
//     keys +0..3 and +8..11; j 8-15 from lanes 32-63: keys +4..7 and
//     +12..15), and the value operand is read in the same order from the
//     row-major V tile by transposing LDS reads.  The two key halves'
//     partial O are added at the end.
// LDS: one K tile and one V tile (35 KB), independent of the prompt length.
constexpr int kFlashLds = kAk * kAkld * 2 + kAk * kAvld * 2;

// Workgroup order: the (KV head, query tile) pairs P = g * ntiles + t are cut
// into chunks of kFlashChunk consecutive tiles (a 1000-token prompt's tiles
// are one chunk); chunk c runs on XCD c % 8 (workgroup b runs on XCD b % 8),
// an XCD takes its chunks in order, a chunk's tiles in order, and the G
// query heads that share the KV head back to back.  The keys and values of a
// row and KV head are then read from one XCD's L2 by all of its tiles and
// heads, instead of from the memory-side cache once per head.
constexpr int kFlashChunk = 16;

int flash_grid(int ntiles, int heads, int kv_heads) {
  const int chunks = (ntiles * kv_heads + kFlashChunk - 1) / kFlashChunk;
  return (chunks + 7) / 8 * 8 * kFlashChunk * (heads / kv_heads);
}

__global__ void __launch_bounds__(256, 2) k_pf_attn_flash(PrefillAttn a, int ntiles) {
  __shared__ __align__(16) unsigned char smem[kFlashLds];
  __shared__ float stat[2][2][32][2];  // [query half][key half][query][max, sum]
  bf16_t* Ks = reinterpret_cast<bf16_t*>(smem);  // [64 keys][136]
  bf16_t* Vs = Ks + kAk * kAkld;                  // [64 keys][144]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int tix, h;
  {
    const int G = a.heads / a.kv_heads;
    const int x = blockIdx.x & 7, s = blockIdx.x >> 3;
    const int k = s / (kFlashChunk * G), rem = s - k * (kFlashChunk * G);
    const int P = (k * 8 + x) * kFlashChunk + rem / G;
    if (P >= ntiles * a.kv_heads) return;  // padding of the last chunks (uniform)
    const int g = P / ntiles;
    tix = P - g * ntiles;
    h = g * G + rem % G;
  }
  const int4 tile = a.tiles[tix];  // first query token, first token of the row, queries, first query's position
  const int m_start = tile.x, r0 = tile.y, nqt = tile.z, p0 = tile.w;
  const int nq = a.heads, kvh = h / (a.heads / a.kv_heads);
  const bf16_t* qkv = static_cast<const bf16_t*>(a.qkv);
  const size_t koff = (size_t)nq * kAd + (size_t)kvh * kAd;
  const size_t voff = (size_t)(nq + a.kv_heads) * kAd + (size_t)kvh * kAd;
  const int nkeys = p0 + nqt;
  const int nkt = (nkeys + kAk - 1) / kAk;
  const int sm = wave >> 1, sn = wave & 1, hi = lane >> 5;
  const int qloc = sm * 32 + (lane & 31);  // this lane's query within the tile
  const int qlim = p0 + qloc;              // its visible keys: j <= qlim
  constexpr float kLog2e = 1.44269504088896340736f;

  // Q fragments (B operand): query qloc (rows past the tile read the last one)
  bf16x8_t qf[kAd / 16];
  {
    const int qi = min(qloc, nqt - 1);
    const bf16_t* qrow = qkv + (size_t)(m_start + qi) * a.ld + (size_t)h * kAd + hi * 8;
#pragma unroll
    for (int ks = 0; ks < kAd / 16; ++ks) qf[ks] = lds_frag(qrow + ks * 16);
  }
  // Key tile in registers: vector v = tid + 256 i is key v / 16, elements
  // (v % 16) * 8 ..+8.  Value tile: key v % 64, elements (v / 64) * 8 ..+8.
  // Both go to LDS row-major.  Keys past the row read the last one.
  re_u32x4 kpre[4], vpre[4];
  auto load_k = [&](int kt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int v = tid + 256 * i;
      const int tok = r0 + min(min(kt, nkt - 1) * kAk + (v >> 4), nkeys - 1);
      kpre[i] = *reinterpret_cast<const re_u32x4*>(qkv + (size_t)tok * a.ld + koff + (v & 15) * 8);
    }
  };
  auto load_v = [&](int kt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int v = tid + 256 * i;
      const int tok = r0 + min(min(kt, nkt - 1) * kAk + (v & 63), nkeys - 1);
      vpre[i] = *reinterpret_cast<const re_u32x4*>(qkv + (size_t)tok * a.ld + voff + (v >> 6) * 8);
    }
  };
  auto store_k = [&]() {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int v = tid + 256 * i;
      *reinterpret_cast<re_u32x4*>(&Ks[(v >> 4) * kAkld + (v & 15) * 8]) = kpre[i];
    }
  };
  auto store_v = [&]() {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int v = tid + 256 * i, key = v & 63, c = (v >> 6) * 8;
      *reinterpret_cast<re_u32x4*>(&Vs[key * kAvld + c]) = vpre[i];
    }
  };
  // Scores of key tile kt for this lane's query: s[v] is key
  // kt * 64 + sn * 32 + 8 (v / 4) + 4 hi + v % 4.  MASKED: the tile reaches
  // past some query's causal limit (the tiles before nfull end at or before
  // the first query's position, so every query sees all of their keys).
  auto scores = [&](int kt, float (&sc)[16], auto masked) {
    f32x16_t acc;
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[v] = 0.f;
#pragma unroll
    for (int ks = 0; ks < kAd / 16; ++ks) {
      const bf16x8_t kf = lds_frag(&Ks[(sn * 32 + (lane & 31)) * kAkld + ks * 16 + hi * 8]);
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[ks], acc, 0, 0, 0);
    }
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const float x = round_bf16(div_sqrt128_bf16(round_bf16(acc[v])));
      if constexpr (decltype(masked)::value) {
        const int j = kt * kAk + sn * 32 + 8 * (v >> 2) + 4 * hi + (v & 3);
        sc[v] = j <= qlim ? x : -INFINITY;
      } else {
        sc[v] = x;
      }
    }
  };
  const int nfull = min(nkt, (p0 + 1) / kAk);

  // Pass 1: row max and sum.  A masked score adds exp2(-inf) = 0; while all
  // of a lane's scores so far are masked (m = -inf) its sum stays 0.
  float m = -INFINITY, l = 0.f;
  auto pass1 = [&](int kt, auto masked) {
#pragma clang fp contract(off)  // the rescaled sum is a product, then a sum
    store_k();
    load_k(kt + 1);
    lds_barrier();
    float sc[16];
    scores(kt, sc, masked);
    float tmax = sc[0];
#pragma unroll
    for (int v = 1; v < 16; ++v) tmax = fmaxf(tmax, sc[v]);
    const float mn = fmaxf(m, tmax);
    const float bn = mn == -INFINITY ? 0.f : mn * kLog2e;
    float add = 0.f;
#pragma unroll
    for (int v = 0; v < 16; ++v) add += __builtin_amdgcn_exp2f(fmaf(sc[v], kLog2e, -bn));
    l = l * __builtin_amdgcn_exp2f(fmaf(m, kLog2e, -bn)) + add;
    m = mn;
    lds_barrier();
  };
  load_k(0);
  {
    int kt = 0;
    for (; kt < nfull; ++kt) pass1(kt, std::false_type{});
    for (; kt < nkt; ++kt) pass1(kt, std::true_type{});
  }
  {
    const float m2 = __shfl_xor(m, 32, 64), l2 = __shfl_xor(l, 32, 64);
    const float mm = fmaxf(m, m2);
    const float bm = mm * kLog2e;
    const float a1 = m == -INFINITY ? 0.f : l * __builtin_amdgcn_exp2f(fmaf(m, kLog2e, -bm));
    const float a2 = m2 == -INFINITY ? 0.f : l2 * __builtin_amdgcn_exp2f(fmaf(m2, kLog2e, -bm));
    m = mm;
    l = a1 + a2;
  }
  if (hi == 0) {
    stat[sm][sn][lane & 31][0] = m;
    stat[sm][sn][lane & 31][1] = l;
  }
  lds_barrier();
  float M, inv;
  {
    const float m0 = stat[sm][0][lane & 31][0], l0 = stat[sm][0][lane & 31][1];
    const float m1 = stat[sm][1][lane & 31][0], l1 = stat[sm][1][lane & 31][1];
    M = fmaxf(m0, m1);
    const float bm = M * kLog2e;
    const float a0 = m0 == -INFINITY ? 0.f : l0 * __builtin_amdgcn_exp2f(fmaf(m0, kLog2e, -bm));
    const float a1 = m1 == -INFINITY ? 0.f : l1 * __builtin_amdgcn_exp2f(fmaf(m1, kLog2e, -bm));
    const float L = a0 + a1;
    inv = L > 0.f ? 1.0f / L : 0.f;
  }
  const float base = M * kLog2e;

  // Pass 2: P V.
  f32x16_t o[4];
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int v = 0; v < 16; ++v) o[t][v] = 0.f;
  // M is finite (key 0 is visible to every query), so a masked score's
  // probability is exp2(-inf) = 0.
  auto pass2 = [&](int kt, auto masked) {
    store_k();
    store_v();
    load_k(kt + 1);
    load_v(kt + 1);
    lds_barrier();
    float sc[16];
    scores(kt, sc, masked);
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      float pv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) pv[e] = __builtin_amdgcn_exp2f(fmaf(sc[8 * b + e], kLog2e, -base)) * inv;
      re_u32x4 pw;
#pragma unroll
      for (int e = 0; e < 4; ++e) pw[e] = f2_to_bf16x2(pv[2 * e], pv[2 * e + 1]);
      const bf16x8_t af = __builtin_bit_cast(bf16x8_t, pw);
      const int kb = sn * 32 + 16 * b + 4 * hi;
      // Value operand by transposing LDS reads (ds_read_b64_tr_b16): in each
      // 16-lane group, lane q + 4 r names the 8 bytes of dims 4 q .. 4 q + 3
      // of key row kb + r, and lane i receives dim i's values of the 4 keys
      // in key order -- the 4 keys lane i's MFMA column needs.
      const int gi = lane & 15, q4 = (gi & 3) * 4, rr = gi >> 2, d16 = ((lane >> 4) & 1) * 16;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const bf16_t* vr = &Vs[(kb + rr) * kAvld + t * 32 + d16 + q4];
        const lds_v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_ptr)vr);
        const lds_v4i16 up = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_ptr)(vr + 8 * kAvld));
        const uint2 l2 = __builtin_bit_cast(uint2, lo), u2 = __builtin_bit_cast(uint2, up);
        const re_u32x4 bw = {l2.x, l2.y, u2.x, u2.y};
        o[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, __builtin_bit_cast(bf16x8_t, bw), o[t], 0, 0, 0);
      }
    }
    lds_barrier();
  };
  load_k(0);
  load_v(0);
  {
    int kt = 0;
    for (; kt < nfull; ++kt) pass2(kt, std::false_type{});
    for (; kt < nkt; ++kt) pass2(kt, std::true_type{});
  }
  // The two key halves' partial O: the sn = 1 waves hand theirs over in LDS
  // (the tiles are free now), the sn = 0 waves add (sn 0 + sn 1) and store.
  float* ox = reinterpret_cast<float*>(smem);  // [2 query halves][4][16][64]
  if (sn == 1) {
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int v = 0; v < 16; ++v) ox[((sm * 4 + t) * 16 + v) * 64 + lane] = o[t][v];
  }
  lds_barrier();
  if (sn == 0) {
    bf16_t* out = static_cast<bf16_t*>(a.out);
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int qi = sm * 32 + 8 * (v >> 2) + 4 * hi + (v & 3);
        const int col = t * 32 + (lane & 31);
        const float y = o[t][v] + ox[((sm * 4 + t) * 16 + v) * 64 + lane];
        if (qi < nqt) out[(size_t)(m_start + qi) * nq * kAd + (size_t)h * kAd + col] = f_to_bf16(y);
      }
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
  if (n % 8 != 0) return hipErrorInvalidValue;  // rows of the intermediate size, a multiple of 8
  const int blocks = static_cast<int>(std::min<long long>((n / 8 + 255) / 256, 16384));
  if (dtype_bytes == 2)
    k_pf_swiglu<bf16_t><<<blocks, 256, 0, stream>>>(gate, up, out, n);
  else
    k_pf_swiglu<float><<<blocks, 256, 0, stream>>>(gate, up, out, n);
  return hipGetLastError();
}

hipError_t launch_prefill_qkv_post(const PrefillQkv& a, int dtype_bytes, hipStream_t stream) {
  if (a.M <= 0) return hipSuccess;
  if (a.head_dim % 16 != 0 || a.ld % 8 != 0) return hipErrorInvalidValue;
  if (dtype_bytes == 2)
    k_pf_qkv_post<bf16_t><<<a.M, 256, 0, stream>>>(a);
  else
    k_pf_qkv_post<float><<<a.M, 256, 0, stream>>>(a);
  return hipGetLastError();
}

hipError_t launch_gemm(const GemmArgs& a, int epi, int dtype_bytes, hipStream_t stream) {
  if (a.M <= 0 || a.N <= 0) return hipSuccess;
  if (dtype_bytes == 2) {
    const bool swiglu = epi == kGemmSwiGlu;
    const bool aligned = ((reinterpret_cast<uintptr_t>(a.A) | reinterpret_cast<uintptr_t>(a.W) |
                           reinterpret_cast<uintptr_t>(a.out) | reinterpret_cast<uintptr_t>(swiglu ? a.W2 : a.W)) &
                          15) == 0;
    if (a.K <= 0 || a.K % kGk != 0 || a.N % 8 != 0 || a.lda % 8 != 0 || a.ldw % 8 != 0 || a.ldo % 8 != 0 ||
        !aligned || (swiglu && a.W2 == nullptr))
      return hipErrorInvalidValue;
    static const hipError_t attr = [] {
      hipError_t e = hipSuccess;
      for (const void* k : {reinterpret_cast<const void*>(k_gemm_bf16<kGemmStore>),
                            reinterpret_cast<const void*>(k_gemm_bf16<kGemmResidual>),
                            reinterpret_cast<const void*>(k_gemm_bf16<kGemmSwiGlu>)})
        if (e == hipSuccess) e = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, kGsmem);
      return e;
    }();
    if (attr != hipSuccess) return attr;
    const int tile_n = swiglu ? kGn / 2 : kGn;
    const int nM = (a.M + kGm - 1) / kGm, nN = (a.N + tile_n - 1) / tile_n;
    if (epi == kGemmStore)
      k_gemm_bf16<kGemmStore><<<nM * nN, kGthreads, kGsmem, stream>>>(a, nM, nN);
    else if (epi == kGemmResidual)
      k_gemm_bf16<kGemmResidual><<<nM * nN, kGthreads, kGsmem, stream>>>(a, nM, nN);
    else
      k_gemm_bf16<kGemmSwiGlu><<<nM * nN, kGthreads, kGsmem, stream>>>(a, nM, nN);
  } else {
    if (a.K <= 0 || epi == kGemmSwiGlu) return hipErrorInvalidValue;
    const dim3 grid((a.N + 63) / 64, (a.M + 63) / 64);
    if (epi == kGemmStore)
      k_gemm_f32<kGemmStore><<<grid, 256, 0, stream>>>(a);
    else
      k_gemm_f32<kGemmResidual><<<grid, 256, 0, stream>>>(a);
  }
  return hipGetLastError();
}

// The MFMA attention serves bf16 models with head_dim 128 (any window: its
// LDS does not depend on the prompt length).
bool prefill_attention_mfma(const Dims& d) { return d.dtype_bytes == 2 && d.head_dim == kAd; }

// Dynamic LDS of the per-(token, head) kernel: the scores of the window.
size_t prefill_attention_lds(const Dims& d, int max_keys) {
  (void)d;
  return (size_t)max_keys * sizeof(float);
}

hipError_t prepare_prefill(const Dims& d) {
  if (prefill_attention_mfma(d)) return hipSuccess;
  const int bytes = static_cast<int>(prefill_attention_lds(d, d.capacity));
  if (d.dtype_bytes == 2)
    return hipFuncSetAttribute(reinterpret_cast<const void*>(k_pf_attn_rows<bf16_t>),
                               hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  return hipFuncSetAttribute(reinterpret_cast<const void*>(k_pf_attn_rows<float>),
                             hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
}

hipError_t launch_prefill_attention(const PrefillAttn& a, const Dims& d, int ntiles, hipStream_t stream) {
  if (a.M <= 0) return hipSuccess;
  if (prefill_attention_mfma(d)) {
    if (ntiles <= 0) return hipErrorInvalidValue;
    if (d.heads % d.kv_heads != 0) return hipErrorInvalidValue;
    k_pf_attn_flash<<<flash_grid(ntiles, d.heads, d.kv_heads), 256, 0, stream>>>(a, ntiles);
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
