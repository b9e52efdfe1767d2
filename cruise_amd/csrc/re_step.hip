// Decoder-step kernels of the resident decode epoch (gfx950).
//
// A decoder step (batched_decoder_step.py:277-417) runs as
//   embed -> L x [qkv | attention | o-proj | gate/up | down (+reduce)] -> LM head.
//
// Every projection is a weight-streaming skinny GEMM: M = batch rows (4 at the
// reference geometry) against an [N, K] weight read exactly once.  A wave owns
// two weight rows over one K-segment of up to 7 x 512 elements (3584: all of
// Qwen2.5-7B's hidden size) and issues all 14 of its 16-byte non-temporal loads
// before touching them -- before the prologue, too -- so one HBM round trip
// covers a whole row pair.  Activations sit in LDS; bf16 pairs go through
// v_dot2 into fp32 accumulators; the 64 lanes are combined by a halving
// exchange.  Norms, RoPE, the paged slot write, SwiGLU, the residual adds and
// the argmax partials are fused into prologues and epilogues; rounding points
// follow the reference decoder (see the per-kernel comments).
#include "re_device.h"
#include "re_layout.h"

namespace re {
namespace {

constexpr int kRowsPerWave = 2;
constexpr int kChunk = 512;     // elements covered by one wave-wide 16-byte load
constexpr int kSegChunks = 7;   // chunks per K-segment
constexpr int kSeg = kChunk * kSegChunks;

__device__ __forceinline__ bool skip_step(const int32_t* done) {
  return done != nullptr && __builtin_nontemporal_load(done) != 0;
}

// Issue the loads of RPW weight rows over the segment [k0, k0 + len): chunk c
// of lane l covers elements k0 + c*512 + l*8 .. +8.  Chunks past len are zero.
template <typename T, int RPW>
__device__ __forceinline__ void load_rows(Vec8<T> (&w)[kSegChunks][RPW], const T* const (&wr)[RPW], int k0,
                                          int len, int lane) {
#pragma unroll
  for (int c = 0; c < kSegChunks; ++c) {
    const int k = c * kChunk + lane * 8;
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      if (k < len)
        w[c][r] = Vec8<T>::load(wr[r] + k0 + k);
      else
        w[c][r] = Vec8<T>{};
    }
  }
}

// acc[r][m] += sum over the segment of W_r[k] * xs[m][k] (xs: LDS, row stride ldx).
template <typename T, int MB, int RPW>
__device__ __forceinline__ void dot_rows(const Vec8<T> (&w)[kSegChunks][RPW], const T* xs, int ldx, int len,
                                         int lane, float (&acc)[RPW][MB]) {
#pragma unroll
  for (int c = 0; c < kSegChunks; ++c) {
    const int k = c * kChunk + lane * 8;
    if (k < len) {
#pragma unroll
      for (int m = 0; m < MB; ++m) {
        const Vec8<T> x = Vec8<T>::load_cached(xs + m * ldx + k);
#pragma unroll
        for (int r = 0; r < RPW; ++r) acc[r][m] = dot8(w[c][r], x, acc[r][m]);
      }
    }
  }
}

// Reduce acc over the wave and leave the totals in red[r*MB + m] (LDS).
template <int MB, int RPW>
__device__ __forceinline__ void wave_totals(float (&acc)[RPW][MB], int lane, float* red) {
  constexpr int N = MB * RPW;
  float v[N];
#pragma unroll
  for (int r = 0; r < RPW; ++r)
#pragma unroll
    for (int m = 0; m < MB; ++m) v[r * MB + m] = acc[r][m];
  wave_reduce_transpose<N>(v, lane);
  if ((lane & (64 / N - 1)) == 0) red[lane / (64 / N)] = v[0];
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
}

// RMSNorm of rows b0..b0+MB-1 of hidden [B, H] into LDS xs [MB, H]
// (batched_decoder_step.py:224-229): fp32 mean of squares, rsqrt(var + eps),
// cast to T, then a T x T product with the weight.  Rows >= B are zero.
// Vec8 slots a 256-thread workgroup needs to hold MB rows of one K-segment.
template <int MB>
constexpr int seg_vecs_per_thread() {
  return (MB * kSeg / 8 + 255) / 256;
}

// Load rows b0..b0+MB-1, columns [k0, k0+len), of X [B, ldg] into registers:
// slot i of thread t holds Vec8 number t + 256*i of the row-major [MB, len]
// block (zero for rows >= B).  All loads are issued before any is used.
template <typename T, int MB>
__device__ __forceinline__ void load_rows_block(Vec8<T> (&v)[seg_vecs_per_thread<MB>()], const T* __restrict__ X,
                                                int ldg, int b0, int B, int k0, int len) {
  const int per_row = len / 8;
#pragma unroll
  for (int i = 0; i < seg_vecs_per_thread<MB>(); ++i) {
    const int idx = threadIdx.x + 256 * i;
    const int m = idx / max(per_row, 1), k = (idx - m * per_row) * 8;
    v[i] = Vec8<T>{};
    if (idx < MB * per_row && b0 + m < B) v[i] = Vec8<T>::load_cached(X + (size_t)(b0 + m) * ldg + k0 + k);
  }
}

// RMSNorm of rows b0..b0+MB-1 of hidden [B, H] into LDS xs [MB, H]
// (batched_decoder_step.py:224-229): fp32 mean of squares, rsqrt(var + eps),
// cast to T, then a T x T product with the weight.  Rows >= B are zero.
// Requires blockDim.x == 256 and H <= kSeg.
template <typename T, int MB>
__device__ void rmsnorm_to_lds(const T* __restrict__ hidden, int b0, int B, const T* __restrict__ w, int H,
                               float eps, T* xs, float* red) {
  constexpr int NV = seg_vecs_per_thread<MB>();
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int per_row = H / 8;
  Vec8<T> hv[NV], wv[NV];
  load_rows_block<T, MB>(hv, hidden, H, b0, B, 0, H);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int idx = tid + 256 * i;
    wv[i] = Vec8<T>{};
    if (idx < MB * per_row) wv[i] = Vec8<T>::load_cached(w + (idx % per_row) * 8);
  }
  float ss[MB];
#pragma unroll
  for (int m = 0; m < MB; ++m) ss[m] = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int idx = tid + 256 * i;
    const int row = idx / per_row;
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float x = hv[i].get(e);
      s = fmaf(x, x, s);
    }
#pragma unroll
    for (int m = 0; m < MB; ++m)
      if (row == m) ss[m] += s;
  }
#pragma unroll
  for (int m = 0; m < MB; ++m) {
    const float s = wave_sum(ss[m]);
    if (lane == 0) red[wave * MB + m] = s;
  }
  __syncthreads();
  float rs[MB];
  const int nw = blockDim.x >> 6;
#pragma unroll
  for (int m = 0; m < MB; ++m) {
    float s = 0.f;
    for (int i = 0; i < nw; ++i) s += red[i * MB + m];
    rs[m] = rsqrtf(s / static_cast<float>(H) + eps);
  }
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int idx = tid + 256 * i;
    if (idx < MB * per_row) {
      const int row = idx / per_row, k = (idx - row * per_row) * 8;
      float r = 0.f;
#pragma unroll
      for (int m = 0; m < MB; ++m)
        if (row == m) r = rs[m];
      float out[8];
#pragma unroll
      for (int e = 0; e < 8; ++e)
        out[e] = b0 + row < B ? Elt<T>::r(Elt<T>::r(hv[i].get(e) * r) * wv[i].get(e)) : 0.f;
      *reinterpret_cast<Vec8<T>*>(xs + row * H + k) = Vec8<T>::from_floats(out);
    }
  }
  __syncthreads();
}

// ---------------------------------------------------------------------------
// Normed projections: RMSNorm prologue + skinny GEMM + fused epilogue.
// ---------------------------------------------------------------------------
enum NormedKind { kQkv = 0, kGateUp = 1, kLmHead = 2 };

struct NormedArgs {
  const int32_t* done;
  const void* hidden;     // T [B, H]
  const void* norm_w;     // T [H]
  const void* w0;         // qkv: stacked [qkv_rows, H]; gate/up: gate [I, H]; lm: [V, H]
  const void* w1;         // gate/up: up [I, H]; qkv: bias [qkv_rows]
  void* out;              // qkv: q [B, NH*d]; gate/up: mlp [B, I]
  float* logits;          // lm head: fp32 [B, V]
  float* am_val;          // lm head argmax partials [gridDim.x, B]
  int32_t* am_idx;
  int32_t* am_bad;
  // qkv epilogue
  const int64_t* pos;
  const int32_t* slot;
  const int32_t* active;
  void* key_cache;        // this layer: [slots, KVH, d]
  void* value_cache;
  const float* inv_freq;  // [d/2]
  long long slots;
  int B, H, units, heads, kv_heads, head_dim;
  float eps;
};

template <int KIND, typename T>
__device__ __forceinline__ void normed_rows(const NormedArgs& a, int u, const T* W0, const T* W1,
                                            const T* (&wr)[kRowsPerWave], int& row0, int& row1) {
  const int H = a.H;
  if constexpr (KIND == kQkv) {
    const int half = a.head_dim >> 1;
    const int hg = u / half, j = u - hg * half;
    row0 = hg * a.head_dim + j;
    row1 = row0 + half;
    wr[0] = W0 + (size_t)row0 * H;
    wr[1] = W0 + (size_t)row1 * H;
  } else if constexpr (KIND == kGateUp) {
    row0 = row1 = u;
    wr[0] = W0 + (size_t)u * H;
    wr[1] = W1 + (size_t)u * H;
  } else {
    row0 = 2 * u;
    row1 = row0 + 1;
    wr[0] = W0 + (size_t)row0 * H;
    wr[1] = W0 + (size_t)row1 * H;
  }
}

template <typename T, int MB, int WAVES, int KIND>
__global__ void __launch_bounds__(WAVES * 64) k_normed(NormedArgs a) {
  if (skip_step(a.done)) return;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  T* xs = reinterpret_cast<T*>(smem_raw);
  float* red = reinterpret_cast<float*>(smem_raw + (size_t)MB * a.H * sizeof(T));
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int b0 = blockIdx.y * MB;
  const int H = a.H;
  const T* W0 = static_cast<const T*>(a.w0);
  const T* W1 = static_cast<const T*>(a.w1);
  float* wred = red + wave * (kRowsPerWave * MB);
  const int stride = gridDim.x * WAVES;
  int u = blockIdx.x * WAVES + wave;

  // The first row pair's weights are requested before the prologue.
  Vec8<T> w[kSegChunks][kRowsPerWave];
  const T* wr[kRowsPerWave];
  int row0 = 0, row1 = 0;
  if (u < a.units) {
    normed_rows<KIND, T>(a, u, W0, W1, wr, row0, row1);
    load_rows<T, kRowsPerWave>(w, wr, 0, H, lane);
  }
  rmsnorm_to_lds<T, MB>(static_cast<const T*>(a.hidden), b0, a.B, static_cast<const T*>(a.norm_w), H, a.eps, xs,
                        red);
  // argmax running state of lane m < MB (batch row b0+m), LM head only
  float best_v = 0.f;
  int best_i = -1;
  int bad = 0;
  auto process = [&](const Vec8<T>(&wv)[kSegChunks][kRowsPerWave], int u, int row0, int row1) {
    float acc[kRowsPerWave][MB];
#pragma unroll
    for (int r = 0; r < kRowsPerWave; ++r)
#pragma unroll
      for (int m = 0; m < MB; ++m) acc[r][m] = 0.f;
    dot_rows<T, MB, kRowsPerWave>(wv, xs, H, H, lane, acc);
    wave_totals<MB, kRowsPerWave>(acc, lane, wred);
    const int m = lane;
    if (m < MB && b0 + m < a.B) {
      const int b = b0 + m;
      const float y0 = wred[0 * MB + m];
      const float y1 = wred[1 * MB + m];
      if constexpr (KIND == kQkv) {
        // F.linear with bias (g4a_linear_t_bias.py:18-21): fp32 sum + bias, one
        // rounding to T.  RoPE (batched_decoder_step.py:231-240, 323-324):
        // q' = q*cos + rotate_half(q)*sin, each product and the sum rounded to T.
        const T* bias = W1;
        const float qa = Elt<T>::r(y0 + Elt<T>::f(bias[row0]));
        const float qb = Elt<T>::r(y1 + Elt<T>::f(bias[row1]));
        const int half = a.head_dim >> 1;
        const int hg = u / half, j = u - hg * half;
        const int nq = a.heads, nkv = a.kv_heads;
        float oa = qa, ob = qb;
        if (hg < nq + nkv) {
          const float ang = static_cast<float>(a.pos[b]) * a.inv_freq[j];
          const float c = Elt<T>::r(cosf(ang));
          const float s = Elt<T>::r(sinf(ang));
          oa = Elt<T>::r(Elt<T>::r(qa * c) + Elt<T>::r(-qb * s));
          ob = Elt<T>::r(Elt<T>::r(qb * c) + Elt<T>::r(qa * s));
        }
        if (hg < nq) {
          T* q = static_cast<T*>(a.out) + (size_t)b * nq * a.head_dim + (size_t)hg * a.head_dim;
          q[j] = Elt<T>::t(oa);
          q[j + half] = Elt<T>::t(ob);
        } else {
          // Paged slot write (batched_decoder_step.py:250-264): active rows only,
          // slots outside [0, P*bs) write nothing.
          const int s = a.slot[b];
          if (a.active[b] != 0 && s >= 0 && s < a.slots) {
            const bool is_key = hg < nq + nkv;
            const int kvh = is_key ? hg - nq : hg - nq - nkv;
            T* cache = static_cast<T*>(is_key ? a.key_cache : a.value_cache) + ((size_t)s * nkv + kvh) * a.head_dim;
            cache[j] = Elt<T>::t(oa);
            cache[j + half] = Elt<T>::t(ob);
          }
        }
      } else if constexpr (KIND == kGateUp) {
        // gate = silu(x Wg^T), up = x Wu^T, product (batched_decoder_step.py:391-398),
        // each result rounded to T.
        const float g = Elt<T>::r(y0);
        const float up = Elt<T>::r(y1);
        const float sg = Elt<T>::r(g / (1.0f + expf(-g)));
        static_cast<T*>(a.out)[(size_t)b * a.units + u] = Elt<T>::t(Elt<T>::r(sg * up));
      } else {
        // LM head in T, then .float() (batched_decoder_step.py:405-408); argmax
        // partials keep the first index of the maximum (CTRL:99-119).
        const float l0 = Elt<T>::r(y0);
        const float l1 = Elt<T>::r(y1);
        const int V = 2 * a.units;
        a.logits[(size_t)b * V + row0] = l0;
        a.logits[(size_t)b * V + row1] = l1;
        if (!isfinite(l0) || !isfinite(l1)) bad = 1;
        if (best_i < 0 || l0 > best_v) {
          best_v = l0;
          best_i = row0;
        }
        if (l1 > best_v) {
          best_v = l1;
          best_i = row1;
        }
      }
    }
  };
  // Double buffer: the next row pair's loads are issued before the current
  // pair is consumed.  Unit indices past the end are clamped to the last unit,
  // so every iteration issues its loads unconditionally (results unused).
  Vec8<T> wb[kSegChunks][kRowsPerWave];
  int rb0 = 0, rb1 = 0;
  const int last = a.units - 1;
  while (u < a.units) {
    int un = u + stride;
    normed_rows<KIND, T>(a, min(un, last), W0, W1, wr, rb0, rb1);
    load_rows<T, kRowsPerWave>(wb, wr, 0, H, lane);
    process(w, u, row0, row1);
    u = un;
    if (u >= a.units) break;
    un = u + stride;
    normed_rows<KIND, T>(a, min(un, last), W0, W1, wr, row0, row1);
    load_rows<T, kRowsPerWave>(w, wr, 0, H, lane);
    process(wb, u, rb0, rb1);
    u = un;
  }
  if constexpr (KIND == kLmHead) {
    // Combine the waves of this workgroup; ties go to the lowest index.
    __syncthreads();
    float* cv = red;                                      // [WAVES][MB]
    int* ci = reinterpret_cast<int*>(red + WAVES * MB);  // [WAVES][MB]
    int* cb = ci + WAVES * MB;                            // [WAVES][MB]
    if (lane < MB) {
      cv[wave * MB + lane] = best_v;
      ci[wave * MB + lane] = best_i;
      cb[wave * MB + lane] = bad;
    }
    __syncthreads();
    if (tid < MB && b0 + tid < a.B) {
      float bv = 0.f;
      int bi = -1, bb = 0;
      for (int wv = 0; wv < WAVES; ++wv) {
        const int i = ci[wv * MB + tid];
        const float v = cv[wv * MB + tid];
        bb |= cb[wv * MB + tid];
        if (i < 0) continue;
        if (bi < 0 || v > bv || (v == bv && i < bi)) {
          bv = v;
          bi = i;
        }
      }
      const size_t o = (size_t)blockIdx.x * a.B + b0 + tid;
      a.am_val[o] = bv;
      a.am_idx[o] = bi;
      a.am_bad[o] = bb;
    }
  }
}

// ---------------------------------------------------------------------------
// Residual projections (o-proj, down-proj): h = h + T(x W^T).  Grid:
// (row groups, K-segments, row tiles).  One segment: the residual epilogue
// runs here.  Several segments: fp32 partials, combined by k_resid_reduce in a
// fixed order (deterministic, no atomics).
// ---------------------------------------------------------------------------
struct ResidArgs {
  const int32_t* done;
  const void* x;      // T [B, K]
  const void* w;      // T [N, K]
  void* hidden;       // T [B, N]
  float* partial;     // [segments, B, N]
  int B, N, K, segments;
};

template <typename T, int MB, int WAVES>
__global__ void __launch_bounds__(WAVES * 64) k_resid(ResidArgs a) {
  if (skip_step(a.done)) return;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  T* xs = reinterpret_cast<T*>(smem_raw);  // [MB][kSeg]
  float* red = reinterpret_cast<float*>(smem_raw + (size_t)MB * kSeg * sizeof(T));
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int seg = blockIdx.y, tile = blockIdx.z;
  const int b0 = tile * MB;
  const int k0 = seg * kSeg;
  const int len = min(a.K - k0, kSeg);
  const int u = blockIdx.x * WAVES + wave;  // rows 2u, 2u+1
  const int units = a.N / 2;
  const T* W = static_cast<const T*>(a.w);
  Vec8<T> w[kSegChunks][kRowsPerWave];
  if (u < units) {
    const T* wr[kRowsPerWave] = {W + (size_t)(2 * u) * a.K, W + (size_t)(2 * u + 1) * a.K};
    load_rows<T, kRowsPerWave>(w, wr, k0, len, lane);
  }
  // stage x[b0.., k0 : k0+len] into LDS: all loads first, then the stores
  constexpr int NV = seg_vecs_per_thread<MB>();
  Vec8<T> xv[NV];
  load_rows_block<T, MB>(xv, static_cast<const T*>(a.x), a.K, b0, a.B, k0, len);
  const int per_row = len / 8;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int idx = tid + 256 * i;
    if (idx < MB * per_row) {
      const int m = idx / per_row, k = (idx - m * per_row) * 8;
      *reinterpret_cast<Vec8<T>*>(xs + m * kSeg + k) = xv[i];
    }
  }
  __syncthreads();
  if (u >= units) return;
  float acc[kRowsPerWave][MB];
#pragma unroll
  for (int r = 0; r < kRowsPerWave; ++r)
#pragma unroll
    for (int m = 0; m < MB; ++m) acc[r][m] = 0.f;
  dot_rows<T, MB, kRowsPerWave>(w, xs, kSeg, len, lane, acc);
  float* wred = red + wave * (kRowsPerWave * MB);
  wave_totals<MB, kRowsPerWave>(acc, lane, wred);
  if (lane >= MB || b0 + lane >= a.B) return;
  const int b = b0 + lane;
  if (a.segments == 1) {
    T* Hd = static_cast<T*>(a.hidden);
#pragma unroll
    for (int r = 0; r < kRowsPerWave; ++r) {
      // o/down projection rounded to T (Bf16Materialize is the identity), then
      // the residual add in T (batched_decoder_step.py:380-386, 399-403).
      const size_t o = (size_t)b * a.N + 2 * u + r;
      Hd[o] = Elt<T>::t(Elt<T>::f(Hd[o]) + Elt<T>::r(wred[r * MB + lane]));
    }
  } else {
#pragma unroll
    for (int r = 0; r < kRowsPerWave; ++r)
      a.partial[((size_t)seg * a.B + b) * a.N + 2 * u + r] = wred[r * MB + lane];
  }
}

// Sum of the segment partials in segment order, rounded to T, residual add.
template <typename T>
__global__ void k_resid_reduce(const int32_t* done, const float* partial, void* hidden, int B, int N,
                               int segments) {
  if (skip_step(done)) return;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= B * N) return;
  float s = 0.f;
  for (int sp = 0; sp < segments; ++sp) s += partial[(size_t)sp * B * N + i];
  T* Hd = static_cast<T*>(hidden);
  Hd[i] = Elt<T>::t(Elt<T>::f(Hd[i]) + Elt<T>::r(s));
}

// ---------------------------------------------------------------------------
// Embedding gather (batched_decoder_step.py:289-291).
// ---------------------------------------------------------------------------
template <typename T>
__global__ void k_embed(const int32_t* done, const int64_t* token, const T* emb, T* hidden, int B, int H, int V) {
  if (skip_step(done)) return;
  const int b = blockIdx.x;
  long long t = token[b];
  if (t < 0 || t >= V) t = 0;  // the controller rejects such ids (CTRL:356); reads stay in bounds
  for (int k = threadIdx.x; k < H; k += blockDim.x) hidden[(size_t)b * H + k] = emb[(size_t)t * H + k];
}

}  // namespace

// ---------------------------------------------------------------------------
// Launcher
// ---------------------------------------------------------------------------
size_t normed_lds_bytes(int mb, int hidden, int dtype_bytes, int waves) {
  return (size_t)mb * hidden * dtype_bytes + 3 * (size_t)waves * mb * kRowsPerWave * sizeof(float);
}
size_t resid_lds_bytes(int mb, int dtype_bytes, int waves) {
  return (size_t)mb * kSeg * dtype_bytes + (size_t)waves * mb * kRowsPerWave * sizeof(float);
}
int k_segment_elems() { return kSeg; }

// The step is a fixed list of launches: embed, then per layer
// [qkv, attention, o-proj, o-reduce, gate/up, down, down-reduce], then the LM
// head.  Reduce entries launch nothing when their projection has a single
// K-segment.  [begin, end) selects a contiguous range of the list.
constexpr int kOpsPerLayer = 7;
constexpr int kGateUpOp = 4;

template <typename T, int MB>
static hipError_t decoder_step_t(const KernelEnv& env, const StepPtrs& st, hipStream_t stream, int begin,
                                 int end) {
  constexpr int WAVES = 4;
  const Dims& d = env.dims;
  const LaunchPlan& p = env.plan;
  const Scratch& sc = env.scratch;
  const int B = d.batch;
  const size_t cache_layer_elems = (size_t)d.slots() * d.kv_dim();
  int op = 0;
  auto want = [&]() {
    const bool w = op >= begin && op < end;
    ++op;
    return w;
  };
  if (want())
    k_embed<T><<<B, 256, 0, stream>>>(st.done, st.token, reinterpret_cast<const T*>(env.weights + env.embedding_off),
                                       static_cast<T*>(sc.hidden), B, d.hidden, d.vocab);
  const size_t normed_smem = normed_lds_bytes(MB, d.hidden, sizeof(T), WAVES);
  const size_t resid_smem = resid_lds_bytes(MB, sizeof(T), WAVES);
  const int reduce_blocks = (B * d.hidden + 255) / 256;
  for (int l = 0; l < d.layers; ++l) {
    const LayerOffsets& lo = env.layer_off[l];
    T* kc = static_cast<T*>(st.key_cache) + l * cache_layer_elems;
    T* vc = static_cast<T*>(st.value_cache) + l * cache_layer_elems;
    NormedArgs q{};
    q.done = st.done;
    q.hidden = sc.hidden;
    q.norm_w = env.weights + lo.input_norm;
    q.w0 = env.weights + lo.qkv_w;
    q.w1 = env.weights + lo.qkv_b;
    q.out = sc.q;
    q.pos = st.pos;
    q.slot = st.slot;
    q.active = st.active;
    q.key_cache = kc;
    q.value_cache = vc;
    q.inv_freq = sc.inv_freq;
    q.slots = d.slots();
    q.B = B;
    q.H = d.hidden;
    q.units = d.qkv_rows() / 2;
    q.heads = d.heads;
    q.kv_heads = d.kv_heads;
    q.head_dim = d.head_dim;
    q.eps = d.rms_eps;
    if (want()) k_normed<T, MB, WAVES, kQkv><<<dim3(p.qkv_grid, p.row_tiles), WAVES * 64, normed_smem, stream>>>(q);

    AttnArgs at{};
    at.done = st.done;
    at.q = sc.q;
    at.key_cache = kc;
    at.value_cache = vc;
    at.len = st.len;
    at.table = st.table;
    at.out = sc.attn;
    at.B = B;
    at.heads = d.heads;
    at.kv_heads = d.kv_heads;
    at.head_dim = d.head_dim;
    at.block_size = d.block_size;
    at.blocks_per_row = d.blocks_per_row;
    at.window = d.capacity;
    at.slots = d.slots();
    if (want()) {
      const hipError_t err = launch_attention(at, d, stream);
      if (err != hipSuccess) return err;
    }

    ResidArgs o{};
    o.done = st.done;
    o.x = sc.attn;
    o.w = env.weights + lo.o_w;
    o.hidden = sc.hidden;
    o.partial = sc.partial;
    o.B = B;
    o.N = d.hidden;
    o.K = d.q_dim();
    o.segments = p.o_segments;
    if (want())
      k_resid<T, MB, WAVES><<<dim3(p.o_grid, p.o_segments, p.row_tiles), WAVES * 64, resid_smem, stream>>>(o);
    if (want() && p.o_segments > 1)
      k_resid_reduce<T><<<reduce_blocks, 256, 0, stream>>>(st.done, sc.partial, sc.hidden, B, d.hidden,
                                                            p.o_segments);

    NormedArgs gu{};
    gu.done = st.done;
    gu.hidden = sc.hidden;
    gu.norm_w = env.weights + lo.post_norm;
    gu.w0 = env.weights + lo.gate_w;
    gu.w1 = env.weights + lo.up_w;
    gu.out = sc.mlp;
    gu.B = B;
    gu.H = d.hidden;
    gu.units = d.intermediate;
    gu.eps = d.rms_eps;
    if (want())
      k_normed<T, MB, WAVES, kGateUp><<<dim3(p.gu_grid, p.row_tiles), WAVES * 64, normed_smem, stream>>>(gu);

    ResidArgs dn{};
    dn.done = st.done;
    dn.x = sc.mlp;
    dn.w = env.weights + lo.down_w;
    dn.hidden = sc.hidden;
    dn.partial = sc.partial;
    dn.B = B;
    dn.N = d.hidden;
    dn.K = d.intermediate;
    dn.segments = p.down_segments;
    if (want())
      k_resid<T, MB, WAVES><<<dim3(p.down_grid, p.down_segments, p.row_tiles), WAVES * 64, resid_smem, stream>>>(dn);
    if (want() && p.down_segments > 1)
      k_resid_reduce<T><<<reduce_blocks, 256, 0, stream>>>(st.done, sc.partial, sc.hidden, B, d.hidden,
                                                            p.down_segments);
  }
  NormedArgs lm{};
  lm.done = st.done;
  lm.hidden = sc.hidden;
  lm.norm_w = env.weights + env.final_norm_off;
  lm.w0 = env.weights + env.lm_head_off;
  lm.logits = st.logits;
  lm.am_val = sc.am_val;
  lm.am_idx = sc.am_idx;
  lm.am_bad = sc.am_bad;
  lm.B = B;
  lm.H = d.hidden;
  lm.units = d.vocab / 2;
  lm.eps = d.rms_eps;
  if (want()) k_normed<T, MB, WAVES, kLmHead><<<dim3(p.lm_grid, p.row_tiles), WAVES * 64, normed_smem, stream>>>(lm);
  return hipGetLastError();
}

// Workgroups of each grid-stride projection: as many as are resident at once
// (from the compiled kernels' occupancy), trimmed so every workgroup runs the
// same number of row groups.
template <typename T, int MB>
static void plan_grids_t(LaunchPlan& p, const Dims& d, int cus) {
  constexpr int WAVES = 4;
  const size_t smem = normed_lds_bytes(MB, d.hidden, sizeof(T), WAVES);
  auto fit = [&](auto kernel, int groups) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, WAVES * 64, smem) != hipSuccess || per_cu < 1)
      per_cu = 1;
    const int resident = per_cu * cus;
    if (groups <= resident) return groups;
    const int iters = (groups + resident - 1) / resident;
    return (groups + iters - 1) / iters;
  };
  p.qkv_grid = fit(k_normed<T, MB, WAVES, kQkv>, (d.qkv_rows() / 2 + WAVES - 1) / WAVES);
  p.gu_grid = fit(k_normed<T, MB, WAVES, kGateUp>, (d.intermediate + WAVES - 1) / WAVES);
  p.lm_grid = fit(k_normed<T, MB, WAVES, kLmHead>, (d.vocab / 2 + WAVES - 1) / WAVES);
  p.lm_wg = p.lm_grid;
}

void plan_grids(LaunchPlan& p, const Dims& d, int cus) {
  const bool bf16 = d.dtype_bytes == 2;
  if (p.mb == 4) {
    if (bf16) plan_grids_t<bf16_t, 4>(p, d, cus);
    else plan_grids_t<float, 4>(p, d, cus);
  } else {
    if (bf16) plan_grids_t<bf16_t, 8>(p, d, cus);
    else plan_grids_t<float, 8>(p, d, cus);
  }
}

int step_op_count(const KernelEnv& env) { return 2 + kOpsPerLayer * env.dims.layers; }
int gateup_op_index(int layer) { return 1 + kOpsPerLayer * layer + kGateUpOp; }

hipError_t launch_step_ops(const KernelEnv& env, const StepPtrs& step, hipStream_t stream, int begin, int end) {
  const bool bf16 = env.dims.dtype_bytes == 2;
  if (env.plan.mb == 4)
    return bf16 ? decoder_step_t<bf16_t, 4>(env, step, stream, begin, end)
                : decoder_step_t<float, 4>(env, step, stream, begin, end);
  return bf16 ? decoder_step_t<bf16_t, 8>(env, step, stream, begin, end)
              : decoder_step_t<float, 8>(env, step, stream, begin, end);
}

hipError_t launch_decoder_step(const KernelEnv& env, const StepPtrs& step, hipStream_t stream) {
  return launch_step_ops(env, step, stream, 0, step_op_count(env));
}

}  // namespace re
