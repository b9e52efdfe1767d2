// Decoder-step kernels of the resident decode epoch (gfx950).
//
// A decoder step (batched_decoder_step.py:277-417) runs as
//   embed -> L x [qkv | attention | o-proj | gate/up | down | down-reduce]
//   -> LM head,
// six launches per layer at Qwen2.5-7B's shape (o-proj and down add a reduce
// launch each when their K spans more than one 3584-element segment).
//
// Every projection is a weight-streaming skinny GEMM: M = batch rows (4 at the
// reference geometry) against an [N, K] weight read exactly once.  A wave owns
// two weight rows over one K-segment of up to 7 x 512 elements (3584: all of
// Qwen2.5-7B's hidden size) and issues all 14 of its 16-byte non-temporal loads
// before touching them, so one HBM round trip covers a whole row pair.
// Activations sit in LDS; bf16 pairs go through v_dot2 into fp32
// accumulators; the 64 lanes are combined by a halving exchange.
//
// The projections that consume a norm (qkv, gate/up, LM head) compute it in
// their prologue from the residual stream: the hidden rows and the norm
// weight are requested first, then the first row pair's weights, so the norm
// is computed while the weights are in flight.  The residual adds happen in
// the epilogue of a single-segment projection (o-proj), or in the reduce
// launch that sums a split-K projection's segment partials in order (down:
// 18944 = five full segments and a tail, one workgroup column each, so every
// segment's loads are in flight at once).
// RoPE cos/sin are tabulated once per step.  RoPE, the paged slot write,
// SwiGLU and the argmax partials are fused into the epilogues; rounding
// points follow the reference decoder (see the per-kernel comments).
#include "re_device.h"
#include "re_gemv.h"
#include "re_layout.h"

namespace re {
namespace {

// Minimum waves per SIMD the bf16 projections are compiled for (register
// budget 512 / NORMED_MIN_WAVES per lane): four resident waves per SIMD with
// one row pair in flight each keep HBM busy.
#ifndef NORMED_MIN_WAVES
#define NORMED_MIN_WAVES 4
#endif

// ---------------------------------------------------------------------------
// Embedding gather (batched_decoder_step.py:289-291) and the step's RoPE table
// (DEC:235-240: fp32 angle pos * inv_freq, cos/sin cast to T; one table for
// every layer, as DEC computes it once per step).  One workgroup per row.
// ---------------------------------------------------------------------------
struct EmbedArgs {
  const int32_t* done;
  const int64_t* token;
  const void* embedding;
  void* hidden;           // T [B, H]
  const int64_t* pos;
  const float* inv_freq;  // [d/2]
  float* rope;            // [B, d/2, 2] cos, sin (rounded to T)
  int B, H, V, half;
};

template <typename T>
__global__ void __launch_bounds__(256) k_embed(EmbedArgs a) {
  if (skip_step(a.done)) return;
  const int b = blockIdx.x, tid = threadIdx.x;
  long long t = a.token[b];
  if (t < 0 || t >= a.V) t = 0;  // the controller rejects such ids (CTRL:356); reads stay in bounds
  for (int j = tid; j < a.half; j += blockDim.x) {
    const float ang = static_cast<float>(a.pos[b]) * a.inv_freq[j];
    a.rope[((size_t)b * a.half + j) * 2] = Elt<T>::r(cosf(ang));
    a.rope[((size_t)b * a.half + j) * 2 + 1] = Elt<T>::r(sinf(ang));
  }
  const T* src = static_cast<const T*>(a.embedding) + (size_t)t * a.H;
  T* dst = static_cast<T*>(a.hidden) + (size_t)b * a.H;
  for (int c = tid; c < a.H / 8; c += blockDim.x)
    *reinterpret_cast<Vec8<T>*>(dst + c * 8) = Vec8<T>::load_cached(src + c * 8);
}

// ---------------------------------------------------------------------------
// Normed projections: norm prologue + skinny GEMM + fused epilogue.
// Workgroup g owns the contiguous unit range [g*per, (g+1)*per) (per = iters
// x waves), so each workgroup's outputs (logits, mlp) form whole lines.
// ---------------------------------------------------------------------------
enum ProjKind { kQkv = 0, kGateUp = 1, kLmHead = 2 };

struct ProjArgs {
  const int32_t* done;
  const void* hidden;     // T [B, H] residual stream
  const void* norm_w;     // T [H]
  const void* w0;         // qkv: stacked [qkv_rows, H]; gate/up: gate [I, H]; lm: [V, H]
  const void* w1;         // gate/up: up [I, H]; qkv: bias [qkv_rows]
  void* out;              // qkv: q [B, NH*d]; gate/up: mlp [B, I]
  float* logits;          // lm head: fp32 [B, V]
  float* am_val;          // lm head argmax partials [gridDim.x, B]
  int32_t* am_idx;
  int32_t* am_bad;
  // qkv epilogue
  const float* rope;      // [B, d/2, 2]
  const int32_t* slot;
  const int32_t* active;
  void* key_cache;        // this layer: [slots, KVH, d]
  void* value_cache;
  long long slots;
  int B, H, units, heads, kv_heads, head_dim;
  float eps;
  // Slot-weighted unit ranges (gate/up and LM head; slot_cus == 0: equal
  // ranges): workgroup i runs in dispatch slot i / slot_cus of its CU and
  // takes a share of the units proportional to slot_w[slot].
  int slot_cus;
  int slot_shift;    // log2(slot_cus) when it is a power of two, else -1
  int slot_base[5];  // first unit of each slot's workgroups; slot_base[4] = units
};

// Unit range of workgroup g when the grid is 4 x slot_cus workgroups,
// dispatched round-robin over the CUs (g in slot g / cus of CU g % cus).
// The SIMD arbiter issues for the oldest waves first, so the later slots of
// a CU stream more slowly; giving them fewer units lets every slot finish
// together, which keeps enough loads in flight until the end.
// The host splits the units over the four slots in proportion to their
// weights (slot_base); inside a slot the workgroups split its units evenly.
// Plain 32-bit arithmetic (a shift where slot_cus is a power of two), so the
// first weight requests leave a few instructions into the kernel.
__device__ __forceinline__ int slot_prefix(const ProjArgs& a, int g) {
  const int cus = a.slot_cus;
  if (g >= 4 * cus) return a.units;
  const int sh = a.slot_shift;
  const int s = sh >= 0 ? g >> sh : g / cus;
  const int i = g - s * cus;
  const int b0 = s == 0 ? a.slot_base[0] : s == 1 ? a.slot_base[1] : s == 2 ? a.slot_base[2] : a.slot_base[3];
  const int b1 = s == 0 ? a.slot_base[1] : s == 1 ? a.slot_base[2] : s == 2 ? a.slot_base[3] : a.slot_base[4];
  const int n = b1 - b0;
  return b0 + (sh >= 0 ? (i * n) >> sh : i * n / cus);
}

template <int KIND, typename T>
__device__ __forceinline__ void proj_rows(const ProjArgs& a, int u, const T* W0, const T* W1,
                                          const T* (&wr)[kRowsPerWave], int& row0, int& row1) {
  const int H = a.H;
  if constexpr (KIND == kQkv) {
    // rows j and j + d/2 of one head: the RoPE pair
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

// Epilogue inputs of one qkv row pair for batch row b = b0 + lane (lanes <
// MB): the two biases and the row's RoPE cos/sin.  Requested together with the
// pair's weights so the epilogue needs no further memory round trip.
struct QkvEpi {
  float bias0, bias1, cos, sin;
  int slot, active;  // the row's paged slot and active flag (key/value rows)
};

template <typename T>
__device__ __forceinline__ QkvEpi qkv_epilogue_inputs(const ProjArgs& a, int u, int row0, int row1, int b) {
  QkvEpi e{0.f, 0.f, 1.f, 0.f, -1, 0};
  const T* bias = static_cast<const T*>(a.w1);
  e.bias0 = Elt<T>::f(bias[row0]);
  e.bias1 = Elt<T>::f(bias[row1]);
  const int half = a.head_dim >> 1;
  const int j = u % half;
  const int bc = min(b, a.B - 1);
  e.cos = a.rope[((size_t)bc * half + j) * 2];
  e.sin = a.rope[((size_t)bc * half + j) * 2 + 1];
  e.slot = a.slot[bc];
  e.active = a.active[bc];
  return e;
}

// Waves per SIMD a projection is compiled for.  qkv runs one row pair per
// wave (2,304 pairs fit the chip at once), so it trades the fourth wave for
// registers: its RoPE epilogue would spill at 128.
template <typename T, int MB, int KIND>
constexpr int proj_min_waves() {
  return (sizeof(T) == 2 && MB == 4) ? (KIND == 0 ? 3 : NORMED_MIN_WAVES) : 2;
}

template <typename T, int MB, int WAVES, int KIND, bool FULL>
__global__ void __launch_bounds__(WAVES * 64, (proj_min_waves<T, MB, KIND>())) k_proj(ProjArgs a) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  T* xs = reinterpret_cast<T*>(smem_raw);
  float* red = reinterpret_cast<float*>(smem_raw + (size_t)MB * a.H * sizeof(T));
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int b0 = blockIdx.y * MB;
  const int H = a.H;
  const T* W0 = static_cast<const T*>(a.w0);
  const T* W1 = static_cast<const T*>(a.w1);
  float* wred = red + wave * (kRowsPerWave * MB);
  int u_begin, u_end;
  if (a.slot_cus > 0) {
    u_begin = slot_prefix(a, blockIdx.x);
    u_end = slot_prefix(a, blockIdx.x + 1);
  } else {
    const int iters = (a.units + gridDim.x * WAVES - 1) / (gridDim.x * WAVES);
    u_begin = blockIdx.x * iters * WAVES;
    u_end = min((int)(blockIdx.x + 1) * iters * WAVES, a.units);
  }
  int u = u_begin + wave;

  // Issue order (loads complete in issue order): the early-exit flag, the
  // hidden rows and norm weight, then the first row pair's weights, so the
  // norm is computed while the weights are in flight.  The flag is uniform:
  // the workgroup leaves together, after the barriers.
  const int32_t stop = a.done != nullptr ? request_flag(a.done) : 0;
  NormIn<T, MB> nin;
  norm_load<T, MB>(nin, static_cast<const T*>(a.hidden), static_cast<const T*>(a.norm_w), b0, a.B, H, tid);
  // Unconditional (a wave past its range loads a valid pair it never uses):
  // with no branch around them the waits below count exactly these 14 loads.
  Vec8<T> w[kSegChunks][kRowsPerWave];
  const T* wr[kRowsPerWave];
  int row0 = 0, row1 = 0;
  proj_rows<KIND, T>(a, min(u, a.units - 1), W0, W1, wr, row0, row1);
  load_rows<T, kRowsPerWave, FULL>(w, wr, 0, H, lane);
  QkvEpi epi{};
  if constexpr (KIND == kQkv) epi = qkv_epilogue_inputs<T>(a, min(u, a.units - 1), row0, row1, b0 + lane);
  __builtin_amdgcn_sched_barrier(0);
  norm_to_lds<T, MB>(nin, b0, a.B, H, a.eps, xs, red + 3 * WAVES * kRowsPerWave * MB, tid);
  if (flag_set(stop)) return;
  // argmax running state of lane m < MB (batch row b0+m), LM head only
  float best_v = 0.f;
  int best_i = -1;
  int bad = 0;
  while (u < u_end) {
    // One row pair per iteration, its 14 loads issued (before the loop or at
    // the end of the previous iteration) before the first product waits; the
    // barriers keep the scheduler from sinking them towards their uses.  The
    // weights are dead during the epilogue, which keeps the register count at
    // four waves per SIMD.
    __builtin_amdgcn_sched_barrier(0);
    float acc[kRowsPerWave][MB];
#pragma unroll
    for (int r = 0; r < kRowsPerWave; ++r)
#pragma unroll
      for (int m = 0; m < MB; ++m) acc[r][m] = 0.f;
    dot_rows<T, MB, kRowsPerWave, FULL>(w, xs, H, 0, H, lane, acc);
    const int cu = u, c0 = row0, c1 = row1;
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
        const float qa = Elt<T>::r(y0 + epi.bias0);
        const float qb = Elt<T>::r(y1 + epi.bias1);
        const int half = a.head_dim >> 1;
        const int hg = cu / half, j = cu - hg * half;
        const int nq = a.heads, nkv = a.kv_heads;
        float oa = qa, ob = qb;
        if (hg < nq + nkv) {
          const float c = epi.cos, s = epi.sin;
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
          const int s = epi.slot;
          if (epi.active != 0 && s >= 0 && s < a.slots) {
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
        static_cast<T*>(a.out)[(size_t)b * a.units + cu] = Elt<T>::t(Elt<T>::r(sg * up));
      } else {
        // LM head in T, then .float() (batched_decoder_step.py:405-408); argmax
        // partials keep the first index of the maximum (CTRL:99-119).
        const float l0 = Elt<T>::r(y0);
        const float l1 = Elt<T>::r(y1);
        const int V = 2 * a.units;
        a.logits[(size_t)b * V + c0] = l0;
        a.logits[(size_t)b * V + c1] = l1;
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
    }
    u += WAVES;
    if (u < u_end) {
      proj_rows<KIND, T>(a, u, W0, W1, wr, row0, row1);
      load_rows<T, kRowsPerWave, FULL>(w, wr, 0, H, lane);
      if constexpr (KIND == kQkv) epi = qkv_epilogue_inputs<T>(a, u, row0, row1, b0 + lane);
    }
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
// qkv with K split over the waves (bf16, B <= 4, hidden = 7 x 512): one
// 7-wave workgroup per CU owns PAIRS RoPE row pairs, and wave w owns elements
// [512 w, 512 w + 512) of every one of them.  A lane needs only its 8
// elements of the 4 hidden rows, so it keeps them (normalized) in registers:
//   requests  the flag, its hidden elements and norm weights, all PAIRS
//             pairs' weights (2 x PAIRS 16-byte loads), the epilogue inputs;
//   RMSNorm   each wave's sums of squares go through LDS once (one barrier),
//             then every lane applies rs to its own elements
//             (batched_decoder_step.py:224-229, as norm_apply);
//   products  per pair a lane dots its elements; the 8 totals (2 rows x 4
//             batch rows) of every pair are reduced over the wave in one
//             transposing exchange and stored per (pair, wave);
//   epilogue  one thread per (pair, batch row) adds the 7 wave totals in wave
//             order, then bias, RoPE and the q / paged K/V writes exactly as
//             k_proj's qkv epilogue.
// No LDS staging of the activations and no barrier between the weights'
// arrival and the products; the sums run in another fp32 order than k_proj's
// (per-wave K ranges added at the end), within the model tolerance.
// ---------------------------------------------------------------------------
constexpr int kQkvKsWaves = 7;
constexpr int kQkvKsPairs = 9;  // Qwen2.5-7B: 2,304 pairs = 256 x 9

template <int PAIRS>
__global__ void __launch_bounds__(kQkvKsWaves * 64, 1) k_qkv_ksplit(ProjArgs a) {
  constexpr int MB = 4;
  __shared__ float nred[kQkvKsWaves][MB];
  __shared__ float pred[PAIRS * kQkvKsWaves * 8];
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_index(tid);
  const int H = a.H;
  const int k0 = wave * kChunk + lane * 8;  // this lane's elements
  const int u0 = blockIdx.x * PAIRS;
  const bf16_t* W0 = static_cast<const bf16_t*>(a.w0);
  const bf16_t* Hd = static_cast<const bf16_t*>(a.hidden);
  const int32_t stop = a.done != nullptr ? request_flag(a.done) : 0;
  Vec8<bf16_t> x[MB];
#pragma unroll
  for (int m = 0; m < MB; ++m) x[m] = Vec8<bf16_t>::load_cached(Hd + (size_t)min(m, a.B - 1) * H + k0);
  const Vec8<bf16_t> nw = Vec8<bf16_t>::load_cached(static_cast<const bf16_t*>(a.norm_w) + k0);
  Vec8<bf16_t> w[PAIRS][2];
#pragma unroll
  for (int p = 0; p < PAIRS; ++p) {
    const bf16_t* wr[kRowsPerWave];
    int row0, row1;
    proj_rows<kQkv, bf16_t>(a, min(u0 + p, a.units - 1), W0, nullptr, wr, row0, row1);
    w[p][0] = Vec8<bf16_t>::load(wr[0] + k0);
    w[p][1] = Vec8<bf16_t>::load(wr[1] + k0);
  }
  // epilogue inputs of thread t < PAIRS * MB: pair t / MB, batch row t % MB
  const int ep = min(tid / MB, PAIRS - 1), em = tid % MB;
  const int eu = min(u0 + ep, a.units - 1);
  int er0 = 0, er1 = 0;
  {
    const bf16_t* wr[kRowsPerWave];
    proj_rows<kQkv, bf16_t>(a, eu, W0, nullptr, wr, er0, er1);
  }
  const QkvEpi epi = qkv_epilogue_inputs<bf16_t>(a, eu, er0, er1, em);
  __builtin_amdgcn_sched_barrier(0);

  // RMSNorm: the rows' sums of squares over the workgroup, rs, then each
  // lane normalizes its own elements.
  float ss[MB];
#pragma unroll
  for (int m = 0; m < MB; ++m) {
    float t = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) t = fmaf(x[m].get(e), x[m].get(e), t);
    ss[m] = t;
  }
  wave_reduce_transpose<MB>(ss, lane);
  if ((lane & (64 / MB - 1)) == 0) nred[wave][lane / (64 / MB)] = ss[0];
  lds_barrier();
  if (flag_set(stop)) return;  // uniform
  Vec8<bf16_t> y[MB];
#pragma unroll
  for (int m = 0; m < MB; ++m) {
    float total = 0.f;
#pragma unroll
    for (int q = 0; q < kQkvKsWaves; ++q) total += nred[q][m];
    y[m] = norm_apply<bf16_t>(x[m], nw, rsqrtf(total / static_cast<float>(H) + a.eps));
  }

  // Products: value index 8 p + 4 r + m for pair p, row r, batch row m.
  float v[PAIRS * 8];
#pragma unroll
  for (int p = 0; p < PAIRS; ++p)
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int m = 0; m < MB; ++m) v[p * 8 + r * 4 + m] = dot8(w[p][r], y[m], 0.f);
  constexpr int kFull = (PAIRS * 8) / 64;  // whole groups of 64 values
  static_assert(PAIRS * 8 - kFull * 64 == 0 || PAIRS * 8 - kFull * 64 == 8, "a tail of one pair at most");
#pragma unroll
  for (int gq = 0; gq < kFull; ++gq) {
    float t[64];
#pragma unroll
    for (int i = 0; i < 64; ++i) t[i] = v[gq * 64 + i];
    wave_reduce_transpose<64>(t, lane);  // lane l: total of value 64 gq + l
    const int idx = gq * 64 + lane;
    pred[((idx >> 3) * kQkvKsWaves + wave) * 8 + (idx & 7)] = t[0];
  }
  if constexpr (PAIRS * 8 > kFull * 64) {
    float t[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) t[i] = v[kFull * 64 + i];
    wave_reduce_transpose<8>(t, lane);  // lane l: total of value 8 kFull + l / 8
    if ((lane & 7) == 0) pred[((kFull * 8) * kQkvKsWaves + wave) * 8 + (lane >> 3)] = t[0];
  }
  lds_barrier();
  if (tid >= PAIRS * MB || u0 + ep >= a.units || em >= a.B) return;
  float y0 = 0.f, y1 = 0.f;
#pragma unroll
  for (int q = 0; q < kQkvKsWaves; ++q) {
    y0 += pred[(ep * kQkvKsWaves + q) * 8 + em];
    y1 += pred[(ep * kQkvKsWaves + q) * 8 + 4 + em];
  }
  // F.linear with bias, then RoPE and the stores: k_proj's qkv epilogue.
  const float qa = Elt<bf16_t>::r(y0 + epi.bias0);
  const float qb = Elt<bf16_t>::r(y1 + epi.bias1);
  const int half = a.head_dim >> 1;
  const int hg = eu / half, j = eu - hg * half;
  const int nq = a.heads, nkv = a.kv_heads;
  float oa = qa, ob = qb;
  if (hg < nq + nkv) {
    oa = Elt<bf16_t>::r(Elt<bf16_t>::r(qa * epi.cos) + Elt<bf16_t>::r(-qb * epi.sin));
    ob = Elt<bf16_t>::r(Elt<bf16_t>::r(qb * epi.cos) + Elt<bf16_t>::r(qa * epi.sin));
  }
  if (hg < nq) {
    bf16_t* q = static_cast<bf16_t*>(a.out) + (size_t)em * nq * a.head_dim + (size_t)hg * a.head_dim;
    q[j] = Elt<bf16_t>::t(oa);
    q[j + half] = Elt<bf16_t>::t(ob);
  } else if (epi.active != 0 && epi.slot >= 0 && epi.slot < a.slots) {
    const bool is_key = hg < nq + nkv;
    const int kvh = is_key ? hg - nq : hg - nq - nkv;
    bf16_t* cache = static_cast<bf16_t*>(is_key ? a.key_cache : a.value_cache) + ((size_t)epi.slot * nkv + kvh) * a.head_dim;
    cache[j] = Elt<bf16_t>::t(oa);
    cache[j + half] = Elt<bf16_t>::t(ob);
  }
}

// ---------------------------------------------------------------------------
// Residual projections, split-K form (o-proj; down when its activations do
// not fit one workgroup's LDS): x W^T per K-segment.  Grid: (row groups,
// K-segments, row tiles).  One segment: the residual add happens here
// (h = T(h + T(x W^T)), batched_decoder_step.py:380-386, 399-403).  Several:
// fp32 partials, added by k_resid_reduce in segment order (deterministic).
// ---------------------------------------------------------------------------
struct ResidArgs {
  const int32_t* done;
  const void* x;      // T [B, K]
  const void* w;      // T [N, K]
  void* hidden;       // T [B, N]
  float* partial;     // [segments, B, N]
  int B, N, K, segments;
};

// The body for one segment kind: FULL segments (len == kSeg) need no guards.
// Each kind is a complete path (loads, staging, products, stores), so the
// waits of one path count only its own loads.
template <typename T, int MB, int WAVES, bool FULL>
__device__ __forceinline__ void resid_segment(const ResidArgs& a, T* xs, float* red, int seg, int len) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int b0 = blockIdx.z * MB;
  const int k0 = seg * kSeg;
  const int u = blockIdx.x * WAVES + wave;  // rows 2u, 2u+1
  const int units = a.N / 2;
  const int uc = min(u, units - 1);
  const T* W = static_cast<const T*>(a.w);
  T* Hd = static_cast<T*>(a.hidden);
  // Flag, residual values (single segment), activations, then weights; the
  // weight loads are unconditional (clamped to a valid pair).
  const int32_t stop = a.done != nullptr ? request_flag(a.done) : 0;
  // (unconditional, clamped: used by lanes < MB of single-segment launches)
  const size_t hrow = (size_t)min(b0 + lane, a.B - 1) * a.N;
  const T h0 = Hd[hrow + 2 * uc], h1 = Hd[hrow + 2 * uc + 1];
  Vec8<T> xv[seg_vecs_per_thread<MB>()];
  load_rows_block<T, MB>(xv, static_cast<const T*>(a.x), a.K, b0, a.B, k0, len, tid);
  Vec8<T> w[kSegChunks][kRowsPerWave];
  const T* wr[kRowsPerWave] = {W + (size_t)(2 * uc) * a.K, W + (size_t)(2 * uc + 1) * a.K};
  load_rows<T, kRowsPerWave, FULL>(w, wr, k0, len, lane);
  __builtin_amdgcn_sched_barrier(0);
  store_rows_block<T, MB>(xv, b0, a.B, len, xs, kSeg, tid);
  if (flag_set(stop) || u >= units) return;
  float acc[kRowsPerWave][MB];
#pragma unroll
  for (int r = 0; r < kRowsPerWave; ++r)
#pragma unroll
    for (int m = 0; m < MB; ++m) acc[r][m] = 0.f;
  dot_rows<T, MB, kRowsPerWave, FULL>(w, xs, kSeg, 0, len, lane, acc);
  float* wred = red + wave * (kRowsPerWave * MB);
  wave_totals<MB, kRowsPerWave>(acc, lane, wred);
  if (lane >= MB || b0 + lane >= a.B) return;
  const int b = b0 + lane;
  if (a.segments == 1) {
    Hd[(size_t)b * a.N + 2 * u] = Elt<T>::t(Elt<T>::f(h0) + Elt<T>::r(wred[0 * MB + lane]));
    Hd[(size_t)b * a.N + 2 * u + 1] = Elt<T>::t(Elt<T>::f(h1) + Elt<T>::r(wred[1 * MB + lane]));
  } else {
#pragma unroll
    for (int r = 0; r < kRowsPerWave; ++r)
      a.partial[((size_t)seg * a.B + b) * a.N + 2 * u + r] = wred[r * MB + lane];
  }
}

template <typename T, int MB, int WAVES>
__global__ void __launch_bounds__(WAVES * 64) k_resid(ResidArgs a) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  T* xs = reinterpret_cast<T*>(smem_raw);  // [MB][kSeg]
  float* red = reinterpret_cast<float*>(smem_raw + (size_t)MB * kSeg * sizeof(T));
  const int seg = blockIdx.y;
  const int len = min(a.K - seg * kSeg, kSeg);
  if (len == kSeg)
    resid_segment<T, MB, WAVES, true>(a, xs, red, seg, len);
  else
    resid_segment<T, MB, WAVES, false>(a, xs, red, seg, len);
}

// ---------------------------------------------------------------------------
// Down projection with the whole K in one workgroup (bf16, B <= 4):
// h = T(h + T(x W^T)) (batched_decoder_step.py:399-403) with no fp32
// partials in global memory and no reduce launch.  One workgroup of 16 waves
// per CU; workgroup g owns the row pairs [g*ppw, (g+1)*ppw).  For one row
// pair, wave w covers its K range (about K/16 elements, down_whole_spans) of
// both rows in up to three 512-element loads per row; each lane dots its elements against the B
// rows and the lanes of a wave are combined by the halving exchange into LDS.
// A lane only ever needs its own elements of the activations x [B, K], so it
// requests them once and keeps them for every pair (the first two chunks in
// registers, the third in its own LDS slot): no workgroup-wide staging of the
// 148 KB of x and no barrier before the first products.  After the
// last pair, one thread per output adds the 16 wave totals in wave order and
// the residual -- a fixed order, so the results do not depend on timing.
// The next pair's weights are in flight while a pair is computed (two
// register sets), and nothing else is requested inside the loop, so every
// wait there is for the pair being computed; a request past the
// workgroup's range reads one 16-byte line for the whole wave.
// ---------------------------------------------------------------------------
constexpr int kWholeWaves = 16;
constexpr int kWholeLoads = 3;   // loads per row and wave: K <= 16 * 3 * 512

struct DownWholeArgs {
  const int32_t* done;
  const void* x;  // bf16 [B, K]
  const void* w;  // bf16 [N, K]
  void* hidden;   // bf16 [B, N]
  int B, N, K, pairs_per_wg;
  int span[4];    // K elements of each wave of wave group w / 4 (sum of 4 x span = K)
};

// Requests the weights of row pair u (rows 2u, 2u+1) for this wave's K range.
__device__ __forceinline__ void whole_issue(Vec8<bf16_t> (&w)[kWholeLoads][2], const bf16_t* W, int K, int u,
                                            int u_end, int k_lo, int span, int lane) {
  const bool real = u < u_end;
#pragma unroll
  for (int j = 0; j < kWholeLoads; ++j) {
    const int k = min(j * kChunk + lane * 8, span - 8);
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const size_t off = real ? (size_t)(2 * u + r) * K + k_lo + k : 0;
      w[j][r] = Vec8<bf16_t>::load(W + off);
    }
  }
}

// K elements per wave of each group of four waves.  The SIMD arbiter serves
// the oldest waves first, so waves 0-3 finish their range first and 12-15
// last; the younger groups take more of K, and every range is a whole number
// of 128-byte lines (64 elements), so no two waves share a line: with
// K = 18,944, 1,088 / 1,152 / 1,216 / 1,280 against 1,184 each (bench 1,476
// -> 1,482 tok/s).  Equal ranges where K is not a multiple of 256 or the
// ramp does not fit three loads per lane.  The fp32 sums follow the ranges
// (wave totals still added in wave order).
void down_whole_spans(int K, int (&span)[4]) {
  for (int q = 0; q < 4; ++q) span[q] = K / kWholeWaves;
  if (K % 256 != 0) return;
  const int n = K / 256, m = n / 4;  // 64-element units per group of four ranges
  const int u[4] = {m - 1, m, m + 1, n - 3 * m};
  for (int q = 0; q < 4; ++q)
    if (u[q] < 1 || u[q] * 64 > kWholeLoads * kChunk || u[q] < u[q > 0 ? q - 1 : 0]) return;
  for (int q = 0; q < 4; ++q) span[q] = u[q] * 64;
}

__global__ void __launch_bounds__(kWholeWaves * 64, 1) k_down_whole(DownWholeArgs a) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  constexpr int MB = 4;
  float* red = reinterpret_cast<float*>(smem_raw);  // [ppw][16][8] wave totals
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_index(tid);
  const int K = a.K, g4 = wave >> 2, span = a.span[g4];
  int k_lo = (wave & 3) * span;
#pragma unroll
  for (int q = 0; q < 3; ++q) k_lo += q < g4 ? 4 * a.span[q] : 0;
  const int units = a.N / 2;
  const int u_begin = blockIdx.x * a.pairs_per_wg;
  const int u_end = min(u_begin + a.pairs_per_wg, units);
  if (u_begin >= u_end) return;  // the whole workgroup
  const bf16_t* W = static_cast<const bf16_t*>(a.w);
  const bf16_t* X = static_cast<const bf16_t*>(a.x);
  bf16_t* Hd = static_cast<bf16_t*>(a.hidden);

  // Issue order: the flag, the residual values of this workgroup's outputs
  // (thread t < 8 x pairs: pair t/8, row (t/4)&1 of the pair, batch row t&3),
  // this wave's slice of the activations, then the first two pairs' weights.
  // A wave only ever reads its own K range of the MB rows (elements k_lo +
  // 512 j + 8 lane), so it keeps that slice in registers for every pair: no
  // LDS staging and no workgroup barrier before the first products.  Loads
  // past the range or the batch are clamped to valid addresses; their
  // products are skipped or never stored.
  const int32_t stop = a.done != nullptr ? request_flag(a.done) : 0;
  const int nout = (u_end - u_begin) * 8;
  const int ot = min(tid, nout - 1);
  const int o_u = u_begin + ot / 8, o_r = (ot >> 2) & 1, o_m = ot & 3;
  const bf16_t h = Hd[(size_t)min(o_m, a.B - 1) * a.N + 2 * o_u + o_r];
  // The last chunk's values wait in this thread's own LDS slot (registers are
  // full at 16 waves per CU); only the thread that wrote a slot reads it.
  constexpr int kReg = kWholeLoads - 1;
  Vec8<bf16_t>* xl = reinterpret_cast<Vec8<bf16_t>*>(smem_raw + (size_t)a.pairs_per_wg * kWholeWaves * 8 * sizeof(float)) +
                     (size_t)tid * MB;
  Vec8<bf16_t> xr[kWholeLoads][MB];
#pragma unroll
  for (int j = 0; j < kWholeLoads; ++j) {
    const int k = min(j * kChunk + lane * 8, span - 8);
#pragma unroll
    for (int m = 0; m < MB; ++m) xr[j][m] = Vec8<bf16_t>::load_cached(X + (size_t)min(m, a.B - 1) * K + k_lo + k);
  }
  Vec8<bf16_t> wa[kWholeLoads][2], wb[kWholeLoads][2];
  whole_issue(wa, W, K, u_begin, u_end, k_lo, span, lane);
  whole_issue(wb, W, K, u_begin + 1, u_end, k_lo, span, lane);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int m = 0; m < MB; ++m) xl[m] = xr[kReg][m];
  if (flag_set(stop)) return;  // uniform over the workgroup

  // One pair: products over this wave's range, wave totals to LDS.
  auto pair = [&](Vec8<bf16_t>(&w)[kWholeLoads][2], int u) {
    __builtin_amdgcn_sched_barrier(0);
    float acc[2][MB];
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int m = 0; m < MB; ++m) acc[r][m] = 0.f;
#pragma unroll
    for (int j = 0; j < kWholeLoads; ++j) {
      const int k = j * kChunk + lane * 8;
      if (k < span) {
#pragma unroll
        for (int m = 0; m < MB; ++m) {
          const Vec8<bf16_t> x = j < kReg ? xr[j][m] : xl[m];
#pragma unroll
          for (int r = 0; r < 2; ++r) acc[r][m] = dot8(w[j][r], x, acc[r][m]);
        }
      }
    }
    const int p = min(u, u_end - 1) - u_begin;  // a pair past the range overwrites the last one's totals
    float totals[2][MB];
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int m = 0; m < MB; ++m) totals[r][m] = u < u_end ? acc[r][m] : 0.f;
    if (u < u_end) wave_totals<MB, 2>(totals, lane, red + (p * kWholeWaves + wave) * 8);
  };
  for (int u = u_begin; u < u_end; u += 2) {
    pair(wa, u);
    whole_issue(wa, W, K, u + 2, u_end, k_lo, span, lane);
    pair(wb, u + 1);
    whole_issue(wb, W, K, u + 3, u_end, k_lo, span, lane);
  }
  lds_barrier();
  if (tid < nout && o_m < a.B) {
    const float* t = red + (ot / 8) * kWholeWaves * 8 + o_r * MB + o_m;
    float s = 0.f;
#pragma unroll
    for (int q = 0; q < kWholeWaves; ++q) s += t[q * 8];
    Hd[(size_t)o_m * a.N + 2 * o_u + o_r] = f_to_bf16(bf16_to_f(h) + round_bf16(s));
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

}  // namespace

// ---------------------------------------------------------------------------
// Launcher
// ---------------------------------------------------------------------------
size_t normed_lds_bytes(int mb, int hidden, int dtype_bytes, int waves) {
  return (size_t)mb * hidden * dtype_bytes + (3 * (size_t)waves * kRowsPerWave + 4) * mb * sizeof(float);
}
size_t down_whole_lds_bytes(int K, int pairs_per_wg) {
  (void)K;  // wave totals, then each thread's slot for its last activation chunk
  return (size_t)pairs_per_wg * kWholeWaves * 8 * sizeof(float) + (size_t)kWholeWaves * 64 * 4 * sizeof(Vec8<bf16_t>);
}
size_t resid_lds_bytes(int mb, int dtype_bytes, int waves) {
  return (size_t)mb * kSeg * dtype_bytes + (size_t)waves * mb * kRowsPerWave * sizeof(float);
}
int k_segment_elems() { return kSeg; }
int row_kernel_max_hidden() { return 8 * 256 * kNormChunks; }

// The step is a fixed list of launches: embed, then per layer [qkv,
// attention, o-proj, o-reduce, gate/up, down, down-reduce], then the LM head.
// The reduce entries launch nothing unless their projection runs split-K.
// [begin, end) selects a contiguous range of the list.
constexpr int kOpsPerLayer = 7;
constexpr int kGateUpOp = 4;

// The guard-free instantiation serves hidden sizes of exactly one K-segment.
template <typename T, int MB, int WAVES, int KIND>
static void launch_proj(const ProjArgs& a, dim3 grid, size_t smem, hipStream_t stream) {
  if (a.H == kSeg)
    k_proj<T, MB, WAVES, KIND, true><<<grid, WAVES * 64, smem, stream>>>(a);
  else
    k_proj<T, MB, WAVES, KIND, false><<<grid, WAVES * 64, smem, stream>>>(a);
}

// Slot-weighted ranges when the plan has them and the grid is exactly four
// workgroups per CU.
static void set_slots(ProjArgs& a, const LaunchPlan& p, int grid) {
  a.slot_cus = 0;
  if (p.slot_cus > 0 && grid == 4 * p.slot_cus && p.row_tiles == 1) {
    a.slot_cus = p.slot_cus;
    a.slot_shift = (p.slot_cus & (p.slot_cus - 1)) == 0 ? __builtin_ctz(static_cast<unsigned>(p.slot_cus)) : -1;
    long long tot = 0, pre = 0;
    for (int s = 0; s < 4; ++s) tot += p.slot_w[s];
    for (int s = 0; s < 4; ++s) {
      a.slot_base[s] = static_cast<int>((long long)a.units * pre / tot);
      pre += p.slot_w[s];
    }
    a.slot_base[4] = a.units;
  }
}

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
  if (want()) {
    EmbedArgs e{};
    e.done = st.done;
    e.token = st.token;
    e.embedding = env.weights + env.embedding_off;
    e.hidden = sc.hidden;
    e.pos = st.pos;
    e.inv_freq = sc.inv_freq;
    e.rope = sc.rope;
    e.B = B;
    e.H = d.hidden;
    e.V = d.vocab;
    e.half = d.head_dim / 2;
    k_embed<T><<<B, 256, 0, stream>>>(e);
  }
  const size_t proj_smem = normed_lds_bytes(MB, d.hidden, sizeof(T), WAVES);
  const size_t resid_smem = resid_lds_bytes(MB, sizeof(T), WAVES);
  const int reduce_blocks = (B * d.hidden + 255) / 256;
  for (int l = 0; l < d.layers; ++l) {
    const LayerOffsets& lo = env.layer_off[l];
    T* kc = static_cast<T*>(st.key_cache) + l * cache_layer_elems;
    T* vc = static_cast<T*>(st.value_cache) + l * cache_layer_elems;
    ProjArgs q{};
    q.done = st.done;
    q.hidden = sc.hidden;
    q.norm_w = env.weights + lo.input_norm;
    q.w0 = env.weights + lo.qkv_w;
    q.w1 = env.weights + lo.qkv_b;
    q.out = sc.q;
    q.rope = sc.rope;
    q.slot = st.slot;
    q.active = st.active;
    q.key_cache = kc;
    q.value_cache = vc;
    q.slots = d.slots();
    q.B = B;
    q.H = d.hidden;
    q.units = d.qkv_rows() / 2;
    q.heads = d.heads;
    q.kv_heads = d.kv_heads;
    q.head_dim = d.head_dim;
    q.eps = d.rms_eps;
    if (want()) {
      if (p.mfma) {
        const hipError_t err = launch_mfma_op(MfmaOp::kQkv, env, st, l, stream);
        if (err != hipSuccess) return err;
      } else if (sizeof(T) == 2 && MB == 4 && p.qkv_ksplit > 0) {
        k_qkv_ksplit<kQkvKsPairs><<<p.qkv_ksplit, kQkvKsWaves * 64, 0, stream>>>(q);
      } else {
        launch_proj<T, MB, WAVES, kQkv>(q, dim3(p.qkv_grid, p.row_tiles), proj_smem, stream);
      }
    }

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
    at.bs_shift = (d.block_size & (d.block_size - 1)) == 0 ? __builtin_ctz(static_cast<unsigned>(d.block_size)) : -1;
    at.grouped = p.grouped_attn;
    at.packed_out = p.mfma;  // the matrix-core o-projection reads its input packed
    at.split_tiles = p.grouped_attn != 1 ? p.attn_split : 0;
    at.sp_scores = sc.sp_scores;
    at.sp_stats = sc.sp_stats;
    at.sp_part = sc.sp_part;
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
    if (want()) {
      if (p.mfma) {
        const hipError_t err = launch_mfma_op(MfmaOp::kO, env, st, l, stream);
        if (err != hipSuccess) return err;
      } else {
        bool launched = false;
        if constexpr (sizeof(T) == 2 && MB == 4) {
          if (p.o_waves == 7) {
            k_resid<T, MB, 7><<<dim3(p.o_grid, p.o_segments, p.row_tiles), 7 * 64, resid_lds_bytes(MB, sizeof(T), 7),
                                stream>>>(o);
            launched = true;
          }
        }
        if (!launched)
          k_resid<T, MB, WAVES><<<dim3(p.o_grid, p.o_segments, p.row_tiles), WAVES * 64, resid_smem, stream>>>(o);
      }
    }
    if (want() && p.o_segments > 1 && !p.mfma)
      k_resid_reduce<T><<<reduce_blocks, 256, 0, stream>>>(st.done, sc.partial, sc.hidden, B, d.hidden,
                                                            p.o_segments);

    ProjArgs gu{};
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
    set_slots(gu, p, p.gu_grid);
    if (want()) {
      if (p.mfma) {
        const hipError_t err = launch_mfma_op(MfmaOp::kGateUp, env, st, l, stream);
        if (err != hipSuccess) return err;
      } else {
        launch_proj<T, MB, WAVES, kGateUp>(gu, dim3(p.gu_grid, p.row_tiles), proj_smem, stream);
      }
    }
    if (p.mfma) {
      if (want()) {
        const hipError_t err = launch_mfma_op(MfmaOp::kDown, env, st, l, stream);
        if (err != hipSuccess) return err;
      }
      (void)want();  // the reduce entry: nothing to reduce
      continue;
    }

    if constexpr (sizeof(T) == 2 && MB == 4) {
      if (p.down_whole_grid > 0) {
        DownWholeArgs dw{};
        dw.done = st.done;
        dw.x = sc.mlp;
        dw.w = env.weights + lo.down_w;
        dw.hidden = sc.hidden;
        dw.B = B;
        dw.N = d.hidden;
        dw.K = d.intermediate;
        dw.pairs_per_wg = (d.hidden / 2 + p.down_whole_grid - 1) / p.down_whole_grid;
        down_whole_spans(d.intermediate, dw.span);
        if (want())
          k_down_whole<<<p.down_whole_grid, kWholeWaves * 64, down_whole_lds_bytes(d.intermediate, dw.pairs_per_wg),
                         stream>>>(dw);
        (void)want();  // the reduce entry: nothing to reduce
        continue;
      }
    }
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
  ProjArgs lm{};
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
  set_slots(lm, p, p.lm_grid);
  if (want()) {
    if (p.mfma) return launch_mfma_op(MfmaOp::kLmHead, env, st, 0, stream);
    launch_proj<T, MB, WAVES, kLmHead>(lm, dim3(p.lm_grid, p.row_tiles), proj_smem, stream);
  }
  return hipGetLastError();
}

// Workgroups of each projection: as many as are resident at once (from the
// compiled kernels' occupancy), trimmed so every workgroup runs the same
// number of row groups.
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
  const bool full = d.hidden == kSeg;
  p.qkv_grid = fit(full ? k_proj<T, MB, WAVES, kQkv, true> : k_proj<T, MB, WAVES, kQkv, false>,
                   (d.qkv_rows() / 2 + WAVES - 1) / WAVES);
  p.qkv_waves = WAVES;
  // qkv with K split over 7 waves (k_qkv_ksplit): the hidden size is 7 x 512
  // and the pairs fill whole workgroups of kQkvKsPairs; the grid, or 0
  p.qkv_ksplit = 0;
  if (sizeof(T) == 2 && MB == 4 && p.row_tiles == 1 && d.hidden == kQkvKsWaves * kChunk &&
      (d.qkv_rows() / 2) % kQkvKsPairs == 0)
    p.qkv_ksplit = d.qkv_rows() / 2 / kQkvKsPairs;
  p.slot_cus = 0;
  p.gu_grid = fit(full ? k_proj<T, MB, WAVES, kGateUp, true> : k_proj<T, MB, WAVES, kGateUp, false>,
                  (d.intermediate + WAVES - 1) / WAVES);
  p.lm_grid = fit(full ? k_proj<T, MB, WAVES, kLmHead, true> : k_proj<T, MB, WAVES, kLmHead, false>,
                  (d.vocab / 2 + WAVES - 1) / WAVES);
  // Slot-weighted ranges for gate/up and the LM head at four workgroups per
  // CU (bf16, one row tile): 1 : 1 : 0.9 : 0.8 measured best on MI355X.
  int per_cu = 0;
  if (sizeof(T) == 2 && p.row_tiles == 1 &&
      hipOccupancyMaxActiveBlocksPerMultiprocessor(
          &per_cu, full ? k_proj<T, MB, WAVES, kGateUp, true> : k_proj<T, MB, WAVES, kGateUp, false>, WAVES * 64,
          smem) == hipSuccess &&
      per_cu == 4 && d.intermediate >= 16 * cus && d.vocab / 2 >= 16 * cus) {
    p.slot_cus = cus;
    const int w[4] = {1000, 1000, 900, 800};
    for (int s = 0; s < 4; ++s) p.slot_w[s] = w[s];
    p.gu_grid = 4 * cus;
    p.lm_grid = 4 * cus;
  }
  p.lm_wg = p.lm_grid;
  // The whole-K down projection: bf16, one row tile of at most four rows,
  // K a multiple of 16 x 8 within three loads per wave, activations in LDS.
  p.down_whole_grid = 0;
  const int whole_grid = std::min(cus, d.hidden / 2);
  const size_t whole_lds = down_whole_lds_bytes(d.intermediate, (d.hidden / 2 + whole_grid - 1) / whole_grid);
  if (sizeof(T) == 2 && MB == 4 && p.row_tiles == 1 && d.intermediate % (kWholeWaves * 8) == 0 &&
      d.intermediate / kWholeWaves <= kWholeLoads * kChunk && d.hidden % 2 == 0 && whole_lds <= 160 * 1024 &&
      hipFuncSetAttribute(reinterpret_cast<const void*>(k_down_whole), hipFuncAttributeMaxDynamicSharedMemorySize,
                          static_cast<int>(whole_lds)) == hipSuccess) {
    p.down_whole_grid = whole_grid;
  }
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

// Whether per-layer op `which` launches a kernel under the engine's plan: the
// o- and down-reduce entries launch only when their projection runs split-K
// on the row-tiled path (the whole-K down and the matrix-core path reduce
// inside the projection).
bool layer_op_launches(const KernelEnv& env, int which) {
  const LaunchPlan& p = env.plan;
  constexpr int kOReduceOp = 3, kDownReduceOp = 6;
  if (which == kOReduceOp) return !p.mfma && p.o_segments > 1;
  if (which == kDownReduceOp) {
    const bool down_whole = env.dims.dtype_bytes == 2 && p.mb == 4 && p.down_whole_grid > 0;
    return !p.mfma && !down_whole && p.down_segments > 1;
  }
  return which >= 0 && which < kOpsPerLayer;
}
int timed_op_index(const KernelEnv& env, int layer) {
  (void)env;
  return 1 + kOpsPerLayer * layer + kGateUpOp;
}

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
