// Building blocks of the weight-streaming skinny GEMMs of the decoder step
// (gfx950; re_step.hip).
//
// A wave owns two weight rows over one K-segment of up to 7 x 512 elements
// and issues all 14 of its 16-byte non-temporal loads before touching them,
// so one HBM round trip covers a whole row pair.  Activations sit in LDS; bf16
// pairs go through v_dot2 into fp32 accumulators; the 64 lanes are combined by
// a halving exchange.
#pragma once

#include "re_device.h"

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
// of lane l covers elements k0 + c*512 + l*8 .. +8.  Chunks past len are left
// unset (dot_rows skips them), so no value merge forces an early wait.
// FULL: the segment holds all kSegChunks chunks (len == kSeg), no guards.
template <typename T, int RPW, bool FULL = false>
__device__ __forceinline__ void load_rows(Vec8<T> (&w)[kSegChunks][RPW], const T* const (&wr)[RPW], int k0,
                                          int len, int lane) {
#pragma unroll
  for (int c = 0; c < kSegChunks; ++c) {
    const int k = c * kChunk + lane * 8;
#pragma unroll
    for (int r = 0; r < RPW; ++r)
      if (FULL || k < len) w[c][r] = Vec8<T>::load(wr[r] + k0 + k);
  }
}

// acc[r][m] += sum over the segment of W_r[k] * xs[m][k0 + k] (xs: LDS, row
// stride ldx).
template <typename T, int MB, int RPW, bool FULL = false>
__device__ __forceinline__ void dot_rows(const Vec8<T> (&w)[kSegChunks][RPW], const T* xs, int ldx, int k0, int len,
                                         int lane, float (&acc)[RPW][MB]) {
#pragma unroll
  for (int c = 0; c < kSegChunks; ++c) {
    const int k = c * kChunk + lane * 8;
    if (FULL || k < len) {
#pragma unroll
      for (int m = 0; m < MB; ++m) {
        const Vec8<T> x = Vec8<T>::load_cached(xs + m * ldx + k0 + k);
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

// Vec8 slots a 256-thread workgroup needs to hold MB rows of one K-segment.
template <int MB>
constexpr int seg_vecs_per_thread() {
  return (MB * kSeg / 8 + 255) / 256;
}

// Load rows b0..b0+MB-1, columns [k0, k0+len), of X [B, ldg] into registers:
// slot i of thread t holds Vec8 number t + 256*i of the row-major [MB, len]
// block.  Within the first 256 threads the loads are unconditional (addresses
// clamped into the block), so every wait counts exactly; store_rows_block
// zeroes what lies outside.  Threads from 256 up (wider workgroups) load
// nothing: each activation line they requested would take one of the CU's
// outstanding-miss slots that the weight stream needs.
template <typename T, int MB>
__device__ __forceinline__ void load_rows_block(Vec8<T> (&v)[seg_vecs_per_thread<MB>()], const T* __restrict__ X,
                                                int ldg, int b0, int B, int k0, int len, int tid) {
  const int per_row = max(len / 8, 1);
  if (tid >= 256) return;  // wave-uniform
#pragma unroll
  for (int i = 0; i < seg_vecs_per_thread<MB>(); ++i) {
    const int idx = min(tid + 256 * i, MB * per_row - 1);
    const int m = idx / per_row, k = (idx - m * per_row) * 8;
    v[i] = Vec8<T>::load_cached(X + (size_t)min(b0 + m, B - 1) * ldg + k0 + k);
  }
}

// Store the block loaded by load_rows_block into LDS xs [MB, ldx] (rows >= B
// as zero), then a workgroup barrier.  Threads from 256 up (workgroups of
// more than four waves) store nothing; they only join the barrier.
template <typename T, int MB>
__device__ __forceinline__ void store_rows_block(const Vec8<T> (&v)[seg_vecs_per_thread<MB>()], int b0, int B, int len,
                                                 T* xs, int ldx, int tid) {
  constexpr int NV = seg_vecs_per_thread<MB>();
  const int per_row = len / 8;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int idx = tid + 256 * i;
    if (tid < 256 && idx < MB * per_row) {
      const int m = idx / per_row, k = (idx - m * per_row) * 8;
      *reinterpret_cast<Vec8<T>*>(xs + m * ldx + k) = b0 + m < B ? v[i] : Vec8<T>{};
    }
  }
  lds_barrier();  // weight loads issued before the staging stay in flight
}

// ---------------------------------------------------------------------------
// Norm prologue: RMSNorm of rows b0..b0+MB-1 of the residual stream into LDS
// (batched_decoder_step.py:224-229): fp32 mean of squares, rsqrt(var + eps),
// cast to T, then a T x T product with the weight.  Thread t < 256 owns
// hidden chunks t and t + 256 (8 elements each) of every row, so it needs the
// norm weight of two chunks only; threads from 256 up (workgroups of more
// than four waves) only take part in the barriers.  Requires
// blockDim.x >= 256, H <= 4096.
// ---------------------------------------------------------------------------
constexpr int kNormChunks = 2;

template <typename T, int MB>
struct NormIn {
  Vec8<T> h[MB][kNormChunks];
  Vec8<T> w[kNormChunks];
};

// The RMSNorm output of eight elements: T(T(h * rs) * w) for each
// (batched_decoder_step.py:227-229).  bf16: the two roundings of an element
// pair go through one packed conversion each, and the result keeps the
// hardware's NaN (the rows stay in LDS as products' inputs, where a NaN's
// payload does not matter): every non-NaN value is the one Elt<T>::r and
// Vec8::from_floats give.
template <typename T>
__device__ __forceinline__ Vec8<T> norm_apply(const Vec8<T>& h, const Vec8<T>& w, float rs) {
  float out[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) out[e] = Elt<T>::r(Elt<T>::r(h.get(e) * rs) * w.get(e));
  return Vec8<T>::from_floats(out);
}
template <>
__device__ __forceinline__ Vec8<bf16_t> norm_apply<bf16_t>(const Vec8<bf16_t>& h, const Vec8<bf16_t>& w, float rs) {
  Vec8<bf16_t> r;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t hp = h.v[i], wp = w.v[i];
    const uint32_t y = f2_to_bf16x2_raw(__uint_as_float(hp << 16) * rs, __uint_as_float(hp & 0xffff0000u) * rs);
    r.v[i] = f2_to_bf16x2_raw(__uint_as_float(y << 16) * __uint_as_float(wp << 16),
                              __uint_as_float(y & 0xffff0000u) * __uint_as_float(wp & 0xffff0000u));
  }
  return r;
}

template <typename T, int MB>
__device__ __forceinline__ void norm_load(NormIn<T, MB>& in, const T* __restrict__ hidden, const T* __restrict__ norm_w,
                                          int b0, int B, int H, int tid) {
  // unconditional (clamped) loads in the owning threads; norm_to_lds ignores
  // what lies outside.  Threads from 256 up own nothing and load nothing (a
  // wave-uniform branch): their requests would only hold miss slots the
  // weight stream needs.
  const int per_row = H / 8;
  if (tid >= 256) return;
#pragma unroll
  for (int j = 0; j < kNormChunks; ++j) {
    const int c = min(tid + 256 * j, per_row - 1);
    in.w[j] = Vec8<T>::load_cached(norm_w + c * 8);
#pragma unroll
    for (int m = 0; m < MB; ++m)
      in.h[m][j] = Vec8<T>::load_cached(hidden + (size_t)min(b0 + m, B - 1) * H + c * 8);
  }
}

// The raw rows go to LDS as they arrive (the per-row sums of squares formed
// on the way), so the hidden values are dead before the block reduction; after
// it each thread normalizes its own chunks in place.  red: LDS scratch of at
// least 4 * MB floats.
template <typename T, int MB>
__device__ __forceinline__ void norm_to_lds(const NormIn<T, MB>& in, int b0, int B, int H, float eps, T* xs,
                                            float* red, int tid) {
  const int lane = tid & 63, wave = wave_index(tid);
  const int per_row = H / 8;
  const bool owner = tid < 256;  // wave-uniform
  float ss[MB];
#pragma unroll
  for (int m = 0; m < MB; ++m) {
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < kNormChunks; ++j) {
      const int c = tid + 256 * j;
      const bool ok = owner && c < per_row && b0 + m < B;
      const Vec8<T> h = ok ? in.h[m][j] : Vec8<T>{};
      if (owner && c < per_row) *reinterpret_cast<Vec8<T>*>(xs + m * H + c * 8) = h;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = h.get(e);
        s = fmaf(x, x, s);
      }
    }
    ss[m] = s;
  }
  wave_reduce_transpose<MB>(ss, lane);
  if (wave < 4 && (lane & (64 / MB - 1)) == 0) red[wave * MB + lane / (64 / MB)] = ss[0];
  lds_barrier();
  float rs[MB];
#pragma unroll
  for (int m = 0; m < MB; ++m) {
    float total = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) total += red[w * MB + m];
    rs[m] = rsqrtf(total / static_cast<float>(H) + eps);
  }
#pragma unroll
  for (int j = 0; j < kNormChunks; ++j) {
    const int c = tid + 256 * j;
    if (owner && c < per_row) {
#pragma unroll
      for (int m = 0; m < MB; ++m) {
        Vec8<T>* p = reinterpret_cast<Vec8<T>*>(xs + m * H + c * 8);
        *p = norm_apply<T>(*p, in.w[j], rs[m]);
      }
    }
  }
  lds_barrier();
}


}  // namespace
}  // namespace re
