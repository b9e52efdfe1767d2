// Device-side helpers shared by the resident-epoch kernels (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef uint16_t bf16_t;
typedef __bf16 re_bf16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t re_u32x4 __attribute__((ext_vector_type(4)));
typedef float re_f32x4 __attribute__((ext_vector_type(4)));

// bf16 <-> fp32.  The fp32 -> bf16 rounding is round-to-nearest-even with
// NaN mapped to 0x7FC0, the conversion torch applies on ``.to(bfloat16)``.
// gfx950's v_cvt_pk_bf16_f32 rounds to nearest even; it agrees with the
// bit-level RNE on every non-NaN fp32 input (all 2^32 patterns checked on
// the device), so only NaN needs the canonical value.
__device__ __forceinline__ float bf16_to_f(bf16_t v) {
  return __uint_as_float(static_cast<uint32_t>(v) << 16);
}
__device__ __forceinline__ bf16_t f_to_bf16(float f) {
  const bf16_t h = __builtin_bit_cast(bf16_t, static_cast<__bf16>(f));
  return f != f ? static_cast<bf16_t>(0x7fc0) : h;
}
// Two values rounded and packed (lo, hi) with one conversion instruction.
__device__ __forceinline__ uint32_t f2_to_bf16x2(float lo, float hi) {
  typedef float f2_t __attribute__((ext_vector_type(2)));
  const f2_t v = {lo, hi};
  uint32_t p = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, re_bf16x2));
  if (lo != lo) p = (p & 0xffff0000u) | 0x7fc0u;
  if (hi != hi) p = (p & 0x0000ffffu) | 0x7fc00000u;
  return p;
}
// Two values rounded to bf16 (RNE) and packed (lo, hi), NaN left as the
// hardware produces it: for values that stay inside a computation.
__device__ __forceinline__ uint32_t f2_to_bf16x2_raw(float lo, float hi) {
  typedef float f2_t __attribute__((ext_vector_type(2)));
  const f2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, re_bf16x2));
}
// Rounding to bf16 inside a computation: a NaN stays a NaN (its payload does
// not matter until a value is stored, and stores canonicalize), so the
// hardware conversion is used as is.
__device__ __forceinline__ float round_bf16(float f) {
  return bf16_to_f(__builtin_bit_cast(bf16_t, static_cast<__bf16>(f)));
}

// x / sqrt(128) for a bf16-valued x whose quotient is rounded to bf16 next
// (the scaled attention score): the product with the rounded reciprocal.
// For every bf16 x the bf16 rounding of the product equals the bf16 rounding
// of the correctly rounded fp32 quotient x / c, c = fp32(sqrt(128)), as the
// reference divides: a quotient of an 8-bit mantissa by c never comes within
// about 1e-5 (relative) of a bf16 rounding boundary, far beyond the product's
// two roundings (the fp32 results differ for 26,650 dividends, the bf16 ones
// for none; tests/test_div_sqrt128.py checks all 65,536 inputs).  Infinities,
// NaN and zeros pass through as in the division.
__device__ __forceinline__ float div_sqrt128_bf16(float x) {
  constexpr float rc = __builtin_bit_cast(float, 0x3db504f3u);  // 1 / fp32(sqrt(128)) rounded to fp32
  return x * rc;
}

// Element traits: the compute dtype T of a model is bf16 or fp32.
template <typename T>
struct Elt;

template <>
struct Elt<bf16_t> {
  static constexpr int kBytes = 2;
  __device__ __forceinline__ static float f(bf16_t v) { return bf16_to_f(v); }
  __device__ __forceinline__ static bf16_t t(float v) { return f_to_bf16(v); }
  __device__ __forceinline__ static float r(float v) { return round_bf16(v); }
};

template <>
struct Elt<float> {
  static constexpr int kBytes = 4;
  __device__ __forceinline__ static float f(float v) { return v; }
  __device__ __forceinline__ static float t(float v) { return v; }
  __device__ __forceinline__ static float r(float v) { return v; }
};

// Eight consecutive elements (16 bytes of bf16, 32 bytes of fp32).
template <typename T>
struct Vec8;

template <>
struct Vec8<bf16_t> {
  re_u32x4 v;
  __device__ __forceinline__ static Vec8 load(const bf16_t* p) {
    Vec8 r;
    r.v = __builtin_nontemporal_load(reinterpret_cast<const re_u32x4*>(p));
    return r;
  }
  __device__ __forceinline__ static Vec8 load_cached(const bf16_t* p) {
    Vec8 r;
    r.v = *reinterpret_cast<const re_u32x4*>(p);
    return r;
  }
  __device__ __forceinline__ float get(int i) const {
    const uint32_t w = v[i >> 1];
    return __uint_as_float((i & 1) ? (w & 0xffff0000u) : (w << 16));
  }
  // Round eight floats to bf16 (RNE) and pack them.
  __device__ __forceinline__ static Vec8 from_floats(const float (&f)[8]) {
    Vec8 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) r.v[i] = f2_to_bf16x2(f[2 * i], f[2 * i + 1]);
    return r;
  }
};

template <>
struct Vec8<float> {
  re_f32x4 a, b;
  __device__ __forceinline__ static Vec8 load(const float* p) {
    Vec8 r;
    r.a = __builtin_nontemporal_load(reinterpret_cast<const re_f32x4*>(p));
    r.b = __builtin_nontemporal_load(reinterpret_cast<const re_f32x4*>(p) + 1);
    return r;
  }
  __device__ __forceinline__ static Vec8 load_cached(const float* p) {
    Vec8 r;
    r.a = reinterpret_cast<const re_f32x4*>(p)[0];
    r.b = reinterpret_cast<const re_f32x4*>(p)[1];
    return r;
  }
  __device__ __forceinline__ float get(int i) const {
    return i < 4 ? a[i] : b[i - 4];
  }
  __device__ __forceinline__ static Vec8 from_floats(const float (&f)[8]) {
    Vec8 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      r.a[i] = f[i];
      r.b[i] = f[i + 4];
    }
    return r;
  }
};

// acc + w.lo*x.lo + w.hi*x.hi for one packed pair of bf16 (fp32 accumulate).
// The operands arrive as plain 32-bit scalars: clang's __builtin_bit_cast of
// an ext-vector element (v.y, v.z, ...) reads element 0 whatever the index,
// so elements are copied out before the cast.
__device__ __forceinline__ float dot2_bf16(uint32_t w, uint32_t x, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(re_bf16x2, w), __builtin_bit_cast(re_bf16x2, x), acc,
                                         false);
}

// acc + sum_i w[i] * x[i] over eight elements, fp32 accumulation.
__device__ __forceinline__ float dot8(const Vec8<bf16_t>& w, const Vec8<bf16_t>& x, float acc) {
  const uint32_t w0 = w.v[0], w1 = w.v[1], w2 = w.v[2], w3 = w.v[3];
  const uint32_t x0 = x.v[0], x1 = x.v[1], x2 = x.v[2], x3 = x.v[3];
  acc = dot2_bf16(w0, x0, acc);
  acc = dot2_bf16(w1, x1, acc);
  acc = dot2_bf16(w2, x2, acc);
  acc = dot2_bf16(w3, x3, acc);
  return acc;
}
__device__ __forceinline__ float dot8(const Vec8<float>& w, const Vec8<float>& x, float acc) {
  acc = fmaf(w.a.x, x.a.x, acc);
  acc = fmaf(w.a.y, x.a.y, acc);
  acc = fmaf(w.a.z, x.a.z, acc);
  acc = fmaf(w.a.w, x.a.w, acc);
  acc = fmaf(w.b.x, x.b.x, acc);
  acc = fmaf(w.b.y, x.b.y, acc);
  acc = fmaf(w.b.z, x.b.z, acc);
  acc = fmaf(w.b.w, x.b.w, acc);
  return acc;
}

// Lane exchanges without the LDS crossbar.  Within a 16-lane row, the value
// of lane l ^ M (M = 1, 2, 4, 8) comes from DPP moves: quad permutations for
// 1 and 2, a rotation by 8 for 8, and for 4 a rotation by 4 or by 12 picked
// by bit 2 of the lane.  Across rows, gfx950's permlane swaps exchange whole
// halves of two registers: permlane32_swap(x, y) trades x's lanes 32-63 with
// y's lanes 0-31, permlane16_swap(x, y) x's odd 16-lane rows with y's even
// ones.  (All checked lane for lane against ds_bpermute on the device.)
template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
constexpr int kDppQuadXor1 = 0xB1;     // quad_perm [1, 0, 3, 2]
constexpr int kDppQuadXor2 = 0x4E;     // quad_perm [2, 3, 0, 1]
constexpr int kDppRowRor4 = 0x124;
constexpr int kDppRowRor8 = 0x128;
constexpr int kDppRowRor12 = 0x12C;
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;

template <int M>
__device__ __forceinline__ float lane_xor_in_row(float v, int lane) {
  static_assert(M == 1 || M == 2 || M == 4 || M == 8, "in-row masks only");
  if constexpr (M == 1) return dpp_move<kDppQuadXor1>(v);
  else if constexpr (M == 2) return dpp_move<kDppQuadXor2>(v);
  else if constexpr (M == 8) return dpp_move<kDppRowRor8>(v);
  else {
    const float a = dpp_move<kDppRowRor4>(v), b = dpp_move<kDppRowRor12>(v);
    return (lane & 4) ? a : b;
  }
}

// x, y -> x + y after the swap of permlane32_swap (M = 32) or permlane16_swap
// (M = 16): lanes whose bit log2(M) is clear get x[l] + x[l + M], the others
// y[l - M] + y[l] -- one level of the transposing reduction below for a pair
// of values, and (with x = y) the step v[l] + v[l ^ M] of a plain sum.
template <int M>
__device__ __forceinline__ float swap_add(float x, float y) {
  static_assert(M == 16 || M == 32, "cross-row masks only");
  const auto r = M == 32 ? __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(y), false, false)
                         : __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(y), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// v + (v of lane l ^ M) and max(v, v of lane l ^ M), M a power of two <= 32.
template <int M>
__device__ __forceinline__ float xor_add(float v, int lane) {
  if constexpr (M >= 16) return swap_add<M>(v, v);
  else return v + lane_xor_in_row<M>(v, lane);
}
template <int M>
__device__ __forceinline__ float xor_max(float v, int lane) {
  if constexpr (M >= 16) {
    const auto r = M == 32 ? __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false)
                           : __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  } else {
    return fmaxf(v, lane_xor_in_row<M>(v, lane));
  }
}

// One level of the halving exchange at mask M over the first NV values: a
// lane whose bit log2(M) is set keeps the upper half and sends the lower one,
// and adds what its partner l ^ M sends (keep + received).  Once one value is
// left (NV == 1) the step is the plain sum v[0] + v[0] of lane l ^ M.
template <int M, int NV, int N>
__device__ __forceinline__ void reduce_step(float (&v)[N], int lane) {
  constexpr int h = NV / 2;
  if constexpr (NV == 1) {
    v[0] = xor_add<M>(v[0], lane);
  } else if constexpr (M >= 16) {
#pragma unroll
    for (int i = 0; i < h; ++i) v[i] = swap_add<M>(v[i], v[i + h]);
  } else {
    const bool upper = (lane & M) != 0;
#pragma unroll
    for (int i = 0; i < h; ++i) {
      // Opaque copies keep the selects on registers: a select between two
      // elements of v is otherwise folded into a read of v at a runtime
      // index, which lowers to a compare-and-select chain over all of v.
      float lo = v[i], hi = v[i + h];
      asm("" : "+v"(lo), "+v"(hi));
      const float send = upper ? lo : hi;
      const float keep = upper ? hi : lo;
      v[i] = keep + lane_xor_in_row<M>(send, lane);
    }
  }
}

// Sum N values (a power of two <= 64) over the 64 lanes of a wavefront by
// halving exchanges: afterwards lane (64/N)*i holds the total of value i.
// Each level halves the values (masks 32, 16, ..., 1); once one is left the
// remaining masks add it across lanes.
template <int N>
__device__ __forceinline__ void wave_reduce_transpose(float (&v)[N], int lane) {
  static_assert(N >= 1 && N <= 64 && (N & (N - 1)) == 0, "N must be a power of two <= 64");
  reduce_step<32, N>(v, lane);
  reduce_step<16, (N >= 2 ? N / 2 : 1)>(v, lane);
  reduce_step<8, (N >= 4 ? N / 4 : 1)>(v, lane);
  reduce_step<4, (N >= 8 ? N / 8 : 1)>(v, lane);
  reduce_step<2, (N >= 16 ? N / 16 : 1)>(v, lane);
  reduce_step<1, (N >= 32 ? N / 32 : 1)>(v, lane);
}

// Workgroup barrier that orders LDS only.  __syncthreads() also orders global
// memory, so it waits for every global load in flight; this one lets weight
// loads issued before it stay in flight across the barrier.
// Packed 64-row activations of the matrix-core path: row m, element k of a
// [rows, K] block at ((m/16 * K/32 + k/32) * 64 + (m%16 + 16 (k%32)/8)) * 8 +
// k%8, so a wave's MFMA fragment of one 16-row tile and one 32-wide k step is
// 1 KB contiguous (rows a multiple of 16, K of 32).
__host__ __device__ __forceinline__ size_t xpack_index(int m, int k, int K) {
  return ((size_t)((m >> 4) * (K >> 5) + (k >> 5)) * 64 + (m & 15) + 16 * ((k & 31) >> 3)) * 8 + (k & 7);
}

__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// The same (wave-uniform) pointer, marked as global memory, so loads and
// stores through it compile to global_* instead of flat_* instructions (a
// flat access also counts against lgkmcnt, so every LDS wait would wait for
// it too).  Needed where the compiler cannot see that a pointer came from a
// kernel argument.  The global-address-space copy passes through an empty
// asm so the compiler cannot fold the two casts back into the generic
// pointer.
template <typename T>
__device__ __forceinline__ T* as_global(T* p) {
  __attribute__((address_space(1))) T* g = (__attribute__((address_space(1))) T*)p;
  asm volatile("" : "+s"(g));
  return (T*)g;
}

// Wait until this wave's vector memory operations have completed (stores
// acknowledged): vmcnt(0), expcnt and lgkmcnt left at their maxima.
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0f70); }

// The wave's index in its workgroup, as a scalar (the compiler cannot always
// tell that threadIdx.x / 64 is the same for every lane of a wave).
__device__ __forceinline__ int wave_index(int tid) { return __builtin_amdgcn_readfirstlane(tid >> 6); }

// The step's early-exit flag, requested as a vector load: its wait then sits
// at the flag's first use (flag_set), after the kernel's weight requests.  A
// plain load of the uniform address becomes a scalar load, which the
// compiler waits for right away -- one more memory round trip ahead of the
// kernel's first request.  The opaque zero index keeps it a vector load.
__device__ __forceinline__ int32_t request_flag(const int32_t* p) {
  int z;
  asm volatile("v_mov_b32 %0, 0" : "=v"(z));
  return __builtin_nontemporal_load(p + z);
}
__device__ __forceinline__ bool flag_set(int32_t v) { return __builtin_amdgcn_readfirstlane(v) != 0; }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}

// The same reductions with the steps inside 16-lane rows on DPP moves (quad
// swaps, then the 8- and 16-lane mirrors: a few cycles each, no LDS round
// trip) and the two steps across rows on permlane swaps.  Every lane ends
// with the same value (each step adds or compares a pair symmetrically).
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += dpp_move<kDppQuadXor1>(v);
  v += dpp_move<kDppQuadXor2>(v);
  v += dpp_move<kDppRowHalfMirror>(v);
  v += dpp_move<kDppRowMirror>(v);
  v = swap_add<16>(v, v);
  v = swap_add<32>(v, v);
  return v;
}
__device__ __forceinline__ float wave_max_dpp(float v) {
  v = fmaxf(v, dpp_move<kDppQuadXor1>(v));
  v = fmaxf(v, dpp_move<kDppQuadXor2>(v));
  v = fmaxf(v, dpp_move<kDppRowHalfMirror>(v));
  v = fmaxf(v, dpp_move<kDppRowMirror>(v));
  v = xor_max<16>(v, 0);
  v = xor_max<32>(v, 0);
  return v;
}
