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
