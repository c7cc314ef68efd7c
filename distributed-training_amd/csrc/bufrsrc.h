// Raw buffer accesses: a wave-uniform resource (base address and byte range),
// a per-lane byte offset that stays fixed over a loop and a wave-uniform byte
// offset, so addressing takes no vector instructions. The range check covers
// the per-lane offset only: an access whose lane offset is at or past the
// range reads 0 and writes nothing, while the wave-uniform offset is added
// unchecked -- every caller that relies on the check puts the whole offset in
// the lane offset. Shared by the attention, GEMM-epilogue and cross-entropy
// kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace dtmi {

typedef __amdgpu_buffer_rsrc_t Rsrc;
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ Rsrc make_rsrc(const void* base, uint64_t bytes) {
  const uint32_t n = bytes < 0xFFFFFFFFull ? (uint32_t)bytes : 0xFFFFFFFFu;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)n, 0x00020000);
}
__device__ __forceinline__ f32x4 buf_load4(Rsrc r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0));
}
__device__ __forceinline__ float buf_load1(Rsrc r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, 0));
}
__device__ __forceinline__ void buf_store4(f32x4 x, Rsrc r, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(__attribute__((ext_vector_type(4))) int, x), r, (int)voff,
                                         (int)soff, 0);
}
__device__ __forceinline__ void buf_store1(float x, Rsrc r, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(int, x), r, (int)voff, (int)soff, 0);
}

}  // namespace dtmi
