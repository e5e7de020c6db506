// Order keys and composites shared by the sampler kernels and the LM-head kernels (device code).
//
// ord_key maps a float to a u32 whose unsigned order is the float order (-0 with +0). A composite
// (key << 32 | ~index) orders elements as the reference's sort does: value descending, then index
// ascending (src/sampler.cpp:72-78), so the largest composite is the first element of the order.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace vsmp {

__device__ __forceinline__ uint32_t ord_key(float v) {
  uint32_t b = __float_as_uint(v);
  if (b == 0x80000000u) b = 0u;  // -0 sorts with +0 (they compare equal in the reference)
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float key_val(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}
__device__ __forceinline__ uint64_t comp(uint32_t key, uint32_t idx) {
  return (static_cast<uint64_t>(key) << 32) | static_cast<uint32_t>(~idx);
}
__device__ __forceinline__ uint32_t comp_key(uint64_t c) { return static_cast<uint32_t>(c >> 32); }
__device__ __forceinline__ int comp_idx(uint64_t c) { return static_cast<int>(~static_cast<uint32_t>(c)); }
__device__ __forceinline__ float comp_val(uint64_t c) { return key_val(comp_key(c)); }

}  // namespace vsmp
