// Device-coherent (agent-scope) word access for hand-offs between work
// groups of one launch: `global_store/load ... sc1` on gfx950, visible
// across the XCDs' separate L2 caches without any cache writeback or
// invalidate. Used by the decode kernel's split-K merge and the prefill
// kernel's key-split merge.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace mv {

__device__ __forceinline__ void store_coherent_u64(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t load_coherent_u64(const uint64_t* p) {
  return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_coherent_u32(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t load_coherent_u32(const uint32_t* p) {
  return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Two fp32 values in one 8-byte word (lo = first in memory).
__device__ __forceinline__ uint64_t pack_f32x2(float lo, float hi) {
  return static_cast<uint64_t>(__float_as_uint(lo)) | (static_cast<uint64_t>(__float_as_uint(hi)) << 32);
}
__device__ __forceinline__ float unpack_lo(uint64_t v) { return __uint_as_float(static_cast<uint32_t>(v)); }
__device__ __forceinline__ float unpack_hi(uint64_t v) { return __uint_as_float(static_cast<uint32_t>(v >> 32)); }

}  // namespace mv
