// In-launch exchange of vectors between workgroups on different XCDs.
//
// A producer publishes 8-byte (data, tag) pairs with agent-scope stores (sc1:
// written through to where every XCD's loads see them); a consumer reads them
// with agent-scope loads and accepts a pair only when its tag is the value the
// current call uses. 8-byte halves of a 16-byte access are single-copy
// atomic, so a pair never mixes two calls' data, and no counter, fence or
// read-modify-write is needed. Waits are bounded in s_memrealtime ticks
// (100 MHz) and report a give-up through a status word.
#pragma once

#include "iron_common.hpp"

namespace iron {
namespace {

typedef unsigned u32x4_v __attribute__((ext_vector_type(4)));
typedef unsigned u32x2_v __attribute__((ext_vector_type(2)));
constexpr int kSc1 = 16;  // cache-policy bits of the buffer builtins: sc1 (agent scope)

__device__ __forceinline__ __amdgpu_buffer_rsrc_t xch_rsrc(const unsigned char* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<unsigned char*>(base), 0, 0x7fffffff, kBufferFlags);
}
// pairs p and p + 1 (p even)
__device__ __forceinline__ u32x4_v ld_pairs2(__amdgpu_buffer_rsrc_t r, int p) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, p * 8, 0, kSc1);
}
__device__ __forceinline__ u32x2_v ld_pair(__amdgpu_buffer_rsrc_t r, int p) {
  return __builtin_amdgcn_raw_buffer_load_b64(r, p * 8, 0, kSc1);
}
__device__ __forceinline__ void st_pairs2(__amdgpu_buffer_rsrc_t r, int p, uint32_t d0, uint32_t d1, unsigned tag) {
  __builtin_amdgcn_raw_buffer_store_b128(u32x4_v{d0, tag, d1, tag}, r, p * 8, 0, kSc1);
}
__device__ __forceinline__ void st_pair(__amdgpu_buffer_rsrc_t r, int p, uint32_t d, unsigned tag) {
  __builtin_amdgcn_raw_buffer_store_b64(u32x2_v{d, tag}, r, p * 8, 0, kSc1);
}

__device__ __forceinline__ unsigned long long now_ticks() { return __builtin_amdgcn_s_memrealtime(); }
__device__ __forceinline__ unsigned read_status(const unsigned* status) {
  return __hip_atomic_load(status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void give_up(unsigned* status, unsigned bit) {
  __hip_atomic_fetch_or(status, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace
}  // namespace iron
