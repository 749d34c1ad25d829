// The records by which the workgroups that share a prefill tile's keys hand
// over their partial states (kernels_prefill.hip, kernels_prefill_f32.hip):
// 16-byte buffer stores and loads with the sc1 cache policy. HIP device code
// only.
#pragma once

#include "ckv_internal.h"

namespace ckv {

// The split tiles' records pass between workgroups as the decode's split-K
// partial records do (kernels_decode.hip), at 16 bytes per access: buffer
// stores and loads with the sc1 cache policy, the same instructions at the
// same policy that LLVM emits for relaxed agent-scope atomic stores and loads
// on gfx950 (global/buffer_store/load sc1: the store writes through, the
// load misses any L2 line that could be stale, so every XCD sees the data in
// memory without an L2 writeback); a wait for the stores' completion before
// one thread's relaxed agent-scope fetch-add counts the share in; the loads
// of the share that arrives last are issued after that fetch-add returns.
#if defined(__HIP_DEVICE_COMPILE__) && !defined(__gfx950__)
#error "the prefill's split-key handoff relies on gfx950's memory system; build for gfx950"
#endif
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
inline constexpr int cache_sc1 = 16; // the buffer builtins' cache-policy operand: sc1

__device__ __forceinline__ __amdgpu_buffer_rsrc_t record_rsrc(float* base, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(base, 0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ void agent_store4(__amdgpu_buffer_rsrc_t r, uint32_t off, float a,
                                             float b, float c, float d)
{
    const u32x4_t v = { __float_as_uint(a), __float_as_uint(b), __float_as_uint(c),
                        __float_as_uint(d) };
    __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, cache_sc1);
}

__device__ __forceinline__ u32x4_t agent_load4(__amdgpu_buffer_rsrc_t r, uint32_t off)
{
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, cache_sc1);
}

// Waits until every vector memory access this wave issued (stores included)
// has completed; a compiler barrier too.
__device__ __forceinline__ void wait_vector_memory()
{
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

} // namespace ckv
