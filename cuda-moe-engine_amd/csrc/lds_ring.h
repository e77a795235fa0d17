// Direct-to-LDS loading helpers shared by the ring kernels (gemm.hip, router.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>
#include <utility>

namespace moe {

constexpr uint32_t kRsrcWord3 = 0x00020000u;  // raw buffer, 32-bit dword format

// Resource descriptor from wave-uniform values, pinned to SGPRs with readfirstlane
// so buffer instructions take it directly (no waterfall loop).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    const uint64_t addr = reinterpret_cast<uint64_t>(base);
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(addr));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(addr >> 32));
    void* uniform_base = reinterpret_cast<void*>((static_cast<uint64_t>(hi) << 32) | lo);
    return __builtin_amdgcn_make_buffer_rsrc(uniform_base, 0, __builtin_amdgcn_readfirstlane(bytes),
                                             kRsrcWord3);
}

// soffset is wave-uniform at every call; readfirstlane states it, so that the
// compiler keeps it in an SGPR. Where it could not prove that (stage indices
// clamped with min() in the prologues), it wrapped each load in a waterfall
// loop of about ten instructions.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t rsrc, char* lds_dst, uint32_t voffset,
                                      uint32_t soffset) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        rsrc, (__attribute__((address_space(3))) void*)(lds_dst), 16, voffset,
        __builtin_amdgcn_readfirstlane(soffset), 0, 0);
}

// s_waitcnt vmcnt(VM) lgkmcnt(LGKM) (gfx9 encoding: vmcnt[3:0] in bits 3:0 and
// vmcnt[5:4] in bits 15:14, expcnt in bits 6:4 with 7 = no wait, lgkmcnt in bits 11:8).
template <int VM, int LGKM = 0>
__device__ __forceinline__ void wait_vm_lgkm() {
    static_assert(VM >= 0 && VM < 64, "vmcnt range");
    static_assert(LGKM >= 0 && LGKM < 16, "lgkmcnt range");
    __builtin_amdgcn_s_waitcnt((VM & 15) | ((VM >> 4) << 14) | (7 << 4) | (LGKM << 8));
}
// Workgroup barrier without the implied wait for all memory operations (the
// explicit wait above bounds what must have landed); the memory clobber keeps
// the compiler from moving LDS accesses across it.
__device__ __forceinline__ void ring_barrier() { asm volatile("s_barrier" ::: "memory"); }

// f(integral_constant<int, 0>) ... f(integral_constant<int, N-1>), unrolled.
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}

}  // namespace moe
