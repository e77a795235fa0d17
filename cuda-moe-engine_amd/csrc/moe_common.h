// Shared device helpers and host-side status plumbing for the gfx950 MoE kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "moe_hip.h"

namespace moe {

constexpr int kWave = 64;        // CDNA wavefront width
constexpr int kMaxExperts = 64;  // one lane per expert in the routing kernels
constexpr int kMaxTopk = 8;
constexpr int kNumXcd = 8;       // MI355X: 8 XCDs, workgroups dispatched round-robin

// ---------------------------------------------------------------------------
// bf16 / fp16 conversion. bf16 is stored as uint16_t bit patterns.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
    return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// Round-to-nearest-even; NaN stays a quiet NaN with its sign.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
    _Float16 v;
    __builtin_memcpy(&v, &h, 2);
    return static_cast<float>(v);
}

__device__ __forceinline__ uint16_t f32_to_f16(float f) {
    _Float16 v = static_cast<_Float16>(f);
    uint16_t h;
    __builtin_memcpy(&h, &v, 2);
    return h;
}

// Element access by storage dtype (MOE_DTYPE_*), used by the transport and
// activation kernels that support fp32 / fp16 / bf16.
template <int DT> struct Elem;
template <> struct Elem<MOE_DTYPE_F32> {
    using T = float;
    static __device__ __forceinline__ float load(T v) { return v; }
    static __device__ __forceinline__ T store(float f) { return f; }
};
template <> struct Elem<MOE_DTYPE_F16> {
    using T = uint16_t;
    static __device__ __forceinline__ float load(T v) { return f16_to_f32(v); }
    static __device__ __forceinline__ T store(float f) { return f32_to_f16(f); }
};
template <> struct Elem<MOE_DTYPE_BF16> {
    using T = uint16_t;
    static __device__ __forceinline__ float load(T v) { return bf16_to_f32(v); }
    static __device__ __forceinline__ T store(float f) { return f32_to_bf16(f); }
};

inline int dtype_size(int dtype) {
    switch (dtype) {
        case MOE_DTYPE_F32: return 4;
        case MOE_DTYPE_F16: return 2;
        case MOE_DTYPE_BF16: return 2;
        default: return 0;
    }
}

// ---------------------------------------------------------------------------
// Host-side error reporting: a status code plus a thread-local message.
// ---------------------------------------------------------------------------
void set_error(const char* fmt, ...);
int fail(int status, const char* fmt, ...);
int check_launch(const char* what);

}  // namespace moe

#define MOE_REQUIRE(cond, status, ...)                \
    do {                                              \
        if (!(cond)) return ::moe::fail(status, __VA_ARGS__); \
    } while (0)
