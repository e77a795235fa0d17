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

// Round-to-nearest-even; NaN becomes the quiet NaN (bits >> 16) | 0x40. gfx950's
// v_cvt_pk_bf16_f32 implements exactly this mapping (checked against the
// integer formulation on all 2^32 inputs), so conversions use the instruction.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float float2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    const float2_t f = {lo, hi};
    const bf16x2_t h = __builtin_convertvector(f, bf16x2_t);
    uint32_t u;
    __builtin_memcpy(&u, &h, 4);
    return u;
}

__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    const __bf16 h = static_cast<__bf16>(f);
    uint16_t u;
    __builtin_memcpy(&u, &h, 2);
    return u;
}

// Value of f rounded to bf16, as fp32.
__device__ __forceinline__ float round_bf16(float f) {
    return __uint_as_float(static_cast<uint32_t>(f32_to_bf16(f)) << 16);
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

// ---------------------------------------------------------------------------
// exp and SiLU with a fixed operation sequence, so a CPU restatement with
// IEEE fp32 operations reproduces them bit for bit: Cody-Waite reduction
// x = n*ln2 + r (ln2 = 16-bit head + tail, so n*ln2_hi is exact), degree-7
// Taylor polynomial of e^r in Horner form with separately rounded multiply and
// add, then ldexp. Within 2 ulp of exp on [-80, 88]; +inf above, 0 below
// (where 1 + e^x already rounds to 1).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float exp_f32(float x) {
#pragma clang fp contract(off)
    if (x != x) return x;
    if (x > 88.0f) return __builtin_inff();
    if (x < -80.0f) return 0.0f;
    const float n = rintf(x * __uint_as_float(0x3fb8aa3bu));  // log2(e)
    float r = x - n * __uint_as_float(0x3f317200u);            // ln2 head
    r = r - n * __uint_as_float(0x35bfbe8eu);                  // ln2 tail
    float p = __uint_as_float(0x39500d01u);                    // 1/7!
    p = p * r + __uint_as_float(0x3ab60b61u);                  // 1/6!
    p = p * r + __uint_as_float(0x3c088889u);                  // 1/5!
    p = p * r + __uint_as_float(0x3d2aaaabu);                  // 1/4!
    p = p * r + __uint_as_float(0x3e2aaaabu);                  // 1/3!
    p = p * r + 0.5f;
    p = p * r + 1.0f;
    p = p * r + 1.0f;
    return ldexpf(p, static_cast<int>(n));
}

// silu(g) = g / (1 + exp(-g)) with a correctly rounded fp32 division.
__device__ __forceinline__ float silu_f32(float g) {
#pragma clang fp contract(off)
    return g / (1.0f + exp_f32(-g));
}

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
