// Routing kernels for gfx950: bias + top-k (ties to the lower expert id) +
// selected-score softmax, on given logits or with the fp32 router projection
// fused in.
//
// Reference behaviour: src/moe_dispatch/csrc/dispatch.cu:325-376 (tie rule
// :331-333, K=2 weight formula :366-374) and src/moe_dispatch/layer.py:122-135.
// The reference handles K in {1,2} with two experts per lane of a 32-lane warp;
// here a 64-lane wavefront holds one expert per lane and K goes up to 8.
#include <climits>
#include <cmath>

#include "moe_common.h"

namespace moe {

// Writes ids and weights for one token from its K selected (value, id) pairs
// (values descending). K=1 -> 1; K=2 -> the reference closed form; K>2 ->
// exp(v_j - v_0) / sum_i exp(v_i - v_0), summed in selection order.
__device__ __forceinline__ void write_route(const float* sel_v, const int* sel_i, int topk,
                                            int64_t token, int32_t* ids32, int64_t* ids64,
                                            float* weights) {
    const int64_t base = token * topk;
    float w[kMaxTopk];
    if (topk == 1) {
        w[0] = 1.0f;
    } else if (topk == 2) {
        const float relative = expf(sel_v[1] - sel_v[0]);
        const float norm = 1.0f / (1.0f + relative);
        w[0] = norm;
        w[1] = relative * norm;
    } else {
        float rel[kMaxTopk];
        float total = 0.0f;
#pragma unroll
        for (int j = 0; j < kMaxTopk; ++j) {
            if (j < topk) {
                rel[j] = expf(sel_v[j] - sel_v[0]);
                total = total + rel[j];
            }
        }
        const float inv = 1.0f / total;
#pragma unroll
        for (int j = 0; j < kMaxTopk; ++j)
            if (j < topk) w[j] = rel[j] * inv;
    }
#pragma unroll
    for (int j = 0; j < kMaxTopk; ++j) {
        if (j < topk) {
            ids32[base + j] = sel_i[j];
            if (ids64) ids64[base + j] = sel_i[j];
            weights[base + j] = w[j];
        }
    }
}

// ---------------------------------------------------------------------------
// Top-k on given logits. Lanes form groups of G = pow2 >= E; each group owns
// one token and each lane one expert. K rounds of a butterfly argmax inside
// the group (larger value wins, equal values go to the lower id).
// ---------------------------------------------------------------------------
template <int G>
__global__ __launch_bounds__(256) void topk_route_kernel(const float* __restrict__ logits,
                                                         const float* __restrict__ bias,
                                                         int32_t* __restrict__ ids32,
                                                         int64_t* __restrict__ ids64,
                                                         float* __restrict__ weights,
                                                         int64_t tokens, int experts, int topk) {
    constexpr int kTokensPerBlock = 256 / G;
    const int lane_g = threadIdx.x % G;
    const int64_t token = static_cast<int64_t>(blockIdx.x) * kTokensPerBlock + threadIdx.x / G;
    const bool live = token < tokens;
    float v = -INFINITY;
    int idx = INT_MAX;
    if (live && lane_g < experts) {
        v = logits[token * experts + lane_g] + bias[lane_g];
        idx = lane_g;
    }
    float sel_v[kMaxTopk];
    int sel_i[kMaxTopk];
#pragma unroll
    for (int k = 0; k < kMaxTopk; ++k) {
        if (k < topk) {
            float bv = v;
            int bi = idx;
#pragma unroll
            for (int m = G / 2; m >= 1; m >>= 1) {
                const float ov = __shfl_xor(bv, m);
                const int oi = __shfl_xor(bi, m);
                if (ov > bv || (ov == bv && oi < bi)) {
                    bv = ov;
                    bi = oi;
                }
            }
            sel_v[k] = bv;
            sel_i[k] = bi;
            if (idx == bi) {  // remove the winner from later rounds
                v = -INFINITY;
                idx = INT_MAX;
            }
        }
    }
    if (live && lane_g == 0) write_route(sel_v, sel_i, topk, token, ids32, ids64, weights);
}

// ---------------------------------------------------------------------------
// Fused router. A block of 256 threads owns 32 tokens, 8 lanes per token.
// The fp32 router matrix is staged through LDS in column chunks shared by the
// 32 tokens; each lane accumulates EB partial dot products over its columns
// (x converted exactly from bf16), then the 8 lanes of a token reduce with a
// butterfly and lane 0 performs the top-k selection.
// ---------------------------------------------------------------------------
constexpr int kRouterTokens = 32;
constexpr int kRouterLdsFloats = 8192;  // 32 KiB of router weights per chunk

template <int EB>
__global__ __launch_bounds__(256) void router_fused_kernel(
    const uint16_t* __restrict__ x, const float* __restrict__ router_w,
    const float* __restrict__ bias, int32_t* __restrict__ ids32, int64_t* __restrict__ ids64,
    float* __restrict__ weights, float* __restrict__ logits_out, int64_t tokens, int hidden,
    int experts, int topk) {
    constexpr int HC = kRouterLdsFloats / EB;  // columns per chunk (multiple of 64)
    __shared__ __attribute__((aligned(16))) float ws[EB * HC];
    const int tid = threadIdx.x;
    const int lane8 = tid & 7;
    const int64_t token = static_cast<int64_t>(blockIdx.x) * kRouterTokens + (tid >> 3);
    const bool live = token < tokens;
    const uint16_t* xrow = x + (live ? token : 0) * static_cast<int64_t>(hidden);

    float acc[EB];
#pragma unroll
    for (int e = 0; e < EB; ++e) acc[e] = 0.0f;

    for (int h0 = 0; h0 < hidden; h0 += HC) {
        // Stage router_w[:, h0:h0+HC] (zero past E or H) as [EB][HC].
        __syncthreads();
        for (int i = tid; i < EB * HC / 4; i += 256) {
            const int e = (i * 4) / HC;
            const int c = (i * 4) % HC;
            float4 val = make_float4(0.f, 0.f, 0.f, 0.f);
            if (e < experts) {
                const int col = h0 + c;
                const float* src = router_w + static_cast<int64_t>(e) * hidden + col;
                if (col + 3 < hidden) {
                    val = *reinterpret_cast<const float4*>(src);
                } else {
                    if (col + 0 < hidden) val.x = src[0];
                    if (col + 1 < hidden) val.y = src[1];
                    if (col + 2 < hidden) val.z = src[2];
                }
            }
            *reinterpret_cast<float4*>(&ws[e * HC + c]) = val;
        }
        __syncthreads();
        const int width = min(HC, hidden - h0);
        for (int c0 = lane8 * 8; c0 < width; c0 += 64) {
            uint4 raw = make_uint4(0, 0, 0, 0);
            if (live) raw = *reinterpret_cast<const uint4*>(xrow + h0 + c0);
            float xv[8];
            xv[0] = bf16_to_f32(raw.x & 0xffff);
            xv[1] = bf16_to_f32(raw.x >> 16);
            xv[2] = bf16_to_f32(raw.y & 0xffff);
            xv[3] = bf16_to_f32(raw.y >> 16);
            xv[4] = bf16_to_f32(raw.z & 0xffff);
            xv[5] = bf16_to_f32(raw.z >> 16);
            xv[6] = bf16_to_f32(raw.w & 0xffff);
            xv[7] = bf16_to_f32(raw.w >> 16);
#pragma unroll
            for (int e = 0; e < EB; ++e) {
                const float4 w0 = *reinterpret_cast<const float4*>(&ws[e * HC + c0]);
                const float4 w1 = *reinterpret_cast<const float4*>(&ws[e * HC + c0 + 4]);
                float s = acc[e];
                s = fmaf(xv[0], w0.x, s);
                s = fmaf(xv[1], w0.y, s);
                s = fmaf(xv[2], w0.z, s);
                s = fmaf(xv[3], w0.w, s);
                s = fmaf(xv[4], w1.x, s);
                s = fmaf(xv[5], w1.y, s);
                s = fmaf(xv[6], w1.z, s);
                s = fmaf(xv[7], w1.w, s);
                acc[e] = s;
            }
        }
    }
    // Reduce the 8 partial sums of each token.
#pragma unroll
    for (int e = 0; e < EB; ++e) {
        float s = acc[e];
        s += __shfl_xor(s, 1);
        s += __shfl_xor(s, 2);
        s += __shfl_xor(s, 4);
        acc[e] = s;
    }
    if (!live || lane8 != 0) return;
    float v[EB];
#pragma unroll
    for (int e = 0; e < EB; ++e) {
        if (e < experts) {
            if (logits_out) logits_out[token * experts + e] = acc[e];
            v[e] = acc[e] + bias[e];
        } else {
            v[e] = -INFINITY;
        }
    }
    float sel_v[kMaxTopk];
    int sel_i[kMaxTopk];
    uint64_t taken = 0;
#pragma unroll
    for (int k = 0; k < kMaxTopk; ++k) {
        if (k < topk) {
            float bv = -INFINITY;
            int bi = INT_MAX;
#pragma unroll
            for (int e = 0; e < EB; ++e) {
                const bool free_e = e < experts && !((taken >> e) & 1ull);
                // Ascending scan with strict '>' keeps the lower id on ties.
                if (free_e && (bi == INT_MAX || v[e] > bv)) {
                    bv = v[e];
                    bi = e;
                }
            }
            sel_v[k] = bv;
            sel_i[k] = bi;
            taken |= 1ull << bi;
        }
    }
    write_route(sel_v, sel_i, topk, token, ids32, ids64, weights);
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
static int group_size(int experts) {
    int g = 1;
    while (g < experts) g <<= 1;
    return g;
}

int launch_topk_route(const float* logits, const float* bias, int32_t* ids32, int64_t* ids64,
                      float* weights, int64_t tokens, int experts, int topk,
                      hipStream_t stream) {
    if (tokens == 0) return MOE_OK;
    const int g = group_size(experts);
    const int64_t per_block = 256 / g;
    const dim3 grid(static_cast<unsigned>((tokens + per_block - 1) / per_block));
#define MOE_TOPK_CASE(GV)                                                                  \
    case GV:                                                                               \
        hipLaunchKernelGGL(topk_route_kernel<GV>, grid, dim3(256), 0, stream, logits, bias, \
                           ids32, ids64, weights, tokens, experts, topk);                   \
        break;
    switch (g) {
        MOE_TOPK_CASE(1)
        MOE_TOPK_CASE(2)
        MOE_TOPK_CASE(4)
        MOE_TOPK_CASE(8)
        MOE_TOPK_CASE(16)
        MOE_TOPK_CASE(32)
        MOE_TOPK_CASE(64)
        default: return fail(MOE_ERR_UNSUPPORTED, "experts=%d exceeds 64", experts);
    }
#undef MOE_TOPK_CASE
    return check_launch("topk_route_kernel");
}

int launch_router_fused(const uint16_t* x, const float* router_w, const float* bias,
                        int32_t* ids32, int64_t* ids64, float* weights, float* logits_out,
                        int64_t tokens, int hidden, int experts, int topk, hipStream_t stream) {
    if (tokens == 0) return MOE_OK;
    const dim3 grid(static_cast<unsigned>((tokens + kRouterTokens - 1) / kRouterTokens));
#define MOE_ROUTER_CASE(EBV)                                                               \
    hipLaunchKernelGGL(router_fused_kernel<EBV>, grid, dim3(256), 0, stream, x, router_w,  \
                       bias, ids32, ids64, weights, logits_out, tokens, hidden, experts,   \
                       topk)
    if (experts <= 8) {
        MOE_ROUTER_CASE(8);
    } else if (experts <= 16) {
        MOE_ROUTER_CASE(16);
    } else if (experts <= 32) {
        MOE_ROUTER_CASE(32);
    } else if (experts <= 64) {
        MOE_ROUTER_CASE(64);
    } else {
        return fail(MOE_ERR_UNSUPPORTED, "experts=%d exceeds 64", experts);
    }
#undef MOE_ROUTER_CASE
    return check_launch("router_fused_kernel");
}

}  // namespace moe
