// Routing kernels for gfx950: bias + top-k (ties to the lower expert id) +
// selected-score softmax, on given logits or with the fp32 router projection
// fused in (on MFMA, see router_fused_kernel).
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
// Fused router on MFMA. logits = x . W^T with x bf16 and W fp32: W is split
// exactly-to-24-bits into three bf16 parts (hi = bf16(W), mid = bf16(W - hi),
// lo = bf16(W - hi - mid)), so x . W = x . hi + x . mid + x . lo with exact
// bf16 x bf16 products accumulated in fp32 by v_mfma_f32_16x16x32_bf16.
// A block (4 wavefronts) owns 16 tokens; the waves split the hidden dimension
// in interleaved 32-wide slices, their partial logits are added in a fixed
// order through LDS, then each wave runs the top-k of 4 tokens with one lane
// per expert. Reading x once is the only HBM traffic of consequence.
// ---------------------------------------------------------------------------
typedef __bf16 rbf16x8_t __attribute__((ext_vector_type(8)));
typedef float rfloatx4_t __attribute__((ext_vector_type(4)));
constexpr int kRouterTokens = 16;

__device__ __forceinline__ void split3(const float (&w)[8], rbf16x8_t& hi, rbf16x8_t& mid, rbf16x8_t& lo) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const float h = round_bf16(w[j]);
        const float r1 = w[j] - h;  // exact
        const float m = round_bf16(r1);
        const float r2 = r1 - m;    // exact
        hi[j] = static_cast<__bf16>(h);
        mid[j] = static_cast<__bf16>(m);
        lo[j] = static_cast<__bf16>(r2);
    }
}

template <int NT>  // expert column tiles of 16: E <= 16 * NT
__global__ __launch_bounds__(256) void router_fused_kernel(
    const uint16_t* __restrict__ x, const float* __restrict__ router_w,
    const float* __restrict__ bias, int32_t* __restrict__ ids32, int64_t* __restrict__ ids64,
    float* __restrict__ weights, float* __restrict__ logits_out, int64_t tokens, int hidden,
    int experts, int topk) {
    __shared__ float part[4][kRouterTokens][16 * NT];
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int64_t t0 = static_cast<int64_t>(blockIdx.x) * kRouterTokens;
    const int m = lane & 15;   // A row (token) and B column (expert within a tile)
    const int kq = lane >> 4;  // 8-element k block within the 32-wide slice
    const bool live = t0 + m < tokens;
    const uint16_t* xrow = x + (live ? t0 + m : t0) * static_cast<int64_t>(hidden);

    rfloatx4_t acc[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[nt] = rfloatx4_t{0.f, 0.f, 0.f, 0.f};

    // Slices are visited in batches of kBatch with every load of a batch issued
    // before its MFMAs, so each wave keeps several 16-byte loads in flight.
    constexpr int kBatch = 8;
    for (int kb = wave * 32; kb < hidden; kb += 128 * kBatch) {
        rbf16x8_t a[kBatch];
        float w[kBatch][NT][8];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            const int k = kb + u * 128 + kq * 8;
            const bool kin = k < hidden;  // hidden % 8 == 0: a block is all in or all out
            if (live && kin) {
                const uint4 raw = *reinterpret_cast<const uint4*>(xrow + k);
                __builtin_memcpy(&a[u], &raw, 16);
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j) a[u][j] = static_cast<__bf16>(0.0f);
            }
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const int e = nt * 16 + m;
                if (e < experts && kin) {
                    const float* src = router_w + static_cast<int64_t>(e) * hidden + k;
                    const float4 w0 = *reinterpret_cast<const float4*>(src);
                    const float4 w1 = *reinterpret_cast<const float4*>(src + 4);
                    w[u][nt][0] = w0.x; w[u][nt][1] = w0.y; w[u][nt][2] = w0.z; w[u][nt][3] = w0.w;
                    w[u][nt][4] = w1.x; w[u][nt][5] = w1.y; w[u][nt][6] = w1.z; w[u][nt][7] = w1.w;
                } else {
#pragma unroll
                    for (int j = 0; j < 8; ++j) w[u][nt][j] = 0.0f;
                }
            }
        }
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                rbf16x8_t hi, mid, lo;
                split3(w[u][nt], hi, mid, lo);
                acc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[u], lo, acc[nt], 0, 0, 0);
                acc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[u], mid, acc[nt], 0, 0, 0);
                acc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[u], hi, acc[nt], 0, 0, 0);
            }
        }
    }
    // 16x16 result: lane l holds tokens 4*(l/16) + r, expert column l%16.
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int r = 0; r < 4; ++r) part[wave][4 * kq + r][nt * 16 + m] = acc[nt][r];
    __syncthreads();

    // Top-k: wave w handles tokens 4w..4w+3, one lane per expert.
    for (int i = 0; i < kRouterTokens / 4; ++i) {
        const int tl = wave * 4 + i;
        const int64_t token = t0 + tl;
        if (token >= tokens) break;
        float v = -INFINITY;
        int idx = INT_MAX;
        if (lane < experts) {
            const float logit = ((part[0][tl][lane] + part[1][tl][lane]) + part[2][tl][lane]) + part[3][tl][lane];
            if (logits_out) logits_out[token * experts + lane] = logit;
            v = logit + bias[lane];
            idx = lane;
        }
        float sel_v[kMaxTopk];
        int sel_i[kMaxTopk];
#pragma unroll
        for (int k = 0; k < kMaxTopk; ++k) {
            if (k < topk) {
                float bv = v;
                int bi = idx;
#pragma unroll
                for (int msk = 32; msk >= 1; msk >>= 1) {
                    const float ov = __shfl_xor(bv, msk);
                    const int oi = __shfl_xor(bi, msk);
                    if (ov > bv || (ov == bv && oi < bi)) {
                        bv = ov;
                        bi = oi;
                    }
                }
                sel_v[k] = bv;
                sel_i[k] = bi;
                if (idx == bi) {
                    v = -INFINITY;
                    idx = INT_MAX;
                }
            }
        }
        if (lane == 0) write_route(sel_v, sel_i, topk, token, ids32, ids64, weights);
    }
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
#define MOE_ROUTER_CASE(NTV)                                                               \
    hipLaunchKernelGGL(router_fused_kernel<NTV>, grid, dim3(256), 0, stream, x, router_w,  \
                       bias, ids32, ids64, weights, logits_out, tokens, hidden, experts,   \
                       topk)
    if (experts <= 16) {
        MOE_ROUTER_CASE(1);
    } else if (experts <= 32) {
        MOE_ROUTER_CASE(2);
    } else if (experts <= 64) {
        MOE_ROUTER_CASE(4);
    } else {
        return fail(MOE_ERR_UNSUPPORTED, "experts=%d exceeds 64", experts);
    }
#undef MOE_ROUTER_CASE
    return check_launch("router_fused_kernel");
}

}  // namespace moe
