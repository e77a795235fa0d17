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
// exactly into three bf16 parts (hi = bf16(W), mid = bf16(W - hi),
// lo = bf16(W - hi - mid); 3 x 8 significant bits cover fp32's 24), so
// x . W = x . hi + x . mid + x . lo with exact bf16 x bf16 products
// accumulated in fp32 by v_mfma_f32_16x16x32_bf16.
//  * router_split_kernel writes the three planes once per call into the
//    caller's scratch ([3][E][H] bf16), so the VALU split is not repeated by
//    every token block.
//  * router_fused_kernel: a block (4 wavefronts) owns 16 tokens; the waves
//    split the hidden dimension in interleaved 32-wide slices, their partial
//    logits are added in a fixed order through LDS, then each wave runs the
//    top-k of 4 tokens with one lane per expert.
// ---------------------------------------------------------------------------
typedef __bf16 rbf16x8_t __attribute__((ext_vector_type(8)));
typedef float rfloatx4_t __attribute__((ext_vector_type(4)));
constexpr int kRouterTokens = 16;

__global__ __launch_bounds__(256) void router_split_kernel(const float* __restrict__ w,
                                                           uint16_t* __restrict__ planes, int64_t n) {
    const int64_t i = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 8;
    if (i >= n) return;
    const float4 w0 = *reinterpret_cast<const float4*>(w + i);
    const float4 w1 = *reinterpret_cast<const float4*>(w + i + 4);
    const float v[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
    uint32_t hi[4], mid[4], lo[4];
#pragma unroll
    for (int j = 0; j < 8; j += 2) {
        float h[2], m[2], l[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            h[t] = round_bf16(v[j + t]);
            const float r1 = v[j + t] - h[t];  // exact
            m[t] = round_bf16(r1);
            l[t] = r1 - m[t];                  // exact, fits bf16
        }
        hi[j / 2] = pack_bf16x2(h[0], h[1]);
        mid[j / 2] = pack_bf16x2(m[0], m[1]);
        lo[j / 2] = pack_bf16x2(l[0], l[1]);
    }
    *reinterpret_cast<uint4*>(planes + i) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
    *reinterpret_cast<uint4*>(planes + n + i) = make_uint4(mid[0], mid[1], mid[2], mid[3]);
    *reinterpret_cast<uint4*>(planes + 2 * n + i) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
}

// NT expert column tiles of 16 (E <= 16 * NT); MT token tiles of 16 per block,
// which share each weight slice a block reads from L2.
template <int NT, int MT>
__global__ __launch_bounds__(256) void router_fused_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ planes,
    const float* __restrict__ bias, int32_t* __restrict__ ids32, int64_t* __restrict__ ids64,
    float* __restrict__ weights, float* __restrict__ logits_out, int64_t tokens, int hidden,
    int experts, int topk) {
    constexpr int TB = kRouterTokens * MT;  // tokens per block
    __shared__ float part[4][TB][16 * NT];
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int64_t t0 = static_cast<int64_t>(blockIdx.x) * TB;
    const int m = lane & 15;   // A row (token) and B column (expert within a tile)
    const int kq = lane >> 4;  // 8-element k block within the 32-wide slice
    const int64_t plane = static_cast<int64_t>(experts) * hidden;
    const uint16_t* xrow[MT];
    bool live[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const int64_t t = t0 + mt * kRouterTokens + m;
        live[mt] = t < tokens;
        xrow[mt] = x + (live[mt] ? t : 0) * static_cast<int64_t>(hidden);
    }

    rfloatx4_t acc[MT][NT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = rfloatx4_t{0.f, 0.f, 0.f, 0.f};

    // Slices are visited in batches of kBatch with every load of a batch issued
    // before its MFMAs, so each wave keeps several 16-byte loads in flight.
    constexpr int kBatch = NT * MT >= 8 ? 2 : (NT * MT >= 4 ? 4 : 8);
    auto load8 = [](const uint16_t* src) {
        rbf16x8_t v;
        const uint4 raw = *reinterpret_cast<const uint4*>(src);
        __builtin_memcpy(&v, &raw, 16);
        return v;
    };
    rbf16x8_t zero;
#pragma unroll
    for (int j = 0; j < 8; ++j) zero[j] = static_cast<__bf16>(0.0f);
    for (int kb = wave * 32; kb < hidden; kb += 128 * kBatch) {
        rbf16x8_t a[kBatch][MT];
        rbf16x8_t w[kBatch][NT][3];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            const int k = kb + u * 128 + kq * 8;
            const bool kin = k < hidden;  // hidden % 8 == 0: a block is all in or all out
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) a[u][mt] = (live[mt] && kin) ? load8(xrow[mt] + k) : zero;
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const int e = nt * 16 + m;
                const bool ok = e < experts && kin;
                const uint16_t* src = planes + static_cast<int64_t>(e) * hidden + k;
#pragma unroll
                for (int q = 0; q < 3; ++q) w[u][nt][q] = ok ? load8(src + q * plane) : zero;
            }
        }
#pragma unroll
        for (int u = 0; u < kBatch; ++u)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) {
                    acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[u][mt], w[u][nt][2], acc[mt][nt], 0, 0, 0);
                    acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[u][mt], w[u][nt][1], acc[mt][nt], 0, 0, 0);
                    acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[u][mt], w[u][nt][0], acc[mt][nt], 0, 0, 0);
                }
    }
    // 16x16 result: lane l holds tokens 4*(l/16) + r of its token tile, expert column l%16.
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int r = 0; r < 4; ++r) part[wave][mt * kRouterTokens + 4 * kq + r][nt * 16 + m] = acc[mt][nt][r];
    __syncthreads();

    // Top-k: wave w handles tokens w*TB/4 .. (w+1)*TB/4 - 1, one lane per expert.
    for (int i = 0; i < TB / 4; ++i) {
        const int tl = wave * (TB / 4) + i;
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

int64_t router_scratch_bytes(int64_t experts, int64_t hidden) { return 3 * experts * hidden * 2; }

int launch_router_fused(const uint16_t* x, const float* router_w, const float* bias,
                        int32_t* ids32, int64_t* ids64, float* weights, float* logits_out,
                        uint16_t* planes, int64_t tokens, int hidden, int experts, int topk,
                        hipStream_t stream) {
    if (tokens == 0) return MOE_OK;
    const int64_t n = static_cast<int64_t>(experts) * hidden;
    hipLaunchKernelGGL(router_split_kernel, dim3(static_cast<unsigned>((n / 8 + 255) / 256)), dim3(256), 0,
                       stream, router_w, planes, n);
    const int rc = check_launch("router_split_kernel");
    if (rc != MOE_OK) return rc;
    // One token tile per block: measured at E=64, H=2048, T=8192, four tiles per
    // block (fewer, longer blocks) ran 1.5x slower than one.
#define MOE_ROUTER_CASE(NTV, MTV)                                                                      \
    hipLaunchKernelGGL((router_fused_kernel<NTV, MTV>),                                                \
                       dim3(static_cast<unsigned>((tokens + kRouterTokens * MTV - 1) / (kRouterTokens * MTV))), \
                       dim3(256), 0, stream, x, planes, bias, ids32, ids64, weights, logits_out, tokens, \
                       hidden, experts, topk)
    if (experts <= 16) {
        MOE_ROUTER_CASE(1, 1);
    } else if (experts <= 32) {
        MOE_ROUTER_CASE(2, 1);
    } else if (experts <= 64) {
        MOE_ROUTER_CASE(4, 1);
    } else {
        return fail(MOE_ERR_UNSUPPORTED, "experts=%d exceeds 64", experts);
    }
#undef MOE_ROUTER_CASE
    return check_launch("router_fused_kernel");
}

}  // namespace moe
