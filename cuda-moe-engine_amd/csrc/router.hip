// Routing kernels for gfx950: bias + top-k (ties to the lower expert id) +
// selected-score softmax, on given logits or with the fp32 router projection
// fused in (on MFMA, see router_ring_kernel).
//
// Reference behaviour: src/moe_dispatch/csrc/dispatch.cu:325-376 (tie rule
// :331-333, K=2 weight formula :366-374) and src/moe_dispatch/layer.py:122-135.
// The reference handles K in {1,2} with two experts per lane of a 32-lane warp;
// here a 64-lane wavefront holds one expert per lane and K goes up to 8.
#include <climits>
#include <cmath>

#include "lds_ring.h"
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
//  * router_ring_kernel (below) multiplies x by the planes and runs top-k.
// ---------------------------------------------------------------------------

constexpr int kRouterTokens = 16;
constexpr int64_t kRankedPrefixMax = 4096;  // routing tiles x experts of a ranked route
constexpr int kRouterSplitTokens = 64;  // split-k routing up to this many tokens (E <= 16)
constexpr int kRouterSplitSlices = 16;
constexpr int kRouterSplitTiles = kRouterSplitTokens / kRouterTokens;
constexpr int64_t kRouterPartialBytes =
    static_cast<int64_t>(kRouterSplitTiles) * kRouterSplitSlices * kRouterTokens * 16 * 4;

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

// Fused router on an LDS ring. A block owns TB = 16*MT tokens and all experts
// (EB = 16*NT slots): per 64-k stage, the x rows (TB x 128 B) and the three
// weight planes (3*EB rows of 128 B, plane q at rows q*EB + e; slots e >= E
// read as zero) arrive in LDS through direct-to-LDS buffer loads of whole
// 128-byte lines, so the planes, which every block needs whole, are read from
// L2 once per block and shared by its waves. Stages sit in a ring of
// STAGES = 4U; each iteration waits for U stages at once, passes one barrier,
// refills the U slots the previous iteration freed (stages s + STAGES - U ..
// s + STAGES - 1) and computes its U stages. U is 4 for E <= 16 and 2 for
// E <= 32 (stages of 8 and 16 KiB), 1 above. Measured at H=4096 (kernel
// time): one token 12.4 -> 11.2 us, 4096 tokens 13.8 -> 12.8 us against one
// stage per barrier. A single token's routing stays bound by one CU issuing
// the 512 loads of the planes and waiting for them.
//  * The MT x NT output tiles of 16 tokens x 16 experts are spread over the
//    four waves; when there are fewer than four tiles, G = 4 / tiles waves
//    share a tile and take every G-th 32-k sub-step, and their partial logits
//    are added in wave order.
//  * Per sub-step a tile takes three MFMAs into one accumulator, lo, mid, hi.
//  * Partial logits go through LDS; then eight lanes per token run the top-k.
// Rows of 128 bytes hold 8 chunks of 16 bytes; chunk c of row r sits at
// physical chunk c ^ ((r >> 1) & 7), so 16 lanes reading 16 consecutive rows
// at one chunk are conflict free.
// Top-k over one token's biased logits held by eight lanes (lane `sub` holds
// experts sub*EPL .. sub*EPL+EPL-1; -inf past E). K rounds of: argmax over
// the lane's values (the lower expert wins a tie), the same across the eight
// lanes with three xor shuffles, then the winner is removed -- the
// reference's iterative argmax with ties to the lower id. Lane 0 writes.
template <int EPL>
__device__ __forceinline__ void select_eight_lanes(float (&v)[EPL], int sub, int topk, int64_t token,
                                                   int32_t* ids32, int64_t* ids64, float* weights,
                                                   int* tile_ids = nullptr) {
    float sel_v[kMaxTopk];
    int sel_i[kMaxTopk];
#pragma unroll
    for (int k = 0; k < kMaxTopk; ++k) {
        if (k < topk) {
            float bv = v[0];
            int bi = sub * EPL;
#pragma unroll
            for (int j = 1; j < EPL; ++j) {
                const bool take = v[j] > bv;
                bv = take ? v[j] : bv;
                bi = take ? sub * EPL + j : bi;
            }
#pragma unroll
            for (int msk = 1; msk < 8; msk <<= 1) {
                const float ov = __shfl_xor(bv, msk);
                const int oi = __shfl_xor(bi, msk);
                const bool take = ov > bv || (ov == bv && oi < bi);
                bv = take ? ov : bv;
                bi = take ? oi : bi;
            }
            sel_v[k] = bv;
            sel_i[k] = bi;
#pragma unroll
            for (int j = 0; j < EPL; ++j) v[j] = (sub * EPL + j == bi) ? -INFINITY : v[j];
        }
    }
    if (sub == 0) {
        write_route(sel_v, sel_i, topk, token, ids32, ids64, weights);
        if (tile_ids) {
#pragma unroll
            for (int k = 0; k < kMaxTopk; ++k)
                if (k < topk) tile_ids[k] = sel_i[k];
        }
    }
}

// In-tile ranks and counts for the dispatch (the work of its count/rank pass,
// done here while the ids are at hand). The block's tile holds tokens t0 ..
// t0 + n_tok - 1; their n = n_tok * K selected ids sit in tile_ids (LDS, flat
// order). One wave walks them in rounds of 64: lanes holding the same id are
// found by intersecting six bit-plane ballots, and a lane's rank is the number
// of such lanes below it plus its expert's count from earlier rounds, which
// lane e keeps in a register (read with a cross-lane shuffle; one ballot per
// expert adds each round's counts). ranks[p] <- rank of assignment p among
// the tile's earlier assignments to the same expert; counts_row[e] <- the
// tile's assignments to expert e.
__device__ __forceinline__ void rank_tile(const int* tile_ids, int n, int64_t p0, int experts, int32_t* ranks,
                                          int32_t* counts_row) {
    const int lane = threadIdx.x & 63;
    const uint64_t lanes_below = lane == 0 ? 0ull : (~0ull >> (kWave - lane));
    int run = 0;  // lane e < experts: the tile's assignments to expert e so far
    for (int base = 0; base < n; base += kWave) {
        const int i = base + lane;
        const bool valid = i < n;
        const int e = valid ? tile_ids[i] : 0;
        uint64_t same = __ballot(valid);
#pragma unroll
        for (int b = 0; b < 6; ++b) {
            const bool bit = (e >> b) & 1;
            const uint64_t plane = __ballot(valid && bit);
            same &= bit ? plane : ~plane;
        }
        const int prior = __shfl(run, e);
        if (valid) ranks[p0 + i] = prior + __popcll(same & lanes_below);
        for (int x = 0; x < experts; ++x) {
            const int c = __popcll(__ballot(valid && e == x));
            if (lane == x) run += c;
        }
    }
    if (lane < experts) counts_row[lane] = run;
}

typedef __bf16 rbf16x8_t __attribute__((ext_vector_type(8)));
typedef float rfloatx4_t __attribute__((ext_vector_type(4)));
constexpr int kRouterRowBytes = 128;  // 64 k of one row
constexpr uint32_t kRouterOob = 0x80000000u;  // a buffer offset past any router operand

__device__ __forceinline__ int router_key(int row) { return (row >> 1) & 7; }

template <int NT, int MT>
struct RouterShape {
    static constexpr int TB = kRouterTokens * MT;
    static constexpr int EB = 16 * NT;
    static constexpr int B_ROWS = 3 * EB;
    static constexpr int TILES = MT * NT;
    static constexpr int TPW = TILES >= 4 ? TILES / 4 : 1;  // tiles per wave
    static constexpr int G = TILES >= 4 ? 1 : 4 / TILES;     // waves per tile
    static constexpr uint32_t A_STAGE = TB * kRouterRowBytes;
    static constexpr uint32_t B_STAGE = B_ROWS * kRouterRowBytes;
    static constexpr int U = A_STAGE + B_STAGE <= 8 * 1024 ? 4 : (A_STAGE + B_STAGE <= 16 * 1024 ? 2 : 1);
    static constexpr int STAGES = 4 * U;                 // stages consumed per iteration, ring depth
    static constexpr uint32_t RING = STAGES * (A_STAGE + B_STAGE);
    static constexpr int LOADS = (TB + B_ROWS) / 8;  // 8 rows per load
    static constexpr int LPW = LOADS / 4;             // loads per wave and stage
    static constexpr int EBP = EB + 1;  // partials row stride (floats): lane-per-token reads hit distinct banks
    static constexpr uint32_t LDS = RING + G * TB * EBP * 4 + EB * 4;  // + bias
    static_assert(LOADS % 4 == 0, "stage loads split evenly over the waves");
    static_assert(TILES % 4 == 0 || 4 % TILES == 0, "tiles map onto the waves");
    static_assert(TPW == 1 || NT % TPW == 0, "a wave's tiles share a token tile");
    static_assert((STAGES - 2 * U) * LPW < 64, "vmcnt range");
    static_assert(LDS <= 160 * 1024, "LDS");
};

// SPLIT (at most kRouterSplitTokens tokens, E <= 16): block b takes token tile
// b / slices and the k-slice b % slices of `per` stages, loads the whole slice
// into its ring at once and writes the slice's partial logits to
// partials[tile][slice][TB][EB]; router_reduce_kernel adds the slices in
// slice order and selects. One token's routing at H=4096 otherwise streams its
// 204 KB of weight planes through one CU, latency-bound (11 us). (A last-block
// reduction inside this kernel needs a device-scope release per block, an L2
// write-back that costs more than the second launch.)
template <int NT, int MT, bool SPLIT = false>
__global__ __launch_bounds__(256) void router_ring_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ planes,
    const float* __restrict__ bias, int32_t* __restrict__ ids32, int64_t* __restrict__ ids64,
    float* __restrict__ weights, float* __restrict__ logits_out, int64_t tokens, int hidden,
    int experts, int topk, float* __restrict__ partials, int slices, int per, int32_t* __restrict__ ranks,
    int32_t* __restrict__ tile_counts) {
    using S = RouterShape<NT, MT>;
    constexpr int TB = S::TB, EB = S::EB, EBP = S::EBP, TPW = S::TPW, G = S::G, LPW = S::LPW;
    constexpr uint32_t A_STAGE = S::A_STAGE, B_STAGE = S::B_STAGE;
    constexpr int U = S::U, STAGES = S::STAGES;
    constexpr uint32_t B_BASE = STAGES * A_STAGE;
    __shared__ __attribute__((aligned(1024))) char lds[S::LDS];
    float* part = reinterpret_cast<float*>(lds + S::RING);  // [G][TB][EBP]
    float* sbias = part + G * TB * EBP;                        // [EB]

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int tile = SPLIT ? static_cast<int>(blockIdx.x) / slices : static_cast<int>(blockIdx.x);
    const int slice = SPLIT ? static_cast<int>(blockIdx.x) - tile * slices : 0;
    const int64_t t0 = static_cast<int64_t>(tile) * TB;
    const int64_t rows = min(static_cast<int64_t>(TB), tokens - t0);
    const int64_t row_bytes = static_cast<int64_t>(hidden) * 2;
    const __amdgpu_buffer_rsrc_t rsrc_x =
        make_rsrc(x + t0 * hidden, static_cast<uint32_t>(rows * row_bytes));
    const __amdgpu_buffer_rsrc_t rsrc_w =
        make_rsrc(planes, static_cast<uint32_t>(3 * static_cast<int64_t>(experts) * row_bytes));

    // This wave's loads: load l covers LDS rows 8*l .. 8*l+7 of the stage
    // (x rows first, then the plane rows), lane -> row l*8 + lane/8, chunk lane%8.
    uint32_t voff[LPW];
    uint32_t ldst[LPW];
    int kchunk[LPW];  // logical 16-byte chunk (8 k) this lane fetches
#pragma unroll
    for (int j = 0; j < LPW; ++j) {
        const int l = wave * LPW + j;
        const int r = l * 8 + (lane >> 3);
        const int chunk = (lane & 7) ^ router_key(r);
        kchunk[j] = chunk;
        if (l < TB / 8) {
            voff[j] = static_cast<uint32_t>(r * row_bytes + chunk * 16);
            ldst[j] = static_cast<uint32_t>(l * 1024);
        } else {
            const int br = r - TB;
            const int q = br / EB, e = br % EB;
            voff[j] = e < experts ? static_cast<uint32_t>((q * experts + e) * row_bytes + chunk * 16) : kRouterOob;
            ldst[j] = B_BASE + static_cast<uint32_t>((l - TB / 8) * 1024);
        }
    }
    // A last stage past `hidden` (hidden % 64 != 0) would run into the next
    // row: its lanes beyond hidden read zero through an out-of-range offset.
    const int k_stages = (hidden + 63) / 64;
    const int tail = hidden % 64;
    auto issue = [&](int stage, int slot) {
        const uint32_t koff = static_cast<uint32_t>(stage) * kRouterRowBytes;
        const bool partial = tail != 0 && stage == k_stages - 1;
#pragma unroll
        for (int j = 0; j < LPW; ++j) {
            const int l = wave * LPW + j;
            const uint32_t vo = partial && kchunk[j] * 8 >= tail ? kRouterOob : voff[j];
            if (l < TB / 8)
                dma16(rsrc_x, lds + ldst[j] + slot * A_STAGE, vo, koff);
            else
                dma16(rsrc_w, lds + ldst[j] + slot * B_STAGE, vo, koff);
        }
    };

    // Tiles of this wave: (token tile mt, expert tiles nt0 .. nt0+TPW-1), k share g.
    const int tile0 = (wave / G) * TPW;
    const int mt = tile0 / NT;
    const int nt0 = tile0 % NT;
    const int g = wave % G;
    const int m = lane & 15, kq = lane >> 4;
    const int ar = mt * 16 + m;
    uint32_t va[2], vb[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        va[h] = static_cast<uint32_t>(ar * kRouterRowBytes + (((4 * h + kq) ^ router_key(ar)) << 4));
        const int br = nt0 * 16 + m;  // plane 0 row; planes 1, 2 add EB rows (same key: EB % 16 == 0)
        vb[h] = B_BASE + static_cast<uint32_t>(br * kRouterRowBytes + (((4 * h + kq) ^ router_key(br)) << 4));
    }
    rfloatx4_t acc[TPW];
#pragma unroll
    for (int t = 0; t < TPW; ++t) acc[t] = rfloatx4_t{0.f, 0.f, 0.f, 0.f};

    if constexpr (SPLIT) {
        // The slice's stages (per <= STAGES, the launcher's condition) go to
        // slots 0 .. n-1 at once; one wait, one barrier.
        const int s_begin = slice * per;
        const int n = min(per, k_stages - s_begin);
        for (int s = 0; s < n; ++s) issue(s_begin + s, s);
        wait_vm_lgkm<0>();
        ring_barrier();
        for (int s = 0; s < n; ++s) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                if ((2 * s + h) % G != g) continue;
                const char* abase = lds + va[h] + s * A_STAGE;
                const char* bbase = lds + vb[h] + s * B_STAGE;
                const rbf16x8_t a = *reinterpret_cast<const rbf16x8_t*>(abase);
#pragma unroll
                for (int t = 0; t < TPW; ++t) {
#pragma unroll
                    for (int q = 2; q >= 0; --q) {
                        const rbf16x8_t b = *reinterpret_cast<const rbf16x8_t*>(
                            bbase + (q * EB + t * 16) * kRouterRowBytes);
                        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[t], 0, 0, 0);
                    }
                }
            }
        }
    } else {
    // Stage s lives in slot s % STAGES; stages past the last are loaded as the
    // last one again (and not computed), so every iteration issues the same loads.
#pragma unroll
    for (int s = 0; s < STAGES - U; ++s) issue(min(s, k_stages - 1), s);
    int group = 0;  // (s0 / U) % 4: slots of this iteration's stages start at group * U
    for (int s0 = 0; s0 < k_stages; s0 += U) {
        // Stages s0 .. s0+U-1 have landed once only stages s0+U .. s0+STAGES-U-1 are
        // younger; every read of the previous iteration's stages (whose slots the
        // next loads reuse) has returned.
        wait_vm_lgkm<(STAGES - 2 * U) * LPW>();
        ring_barrier();
        const int refill = (group == 0 ? 3 : group - 1) * U;  // the previous iteration's slots
#pragma unroll
        for (int u = 0; u < U; ++u) issue(min(s0 + STAGES - U + u, k_stages - 1), refill + u);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int s = s0 + u;
            if (s >= k_stages) break;
            const int slot = group * U + u;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                if ((2 * s + h) % G != g) continue;
                const char* abase = lds + va[h] + slot * A_STAGE;
                const char* bbase = lds + vb[h] + slot * B_STAGE;
                const rbf16x8_t a = *reinterpret_cast<const rbf16x8_t*>(abase);
#pragma unroll
                for (int t = 0; t < TPW; ++t) {
#pragma unroll
                    for (int q = 2; q >= 0; --q) {
                        const rbf16x8_t b = *reinterpret_cast<const rbf16x8_t*>(
                            bbase + (q * EB + t * 16) * kRouterRowBytes);
                        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[t], 0, 0, 0);
                    }
                }
            }
        }
        group = group == 3 ? 0 : group + 1;
    }
    wait_vm_lgkm<0>();
    }
    if (!SPLIT && threadIdx.x < experts) sbias[threadIdx.x] = bias[threadIdx.x];
    // 16x16 result: lane l holds tokens 4*(l/16) + r of token tile mt, expert column l%16.
#pragma unroll
    for (int t = 0; t < TPW; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r)
            part[(g * TB + mt * 16 + 4 * kq + r) * EBP + (nt0 + t) * 16 + m] = acc[t][r];
    __syncthreads();
    if constexpr (SPLIT) {
        // The slice's partial logits, its waves' partials added in wave order.
        for (int i = threadIdx.x; i < TB * EB; i += 256) {
            const int tl = i / EB, e = i % EB;
            float logit = part[tl * EBP + e];
#pragma unroll
            for (int gg = 1; gg < G; ++gg) logit = logit + part[(gg * TB + tl) * EBP + e];
            partials[((static_cast<int64_t>(tile) * slices + slice) * TB + tl) * EB + e] = logit;
        }
        return;
    }

    constexpr int EPL = EB / 8;
    static_assert(EPL >= 1 && TB <= 32, "eight lanes per token, at most 32 tokens per block");
    __shared__ int tile_ids[TB * kMaxTopk];
    const int tl = wave * 8 + (lane >> 3);
    const int sub = lane & 7;
    const int64_t token = t0 + tl;
    if (tl < TB && token < tokens) {  // uniform across each group of eight lanes
        float v[EPL];
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            const int e = sub * EPL + j;
            v[j] = -INFINITY;
            if (e < experts) {
                float logit = part[tl * EBP + e];
#pragma unroll
                for (int gg = 1; gg < G; ++gg) logit = logit + part[(gg * TB + tl) * EBP + e];
                if (logits_out) logits_out[token * experts + e] = logit;
                v[j] = logit + sbias[e];
            }
        }
        select_eight_lanes<EPL>(v, sub, topk, token, ids32, ids64, weights, ranks ? tile_ids + tl * topk : nullptr);
    }
    if (ranks) {
        __syncthreads();
        if (threadIdx.x < kWave)
            rank_tile(tile_ids, static_cast<int>(rows) * topk, t0 * topk, experts, ranks,
                      tile_counts + static_cast<int64_t>(tile) * experts);
    }
}

// Fused router for E <= 16 on loads straight into VGPRs (no LDS ring).
//
// Operands reach VGPRs through buffer loads, already in MFMA fragment layout
// (lane l supplies row l%16 and k 8*(l/16) .. +7 of a 16 x 32 operand). Each
// 16x16x32 product covers 8 tokens and a 64-k step: operand row 2t + h is
// token t's k half h (k0 + 32h ..), so the eight lanes of a token read one
// whole 128-byte line and a token load reads 8 full lines; a layout with one
// token per row reads 64 bytes of 16 lines (H=4096, 4096 tokens: 9.1 against
// 7.7 us). The weight operand's column 2r + h holds plane row r (r = q*E
// + e: plane q, expert e) at k half h, so output (2t + h, 2r + h) is token t's
// k-half-h product with plane row r (the other outputs mix the halves and are
// not used). The planes are read from a copy in this fragment order
// (router_fragment_kernel): per 64-k step, F = ceil(6E/16) fragments of 1 KiB,
// lane l's 16 bytes at byte 16*l, rows >= 3E zero, so a weight load reads 1
// KiB of contiguous, fully used lines. Each (token group, fragment) pair has
// its own accumulator; per token and plane row the block sums the halves and
// the waves in order, and the logit is (lo + mid) + hi.
//
// A block owns 16 tokens (two groups of 8); its two waves split the 64-k
// steps into two contiguous ranges of at most PER (at H=4096, 4096 tokens:
// 7.7, 7.3 and 7.3 us with eight, four and two waves; fewer partials to add,
// longer load streams per wave; 8.5 us with sixteen). The range is unrolled at
// compile time with the loads D steps ahead of the multiplies, so the code is
// straight-line and the compiler's wait before each multiply counts only the
// loads issued after that step's (a runtime loop carried the in-flight
// fragments through register copies that waited for every load). Lanes of
// steps past the wave's range and of k past `hidden` read zero through an
// out-of-range offset, with no memory traffic.
//
// Why no LDS ring here: the ring kernel moved every operand byte through
// direct-to-LDS loads, 8 KiB per 64-k stage for 16 tokens (x, the planes and
// the zero rows of unused expert slots), and at H=4096, 4096 tokens its time
// did not move when either the x or the plane loads were replaced by
// out-of-range (zero, no traffic) ones: 12.3 us.
constexpr int kDirectWaves = 2;
constexpr int kDirectMaxPer = 64;   // 64-k steps per wave: hidden <= 2 * 64 * 64 = 8192
constexpr int kDirectMaxExperts = 16;

__host__ __device__ constexpr int router_fragments(int experts) { return (6 * experts + 15) / 16; }

// Plane fragments from the row-major planes ([3][E][H] bf16): one thread per
// 16-byte lane chunk (64-k step s, fragment f, lane l = (column n, k chunk kq)).
__global__ __launch_bounds__(256) void router_fragment_kernel(const uint16_t* __restrict__ planes,
                                                              uint16_t* __restrict__ frags, int experts,
                                                              int hidden, int64_t chunks) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= chunks) return;
    const int F = router_fragments(experts);
    const int lane = static_cast<int>(i & 63);
    const int64_t sf = i >> 6;
    const int f = static_cast<int>(sf % F);
    const int64_t s = sf / F;
    const int c = f * 16 + (lane & 15);
    const int r = c >> 1, h = c & 1;
    const int64_t k = s * 64 + h * 32 + (lane >> 4) * 8;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (r < 3 * experts && k < hidden) v = *reinterpret_cast<const uint4*>(planes + r * static_cast<int64_t>(hidden) + k);
    *reinterpret_cast<uint4*>(frags + i * 8) = v;
}

typedef uint32_t ru32x4_t __attribute__((ext_vector_type(4)));

// Loads in flight ahead of the multiplies: about 48 (vmcnt holds 63), and
// fewer steps when the fragments are many (VGPRs).
template <int PER, int F>
constexpr int direct_depth() {
    constexpr int d = F > 3 ? 4 : 48 / (2 + F);
    return d < PER ? d : PER;
}

template <int PER, int F>
__global__ __launch_bounds__(kDirectWaves * 64) void router_direct_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ frags, const float* __restrict__ bias,
    int32_t* __restrict__ ids32, int64_t* __restrict__ ids64, float* __restrict__ weights,
    float* __restrict__ logits_out, int64_t tokens, int hidden, int experts, int topk, int32_t* __restrict__ ranks,
    int32_t* __restrict__ tile_counts) {
    constexpr int TB = kRouterTokens, PR = 8 * F, PRP = 2 * PR + 1;
    constexpr int D = direct_depth<PER, F>();
    static_assert(kDirectWaves * 8 >= TB, "the selection takes eight lanes per token");
    __shared__ float part[kDirectWaves][TB][PRP];  // [wave][token][half * PR + plane row]
    __shared__ float sbias[kDirectMaxExperts];
    __shared__ int tile_ids[TB * kMaxTopk];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t t0 = static_cast<int64_t>(blockIdx.x) * TB;
    const int64_t rows = min(static_cast<int64_t>(TB), tokens - t0);
    const uint32_t row_bytes = static_cast<uint32_t>(hidden) * 2;
    const int steps = (hidden + 63) / 64;
    const __amdgpu_buffer_rsrc_t rsrc_x = make_rsrc(x + t0 * hidden, static_cast<uint32_t>(rows) * row_bytes);
    const __amdgpu_buffer_rsrc_t rsrc_f = make_rsrc(frags, static_cast<uint32_t>(steps) * F * 1024u);
    const int per = (steps + kDirectWaves - 1) / kDirectWaves;  // <= PER (the launcher's choice)
    const int s_begin = min(steps, wave * per);
    const int s_end = min(steps, s_begin + per);
    const int m = lane & 15, kq = lane >> 4, h = m & 1;
    const int k_lane = h * 32 + kq * 8;  // this lane's k inside a step
    const uint32_t x_off = static_cast<uint32_t>(m >> 1) * row_bytes + k_lane * 2;

    struct Frag {
        ru32x4_t a[2], b[F];
    };
    auto load = [&](int s, Frag& fr) {
        const bool in = s < s_end;
        const bool k_in = in && s * 64 + k_lane < hidden;
        const uint32_t k_bytes = static_cast<uint32_t>(s) * 128;
#pragma unroll
        for (int g = 0; g < 2; ++g)
            fr.a[g] = __builtin_amdgcn_raw_buffer_load_b128(
                rsrc_x, k_in ? x_off + g * 8 * row_bytes + k_bytes : kRouterOob, 0, 0);
#pragma unroll
        for (int f = 0; f < F; ++f)
            fr.b[f] = __builtin_amdgcn_raw_buffer_load_b128(
                rsrc_f, in ? static_cast<uint32_t>((s * F + f) * 64 + lane) * 16 : kRouterOob, 0, 0);
    };
    rfloatx4_t acc[2][F];
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
        for (int f = 0; f < F; ++f) acc[g][f] = rfloatx4_t{0.f, 0.f, 0.f, 0.f};
    Frag fr[D];
    static_for<D>([&](auto u_c) { load(s_begin + decltype(u_c)::value, fr[decltype(u_c)::value]); });
    static_for<PER>([&](auto i_c) {
        constexpr int i = decltype(i_c)::value;
#pragma unroll
        for (int g = 0; g < 2; ++g)
#pragma unroll
            for (int f = 0; f < F; ++f)
                acc[g][f] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(rbf16x8_t, fr[i % D].a[g]),
                                                                    __builtin_bit_cast(rbf16x8_t, fr[i % D].b[f]),
                                                                    acc[g][f], 0, 0, 0);
        if constexpr (i + D < PER) load(s_begin + i + D, fr[i % D]);
        __builtin_amdgcn_sched_barrier(0);
    });
    // 16x16 results: lane l holds operand rows 4*(l/16) + j and column c = 16f
    // + l%16; the useful ones have the row's half equal to the column's (j % 2
    // == c % 2): token 8g + 2*(l/16) + j/2, plane row c/2, half c%2.
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
        for (int f = 0; f < F; ++f)
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) {
                const int j = 2 * jj + h;
                part[wave][8 * g + 2 * kq + jj][h * PR + 8 * f + (m >> 1)] = acc[g][f][j];
            }
    if (threadIdx.x < experts) sbias[threadIdx.x] = bias[threadIdx.x];
    __syncthreads();
    constexpr int EPL = kDirectMaxExperts / 8;
    const int tl = wave * 8 + (lane >> 3);
    const int sub = lane & 7;
    const int64_t token = t0 + tl;
    if (tl < TB && token < tokens) {  // uniform across each group of eight lanes
        float v[EPL];
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            const int e = sub * EPL + j;
            v[j] = -INFINITY;
            if (e < experts) {
                float q[3];
#pragma unroll
                for (int p = 0; p < 3; ++p) {
                    const int pr = p * experts + e;
                    float sum = part[0][tl][pr] + part[0][tl][PR + pr];
#pragma unroll
                    for (int w = 1; w < kDirectWaves; ++w) sum = sum + (part[w][tl][pr] + part[w][tl][PR + pr]);
                    q[p] = sum;
                }
                const float logit = (q[2] + q[1]) + q[0];
                if (logits_out) logits_out[token * experts + e] = logit;
                v[j] = logit + sbias[e];
            }
        }
        select_eight_lanes<EPL>(v, sub, topk, token, ids32, ids64, weights, ranks ? tile_ids + tl * topk : nullptr);
    }
    if (ranks) {
        __syncthreads();
        if (threadIdx.x < kWave)
            rank_tile(tile_ids, static_cast<int>(rows) * topk, t0 * topk, experts, ranks,
                      tile_counts + static_cast<int64_t>(blockIdx.x) * experts);
    }
}

// Fused router for 16 < E <= 64 on the same VGPR loads and fragment-order
// planes as router_direct_kernel, organised for many experts: a block owns
// 32 tokens (four groups of 8, two tokens per operand row as above) and its
// four waves split the weight fragments (wave w: fragments w*FW .. w*FW+FW-1
// of F = ceil(6E/16)), each over the whole k range, so no wave partials need
// adding; every wave loads the four token fragments itself (they come from
// L1/L2 after the first). Loads run up to about 40 ahead of the multiplies.
// At E = 64, H = 2048, 8192 tokens: 23-24 us, against 25-37 us for the LDS
// ring kernel. There the x stream, the weight stream and the MFMAs add up
// rather than overlap (timing variants with either load stream out of range:
// 15 us each; MFMAs alone 8.4 us), and load depths of 2 to 6 steps, or the
// loads interleaved with the multiplies, measured the same.
constexpr int kWideTokens = 32;
constexpr int kWideWaves = 4;
constexpr int kWideMaxPer = 64;  // 64-k steps: hidden <= 4096

template <int PER, int FW>
constexpr int wide_depth() {
    constexpr int d = 40 / (4 + FW);
    return d < PER ? d : PER;
}

template <int PER, int FW>
__global__ __launch_bounds__(kWideWaves * 64) void router_wide_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ frags, const float* __restrict__ bias,
    int32_t* __restrict__ ids32, int64_t* __restrict__ ids64, float* __restrict__ weights,
    float* __restrict__ logits_out, int64_t tokens, int hidden, int experts, int topk, int32_t* __restrict__ ranks,
    int32_t* __restrict__ tile_counts) {
    constexpr int TB = kWideTokens, G = TB / 8, PR = 8 * FW * kWideWaves, PRP = 2 * PR + 1;
    constexpr int D = wide_depth<PER, FW>();
    static_assert(kWideWaves * 8 == TB, "the selection takes eight lanes per token");
    __shared__ float part[TB][PRP];  // [token][half * PR + plane row]
    __shared__ float sbias[kMaxExperts];
    __shared__ int tile_ids[TB * kMaxTopk];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t t0 = static_cast<int64_t>(blockIdx.x) * TB;
    const int64_t rows = min(static_cast<int64_t>(TB), tokens - t0);
    const uint32_t row_bytes = static_cast<uint32_t>(hidden) * 2;
    const int steps = (hidden + 63) / 64;  // <= PER (the launcher's choice)
    const int F = router_fragments(experts);
    const __amdgpu_buffer_rsrc_t rsrc_x = make_rsrc(x + t0 * hidden, static_cast<uint32_t>(rows) * row_bytes);
    const __amdgpu_buffer_rsrc_t rsrc_f = make_rsrc(frags, static_cast<uint32_t>(steps) * F * 1024u);
    const int m = lane & 15, kq = lane >> 4, h = m & 1;
    const int k_lane = h * 32 + kq * 8;
    const uint32_t x_off = static_cast<uint32_t>(m >> 1) * row_bytes + k_lane * 2;
    const int f0 = wave * FW;  // this wave's first fragment

    struct Frag {
        ru32x4_t a[G], b[FW];
    };
    auto load = [&](int s, Frag& fr) {
        const bool in = s < steps;
        const bool k_in = in && s * 64 + k_lane < hidden;
        const uint32_t k_bytes = static_cast<uint32_t>(s) * 128;
#pragma unroll
        for (int g = 0; g < G; ++g)
            fr.a[g] = __builtin_amdgcn_raw_buffer_load_b128(
                rsrc_x, k_in ? x_off + g * 8 * row_bytes + k_bytes : kRouterOob, 0, 0);
#pragma unroll
        for (int f = 0; f < FW; ++f)
            fr.b[f] = __builtin_amdgcn_raw_buffer_load_b128(
                rsrc_f, in && f0 + f < F ? static_cast<uint32_t>((s * F + f0 + f) * 64 + lane) * 16 : kRouterOob,
                0, 0);
    };
    rfloatx4_t acc[G][FW];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int f = 0; f < FW; ++f) acc[g][f] = rfloatx4_t{0.f, 0.f, 0.f, 0.f};
    Frag fr[D];
    static_for<D>([&](auto u_c) { load(decltype(u_c)::value, fr[decltype(u_c)::value]); });
    static_for<PER>([&](auto i_c) {
        constexpr int i = decltype(i_c)::value;
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int f = 0; f < FW; ++f)
                acc[g][f] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(rbf16x8_t, fr[i % D].a[g]),
                                                                    __builtin_bit_cast(rbf16x8_t, fr[i % D].b[f]),
                                                                    acc[g][f], 0, 0, 0);
        if constexpr (i + D < PER) load(i + D, fr[i % D]);
        __builtin_amdgcn_sched_barrier(0);
    });
    // As in router_direct_kernel: lane l holds rows 4*(l/16) + j and column
    // 16f + l%16 of fragment f; the useful outputs have equal halves.
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int f = 0; f < FW; ++f)
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) {
                const int j = 2 * jj + h;
                part[8 * g + 2 * kq + jj][h * PR + 8 * (f0 + f) + (m >> 1)] = acc[g][f][j];
            }
    if (threadIdx.x < experts) sbias[threadIdx.x] = bias[threadIdx.x];
    __syncthreads();
    constexpr int EPL = kMaxExperts / 8;
    const int tl = wave * 8 + (lane >> 3);
    const int sub = lane & 7;
    const int64_t token = t0 + tl;
    if (token < tokens) {  // uniform across each group of eight lanes
        float v[EPL];
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            const int e = sub * EPL + j;
            v[j] = -INFINITY;
            if (e < experts) {
                float q[3];
#pragma unroll
                for (int p = 0; p < 3; ++p) {
                    const int pr = p * experts + e;
                    q[p] = part[tl][pr] + part[tl][PR + pr];
                }
                const float logit = (q[2] + q[1]) + q[0];
                if (logits_out) logits_out[token * experts + e] = logit;
                v[j] = logit + sbias[e];
            }
        }
        select_eight_lanes<EPL>(v, sub, topk, token, ids32, ids64, weights, ranks ? tile_ids + tl * topk : nullptr);
    }
    if (ranks) {
        __syncthreads();
        if (threadIdx.x < kWave)
            rank_tile(tile_ids, static_cast<int>(rows) * topk, t0 * topk, experts, ranks,
                      tile_counts + static_cast<int64_t>(blockIdx.x) * experts);
    }
}

// Sum of a token tile's k-slices in slice order, the bias, and the same
// selection as router_ring_kernel (16 tokens x 16 expert slots, E <= 16).
__global__ __launch_bounds__(256) void router_reduce_kernel(
    const float* __restrict__ partials, const float* __restrict__ bias, int32_t* __restrict__ ids32,
    int64_t* __restrict__ ids64, float* __restrict__ weights, float* __restrict__ logits_out,
    int64_t tokens, int experts, int topk, int slices, int32_t* __restrict__ ranks,
    int32_t* __restrict__ tile_counts) {
    constexpr int TB = kRouterTokens, EB = 16, EPL = EB / 8;
    static_assert(TB * EB == 256, "one thread per (token, expert)");
    __shared__ float lg[TB][EB + 1];
    __shared__ int tile_ids[TB * kMaxTopk];
    const int tile = blockIdx.x;
    {
        const int tl = threadIdx.x / EB, e = threadIdx.x % EB;
        const float* p = partials + (static_cast<int64_t>(tile) * slices * TB + tl) * EB + e;
        float logit = p[0];
        for (int s = 1; s < slices; ++s) logit = logit + p[static_cast<int64_t>(s) * TB * EB];
        lg[tl][e] = logit;
    }
    __syncthreads();
    const int lane = threadIdx.x & 63;
    const int tl = (threadIdx.x >> 6) * 8 + (lane >> 3);
    const int sub = lane & 7;
    const int64_t token = static_cast<int64_t>(tile) * TB + tl;
    if (tl < TB && token < tokens) {  // 32 lane groups, 16 tokens; uniform across each group of eight lanes
        float v[EPL];
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            const int e = sub * EPL + j;
            v[j] = -INFINITY;
            if (e < experts) {
                const float logit = lg[tl][e];
                if (logits_out) logits_out[token * experts + e] = logit;
                v[j] = logit + bias[e];
            }
        }
        select_eight_lanes<EPL>(v, sub, topk, token, ids32, ids64, weights, ranks ? tile_ids + tl * topk : nullptr);
    }
    if (ranks) {
        __syncthreads();
        const int64_t t0 = static_cast<int64_t>(tile) * TB;
        const int n_tok = static_cast<int>(min(static_cast<int64_t>(TB), tokens - t0));
        if (threadIdx.x < kWave)
            rank_tile(tile_ids, n_tok * topk, t0 * topk, experts, ranks,
                      tile_counts + static_cast<int64_t>(tile) * experts);
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

// The three bf16 planes, then (256-byte aligned) the split path's partial
// logits [tiles][slices][16 tokens][16 experts] fp32, then the planes in
// fragment order ([ceil(H/64)][F][64 lanes][16 bytes]).
static int64_t router_partials_offset(int64_t experts, int64_t hidden) {
    return (3 * experts * hidden * 2 + 255) & ~static_cast<int64_t>(255);
}

static int64_t router_fragments_offset(int64_t experts, int64_t hidden) {
    return router_partials_offset(experts, hidden) + kRouterPartialBytes;
}

static int64_t router_fragment_chunks(int64_t experts, int64_t hidden) {
    return (hidden + 63) / 64 * router_fragments(static_cast<int>(experts)) * 64;
}

int64_t router_scratch_bytes(int64_t experts, int64_t hidden) {
    return router_fragments_offset(experts, hidden) + router_fragment_chunks(experts, hidden) * 16;
}

int launch_router_split(const float* router_w, uint16_t* planes, int experts, int hidden, hipStream_t stream) {
    const int64_t n = static_cast<int64_t>(experts) * hidden;
    hipLaunchKernelGGL(router_split_kernel, dim3(static_cast<unsigned>((n / 8 + 255) / 256)), dim3(256), 0, stream,
                       router_w, planes, n);
    const int rc = check_launch("router_split_kernel");
    const int64_t chunks = router_fragment_chunks(experts, hidden);
    if (rc != MOE_OK || chunks == 0) return rc;
    uint16_t* frags = reinterpret_cast<uint16_t*>(reinterpret_cast<char*>(planes) +
                                                  router_fragments_offset(experts, hidden));
    hipLaunchKernelGGL(router_fragment_kernel, dim3(static_cast<unsigned>((chunks + 255) / 256)), dim3(256), 0,
                       stream, planes, frags, experts, hidden, chunks);
    return check_launch("router_fragment_kernel");
}

// Tokens per routing block: the tile whose in-tile ranks and counts the
// ranked router writes (16 for E <= 16, 32 above), or 0 when the tile table
// (tiles x E entries, which every pack block sums) would exceed
// kRankedPrefixMax or there are no tokens.
int64_t router_rank_tile(int64_t tokens, int64_t experts) {
    const int64_t tile = experts <= 16 ? kRouterTokens : 2 * kRouterTokens;
    if (tokens <= 0 || (tokens + tile - 1) / tile * experts > kRankedPrefixMax) return 0;
    return tile;
}

int launch_router_fused(const uint16_t* x, const float* router_w, const float* bias,
                        int32_t* ids32, int64_t* ids64, float* weights, float* logits_out,
                        uint16_t* planes, int64_t tokens, int hidden, int experts, int topk,
                        int32_t* ranks, int32_t* tile_counts, hipStream_t stream) {
    if (tokens == 0) return MOE_OK;
    if (router_w != nullptr) {  // else planes already holds the split
        const int rc = launch_router_split(router_w, planes, experts, hidden, stream);
        if (rc != MOE_OK) return rc;
    }
    // Buffer offsets are 32-bit: 3*E*H*2 bytes of planes and 32 rows of x must fit.
    MOE_REQUIRE(hidden <= (1 << 20), MOE_ERR_UNSUPPORTED, "fused router supports hidden <= 1048576 (got %d)",
                hidden);
    const int k_stages = (hidden + 63) / 64;
    constexpr int kSplitMaxPer = RouterShape<1, 1>::STAGES;  // a slice fits the ring at once
    if (experts <= 16 && tokens <= kRouterSplitTokens && k_stages >= 16 &&
        k_stages <= kRouterSplitSlices * kSplitMaxPer) {
        // Split k: slices of about 8 stages (64 KiB of loads per workgroup),
        // none empty.
        const int per = (k_stages + min(kRouterSplitSlices, (k_stages + 7) / 8) - 1) /
                        min(kRouterSplitSlices, (k_stages + 7) / 8);
        const int slices = (k_stages + per - 1) / per;
        const int tiles = static_cast<int>((tokens + kRouterTokens - 1) / kRouterTokens);
        float* partials = reinterpret_cast<float*>(reinterpret_cast<char*>(planes) +
                                                   router_partials_offset(experts, hidden));
        hipLaunchKernelGGL((router_ring_kernel<1, 1, true>), dim3(static_cast<unsigned>(tiles * slices)),
                           dim3(256), 0, stream, x, planes, bias, ids32, ids64, weights, logits_out, tokens,
                           hidden, experts, topk, partials, slices, per, nullptr, nullptr);
        const int rs = check_launch("router_ring_kernel");
        if (rs != MOE_OK) return rs;
        hipLaunchKernelGGL(router_reduce_kernel, dim3(static_cast<unsigned>(tiles)), dim3(256), 0, stream,
                           partials, bias, ids32, ids64, weights, logits_out, tokens, experts, topk, slices,
                           ranks, tile_counts);
        return check_launch("router_reduce_kernel");
    }
#define MOE_ROUTER_CASE(NTV, MTV)                                                                      \
    hipLaunchKernelGGL((router_ring_kernel<NTV, MTV>),                                                 \
                       dim3(static_cast<unsigned>((tokens + kRouterTokens * MTV - 1) / (kRouterTokens * MTV))), \
                       dim3(256), 0, stream, x, planes, bias, ids32, ids64, weights, logits_out, tokens, \
                       hidden, experts, topk, nullptr, 1, 0, ranks, tile_counts)
    // E <= 16 and hidden <= 8192: the VGPR-load kernel, 16 tokens per block.
    // Otherwise the LDS ring: one token tile per block for E <= 16 (the four
    // waves split k), two above (the waves split the 16x16 output tiles).
    const int per = ((hidden + 63) / 64 + kDirectWaves - 1) / kDirectWaves;
    if (experts <= kDirectMaxExperts && per <= kDirectMaxPer) {
        const uint16_t* frags = reinterpret_cast<const uint16_t*>(reinterpret_cast<const char*>(planes) +
                                                                  router_fragments_offset(experts, hidden));
        const dim3 grid(static_cast<unsigned>((tokens + kRouterTokens - 1) / kRouterTokens));
        const int f = router_fragments(experts);
#define MOE_DIRECT_CASE(P, FV)                                                                              \
    hipLaunchKernelGGL((router_direct_kernel<P, FV>), grid, dim3(kDirectWaves * 64), 0, stream, x, frags, \
                       bias, ids32, ids64, weights, logits_out, tokens, hidden, experts, topk, ranks, tile_counts)
#define MOE_DIRECT_PER(FV)                    \
    if (per <= 2) MOE_DIRECT_CASE(2, FV);       \
    else if (per <= 4) MOE_DIRECT_CASE(4, FV);  \
    else if (per <= 8) MOE_DIRECT_CASE(8, FV);  \
    else if (per <= 16) MOE_DIRECT_CASE(16, FV);  \
    else if (per <= 32) MOE_DIRECT_CASE(32, FV);  \
    else MOE_DIRECT_CASE(64, FV);
        switch (f) {
            case 1: MOE_DIRECT_PER(1) break;
            case 2: MOE_DIRECT_PER(2) break;
            case 3: MOE_DIRECT_PER(3) break;
            case 4: MOE_DIRECT_PER(4) break;
            case 5: MOE_DIRECT_PER(5) break;
            default: MOE_DIRECT_PER(6) break;
        }
#undef MOE_DIRECT_PER
#undef MOE_DIRECT_CASE
        return check_launch("router_direct_kernel");
    }
    const int steps = (hidden + 63) / 64;
    if (experts > kDirectMaxExperts && steps <= kWideMaxPer) {
        const uint16_t* frags = reinterpret_cast<const uint16_t*>(reinterpret_cast<const char*>(planes) +
                                                                  router_fragments_offset(experts, hidden));
        const dim3 grid(static_cast<unsigned>((tokens + kWideTokens - 1) / kWideTokens));
        const int fw = (router_fragments(experts) + kWideWaves - 1) / kWideWaves;
#define MOE_WIDE_CASE(P, FV)                                                                              \
    hipLaunchKernelGGL((router_wide_kernel<P, FV>), grid, dim3(kWideWaves * 64), 0, stream, x, frags, bias, \
                       ids32, ids64, weights, logits_out, tokens, hidden, experts, topk, ranks, tile_counts)
#define MOE_WIDE_PER(FV)                     \
    if (steps <= 8) MOE_WIDE_CASE(8, FV);      \
    else if (steps <= 16) MOE_WIDE_CASE(16, FV); \
    else if (steps <= 32) MOE_WIDE_CASE(32, FV); \
    else MOE_WIDE_CASE(64, FV);
        switch (fw) {
            case 2: MOE_WIDE_PER(2) break;
            case 3: MOE_WIDE_PER(3) break;
            case 4: MOE_WIDE_PER(4) break;
            case 5: MOE_WIDE_PER(5) break;
            default: MOE_WIDE_PER(6) break;
        }
#undef MOE_WIDE_PER
#undef MOE_WIDE_CASE
        return check_launch("router_wide_kernel");
    }
    if (experts <= 16) {
        MOE_ROUTER_CASE(1, 1);
    } else if (experts <= 32) {
        MOE_ROUTER_CASE(2, 2);
    } else if (experts <= 64) {
        MOE_ROUTER_CASE(4, 2);
    } else {
        return fail(MOE_ERR_UNSUPPORTED, "experts=%d exceeds 64", experts);
    }
#undef MOE_ROUTER_CASE
    return check_launch("router_ring_kernel");
}

}  // namespace moe
