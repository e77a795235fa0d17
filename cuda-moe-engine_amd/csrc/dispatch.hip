// Token transport kernels for gfx950: deterministic dispatch (per-chunk
// histogram and stable ranks, then one pack kernel that rebuilds the expert
// prefix from the small per-chunk table, writes destinations, copies rows and
// zeroes padding; for at most 1024 assignments the pack kernel ranks them
// itself) and the atomic-free weighted combine. Plus the standalone SwiGLU
// kept for API parity.
//
// Reference behaviour: src/moe_dispatch/csrc/dispatch.cu:13-93 (count, scan,
// pack, combine), :194-275 (aligned layout and padding), :277-323 (SwiGLU).
// The reference assigns slots with global atomicAdd, so its slot order varies
// from run to run; here slots follow the flat assignment order, computed with
// wavefront ballots and per-chunk counts, and every output is deterministic.
#include <algorithm>

#include "moe_common.h"

namespace moe {

// Assignments are grouped in chunks of chunk_tokens consecutive tokens (16
// times a power of two, chosen on the host so that n_chunks * E <=
// prefix_max(E)). Every pack block reads the whole table, so it stays small
// for few experts; for many, a small table leaves the counting kernel few,
// long blocks (8192 tokens, E=64, K=6: 16 blocks of 3072 assignments, dispatch
// 42.5 us; with 4096 entries 64 blocks of 768, 40.0 us; at 4096 tokens, E=8,
// K=2, 4096 entries measured 13.7 -> 13.9 us).
constexpr int kPrefixMax = 4096;
__host__ __device__ constexpr int prefix_max(int64_t experts) { return experts > 16 ? kPrefixMax : 1024; }
constexpr int kRankThreads = 1024;
constexpr int kRankWaves = kRankThreads / kWave;

// ---------------------------------------------------------------------------
// Stage 1: per-chunk histogram and in-chunk stable rank (one block per chunk,
// rounds of 1024 assignments). slots[p] <- rank of p among the chunk's earlier
// assignments to the same expert (-1 for an out-of-range id);
// chunk_counts[c][e] <- assignments of chunk c to expert e.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kRankThreads) void count_rank_kernel(
    const int32_t* __restrict__ ids, int32_t* __restrict__ slots,
    int32_t* __restrict__ chunk_counts, int64_t n_assign, int experts, int64_t chunk_assign) {
    __shared__ int running[kMaxExperts];
    __shared__ int wave_counts[kRankWaves][kMaxExperts];
    const int tid = threadIdx.x;
    const int wave = tid / kWave;
    const int lane = tid % kWave;
    const uint64_t lanes_below = (lane == 0) ? 0ull : (~0ull >> (kWave - lane));
    const int64_t p0 = static_cast<int64_t>(blockIdx.x) * chunk_assign;
    const int64_t p1 = min(p0 + chunk_assign, n_assign);
    if (tid < kMaxExperts) running[tid] = 0;
    for (int64_t base = p0; base < p1; base += kRankThreads) {
        for (int i = tid; i < kRankWaves * kMaxExperts; i += kRankThreads) (&wave_counts[0][0])[i] = 0;
        __syncthreads();
        const int64_t p = base + tid;
        const bool valid = p < p1;
        const int e = valid ? ids[p] : -1;
        const bool in_range = valid && e >= 0 && e < experts;
        // Lanes holding the same expert id: intersect 6 bit-plane ballots.
        uint64_t same = __ballot(in_range);
#pragma unroll
        for (int b = 0; b < 6; ++b) {
            const bool bit = (e >> b) & 1;
            const uint64_t plane = __ballot(in_range && bit);
            same &= bit ? plane : ~plane;
        }
        const int rank = __popcll(same & lanes_below);
        if (in_range && rank == 0) wave_counts[wave][e] = __popcll(same);
        __syncthreads();
        if (valid) {
            int s = -1;
            if (in_range) {
                s = running[e] + rank;
                for (int w = 0; w < wave; ++w) s += wave_counts[w][e];
            }
            slots[p] = s;
        }
        __syncthreads();
        if (tid < experts) {
            int add = 0;
            for (int w = 0; w < kRankWaves; ++w) add += wave_counts[w][tid];
            running[tid] += add;
        }
        __syncthreads();
    }
    if (tid < experts) chunk_counts[static_cast<int64_t>(blockIdx.x) * experts + tid] = running[tid];
}

// ---------------------------------------------------------------------------
// Stage 2: prefix + pack + padding. A block owns `pack_tokens` tokens of one
// chunk. It rebuilds, from chunk_counts, the expert totals (-> counts and
// aligned offsets, written by block 0) and the counts of earlier chunks, turns
// in-chunk ranks into within-expert slots and destinations, and copies each
// token row once from x to its K destinations with VB-byte accesses. Blocks
// e, e+grid, ... also zero the padding rows of expert e.
//
// The source rows do not depend on the destinations, so each thread loads its
// first kPackEarly vectors of x before the prefix work and stores them after:
// all blocks start together, and the prefix's dependent global reads and
// barriers (a few microseconds) would otherwise pass with no copy traffic
// (H=4096, 4096 tokens: 19.7 us before).
// ---------------------------------------------------------------------------
constexpr int kPackThreads = 256;
constexpr int kPackMaxAssign = 256;  // pack_tokens * K upper bound
constexpr int kPackEarly = 4;        // vectors of x per thread loaded before the prefix

template <int VB> struct VecOf;
template <> struct VecOf<16> { using T = uint4; };
template <> struct VecOf<8> { using T = uint2; };
template <> struct VecOf<4> { using T = uint32_t; };
template <> struct VecOf<2> { using T = uint16_t; };

template <typename V> __device__ __forceinline__ V zero_vec();
template <> __device__ __forceinline__ uint4 zero_vec<uint4>() { return make_uint4(0, 0, 0, 0); }
template <> __device__ __forceinline__ uint2 zero_vec<uint2>() { return make_uint2(0, 0); }
template <> __device__ __forceinline__ uint32_t zero_vec<uint32_t>() { return 0u; }
template <> __device__ __forceinline__ uint16_t zero_vec<uint16_t>() { return 0; }

// COUNT (at most kSmallAssign assignments): no count_rank_kernel; every block
// ranks all assignments itself (the same ballots, in flat order) and keeps
// the expert totals and its own assignments' ranks, which saves a launch for
// small batches. The ranks, and so every output, are the same as the
// two-kernel path's.
constexpr int kSmallAssign = 1024;

// Ranks (in-chunk, !COUNT) come from `ranks`: the count/rank pass writes them
// into slots itself, a ranked route into a buffer of its own. Destination and
// padding rows are kept below packed_rows (they are for consistent counts and
// ranks; a caller's inconsistent pair is not written out of bounds).
// ROWS: the layout without the rows. Instead of copying x rows into packed,
// row_src[r] receives the token whose row packed row r would hold (-1 for
// padding rows), for a GEMM that reads its A rows from x through it.
template <int VB, bool COUNT, bool ROWS>
__global__ __launch_bounds__(kPackThreads) void pack_kernel(
    const char* __restrict__ x, const int32_t* __restrict__ ids, int32_t* slots,
    const int32_t* ranks, const int32_t* __restrict__ chunk_counts, int32_t* __restrict__ counts,
    int32_t* __restrict__ offsets, char* __restrict__ packed, int32_t* __restrict__ inverse,
    int32_t* __restrict__ row_src, int64_t tokens, int64_t row_bytes, int experts, int topk, int alignment,
    int64_t chunk_tokens, int pack_tokens, int n_chunks, int experts_pow2, int64_t packed_rows) {
    using V = typename VecOf<VB>::T;
    __shared__ int part_all[kPackThreads / kWave][kMaxExperts];
    __shared__ int part_before[kPackThreads / kWave][kMaxExperts];
    __shared__ int total[kMaxExperts];
    __shared__ int before[kMaxExperts];
    __shared__ int offs[kMaxExperts + 1];
    __shared__ int64_t dest[kPackMaxAssign];
    __shared__ int own_rank[COUNT ? kPackMaxAssign : 1];

    const int tid = threadIdx.x;
    const int wave = tid / kWave;
    const int lane = tid % kWave;
    const int64_t t0 = static_cast<int64_t>(blockIdx.x) * pack_tokens;
    const int my_chunk = static_cast<int>(t0 / chunk_tokens);
    const int64_t t_end = min(t0 + pack_tokens, tokens);
    const int n_tok = static_cast<int>(max<int64_t>(t_end - t0, 0));
    // Item i of this block is vector i % nv of token t0 + i / nv (the launcher
    // keeps pack_tokens * nv within int32).
    const int nv = static_cast<int>(row_bytes / VB);
    const int items = n_tok * nv;
    auto src = [&](int i) {
        const int tl = i / nv;
        return reinterpret_cast<const V*>(x + (t0 + tl) * row_bytes)[i - tl * nv];
    };
    V early[kPackEarly];
    if constexpr (!ROWS) {
#pragma unroll
        for (int j = 0; j < kPackEarly; ++j) {
            const int i = tid + j * kPackThreads;
            if (i < items) early[j] = src(i);
        }
    }
    // This thread's assignment (n_tok * K <= kPackMaxAssign == kPackThreads):
    // its expert and in-chunk rank do not depend on the prefix either.
    static_assert(kPackMaxAssign <= kPackThreads, "one assignment per thread");
    const int n_local = n_tok * topk;
    const int64_t my_p = t0 * topk + tid;
    const int my_e = tid < n_local ? ids[my_p] : -1;
    int my_rank = -1;
    if constexpr (!COUNT) {
        if (tid < n_local) my_rank = ranks[my_p];
    }

    if constexpr (COUNT) {
        // (a') Every assignment in rounds of kPackThreads: totals in `total`, and
        //      for this block's assignments the rank among earlier assignments
        //      to the same expert (-1 for an out-of-range id).
        const uint64_t lanes_below = (lane == 0) ? 0ull : (~0ull >> (kWave - lane));
        const int64_t n_assign = tokens * topk;
        const int64_t own_lo = t0 * topk;
        const int64_t own_hi = min(t0 + pack_tokens, tokens) * topk;
        if (tid < kMaxExperts) total[tid] = 0;
        for (int64_t base = 0; base < n_assign; base += kPackThreads) {
            for (int i = tid; i < (kPackThreads / kWave) * kMaxExperts; i += kPackThreads)
                (&part_all[0][0])[i] = 0;
            __syncthreads();
            const int64_t p = base + tid;
            const bool valid = p < n_assign;
            const int e = valid ? ids[p] : -1;
            const bool in_range = valid && e >= 0 && e < experts;
            uint64_t same = __ballot(in_range);
#pragma unroll
            for (int b = 0; b < 6; ++b) {
                const bool bit = (e >> b) & 1;
                const uint64_t plane = __ballot(in_range && bit);
                same &= bit ? plane : ~plane;
            }
            const int rank = __popcll(same & lanes_below);
            if (in_range && rank == 0) part_all[wave][e] = __popcll(same);
            __syncthreads();
            if (valid && p >= own_lo && p < own_hi) {
                int s = -1;
                if (in_range) {
                    s = total[e] + rank;
                    for (int w = 0; w < wave; ++w) s += part_all[w][e];
                }
                own_rank[p - own_lo] = s;
            }
            __syncthreads();
            if (tid < experts) {
                int add = 0;
                for (int w = 0; w < kPackThreads / kWave; ++w) add += part_all[w][tid];
                total[tid] += add;
            }
            __syncthreads();
        }
    } else {
    // (a) Column sums of chunk_counts: all chunks, and chunks before mine.
    //     Thread tid always sees expert tid % experts_pow2 (a divisor of 256).
    //     Loads go out eight at a time (independent), not one per loop trip:
    //     the table has up to 4096 entries (16 per thread) and each trip's L2
    //     latency would otherwise add up on every block's critical path.
    {
        const int e = tid % experts_pow2;
        const int stride = kPackThreads / experts_pow2;
        int s_all = 0, s_before = 0;
        if (e < experts) {
            for (int c0 = tid / experts_pow2; c0 < n_chunks; c0 += 8 * stride) {
                int v[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int c = c0 + j * stride;
                    v[j] = c < n_chunks ? chunk_counts[static_cast<int64_t>(c) * experts + e] : 0;
                }
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    s_all += v[j];
                    if (c0 + j * stride < my_chunk) s_before += v[j];
                }
            }
        }
        for (int m = experts_pow2; m < kWave; m <<= 1) {
            s_all += __shfl_xor(s_all, m);
            s_before += __shfl_xor(s_before, m);
        }
        if (lane < experts_pow2 && lane < kMaxExperts) {
            part_all[wave][lane] = s_all;
            part_before[wave][lane] = s_before;
        }
    }
    __syncthreads();
    }
    if (wave == 0) {
        int tot = 0, bef = 0;
        if (lane < experts) {
            if constexpr (COUNT) {
                tot = total[lane];  // ranks are already global: nothing before
            } else {
                for (int w = 0; w < kPackThreads / kWave; ++w) {
                    tot += part_all[w][lane];
                    bef += part_before[w][lane];
                }
            }
        }
        const int span = (tot + alignment - 1) / alignment * alignment;
        int incl = span;  // inclusive scan over the wavefront
        for (int d = 1; d < kWave; d <<= 1) {
            const int up = __shfl_up(incl, d);
            if (lane >= d) incl += up;
        }
        if (lane < experts) {
            total[lane] = tot;
            before[lane] = bef;
            offs[lane + 1] = incl;
        }
        if (lane == 0) offs[0] = 0;
    }
    __syncthreads();
    if (blockIdx.x == 0) {
        if (tid < experts) counts[tid] = total[tid];
        if (tid <= experts) offsets[tid] = offs[tid];
    }

    // (b) Destinations of this block's assignments.
    if (tid < n_local) {
        const int e = my_e;
        int64_t d = -1;
        if (e >= 0 && e < experts) {
            const int r = COUNT ? own_rank[tid] : my_rank;
            const int64_t slot = static_cast<int64_t>(before[e]) + r;
            const int64_t row = static_cast<int64_t>(offs[e]) + slot;
            if (r >= 0 && slot >= 0 && row >= 0 && row < packed_rows) {
                d = row;
                slots[my_p] = static_cast<int32_t>(slot);
                inverse[my_p] = static_cast<int32_t>(d);
                if constexpr (ROWS) row_src[d] = static_cast<int32_t>(t0 + tid / topk);
            }
        } else {
            slots[my_p] = -1;  // out-of-range id (the count/rank pass also writes -1)
        }
        dest[tid] = d;
    }
    __syncthreads();

    // (c) Row copies: each x row is read once and written to its K rows.
    auto store = [&](int i, const V& val) {
        const int tl = i / nv;
        const int v = i - tl * nv;
        for (int k = 0; k < topk; ++k) {
            const int64_t d = dest[tl * topk + k];
            if (d >= 0) reinterpret_cast<V*>(packed + d * row_bytes)[v] = val;
        }
    };
    if constexpr (!ROWS) {
#pragma unroll
        for (int j = 0; j < kPackEarly; ++j) {
            const int i = tid + j * kPackThreads;
            if (i < items) store(i, early[j]);
        }
        for (int i = tid + kPackEarly * kPackThreads; i < items; i += kPackThreads) store(i, src(i));
    }

    // (d) Padding rows [offs[e] + total[e], offs[e+1]) are zero (ROWS: map to -1).
    for (int e = blockIdx.x; e < experts; e += gridDim.x) {
        const int64_t r0 = max(static_cast<int64_t>(offs[e]) + total[e], static_cast<int64_t>(0));
        const int64_t r1 = min(static_cast<int64_t>(offs[e + 1]), packed_rows);
        if constexpr (ROWS) {
            for (int64_t r = r0 + tid; r < r1; r += kPackThreads) row_src[r] = -1;
        } else {
            const int64_t pad_items = (r1 - r0) * nv;
            V* base = reinterpret_cast<V*>(packed + r0 * row_bytes);
            for (int64_t i = tid; i < pad_items; i += kPackThreads) base[i] = zero_vec<V>();
        }
    }
}

// ---------------------------------------------------------------------------
// Combine: out[t] = round(sum_k w[t,k] * y[inverse[t,k]]) in fp32, k order,
// separate multiply and add (no contraction), skipped rows outside [0, R).
// Each thread owns VECS VE-element vectors of one token and issues all
// K * VECS gathers before reducing.
// ---------------------------------------------------------------------------
template <int DT, int VE, int VECS>
__global__ __launch_bounds__(256) void combine_kernel(
    const typename Elem<DT>::T* __restrict__ y, const int32_t* __restrict__ inverse,
    const float* __restrict__ weights, typename Elem<DT>::T* __restrict__ out, int64_t tokens,
    int64_t hidden, int topk, int64_t rows) {
#pragma clang fp contract(off)
    using T = typename Elem<DT>::T;
    struct alignas(sizeof(T) * VE) Pack {
        T v[VE];
    };
    const int64_t nv = hidden / VE;
    const int64_t groups = (nv + VECS - 1) / VECS;  // vector groups per token
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    const int64_t t = idx / groups;
    if (t >= tokens) return;
    const int64_t v0 = (idx - t * groups) * VECS;
    float acc[VECS][VE];
#pragma unroll
    for (int u = 0; u < VECS; ++u)
#pragma unroll
        for (int j = 0; j < VE; ++j) acc[u][j] = 0.0f;
    for (int k0 = 0; k0 < topk; k0 += 2) {
        Pack in[2][VECS];
        float w[2];
        bool ok[2];
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            const int k = k0 + kk;
            ok[kk] = false;
            w[kk] = 0.0f;
            if (k < topk) {
                const int64_t pa = t * topk + k;
                const int row = inverse[pa];
                ok[kk] = row >= 0 && row < rows;
                if (ok[kk]) {
                    w[kk] = weights[pa];
                    const Pack* src = reinterpret_cast<const Pack*>(y + static_cast<int64_t>(row) * hidden);
#pragma unroll
                    for (int u = 0; u < VECS; ++u)
                        if (v0 + u < nv) in[kk][u] = src[v0 + u];
                }
            }
        }
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            if (!ok[kk]) continue;
#pragma unroll
            for (int u = 0; u < VECS; ++u)
#pragma unroll
                for (int j = 0; j < VE; ++j) {
                    const float prod = w[kk] * Elem<DT>::load(in[kk][u].v[j]);
                    acc[u][j] = acc[u][j] + prod;
                }
        }
    }
#pragma unroll
    for (int u = 0; u < VECS; ++u) {
        if (v0 + u >= nv) continue;
        Pack o;
#pragma unroll
        for (int j = 0; j < VE; ++j) o.v[j] = Elem<DT>::store(acc[u][j]);
        reinterpret_cast<Pack*>(out + t * hidden)[v0 + u] = o;
    }
}

// ---------------------------------------------------------------------------
// Standalone SwiGLU (API parity; the block fuses it into the gate/up GEMM).
// ---------------------------------------------------------------------------
template <int DT>
__global__ __launch_bounds__(256) void swiglu_kernel(const typename Elem<DT>::T* __restrict__ proj,
                                                     const int32_t* __restrict__ valid_rows,
                                                     typename Elem<DT>::T* __restrict__ out,
                                                     int64_t rows, int64_t width) {
    const int64_t elements = rows * width;
    const int64_t valid = *valid_rows;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < elements;
         i += static_cast<int64_t>(gridDim.x) * 256) {
        const int64_t r = i / width;
        const int64_t c = i - r * width;
        if (r >= valid) {
            out[i] = Elem<DT>::store(0.0f);
            continue;
        }
        const int64_t base = r * width * 2 + c;
        const float g = Elem<DT>::load(proj[base]);
        const float u = Elem<DT>::load(proj[base + width]);
        out[i] = Elem<DT>::store(silu_f32(g) * u);
    }
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
struct DispatchPlan {
    int64_t chunk_tokens;
    int64_t n_chunks;
    int pack_tokens;
    int64_t pack_blocks;
};

static int64_t pow2_at_least(int64_t v) {
    int64_t p = 1;
    while (p < v) p <<= 1;
    return p;
}

// Chunk size keeps n_chunks * E <= prefix_max(E) (each pack block rebuilds its
// prefix from the whole chunk_counts table) unless the chunks are given (the
// router's tiles); pack blocks move about 16 KiB of rows.
static DispatchPlan plan_dispatch(int64_t tokens, int64_t experts, int64_t topk, int64_t row_bytes,
                                  int64_t given_chunk = 0) {
    DispatchPlan p{};
    int64_t chunk = 16;
    while (chunk < tokens && ((tokens + chunk - 1) / chunk) * experts > prefix_max(experts)) chunk <<= 1;
    if (given_chunk > 0) chunk = given_chunk;
    p.chunk_tokens = chunk;
    p.n_chunks = tokens > 0 ? (tokens + chunk - 1) / chunk : 0;
    int64_t pt = 1;
    const int64_t max_pt = kPackMaxAssign / topk;
    while (pt * 2 <= max_pt && pt * 2 <= chunk && pt * row_bytes < 16384) pt <<= 1;
    p.pack_tokens = static_cast<int>(pt);
    p.pack_blocks = tokens > 0 ? (tokens + pt - 1) / pt : 1;
    // Block b also zeroes the padding rows of experts b, b + grid, ...: at
    // least one block per expert, so that a few tokens' padding (up to a-1
    // rows per expert) is not written by one block alone (T=1, H=4096, a=8:
    // 5.2 us with one block).
    if (p.pack_blocks < experts) p.pack_blocks = experts;
    return p;
}

int64_t dispatch_scratch_bytes(int64_t tokens, int64_t experts, int64_t topk) {
    const DispatchPlan p = plan_dispatch(tokens, experts, topk, 16);
    const int64_t n = p.n_chunks * experts;
    return (n > 0 ? n : 1) * static_cast<int64_t>(sizeof(int32_t));
}

static int launch_pack(const void* x, int dtype, const int32_t* ids, int32_t* counts, int32_t* offsets,
                       int32_t* slots, const int32_t* ranks, void* packed, int32_t* inverse,
                       const int32_t* chunk_counts, int64_t tokens, int64_t hidden, int experts, int topk,
                       int alignment, int64_t packed_rows, bool vectorized, const DispatchPlan& plan,
                       bool count_in_pack, hipStream_t stream, int32_t* row_src = nullptr);

int launch_dispatch(const void* x, int dtype, const int32_t* ids, int32_t* counts,
                    int32_t* offsets, int32_t* slots, void* packed, int32_t* inverse,
                    int32_t* chunk_counts, int64_t tokens, int64_t hidden, int experts, int topk,
                    int alignment, int64_t packed_rows, bool vectorized, hipStream_t stream) {
    const int64_t row_bytes = hidden * dtype_size(dtype);
    const DispatchPlan plan = plan_dispatch(tokens, experts, topk, row_bytes);
    const int64_t n_assign = tokens * topk;
    const bool count_in_pack = n_assign <= kSmallAssign;
    if (plan.n_chunks > 0 && !count_in_pack) {
        hipLaunchKernelGGL(count_rank_kernel, dim3(static_cast<unsigned>(plan.n_chunks)),
                           dim3(kRankThreads), 0, stream, ids, slots, chunk_counts, n_assign,
                           experts, plan.chunk_tokens * topk);
        int rc = check_launch("count_rank_kernel");
        if (rc != MOE_OK) return rc;
    }
    return launch_pack(x, dtype, ids, counts, offsets, slots, slots, packed, inverse, chunk_counts, tokens,
                       hidden, experts, topk, alignment, packed_rows, vectorized, plan, count_in_pack, stream);
}

// Dispatch after a ranked route: `ranks` holds the in-tile ranks and
// tile_counts the per-tile counts of tiles of tile_tokens tokens (the
// count/rank pass's formats, with the tiles as chunks), so only the pack
// kernel runs. It does not write `ranks`, so it can run again on them.
int launch_dispatch_ranked(const void* x, int dtype, const int32_t* ids, int32_t* counts, int32_t* offsets,
                           int32_t* slots, void* packed, int32_t* inverse, const int32_t* ranks,
                           const int32_t* tile_counts, int64_t tile_tokens, int64_t tokens, int64_t hidden,
                           int experts, int topk, int alignment, int64_t packed_rows, bool vectorized,
                           hipStream_t stream) {
    const int64_t row_bytes = hidden * dtype_size(dtype);
    const DispatchPlan plan = plan_dispatch(tokens, experts, topk, row_bytes, tile_tokens);
    return launch_pack(x, dtype, ids, counts, offsets, slots, ranks, packed, inverse, tile_counts, tokens,
                       hidden, experts, topk, alignment, packed_rows, vectorized, plan, false, stream);
}

// The layout without the rows: counts, offsets, slots and inverse as
// launch_dispatch writes them, and row_src (packed_rows int32) the token of
// each packed row (-1 for padding; rows >= offsets[E] untouched). With
// `ranks` (a ranked route's tiles of tile_tokens tokens) the pack kernel
// alone; otherwise the counting kernel first, into chunk_counts.
int launch_dispatch_rows(const int32_t* ids, int32_t* counts, int32_t* offsets, int32_t* slots, int32_t* inverse,
                         int32_t* row_src, const int32_t* ranks, int32_t* chunk_counts, int64_t tile_tokens,
                         int64_t tokens, int experts, int topk, int alignment, int64_t packed_rows,
                         hipStream_t stream) {
    // 16-byte "rows": a block takes as many tokens as its assignment budget allows.
    const DispatchPlan plan = plan_dispatch(tokens, experts, topk, 16, ranks ? tile_tokens : 0);
    const int64_t n_assign = tokens * topk;
    const bool count_in_pack = ranks == nullptr && n_assign <= kSmallAssign;
    if (ranks == nullptr && plan.n_chunks > 0 && !count_in_pack) {
        hipLaunchKernelGGL(count_rank_kernel, dim3(static_cast<unsigned>(plan.n_chunks)), dim3(kRankThreads), 0,
                           stream, ids, slots, chunk_counts, n_assign, experts, plan.chunk_tokens * topk);
        const int rc = check_launch("count_rank_kernel");
        if (rc != MOE_OK) return rc;
    }
    return launch_pack(nullptr, 0, ids, counts, offsets, slots, ranks ? ranks : slots, nullptr, inverse,
                       chunk_counts, tokens, 0, experts, topk, alignment, packed_rows, false, plan, count_in_pack,
                       stream, row_src);
}

static int launch_pack(const void* x, int dtype, const int32_t* ids, int32_t* counts, int32_t* offsets,
                       int32_t* slots, const int32_t* ranks, void* packed, int32_t* inverse,
                       const int32_t* chunk_counts, int64_t tokens, int64_t hidden, int experts, int topk,
                       int alignment, int64_t packed_rows, bool vectorized, const DispatchPlan& plan,
                       bool count_in_pack, hipStream_t stream, int32_t* row_src) {
    const int experts_pow2_rows = static_cast<int>(pow2_at_least(experts));
    if (row_src != nullptr) {  // the row table instead of the rows (x and packed unused)
#define MOE_ROWS_LAUNCH(CNT)                                                                             \
    hipLaunchKernelGGL((pack_kernel<16, CNT, true>), dim3(static_cast<unsigned>(plan.pack_blocks)),       \
                       dim3(kPackThreads), 0, stream, nullptr, ids, slots, ranks, chunk_counts, counts,    \
                       offsets, nullptr, inverse, row_src, tokens, int64_t{16}, experts, topk, alignment, \
                       plan.chunk_tokens, plan.pack_tokens, static_cast<int>(plan.n_chunks),              \
                       experts_pow2_rows, packed_rows)
        if (count_in_pack)
            MOE_ROWS_LAUNCH(true);
        else
            MOE_ROWS_LAUNCH(false);
#undef MOE_ROWS_LAUNCH
        return check_launch("pack_kernel");
    }
    const int64_t elem = dtype_size(dtype);
    const int64_t row_bytes = hidden * elem;
    // The widest access that divides the row size and both base addresses (an
    // offset view of a larger tensor may start at any element).
    int vb = static_cast<int>(elem);
    if (vectorized) {
        const uint64_t bits = static_cast<uint64_t>(row_bytes) | reinterpret_cast<uintptr_t>(x) |
                              reinterpret_cast<uintptr_t>(packed);
        for (int w : {16, 8, 4}) {
            if (w > vb && bits % w == 0) {
                vb = w;
                break;
            }
        }
    }
    MOE_REQUIRE(plan.pack_tokens * (row_bytes / vb) <= INT32_MAX, MOE_ERR_UNSUPPORTED,
                "row of %lld bytes too large for the pack kernel", (long long)row_bytes);
    const int experts_pow2 = static_cast<int>(pow2_at_least(experts));
    const dim3 grid(static_cast<unsigned>(plan.pack_blocks));
#define MOE_PACK_LAUNCH(VBV, CNT)                                                              \
    hipLaunchKernelGGL((pack_kernel<VBV, CNT, false>), grid, dim3(kPackThreads), 0, stream,     \
                       static_cast<const char*>(x), ids, slots, ranks, chunk_counts, counts, offsets, \
                       static_cast<char*>(packed), inverse, nullptr, tokens, row_bytes, experts, topk, \
                       alignment, plan.chunk_tokens, plan.pack_tokens,                          \
                       static_cast<int>(plan.n_chunks), experts_pow2, packed_rows)
#define MOE_PACK_CASE(VBV)                 \
    if (count_in_pack)                     \
        MOE_PACK_LAUNCH(VBV, true);        \
    else                                   \
        MOE_PACK_LAUNCH(VBV, false)
    switch (vb) {
        case 16: MOE_PACK_CASE(16); break;
        case 8: MOE_PACK_CASE(8); break;
        case 4: MOE_PACK_CASE(4); break;
        case 2: MOE_PACK_CASE(2); break;
        default: return fail(MOE_ERR_UNSUPPORTED, "row size %lld bytes", (long long)row_bytes);
    }
#undef MOE_PACK_CASE
#undef MOE_PACK_LAUNCH
    return check_launch("pack_kernel");
}

template <int DT, int VE>
static void launch_combine_t(const void* y, const int32_t* inverse, const float* weights,
                             void* out, int64_t tokens, int64_t hidden, int topk, int64_t rows,
                             hipStream_t stream) {
    using T = typename Elem<DT>::T;
    // Two vectors per thread, one for rows of 8 KiB and up (vectorized): at
    // H=4096 bf16, 4096 tokens, top-2, 17.7 against 18.6 us; at H=2048 one
    // vector took 9.85 against 9.46 us.
    auto go = [&](auto vecs_c) {
        constexpr int VECS = decltype(vecs_c)::value;
        const int64_t groups = (hidden / VE + VECS - 1) / VECS;
        const int64_t threads = tokens * groups;
        const dim3 grid(static_cast<unsigned>((threads + 255) / 256));
        hipLaunchKernelGGL((combine_kernel<DT, VE, VECS>), grid, dim3(256), 0, stream,
                           static_cast<const T*>(y), inverse, weights, static_cast<T*>(out), tokens,
                           hidden, topk, rows);
    };
    if (VE > 1 && hidden * static_cast<int64_t>(sizeof(T)) >= 8192)
        go(std::integral_constant<int, 1>{});
    else
        go(std::integral_constant<int, 2>{});
}

int launch_combine(const void* y, int dtype, const int32_t* inverse, const float* weights,
                   void* out, int64_t tokens, int64_t hidden, int topk, int64_t rows,
                   hipStream_t stream) {
    if (tokens == 0) return MOE_OK;
    // 16-byte vectors need both row arrays 16-byte aligned (rows then are too).
    const bool vec_ok = (reinterpret_cast<uintptr_t>(y) | reinterpret_cast<uintptr_t>(out)) % 16 == 0;
    switch (dtype) {
        case MOE_DTYPE_BF16:
            if (vec_ok && hidden % 8 == 0) launch_combine_t<MOE_DTYPE_BF16, 8>(y, inverse, weights, out, tokens, hidden, topk, rows, stream);
            else launch_combine_t<MOE_DTYPE_BF16, 1>(y, inverse, weights, out, tokens, hidden, topk, rows, stream);
            break;
        case MOE_DTYPE_F16:
            if (vec_ok && hidden % 8 == 0) launch_combine_t<MOE_DTYPE_F16, 8>(y, inverse, weights, out, tokens, hidden, topk, rows, stream);
            else launch_combine_t<MOE_DTYPE_F16, 1>(y, inverse, weights, out, tokens, hidden, topk, rows, stream);
            break;
        case MOE_DTYPE_F32:
            if (vec_ok && hidden % 4 == 0) launch_combine_t<MOE_DTYPE_F32, 4>(y, inverse, weights, out, tokens, hidden, topk, rows, stream);
            else launch_combine_t<MOE_DTYPE_F32, 1>(y, inverse, weights, out, tokens, hidden, topk, rows, stream);
            break;
        default: return fail(MOE_ERR_INVALID_ARGUMENT, "unknown dtype %d", dtype);
    }
    return check_launch("combine_kernel");
}

int launch_swiglu(const void* proj, int dtype, const int32_t* valid_rows, void* out, int64_t rows,
                  int64_t width, hipStream_t stream) {
    const int64_t elements = rows * width;
    if (elements == 0) return MOE_OK;
    const int64_t blocks = std::min<int64_t>((elements + 255) / 256, 1 << 20);
    const dim3 grid(static_cast<unsigned>(blocks));
    switch (dtype) {
        case MOE_DTYPE_BF16:
            hipLaunchKernelGGL(swiglu_kernel<MOE_DTYPE_BF16>, grid, dim3(256), 0, stream,
                               static_cast<const uint16_t*>(proj), valid_rows,
                               static_cast<uint16_t*>(out), rows, width);
            break;
        case MOE_DTYPE_F16:
            hipLaunchKernelGGL(swiglu_kernel<MOE_DTYPE_F16>, grid, dim3(256), 0, stream,
                               static_cast<const uint16_t*>(proj), valid_rows,
                               static_cast<uint16_t*>(out), rows, width);
            break;
        case MOE_DTYPE_F32:
            hipLaunchKernelGGL(swiglu_kernel<MOE_DTYPE_F32>, grid, dim3(256), 0, stream,
                               static_cast<const float*>(proj), valid_rows,
                               static_cast<float*>(out), rows, width);
            break;
        default: return fail(MOE_ERR_INVALID_ARGUMENT, "unknown dtype %d", dtype);
    }
    return check_launch("swiglu_kernel");
}

}  // namespace moe
