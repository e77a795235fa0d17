// Grouped bf16 expert GEMMs on CDNA4 MFMA (v_mfma_f32_16x16x32_bf16; 32x32x16 on the generic path).
//
// Problem: for every expert e, rows r in [offsets[e], offsets[e+1]) of A
// [R, K] multiply B[e]^T (B is [E, N, K], K-contiguous like A) into C [R, N].
// Reference behaviour: src/moe_dispatch/experts.py:21-35 and the persistent
// Triton kernel src/moe_dispatch/_triton_gemm.py:16-72 (device-resident
// ENDS = offsets[1:], masked partial row tiles, fp32 accumulation, bf16
// output). The gate/up variant fuses the SwiGLU of csrc/dispatch.cu:277-292
// into the epilogue: gate and up columns of the same output column land in the
// same lane, so the activation is computed in registers.
//
// Design (gfx950):
//  * Fast path (K % 32 == 0, the block's shapes): ring_tile / grouped_gemm_ring_kernel
//    below -- 256 x 256 tiles on four wavefronts of 128 x 128 (16x16x32 MFMAs),
//    direct-to-LDS buffer loads into a four-stage LDS ring, loads three k-steps
//    ahead, MFMAs interleaved with fragment reads, XCD-aware two-phase order.
//  * Generic path (any K % 8 == 0): grouped_gemm_kernel -- global -> register ->
//    LDS double buffering with one barrier per 64-wide k-step; LDS rows are 128
//    bytes with 16-byte chunks XOR-swizzled per row (swz).
//  * Tile schedule is built on the device from offsets: expert e contributes
//    ceil(span_e/256) row tiles per column tile (0 for an empty expert). The grid
//    is a host-side upper bound; surplus workgroups exit at once, and no offsets
//    are read on the host.
//  * Every output element is one MFMA chain in ascending k with one fp32
//    accumulator, whichever path and tile shape computes it.
#include <type_traits>
#include <utility>

#include "moe_common.h"

namespace moe {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kGemmThreads = 256;
constexpr int kBK = 64;  // k-step: one 128-byte LDS row

struct GemmParams {
    const uint16_t* a;        // [R, K]
    const uint16_t* b;        // [E, NB, K]  (NB = N, or 2I for gate/up)
    uint16_t* c;              // [R, ldc]
    const int32_t* offsets;   // [E + 1]
    int64_t k;                // reduction length (H or I)
    int64_t nb;               // rows of one expert's B
    int64_t n_out;            // output columns (N, or I for gate/up)
    int64_t ldc;
    int64_t rows;             // rows of A and C; spans are clamped to it
    int experts;
    int n_tiles;              // output column tiles
    int n_cu;                 // compute units of the device (tail balancing)
};

// 16-byte chunk c of LDS row r lives at physical chunk c ^ f(r), f(r) = (r ^ (r >> 3)) & 7.
// A 16-byte read is serviced 16 lanes at a time across 64 four-byte banks (two
// 128-byte rows); with this f, 16 consecutive rows at one logical chunk hit 16
// distinct (row parity, chunk) bank groups, so fragment reads are conflict free
// (and so are 8-lane groups on a 32-bank LDS).
__device__ __forceinline__ int swz_key(int row) { return (row ^ (row >> 3)) & 7; }
__device__ __forceinline__ int swz(int row, int chunk) { return row * kBK + ((chunk ^ swz_key(row)) << 3); }

template <int BM, int BN, int WAVES_M, int WAVES_N, bool SWIGLU>
__global__ __launch_bounds__(kGemmThreads) void grouped_gemm_kernel(GemmParams p) {
    constexpr int WTM = BM / WAVES_M;
    constexpr int WTN = BN / WAVES_N;
    constexpr int SM = WTM / 32;
    constexpr int SN = WTN / 32;
    constexpr int A_LOADS = BM * kBK / 8 / kGemmThreads;  // 16-byte chunks per thread
    constexpr int B_LOADS = BN * kBK / 8 / kGemmThreads;
    static_assert(WAVES_M * WAVES_N == 4, "4 wavefronts");
    static_assert(A_LOADS >= 1 && B_LOADS >= 1, "tile too small");
    static_assert(!SWIGLU || (SN % 2 == 0), "gate/up pairing needs an even sub-tile count");

    __shared__ __attribute__((aligned(16))) uint16_t lds_a[2][BM * kBK];
    __shared__ __attribute__((aligned(16))) uint16_t lds_b[2][BN * kBK];

    // ---- tile lookup -------------------------------------------------------
    const int32_t* __restrict__ offs = p.offsets;
    int total = 0;
    for (int e = 0; e < p.experts; ++e) {
        const int span = offs[e + 1] - offs[e];
        total += ((span + BM - 1) / BM) * p.n_tiles;
    }
    const int per_xcd = (total + kNumXcd - 1) / kNumXcd;
    const int slot = blockIdx.x / kNumXcd;
    if (slot >= per_xcd) return;
    const int tile = (blockIdx.x % kNumXcd) * per_xcd + slot;
    if (tile >= total) return;
    int expert = 0, base = 0, m_tiles = 0;
    for (; expert < p.experts; ++expert) {
        const int span = offs[expert + 1] - offs[expert];
        m_tiles = (span + BM - 1) / BM;
        const int t = m_tiles * p.n_tiles;
        if (tile < base + t) break;
        base += t;
    }
    const int rel = tile - base;
    const int n_tile = rel / m_tiles;
    const int m_tile = rel - n_tile * m_tiles;
    const int64_t row0 = offs[expert] + static_cast<int64_t>(m_tile) * BM;
    const int64_t row_end = min(static_cast<int64_t>(offs[expert + 1]), p.rows);
    if (row0 < 0 || row0 >= row_end) return;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WAVES_N;
    const int wn = wave % WAVES_N;

    // ---- per-thread global chunk pointers ----------------------------------
    const uint16_t* a_src[A_LOADS];
    int a_dst[A_LOADS];
    bool a_ok[A_LOADS];
    int a_kc[A_LOADS];
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
        const int chunk = tid + i * kGemmThreads;
        const int r = chunk >> 3, c = chunk & 7;
        const int64_t grow = row0 + r;
        a_ok[i] = grow < row_end;
        a_src[i] = p.a + (a_ok[i] ? grow : row0) * p.k + c * 8;
        a_dst[i] = swz(r, c);
        a_kc[i] = c * 8;
    }
    const uint16_t* b_src[B_LOADS];
    int b_dst[B_LOADS];
    bool b_ok[B_LOADS];
    int b_kc[B_LOADS];
    const uint16_t* b_expert = p.b + static_cast<int64_t>(expert) * p.nb * p.k;
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i) {
        const int chunk = tid + i * kGemmThreads;
        const int r = chunk >> 3, c = chunk & 7;
        int64_t brow;
        bool ok;
        if constexpr (SWIGLU) {
            // LDS row r -> wave column block r / WTN; first half gate, second half up.
            const int wcol = r / WTN, w = r % WTN;
            constexpr int HALF = WTN / 2;
            const int64_t col = static_cast<int64_t>(n_tile) * (BN / 2) + wcol * HALF + (w % HALF);
            ok = col < p.n_out;
            brow = (w < HALF) ? col : p.n_out + col;
        } else {
            const int64_t col = static_cast<int64_t>(n_tile) * BN + r;
            ok = col < p.n_out;
            brow = col;
        }
        b_ok[i] = ok;
        b_src[i] = b_expert + (ok ? brow : 0) * p.k + c * 8;
        b_dst[i] = swz(r, c);
        b_kc[i] = c * 8;
    }

    floatx16 acc[SM][SN];
#pragma unroll
    for (int i = 0; i < SM; ++i)
#pragma unroll
        for (int j = 0; j < SN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    uint4 ra[A_LOADS], rb[B_LOADS];
    const int64_t K = p.k;
    const int k_steps = static_cast<int>((K + kBK - 1) / kBK);

    auto load_tile = [&](int64_t k0) {
#pragma unroll
        for (int i = 0; i < A_LOADS; ++i)
            ra[i] = (a_ok[i] && k0 + a_kc[i] < K) ? *reinterpret_cast<const uint4*>(a_src[i] + k0)
                                                  : make_uint4(0, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < B_LOADS; ++i)
            rb[i] = (b_ok[i] && k0 + b_kc[i] < K) ? *reinterpret_cast<const uint4*>(b_src[i] + k0)
                                                  : make_uint4(0, 0, 0, 0);
    };
    auto store_tile = [&](int buf) {
#pragma unroll
        for (int i = 0; i < A_LOADS; ++i) *reinterpret_cast<uint4*>(&lds_a[buf][a_dst[i]]) = ra[i];
#pragma unroll
        for (int i = 0; i < B_LOADS; ++i) *reinterpret_cast<uint4*>(&lds_b[buf][b_dst[i]]) = rb[i];
    };

    load_tile(0);
    store_tile(0);
    __syncthreads();

    const int frag_row = lane & 31;
    const int frag_half = lane >> 5;
    for (int kt = 0; kt < k_steps; ++kt) {
        const int buf = kt & 1;
        const bool has_next = kt + 1 < k_steps;
        if (has_next) load_tile(static_cast<int64_t>(kt + 1) * kBK);
        const uint16_t* la = lds_a[buf];
        const uint16_t* lb = lds_b[buf];
#pragma unroll
        for (int kk = 0; kk < kBK / 16; ++kk) {
            const int chunk = kk * 2 + frag_half;
            bf16x8_t af[SM], bfr[SN];
#pragma unroll
            for (int i = 0; i < SM; ++i) {
                const int r = wm * WTM + i * 32 + frag_row;
                af[i] = *reinterpret_cast<const bf16x8_t*>(&la[swz(r, chunk)]);
            }
#pragma unroll
            for (int j = 0; j < SN; ++j) {
                const int r = wn * WTN + j * 32 + frag_row;
                bfr[j] = *reinterpret_cast<const bf16x8_t*>(&lb[swz(r, chunk)]);
            }
#pragma unroll
            for (int i = 0; i < SM; ++i)
#pragma unroll
                for (int j = 0; j < SN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
        }
        if (has_next) store_tile(buf ^ 1);
        __syncthreads();
    }

    // ---- epilogue ------------------------------------------------------------
    // Accumulator register r of a 32x32 sub-tile holds row 8*(r/4) + 4*(lane/32) + r%4,
    // column lane%32.
    const int col_in = lane & 31;
    const int row_in = (lane >> 5) * 4;
    if constexpr (SWIGLU) {
        constexpr int HALF_SN = SN / 2;
#pragma unroll
        for (int i = 0; i < SM; ++i) {
#pragma unroll
            for (int j = 0; j < HALF_SN; ++j) {
                const int64_t col = static_cast<int64_t>(n_tile) * (BN / 2) + wn * (WTN / 2) + j * 32 + col_in;
                if (col >= p.n_out) continue;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int64_t grow = row0 + wm * WTM + i * 32 + (r >> 2) * 8 + row_in + (r & 3);
                    if (grow < row_end) {
                        const float g = bf16_to_f32(f32_to_bf16(acc[i][j][r]));
                        const float u = bf16_to_f32(f32_to_bf16(acc[i][j + HALF_SN][r]));
                        p.c[grow * p.ldc + col] = f32_to_bf16(silu_f32(g) * u);
                    }
                }
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < SM; ++i) {
#pragma unroll
            for (int j = 0; j < SN; ++j) {
                const int64_t col = static_cast<int64_t>(n_tile) * BN + wn * WTN + j * 32 + col_in;
                if (col >= p.n_out) continue;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int64_t grow = row0 + wm * WTM + i * 32 + (r >> 2) * 8 + row_in + (r & 3);
                    if (grow < row_end) p.c[grow * p.ldc + col] = f32_to_bf16(acc[i][j][r]);
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Fast path (K % 32 == 0): 256 x 256 output tiles computed by four wavefronts
// (one per SIMD), each owning 128 x 128 (or (TM/2) x (BNT/2) for the short last
// row tile of an expert and the split tail pieces) as a grid of 16 x 16 blocks
// on v_mfma_f32_16x16x32_bf16.
//
//  * Operands reach LDS through direct-to-LDS buffer loads
//    (buffer_load_dwordx4 ... lds): a wavefront load moves 16 rows of 64 bytes
//    (1 KiB), lane l landing at byte 16*l, i.e. row l/4, physical chunk l%4, so
//    it fetches the logical chunk the swizzle maps there. Buffer resources
//    bound the valid bytes: rows past the expert's span and weight rows past the
//    expert read as zero with no per-lane predicate.
//  * LDS is a ring of stages of 32 k (A TM x 64 B + B BNT x 64 B each; four for
//    a full 256 x 256 tile, six for the 64-row tiles). The loads of k-step
//    kt+STAGES-1 are issued while k-step kt computes, and the one barrier per
//    k-step waits only for the stage about to be read (vmcnt leaves the younger
//    stages in flight), so global latency hides behind STAGES-1 k-steps.
//  * Rows of 64 bytes hold 4 chunks of 16 bytes; chunk c of row r sits at
//    physical chunk c ^ ((r >> 2) & 3), so 16 lanes reading 16 consecutive rows
//    at one chunk touch all 64 banks once (conflict free).
//  * Fragment reads of the next stage are spread between the MFMAs of the
//    current one, each well ahead of its use, and a single set of fragment
//    registers is live (see ring_tile). sched_barrier fences pin the order.
//  * The k order of each output's MFMA chain (ascending k in groups of 8, one
//    accumulator) is the same as the generic path, whatever the tile shape.
// ---------------------------------------------------------------------------
constexpr uint32_t kRsrcWord3 = 0x00020000u;  // raw buffer, 32-bit dword format
constexpr int kRingK = 32;                     // k per LDS stage
constexpr int kRingThreads = 256;
constexpr uint32_t kRingBytes = 128 * 1024;
// Stages that fit for a tile of TM activation rows and BNT weight rows (k = 32
// per stage, 64 bytes per row), at most 6.
constexpr int ring_stages(int tm, int bnt) {
    const int fit = static_cast<int>(kRingBytes / ((tm + bnt) * kRingK * 2));
    return fit < 6 ? fit : 6;
}

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

__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t rsrc, char* lds_dst, uint32_t voffset,
                                      uint32_t soffset) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        rsrc, (__attribute__((address_space(3))) void*)(lds_dst), 16, voffset, soffset,
        0, 0);
}

// s_waitcnt vmcnt(VM) lgkmcnt(0) (gfx9 encoding: vmcnt[3:0] in bits 3:0 and
// vmcnt[5:4] in bits 15:14, expcnt in bits 6:4 with 7 = no wait, lgkmcnt in bits 11:8).
template <int VM>
__device__ __forceinline__ void wait_vm_lgkm0() {
    static_assert(VM >= 0 && VM < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((VM & 15) | ((VM >> 4) << 14) | (7 << 4));
}
// Workgroup barrier without the implied wait for all memory operations (the
// explicit wait above bounds what must have landed); the memory clobber keeps
// the compiler from moving LDS accesses across it.
__device__ __forceinline__ void ring_barrier() { asm volatile("s_barrier" ::: "memory"); }

__device__ __forceinline__ int ring_key(int row) { return (row >> 2) & 3; }

// f(integral_constant<int, 0>) ... f(integral_constant<int, N-1>), unrolled.
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// silu(g) * u for the fused epilogue: hardware exp2 and reciprocal
// (v_exp_f32, v_rcp_f32; about 1 ulp each), g and u already rounded to bf16.
__device__ __forceinline__ float swiglu_fast(float g, float u) {
    const float e = __builtin_amdgcn_exp2f(-g * 1.4426950408889634f);
    return (g * u) * __builtin_amdgcn_rcpf(1.0f + e);
}

// One output tile on v_mfma_f32_16x16x32_bf16: rows [row0, row0 + SMT*64) of one
// expert (clamped to row_end) by BNT weight rows starting at output column
// col0. A k-step is one 32-k stage: every wave multiplies its (WTM/16) x (WTN/16)
// grid of 16x16 blocks with one MFMA each while it reads the next stage's
// fragments and issues loads for a stage AHEAD steps on. The 16x16x32 form
// sustains a higher clock than 32x32x16 under the power limit (measured on
// MI355X: 1.91 vs 1.66 GHz with the same read and load mix), so it moves the
// same FLOPs about 10% faster.
template <int SMT, int BNT, bool SWIGLU>
__device__ __forceinline__ void ring_tile(const GemmParams& p, char* lds, int expert, int64_t col0,
                                          int64_t row0, int64_t row_end) {
    constexpr int WAVES = kRingThreads / kWave;
    constexpr int TM = SMT * 64;
    constexpr int WTM = TM / 2;
    constexpr int WTN = BNT / 2;
    constexpr int FA = WTM / 16;       // 16-row A fragments per wave
    constexpr int FB = WTN / 16;       // 16-row B fragments per wave
    constexpr int A_LOADS = TM / 16 / WAVES;
    constexpr int B_LOADS = BNT / 16 / WAVES;
    constexpr int LOADS = A_LOADS + B_LOADS;
    constexpr uint32_t A_STAGE = TM * kRingK * 2;   // bytes of one stage of A
    constexpr uint32_t B_STAGE = BNT * kRingK * 2;  // bytes of one stage of B
    constexpr int STAGES = ring_stages(TM, BNT) >= 6 ? 6 : 4;  // 4 for 256x256 and 256x128 tiles
    constexpr int AHEAD = STAGES - 1;               // k-step kt+AHEAD loads during kt
    constexpr uint32_t B_BASE = STAGES * A_STAGE;   // B stages follow the A stages
    static_assert(A_LOADS >= 1 && B_LOADS >= 1 && FA >= 1 && FB >= 2, "tile shape");
    static_assert(!SWIGLU || FB % 2 == 0, "gate/up pairing needs an even fragment count");
    static_assert(STAGES * (A_STAGE + B_STAGE) <= kRingBytes, "ring does not fit");
    static_assert((FA - 1) * 1024 < 65536 && (FB - 1) * 1024 < 65536, "fragment offsets fit the instruction offset");
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / 2;
    const int wn = wave % 2;
    const int64_t K = p.k;

    const int64_t a_rows = min<int64_t>(row_end - row0, TM);
    const __amdgpu_buffer_rsrc_t rsrc_a = make_rsrc(p.a + row0 * K, static_cast<uint32_t>(a_rows * K * 2));
    const __amdgpu_buffer_rsrc_t rsrc_b =
        make_rsrc(p.b + static_cast<int64_t>(expert) * p.nb * K, static_cast<uint32_t>(p.nb * K * 2));

    const int lrow = lane >> 2;
    uint32_t a_off[A_LOADS], b_off[B_LOADS];
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
        const int r = (wave * A_LOADS + i) * 16 + lrow;
        const int lchunk = (lane & 3) ^ ring_key(r);
        a_off[i] = static_cast<uint32_t>((r * K + lchunk * 8) * 2);
    }
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i) {
        const int r = (wave * B_LOADS + i) * 16 + lrow;
        const int lchunk = (lane & 3) ^ ring_key(r);
        int64_t brow;
        if constexpr (SWIGLU) {
            // Wave column wc owns gate columns [wc*WTN/2, (wc+1)*WTN/2) of the
            // tile and the matching up rows (I further on).
            const int wcol = r / WTN, w = r % WTN;
            constexpr int HALF = WTN / 2;
            const int64_t col = col0 + wcol * HALF + (w % HALF);
            brow = (w < HALF) ? col : p.n_out + col;
        } else {
            brow = col0 + r;
        }
        b_off[i] = static_cast<uint32_t>((brow * K + lchunk * 8) * 2);
    }
    // Loads [first, first + count) of the A-then-B list for k-step kt into stage st.
    auto issue = [&](int kt, int st, int first, int count) {
        const uint32_t koff = static_cast<uint32_t>(kt) * kRingK * 2;
#pragma unroll
        for (int i = 0; i < LOADS; ++i) {
            if (i < first || i >= first + count) continue;
            if (i < A_LOADS)
                dma16(rsrc_a, lds + st * A_STAGE + (wave * A_LOADS + i) * 1024, a_off[i], koff);
            else
                dma16(rsrc_b, lds + B_BASE + st * B_STAGE + (wave * B_LOADS + (i - A_LOADS)) * 1024,
                      b_off[i - A_LOADS], koff);
        }
    };

    // Per-lane fragment addresses: lane l reads row (l%16) of a fragment at k
    // chunk l/16 (all 32 k of the stage in one 16-byte read). Fragments 16 rows
    // apart share the swizzle key, so fragment and stage only add constants
    // (instruction offsets); stages from SPLIT on use second bases to keep those
    // offsets below 64 KiB.
    const int frag_row = lane & 15;
    const int chunk = lane >> 4;
    const int ar = wm * WTM + frag_row;
    const int br = wn * WTN + frag_row;
    const uint32_t va = static_cast<uint32_t>((ar * kRingK + ((chunk ^ ring_key(ar)) << 3)) * 2);
    const uint32_t vb = B_BASE + static_cast<uint32_t>((br * kRingK + ((chunk ^ ring_key(br)) << 3)) * 2);

    floatx4 acc[FA][FB];
#pragma unroll
    for (int i = 0; i < FA; ++i)
#pragma unroll
        for (int j = 0; j < FB; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[i][j][r] = 0.0f;

    // Fragment reads at a stage base (per-lane address of stage st, computed
    // once per k-step); the fragment index is an instruction offset.
    auto read_at = [&](uint32_t base, int idx) {
        return *reinterpret_cast<const bf16x8_t*>(lds + base + idx * 1024);
    };
    auto fence = [] { __builtin_amdgcn_sched_barrier(0); };

    // Weights fragment as src0, activations as src1: the 16x16 result comes out
    // transposed, so lane l holds row l%16 and the four consecutive columns
    // 4*(l/16) + 0..3 (packed 8-byte stores).
    //
    // One set of fragments (FA A + FB B) is live. A k-step runs in two halves:
    // B fragments [0, FB/2) with every A fragment, then [FB/2, FB). During the
    // first half this stage's B fragments [FB/2, FB) are read (their previous
    // values were last used by the previous step's second half); during the
    // second half the next stage's A fragment i is read right after its last
    // MFMA, and the next stage's B fragments [0, FB/2). Every read has at least
    // about a quarter of a k-step of MFMA work before its first use. The k-loop
    // is not unrolled (stage addresses are computed per step), so each
    // accumulator keeps one register through the loop.
    constexpr int HB = FB / 2;
    constexpr int HM = FA * HB;        // MFMAs per half
    static_assert(HB >= 1 && HM >= HB, "half-step shape");
    bf16x8_t fa[FA], fb[FB];
    const int k_steps = static_cast<int>(K / kRingK);
    // Loads go in two blocks per k-step: one load between each pair of MFMAs
    // makes the register allocator shuffle the accumulators through copies.
#pragma unroll
    for (int st = 0; st < AHEAD; ++st) issue(min(st, k_steps - 1), st, 0, LOADS);
    wait_vm_lgkm0<(AHEAD - 1) * LOADS>();
    ring_barrier();
    fence();
#pragma unroll
    for (int i = 0; i < FA; ++i) fa[i] = read_at(va, i);
#pragma unroll
    for (int j = 0; j < HB; ++j) fb[j] = read_at(vb, j);
    int st = 0;
    for (int kt = 0; kt < k_steps; ++kt) {
        // k-step kt in stage st; its loads (k-step kt+AHEAD) go to stage
        // (st+AHEAD)%STAGES, whose reads all ended before the previous barrier.
        const int nx = st + 1 == STAGES ? 0 : st + 1;
        const int lst = st == 0 ? STAGES - 1 : st - 1;
        const int ahead = min(kt + AHEAD, k_steps - 1);
        const uint32_t b_cur = vb + st * B_STAGE;
        const uint32_t a_nx = va + nx * A_STAGE, b_nx = vb + nx * B_STAGE;
        fence();
        // Stage kt+1 has landed once at most k-steps kt+2 .. kt+AHEAD-1 are younger.
        wait_vm_lgkm0<(AHEAD - 2) * LOADS>();
        ring_barrier();
        fence();
        issue(ahead, lst, 0, LOADS / 2);
        fence();
        static_for<HM>([&](auto m_c) {
            constexpr int m = decltype(m_c)::value;
            constexpr int i = m / HB, j = m % HB;
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fb[j], fa[i], acc[i][j], 0, 0, 0);
            if constexpr (m % 2 == 0 && m / 2 < HB) fb[HB + m / 2] = read_at(b_cur, HB + m / 2);
            fence();
        });
        issue(ahead, lst, LOADS / 2, LOADS - LOADS / 2);
        fence();
        static_for<HM>([&](auto m_c) {
            constexpr int m = decltype(m_c)::value;
            constexpr int i = m / HB, j = HB + m % HB;
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fb[j], fa[i], acc[i][j], 0, 0, 0);
            if constexpr (m % 2 == 1 && m / 2 < HB) fb[m / 2] = read_at(b_nx, m / 2);
            if constexpr (m % HB == HB - 1) fa[i] = read_at(a_nx, i);
            fence();
        });
        st = nx;
    }
    wait_vm_lgkm0<0>();

    // Epilogue: one row per lane, four consecutive columns per 8-byte store.
    // Each row of accumulators is first moved to VGPRs through an empty asm
    // operand: without it the register allocator shapes the accumulators' AGPR
    // assignment after the epilogue's register pairs and copies them inside the
    // k-loop on every step.
    const int col4 = 4 * (lane >> 4);
#pragma unroll
    for (int i = 0; i < FA; ++i) {
#pragma unroll
        for (int j = 0; j < FB; ++j) asm volatile("" : "+v"(acc[i][j]));
        const int64_t grow = row0 + wm * WTM + i * 16 + (lane & 15);
        if (grow >= row_end) continue;
        uint16_t* crow = p.c + grow * p.ldc;
        if constexpr (SWIGLU) {
#pragma unroll
            for (int j = 0; j < FB / 2; ++j) {
                const int64_t col = col0 + wn * (WTN / 2) + j * 16 + col4;
                if (col >= p.n_out) continue;
                float act[4];
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const uint32_t gu = pack_bf16x2(acc[i][j][t], acc[i][j + FB / 2][t]);
                    act[t] = swiglu_fast(__uint_as_float(gu << 16), __uint_as_float(gu & 0xffff0000u));
                }
                *reinterpret_cast<uint2*>(crow + col) =
                    make_uint2(pack_bf16x2(act[0], act[1]), pack_bf16x2(act[2], act[3]));
            }
        } else {
#pragma unroll
            for (int j = 0; j < FB; ++j) {
                const int64_t col = col0 + wn * WTN + j * 16 + col4;
                if (col >= p.n_out) continue;
                *reinterpret_cast<uint2*>(crow + col) =
                    make_uint2(pack_bf16x2(acc[i][j][0], acc[i][j][1]), pack_bf16x2(acc[i][j][2], acc[i][j][3]));
            }
        }
    }
}

// Work list, built on the device from offsets. Row tiles of more than 128 rows
// form phase 1 (equal cost) and the short last row tile of an expert (at most
// 128 rows) forms phase 2, so the CUs of an XCD run phase-1 tiles in lockstep
// rounds and share A and B k-slices in L2. Inside a phase, tiles go expert by
// expert, column tile by column tile, row tiles fastest, and each phase is
// spread over the XCDs in contiguous ranges (workgroup i runs on XCD i % 8).
// For the plain GEMM a short last round of a phase (at most half of the CUs)
// is split into 128-column pieces; every piece still runs the whole k chain
// in order, so results do not change.
struct RingPhase {
    int count;   // tiles
    int main;    // tiles mapped XCD-contiguously
    int blocks;  // workgroups of the main part (multiple of 8)
    int pieces;  // split tail pieces (2 per split tile)
};

__device__ __forceinline__ RingPhase ring_phase(int count, int n_cu, bool allow_split) {
    RingPhase ph;
    ph.count = count;
    const int rem = n_cu > 0 ? count % n_cu : 0;
    const bool split = allow_split && rem > 0 && 2 * rem <= n_cu;
    ph.main = split ? count - rem : count;
    ph.blocks = (ph.main + kNumXcd - 1) / kNumXcd * kNumXcd;
    ph.pieces = split ? 2 * rem : 0;
    return ph;
}

template <bool SWIGLU>
__global__ __launch_bounds__(kRingThreads) void grouped_gemm_ring_kernel(GemmParams p) {
    __shared__ __attribute__((aligned(1024))) char lds[kRingBytes];
    const int32_t* __restrict__ offs = p.offsets;
    auto full_tiles = [](int span) { return span / 256 + ((span % 256) > 128 ? 1 : 0); };
    int n_full = 0, n_part = 0;
    for (int e = 0; e < p.experts; ++e) {
        const int span = offs[e + 1] - offs[e];
        const int mf = full_tiles(span);
        n_full += mf * p.n_tiles;
        n_part += ((span + 255) / 256 - mf) * p.n_tiles;
    }
    const RingPhase ph1 = ring_phase(n_full, p.n_cu, !SWIGLU);
    const RingPhase ph2 = ring_phase(n_part, p.n_cu, !SWIGLU);
    int q = blockIdx.x;
    int phase = -1, tile = 0, piece = -1;
    const RingPhase* phs[2] = {&ph1, &ph2};
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const RingPhase& ph = *phs[k];
        if (phase >= 0) break;
        if (q < ph.blocks) {
            const int per = ph.blocks / kNumXcd;
            tile = (q % kNumXcd) * per + q / kNumXcd;
            if (tile >= ph.main) return;
            phase = k;
        } else if (q < ph.blocks + ph.pieces) {
            const int r = q - ph.blocks;
            tile = ph.main + r / 2;
            piece = r % 2;
            phase = k;
        } else {
            q -= ph.blocks + ph.pieces;
        }
    }
    if (phase < 0) return;
    int expert = 0, base = 0, span = 0, mf = 0;
    for (; expert < p.experts; ++expert) {
        span = offs[expert + 1] - offs[expert];
        mf = full_tiles(span);
        const int t = (phase == 0 ? mf : (span + 255) / 256 - mf) * p.n_tiles;
        if (tile < base + t) break;
        base += t;
    }
    if (expert >= p.experts) return;
    const int rel = tile - base;
    int n_tile, m_tile;
    if (phase == 0) {
        n_tile = rel / mf;
        m_tile = rel - n_tile * mf;
    } else {
        n_tile = rel;
        m_tile = mf;
    }
    const int64_t row0 = offs[expert] + static_cast<int64_t>(m_tile) * 256;
    const int64_t row_end = min(static_cast<int64_t>(offs[expert + 1]), p.rows);
    if (row0 < 0 || row0 >= row_end) return;
    const int rem_rows = span - m_tile * 256;  // rows left from this tile on
    if constexpr (SWIGLU) {
        const int64_t col0 = static_cast<int64_t>(n_tile) * 128;
        if (rem_rows > 128) ring_tile<4, 256, true>(p, lds, expert, col0, row0, row_end);
        else if (rem_rows > 64) ring_tile<2, 256, true>(p, lds, expert, col0, row0, row_end);
        else ring_tile<1, 256, true>(p, lds, expert, col0, row0, row_end);
    } else if (piece < 0) {
        const int64_t col0 = static_cast<int64_t>(n_tile) * 256;
        if (rem_rows > 128) ring_tile<4, 256, false>(p, lds, expert, col0, row0, row_end);
        else if (rem_rows > 64) ring_tile<2, 256, false>(p, lds, expert, col0, row0, row_end);
        else ring_tile<1, 256, false>(p, lds, expert, col0, row0, row_end);
    } else {
        const int64_t col0 = static_cast<int64_t>(n_tile) * 256 + piece * 128;
        if (rem_rows > 128) ring_tile<4, 128, false>(p, lds, expert, col0, row0, row_end);
        else if (rem_rows > 64) ring_tile<2, 128, false>(p, lds, expert, col0, row0, row_end);
        else ring_tile<1, 128, false>(p, lds, expert, col0, row0, row_end);
    }
}

// Decode-sized launches (at most 128 rows in all): every expert has at most one
// row tile, so the work is streaming the active experts' weights. Tiles are 64
// output columns wide, four times as many as the 256-wide tiles, so that a
// single token's two experts still spread over the CUs. Each output is the
// same MFMA chain in k order as on the wide path. MAX_ROWS (64 or 128) bounds
// every expert's span; the 64-row instance needs less LDS, so more blocks share
// a CU.
constexpr int kNarrowCols = 64;

template <bool SWIGLU, int MAX_ROWS>
__global__ __launch_bounds__(kRingThreads) void grouped_gemm_narrow_kernel(GemmParams p) {
    constexpr int BNT = SWIGLU ? 2 * kNarrowCols : kNarrowCols;
    constexpr uint32_t kLds = 6 * (MAX_ROWS + BNT) * kRingK * 2;  // six stages of the largest tile
    static_assert(MAX_ROWS == 64 || MAX_ROWS == 128, "narrow row tiles");
    static_assert(ring_stages(MAX_ROWS, BNT) >= 6 && ring_stages(64, BNT) >= 6, "narrow tiles use six stages");
    __shared__ __attribute__((aligned(1024))) char lds[kLds];
    const int expert = blockIdx.x / p.n_tiles;
    const int n_tile = blockIdx.x - expert * p.n_tiles;
    if (expert >= p.experts) return;
    const int64_t row0 = p.offsets[expert];
    const int64_t row_end = min(static_cast<int64_t>(p.offsets[expert + 1]), p.rows);
    if (row0 < 0 || row0 >= row_end) return;
    const int64_t span = row_end - row0;  // <= p.rows <= MAX_ROWS (checked by the launcher)
    const int64_t col0 = static_cast<int64_t>(n_tile) * kNarrowCols;
    if constexpr (MAX_ROWS == 128) {
        if (span > 64) {
            ring_tile<2, BNT, SWIGLU>(p, lds, expert, col0, row0, row_end);
            return;
        }
    }
    ring_tile<1, BNT, SWIGLU>(p, lds, expert, col0, row0, row_end);
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
// Compute units of the current device, cached per device id.
static int device_cu_count() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cached[dev] == 0) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
        cached[dev] = cus;
    }
    return cached[dev];
}

template <int BM, int BN, int WAVES_M, int WAVES_N, bool SWIGLU>
static int launch_gemm_t(GemmParams p, int64_t rows, hipStream_t stream) {
    const int64_t out_per_tile = SWIGLU ? BN / 2 : BN;
    p.n_tiles = static_cast<int>((p.n_out + out_per_tile - 1) / out_per_tile);
    // Upper bound on row tiles: sum_e ceil(span_e/BM) <= ceil(R/BM) + E.
    const int64_t m_bound = (rows + BM - 1) / BM + p.experts;
    int64_t blocks = m_bound * p.n_tiles;
    if (blocks == 0) return MOE_OK;
    p.n_cu = device_cu_count();
    if (BM == 256 && BN == 256 && p.k % kRingK == 0 && rows <= 128) {
        GemmParams q = p;
        q.n_tiles = static_cast<int>((p.n_out + kNarrowCols - 1) / kNarrowCols);
        const int64_t narrow_blocks = static_cast<int64_t>(p.experts) * q.n_tiles;
        if (narrow_blocks > INT32_MAX) return fail(MOE_ERR_CAPACITY, "grouped GEMM grid too large");
        if (rows <= 64)
            hipLaunchKernelGGL((grouped_gemm_narrow_kernel<SWIGLU, 64>), dim3(static_cast<unsigned>(narrow_blocks)),
                               dim3(kRingThreads), 0, stream, q);
        else
            hipLaunchKernelGGL((grouped_gemm_narrow_kernel<SWIGLU, 128>), dim3(static_cast<unsigned>(narrow_blocks)),
                               dim3(kRingThreads), 0, stream, q);
        return check_launch("grouped_gemm_narrow_kernel");
    }
    if (BM == 256 && BN == 256 && p.k % kRingK == 0) {
        // Two phases, each rounded up to the XCD count, plus room for the split
        // tail pieces (at most n_cu per phase).
        int64_t ring_blocks = blocks + 2 * kNumXcd;
        if (!SWIGLU) ring_blocks += 2 * static_cast<int64_t>(p.n_cu);
        if (ring_blocks > INT32_MAX) return fail(MOE_ERR_CAPACITY, "grouped GEMM grid too large");
        hipLaunchKernelGGL((grouped_gemm_ring_kernel<SWIGLU>), dim3(static_cast<unsigned>(ring_blocks)),
                           dim3(kRingThreads), 0, stream, p);
        return check_launch("grouped_gemm_ring_kernel");
    }
    if (blocks > INT32_MAX) return fail(MOE_ERR_CAPACITY, "grouped GEMM grid too large");
    hipLaunchKernelGGL((grouped_gemm_kernel<BM, BN, WAVES_M, WAVES_N, SWIGLU>),
                       dim3(static_cast<unsigned>(blocks)), dim3(kGemmThreads), 0, stream, p);
    return check_launch("grouped_gemm_kernel");
}

int launch_grouped_gemm(const uint16_t* a, const uint16_t* b, uint16_t* c, const int32_t* offsets,
                        int64_t rows, int64_t n, int64_t k, int experts, hipStream_t stream) {
    GemmParams p{};
    p.rows = rows;
    p.a = a;
    p.b = b;
    p.c = c;
    p.offsets = offsets;
    p.k = k;
    p.nb = n;
    p.n_out = n;
    p.ldc = n;
    p.experts = experts;
    return launch_gemm_t<256, 256, 2, 2, false>(p, rows, stream);
}

int launch_gateup_swiglu(const uint16_t* a, const uint16_t* gate_up, uint16_t* act,
                         const int32_t* offsets, int64_t rows, int64_t hidden,
                         int64_t intermediate, int experts, hipStream_t stream) {
    GemmParams p{};
    p.rows = rows;
    p.a = a;
    p.b = gate_up;
    p.c = act;
    p.offsets = offsets;
    p.k = hidden;
    p.nb = 2 * intermediate;
    p.n_out = intermediate;
    p.ldc = intermediate;
    p.experts = experts;
    return launch_gemm_t<256, 256, 2, 2, true>(p, rows, stream);
}

}  // namespace moe
