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
//  * Fast path (K % 64 == 0, the block's shapes): ring_tile / grouped_gemm_persistent_kernel
//    below -- 256 x 256 tiles on four wavefronts of 128 x 128 (16x16x32 MFMAs),
//    direct-to-LDS buffer loads of whole 128-byte lines into an LDS ring of
//    64-k stages, MFMAs interleaved with fragment reads and loads, XCD-aware
//    rounds of full row tiles with the experts' short last row tiles carried
//    beside them; 32- and 64-column tiles for decode-sized launches.
//  * Generic path (any K % 8 == 0): grouped_gemm_kernel -- global -> register ->
//    LDS double buffering with one barrier per 64-wide k-step; LDS rows are 128
//    bytes with 16-byte chunks XOR-swizzled per row (swz).
//  * Tile schedule is built on the device from offsets: expert e contributes
//    ceil(span_e/256) row tiles per column tile (0 for an empty expert). No
//    offsets are read on the host: the generic grid is an upper bound whose
//    surplus workgroups exit at once, and the persistent grid is one workgroup
//    per CU.
//  * Every output element is one MFMA chain in ascending k with one fp32
//    accumulator, whichever path and tile shape computes it.
#include <atomic>
#include <type_traits>
#include <utility>

#include "lds_ring.h"
#include "moe_common.h"

namespace moe {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kGemmThreads = 256;
constexpr int kBK = 64;  // k-step: one 128-byte LDS row

struct GemmParams {
    const uint16_t* a;        // [R, K], or with a_rows the [a_src_rows, K] rows they index
    const uint16_t* b;        // [E, NB, ldb]: K values per row, rows ldb apart (NB = N, or 2I for gate/up)
    uint16_t* c;              // [R, ldc]
    const int32_t* offsets;   // [E + 1]
    int64_t k;                // reduction length (H or I)
    int64_t ldb;              // elements from one row of B to the next (>= k)
    int64_t nb;               // rows of one expert's B
    int64_t n_out;            // output columns (N, or I for gate/up)
    int64_t ldc;
    int64_t rows;             // rows of A and C; spans are clamped to it
    int experts;
    int n_tiles;              // output column tiles
    // Gathered A (gate/up GEMM of the ring kernels only): row r of the
    // product reads row a_rows[r] of `a` (zero when negative); null: row r.
    const int32_t* a_rows;
    int64_t a_src_rows;
};

// A buffer offset past every buffer's range (buffers hold at most 2 GiB): the
// load returns zero and moves no data.
constexpr uint32_t kOutOfRange = 0x80000000u;

// Expert e's first row and row count from the offsets, clamped to [0, rows].
// The offsets are read from the caller's device memory: values past the
// buffer (a caller's mistake: counts that disagree with the rows) would
// otherwise size the persistent kernels' tile walks (garbage counts once made
// one launch walk empty tiles for a second). Valid offsets are unchanged.
__device__ __forceinline__ void expert_rows(const GemmParams& p, int e, int& off, int& span) {
    const int64_t lo = min(max(static_cast<int64_t>(p.offsets[e]), int64_t{0}), p.rows);
    const int64_t hi = min(max(static_cast<int64_t>(p.offsets[e + 1]), lo), p.rows);
    off = static_cast<int>(lo);
    span = static_cast<int>(hi - lo);
}

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
    const uint16_t* b_expert = p.b + static_cast<int64_t>(expert) * p.nb * p.ldb;
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
        b_src[i] = b_expert + (ok ? brow : 0) * p.ldb + c * 8;
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
// Fast path (K % 64 == 0): 256 x 256 output tiles computed by four wavefronts
// (one per SIMD), each owning 128 x 128 (or (TM/2) x (BNT/2) for the short last
// row tile of an expert, the split tail pieces and decode tiles) as a grid of
// 16 x 16 blocks on v_mfma_f32_16x16x32_bf16.
//
//  * Operands reach LDS through direct-to-LDS buffer loads
//    (buffer_load_dwordx4 ... lds). One wavefront load moves 8 rows of 128
//    bytes (64 k), lane l landing at byte 16*l, i.e. row l/8, physical chunk
//    l%8, so it fetches the logical chunk the swizzle maps there. Each group of
//    8 lanes covers one whole 128-byte line: the vector L1 sends full-line
//    requests to L2. With 64-byte (32-k) rows every line took two requests, and
//    the number of requests a CU keeps in flight capped the load rate (measured:
//    the gate/up GEMM 9% and the down GEMM 13% slower). Buffer resources bound
//    the valid bytes: rows past the expert's span and weight rows past the
//    expert read as zero with no per-lane predicate.
//  * LDS holds two rings of 64-k stages: SA stages of A (TM x 128 B each) and
//    SB >= SA stages of B (BNT x 128 B each); a full 256 x 256 tile uses all
//    160 KiB as two A and three B stages, smaller tiles three or four of each.
//    One barrier per stage, placed before the first read of the next stage,
//    waits for that stage and frees the slots of the one just finished. Their
//    refills go out while the next stage computes: A (stage SA on) in its
//    first quarter, B (stage SB on) in its second and third, so every load has
//    at least three quarters of a stage to land, and B loads SB-1 stages.
//  * Rows of 128 bytes hold 8 chunks of 16 bytes; chunk c of row r sits at
//    physical chunk c ^ ((r >> 1) & 7), so 16 lanes reading 16 consecutive rows
//    at one chunk touch 16 distinct (row parity, chunk) bank groups, all 64
//    banks once (conflict free).
//  * Fragment reads of the next 32-k sub-step are spread between the MFMAs of
//    the current one, each well ahead of its use, and a single set of fragment
//    registers is live (see ring_tile). sched_barrier fences pin the order.
//  * The k order of each output's MFMA chain (ascending k in groups of 8, one
//    accumulator) is the same as the generic path, whatever the tile shape.
// ---------------------------------------------------------------------------
constexpr int kStageK = 64;                    // k per LDS stage
constexpr int kRowBytes = kStageK * 2;         // one 128-byte line per row and stage
constexpr int kRingThreads = 256;
constexpr uint32_t kRingBytes = 160 * 1024;    // all of a gfx950 CU's LDS
// Ring depths for stages of a_stage (A) and b_stage (B) bytes in `bytes` of
// LDS. When three or more whole stages fit, both rings get that many (at most
// 4): small tiles compute a stage in a few hundred cycles, so A needs the same
// lead as B. Otherwise (the 256 x 256 tile) A gets two stages and B as many as
// fit beside them.
constexpr int ring_equal_stages(uint32_t a_stage, uint32_t b_stage, uint32_t bytes, int cap = 4) {
    const int fit = static_cast<int>(bytes / (a_stage + b_stage));
    return fit < cap ? fit : cap;
}
constexpr int ring_b_stages(uint32_t a_stage, uint32_t b_stage, uint32_t bytes, int cap = 4) {
    if (ring_equal_stages(a_stage, b_stage, bytes, cap) >= 3) return ring_equal_stages(a_stage, b_stage, bytes, cap);
    const int fit = bytes < 2 * a_stage ? 0 : static_cast<int>((bytes - 2 * a_stage) / b_stage);
    return fit < cap ? fit : cap;
}
constexpr int ring_a_stages(uint32_t a_stage, uint32_t b_stage, uint32_t bytes, int cap = 4) {
    if (ring_equal_stages(a_stage, b_stage, bytes, cap) >= 3) return ring_equal_stages(a_stage, b_stage, bytes, cap);
    const int sb = ring_b_stages(a_stage, b_stage, bytes, cap);
    const int fit = static_cast<int>((bytes - sb * b_stage) / a_stage);
    return fit < sb ? fit : sb;
}

__device__ __forceinline__ int ring_key(int row) { return (row >> 1) & 7; }

// silu(g) * u for the fused epilogue: hardware exp2 and reciprocal
// (v_exp_f32, v_rcp_f32; about 1 ulp each), g and u already rounded to bf16.
__device__ __forceinline__ float swiglu_fast(float g, float u) {
    const float e = __builtin_amdgcn_exp2f(-g * 1.4426950408889634f);
    return (g * u) * __builtin_amdgcn_rcpf(1.0f + e);
}

// The ring's shape and direct-to-LDS loads for one tile: rows [row0,
// row0 + TMR) of one expert (clamped to row_end) by BNT weight rows from
// output column col0, in the first LDS_BYTES of `lds`, at most MAXS stages
// deep. The four waves split the tile as (4/WC) row blocks x WC column blocks.
template <int TMR, int BNT, bool SWIGLU, uint32_t LDS_BYTES, int WC = 2, int MAXS = 4, bool GATHER = false>
struct RingOps {
    static_assert(!GATHER || SWIGLU, "only the gate/up GEMM gathers its rows");
    static constexpr int WAVES = kRingThreads / kWave;
    static constexpr int TM = TMR;
    static constexpr int WTM = TM / (WAVES / WC);  // the four waves as (4/WC) x WC
    static constexpr int WTN = BNT / WC;
    static constexpr int FA = WTM / 16;       // 16-row A fragments per wave
    static constexpr int FB = WTN / 16;       // 16-row B fragments per wave
    static constexpr int A_LOADS = TM / 8 / WAVES;    // loads of 8 rows x 128 B per wave and stage
    static constexpr int B_LOADS = BNT / 8 / WAVES;
    static constexpr int LOADS = A_LOADS + B_LOADS;
    static constexpr uint32_t A_STAGE = TM * kRowBytes;   // bytes of one stage of A
    static constexpr uint32_t B_STAGE = BNT * kRowBytes;  // bytes of one stage of B
    static constexpr int SB = ring_b_stages(A_STAGE, B_STAGE, LDS_BYTES, MAXS);
    static constexpr int SA = ring_a_stages(A_STAGE, B_STAGE, LDS_BYTES, MAXS);
    static constexpr uint32_t B_BASE = SA * A_STAGE;      // B stages follow the A stages
    static constexpr uint32_t FRAG = 16 * kRowBytes;      // bytes between 16-row fragments
    static_assert(A_LOADS >= 1 && B_LOADS >= 1 && FA >= 1 && FB >= 2, "tile shape");
    static_assert(!SWIGLU || FB % 2 == 0, "gate/up pairing needs an even fragment count");
    static_assert(SA >= 2 && SA <= SB && SA * A_STAGE + SB * B_STAGE <= LDS_BYTES, "ring does not fit");
    // Loads complete in order. Each stage's window issues A (stage SA on) and
    // then B (stage SB on). Before stage u+1 is read, its newest loads are its
    // A loads when SB > SA (its B loads went out SB-SA windows earlier), with
    // one window's B loads and SA-2 whole windows younger; when SB == SA they
    // are its B loads, with SA-2 whole windows younger.
    static constexpr int VM_STEADY = (SB > SA ? B_LOADS : 0) + (SA - 2) * LOADS;
    static constexpr int VM_FIRST = (SB > SA ? B_LOADS : 0) + (SA - 1) * LOADS;
    static_assert(VM_FIRST < 64, "in-flight loads fit the vmcnt field");
    static_assert((FA - 1) * FRAG < 65536 && (FB - 1) * FRAG < 65536, "fragment offsets fit the instruction offset");
    __amdgpu_buffer_rsrc_t rsrc_a, rsrc_b;
    uint32_t a_off[A_LOADS], b_off[B_LOADS];
    char* lds;
    int wave;

    // A tile's two buffer resources and its per-lane A offsets. B: the
    // expert's weight rows from the tile's first column on (so the per-lane B
    // offsets below do not depend on the tile). A: the tile's rows of A, read
    // at offsets relative to its first row; or, gathered (gate/up with
    // a_rows), the whole source at each row's own offset. Rows past the tile
    // (or the expert), and gathered rows mapped to a negative index, read as
    // zero (out of the buffer's range). Load l of a stage covers LDS rows
    // (wave * X_LOADS + l) * 8 + lane / 8.
    struct Rsrc {
        __amdgpu_buffer_rsrc_t a, b;
        uint32_t a_off[A_LOADS];
    };
    // GATHER with `offsets` false leaves a_off to the caller (its table loads
    // belong where the tile's prologue is issued, see ring_tile's a_carry).
    static __device__ __forceinline__ Rsrc tile_rsrc(const GemmParams& p, int expert, int64_t col0, int64_t row0,
                                                     int64_t row_end, bool offsets = true) {
        const int64_t K = p.k;
        const int lane = threadIdx.x & 63;
        const int wave_ = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
        const int lrow = lane >> 3;
        const int pchunk = lane & 7;
        Rsrc r;
        // The expert's weight rows from col0 on. Every caller has col0 < n_out
        // <= nb (ring_locate drops pieces at or past n_out; whole and decode
        // tiles start below n_out), so the range cannot wrap. A clamp here at
        // zero rows costs the gate/up persistent kernel 28 VGPRs, and at 4096
        // tokens, H=4096, I=14336, 8 experts, top-2, 14% of gate/up's time and
        // 10% of down's.
        r.b = make_rsrc(p.b + (static_cast<int64_t>(expert) * p.nb + col0) * p.ldb,
                        static_cast<uint32_t>((p.nb - col0) * p.ldb * 2));
        if constexpr (GATHER) {
            r.a = make_rsrc(p.a, static_cast<uint32_t>(p.a_src_rows * K * 2));
            if (!offsets) return r;
            // All table loads first, at in-range indices, and the row bound
            // after: a load under a branch gets a wait of its own, and every
            // wait also waits for the ring loads already in flight.
            int src[A_LOADS];
#pragma unroll
            for (int i = 0; i < A_LOADS; ++i)
                src[i] = p.a_rows[min(row0 + (wave_ * A_LOADS + i) * 8 + lrow, p.rows - 1)];
#pragma unroll
            for (int i = 0; i < A_LOADS; ++i) {
                const int rr = (wave_ * A_LOADS + i) * 8 + lrow;
                const int s = row0 + rr < row_end ? src[i] : -1;
                r.a_off[i] = s >= 0 && s < p.a_src_rows
                                 ? static_cast<uint32_t>((s * K + (pchunk ^ ring_key(rr)) * 8) * 2)
                                 : kOutOfRange;
            }
        } else {
            const int64_t a_rows = min<int64_t>(row_end - row0, TM);
            r.a = make_rsrc(p.a + row0 * K, static_cast<uint32_t>(a_rows * K * 2));
#pragma unroll
            for (int i = 0; i < A_LOADS; ++i) {
                const int rr = (wave_ * A_LOADS + i) * 8 + lrow;
                r.a_off[i] = static_cast<uint32_t>((rr * K + (pchunk ^ ring_key(rr)) * 8) * 2);
            }
        }
        return r;
    }

    __device__ __forceinline__ RingOps(const GemmParams& p, char* lds_, int expert, int64_t col0,
                                       int64_t row0, int64_t row_end)
        : RingOps(p, lds_, tile_rsrc(p, expert, col0, row0, row_end)) {}

    // From a tile's resources already formed: a chained next tile's, or a
    // gathered tile's whose A offsets were carried in.
    __device__ __forceinline__ RingOps(const GemmParams& p, char* lds_, const Rsrc& res) : lds(lds_) {
        const int lane = threadIdx.x & 63;
        wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
        rsrc_a = res.a;
        rsrc_b = res.b;
        const int lrow = lane >> 3;
        const int pchunk = lane & 7;
#pragma unroll
        for (int i = 0; i < A_LOADS; ++i) a_off[i] = res.a_off[i];
#pragma unroll
        for (int i = 0; i < B_LOADS; ++i) {
            const int r = (wave * B_LOADS + i) * 8 + lrow;
            int64_t brow;
            if constexpr (SWIGLU) {
                // Wave column wc owns gate columns [wc*WTN/2, (wc+1)*WTN/2) of the
                // tile and the matching up rows (I further on).
                const int wcol = r / WTN, w = r % WTN;
                static constexpr int HALF = WTN / 2;
                const int64_t col = wcol * HALF + (w % HALF);  // from the tile's first column
                brow = (w < HALF) ? col : p.n_out + col;
            } else {
                brow = r;
            }
            b_off[i] = static_cast<uint32_t>((brow * p.ldb + (pchunk ^ ring_key(r)) * 8) * 2);
        }
    }
    // Load l of stage kt into ring slot st, of A and of B (of this tile, or of
    // the tile whose resources are given).
    __device__ __forceinline__ void issue_a(int kt, int st, int l) const { issue_a(rsrc_a, kt, st, l, a_off[l]); }
    __device__ __forceinline__ void issue_b(int kt, int st, int l) const { issue_b(rsrc_b, kt, st, l); }
    __device__ __forceinline__ void issue_a(__amdgpu_buffer_rsrc_t r, int kt, int st, int l, uint32_t off) const {
        dma16(r, lds + st * A_STAGE + (wave * A_LOADS + l) * 1024, off, static_cast<uint32_t>(kt) * kRowBytes);
    }
    __device__ __forceinline__ void issue_b(__amdgpu_buffer_rsrc_t r, int kt, int st, int l) const {
        dma16(r, lds + B_BASE + st * B_STAGE + (wave * B_LOADS + l) * 1024, b_off[l],
              static_cast<uint32_t>(kt) * kRowBytes);
    }
    // The windows before stage 0, in the steady-state order (A of stage
    // v+SA, then B of stage v+SB, for v = -SB .. -1; only v = -1 when `last`).
    // Stage s goes to slots (a0 + s) % SA and (b0 + s) % SB. Stages past the
    // last are loaded as the last one again, so every window issues the same
    // loads and the vmcnt accounting stays uniform.
    __device__ __forceinline__ void prologue(int k_steps, int a0 = 0, int b0 = 0, bool last = false) const {
#pragma unroll
        for (int v = -SB; v < 0; ++v) {
            if (last && v != -1) continue;
            if (v + SA >= 0) {
                const int st = a0 + v + SA >= SA ? a0 + v : a0 + v + SA;
#pragma unroll
                for (int l = 0; l < A_LOADS; ++l) issue_a(min(v + SA, k_steps - 1), st, l);
            }
            const int st = b0 + v + SB >= SB ? b0 + v : b0 + v + SB;
#pragma unroll
            for (int l = 0; l < B_LOADS; ++l) issue_b(min(v + SB, k_steps - 1), st, l);
        }
    }

};

// No work between a tile's k-loop and its epilogue.
struct NoHook {
    __device__ void operator()() const {}
};

// One output tile on v_mfma_f32_16x16x32_bf16 (shape as in RingOps). A 64-k
// stage is two 32-k sub-steps; in each, every wave multiplies its (WTM/16) x
// (WTN/16) grid of 16x16 blocks with one MFMA each while it reads the
// fragments of the next sub-step. The 16x16x32 form sustains a higher clock
// than 32x32x16 under the power limit (measured on MI355X: 1.91 vs 1.66 GHz
// with the same read and load mix), so it moves the same FLOPs about 10%
// faster.
//
// own_prologue: issue the prologue loads here (else a previous call's hook
// issued them). wait_all: a previous epilogue's stores may be in flight, and
// on gfx9 stores share vmcnt with loads, so wait for every outstanding access
// before the first read instead of counting loads. hook: runs once the
// k-loop is done and every wave has finished with the ring (it may refill
// LDS), before the epilogue.
//
// Chaining (persistent kernels): the ring's stage s sits in slots (sa0 + s) % SA
// and (sb0 + s) % SB. With `chain`, the windows that would reload this tile's
// last stage instead load the next tile's first stages (resources `next`, a
// tile of the same shape and k) into the slots that follow, so the next tile
// starts at slots (sa0 + k_steps) % SA and (sb0 + k_steps) % SB and its hook
// only issues the prologue's last window. Requires k_steps >= SB.
template <int TMR, int BNT, bool SWIGLU, uint32_t LDS_BYTES, typename Hook = NoHook, int WC = 2, int MAXS = 4,
          bool GATHER = false>
__device__ __forceinline__ void ring_tile(const GemmParams& p, char* lds, int expert, int64_t col0,
                                          int64_t row0, int64_t row_end, bool own_prologue = true,
                                          bool wait_all = false, const Hook& hook = Hook{}, int sa0 = 0, int sb0 = 0,
                                          bool chain = false,
                                          typename RingOps<TMR, BNT, SWIGLU, LDS_BYTES, WC, MAXS, GATHER>::Rsrc next = {},
                                          const uint32_t* a_carry = nullptr) {
    using R = RingOps<TMR, BNT, SWIGLU, LDS_BYTES, WC, MAXS, GATHER>;
    constexpr int WTM = R::WTM, WTN = R::WTN, FA = R::FA, FB = R::FB;
    constexpr int A_LOADS = R::A_LOADS, B_LOADS = R::B_LOADS;
    constexpr int SA = R::SA, SB = R::SB;
    constexpr uint32_t A_STAGE = R::A_STAGE, B_STAGE = R::B_STAGE, B_BASE = R::B_BASE, FRAG = R::FRAG;
    constexpr int VM_STEADY = R::VM_STEADY, VM_FIRST = R::VM_FIRST;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / WC;
    const int wn = wave % WC;
    const int64_t K = p.k;
    // Gathered rows: the tile's A offsets were formed where its prologue was
    // issued (a_carry). Forming them here would load the row table after the
    // ring's loads, and the first refill's wait for it would drain the ring.
    typename R::Rsrc cur = R::tile_rsrc(p, expert, col0, row0, row_end, !GATHER);
    if constexpr (GATHER) {
#pragma unroll
        for (int i = 0; i < R::A_LOADS; ++i) cur.a_off[i] = a_carry[i];
    }
    const R ops(p, lds, cur);

    // Per-lane fragment addresses: lane l reads row (l%16) of a fragment at k
    // chunk l/16 of the sub-step (all 32 k of it in one 16-byte read). Fragments
    // 16 rows apart share the swizzle key, so the fragment only adds a constant
    // (an instruction offset); each ring slot and sub-step has its own base.
    const int frag_row = lane & 15;
    const int chunk = lane >> 4;
    const int ar = wm * WTM + frag_row;
    const int br = wn * WTN + frag_row;
    uint32_t va[2], vb[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        va[h] = static_cast<uint32_t>(ar * kRowBytes + (((4 * h + chunk) ^ ring_key(ar)) << 4));
        vb[h] = B_BASE + static_cast<uint32_t>(br * kRowBytes + (((4 * h + chunk) ^ ring_key(br)) << 4));
    }

    floatx4 acc[FA][FB];
#pragma unroll
    for (int i = 0; i < FA; ++i)
#pragma unroll
        for (int j = 0; j < FB; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[i][j][r] = 0.0f;

    auto read_at = [&](uint32_t base, int idx) {
        return *reinterpret_cast<const bf16x8_t*>(lds + base + idx * FRAG);
    };
    auto fence = [] { __builtin_amdgcn_sched_barrier(0); };

    // Weights fragment as src0, activations as src1: the 16x16 result comes out
    // transposed, so lane l holds row l%16 and the four consecutive columns
    // 4*(l/16) + 0..3 (packed 8-byte stores).
    //
    // One set of fragments (FA A + FB B) is live. A 32-k sub-step runs in two
    // halves: B fragments [0, FB/2) with every A fragment, then [FB/2, FB).
    // Inside a half the MFMAs go A fragment by A fragment with the B fragments
    // in snake order (forward for even A fragments, backward for odd ones), so
    // consecutive MFMAs change one operand, never both: the kernel is power-
    // limited, and the fewer operand bits toggle, the higher the clock it holds
    // (measured on MI355X: 0.5-1.2% faster than restarting each row at B 0).
    // During the first half this sub-step's B fragments [FB/2, FB) are read
    // (their previous values were last used by the previous second half);
    // during the second half the next sub-step's A fragment i is read right
    // after its last MFMA, and its B fragments [0, FB/2). Every read has at
    // least about a quarter of a sub-step of MFMA work before its first use.
    constexpr int HB = FB / 2;
    constexpr int HM = FA * HB;        // MFMAs per half sub-step
    static_assert(HB >= 1 && HM >= HB, "half-step shape");
    // MFMA slots of the B fragment reads: this sub-step's fragment HB+b in
    // the first half, the next sub-step's fragment b in the second, one every
    // other MFMA (all at the last MFMA of a half that has fewer).
    constexpr auto first_read_slot = [](int b) constexpr { return 2 * b < HM - 1 ? 2 * b : HM - 1; };
    constexpr auto second_read_slot = [](int b) constexpr { return 2 * b + 1 < HM - 1 ? 2 * b + 1 : HM - 1; };
    constexpr int LOADS = A_LOADS + B_LOADS;
    // Slots of a window's loads: A in its first quarter and B over its second
    // and third (gate/up) or second to fourth (plain GEMM: C4's down GEMM 1%
    // faster, the gate/up GEMM 1% slower that way) when they fit one per MFMA;
    // otherwise all spread evenly, A first (small tiles with few MFMAs per
    // quarter). Either way a window issues its A loads before its B loads.
    constexpr bool kQuarters = A_LOADS <= HM && B_LOADS <= 2 * HM;
    bf16x8_t fa[FA], fb[FB];
    // The refills of one window, at the slots above.
    struct Refill {
        int kt_a, slot_a, kt_b, slot_b;
        __amdgpu_buffer_rsrc_t ra, rb;  // this tile's or (chained) the next tile's
        bool a_next;                    // A loads of the next tile (its own offsets when gathered)
    };
    auto refill_at = [&](auto g_c, const Refill& r) {
        constexpr int g = decltype(g_c)::value;  // MFMA slot in the window
        static_for<A_LOADS>([&](auto l_c) {
            constexpr int l = decltype(l_c)::value;
            constexpr int slot = kQuarters ? l * HM / A_LOADS : l * 4 * HM / LOADS;
            if constexpr (slot == g)
                ops.issue_a(r.ra, r.kt_a, r.slot_a, l, GATHER && r.a_next ? next.a_off[l] : ops.a_off[l]);
        });
        static_for<B_LOADS>([&](auto l_c) {
            constexpr int l = decltype(l_c)::value;
            constexpr int slot = kQuarters ? HM + l * (SWIGLU ? 2 : 3) * HM / B_LOADS : (A_LOADS + l) * 4 * HM / LOADS;
            if constexpr (slot == g) ops.issue_b(r.rb, r.kt_b, r.slot_b, l);
        });
    };
    // First half: B [0, HB) x A, reading this sub-step's B [HB, FB) at `bh`.
    // Quarter q >= 0 of a window carries its share of the refills.
    auto first_half = [&](uint32_t bh, auto q_c, const Refill& rf) {
        constexpr int q = decltype(q_c)::value;
        static_for<HM>([&](auto m_c) {
            constexpr int m = decltype(m_c)::value;
            constexpr int i = m / HB, j = (i % 2) ? HB - 1 - m % HB : m % HB;  // snake order
            if constexpr (q >= 0) refill_at(std::integral_constant<int, q * HM + m>{}, rf);
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fb[j], fa[i], acc[i][j], 0, 0, 0);
            static_for<HB>([&](auto b_c) {
                constexpr int b = decltype(b_c)::value;
                if constexpr (first_read_slot(b) == m) fb[HB + b] = read_at(bh, HB + b);
            });
            fence();
        });
    };
    // Second half: B [HB, FB) x A, reading the next sub-step's A and B [0, HB)
    // at (an, bn) unless `last`.
    auto second_half = [&](uint32_t an, uint32_t bn, auto last_c, auto q_c, const Refill& rf) {
        constexpr bool last = decltype(last_c)::value;
        constexpr int q = decltype(q_c)::value;
        static_for<HM>([&](auto m_c) {
            constexpr int m = decltype(m_c)::value;
            constexpr int i = m / HB, j = HB + ((i % 2) ? HB - 1 - m % HB : m % HB);  // snake order
            if constexpr (q >= 0) refill_at(std::integral_constant<int, q * HM + m>{}, rf);
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fb[j], fa[i], acc[i][j], 0, 0, 0);
            if constexpr (!last) {
                static_for<HB>([&](auto b_c) {
                    constexpr int b = decltype(b_c)::value;
                    if constexpr (second_read_slot(b) == m) fb[b] = read_at(bn, b);
                });
                if constexpr (m % HB == HB - 1) fa[i] = read_at(an, i);
            }
            fence();
        });
    };

    const int k_steps = static_cast<int>(K / kStageK);
    if (own_prologue) ops.prologue(k_steps, sa0, sb0);
    if (wait_all)
        wait_vm_lgkm<0>();
    else
        wait_vm_lgkm<VM_FIRST>();
    ring_barrier();
    fence();
    // Sub-step 0's fragments, in the order the second half reads them.
    const uint32_t a_first = sa0 * A_STAGE, b_first = sb0 * B_STAGE;
    static_for<HM>([&](auto m_c) {
        constexpr int m = decltype(m_c)::value;
        constexpr int i = m / HB;
        static_for<HB>([&](auto b_c) {
            constexpr int b = decltype(b_c)::value;
            if constexpr (second_read_slot(b) == m) fb[b] = read_at(vb[0] + b_first, b);
        });
        if constexpr (m % HB == HB - 1) fa[i] = read_at(va[0] + a_first, i);
    });
    // Stage 0 up to its last quarter, then per stage u: [barrier] the last
    // quarter of stage u (reading stage u+1), then the first three quarters of
    // stage u+1; this window refills the slots stage u just freed.
    using NoLoads = std::integral_constant<int, -1>;
    using More = std::false_type;
    const Refill none{0, 0, 0, 0, ops.rsrc_a, ops.rsrc_b, false};
    first_half(vb[0] + b_first, NoLoads{}, none);
    second_half(va[1] + a_first, vb[1] + b_first, More{}, NoLoads{}, none);
    first_half(vb[1] + b_first, NoLoads{}, none);
    int sa = sa0, sb = sb0;  // ring slots of stage u
    // The window after the barrier that precedes stage u+1's first read.
    auto window = [&](const Refill& rf, int na, int nb) {
        const uint32_t a0 = va[0] + na * A_STAGE, a1 = va[1] + na * A_STAGE;
        const uint32_t b0 = vb[0] + nb * B_STAGE, b1 = vb[1] + nb * B_STAGE;
        fence();
        // Stage u+1 has landed, and every read of stage u (the last in the
        // quarter just done) has returned.
        wait_vm_lgkm<VM_STEADY>();
        ring_barrier();
        fence();
        second_half(a0, b0, More{}, std::integral_constant<int, 0>{}, rf);
        first_half(b0, std::integral_constant<int, 1>{}, rf);
        second_half(a1, b1, More{}, std::integral_constant<int, 2>{}, rf);
        first_half(b1, std::integral_constant<int, 3>{}, rf);
    };
    // With one wave per SIMD, every scalar instruction between two MFMAs takes
    // an issue slot of the wave, and a burst of them before the barrier left
    // the MFMA pipe idle (the refill's resource selects: about 40 scalar
    // instructions per stage). So the stages whose refills come from this
    // tile, at stages u+SA and u+SB, run in a loop of their own without
    // selects; only the last SB-1 windows (clamped stages, or the next tile's
    // first stages when chained) compute their refill in full.
    int u = 0;
    for (; u < k_steps - SB; ++u) {
        const int na = sa + 1 == SA ? 0 : sa + 1;
        const int nb = sb + 1 == SB ? 0 : sb + 1;
        window(Refill{u + SA, sa, u + SB, sb, ops.rsrc_a, ops.rsrc_b, false}, na, nb);
        sa = na;
        sb = nb;
    }
    for (; u + 1 < k_steps; ++u) {
        const int na = sa + 1 == SA ? 0 : sa + 1;
        const int nb = sb + 1 == SB ? 0 : sb + 1;
        // Stages past this tile's last: the next tile's first ones when
        // chained, else this tile's last one again.
        const bool a_next = chain && u + SA >= k_steps;
        const bool b_next = chain && u + SB >= k_steps;
        window(Refill{a_next ? u + SA - k_steps : min(u + SA, k_steps - 1), sa,
                      b_next ? u + SB - k_steps : min(u + SB, k_steps - 1), sb,
                      a_next ? next.a : ops.rsrc_a, b_next ? next.b : ops.rsrc_b, a_next},
               na, nb);
        sa = na;
        sb = nb;
    }
    second_half(0u, 0u, std::true_type{}, NoLoads{}, none);
    wait_vm_lgkm<0>();
    if constexpr (!std::is_same_v<Hook, NoHook>) {
        ring_barrier();
        hook();
    }

    // Epilogue. Lane l holds, in each 16 x 16 block, row l%16 and columns
    // 4*(l/16) + 0..3. For each pair of neighbouring blocks a
    // v_permlane16_swap per dword exchanges data between lane rows 0<->1 and
    // 2<->3 (lanes 16 apart hold the same output row), after which lane row g
    // holds the 8 consecutive columns 8 * (0, 2, 1, 3)[g] of the pair's 32:
    // one 16-byte store where there were two 8-byte ones, and each store
    // instruction writes 64 contiguous bytes per output row instead of 32.
    // Each row of accumulators is first moved to VGPRs through an empty asm
    // operand: without it the register allocator shapes the accumulators' AGPR
    // assignment after the epilogue's register pairs and copies them inside the
    // k-loop on every step. The swaps run on every lane (before the row test).
    const int lane_row = lane >> 4;
    const int col4 = 4 * lane_row;
    const int col8 = 8 * (((lane_row & 1) << 1) | (lane_row >> 1));
    // Blocks b0 and b0 + 1 of a row fragment, as four bf16 each, into crow from
    // column `base` (the first column of block b0).
    auto store_pair = [&](uint16_t* crow, bool row_ok, int64_t base, uint2 x, uint2 y) {
        const auto s0 = __builtin_amdgcn_permlane16_swap(x.x, y.x, false, false);
        const auto s1 = __builtin_amdgcn_permlane16_swap(x.y, y.y, false, false);
        const int64_t col = base + col8;
        if (row_ok && col < p.n_out)
            *reinterpret_cast<uint4*>(crow + col) = make_uint4(s0[0], s1[0], s0[1], s1[1]);
    };
    auto store_one = [&](uint16_t* crow, bool row_ok, int64_t base, uint2 x) {
        const int64_t col = base + col4;
        if (row_ok && col < p.n_out) *reinterpret_cast<uint2*>(crow + col) = x;
    };
    constexpr int OUT_BLOCKS = SWIGLU ? FB / 2 : FB;  // 16-column output blocks per wave
#pragma unroll
    for (int i = 0; i < FA; ++i) {
#pragma unroll
        for (int j = 0; j < FB; ++j) asm volatile("" : "+v"(acc[i][j]));
        const int64_t grow = row0 + wm * WTM + i * 16 + (lane & 15);
        const bool row_ok = grow < row_end;
        uint16_t* crow = p.c + (row_ok ? grow : row0) * p.ldc;
        const int64_t first_col = col0 + wn * (SWIGLU ? WTN / 2 : WTN);
        uint2 out[OUT_BLOCKS];
#pragma unroll
        for (int j = 0; j < OUT_BLOCKS; ++j) {
            if constexpr (SWIGLU) {
                float act[4];
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const uint32_t gu = pack_bf16x2(acc[i][j][t], acc[i][j + FB / 2][t]);
                    act[t] = swiglu_fast(__uint_as_float(gu << 16), __uint_as_float(gu & 0xffff0000u));
                }
                out[j] = make_uint2(pack_bf16x2(act[0], act[1]), pack_bf16x2(act[2], act[3]));
            } else {
                out[j] = make_uint2(pack_bf16x2(acc[i][j][0], acc[i][j][1]), pack_bf16x2(acc[i][j][2], acc[i][j][3]));
            }
        }
#pragma unroll
        for (int j = 0; j + 1 < OUT_BLOCKS; j += 2) store_pair(crow, row_ok, first_col + j * 16, out[j], out[j + 1]);
        if constexpr (OUT_BLOCKS % 2 == 1)
            store_one(crow, row_ok, first_col + (OUT_BLOCKS - 1) * 16, out[OUT_BLOCKS - 1]);
    }
}

// Work list, built on the device from offsets (the same in every workgroup).
// Row tiles of more than 128 rows form phase 1: they cost about the same and
// are compute-bound. The short last row tile of an expert (at most 128 rows)
// forms phase 2: it reads a whole 256-row weight slab for a quarter or half of
// the arithmetic, so its cost is streaming that slab at one CU's request rate
// (about half of a phase-1 tile: 49 vs 101 us at H=4096, I=14336), and many of
// them at once are HBM-bound. With balanced row tiles (ring_table) only experts
// of at most 128 rows have a phase-2 tile.
//
// The grid (G workgroups, workgroup i on XCD i % 8) walks virtual workgroups
// q = blockIdx.x, blockIdx.x + G, ..., i.e. in rounds of G. Phase 1 is cut
// into 8 contiguous ranges, one per XCD, and each XCD runs its range in order,
// cpr tiles per round, so the CUs of an XCD run neighbouring tiles (same
// expert and column tile, adjacent row tiles) in lockstep and share A and B
// k-slices in L2. The other slots of the rounds take one or two phase-2 tiles
// each, so their weight streaming runs beside the compute-bound tiles, within
// the HBM headroom, instead of after them at the HBM limit. The round count is
// the minimum for phase 1, plus one when more than one phase-2 tile per
// workgroup would otherwise be left over; leftover phase-2 tiles run after the
// rounds, one per slot. Inside a phase, tiles go expert by expert, column tile
// by column tile, row tiles fastest. Measured at H=4096, I=14336, 4096 tokens:
// the short tiles took 250 us after the 1418 us of phase 1 when run last.
//
// For the plain GEMM a short last round (at most half of the slots busy) of
// phase 1 (when there is no phase 2) or of the leftover phase-2 tiles is split
// into 128-column pieces, and leftover phase-2 tiles into 64-column quarters
// when at most a quarter of the slots would be busy. When phase 1 fills at
// most half of the slots of one round beside a phase 2, its tiles run as
// 128-column halves (the two halves of a tile in neighbouring slots of one
// XCD, sharing the A slab in L2): at H=1024, I=2048, E=16, 4096 tokens the
// down GEMM's 128 full tiles otherwise took one whole K=2048 chain on half of
// the CUs. Every tile or piece runs its whole k chain in order on one
// workgroup, so results do not depend on the schedule or on G.
struct RingPhase {
    int count;   // tiles
    int main;    // tiles mapped XCD-contiguously
    int blocks;  // virtual workgroups of the main part (multiple of 8)
    int pieces;  // split tail pieces (`ways` per split tile)
    int ways;    // 2 (128-column pieces) or 4 (64-column pieces of short tiles)
};

// Short tiles (phase 2) split four ways when that still fits the slots: their
// cost is streaming the weight slab, which more CUs pull faster.
__device__ __forceinline__ RingPhase ring_phase(int count, int grid, bool allow_split, bool short_tiles) {
    RingPhase ph;
    ph.count = count;
    const int rem = count % grid;
    const bool split = allow_split && rem > 0 && 2 * rem <= grid;
    ph.ways = short_tiles && 4 * rem <= grid ? 4 : 2;
    ph.main = split ? count - rem : count;
    ph.blocks = (ph.main + kNumXcd - 1) / kNumXcd * kNumXcd;
    ph.pieces = split ? ph.ways * rem : 0;
    return ph;
}

struct RingPlan {
    int n1;           // phase-1 tiles
    int n2;           // phase-2 tiles
    bool half1;       // phase 1 runs as 128-column halves in the rounds
    int u1;           // phase-1 units of the rounds (tiles, or halves)
    int per1;         // phase-1 tiles per XCD range
    int cpr;          // phase-1 tiles per XCD and round
    int rounds;       // interleaved rounds (0: none)
    int full_rounds;  // rounds that run cpr phase-1 tiles per XCD
    int last_cols;    // phase-1 tiles per XCD in round full_rounds
    int slots;        // phase-2 slots in the rounds
    int carried;      // phase-2 tiles the rounds take (at most two per slot)
    RingPhase rest;   // after the rounds: phase 1 (no phase 2) or the leftover phase-2 tiles
    int virtual_blocks;
};

// grid is a positive multiple of 8.
__device__ __forceinline__ RingPlan ring_plan(int n1, int n2, int grid, bool allow_split) {
    RingPlan pl{};
    pl.n1 = n1;
    pl.n2 = n2;
    pl.half1 = allow_split && n2 > 0 && n1 > 0 && 2 * n1 <= grid;
    pl.u1 = pl.half1 ? 2 * n1 : n1;
    if (n2 > 0 && n1 > 0) {
        pl.per1 = (pl.u1 + kNumXcd - 1) / kNumXcd;
        int rounds = (pl.per1 + grid / kNumXcd - 1) / (grid / kNumXcd);
        if (n2 - 2 * (rounds * grid - kNumXcd * pl.per1) > grid) ++rounds;
        pl.rounds = rounds;
        pl.cpr = (pl.per1 + rounds - 1) / rounds;
        pl.full_rounds = pl.per1 / pl.cpr;
        pl.last_cols = pl.per1 - pl.full_rounds * pl.cpr;
        pl.slots = rounds * grid - kNumXcd * pl.per1;
        pl.carried = min(n2, 2 * pl.slots);
    }
    pl.rest = ring_phase(n2 > 0 ? n2 - pl.carried : n1, grid, allow_split, n2 > 0);
    pl.virtual_blocks = pl.rounds * grid + pl.rest.blocks + pl.rest.pieces;
    return pl;
}

struct RingSlot {
    int phase;  // 0 / 1 for phase 1 / 2; -1: no tile
    int tile;   // index inside the phase of the first tile
    int piece;  // -1; 0 / 1 for the two 128-column halves; 4 + q for 64-column quarter q
    int count;  // tiles tile, tile + 1, ... of this slot (0 to 2)
};

// The tiles of virtual workgroup q.
__device__ __forceinline__ RingSlot ring_slot(const RingPlan& pl, int grid, int q) {
    RingSlot s{-1, 0, -1, 0};
    const int base = pl.rounds * grid;
    if (q < base) {
        // Column j of the XCD's slots, rotated by the round so that the
        // phase-2 slots move to other CUs each round (a CU that always carried
        // them would fall further behind its XCD's lockstep every round).
        const int per_xcd = grid / kNumXcd, r = q / grid, pos = q - r * grid;
        const int j = (pos / kNumXcd + r * (per_xcd - pl.cpr)) % per_xcd;
        const int cols = r < pl.full_rounds ? pl.cpr : (r == pl.full_rounds ? pl.last_cols : 0);
        if (j < cols) {
            const int unit = (pos % kNumXcd) * pl.per1 + r * pl.cpr + j;
            if (unit < pl.u1) s = pl.half1 ? RingSlot{0, unit >> 1, unit & 1, 1} : RingSlot{0, unit, -1, 1};
            return s;
        }
        // A phase-2 slot: its index among the rounds' phase-2 slots, in q order.
        const int per_round = grid - kNumXcd * pl.cpr;
        int idx = r <= pl.full_rounds
                      ? r * per_round
                      : pl.full_rounds * per_round + grid - kNumXcd * pl.last_cols +
                            (r - pl.full_rounds - 1) * grid;
        idx += (j - cols) * kNumXcd + pos % kNumXcd;
        const int lo = static_cast<int>(static_cast<int64_t>(idx) * pl.carried / pl.slots);
        const int hi = static_cast<int>(static_cast<int64_t>(idx + 1) * pl.carried / pl.slots);
        if (lo < hi) s = RingSlot{1, lo, -1, hi - lo};
        return s;
    }
    const int phase = pl.n2 > 0 ? 1 : 0;
    const int first = pl.n2 > 0 ? pl.carried : 0;
    const RingPhase& ph = pl.rest;
    const int v = q - base;
    if (v < ph.blocks) {
        const int per = ph.blocks / kNumXcd;
        const int tile = (v % kNumXcd) * per + v / kNumXcd;
        if (tile < ph.main) s = RingSlot{phase, first + tile, -1, 1};
    } else if (v - ph.blocks < ph.pieces) {
        const int r = v - ph.blocks;
        s = RingSlot{phase, first + ph.main + r / ph.ways, ph.ways == 4 ? 4 + r % 4 : r % 2, 1};
    }
    return s;
}

// The fast-path kernel is persistent: one workgroup per CU walks its virtual
// workgroups and, once a tile's k-loop is done, issues the next tile's first
// stages before running the epilogue, so their latency hides behind the
// epilogue's arithmetic and stores, and the per-workgroup start-up is paid
// once per CU. Tiles are decoded from a per-wave table (lane e = expert e)
// instead of a loop over the offsets per tile. Measured: C3 and C5 expert
// GEMMs 5-11% faster, C4 T=4096 about 1%.
struct RingWork {
    bool valid;
    int expert;
    int variant;  // row tile 256 / 128 / 64 = 0 / 1 / 2; +3 for a 128-column piece, +6 for a 64-column one;
                  // whole 256-column tiles of 32 / 224 / 192 / 160 rows = 9 / 10 / 11 / 12
    int64_t row0, row_end, col0;
};

struct RingTable {
    int off, span, mf, s1, s2, c1, c2;  // lane e: expert e's first row, rows, phase-1 row tiles,
                                        // first tile and tile count in phase 1 and 2
    int n_full, n_part;                 // tiles per phase (uniform)
    bool balanced;                      // phase-1 row tiles of equal height (uniform)
};

__device__ __forceinline__ int wave_inclusive_sum(int x) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
        const int t = __shfl_up(x, d);
        if (lane >= d) x += t;
    }
    return x;
}

// Row tiles: ceil(rows / 256) per expert. Plain: 256-row tiles, the last in
// phase 1 when it has more than 128 rows, else in phase 2. Balanced: an
// expert of more than 128 rows has all its tiles in phase 1, of equal height
// (ring_locate); one of at most 128 rows is a phase-2 tile.
__device__ __forceinline__ RingTable ring_table(const GemmParams& p, bool balanced) {
    RingTable t;
    t.balanced = balanced;
    const int lane = threadIdx.x & 63;
    t.off = 0;
    t.span = 0;
    if (lane < p.experts) expert_rows(p, lane, t.off, t.span);
    const int tiles = (t.span + 255) / 256;
    t.mf = balanced ? (t.span > 128 ? tiles : 0) : t.span / 256 + ((t.span % 256) > 128 ? 1 : 0);
    t.c1 = t.mf * p.n_tiles;
    t.c2 = (tiles - t.mf) * p.n_tiles;
    const int i1 = wave_inclusive_sum(t.c1), i2 = wave_inclusive_sum(t.c2);
    t.s1 = i1 - t.c1;
    t.s2 = i2 - t.c2;
    t.n_full = __builtin_amdgcn_readlane(i1, kWave - 1);
    t.n_part = __builtin_amdgcn_readlane(i2, kWave - 1);
    return t;
}

// Slot -> tile: expert, rows, columns and ring variant.
template <bool SWIGLU>
__device__ __forceinline__ RingWork ring_locate(const GemmParams& p, const RingTable& t, const RingSlot& s) {
    RingWork w{false, 0, 0, 0, 0, 0};
    if (s.phase < 0) return w;
    const int lane = threadIdx.x & 63;
    const int first = s.phase == 0 ? t.s1 : t.s2;
    const int count = s.phase == 0 ? t.c1 : t.c2;
    // The tile's expert: the last one (in order) with tiles in this phase starting at or before it.
    const uint64_t owners = __ballot(lane < p.experts && count > 0 && first <= s.tile);
    if (owners == 0) return w;
    const int e = 63 - __builtin_clzll(owners);
    const int rel = s.tile - __builtin_amdgcn_readlane(first, e);
    const int mf = __builtin_amdgcn_readlane(t.mf, e);
    const int span = __builtin_amdgcn_readlane(t.span, e);
    const int off = __builtin_amdgcn_readlane(t.off, e);
    // Phase 1: the expert's mf row tiles of h rows each (256, or balanced: the
    // multiple of 32 that spreads the rows evenly, 160-256 when mf >= 2); the
    // last may hold fewer. Phase 2: the expert's last tile (at most 128 rows).
    int n_tile, m_tile, h;
    if (s.phase == 0) {
        // The expert's row tiles in groups of at most 8 (of balanced heights),
        // column tiles fastest inside a group, row tiles fastest inside a
        // column. An XCD's round of about 32 neighbouring tiles then spans at
        // most 8 row tiles by 4 or more column tiles, about 12 operand slabs.
        // In plain row-tiles-fastest order an expert of 32 row tiles ran each
        // round as one column tile by 32 row tiles: 33 slabs, and every round
        // streamed the expert's whole A again (H=2048, I=1408, E=64 Zipf:
        // gate/up 2.66 GB and down 1.53 GB fetched per launch, about three
        // times their operands). Experts of at most 8 row tiles keep that
        // order. Each tile still runs its whole k chain on one workgroup.
        const int groups = (mf + 7) / 8;
        const int hg = (mf + groups - 1) / groups;
        const int full = hg * p.n_tiles;  // tiles of a group of hg row tiles
        const int g = rel / full;
        const int height = min(hg, mf - g * hg);
        const int r = rel - g * full;
        n_tile = r / height;
        m_tile = g * hg + (r - n_tile * height);
        h = t.balanced ? ((span + mf - 1) / mf + 31) / 32 * 32 : 256;
    } else {
        n_tile = rel;
        m_tile = mf;
        h = 256;
    }
    w.row0 = off + static_cast<int64_t>(m_tile) * h;
    w.row_end = min(min(w.row0 + h, static_cast<int64_t>(off) + span), p.rows);
    if (w.row0 < 0 || w.row0 >= w.row_end) return w;
    if (s.phase != 0) h = static_cast<int>(w.row_end - w.row0);
    // The tile runs the smallest row variant that holds h rows, so all row
    // tiles of one expert run the same variant (and keep pace with each other).
    // Phase-2 tiles of at most 32 rows (at H=4096, 4096 tokens: 336 of the 448
    // gate/up short tiles) run a 32-row tile: half the MFMA work of the 64-row
    // one. Column pieces exist for 256-, 128- and 64-row tiles.
    if (s.piece >= 0)
        w.variant = h > 128 ? 0 : (h > 64 ? 1 : 2);
    else
        w.variant = h > 224   ? 0
                    : h > 192 ? 10
                    : h > 160 ? 11
                    : h > 128 ? 12
                    : h > 64  ? 1
                    : h > 32  ? 2
                              : 9;
    if constexpr (SWIGLU) {
        w.col0 = static_cast<int64_t>(n_tile) * 128;
    } else if (s.piece < 0) {
        w.col0 = static_cast<int64_t>(n_tile) * 256;
    } else if (s.piece < 4) {
        w.col0 = static_cast<int64_t>(n_tile) * 256 + s.piece * 128;
        w.variant += 3;
    } else {
        w.col0 = static_cast<int64_t>(n_tile) * 256 + (s.piece - 4) * 64;
        w.variant += 6;
    }
    // A piece of the last column tile can start at or past the last output
    // column (N < 256, or a last tile of at most 192 columns): it has no
    // work, and its weight rows would start past the expert's.
    if (w.col0 >= p.n_out) return w;
    w.expert = e;
    w.valid = true;
    return w;
}

// Issues tile w's prologue; with GATHER also leaves its A offsets in a_carry.
template <bool SWIGLU, bool GATHER>
__device__ __forceinline__ void ring_prologue(const GemmParams& p, char* lds, const RingWork& w, uint32_t* a_carry) {
    const int k_steps = static_cast<int>(p.k / kStageK);
    auto go = [&](auto ops) {
        ops.prologue(k_steps);
        if constexpr (GATHER) {
#pragma unroll
            for (int i = 0; i < decltype(ops)::A_LOADS; ++i) a_carry[i] = ops.a_off[i];
        }
    };
    switch (w.variant) {
        case 0: go(RingOps<256, 256, SWIGLU, kRingBytes, 2, 4, GATHER>(p, lds, w.expert, w.col0, w.row0, w.row_end)); break;
        case 1: go(RingOps<128, 256, SWIGLU, kRingBytes, 2, 4, GATHER>(p, lds, w.expert, w.col0, w.row0, w.row_end)); break;
        case 2: go(RingOps<64, 256, SWIGLU, kRingBytes, 2, 4, GATHER>(p, lds, w.expert, w.col0, w.row0, w.row_end)); break;
        case 9: go(RingOps<32, 256, SWIGLU, kRingBytes, 2, 4, GATHER>(p, lds, w.expert, w.col0, w.row0, w.row_end)); break;
        case 10: go(RingOps<224, 256, SWIGLU, kRingBytes, 2, 4, GATHER>(p, lds, w.expert, w.col0, w.row0, w.row_end)); break;
        case 11: go(RingOps<192, 256, SWIGLU, kRingBytes, 2, 4, GATHER>(p, lds, w.expert, w.col0, w.row0, w.row_end)); break;
        case 12: go(RingOps<160, 256, SWIGLU, kRingBytes, 2, 4, GATHER>(p, lds, w.expert, w.col0, w.row0, w.row_end)); break;
        default:
            if constexpr (!SWIGLU) {
                if (w.variant == 3) go(RingOps<256, 128, false, kRingBytes>(p, lds, w.expert, w.col0, w.row0, w.row_end));
                else if (w.variant == 4) go(RingOps<128, 128, false, kRingBytes>(p, lds, w.expert, w.col0, w.row0, w.row_end));
                else if (w.variant == 5) go(RingOps<64, 128, false, kRingBytes>(p, lds, w.expert, w.col0, w.row0, w.row_end));
                else if (w.variant == 6) go(RingOps<256, 64, false, kRingBytes>(p, lds, w.expert, w.col0, w.row0, w.row_end));
                else if (w.variant == 7) go(RingOps<128, 64, false, kRingBytes>(p, lds, w.expert, w.col0, w.row0, w.row_end));
                else go(RingOps<64, 64, false, kRingBytes>(p, lds, w.expert, w.col0, w.row0, w.row_end));
            }
    }
}

// Runs tile `w` starting at ring slots (sa, sb) (updated for the next tile).
// When the next tile `nxt` has the same ring shape and the k chain is long
// enough, the two are chained (see ring_tile): `w`'s last windows load `nxt`'s
// first stages and its hook issues only the prologue's last window. Otherwise
// the hook issues `nxt`'s whole prologue at slots 0.
template <int TMR, int BNT, bool SWIGLU, bool GATHER = false>
__device__ __forceinline__ void ring_run_shape(const GemmParams& p, char* lds, const RingWork& w,
                                               const RingWork& nxt, bool wait_all, int& sa, int& sb,
                                               uint32_t* a_carry) {
    using R = RingOps<TMR, BNT, SWIGLU, kRingBytes, 2, 4, GATHER>;
    const int k_steps = static_cast<int>(p.k / kStageK);
    // Wave-uniform (it selects buffer resources, which live in SGPRs).
    const bool chain = __builtin_amdgcn_readfirstlane(nxt.valid && nxt.variant == w.variant && k_steps >= R::SB) != 0;
    typename R::Rsrc next{};
    if (chain) next = R::tile_rsrc(p, nxt.expert, nxt.col0, nxt.row0, nxt.row_end);
    // The hook reads the gathered offsets from their own array, not from
    // `next`: a hook that refers to `next` keeps its buffer resources in
    // scratch memory, and the hook's reload of them waits for the ring.
    uint32_t next_off[R::A_LOADS];
#pragma unroll
    for (int i = 0; i < R::A_LOADS; ++i) next_off[i] = next.a_off[i];
    const int na = (sa + k_steps) % R::SA, nb = (sb + k_steps) % R::SB;
    auto hook = [&] {
        if (!nxt.valid) return;
        if (chain) {
            // Gathered rows: the next tile's offsets, formed before its k-loop;
            // otherwise they do not depend on the tile.
            if constexpr (GATHER) {
                typename R::Rsrc res = R::tile_rsrc(p, nxt.expert, nxt.col0, nxt.row0, nxt.row_end, false);
#pragma unroll
                for (int i = 0; i < R::A_LOADS; ++i) res.a_off[i] = next_off[i];
                R(p, lds, res).prologue(k_steps, na, nb, true);
#pragma unroll
                for (int i = 0; i < R::A_LOADS; ++i) a_carry[i] = next_off[i];
            } else {
                R(p, lds, nxt.expert, nxt.col0, nxt.row0, nxt.row_end).prologue(k_steps, na, nb, true);
            }
        } else {
            ring_prologue<SWIGLU, GATHER>(p, lds, nxt, a_carry);
        }
    };
    ring_tile<TMR, BNT, SWIGLU, kRingBytes, decltype(hook), 2, 4, GATHER>(p, lds, w.expert, w.col0, w.row0, w.row_end,
                                                                           false, wait_all, hook, sa, sb, chain, next,
                                                                           a_carry);
    sa = chain ? na : 0;
    sb = chain ? nb : 0;
}

template <bool SWIGLU, bool GATHER>
__device__ __forceinline__ void ring_run(const GemmParams& p, char* lds, const RingWork& w, const RingWork& nxt,
                                         bool wait_all, int& sa, int& sb, uint32_t* a_carry) {
    switch (w.variant) {
        case 0: ring_run_shape<256, 256, SWIGLU, GATHER>(p, lds, w, nxt, wait_all, sa, sb, a_carry); break;
        case 1: ring_run_shape<128, 256, SWIGLU, GATHER>(p, lds, w, nxt, wait_all, sa, sb, a_carry); break;
        case 2: ring_run_shape<64, 256, SWIGLU, GATHER>(p, lds, w, nxt, wait_all, sa, sb, a_carry); break;
        case 9: ring_run_shape<32, 256, SWIGLU, GATHER>(p, lds, w, nxt, wait_all, sa, sb, a_carry); break;
        case 10: ring_run_shape<224, 256, SWIGLU, GATHER>(p, lds, w, nxt, wait_all, sa, sb, a_carry); break;
        case 11: ring_run_shape<192, 256, SWIGLU, GATHER>(p, lds, w, nxt, wait_all, sa, sb, a_carry); break;
        case 12: ring_run_shape<160, 256, SWIGLU, GATHER>(p, lds, w, nxt, wait_all, sa, sb, a_carry); break;
        default:
            if constexpr (!SWIGLU) {
                if (w.variant == 3) ring_run_shape<256, 128, false>(p, lds, w, nxt, wait_all, sa, sb, a_carry);
                else if (w.variant == 4) ring_run_shape<128, 128, false>(p, lds, w, nxt, wait_all, sa, sb, a_carry);
                else if (w.variant == 5) ring_run_shape<64, 128, false>(p, lds, w, nxt, wait_all, sa, sb, a_carry);
                else if (w.variant == 6) ring_run_shape<256, 64, false>(p, lds, w, nxt, wait_all, sa, sb, a_carry);
                else if (w.variant == 7) ring_run_shape<128, 64, false>(p, lds, w, nxt, wait_all, sa, sb, a_carry);
                else ring_run_shape<64, 64, false>(p, lds, w, nxt, wait_all, sa, sb, a_carry);
            }
    }
}

template <bool SWIGLU, bool GATHER>
__global__ __launch_bounds__(kRingThreads) void grouped_gemm_persistent_kernel(GemmParams p) {
    __shared__ __attribute__((aligned(1024))) char lds[kRingBytes];
    // Balanced row tiles for the gate/up GEMM at K >= 2048. There a short last
    // tile's cost is streaming its 256 x K weight slab once more, and the
    // expert's equal-height tiles share that slab in L2 instead (H=4096, I=14336,
    // 4096 tokens: 1625 -> 1587 us; H=2048, I=1408, E=64 Zipf: 661 -> 651 us).
    // Not at H=1024 (77 -> 81 us), nor for the down GEMM, whose short tiles run
    // as column pieces on every CU (781 -> 800 us at H=4096, I=14336).
    const RingTable table = ring_table(p, SWIGLU && p.k >= 2048);
    const int grid = static_cast<int>(gridDim.x);
    const RingPlan plan = ring_plan(table.n_full, table.n_part, grid, !SWIGLU);
    // The next tile of this workgroup at or after tile `sub` of virtual workgroup q.
    auto next = [&](int& q, int& sub) {
        RingWork w{false, 0, 0, 0, 0, 0};
        for (; q < plan.virtual_blocks; q += grid, sub = 0) {
            const RingSlot s = ring_slot(plan, grid, q);
            for (; sub < s.count; ++sub) {
                w = ring_locate<SWIGLU>(p, table, RingSlot{s.phase, s.tile + sub, s.piece, 1});
                if (w.valid) return w;
            }
        }
        return w;
    };
    int q = blockIdx.x, sub = 0;
    RingWork cur = next(q, sub);
    if (!cur.valid) return;
    uint32_t a_carry[8];  // GATHER: the next tile's A offsets (at most 8 loads per wave and stage)
    ring_prologue<SWIGLU, GATHER>(p, lds, cur, a_carry);
    bool after_epilogue = false;
    int sa = 0, sb = 0;  // ring slots of the current tile's first stage
    for (;;) {
        int qn = q, sn = sub + 1;
        RingWork nxt = next(qn, sn);
        // Wave-uniform, opaque copies: nothing derived from the next tile may be
        // hoisted into (and kept live through) the current tile's k-loop.
        {
            int r0 = __builtin_amdgcn_readfirstlane(static_cast<int>(nxt.row0));
            int r1 = __builtin_amdgcn_readfirstlane(static_cast<int>(nxt.row_end));
            int c = __builtin_amdgcn_readfirstlane(static_cast<int>(nxt.col0));
            int e = __builtin_amdgcn_readfirstlane(nxt.expert), v = __builtin_amdgcn_readfirstlane(nxt.variant);
            nxt.valid = __builtin_amdgcn_readfirstlane(nxt.valid ? 1 : 0) != 0;
            asm volatile("" : "+s"(r0), "+s"(r1), "+s"(c), "+s"(e), "+s"(v));
            nxt.row0 = r0;
            nxt.row_end = r1;
            nxt.col0 = c;
            nxt.expert = e;
            nxt.variant = v;
        }
        ring_run<SWIGLU, GATHER>(p, lds, cur, nxt, after_epilogue, sa, sb, a_carry);
        if (!nxt.valid) break;
        cur = nxt;
        q = qn;
        sub = sn;
        after_epilogue = true;
    }
}

// Weight-streaming launches (decode sizes, and small batches over many
// experts; the launcher's rule is below): the work is streaming
// the active experts' weights (at T=1, 2 x 235 MB for the gate/up GEMM). The
// kernel is persistent like the wide one: workgroups walk the tiles (row
// tiles of at most MAX_ROWS rows, expert by expert, column tile by column
// tile) and issue the next tile's first stages before the current tile's
// epilogue. Tiles are narrow so that a single token's two
// experts still spread over the CUs: 64 activation columns (128 weight rows,
// waves 2 x 2) for the gate/up GEMM, 64 output columns for the down GEMM, and
// 32 (waves 4 x 1) when at most 64 rows are packed (at T=16 the 4 x 1 waves,
// which all read every B fragment, ran 7% slower than 64 columns). Their
// stages are small (12-32 KiB), so the ring holds up to eight: a CU has to
// keep about 32 KiB of loads in flight to stream at the HBM rate (a plain
// read kernel reaches 6.3-6.4 TB/s with 32 KiB per CU, 5.2 TB/s with 16 KiB).
// The 64-row gate/up instance is the exception: it keeps three stages (72
// KiB) so that two workgroups share a CU, which suits a token's 448 tiles
// better than one workgroup per CU with a deeper ring (T=1: 93 vs 97 us).
// Each output is the same MFMA chain in k order as on the wide path. MAX_ROWS
// is 64 when the launch has at most 64 rows, else 128; a row tile of at most
// 64 rows runs the 64-row instance. At C1 (T=128, E=8: about 32 rows per
// expert) the wide tiles kept 64 (gate/up) and 16 (down) CUs busy.
template <bool SWIGLU, int MAX_ROWS>
constexpr int narrow_cols() { return SWIGLU || MAX_ROWS == 128 ? 64 : 32; }

constexpr int kDecodeStages = 8;

template <bool SWIGLU, int MAX_ROWS>
constexpr uint32_t decode_lds_bytes() {
    return SWIGLU && MAX_ROWS == 64 ? 3 * (64 + 2 * narrow_cols<SWIGLU, MAX_ROWS>()) * kRowBytes : kRingBytes;
}

template <bool SWIGLU, int MAX_ROWS, bool GATHER>
__global__ __launch_bounds__(kRingThreads) void grouped_gemm_decode_kernel(GemmParams p) {
    constexpr int COLS = narrow_cols<SWIGLU, MAX_ROWS>();
    constexpr int BNT = SWIGLU ? 2 * COLS : COLS;
    constexpr int WC = BNT == 32 ? 1 : 2;
    constexpr uint32_t kLds = decode_lds_bytes<SWIGLU, MAX_ROWS>();
    static_assert(MAX_ROWS == 64 || MAX_ROWS == 128, "decode row tiles");
    __shared__ __attribute__((aligned(1024))) char lds[kLds];
    const int lane = threadIdx.x & 63;
    // Lane e: expert e's first row, rows, row tiles of at most MAX_ROWS rows,
    // and its first tile. Tiles go expert by expert, column tile by column
    // tile, row tiles fastest (so an expert's row tiles share a weight slab).
    int off = 0, span = 0;
    if (lane < p.experts) expert_rows(p, lane, off, span);
    const int m_tiles = (span + MAX_ROWS - 1) / MAX_ROWS;
    const int count = m_tiles * p.n_tiles;
    const int incl = wave_inclusive_sum(count);
    const int first = incl - count;
    const int tiles = __builtin_amdgcn_readlane(incl, kWave - 1);
    const int k_steps = static_cast<int>(p.k / kStageK);
    struct Work {
        bool valid;
        int tall, expert, row0, row_end, col0;  // tall: more than 64 rows
    };
    auto locate = [&](int t) {
        Work w{false, 0, 0, 0, 0, 0};
        if (t >= tiles) return w;
        const uint64_t owner = __ballot(lane < p.experts && count > 0 && first <= t);
        if (owner == 0) return w;
        const int e = 63 - __builtin_clzll(owner);
        const int rel = t - __builtin_amdgcn_readlane(first, e);
        const int me = __builtin_amdgcn_readlane(m_tiles, e);
        const int n_tile = rel / me;
        const int base = __builtin_amdgcn_readlane(off, e);
        w.row0 = base + (rel - n_tile * me) * MAX_ROWS;
        w.row_end = static_cast<int>(min(static_cast<int64_t>(base) + __builtin_amdgcn_readlane(span, e), p.rows));
        if (w.row0 < 0 || w.row0 >= w.row_end) return w;
        w.tall = MAX_ROWS == 128 && w.row_end - w.row0 > 64;
        w.expert = e;
        w.col0 = n_tile * COLS;
        w.valid = true;
        return w;
    };
    uint32_t a_carry[8];  // GATHER: the next tile's A offsets, formed where its prologue is issued
    auto issue = [&](auto ops) {
        ops.prologue(k_steps);
        if constexpr (GATHER) {
#pragma unroll
            for (int i = 0; i < decltype(ops)::A_LOADS; ++i) a_carry[i] = ops.a_off[i];
        }
    };
    auto prologue = [&](const Work& w) {
        if constexpr (MAX_ROWS == 128) {
            if (w.tall) {
                issue(RingOps<128, BNT, SWIGLU, kLds, WC, kDecodeStages, GATHER>(p, lds, w.expert, w.col0, w.row0,
                                                                                 w.row_end));
                return;
            }
        }
        issue(RingOps<64, BNT, SWIGLU, kLds, WC, kDecodeStages, GATHER>(p, lds, w.expert, w.col0, w.row0, w.row_end));
    };
    auto run = [&](const Work& w, bool wait_all, const auto& hook) {
        using Hook = std::decay_t<decltype(hook)>;
        if constexpr (MAX_ROWS == 128) {
            if (w.tall) {
                ring_tile<128, BNT, SWIGLU, kLds, Hook, WC, kDecodeStages, GATHER>(
                    p, lds, w.expert, w.col0, w.row0, w.row_end, false, wait_all, hook, 0, 0, false, {}, a_carry);
                return;
            }
        }
        ring_tile<64, BNT, SWIGLU, kLds, Hook, WC, kDecodeStages, GATHER>(
            p, lds, w.expert, w.col0, w.row0, w.row_end, false, wait_all, hook, 0, 0, false, {}, a_carry);
    };
    int t = blockIdx.x;
    Work cur = locate(t);
    if (!cur.valid) return;
    prologue(cur);
    bool after_epilogue = false;
    for (;;) {
        const int tn = t + static_cast<int>(gridDim.x);
        const Work nxt = locate(tn);
        auto hook = [&] {
            if (!nxt.valid) return;
            // Opaque copies, as in the wide kernel: nothing derived from the
            // next tile is hoisted into the current tile's k-loop. (The values
            // are uniform; they go back to scalar registers after the asm.)
            Work w = nxt;
            asm volatile("" : "+v"(w.tall), "+v"(w.expert), "+v"(w.row0), "+v"(w.row_end), "+v"(w.col0));
            w.tall = __builtin_amdgcn_readfirstlane(w.tall);
            w.expert = __builtin_amdgcn_readfirstlane(w.expert);
            w.row0 = __builtin_amdgcn_readfirstlane(w.row0);
            w.row_end = __builtin_amdgcn_readfirstlane(w.row_end);
            w.col0 = __builtin_amdgcn_readfirstlane(w.col0);
            prologue(w);
        };
        run(cur, after_epilogue, hook);
        if (!nxt.valid) break;
        cur = nxt;
        t = tn;
        after_epilogue = true;
    }
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
// Upper bound on the persistent GEMM's workgroups (0: one per CU), process-wide.
static std::atomic<int> g_gemm_workgroup_limit{0};

void set_gemm_workgroup_limit(int workgroups) {
    g_gemm_workgroup_limit.store(workgroups, std::memory_order_relaxed);
}

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
    // Narrow tiles for weight streaming: at most 128 rows in all, or at most 128
    // per expert on average when the wide tiles (rows spread evenly over the
    // experts) would not give every CU one. Measured at C1 (E=8, ~32 rows each):
    // gate/up 9.4 -> 7.2 us, down 11.6 -> 7.4 us; at C3 T=256 the gate/up GEMM's
    // 256 wide tiles streamed faster than narrow ones (22.9 vs 24.9 us).
    const int64_t per_expert = (rows + p.experts - 1) / p.experts;
    const int64_t wide_tiles = static_cast<int64_t>(p.experts) * ((per_expert + BM - 1) / BM) * p.n_tiles;
    const bool narrow = rows <= 128 || (rows <= 128 * static_cast<int64_t>(p.experts) &&
                                        wide_tiles < device_cu_count());
    if (BM == 256 && BN == 256 && p.k % kStageK == 0 && narrow) {
        GemmParams q = p;
        const int max_rows = rows <= 64 ? 64 : 128;
        const int cols = max_rows == 64 ? narrow_cols<SWIGLU, 64>() : narrow_cols<SWIGLU, 128>();
        q.n_tiles = static_cast<int>((p.n_out + cols - 1) / cols);
        // Upper bound on row tiles: sum_e ceil(span_e/max_rows) <= ceil(R/max_rows) + E.
        const int64_t tiles = ((rows + max_rows - 1) / max_rows + p.experts) * q.n_tiles;
        if (tiles > INT32_MAX) return fail(MOE_ERR_CAPACITY, "grouped GEMM grid too large");
        // As many workgroups as fit the CUs' LDS, at most one per tile.
        const uint32_t lds = rows <= 64 ? decode_lds_bytes<SWIGLU, 64>() : decode_lds_bytes<SWIGLU, 128>();
        int64_t grid = static_cast<int64_t>(device_cu_count()) * (kRingBytes / lds);
        if (tiles < grid) grid = tiles;
        auto launch = [&](auto gather_c) {
            constexpr bool G = decltype(gather_c)::value;
            if (rows <= 64)
                hipLaunchKernelGGL((grouped_gemm_decode_kernel<SWIGLU, 64, G>), dim3(static_cast<unsigned>(grid)),
                                   dim3(kRingThreads), 0, stream, q);
            else
                hipLaunchKernelGGL((grouped_gemm_decode_kernel<SWIGLU, 128, G>), dim3(static_cast<unsigned>(grid)),
                                   dim3(kRingThreads), 0, stream, q);
        };
        if constexpr (SWIGLU) {
            if (p.a_rows != nullptr)
                launch(std::true_type{});
            else
                launch(std::false_type{});
        } else {
            launch(std::false_type{});
        }
        return check_launch("grouped_gemm_decode_kernel");
    }
    if (BM == 256 && BN == 256 && p.k % kStageK == 0) {
        // One workgroup per CU (the ring fills a CU's LDS), each walking the
        // virtual workgroups of the device-side plan, whose XCD ranges need a
        // multiple of 8 workgroups. Row offsets fit 32 bits (checked by the ABI).
        if (blocks > INT32_MAX) return fail(MOE_ERR_CAPACITY, "grouped GEMM grid too large");
        int64_t grid = device_cu_count();
        const int limit = g_gemm_workgroup_limit.load(std::memory_order_relaxed);
        if (limit > 0 && limit < grid) grid = limit;
        // At most one workgroup per unit of work: tiles, or for the plain GEMM
        // the halves and quarters the plan may split them into.
        const int64_t units = SWIGLU ? blocks : 4 * blocks;
        if (units < grid) grid = units;
        grid = grid / kNumXcd * kNumXcd;
        if (grid < kNumXcd) grid = kNumXcd;
        if constexpr (SWIGLU) {
            if (p.a_rows != nullptr)
                hipLaunchKernelGGL((grouped_gemm_persistent_kernel<true, true>), dim3(static_cast<unsigned>(grid)),
                                   dim3(kRingThreads), 0, stream, p);
            else
                hipLaunchKernelGGL((grouped_gemm_persistent_kernel<true, false>), dim3(static_cast<unsigned>(grid)),
                                   dim3(kRingThreads), 0, stream, p);
        } else {
            hipLaunchKernelGGL((grouped_gemm_persistent_kernel<false, false>), dim3(static_cast<unsigned>(grid)),
                               dim3(kRingThreads), 0, stream, p);
        }
        return check_launch("grouped_gemm_persistent_kernel");
    }
    if (p.a_rows != nullptr) return fail(MOE_ERR_UNSUPPORTED, "gathered A rows need K a multiple of 64");
    // The generic kernel maps workgroup b to tile (b % 8) * per_xcd + b / 8 with
    // per_xcd = ceil(tiles / 8), which reaches every tile only when the grid
    // holds all 8 * per_xcd slots: round the upper bound up to a multiple of 8.
    blocks = (blocks + kNumXcd - 1) / kNumXcd * kNumXcd;
    if (blocks > INT32_MAX) return fail(MOE_ERR_CAPACITY, "grouped GEMM grid too large");
    hipLaunchKernelGGL((grouped_gemm_kernel<BM, BN, WAVES_M, WAVES_N, SWIGLU>),
                       dim3(static_cast<unsigned>(blocks)), dim3(kGemmThreads), 0, stream, p);
    return check_launch("grouped_gemm_kernel");
}

int launch_grouped_gemm(const uint16_t* a, const uint16_t* b, int64_t ldb, uint16_t* c, const int32_t* offsets,
                        int64_t rows, int64_t n, int64_t k, int experts, hipStream_t stream) {
    GemmParams p{};
    p.rows = rows;
    p.a = a;
    p.b = b;
    p.c = c;
    p.offsets = offsets;
    p.k = k;
    p.ldb = ldb;
    p.nb = n;
    p.n_out = n;
    p.ldc = n;
    p.experts = experts;
    return launch_gemm_t<256, 256, 2, 2, false>(p, rows, stream);
}

int launch_gateup_swiglu(const uint16_t* a, const uint16_t* gate_up, int64_t ldb, uint16_t* act,
                         const int32_t* offsets, int64_t rows, int64_t hidden,
                         int64_t intermediate, int experts, hipStream_t stream) {
    GemmParams p{};
    p.rows = rows;
    p.a = a;
    p.b = gate_up;
    p.c = act;
    p.offsets = offsets;
    p.k = hidden;
    p.ldb = ldb;
    p.nb = 2 * intermediate;
    p.n_out = intermediate;
    p.ldc = intermediate;
    p.experts = experts;
    return launch_gemm_t<256, 256, 2, 2, true>(p, rows, stream);
}

// launch_gateup_swiglu with A row r read from row a_rows[r] of x (zero when
// negative): the dispatch's row table instead of its packed copy. Needs the
// ring kernels (hidden a multiple of 64; the ABI checks it).
int launch_gateup_swiglu_gathered(const uint16_t* x, const int32_t* a_rows, int64_t x_rows, const uint16_t* gate_up,
                                  int64_t ldb, uint16_t* act, const int32_t* offsets, int64_t rows, int64_t hidden,
                                  int64_t intermediate, int experts, hipStream_t stream) {
    GemmParams p{};
    p.rows = rows;
    p.a = x;
    p.a_rows = a_rows;
    p.a_src_rows = x_rows;
    p.b = gate_up;
    p.c = act;
    p.offsets = offsets;
    p.k = hidden;
    p.ldb = ldb;
    p.nb = 2 * intermediate;
    p.n_out = intermediate;
    p.ldc = intermediate;
    p.experts = experts;
    return launch_gemm_t<256, 256, 2, 2, true>(p, rows, stream);
}

}  // namespace moe
