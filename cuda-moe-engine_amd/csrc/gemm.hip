// Grouped bf16 expert GEMMs on CDNA4 MFMA (v_mfma_f32_32x32x16_bf16).
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
//  * Block tile BM x BN x 64, 4 wavefronts in a WAVES_M x WAVES_N grid, each
//    wave owns (BM/WAVES_M) x (BN/WAVES_N) as 32x32 MFMA sub-tiles; the fp32
//    accumulators live in the AGPR/VGPR file (one wave per SIMD).
//  * Global -> register -> LDS double buffering with one barrier per k-step.
//    LDS rows are 128 bytes; 16-byte chunks are XOR-swizzled per row (swz) so
//    both the 16-byte stores and the MFMA fragment reads are conflict free.
//  * Tile schedule is built on the device from offsets: expert e contributes
//    ceil(span_e/BM) x n_tiles tiles (0 for an empty expert). The grid is a
//    host-side upper bound; surplus workgroups exit at once.
//  * XCD-aware order: workgroup i runs on XCD i % 8, so logical tiles are
//    remapped to give each XCD a contiguous range; inside an expert tiles go
//    N-major so the row tiles of one expert share each weight slice in L2.
#include "moe_common.h"

namespace moe {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

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
// Fast path (K % 64 == 0): 256 x 256 x 64 tiles fed by direct-to-LDS buffer
// loads (buffer_load_dwordx4 ... lds). Each wavefront load moves 8 LDS rows
// (1 KiB); lane l lands at byte 16*l of that block, i.e. row l/8, physical
// chunk l%8, so it fetches the logical chunk that the swizzle maps there. Buffer resources bound the valid bytes: rows past the
// expert's span and weight rows past the expert read as zero without
// per-lane predicates. The last row tile of an expert is 64, 128 or 256 rows
// high (the smallest that holds the remainder), so skewed and ragged spans do
// not pay for a full 256-row tile. The k order of the MFMA chain (ascending,
// one accumulator) is the same as the generic path.
// ---------------------------------------------------------------------------
constexpr uint32_t kRsrcWord3 = 0x00020000u;  // raw buffer, 32-bit dword format
constexpr int kFastStage = (256 + 256) * kBK;  // bf16 elements per LDS stage (A then B)
#ifndef MOE_FAST_WAVE_COLS
#define MOE_FAST_WAVE_COLS 4
#endif
constexpr int kFastWaveCols = MOE_FAST_WAVE_COLS;  // 4 -> 8 wavefronts per tile

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

__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t rsrc, uint16_t* lds_dst, uint32_t voffset,
                                      uint32_t soffset) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        rsrc, (__attribute__((address_space(3))) void*)(lds_dst), 16, voffset, soffset,
        0, 0);
}

// WN wave columns x 2 wave rows; WN = 4 gives 8 wavefronts (2 per SIMD), each
// owning (TM/2) x 64, so one wave's stalls are covered by the other's MFMAs.
// BNT weight rows per tile (256, or 128 for the split tail pieces); col0 is the
// first output column of the tile.
template <int SMT, int WN, int BNT, bool SWIGLU>
__device__ __forceinline__ void fast_tile(const GemmParams& p, uint16_t* lds, int expert, int64_t col0,
                                          int64_t row0, int64_t row_end) {
    constexpr int WAVES = 2 * WN;
    constexpr int TM = SMT * 64;        // rows of this tile (2 wave rows x SMT x 32)
    constexpr int WTM = TM / 2;
    constexpr int WTN = BNT / WN;
    constexpr int SN = WTN / 32;
    constexpr int A_LOADS = TM / 8 / WAVES;   // 8-row wavefront loads per wave
    constexpr int B_LOADS = BNT / 8 / WAVES;
    static_assert(A_LOADS >= 1 && B_LOADS >= 1 && SN >= 1, "tile shape");
    static_assert(!SWIGLU || SN % 2 == 0, "gate/up pairing needs an even sub-tile count");
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN;
    const int wn = wave % WN;
    const int64_t K = p.k;

    const int64_t a_rows = min<int64_t>(row_end - row0, TM);
    const __amdgpu_buffer_rsrc_t rsrc_a = make_rsrc(p.a + row0 * K, static_cast<uint32_t>(a_rows * K * 2));
    const __amdgpu_buffer_rsrc_t rsrc_b =
        make_rsrc(p.b + static_cast<int64_t>(expert) * p.nb * K, static_cast<uint32_t>(p.nb * K * 2));

    // Lane l of an 8-row wavefront load lands at row r0 + l/8, physical chunk l%8,
    // so it fetches logical chunk (l%8) ^ swz_key(row).
    const int lrow = lane >> 3;
    uint32_t a_off[A_LOADS], b_off[B_LOADS];
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
        const int r = (wave * A_LOADS + i) * 8 + lrow;
        const int lchunk = (lane & 7) ^ swz_key(r);
        a_off[i] = static_cast<uint32_t>((r * K + lchunk * 8) * 2);
    }
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i) {
        const int r = (wave * B_LOADS + i) * 8 + lrow;
        const int lchunk = (lane & 7) ^ swz_key(r);
        int64_t brow;
        if constexpr (SWIGLU) {
            const int wcol = r / WTN, w = r % WTN;
            constexpr int HALF = WTN / 2;
            const int64_t col = col0 + wcol * HALF + (w % HALF);
            brow = (w < HALF) ? col : p.n_out + col;
        } else {
            brow = col0 + r;
        }
        b_off[i] = static_cast<uint32_t>((brow * K + lchunk * 8) * 2);
    }

    auto issue = [&](int kt, int stage) {
        const uint32_t koff = static_cast<uint32_t>(kt) * kBK * 2;
        uint16_t* sa = lds + stage * kFastStage;
        uint16_t* sb = sa + 256 * kBK;
#pragma unroll
        for (int i = 0; i < A_LOADS; ++i) dma16(rsrc_a, sa + (wave * A_LOADS + i) * 8 * kBK, a_off[i], koff);
#pragma unroll
        for (int i = 0; i < B_LOADS; ++i) dma16(rsrc_b, sb + (wave * B_LOADS + i) * 8 * kBK, b_off[i], koff);
    };

    floatx16 acc[SMT][SN];
#pragma unroll
    for (int i = 0; i < SMT; ++i)
#pragma unroll
        for (int j = 0; j < SN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    const int frag_row = lane & 31;
    const int frag_half = lane >> 5;
    const int k_steps = static_cast<int>(K / kBK);

    // Fragment reads of one 16-wide k slice and the MFMAs that consume them.
    auto read = [&](const uint16_t* sa, const uint16_t* sb, int kk, bf16x8_t (&fa)[SMT], bf16x8_t (&fb)[SN]) {
        const int chunk = kk * 2 + frag_half;
#pragma unroll
        for (int i = 0; i < SMT; ++i) {
            const int r = wm * WTM + i * 32 + frag_row;
            fa[i] = *reinterpret_cast<const bf16x8_t*>(&sa[swz(r, chunk)]);
        }
#pragma unroll
        for (int j = 0; j < SN; ++j) {
            const int r = wn * WTN + j * 32 + frag_row;
            fb[j] = *reinterpret_cast<const bf16x8_t*>(&sb[swz(r, chunk)]);
        }
    };
    // Weights fragment as src0, activations as src1: the 32x32 result comes out
    // transposed, so lane l holds row l%32 and, in registers 4q..4q+3, the four
    // consecutive columns 8q + 4*(l/32) + 0..3 (packed 8-byte stores). The
    // products and their k grouping are unchanged.
    auto mma = [&](const bf16x8_t (&fa)[SMT], const bf16x8_t (&fb)[SN]) {
#pragma unroll
        for (int i = 0; i < SMT; ++i)
#pragma unroll
            for (int j = 0; j < SN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[j], fa[i], acc[i][j], 0, 0, 0);
    };
    // sched_barrier(0) fences keep each phase in place: the fragment reads of
    // slice kk+1 are issued before the MFMAs of slice kk, so LDS latency hides
    // under the matrix pipe and two fragment sets stay live.
    auto fence = [] { __builtin_amdgcn_sched_barrier(0); };

    bf16x8_t fa0[SMT], fb0[SN], fa1[SMT], fb1[SN];
    issue(0, 0);
    __syncthreads();
    read(lds, lds + 256 * kBK, 0, fa0, fb0);
    for (int kt = 0; kt < k_steps; ++kt) {
        const int stage = kt & 1;
        const uint16_t* sa = lds + stage * kFastStage;
        const uint16_t* sb = sa + 256 * kBK;
        const uint16_t* na = lds + (stage ^ 1) * kFastStage;
        const uint16_t* nb = na + 256 * kBK;
        // Next tile into the other stage (the last step reloads the final tile,
        // keeping the body branch free; the copy is never read).
        issue(min(kt + 1, k_steps - 1), stage ^ 1);
        read(sa, sb, 1, fa1, fb1);
        fence();
        mma(fa0, fb0);
        fence();
        read(sa, sb, 2, fa0, fb0);
        fence();
        mma(fa1, fb1);
        fence();
        read(sa, sb, 3, fa1, fb1);
        fence();
        mma(fa0, fb0);
        fence();
        // All waves are done with this stage's fragments and the next stage has landed.
        __syncthreads();
        read(na, nb, 0, fa0, fb0);
        fence();
        mma(fa1, fb1);
        fence();
    }

    // Epilogue: one row per lane, four consecutive columns per 8-byte store.
    const int col4 = 4 * (lane >> 5);
#pragma unroll
    for (int i = 0; i < SMT; ++i) {
        const int64_t grow = row0 + wm * WTM + i * 32 + (lane & 31);
        if (grow >= row_end) continue;
        uint16_t* crow = p.c + grow * p.ldc;
        if constexpr (SWIGLU) {
#pragma unroll
            for (int j = 0; j < SN / 2; ++j) {
                const int64_t cbase = col0 + wn * (WTN / 2) + j * 32 + col4;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int64_t col = cbase + 8 * q;
                    if (col >= p.n_out) continue;
                    float act[4];
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        const uint32_t gu = pack_bf16x2(acc[i][j][4 * q + t], acc[i][j + SN / 2][4 * q + t]);
                        const float g = __uint_as_float(gu << 16);
                        const float u = __uint_as_float(gu & 0xffff0000u);
                        act[t] = silu_f32(g) * u;
                    }
                    *reinterpret_cast<uint2*>(crow + col) =
                        make_uint2(pack_bf16x2(act[0], act[1]), pack_bf16x2(act[2], act[3]));
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < SN; ++j) {
                const int64_t cbase = col0 + wn * WTN + j * 32 + col4;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int64_t col = cbase + 8 * q;
                    if (col >= p.n_out) continue;
                    *reinterpret_cast<uint2*>(crow + col) =
                        make_uint2(pack_bf16x2(acc[i][j][4 * q], acc[i][j][4 * q + 1]),
                                   pack_bf16x2(acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]));
                }
            }
        }
    }
}

// Work list: full tiles in XCD-aware order, then (plain GEMM only) the tail.
// When the last round of full tiles would occupy at most half of the CUs,
// those tiles are split into two 128-column pieces each; every piece still
// runs the whole k chain in order, so results are unchanged.
template <int WN, bool SWIGLU>
__global__ __launch_bounds__(128 * WN) void grouped_gemm_fast_kernel(GemmParams p) {
    __shared__ __attribute__((aligned(1024))) uint16_t lds[2 * kFastStage];
    const int32_t* __restrict__ offs = p.offsets;
    int total = 0;
    for (int e = 0; e < p.experts; ++e) total += ((offs[e + 1] - offs[e] + 255) / 256) * p.n_tiles;
    const int rem = p.n_cu > 0 ? total % p.n_cu : 0;
    const bool split = !SWIGLU && rem > 0 && 2 * rem <= p.n_cu;
    const int main_tiles = split ? total - rem : total;
    const int per_xcd = (main_tiles + kNumXcd - 1) / kNumXcd;
    int tile, piece = -1;
    if (static_cast<int>(blockIdx.x) < kNumXcd * per_xcd) {
        tile = (blockIdx.x % kNumXcd) * per_xcd + blockIdx.x / kNumXcd;
        if (tile >= main_tiles) return;
    } else {
        const int q = blockIdx.x - kNumXcd * per_xcd;
        if (!split || q >= 2 * rem) return;
        tile = main_tiles + q / 2;
        piece = q % 2;
    }
    int expert = 0, base = 0, m_tiles = 0, span = 0;
    for (; expert < p.experts; ++expert) {
        span = offs[expert + 1] - offs[expert];
        m_tiles = (span + 255) / 256;
        const int t = m_tiles * p.n_tiles;
        if (tile < base + t) break;
        base += t;
    }
    const int rel = tile - base;
    const int n_tile = rel / m_tiles;
    const int m_tile = rel - n_tile * m_tiles;
    const int64_t row0 = offs[expert] + static_cast<int64_t>(m_tile) * 256;
    const int64_t row_end = min(static_cast<int64_t>(offs[expert + 1]), p.rows);
    if (row0 < 0 || row0 >= row_end) return;
    const int rem_rows = span - m_tile * 256;  // rows left from this tile on
    if constexpr (SWIGLU) {
        const int64_t col0 = static_cast<int64_t>(n_tile) * 128;
        if (rem_rows > 128) fast_tile<4, WN, 256, true>(p, lds, expert, col0, row0, row_end);
        else if (rem_rows > 64) fast_tile<2, WN, 256, true>(p, lds, expert, col0, row0, row_end);
        else fast_tile<1, WN, 256, true>(p, lds, expert, col0, row0, row_end);
    } else if (piece < 0) {
        const int64_t col0 = static_cast<int64_t>(n_tile) * 256;
        if (rem_rows > 128) fast_tile<4, WN, 256, false>(p, lds, expert, col0, row0, row_end);
        else if (rem_rows > 64) fast_tile<2, WN, 256, false>(p, lds, expert, col0, row0, row_end);
        else fast_tile<1, WN, 256, false>(p, lds, expert, col0, row0, row_end);
    } else {
        const int64_t col0 = static_cast<int64_t>(n_tile) * 256 + piece * 128;
        if (rem_rows > 128) fast_tile<4, WN, 128, false>(p, lds, expert, col0, row0, row_end);
        else if (rem_rows > 64) fast_tile<2, WN, 128, false>(p, lds, expert, col0, row0, row_end);
        else fast_tile<1, WN, 128, false>(p, lds, expert, col0, row0, row_end);
    }
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
    blocks = (blocks + kNumXcd - 1) / kNumXcd * kNumXcd;
    if (blocks == 0) return MOE_OK;
    p.n_cu = device_cu_count();
    if (!SWIGLU) blocks += 2 * p.n_cu;  // room for the split tail pieces
    if (blocks > INT32_MAX) return fail(MOE_ERR_CAPACITY, "grouped GEMM grid too large");
    if (BM == 256 && BN == 256 && p.k % kBK == 0) {
        hipLaunchKernelGGL((grouped_gemm_fast_kernel<kFastWaveCols, SWIGLU>),
                           dim3(static_cast<unsigned>(blocks)), dim3(128 * kFastWaveCols), 0, stream, p);
        return check_launch("grouped_gemm_fast_kernel");
    }
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
