/*
 * moe_hip.h - C ABI of the gfx950 (MI355X) MoE feed-forward kernels.
 *
 * Every entry point takes raw device pointers, 64-bit sizes and a HIP stream
 * (hipStream_t passed as void*; NULL means the default stream). Calls are
 * asynchronous on that stream, never synchronise the host, and never allocate
 * or free device memory: the caller owns every buffer, including the scratch
 * that moe_dispatch needs (size from moe_dispatch_scratch_bytes).
 *
 * Return value: MOE_OK (0) or a moe_status_t error code. moe_last_error()
 * returns a thread-local message describing the most recent failure.
 *
 * Layouts (all row-major, contiguous):
 *   x            [T, H]       activations (bf16 for the block; f32/f16/bf16 transport)
 *   router_w     [E, H]       fp32
 *   ids32/ids64  [T, K]       selected experts, flat assignment index p = t*K + k
 *   weights      [T, K]       fp32 routing weights
 *   counts       [E]          int32 assignments per expert
 *   offsets      [E+1]        int32 start row of each expert's span in `packed`
 *   slots        [T*K]        int32 within-expert slot of each assignment
 *   inverse      [T, K]       int32 packed row of each assignment
 *   packed       [R, H]       rows grouped by expert; span e = [offsets[e], offsets[e+1])
 *   gate_up      [E, 2I, H]   bf16; rows 0..I-1 gate, I..2I-1 up
 *   down         [E, H, I]    bf16
 *   (the *_strided GEMM entry points also take weight rows further apart)
 *
 * Slot order is canonical (deterministic): within an expert, assignments
 * appear in increasing flat index p. No global atomics are used.
 */
#ifndef MOE_HIP_H_
#define MOE_HIP_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MOE_ABI_VERSION 8

typedef enum {
    MOE_DTYPE_F32 = 0,
    MOE_DTYPE_F16 = 1,
    MOE_DTYPE_BF16 = 2,
} moe_dtype_t;

typedef enum {
    MOE_OK = 0,
    MOE_ERR_INVALID_ARGUMENT = 1, /* shape, pointer or dtype mismatch */
    MOE_ERR_UNSUPPORTED = 2,      /* valid request outside this build's limits */
    MOE_ERR_CAPACITY = 3,         /* exceeds int32 indexing capacity */
    MOE_ERR_WORKSPACE = 4,        /* caller buffer too small */
    MOE_ERR_HIP = 5,              /* HIP runtime / launch failure */
} moe_status_t;

/* ABI version of the loaded library (MOE_ABI_VERSION at build time). */
int moe_abi_version(void);

/* Static description of a status code. */
const char* moe_status_string(int status);

/* Thread-local message for the most recent non-OK return on this thread. */
const char* moe_last_error(void);

/*
 * Top-k routing on given fp32 logits.
 * Replaces topk_route_out (reference src/moe_dispatch/csrc/dispatch.cu:378-402,
 * kernel :338-376, tie rule :325-336; binding csrc/bindings.cpp:12-13).
 * v = logits + bias; top-k by value with ties to the lower expert index;
 * weights: K=1 -> 1, K=2 -> w0 = 1/(1+exp(v1-v0)), w1 = exp(v1-v0)*w0,
 * K>2 -> exp(v_j - v_0) / sum_i exp(v_i - v_0).
 * Limits: 1 <= E <= 64, 1 <= K <= min(E, 8), T*E <= INT32_MAX. Logits must be finite.
 */
int moe_topk_route(const float* logits, const float* bias, int32_t* ids32, int64_t* ids64,
                   float* weights, int64_t tokens, int64_t experts, int64_t topk, void* stream);

/* Bytes of scratch moe_router_fused needs for (E, H): the bf16 split of
 * router_w, then 64 KiB of partial logits for the small-batch (T <= 64,
 * E <= 16) split-k path, then a copy of the split in the MFMA operand order
 * the VGPR-load kernels read (ceil(H/64) * ceil(6E/16) KiB). */
int64_t moe_router_scratch_bytes(int64_t experts, int64_t hidden);

/*
 * Fused router: logits = float(x) . router_w^T in fp32, then moe_topk_route's
 * selection. Replaces the F.linear + topk_route_out pair of MoEBlock.route
 * (reference src/moe_dispatch/layer.py:122-135). x is bf16 [T,H]. logits_out
 * ([T,E] fp32) is optional (NULL to skip). ids64 may be NULL.
 * router_w is split exactly into three bf16 planes (hi, mid, lo) in scratch
 * (moe_router_scratch_bytes bytes, 16-byte aligned) once per call; the
 * products x * part are exact and accumulate in fp32 on MFMA.
 * router_w == NULL skips the split and uses the planes scratch already holds
 * from an earlier call with the same E and H (for callers that know the
 * router weights have not changed since; no reference counterpart).
 * Precondition: moe_router_split, or a moe_router_fused call with router_w,
 * wrote that scratch for this E and H. Without it the kernels read whatever
 * the scratch holds and the ids and weights are meaningless; the call cannot
 * tell (it reads no device memory on the host) and returns MOE_OK.
 * Calls that share one scratch must not overlap in time.
 */
int moe_router_fused(const void* x, const float* router_w, const float* bias, int32_t* ids32,
                     int64_t* ids64, float* weights, float* logits_out, void* scratch,
                     int64_t scratch_bytes, int64_t tokens, int64_t hidden, int64_t experts,
                     int64_t topk, void* stream);

/*
 * The bf16 split of router_w that moe_router_fused keeps in its scratch, alone:
 * writes the planes a later moe_router_fused(router_w = NULL, ...) call reads.
 * For callers that keep the split current outside a captured graph, so that
 * replays of a forward captured with router_w = NULL do not redo it. No
 * counterpart in the reference (its router has no such split).
 */
int moe_router_split(const float* router_w, void* scratch, int64_t scratch_bytes, int64_t experts,
                     int64_t hidden, void* stream);

/*
 * Tokens per tile of moe_router_fused_ranked for (T, E): 16 for E <= 16, 32
 * above, or 0 when ceil(T / tile) * E > 4096 or T == 0 (then route with
 * moe_router_fused and dispatch with moe_dispatch); -1 for invalid E or T.
 * No counterpart in the reference.
 */
int64_t moe_router_rank_tile(int64_t tokens, int64_t experts);

/*
 * moe_router_fused that also does the counting pass of the dispatch for the
 * routes it selects: for each tile of `tile` = moe_router_rank_tile(T, E)
 * consecutive tokens, tile_counts[tile_index * E + e] = the tile's
 * assignments to expert e, and ranks[p] = #{p' < p in p's tile : ids[p'] ==
 * ids[p]} (flat order p = t*K + k; ranks holds T*K int32). moe_dispatch_ranked
 * then skips its own counting pass (one launch less per forward).
 * tile_counts_bytes >= ceil(T / tile) * E * 4; MOE_ERR_UNSUPPORTED when
 * moe_router_rank_tile returns 0. router_w == NULL carries moe_router_fused's
 * precondition; here meaningless ranks and tile counts would also misplace the
 * pack's rows (moe_dispatch_ranked keeps every write inside packed_rows, but
 * the layout is then wrong). No counterpart in the reference (its router and
 * dispatch are separate passes).
 */
int moe_router_fused_ranked(const void* x, const float* router_w, const float* bias, int32_t* ids32,
                            int64_t* ids64, float* weights, float* logits_out, void* scratch,
                            int64_t scratch_bytes, int64_t tokens, int64_t hidden, int64_t experts,
                            int64_t topk, int32_t* ranks, int32_t* tile_counts, int64_t tile_counts_bytes,
                            void* stream);

/* Bytes of scratch moe_dispatch needs for (T, E, K). */
int64_t moe_dispatch_scratch_bytes(int64_t tokens, int64_t experts, int64_t topk);

/*
 * Token dispatch: expert histogram, prefix scan and stable pack.
 * Replaces dispatch_out (alignment == 1; reference csrc/dispatch.cu:102-158)
 * and dispatch_aligned_out (alignment > 1; :218-275), binding
 * csrc/bindings.cpp:3-5,8-10.
 *   counts[e]  = #{p : ids[p] == e}
 *   offsets[0] = 0, offsets[e+1] = offsets[e] + ceil(counts[e]/a)*a
 *   slots[p]   = #{p' < p : ids[p'] == ids[p]}     (canonical order)
 *   inverse[p] = offsets[ids[p]] + slots[p]
 *   packed[inverse[p]] = x[p / K]; rows [offsets[e]+counts[e], offsets[e+1]) = 0.
 * Rows >= offsets[E] are not written. Out-of-range ids are skipped (slot -1,
 * inverse untouched) as in the reference kernels.
 * vectorized != 0 copies rows with 16-byte accesses when the row size allows.
 * packed_rows must be >= T*K (alignment 1) or the aligned capacity
 * ceil((T*K + E*(a-1) + 1)/a)*a (reference src/moe_dispatch/workspace.py:29-34).
 * Limits: 1 <= E <= 64, 1 <= K <= 8, 1 <= a <= 128, H >= 1.
 */
int moe_dispatch(const void* x, int dtype, const int32_t* ids, int32_t* counts, int32_t* offsets,
                 int32_t* slots, void* packed, int32_t* inverse, void* scratch,
                 int64_t scratch_bytes, int64_t tokens, int64_t hidden, int64_t experts,
                 int64_t topk, int64_t alignment, int64_t packed_rows, int vectorized,
                 void* stream);

/*
 * moe_dispatch with no scratch argument, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc). No counterpart in the reference. It allocates
 * nothing: the kernels' per-chunk count table (at most 16384 bytes for every
 * valid shape; larger needs return MOE_ERR_WORKSPACE) lives in a static device
 * array of the library, one per GPU, kept until the process ends. Every call
 * on one GPU uses that GPU's array, so calls that overlap in time on one GPU
 * (other streams or host threads) race; calls on one stream are ordered. The
 * current device must be the one the pointers and the stream belong to.
 * The first call on each device looks the array's address up (a runtime call,
 * not a stream operation); made while `stream` is capturing, that first call
 * returns MOE_ERR_UNSUPPORTED, so make one call per device before capturing.
 * Arguments, results and errors are otherwise moe_dispatch's.
 */
int moe_dispatch_noalloc(const void* x, int dtype, const int32_t* ids, int32_t* counts,
                         int32_t* offsets, int32_t* slots, void* packed, int32_t* inverse,
                         int64_t tokens, int64_t hidden, int64_t experts, int64_t topk,
                         int64_t alignment, int64_t packed_rows, int vectorized, void* stream);

/*
 * moe_dispatch after moe_router_fused_ranked: ids, ranks and tile_counts are
 * that call's outputs and tile_tokens its tile (moe_router_rank_tile(T, E);
 * other values return MOE_ERR_INVALID_ARGUMENT). Runs only the pack pass
 * (reference csrc/dispatch.cu:218-275, with the count and scan of :13-53
 * folded into the router); counts, offsets, slots, inverse and packed are
 * moe_dispatch's, bit for bit. ranks is only read, so the call can be
 * repeated. No scratch argument: the tile table is the count table.
 * Destination and padding rows stay below packed_rows whatever ranks and
 * tile_counts hold. No counterpart in the reference.
 */
int moe_dispatch_ranked(const void* x, int dtype, const int32_t* ids, int32_t* counts, int32_t* offsets,
                        int32_t* slots, void* packed, int32_t* inverse, const int32_t* ranks,
                        const int32_t* tile_counts, int64_t tile_counts_bytes, int64_t tile_tokens, int64_t tokens,
                        int64_t hidden, int64_t experts, int64_t topk, int64_t alignment, int64_t packed_rows,
                        int vectorized, void* stream);

/*
 * The dispatch layout without the rows, for moe_grouped_gateup_swiglu_gathered:
 * counts, offsets, slots and inverse exactly as moe_dispatch writes them, and
 * instead of packed rows the row table row_src (packed_rows int32):
 *   row_src[inverse[p]] = p / K for every assignment p, row_src[r] = -1 for the
 *   padding rows [offsets[e] + counts[e], offsets[e+1]); rows >= offsets[E]
 *   are not written.
 * moe_dispatch_rows counts with its scratch like moe_dispatch;
 * moe_dispatch_ranked_rows takes a ranked route's ranks and tile counts like
 * moe_dispatch_ranked. No counterpart in the reference (its dispatch always
 * copies the rows): the expert GEMM reads x through the table instead, which
 * saves writing and reading back T*K rows.
 */
int moe_dispatch_rows(const int32_t* ids, int32_t* counts, int32_t* offsets, int32_t* slots, int32_t* inverse,
                      int32_t* row_src, void* scratch, int64_t scratch_bytes, int64_t tokens, int64_t experts,
                      int64_t topk, int64_t alignment, int64_t packed_rows, void* stream);
int moe_dispatch_ranked_rows(const int32_t* ids, int32_t* counts, int32_t* offsets, int32_t* slots,
                             int32_t* inverse, int32_t* row_src, const int32_t* ranks, const int32_t* tile_counts,
                             int64_t tile_counts_bytes, int64_t tile_tokens, int64_t tokens, int64_t experts,
                             int64_t topk, int64_t alignment, int64_t packed_rows, void* stream);

/*
 * Weighted combine: out[t] = round(sum_k w[t,k] * float(y[inverse[t,k]])),
 * fp32 products and running sum in k order (no fused multiply-add), rows
 * outside [0, packed_rows) skipped, no atomics.
 * Replaces combine_out (reference csrc/dispatch.cu:160-192, kernel :76-93;
 * binding csrc/bindings.cpp:6-7).
 */
int moe_combine(const void* expert_output, int dtype, const int32_t* inverse,
                const float* weights, void* output, int64_t tokens, int64_t hidden,
                int64_t topk, int64_t packed_rows, void* stream);

/*
 * SwiGLU: out[r, j] = round(silu(g) * u), g = proj[r, j], u = proj[r, I + j],
 * fp32 math, one cast; rows >= *valid_rows (device int32) are exactly zero.
 * Replaces swiglu_out (reference csrc/dispatch.cu:294-323, kernel :277-292;
 * binding csrc/bindings.cpp:11).
 */
int moe_swiglu(const void* projection, int dtype, const int32_t* valid_rows, void* output,
               int64_t rows, int64_t width, void* stream);

/*
 * Grouped bf16 GEMM on MFMA: for every expert e and row r in
 * [offsets[e], offsets[e+1]):  c[r, :] = round_bf16(a[r, :] . b[e]^T)
 * with fp32 accumulation. a [rows, k], b [E, n, k], c [rows, n].
 * Rows at or past offsets[E] are not written. The offsets are read on the
 * device and not validated: whatever they hold, only rows [0, rows) of a and
 * c are accessed, and the persistent kernels clamp each span to [0, rows]
 * before they size their tile walk (so offsets past the buffer cost no time).
 * Replaces grouped_linear -> grouped_mm (reference src/moe_dispatch/experts.py:21-35,
 * _triton_gemm.py:16-104; ENDS = offsets[1:]). Requires n % 8 == 0, k % 8 == 0.
 */
int moe_grouped_gemm(const void* a, const void* b, void* c, const int32_t* offsets,
                     int64_t rows, int64_t n, int64_t k, int64_t experts, void* stream);

/*
 * Grouped gate/up GEMM with the SwiGLU epilogue fused:
 *   g = round_bf16(a[r] . gate_up[e, j]), u = round_bf16(a[r] . gate_up[e, I + j])
 *   act[r, j] = round_bf16(silu(g) * u)
 * the computation of grouped_gemm followed by swiglu (reference
 * layer.py:161-172, csrc/dispatch.cu:277-292). g and u are the same bf16
 * values; the epilogue evaluates silu(g) * u as (g * u) / (1 + 2^(-g log2 e))
 * with the hardware exp2 and reciprocal (about 1 ulp each) where moe_swiglu
 * uses a correctly reduced exp, so a few outputs per 100 000 differ from the
 * unfused pair by one bf16 step. Rows at or past offsets[E] are not written.
 * Requires hidden % 8 == 0, intermediate % 8 == 0.
 */
int moe_grouped_gateup_swiglu(const void* a, const void* gate_up, void* act,
                              const int32_t* offsets, int64_t rows, int64_t hidden,
                              int64_t intermediate, int64_t experts, void* stream);

/*
 * moe_grouped_gateup_swiglu with row r of A read from row row_src[r] of x
 * ([x_rows, hidden] bf16; a negative entry reads zeros): with the row table
 * of moe_dispatch_rows this equals moe_grouped_gateup_swiglu on that
 * dispatch's packed rows, bit for bit. No counterpart in the reference (its
 * grouped GEMM reads the packed copy). Requires hidden % 64 == 0 and x below
 * 2 GiB.
 */
int moe_grouped_gateup_swiglu_gathered(const void* x, const int32_t* row_src, int64_t x_rows, const void* gate_up,
                                       void* act, const int32_t* offsets, int64_t rows, int64_t hidden,
                                       int64_t intermediate, int64_t experts, void* stream);

/*
 * The three GEMMs above with the weights' rows a given number of elements
 * apart: row j of expert e's weights starts at element (e * NB + j) * stride
 * (NB = n, or 2 * intermediate for gate/up), and its first k (or hidden)
 * elements are read. With stride equal to the row length they are the calls
 * above (which call these). Every output is the same MFMA chain, so results
 * equal those on a contiguous copy of the weights bit for bit. For weights
 * stored with padded rows: rows a power of two bytes apart (gate/up at
 * H = 4096) are read in lockstep by the weight-streaming kernels, and 64
 * elements of padding per row make the gate/up GEMM at 1 and 16 tokens,
 * H = 4096, 10-11% faster. Requires stride >= the row length, stride % 8
 * == 0, and one expert's rows * stride * 2 bytes below 4 GiB. No counterpart
 * in the reference (its weights are contiguous tensors).
 */
int moe_grouped_gemm_strided(const void* a, const void* b, int64_t b_row_stride, void* c, const int32_t* offsets,
                             int64_t rows, int64_t n, int64_t k, int64_t experts, void* stream);
int moe_grouped_gateup_swiglu_strided(const void* a, const void* gate_up, int64_t gate_up_row_stride, void* act,
                                      const int32_t* offsets, int64_t rows, int64_t hidden, int64_t intermediate,
                                      int64_t experts, void* stream);
int moe_grouped_gateup_swiglu_gathered_strided(const void* x, const int32_t* row_src, int64_t x_rows,
                                               const void* gate_up, int64_t gate_up_row_stride, void* act,
                                               const int32_t* offsets, int64_t rows, int64_t hidden,
                                               int64_t intermediate, int64_t experts, void* stream);

/*
 * Upper bound on the workgroups of the persistent grouped GEMM (both
 * moe_grouped_gemm and moe_grouped_gateup_swiglu): 0 (the default) runs one
 * per CU; n > 0 runs min(n, CUs), rounded down to a multiple of 8 (at least 8).
 * Process-wide; it takes effect at the next launch. Scheduling only: every
 * output tile is computed by one workgroup with the same MFMA chain, so
 * results are identical for every value. For callers that leave CUs to
 * concurrent work on other streams, and for tests of the schedule. No
 * counterpart in the reference (its GEMM is torch's grouped_mm).
 */
int moe_set_gemm_workgroups(int64_t workgroups);

#ifdef __cplusplus
}
#endif

#endif /* MOE_HIP_H_ */
