// extern "C" entry points: argument validation (the checks the reference
// performs with TORCH_CHECK in src/moe_dispatch/csrc/dispatch.cu:95-129,
// :160-182, :218-243, :294-313, :378-395), then kernel launches on the
// caller's stream. Nothing here allocates device memory or synchronises.
#include <climits>
#include <cstdarg>
#include <cstdio>

#include "moe_common.h"

namespace moe {

int launch_topk_route(const float*, const float*, int32_t*, int64_t*, float*, int64_t, int, int,
                      hipStream_t);
int launch_router_fused(const uint16_t*, const float*, const float*, int32_t*, int64_t*, float*,
                        float*, uint16_t*, int64_t, int, int, int, int32_t*, int32_t*, hipStream_t);
int64_t router_rank_tile(int64_t, int64_t);
int launch_router_split(const float*, uint16_t*, int, int, hipStream_t);
int64_t router_scratch_bytes(int64_t, int64_t);
int64_t dispatch_scratch_bytes(int64_t, int64_t, int64_t);
int launch_dispatch(const void*, int, const int32_t*, int32_t*, int32_t*, int32_t*, void*,
                    int32_t*, int32_t*, int64_t, int64_t, int, int, int, int64_t, bool, hipStream_t);
int launch_dispatch_ranked(const void*, int, const int32_t*, int32_t*, int32_t*, int32_t*, void*, int32_t*,
                           const int32_t*, const int32_t*, int64_t, int64_t, int64_t, int, int, int, int64_t, bool,
                           hipStream_t);
int launch_combine(const void*, int, const int32_t*, const float*, void*, int64_t, int64_t, int,
                   int64_t, hipStream_t);
int launch_swiglu(const void*, int, const int32_t*, void*, int64_t, int64_t, hipStream_t);
int launch_grouped_gemm(const uint16_t*, const uint16_t*, int64_t, uint16_t*, const int32_t*, int64_t,
                        int64_t, int64_t, int, hipStream_t);
int launch_gateup_swiglu(const uint16_t*, const uint16_t*, int64_t, uint16_t*, const int32_t*, int64_t,
                         int64_t, int64_t, int, hipStream_t);
int launch_gateup_swiglu_gathered(const uint16_t*, const int32_t*, int64_t, const uint16_t*, int64_t, uint16_t*,
                                  const int32_t*, int64_t, int64_t, int64_t, int, hipStream_t);
int launch_dispatch_rows(const int32_t*, int32_t*, int32_t*, int32_t*, int32_t*, int32_t*, const int32_t*, int32_t*,
                         int64_t, int64_t, int, int, int, int64_t, hipStream_t);
void set_gemm_workgroup_limit(int);

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
}

int fail(int status, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return status;
}

int check_launch(const char* what) {
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return fail(MOE_ERR_HIP, "%s: %s", what, hipGetErrorString(err));
    return MOE_OK;
}

static bool valid_dtype(int dtype) {
    return dtype == MOE_DTYPE_F32 || dtype == MOE_DTYPE_F16 || dtype == MOE_DTYPE_BF16;
}

// True when p is a multiple of `bytes` (a null pointer counts as aligned: the
// null checks report it).
static bool aligned_to(const void* p, uintptr_t bytes) {
    return reinterpret_cast<uintptr_t>(p) % bytes == 0;
}

static int64_t aligned_capacity(int64_t n, int64_t experts, int64_t alignment) {
    if (alignment == 1) return n;
    return (n + experts * (alignment - 1) + 1 + alignment - 1) / alignment * alignment;
}

}  // namespace moe

using namespace moe;

extern "C" {

int moe_abi_version(void) { return MOE_ABI_VERSION; }

const char* moe_status_string(int status) {
    switch (status) {
        case MOE_OK: return "ok";
        case MOE_ERR_INVALID_ARGUMENT: return "invalid argument";
        case MOE_ERR_UNSUPPORTED: return "unsupported configuration";
        case MOE_ERR_CAPACITY: return "exceeds int32 indexing capacity";
        case MOE_ERR_WORKSPACE: return "workspace too small";
        case MOE_ERR_HIP: return "HIP runtime error";
        default: return "unknown status";
    }
}

const char* moe_last_error(void) { return g_last_error; }

int moe_topk_route(const float* logits, const float* bias, int32_t* ids32, int64_t* ids64,
                   float* weights, int64_t tokens, int64_t experts, int64_t topk, void* stream) {
    MOE_REQUIRE(tokens >= 0, MOE_ERR_INVALID_ARGUMENT, "tokens must be >= 0");
    MOE_REQUIRE(experts >= 1 && experts <= kMaxExperts, MOE_ERR_UNSUPPORTED,
                "routing supports 1..64 experts (got %lld)", (long long)experts);
    MOE_REQUIRE(topk >= 1 && topk <= kMaxTopk && topk <= experts, MOE_ERR_UNSUPPORTED,
                "topk must be in 1..min(experts, 8) (got %lld)", (long long)topk);
    MOE_REQUIRE(tokens <= INT_MAX / experts, MOE_ERR_CAPACITY, "tokens*experts exceeds int32");
    if (tokens == 0) return MOE_OK;
    MOE_REQUIRE(logits && bias && ids32 && weights, MOE_ERR_INVALID_ARGUMENT, "null pointer");
    MOE_REQUIRE(aligned_to(logits, 4) && aligned_to(bias, 4) && aligned_to(ids32, 4) &&
                    aligned_to(weights, 4) && aligned_to(ids64, 8),
                MOE_ERR_INVALID_ARGUMENT, "pointers must be aligned to their element size");
    return launch_topk_route(logits, bias, ids32, ids64, weights, tokens, (int)experts, (int)topk,
                             static_cast<hipStream_t>(stream));
}

int64_t moe_router_scratch_bytes(int64_t experts, int64_t hidden) {
    if (experts < 1 || experts > kMaxExperts || hidden < 8 || hidden % 8 != 0) return -1;
    return router_scratch_bytes(experts, hidden);
}

// The fused router's checks (both entry points); MOE_OK when it may launch.
static int check_router_fused(const void* x, const float* router_w, const float* bias, int32_t* ids32,
                              int64_t* ids64, float* weights, float* logits_out, void* scratch,
                              int64_t scratch_bytes, int64_t tokens, int64_t hidden, int64_t experts,
                              int64_t topk) {
    MOE_REQUIRE(tokens >= 0, MOE_ERR_INVALID_ARGUMENT, "tokens must be >= 0");
    MOE_REQUIRE(hidden >= 8 && hidden % 8 == 0 && hidden <= INT_MAX, MOE_ERR_UNSUPPORTED,
                "fused router needs hidden a positive multiple of 8");
    MOE_REQUIRE(experts >= 1 && experts <= kMaxExperts, MOE_ERR_UNSUPPORTED,
                "routing supports 1..64 experts");
    MOE_REQUIRE(topk >= 1 && topk <= kMaxTopk && topk <= experts, MOE_ERR_UNSUPPORTED,
                "topk must be in 1..min(experts, 8)");
    MOE_REQUIRE(tokens <= INT_MAX / experts, MOE_ERR_CAPACITY, "tokens*experts exceeds int32");
    if (tokens == 0) return MOE_OK;
    // router_w == NULL: scratch already holds the split planes.
    MOE_REQUIRE(x && bias && ids32 && weights, MOE_ERR_INVALID_ARGUMENT, "null pointer");
    const int64_t need = router_scratch_bytes(experts, hidden);
    MOE_REQUIRE(scratch && scratch_bytes >= need, MOE_ERR_WORKSPACE,
                "router scratch needs %lld bytes, got %lld", (long long)need, (long long)scratch_bytes);
    // x, the weights and the scratch planes are read with 16-byte (direct-to-LDS) loads.
    MOE_REQUIRE(aligned_to(x, 16) && aligned_to(scratch, 16) && aligned_to(router_w, 16),
                MOE_ERR_INVALID_ARGUMENT, "x, router weights and scratch must be 16-byte aligned");
    MOE_REQUIRE(aligned_to(bias, 4) && aligned_to(ids32, 4) && aligned_to(weights, 4) &&
                    aligned_to(logits_out, 4) && aligned_to(ids64, 8),
                MOE_ERR_INVALID_ARGUMENT, "pointers must be aligned to their element size");
    return MOE_OK;
}

int moe_router_fused(const void* x, const float* router_w, const float* bias, int32_t* ids32,
                     int64_t* ids64, float* weights, float* logits_out, void* scratch,
                     int64_t scratch_bytes, int64_t tokens, int64_t hidden, int64_t experts,
                     int64_t topk, void* stream) {
    const int rc = check_router_fused(x, router_w, bias, ids32, ids64, weights, logits_out, scratch,
                                      scratch_bytes, tokens, hidden, experts, topk);
    if (rc != MOE_OK || tokens == 0) return rc;
    return launch_router_fused(static_cast<const uint16_t*>(x), router_w, bias, ids32, ids64,
                               weights, logits_out, static_cast<uint16_t*>(scratch), tokens,
                               (int)hidden, (int)experts, (int)topk, nullptr, nullptr,
                               static_cast<hipStream_t>(stream));
}

int64_t moe_router_rank_tile(int64_t tokens, int64_t experts) {
    if (tokens < 0 || experts < 1 || experts > kMaxExperts) return -1;
    return router_rank_tile(tokens, experts);
}

int moe_router_fused_ranked(const void* x, const float* router_w, const float* bias, int32_t* ids32,
                            int64_t* ids64, float* weights, float* logits_out, void* scratch,
                            int64_t scratch_bytes, int64_t tokens, int64_t hidden, int64_t experts,
                            int64_t topk, int32_t* ranks, int32_t* tile_counts, int64_t tile_counts_bytes,
                            void* stream) {
    const int rc = check_router_fused(x, router_w, bias, ids32, ids64, weights, logits_out, scratch,
                                      scratch_bytes, tokens, hidden, experts, topk);
    if (rc != MOE_OK || tokens == 0) return rc;
    const int64_t tile = router_rank_tile(tokens, experts);
    MOE_REQUIRE(tile > 0, MOE_ERR_UNSUPPORTED,
                "ranked routing needs ceil(tokens/tile) * experts <= 4096 (moe_router_rank_tile returned 0)");
    const int64_t need = (tokens + tile - 1) / tile * experts * 4;
    MOE_REQUIRE(tile_counts_bytes >= need, MOE_ERR_WORKSPACE, "tile counts need %lld bytes, got %lld",
                (long long)need, (long long)tile_counts_bytes);
    MOE_REQUIRE(ranks && tile_counts, MOE_ERR_INVALID_ARGUMENT, "null pointer");
    MOE_REQUIRE(aligned_to(ranks, 4) && aligned_to(tile_counts, 4), MOE_ERR_INVALID_ARGUMENT,
                "index buffers must be 4-byte aligned");
    return launch_router_fused(static_cast<const uint16_t*>(x), router_w, bias, ids32, ids64,
                               weights, logits_out, static_cast<uint16_t*>(scratch), tokens,
                               (int)hidden, (int)experts, (int)topk, ranks, tile_counts,
                               static_cast<hipStream_t>(stream));
}

int moe_router_split(const float* router_w, void* scratch, int64_t scratch_bytes, int64_t experts,
                     int64_t hidden, void* stream) {
    MOE_REQUIRE(hidden >= 8 && hidden % 8 == 0 && hidden <= (1 << 20), MOE_ERR_UNSUPPORTED,
                "fused router needs hidden a positive multiple of 8 up to 1048576");
    MOE_REQUIRE(experts >= 1 && experts <= kMaxExperts, MOE_ERR_UNSUPPORTED, "routing supports 1..64 experts");
    const int64_t need = router_scratch_bytes(experts, hidden);
    MOE_REQUIRE(router_w && scratch, MOE_ERR_INVALID_ARGUMENT, "null pointer");
    MOE_REQUIRE(scratch_bytes >= need, MOE_ERR_WORKSPACE, "router scratch needs %lld bytes, got %lld",
                (long long)need, (long long)scratch_bytes);
    MOE_REQUIRE(aligned_to(router_w, 16) && aligned_to(scratch, 16), MOE_ERR_INVALID_ARGUMENT,
                "router weights and scratch must be 16-byte aligned");
    return launch_router_split(router_w, static_cast<uint16_t*>(scratch), (int)experts, (int)hidden,
                               static_cast<hipStream_t>(stream));
}

int64_t moe_dispatch_scratch_bytes(int64_t tokens, int64_t experts, int64_t topk) {
    if (tokens < 0 || experts < 1 || experts > kMaxExperts || topk < 1 || topk > kMaxTopk)
        return -1;
    return dispatch_scratch_bytes(tokens, experts, topk);
}

// The dispatch checks shared by moe_dispatch and moe_dispatch_ranked (all but the scratch).
static int check_dispatch(const void* x, int dtype, const int32_t* ids, int32_t* counts, int32_t* offsets,
                          int32_t* slots, void* packed, int32_t* inverse, int64_t tokens, int64_t hidden,
                          int64_t experts, int64_t topk, int64_t alignment, int64_t packed_rows) {
    MOE_REQUIRE(valid_dtype(dtype), MOE_ERR_INVALID_ARGUMENT, "only FP32, FP16 and BF16 are supported");
    MOE_REQUIRE(tokens >= 0 && hidden > 0, MOE_ERR_INVALID_ARGUMENT, "incompatible token dimensions");
    MOE_REQUIRE(experts >= 1 && experts <= kMaxExperts, MOE_ERR_UNSUPPORTED, "supports 1..64 experts");
    MOE_REQUIRE(topk >= 1 && topk <= kMaxTopk, MOE_ERR_UNSUPPORTED, "topk must be in 1..8");
    MOE_REQUIRE(alignment >= 1 && alignment <= 128, MOE_ERR_INVALID_ARGUMENT, "alignment must be 1..128");
    const int64_t n = tokens * topk;
    const int64_t required = aligned_capacity(n, experts, alignment);
    MOE_REQUIRE(n <= INT_MAX && hidden <= INT_MAX && required <= INT_MAX, MOE_ERR_CAPACITY,
                "shape exceeds int32 indexing capacity");
    MOE_REQUIRE(packed_rows >= required, MOE_ERR_WORKSPACE,
                "packed workspace has %lld rows, needs %lld", (long long)packed_rows,
                (long long)required);
    MOE_REQUIRE(counts && offsets, MOE_ERR_INVALID_ARGUMENT, "null pointer");
    MOE_REQUIRE(n == 0 || (x && ids && slots && packed && inverse), MOE_ERR_INVALID_ARGUMENT,
                "null pointer");
    return MOE_OK;
}

static int check_dispatch_alignment(const void* x, int dtype, void* packed, const int32_t* ids, int32_t* counts,
                                    int32_t* offsets, int32_t* slots, int32_t* inverse, const void* table) {
    // Rows are copied with the widest access that the row size and both base
    // addresses allow (launch_dispatch), down to one element.
    const uintptr_t elem = static_cast<uintptr_t>(dtype_size(dtype));
    MOE_REQUIRE(aligned_to(x, elem) && aligned_to(packed, elem), MOE_ERR_INVALID_ARGUMENT,
                "x and packed must be aligned to their element size");
    MOE_REQUIRE(aligned_to(ids, 4) && aligned_to(counts, 4) && aligned_to(offsets, 4) &&
                    aligned_to(slots, 4) && aligned_to(inverse, 4) && aligned_to(table, 4),
                MOE_ERR_INVALID_ARGUMENT, "index buffers must be 4-byte aligned");
    return MOE_OK;
}

int moe_dispatch(const void* x, int dtype, const int32_t* ids, int32_t* counts, int32_t* offsets,
                 int32_t* slots, void* packed, int32_t* inverse, void* scratch,
                 int64_t scratch_bytes, int64_t tokens, int64_t hidden, int64_t experts,
                 int64_t topk, int64_t alignment, int64_t packed_rows, int vectorized,
                 void* stream) {
    const int rc = check_dispatch(x, dtype, ids, counts, offsets, slots, packed, inverse, tokens, hidden,
                                  experts, topk, alignment, packed_rows);
    if (rc != MOE_OK) return rc;
    const int64_t need = dispatch_scratch_bytes(tokens, experts, topk);
    MOE_REQUIRE(scratch_bytes >= need, MOE_ERR_WORKSPACE, "dispatch scratch has %lld bytes, needs %lld",
                (long long)scratch_bytes, (long long)need);
    MOE_REQUIRE(scratch, MOE_ERR_INVALID_ARGUMENT, "null pointer");
    const int ra = check_dispatch_alignment(x, dtype, packed, ids, counts, offsets, slots, inverse, scratch);
    if (ra != MOE_OK) return ra;
    return launch_dispatch(x, dtype, ids, counts, offsets, slots, packed, inverse,
                           static_cast<int32_t*>(scratch), tokens, hidden, (int)experts, (int)topk,
                           (int)alignment, packed_rows, vectorized != 0, static_cast<hipStream_t>(stream));
}

int moe_dispatch_ranked(const void* x, int dtype, const int32_t* ids, int32_t* counts, int32_t* offsets,
                        int32_t* slots, void* packed, int32_t* inverse, const int32_t* ranks,
                        const int32_t* tile_counts, int64_t tile_counts_bytes, int64_t tile_tokens, int64_t tokens,
                        int64_t hidden, int64_t experts, int64_t topk, int64_t alignment, int64_t packed_rows,
                        int vectorized, void* stream) {
    const int rc = check_dispatch(x, dtype, ids, counts, offsets, slots, packed, inverse, tokens, hidden,
                                  experts, topk, alignment, packed_rows);
    if (rc != MOE_OK) return rc;
    const int64_t tile = router_rank_tile(tokens, experts);
    MOE_REQUIRE(tokens == 0 || (tile > 0 && tile_tokens == tile), MOE_ERR_INVALID_ARGUMENT,
                "tile_tokens %lld is not the ranked route's tile (%lld) for this shape", (long long)tile_tokens,
                (long long)tile);
    if (tokens > 0) {
        const int64_t need = (tokens + tile - 1) / tile * experts * 4;
        MOE_REQUIRE(tile_counts_bytes >= need, MOE_ERR_WORKSPACE, "tile counts need %lld bytes, got %lld",
                    (long long)need, (long long)tile_counts_bytes);
        MOE_REQUIRE(ranks && tile_counts, MOE_ERR_INVALID_ARGUMENT, "null pointer");
    }
    int ra = check_dispatch_alignment(x, dtype, packed, ids, counts, offsets, slots, inverse, tile_counts);
    if (ra != MOE_OK) return ra;
    MOE_REQUIRE(aligned_to(ranks, 4), MOE_ERR_INVALID_ARGUMENT, "index buffers must be 4-byte aligned");
    if (tokens == 0)  // no assignments: counts and offsets are zero (no tile table is read)
        return launch_dispatch(x, dtype, ids, counts, offsets, slots, packed, inverse, nullptr, tokens, hidden,
                               (int)experts, (int)topk, (int)alignment, packed_rows, vectorized != 0,
                               static_cast<hipStream_t>(stream));
    return launch_dispatch_ranked(x, dtype, ids, counts, offsets, slots, packed, inverse, ranks, tile_counts,
                                  tile, tokens, hidden, (int)experts, (int)topk, (int)alignment, packed_rows,
                                  vectorized != 0, static_cast<hipStream_t>(stream));
}

// The checks of the row-table dispatch entry points (no x, no packed rows).
static int check_dispatch_rows(const int32_t* ids, int32_t* counts, int32_t* offsets, int32_t* slots,
                               int32_t* inverse, int32_t* row_src, const void* table, int64_t tokens,
                               int64_t experts, int64_t topk, int64_t alignment, int64_t packed_rows) {
    MOE_REQUIRE(tokens >= 0, MOE_ERR_INVALID_ARGUMENT, "incompatible token dimensions");
    MOE_REQUIRE(experts >= 1 && experts <= kMaxExperts, MOE_ERR_UNSUPPORTED, "supports 1..64 experts");
    MOE_REQUIRE(topk >= 1 && topk <= kMaxTopk, MOE_ERR_UNSUPPORTED, "topk must be in 1..8");
    MOE_REQUIRE(alignment >= 1 && alignment <= 128, MOE_ERR_INVALID_ARGUMENT, "alignment must be 1..128");
    const int64_t n = tokens * topk;
    const int64_t required = aligned_capacity(n, experts, alignment);
    MOE_REQUIRE(n <= INT_MAX && required <= INT_MAX, MOE_ERR_CAPACITY, "shape exceeds int32 indexing capacity");
    MOE_REQUIRE(packed_rows >= required, MOE_ERR_WORKSPACE, "row table has %lld rows, needs %lld",
                (long long)packed_rows, (long long)required);
    MOE_REQUIRE(counts && offsets, MOE_ERR_INVALID_ARGUMENT, "null pointer");
    MOE_REQUIRE(n == 0 || (ids && slots && inverse && row_src), MOE_ERR_INVALID_ARGUMENT, "null pointer");
    MOE_REQUIRE(aligned_to(ids, 4) && aligned_to(counts, 4) && aligned_to(offsets, 4) && aligned_to(slots, 4) &&
                    aligned_to(inverse, 4) && aligned_to(row_src, 4) && aligned_to(table, 4),
                MOE_ERR_INVALID_ARGUMENT, "index buffers must be 4-byte aligned");
    return MOE_OK;
}

int moe_dispatch_rows(const int32_t* ids, int32_t* counts, int32_t* offsets, int32_t* slots, int32_t* inverse,
                      int32_t* row_src, void* scratch, int64_t scratch_bytes, int64_t tokens, int64_t experts,
                      int64_t topk, int64_t alignment, int64_t packed_rows, void* stream) {
    const int rc = check_dispatch_rows(ids, counts, offsets, slots, inverse, row_src, scratch, tokens, experts,
                                       topk, alignment, packed_rows);
    if (rc != MOE_OK) return rc;
    const int64_t need = dispatch_scratch_bytes(tokens, experts, topk);
    MOE_REQUIRE(scratch_bytes >= need, MOE_ERR_WORKSPACE, "dispatch scratch has %lld bytes, needs %lld",
                (long long)scratch_bytes, (long long)need);
    MOE_REQUIRE(scratch, MOE_ERR_INVALID_ARGUMENT, "null pointer");
    return launch_dispatch_rows(ids, counts, offsets, slots, inverse, row_src, nullptr, static_cast<int32_t*>(scratch),
                                0, tokens, (int)experts, (int)topk, (int)alignment, packed_rows,
                                static_cast<hipStream_t>(stream));
}

int moe_dispatch_ranked_rows(const int32_t* ids, int32_t* counts, int32_t* offsets, int32_t* slots,
                             int32_t* inverse, int32_t* row_src, const int32_t* ranks, const int32_t* tile_counts,
                             int64_t tile_counts_bytes, int64_t tile_tokens, int64_t tokens, int64_t experts,
                             int64_t topk, int64_t alignment, int64_t packed_rows, void* stream) {
    const int rc = check_dispatch_rows(ids, counts, offsets, slots, inverse, row_src, tile_counts, tokens, experts,
                                       topk, alignment, packed_rows);
    if (rc != MOE_OK) return rc;
    const int64_t tile = router_rank_tile(tokens, experts);
    MOE_REQUIRE(tokens == 0 || (tile > 0 && tile_tokens == tile), MOE_ERR_INVALID_ARGUMENT,
                "tile_tokens %lld is not the ranked route's tile (%lld) for this shape", (long long)tile_tokens,
                (long long)tile);
    if (tokens > 0) {
        const int64_t need = (tokens + tile - 1) / tile * experts * 4;
        MOE_REQUIRE(tile_counts_bytes >= need, MOE_ERR_WORKSPACE, "tile counts need %lld bytes, got %lld",
                    (long long)need, (long long)tile_counts_bytes);
        MOE_REQUIRE(ranks && tile_counts, MOE_ERR_INVALID_ARGUMENT, "null pointer");
    }
    MOE_REQUIRE(aligned_to(ranks, 4), MOE_ERR_INVALID_ARGUMENT, "index buffers must be 4-byte aligned");
    if (tokens == 0)  // no assignments: counts and offsets are zero (the count-in-pack path reads no table)
        return launch_dispatch_rows(ids, counts, offsets, slots, inverse, row_src, nullptr, nullptr, 0, tokens,
                                    (int)experts, (int)topk, (int)alignment, packed_rows,
                                    static_cast<hipStream_t>(stream));
    return launch_dispatch_rows(ids, counts, offsets, slots, inverse, row_src, ranks,
                                const_cast<int32_t*>(tile_counts), tile, tokens, (int)experts, (int)topk,
                                (int)alignment, packed_rows, static_cast<hipStream_t>(stream));
}

int moe_combine(const void* expert_output, int dtype, const int32_t* inverse,
                const float* weights, void* output, int64_t tokens, int64_t hidden,
                int64_t topk, int64_t packed_rows, void* stream) {
    MOE_REQUIRE(valid_dtype(dtype), MOE_ERR_INVALID_ARGUMENT, "unsupported output dtype");
    MOE_REQUIRE(topk >= 1 && topk <= kMaxTopk, MOE_ERR_UNSUPPORTED, "topk must be in 1..8");
    MOE_REQUIRE(tokens >= 0 && hidden > 0, MOE_ERR_INVALID_ARGUMENT, "invalid output shape");
    MOE_REQUIRE(tokens * topk <= INT_MAX && hidden <= INT_MAX && packed_rows <= INT_MAX,
                MOE_ERR_CAPACITY, "invalid output shape");
    MOE_REQUIRE(packed_rows >= tokens * topk, MOE_ERR_INVALID_ARGUMENT, "shape/dtype mismatch");
    if (tokens == 0) return MOE_OK;
    MOE_REQUIRE(expert_output && inverse && weights && output, MOE_ERR_INVALID_ARGUMENT, "null pointer");
    // 16-byte vectors when both row arrays allow them (launch_combine), else elements.
    const uintptr_t elem = static_cast<uintptr_t>(dtype_size(dtype));
    MOE_REQUIRE(aligned_to(expert_output, elem) && aligned_to(output, elem), MOE_ERR_INVALID_ARGUMENT,
                "expert output and output must be aligned to their element size");
    MOE_REQUIRE(aligned_to(inverse, 4) && aligned_to(weights, 4), MOE_ERR_INVALID_ARGUMENT,
                "inverse and weights must be 4-byte aligned");
    return launch_combine(expert_output, dtype, inverse, weights, output, tokens, hidden,
                          (int)topk, packed_rows, static_cast<hipStream_t>(stream));
}

int moe_swiglu(const void* projection, int dtype, const int32_t* valid_rows, void* output,
               int64_t rows, int64_t width, void* stream) {
    MOE_REQUIRE(valid_dtype(dtype), MOE_ERR_INVALID_ARGUMENT, "unsupported dtype");
    MOE_REQUIRE(rows >= 0 && width >= 0 && rows <= INT_MAX && width <= INT_MAX, MOE_ERR_CAPACITY,
                "shape exceeds index capacity");
    if (rows * width == 0) return MOE_OK;
    MOE_REQUIRE(projection && valid_rows && output, MOE_ERR_INVALID_ARGUMENT, "null pointer");
    const uintptr_t elem = static_cast<uintptr_t>(dtype_size(dtype));
    MOE_REQUIRE(aligned_to(projection, elem) && aligned_to(output, elem) && aligned_to(valid_rows, 4),
                MOE_ERR_INVALID_ARGUMENT, "pointers must be aligned to their element size");
    return launch_swiglu(projection, dtype, valid_rows, output, rows, width,
                         static_cast<hipStream_t>(stream));
}

// The weights' row stride: at least the row length, a multiple of 8 (rows
// start 16-byte aligned), and with rows * stride within the kernels' 32-bit
// buffer ranges (one expert's weights, and a 256-row tile).
static int check_row_stride(int64_t stride, int64_t k, int64_t weight_rows) {
    MOE_REQUIRE(stride >= k && stride % 8 == 0 && stride <= INT_MAX, MOE_ERR_UNSUPPORTED,
                "weight row stride must be a multiple of 8 and at least the row length");
    MOE_REQUIRE(256 * stride * 2 <= UINT32_MAX && weight_rows <= UINT32_MAX / (2 * stride), MOE_ERR_CAPACITY,
                "one expert's weight matrix must be below 4 GiB");
    return MOE_OK;
}

int moe_grouped_gemm(const void* a, const void* b, void* c, const int32_t* offsets, int64_t rows,
                     int64_t n, int64_t k, int64_t experts, void* stream) {
    return moe_grouped_gemm_strided(a, b, k, c, offsets, rows, n, k, experts, stream);
}

int moe_grouped_gemm_strided(const void* a, const void* b, int64_t b_row_stride, void* c, const int32_t* offsets,
                             int64_t rows, int64_t n, int64_t k, int64_t experts, void* stream) {
    MOE_REQUIRE(experts >= 1 && experts <= kMaxExperts, MOE_ERR_UNSUPPORTED, "supports 1..64 experts");
    MOE_REQUIRE(rows >= 0 && rows <= INT_MAX, MOE_ERR_CAPACITY, "rows exceed int32");
    MOE_REQUIRE(n > 0 && k > 0 && n % 8 == 0 && k % 8 == 0, MOE_ERR_UNSUPPORTED,
                "grouped GEMM dimensions must be positive multiples of 8");
    // The kernels bound each expert's weights and row tile with 32-bit buffer ranges.
    MOE_REQUIRE(n <= INT_MAX && k <= INT_MAX, MOE_ERR_CAPACITY, "one expert's weight matrix must be below 4 GiB");
    if (int status = check_row_stride(b_row_stride, k, n); status != MOE_OK) return status;
    if (rows == 0) return MOE_OK;
    MOE_REQUIRE(a && b && c && offsets, MOE_ERR_INVALID_ARGUMENT, "null pointer");
    // Operands are read with 16-byte buffer loads and results stored 8 bytes at a time.
    MOE_REQUIRE(aligned_to(a, 16) && aligned_to(b, 16) && aligned_to(c, 16) && aligned_to(offsets, 4),
                MOE_ERR_INVALID_ARGUMENT, "a, b and c must be 16-byte aligned (offsets 4-byte)");
    return launch_grouped_gemm(static_cast<const uint16_t*>(a), static_cast<const uint16_t*>(b), b_row_stride,
                               static_cast<uint16_t*>(c), offsets, rows, n, k, (int)experts,
                               static_cast<hipStream_t>(stream));
}

int moe_grouped_gateup_swiglu(const void* a, const void* gate_up, void* act,
                              const int32_t* offsets, int64_t rows, int64_t hidden,
                              int64_t intermediate, int64_t experts, void* stream) {
    return moe_grouped_gateup_swiglu_strided(a, gate_up, hidden, act, offsets, rows, hidden, intermediate, experts,
                                             stream);
}

int moe_grouped_gateup_swiglu_strided(const void* a, const void* gate_up, int64_t gate_up_row_stride, void* act,
                                      const int32_t* offsets, int64_t rows, int64_t hidden, int64_t intermediate,
                                      int64_t experts, void* stream) {
    MOE_REQUIRE(experts >= 1 && experts <= kMaxExperts, MOE_ERR_UNSUPPORTED, "supports 1..64 experts");
    MOE_REQUIRE(rows >= 0 && rows <= INT_MAX, MOE_ERR_CAPACITY, "rows exceed int32");
    MOE_REQUIRE(hidden > 0 && intermediate > 0 && hidden % 8 == 0 && intermediate % 8 == 0,
                MOE_ERR_UNSUPPORTED, "grouped GEMM dimensions must be positive multiples of 8");
    MOE_REQUIRE(hidden <= INT_MAX && intermediate <= INT_MAX, MOE_ERR_CAPACITY,
                "one expert's weight matrix must be below 4 GiB");
    if (int status = check_row_stride(gate_up_row_stride, hidden, 2 * intermediate); status != MOE_OK) return status;
    if (rows == 0) return MOE_OK;
    MOE_REQUIRE(a && gate_up && act && offsets, MOE_ERR_INVALID_ARGUMENT, "null pointer");
    MOE_REQUIRE(aligned_to(a, 16) && aligned_to(gate_up, 16) && aligned_to(act, 16) && aligned_to(offsets, 4),
                MOE_ERR_INVALID_ARGUMENT, "a, gate_up and act must be 16-byte aligned (offsets 4-byte)");
    return launch_gateup_swiglu(static_cast<const uint16_t*>(a), static_cast<const uint16_t*>(gate_up),
                                gate_up_row_stride, static_cast<uint16_t*>(act),
                                offsets, rows, hidden, intermediate, (int)experts,
                                static_cast<hipStream_t>(stream));
}

int moe_grouped_gateup_swiglu_gathered(const void* x, const int32_t* row_src, int64_t x_rows, const void* gate_up,
                                       void* act, const int32_t* offsets, int64_t rows, int64_t hidden,
                                       int64_t intermediate, int64_t experts, void* stream) {
    return moe_grouped_gateup_swiglu_gathered_strided(x, row_src, x_rows, gate_up, hidden, act, offsets, rows, hidden,
                                                      intermediate, experts, stream);
}

int moe_grouped_gateup_swiglu_gathered_strided(const void* x, const int32_t* row_src, int64_t x_rows,
                                               const void* gate_up, int64_t gate_up_row_stride, void* act,
                                               const int32_t* offsets, int64_t rows, int64_t hidden,
                                               int64_t intermediate, int64_t experts, void* stream) {
    MOE_REQUIRE(experts >= 1 && experts <= kMaxExperts, MOE_ERR_UNSUPPORTED, "supports 1..64 experts");
    MOE_REQUIRE(rows >= 0 && rows <= INT_MAX && x_rows >= 0 && x_rows <= INT_MAX, MOE_ERR_CAPACITY,
                "rows exceed int32");
    MOE_REQUIRE(hidden > 0 && intermediate > 0 && hidden % 64 == 0 && intermediate % 8 == 0, MOE_ERR_UNSUPPORTED,
                "gathered gate/up needs hidden a positive multiple of 64 and intermediate of 8");
    MOE_REQUIRE(hidden <= INT_MAX && intermediate <= INT_MAX, MOE_ERR_CAPACITY,
                "one expert's weight matrix must be below 4 GiB");
    if (int status = check_row_stride(gate_up_row_stride, hidden, 2 * intermediate); status != MOE_OK) return status;
    // x is one buffer of 32-bit offsets, with 2 GiB and up left for the out-of-range marker.
    MOE_REQUIRE(x_rows * hidden * 2 < (int64_t{1} << 31), MOE_ERR_CAPACITY, "x must be below 2 GiB");
    if (rows == 0) return MOE_OK;
    MOE_REQUIRE(x && row_src && gate_up && act && offsets, MOE_ERR_INVALID_ARGUMENT, "null pointer");
    MOE_REQUIRE(aligned_to(x, 16) && aligned_to(gate_up, 16) && aligned_to(act, 16) && aligned_to(offsets, 4) &&
                    aligned_to(row_src, 4),
                MOE_ERR_INVALID_ARGUMENT, "x, gate_up and act must be 16-byte aligned (index buffers 4-byte)");
    return launch_gateup_swiglu_gathered(static_cast<const uint16_t*>(x), row_src, x_rows,
                                         static_cast<const uint16_t*>(gate_up), gate_up_row_stride,
                                         static_cast<uint16_t*>(act), offsets,
                                         rows, hidden, intermediate, (int)experts, static_cast<hipStream_t>(stream));
}

int moe_set_gemm_workgroups(int64_t workgroups) {
    MOE_REQUIRE(workgroups >= 0 && workgroups <= INT_MAX, MOE_ERR_INVALID_ARGUMENT,
                "workgroups must be in [0, INT_MAX]");
    set_gemm_workgroup_limit(static_cast<int>(workgroups));
    return MOE_OK;
}

}  // extern "C"
