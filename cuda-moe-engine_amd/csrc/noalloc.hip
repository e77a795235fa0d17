// moe_dispatch_noalloc: moe_dispatch for callers that cannot allocate device
// memory (code under HIP graph capture, tight serving loops, harnesses that
// forbid hipMalloc). The dispatch kernels' only scratch, the per-chunk count
// table, lives in a static device array of this library instead of a buffer
// the caller passes; everything else (inputs, outputs, validation, kernels)
// is moe_dispatch's.
//
// The dispatch plan sizes chunks so that chunks * experts <= 4096 for every
// valid shape (dispatch.hip, plan_dispatch), so 4096 int32 counters always
// suffice. count_rank_kernel writes every counter a call reads, so nothing
// needs clearing between calls. Each GPU holds one copy of the array for the
// life of the process, and every call on that GPU uses it: calls on one GPU
// that overlap in time (different streams, or host threads) race on it.
#include <mutex>

#include "moe_common.h"

namespace moe {

constexpr int64_t kStaticScratchBytes = 16384;

// The static scratch array. In host code its name is a host-side stand-in, not
// a device address: it is never passed to a kernel or a copy. The device
// address of each GPU's copy comes from hipGetSymbolAddress.
static __device__ __align__(256) int32_t scratch[kStaticScratchBytes / sizeof(int32_t)];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mutex;
static void* g_scratch_address[kMaxDevices] = {};

// Device address of the current device's copy of `scratch`, looked up once per
// device. The lookup is a runtime call that graph capture need not allow, so a
// first call on a device while `stream` is capturing is refused with an error
// (make one call on each device before capturing); later calls only read the
// cached address.
static int static_scratch(void** address, hipStream_t stream) {
    int device = -1;
    hipError_t err = hipGetDevice(&device);
    if (err != hipSuccess) return fail(MOE_ERR_HIP, "hipGetDevice: %s", hipGetErrorString(err));
    if (device < 0 || device >= kMaxDevices)
        return fail(MOE_ERR_UNSUPPORTED, "device %d beyond the %d this build tracks", device, kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_address[device] == nullptr) {
        hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
        err = hipStreamIsCapturing(stream, &capture);
        if (err != hipSuccess) return fail(MOE_ERR_HIP, "hipStreamIsCapturing: %s", hipGetErrorString(err));
        if (capture != hipStreamCaptureStatusNone)
            return fail(MOE_ERR_UNSUPPORTED,
                        "the first moe_dispatch_noalloc call on device %d is under graph capture: make one call "
                        "on this device before capturing", device);
        void* ptr = nullptr;
        err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (err != hipSuccess || ptr == nullptr)
            return fail(MOE_ERR_HIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(err));
        g_scratch_address[device] = ptr;
    }
    *address = g_scratch_address[device];
    return MOE_OK;
}

}  // namespace moe

using namespace moe;

extern "C" int moe_dispatch_noalloc(const void* x, int dtype, const int32_t* ids, int32_t* counts,
                                    int32_t* offsets, int32_t* slots, void* packed, int32_t* inverse,
                                    int64_t tokens, int64_t hidden, int64_t experts, int64_t topk,
                                    int64_t alignment, int64_t packed_rows, int vectorized,
                                    void* stream) {
    const int64_t need = moe_dispatch_scratch_bytes(tokens, experts, topk);
    MOE_REQUIRE(need >= 0, MOE_ERR_UNSUPPORTED, "supports T>=0, 1..64 experts and topk 1..8");
    MOE_REQUIRE(need <= kStaticScratchBytes, MOE_ERR_WORKSPACE,
                "dispatch needs %lld bytes of scratch, beyond the static %lld", (long long)need,
                (long long)kStaticScratchBytes);
    void* address = nullptr;
    const int rc = static_scratch(&address, static_cast<hipStream_t>(stream));
    if (rc != MOE_OK) return rc;
    return moe_dispatch(x, dtype, ids, counts, offsets, slots, packed, inverse, address,
                        kStaticScratchBytes, tokens, hidden, experts, topk, alignment, packed_rows,
                        vectorized, stream);
}
