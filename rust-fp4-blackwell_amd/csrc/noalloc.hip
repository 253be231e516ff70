// Allocation-free attention (attn_decode_f16_noalloc, include/rfp4.h): for
// callers that cannot allocate device memory (code under HIP graph capture,
// tight serving loops, harnesses that forbid hipMalloc).  Its split-K states
// live in a file-scope device array instead of the library workspace that
// rfp4_init allocates, so the call allocates nothing: no hipMalloc, no
// hipFree, no allocating library routine.
//
// The array is a host-side stand-in in host code: its device address is
// looked up once per device with hipGetSymbolAddress (noalloc_setup, called
// by rfp4_init with that device current) and only that address is handed to
// kernels.  Every call on a device shares the device's copy, which keeps the
// last call's contents: calls that overlap on one device race.  Each call
// writes every split state it reads before reading it (the split kernel
// writes all states of the call, the merge kernel then reads them, in stream
// order), so nothing in the array must start at zero.
#include <hip/hip_runtime.h>

#include "runtime.h"

namespace {

// [n_heads][splits][head_dim + 4] floats of split state: 4 MiB per device,
// e.g. 32 heads x 248 splits at head_dim 128 (a 35k-token context at the
// library's plan of 144 tokens per split).
constexpr size_t kScratchFloats = (size_t)1 << 20;
static __device__ __align__(256) float scratch[kScratchFloats];

constexpr int kMaxDevices = 64;
float *g_scratch[kMaxDevices]; // per device: the address of its copy (set once, under rfp4_init's lock)

} // namespace

namespace rfp4 {

int noalloc_setup(int device)
{
    if (device < 0 || device >= kMaxDevices)
        return set_error(RFP4_E_INVALID, "noalloc: device %d out of range (%d)", device, kMaxDevices);
    if (g_scratch[device]) return RFP4_OK;
    void *p = nullptr;
    int rc = hip_check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    if (rc) return rc;
    g_scratch[device] = (float *)p;
    return RFP4_OK;
}

} // namespace rfp4

extern "C" int attn_decode_f16_noalloc(rfp4_stream_t stream, uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim,
                                       uint32_t seq, const float *q, const uint16_t *kc, const uint16_t *vc,
                                       uint64_t token_stride, uint64_t head_stride, float *out)
{
    using namespace rfp4;
    Runtime *rt = runtime();
    if (!rt) return set_error(RFP4_E_NOT_INIT, "rfp4_init has not been called");
    float *ptr = (rt->device >= 0 && rt->device < kMaxDevices) ? g_scratch[rt->device] : nullptr;
    if (!ptr) return set_error(RFP4_E_NOT_INIT, "attn_decode_f16_noalloc: scratch of device %d not set up", rt->device);
    return attn_decode_ws((hipStream_t)stream, n_heads, n_kv_heads, head_dim, seq, q, kc, vc, token_stride, head_stride,
                          out, 1, ptr, kScratchFloats, false);
}
