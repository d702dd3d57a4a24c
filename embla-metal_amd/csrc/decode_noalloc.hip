// embla_decode_int8 for callers that cannot allocate (code under HIP graph capture, serving loops
// that forbid hipMalloc): the split-K partials live in a file-scope device array instead of a
// caller workspace. The kernels are embla_decode_int8's (decode_full.hip); only where the partials
// go differs.
//
// The array is `scratch`, 4.125 MiB: 256 chunks x 32 query heads x 132 floats. Each GPU the library
// runs on holds its own copy until the process ends. Host code never passes the array's name to a
// kernel (on the host it is a stand-in symbol, not a device address): the first call on a device
// resolves that device's address with hipGetSymbolAddress, with the device current, and keeps it.
// Every call on one GPU shares that GPU's array, so calls that overlap on one GPU (two streams, or
// two host threads) race; calls on one stream are ordered. Nothing needs clearing between calls:
// the split-K pass writes every partial record the merge then reads.
#include <mutex>
#include "common.hpp"
#include "embla_internal.hpp"

namespace {

constexpr size_t kScratchFloats = (size_t)256 * 32 * 132;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) float scratch[kScratchFloats];

std::mutex g_mu;
float* g_ptr[kMaxDevices];   // scratch's address on each device, once resolved

/// scratch's device address on the current device (resolved once a device), or nullptr.
float* scratch_ptr(int& rc) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        rc = EMBLA_ERR_HIP;
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_ptr[dev]) {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) {
            rc = EMBLA_ERR_HIP;
            return nullptr;
        }
        g_ptr[dev] = (float*)p;
    }
    rc = EMBLA_OK;
    return g_ptr[dev];
}

}  // namespace

extern "C" {

size_t embla_decode_int8_noalloc_max_bytes(void) { return kScratchFloats * sizeof(float); }

int embla_decode_int8_noalloc(const void* q, const void* kc, const void* vc, void* o, float* scores, int S, int max_s,
                              int n_q, int n_kv, int weights, int scale_dtype, int out_dtype, int chunk,
                              hipStream_t stream) {
    if (!q || !kc || !vc || !o) return EMBLA_ERR_INVALID;
    embla::FullDecodeArgs a;
    int rc = embla::full_decode_plan(q, kc, vc, o, scores, S, max_s, n_q, n_kv, weights, scale_dtype, out_dtype,
                                     chunk, a);
    if (rc) return rc;
    if (a.C > 1) {
        if ((size_t)a.C * n_q * 132 > kScratchFloats) return EMBLA_ERR_WORKSPACE;   // beyond the array
        a.part = scratch_ptr(rc);
        if (rc) return rc;
    }
    return embla::launch_full_decode(a, stream);
}

}  // extern "C"
