// ct_forward_linear_static: ct_forward_linear for callers that cannot allocate device
// memory (tight serving loops, harnesses that forbid hipMalloc). Its scratch space -- the split partials of few-row problems and, from 512 rows
// on, the decoded bf16 weight -- lives in one file-scope device array of
// CT_STATIC_SCRATCH_BYTES per GPU instead of a caller's workspace. The array is created
// when the library's code object loads on a device and held until the process ends.
//
// Host code never passes the array's name to a kernel: on the host that name is only a
// stand-in. The device address is looked up once per device with hipGetSymbolAddress
// (with that device current) by ct_init_device, the library's set-up call, and kept;
// every later call on that device uses the kept address (a first static call on a device
// that was never set up looks it up itself). All calls on one GPU share its array, so calls that overlap on one GPU (two
// streams, two threads) race on it; the array keeps the last call's contents, and every
// kernel that reads it first writes what it reads (split partials are fully written
// before the reduction, the decoded weight before the GEMM).

#include <atomic>
#include <mutex>

#include "common.hpp"

static __device__ __align__(256) unsigned char scratch[CT_STATIC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;

std::mutex g_lookup;
std::atomic<void *> g_address[kMaxDevices];

// Device address of the current device's scratch array (looked up once per device).
int scratch_address(void **out) {
    int device = -1;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess) return (int)e;
    if (device < 0 || device >= kMaxDevices) return -CT_EINVAL_SHAPE;
    void *p = g_address[device].load(std::memory_order_acquire);
    if (!p) {
        std::lock_guard<std::mutex> lock(g_lookup);
        p = g_address[device].load(std::memory_order_relaxed);
        if (!p) {
            e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
            if (e != hipSuccess) return (int)e;
            if (!p) return (int)hipErrorInvalidSymbol;
            g_address[device].store(p, std::memory_order_release);
        }
    }
    *out = p;
    return 0;
}

}  // namespace

extern "C" int ct_init_device(void) {
    void *p = nullptr;
    return scratch_address(&p);
}

extern "C" int ct_forward_linear_static(const void *x, int64_t ldx, const void *w_dense, const ct_nf4_weight *w_nf4,
                                        const void *a, const void *b, const void *bias, void *out, int64_t ldo,
                                        void *xa, int64_t ldxa, int32_t xa_given, int64_t m, int64_t n, int64_t k,
                                        int64_t r, const ct_epilogue *epilogue, hipStream_t stream) {
    if (m < 0 || n < 0 || k < 0 || r < 0) return -CT_EINVAL_SHAPE;
    if (m == 0 || n == 0) return 0;
    const int32_t kind = w_nf4 ? (w_nf4->nested ? 1 : 2) : 0;
    const int64_t need = ct_forward_linear_workspace(m, n, k, r, kind);
    if (need < 0 || need > (int64_t)CT_STATIC_SCRATCH_BYTES) return -CT_EINVAL_WORKSPACE;
    void *ws = nullptr;
    if (need > 0) {
        const int st = scratch_address(&ws);
        if (st) return st;
    }
    return ct_forward_linear(x, ldx, w_dense, w_nf4, a, b, bias, out, ldo, xa, ldxa, xa_given, m, n, k, r, epilogue,
                             ws, need, stream);
}
