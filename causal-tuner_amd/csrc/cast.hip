// Several fp32 tensors rounded to bf16 in one launch, gfx950: the per-call casts of a
// projection group's fp32 LoRA factors to the compute dtype (the reference's a.to(dtype),
// b.to(dtype) for every projection in kernels/linear.py:70,108 and kernels/mlp_cuda.py:62,
// 110), which otherwise cost one launch per tensor. Round to nearest even, NaN kept quiet,
// as torch's cast. HBM-bound: 4 bytes read and 2 written per element.
//
// The table of tensors travels in the kernel arguments (no device-side table, so nothing
// is copied from the host per call). Workgroup b converts elements [b, b + 1) * kSpan of
// the tensors laid end to end; 8 elements per lane per step with 16-byte loads where the
// tensor and its offset allow it.

#include "common.hpp"

namespace ct {
namespace {

constexpr int kCastThreads = 256;
constexpr int64_t kSpan = 8 * kCastThreads * 4;  // elements per workgroup

struct CastTable {
    const float *src[CT_CAST_MAX];
    uint16_t *dst[CT_CAST_MAX];
    int64_t begin[CT_CAST_MAX + 1];  // prefix sums of the element counts
    int count;
};

__global__ __launch_bounds__(kCastThreads) void cast_f32_bf16(const CastTable t) {
    const int64_t g0 = (int64_t)blockIdx.x * kSpan;
    const int64_t g1 = g0 + kSpan < t.begin[t.count] ? g0 + kSpan : t.begin[t.count];
    // the tensors overlapping [g0, g1): a workgroup may straddle several small ones
    for (int i = 0; i < t.count; ++i) {
        const int64_t lo = t.begin[i] > g0 ? t.begin[i] : g0;
        const int64_t hi = t.begin[i + 1] < g1 ? t.begin[i + 1] : g1;
        if (lo >= hi) continue;
        const float *src = t.src[i];
        uint16_t *dst = t.dst[i];
        const int64_t base = t.begin[i];
        int64_t e = lo - base, end = hi - base;
        // 8-element groups when both ends are 16-byte aligned for this tensor
        const bool vec = ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15) == 0 &&
                         (e & 7) == 0;
        if (vec) {
            // at most kSpan / (8 * kCastThreads) = 4 groups per lane: every load is issued
            // before the first store, so the lane waits on memory once
            constexpr int kGroups = kSpan / (8 * kCastThreads);
            const int64_t full = e + ((end - e) & ~int64_t{7});
            float4 a[kGroups], b[kGroups];
#pragma unroll
            for (int u = 0; u < kGroups; ++u) {
                const int64_t j = e + 8 * ((int64_t)threadIdx.x + (int64_t)u * kCastThreads);
                if (j < full) {
                    a[u] = *reinterpret_cast<const float4 *>(src + j);
                    b[u] = *reinterpret_cast<const float4 *>(src + j + 4);
                }
            }
#pragma unroll
            for (int u = 0; u < kGroups; ++u) {
                const int64_t j = e + 8 * ((int64_t)threadIdx.x + (int64_t)u * kCastThreads);
                if (j < full)
                    *reinterpret_cast<uint4 *>(dst + j) =
                        make_uint4(pack_bf16x2(a[u].x, a[u].y), pack_bf16x2(a[u].z, a[u].w),
                                   pack_bf16x2(b[u].x, b[u].y), pack_bf16x2(b[u].z, b[u].w));
            }
            e = full;
        }
        for (int64_t j = e + threadIdx.x; j < end; j += kCastThreads) dst[j] = bf16_bits(src[j]);
    }
}

}  // namespace
}  // namespace ct

using namespace ct;

extern "C" int ct_cast_f32_bf16(const float *const *src, uint16_t *const *dst, const int64_t *counts,
                                int32_t count, hipStream_t stream) {
    if (count < 0 || count > CT_CAST_MAX) return -CT_EINVAL_SHAPE;
    if (count == 0) return 0;
    if (!src || !dst || !counts) return -CT_EINVAL_POINTER;
    CastTable t{};
    t.count = count;
    t.begin[0] = 0;
    for (int i = 0; i < count; ++i) {
        if (counts[i] < 0) return -CT_EINVAL_SHAPE;
        if (counts[i] > 0 && (!src[i] || !dst[i])) return -CT_EINVAL_POINTER;
        t.src[i] = src[i];
        t.dst[i] = dst[i];
        t.begin[i + 1] = t.begin[i] + counts[i];
    }
    const int64_t total = t.begin[count];
    if (total == 0) return 0;
    const int64_t blocks = cdiv(total, kSpan);
    if (blocks > 0x7fffffff) return -CT_EINVAL_SHAPE;
    cast_f32_bf16<<<dim3((unsigned)blocks), dim3(kCastThreads), 0, stream>>>(t);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : (int)e;
}
