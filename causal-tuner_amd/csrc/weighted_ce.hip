// Weighted cross-entropy over a block of logits, gfx950 (the reference's
// kernels/loss_cuda.py:11-70: _statistics, _finish behind weighted_ce):
//
//   lse[r]  = log sum_c exp(logits[r, c])                       (fp32)
//   loss[r] = weight[r] * (lse[r] - logits[r, target[r]])       (0 for a target outside [0, vocab))
//   with gradient: logits[r, c] <- (exp(logits[r, c] - lse[r]) - [c == target[r]]) * weight[r]
//                  (overwritten in place, rounded to the logits' dtype)
//
// One workgroup per row. Pass one keeps a running (maximum, sum of exp(v - maximum)) per
// thread and combines the 256 pairs in a fixed tree, so the result does not depend on
// timing; pass two (with gradient) reads the row again, mostly from L2, and writes the
// derivative. HBM-bound: one read of the logits, plus one write with gradient.

#include <math.h>

#include "common.hpp"

namespace ct {
namespace {

constexpr int kCeThreads = 256;

template <int DT>
__device__ __forceinline__ float ce_load(const void *p, int64_t i) {
    if constexpr (DT == CT_BF16) return bf16_to_f32(static_cast<const uint16_t *>(p)[i]);
    else if constexpr (DT == CT_F16) return f16_to_f32(static_cast<const uint16_t *>(p)[i]);
    else return static_cast<const float *>(p)[i];
}

template <int DT>
__device__ __forceinline__ void ce_store(void *p, int64_t i, float v) {
    if constexpr (DT == CT_BF16) static_cast<uint16_t *>(p)[i] = bf16_bits(v);
    else if constexpr (DT == CT_F16) static_cast<uint16_t *>(p)[i] = f16_bits(v);
    else static_cast<float *>(p)[i] = v;
}

// (m, s) represents s * exp(m); combining keeps the larger maximum.
__device__ __forceinline__ void combine(float &m, float &s, float m2, float s2) {
    if (m2 > m) {
        s = s * __expf(m - m2) + s2;
        m = m2;
    } else if (m2 > -INFINITY) {
        s += s2 * __expf(m2 - m);
    }
}

template <int DT>
__global__ __launch_bounds__(kCeThreads) void weighted_ce_rows(void *logits, int64_t vocab, int64_t ld,
                                                              const int64_t *__restrict__ targets,
                                                              const float *__restrict__ weights,
                                                              float *__restrict__ loss, int gradient) {
    __shared__ float lm[kCeThreads], ls[kCeThreads];
    __shared__ float selected;
    const int tid = threadIdx.x;
    const int64_t row = blockIdx.x;
    const int64_t base = row * ld;
    const int64_t target = targets[row];
    if (tid == 0) selected = (target >= 0 && target < vocab) ? ce_load<DT>(logits, base + target) : 0.f;
    float m = -INFINITY, s = 0.f;
    for (int64_t c = tid; c < vocab; c += kCeThreads) combine(m, s, ce_load<DT>(logits, base + c), 1.f);
    lm[tid] = m;
    ls[tid] = s;
    __syncthreads();
    for (int h = kCeThreads / 2; h > 0; h >>= 1) {
        if (tid < h) {
            float a = lm[tid], b = ls[tid];
            combine(a, b, lm[tid + h], ls[tid + h]);
            lm[tid] = a;
            ls[tid] = b;
        }
        __syncthreads();
    }
    const float lse = lm[0] + logf(ls[0]);
    const float weight = weights[row];
    if (tid == 0) loss[row] = weight * (lse - selected);
    if (!gradient) return;
    // (the target logit was read before the barriers above; nothing is overwritten earlier)
    for (int64_t c = tid; c < vocab; c += kCeThreads) {
        const float v = ce_load<DT>(logits, base + c);
        const float onehot = c == target ? 1.f : 0.f;
        ce_store<DT>(logits, base + c, (__expf(v - lse) - onehot) * weight);
    }
}

}  // namespace
}  // namespace ct

using namespace ct;

extern "C" int ct_weighted_ce(void *logits, int32_t dtype, int64_t rows, int64_t vocab, int64_t ld,
                              const int64_t *targets, const float *weights, float *loss, int32_t gradient,
                              hipStream_t stream) {
    if (rows < 0 || vocab < 0 || ld < vocab) return -CT_EINVAL_SHAPE;
    if (dtype != CT_BF16 && dtype != CT_F16 && dtype != CT_F32) return -CT_EINVAL_DTYPE;
    if (rows == 0) return 0;
    if (vocab == 0) return -CT_EINVAL_SHAPE;
    if (!logits || !targets || !weights || !loss) return -CT_EINVAL_POINTER;
    if (rows > 0x7fffffff) return -CT_EINVAL_SHAPE;
    const dim3 grid((unsigned)rows), block(kCeThreads);
    switch (dtype) {
        case CT_BF16: weighted_ce_rows<CT_BF16><<<grid, block, 0, stream>>>(logits, vocab, ld, targets, weights, loss, gradient); break;
        case CT_F16: weighted_ce_rows<CT_F16><<<grid, block, 0, stream>>>(logits, vocab, ld, targets, weights, loss, gradient); break;
        default: weighted_ce_rows<CT_F32><<<grid, block, 0, stream>>>(logits, vocab, ld, targets, weights, loss, gradient); break;
    }
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : (int)e;
}
