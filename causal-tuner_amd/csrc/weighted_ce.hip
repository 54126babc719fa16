// Weighted cross-entropy over a block of logits, gfx950 (the reference's
// kernels/loss_cuda.py:11-70: _statistics, _finish behind weighted_ce):
//
//   lse[r]  = log sum_c exp(logits[r, c])                       (fp32)
//   loss[r] = weight[r] * (lse[r] - logits[r, target[r]])       (the target term is 0 for a
//                                                                target outside [0, vocab))
//   with gradient: logits[r, c] <- (exp(logits[r, c] - lse[r]) - [c == target[r]]) * weight[r]
//                  (overwritten in place, rounded to the logits' dtype)
//
// Two launches over (column splits of kSplit, rows), as the reference splits the vocabulary:
// the first keeps a running (maximum, sum of exp(v - maximum)) per thread, combines the 256
// pairs of the workgroup in a fixed tree and stores one pair per split (plus the target's
// logit, read before anything is overwritten); the second combines a row's pairs in split
// order (every workgroup of the row gets the same lse), writes the loss, and with gradient
// rewrites its split. Both read 16 bytes per lane per load. HBM-bound: the logits are read
// twice (the second time mostly from L2/MALL at these sizes) and written once.

#include <math.h>

#include "common.hpp"

namespace ct {
namespace {

constexpr int kCeThreads = 256;
constexpr int64_t kSplit = 4096;  // columns per workgroup

template <int DT>
struct CeVec {  // elements per 16-byte load
    static constexpr int N = DT == CT_F32 ? 4 : 8;
};

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

// The 16 bytes at element i (i a multiple of CeVec<DT>::N, 16-byte aligned) as floats.
template <int DT>
__device__ __forceinline__ void ce_load_vec(const void *p, int64_t i, float (&v)[CeVec<DT>::N]) {
    const uint4 q = *reinterpret_cast<const uint4 *>(static_cast<const char *>(p) + i * (DT == CT_F32 ? 4 : 2));
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
    if constexpr (DT == CT_F32) {
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = __builtin_bit_cast(float, w[j]);
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint16_t h = (uint16_t)(j & 1 ? w[j / 2] >> 16 : w[j / 2] & 0xffffu);
            v[j] = DT == CT_BF16 ? bf16_to_f32(h) : f16_to_f32(h);
        }
    }
}

template <int DT>
__device__ __forceinline__ void ce_store_vec(void *p, int64_t i, const float (&v)[CeVec<DT>::N]) {
    uint32_t w[4];
    if constexpr (DT == CT_F32) {
#pragma unroll
        for (int j = 0; j < 4; ++j) w[j] = __builtin_bit_cast(uint32_t, v[j]);
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if constexpr (DT == CT_BF16) w[j] = pack_bf16x2(v[2 * j], v[2 * j + 1]);
            else w[j] = (uint32_t)f16_bits(v[2 * j]) | ((uint32_t)f16_bits(v[2 * j + 1]) << 16);
        }
    }
    *reinterpret_cast<uint4 *>(static_cast<char *>(p) + i * (DT == CT_F32 ? 4 : 2)) = make_uint4(w[0], w[1], w[2], w[3]);
}

// (m, s) represents s * exp(m); combining keeps the larger maximum. A NaN on either side
// makes the pair NaN, so a NaN logit gives a NaN loss as sum(exp(values - max)) does.
__device__ __forceinline__ void combine(float &m, float &s, float m2, float s2) {
    if (__builtin_isnan(m2) || __builtin_isnan(s2)) {
        m = s = __builtin_nanf("");
    } else if (m2 > m) {
        s = s * __expf(m - m2) + s2;
        m = m2;
    } else if (m2 > -INFINITY) {
        s += s2 * __expf(m2 - m);
    }
}

// Columns [c0, c1) of one row, in 16-byte groups per lane when `vec` (row start aligned
// and c0 a multiple of the group), else one element per lane.
template <int DT, class F>
__device__ __forceinline__ void for_split(const void *row, int64_t c0, int64_t c1, bool vec, F &&f) {
    constexpr int N = CeVec<DT>::N;
    int64_t c = c0;
    if (vec) {
        const int64_t full = c0 + ((c1 - c0) / N) * N;
        for (int64_t j = c0 + (int64_t)threadIdx.x * N; j < full; j += (int64_t)kCeThreads * N) {
            float v[N];
            ce_load_vec<DT>(row, j, v);
#pragma unroll
            for (int e = 0; e < N; ++e) f(j + e, v[e]);
        }
        c = full;
    }
    for (int64_t j = c + threadIdx.x; j < c1; j += kCeThreads) f(j, ce_load<DT>(row, j));
}

template <int DT>
__global__ __launch_bounds__(kCeThreads) void weighted_ce_stats(const void *logits, int64_t vocab, int64_t ld,
                                                                const int64_t *__restrict__ targets,
                                                                float2 *__restrict__ partial,
                                                                float *__restrict__ selected, int vec) {
    __shared__ float lm[kCeThreads], ls[kCeThreads];
    const int tid = threadIdx.x;
    const int64_t split = blockIdx.x, row = blockIdx.y, splits = gridDim.x;
    const int64_t c0 = split * kSplit, c1 = c0 + kSplit < vocab ? c0 + kSplit : vocab;
    const char *rowp = static_cast<const char *>(logits) + row * ld * (DT == CT_F32 ? 4 : 2);
    const int64_t target = targets[row];
    if (tid == 0 && target >= c0 && target < c1) selected[row] = ce_load<DT>(rowp, target);
    float m = -INFINITY, s = 0.f;
    for_split<DT>(rowp, c0, c1, vec != 0, [&](int64_t, float v) { combine(m, s, v, 1.f); });
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
    if (tid == 0) partial[row * splits + split] = make_float2(lm[0], ls[0]);
}

template <int DT>
__global__ __launch_bounds__(kCeThreads) void weighted_ce_finish(void *logits, int64_t vocab, int64_t ld,
                                                                 const int64_t *__restrict__ targets,
                                                                 const float *__restrict__ weights,
                                                                 const float2 *__restrict__ partial,
                                                                 const float *__restrict__ selected,
                                                                 int64_t splits, float *__restrict__ loss,
                                                                 int gradient, int vec) {
    const int64_t split = blockIdx.x, row = blockIdx.y;
    float m = -INFINITY, s = 0.f;
    for (int64_t z = 0; z < splits; ++z) {  // split order: the same lse in every workgroup
        const float2 p = partial[row * splits + z];
        combine(m, s, p.x, p.y);
    }
    const float lse = m + logf(s);
    const float weight = weights[row];
    const int64_t target = targets[row];
    if (split == 0 && threadIdx.x == 0) {
        const float chosen = (target >= 0 && target < vocab) ? selected[row] : 0.f;
        loss[row] = weight * (lse - chosen);
    }
    if (!gradient) return;
    const int64_t c0 = split * kSplit, c1 = c0 + kSplit < vocab ? c0 + kSplit : vocab;
    char *rowp = static_cast<char *>(logits) + row * ld * (DT == CT_F32 ? 4 : 2);
    constexpr int N = CeVec<DT>::N;
    int64_t c = c0;
    if (vec) {
        const int64_t full = c0 + ((c1 - c0) / N) * N;
        for (int64_t j = c0 + (int64_t)threadIdx.x * N; j < full; j += (int64_t)kCeThreads * N) {
            float v[N];
            ce_load_vec<DT>(rowp, j, v);
#pragma unroll
            for (int e = 0; e < N; ++e) v[e] = (__expf(v[e] - lse) - (j + e == target ? 1.f : 0.f)) * weight;
            ce_store_vec<DT>(rowp, j, v);
        }
        c = full;
    }
    for (int64_t j = c + threadIdx.x; j < c1; j += kCeThreads) {
        const float v = ce_load<DT>(rowp, j);
        ce_store<DT>(rowp, j, (__expf(v - lse) - (j == target ? 1.f : 0.f)) * weight);
    }
}

template <int DT>
hipError_t launch_ce(void *logits, int64_t rows, int64_t vocab, int64_t ld, const int64_t *targets,
                     const float *weights, float *loss, int gradient, void *workspace, hipStream_t stream) {
    const int64_t splits = cdiv(vocab, kSplit);
    float2 *partial = static_cast<float2 *>(workspace);
    float *selected = reinterpret_cast<float *>(partial + rows * splits);
    const int elem = DT == CT_F32 ? 4 : 2;
    const int vec = (reinterpret_cast<uintptr_t>(logits) % 16 == 0 && (ld * elem) % 16 == 0) ? 1 : 0;
    weighted_ce_stats<DT><<<dim3((unsigned)splits, (unsigned)rows), dim3(kCeThreads), 0, stream>>>(
        logits, vocab, ld, targets, partial, selected, vec);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    weighted_ce_finish<DT><<<dim3(gradient ? (unsigned)splits : 1u, (unsigned)rows), dim3(kCeThreads), 0, stream>>>(
        logits, vocab, ld, targets, weights, partial, selected, splits, loss, gradient, vec);
    return hipGetLastError();
}

}  // namespace
}  // namespace ct

using namespace ct;

extern "C" int64_t ct_weighted_ce_workspace(int64_t rows, int64_t vocab) {
    if (rows <= 0 || vocab <= 0) return 0;
    return rows * cdiv(vocab, kSplit) * (int64_t)sizeof(float2) + rows * (int64_t)sizeof(float);
}

extern "C" int ct_weighted_ce(void *logits, int32_t dtype, int64_t rows, int64_t vocab, int64_t ld,
                              const int64_t *targets, const float *weights, float *loss, int32_t gradient,
                              void *workspace, int64_t workspace_bytes, hipStream_t stream) {
    if (rows < 0 || vocab < 0 || ld < vocab) return -CT_EINVAL_SHAPE;
    if (dtype != CT_BF16 && dtype != CT_F16 && dtype != CT_F32) return -CT_EINVAL_DTYPE;
    if (rows == 0) return 0;
    if (vocab == 0) return -CT_EINVAL_SHAPE;
    if (!logits || !targets || !weights || !loss) return -CT_EINVAL_POINTER;
    if (rows > 65535 || cdiv(vocab, kSplit) > 0x7fffffff) return -CT_EINVAL_SHAPE;
    if (!workspace || workspace_bytes < ct_weighted_ce_workspace(rows, vocab) ||
        reinterpret_cast<uintptr_t>(workspace) % 8)
        return -CT_EINVAL_WORKSPACE;
    hipError_t e;
    switch (dtype) {
        case CT_BF16: e = launch_ce<CT_BF16>(logits, rows, vocab, ld, targets, weights, loss, gradient, workspace, stream); break;
        case CT_F16: e = launch_ce<CT_F16>(logits, rows, vocab, ld, targets, weights, loss, gradient, workspace, stream); break;
        default: e = launch_ce<CT_F32>(logits, rows, vocab, ld, targets, weights, loss, gradient, workspace, stream); break;
    }
    return e == hipSuccess ? 0 : (int)e;
}
