// AdamW step over many parameter tensors in one launch, gfx950: the update torch's fused
// AdamW applies for the reference's optimizer (training/engine.py:10-16, torch.optim.AdamW
// with fused=True, amsgrad off), restated from the published algorithm (decoupled weight
// decay, Loshchilov & Hutter) with torch's rounding points:
//
//   step s = *step (already incremented for this update), bc1 = 1 - beta1^s,
//   bc2s = sqrt(1 - beta2^s)                                   (fp32)
//   g = maximize ? -grad : grad
//   p = p - lr * weight_decay * p                               (double, rounded to fp32)
//   m = beta1 * m + (1 - beta1) * g                             (double, rounded to fp32)
//   v = beta2 * v + (1 - beta2) * g * g                         (double, rounded to fp32)
//   p = p - (lr / bc1) * m / (sqrt(v) / bc2s + eps)             (fp32)
//
// then p, m, v are stored in the parameter's dtype (fp32 or bf16; the states share it).
// HBM-bound: per element it reads p, g, m, v and writes p, m, v.
//
// The tensor table and the chunk list live in device memory (the caller builds them once
// per parameter set); each workgroup takes one chunk of one tensor, so a whole model's
// adapters update in a single launch.

#include <math.h>

#include "common.hpp"

namespace ct {
namespace {

constexpr int kAdamThreads = 256;

template <int DT>
__device__ __forceinline__ float ld_elem(const void *p, int64_t i) {
    if constexpr (DT == CT_BF16) return bf16_to_f32(static_cast<const uint16_t *>(p)[i]);
    else return static_cast<const float *>(p)[i];
}
template <int DT>
__device__ __forceinline__ void st_elem(void *p, int64_t i, float v) {
    if constexpr (DT == CT_BF16) static_cast<uint16_t *>(p)[i] = bf16_bits(v);
    else static_cast<float *>(p)[i] = v;
}

struct AdamScalars {
    double lr, beta1, beta2, eps, weight_decay;
    int maximize;
};

template <int DT>
__device__ __forceinline__ void adam_elem(void *param, const void *grad, void *exp_avg, void *exp_avg_sq,
                                          int64_t i, const AdamScalars &h, float step_size_bc1,
                                          float bc2s) {
    float p = ld_elem<DT>(param, i);
    float g = ld_elem<DT>(grad, i);
    if (h.maximize) g = -g;
    float m = ld_elem<DT>(exp_avg, i);
    float v = ld_elem<DT>(exp_avg_sq, i);
    if (h.weight_decay != 0.0) p = (float)((double)p - h.lr * h.weight_decay * (double)p);
    m = (float)(h.beta1 * (double)m + (1.0 - h.beta1) * (double)g);
    v = (float)(h.beta2 * (double)v + (1.0 - h.beta2) * (double)g * (double)g);
    const float denom = (float)((double)(sqrtf(v) / bc2s) + h.eps);
    p = p - step_size_bc1 * m / denom;
    st_elem<DT>(param, i, p);
    st_elem<DT>(exp_avg, i, m);
    st_elem<DT>(exp_avg_sq, i, v);
}

template <int DT>
__global__ __launch_bounds__(kAdamThreads) void adamw_chunks(const ct_adamw_tensor *__restrict__ tensors,
                                                            const int64_t *__restrict__ chunks,
                                                            int64_t chunk_elems, AdamScalars h) {
    const int64_t t = chunks[2 * blockIdx.x], start = chunks[2 * blockIdx.x + 1];
    const ct_adamw_tensor d = tensors[t];
    const double s = (double)*d.step;
    const float bc1 = (float)(1.0 - pow(h.beta1, s));
    const float bc2s = sqrtf((float)(1.0 - pow(h.beta2, s)));
    const float step_size = (float)(h.lr / (double)bc1);
    const int64_t end = start + chunk_elems < d.numel ? start + chunk_elems : d.numel;
    for (int64_t i = start + threadIdx.x; i < end; i += kAdamThreads)
        adam_elem<DT>(d.param, d.grad, d.exp_avg, d.exp_avg_sq, i, h, step_size, bc2s);
}

// state steps += 1, one lane per tensor (the step counters of the update about to run).
__global__ __launch_bounds__(256) void adamw_count(const ct_adamw_tensor *__restrict__ tensors, int64_t count) {
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t < count) *const_cast<float *>(tensors[t].step) += 1.0f;
}

}  // namespace
}  // namespace ct

using namespace ct;

extern "C" int ct_adamw_step(const ct_adamw_tensor *tensors, int64_t count, const int64_t *chunks,
                             int64_t n_chunks, int64_t chunk_elems, int32_t dtype, double lr, double beta1,
                             double beta2, double eps, double weight_decay, int32_t maximize,
                             int32_t count_step, hipStream_t stream) {
    if (count < 0 || n_chunks < 0 || chunk_elems <= 0) return -CT_EINVAL_SHAPE;
    if (dtype != CT_F32 && dtype != CT_BF16) return -CT_EINVAL_DTYPE;
    if (count == 0 || n_chunks == 0) return 0;
    if (!tensors || !chunks) return -CT_EINVAL_POINTER;
    if (n_chunks > 0x7fffffff) return -CT_EINVAL_SHAPE;
    if (count_step) {
        adamw_count<<<dim3((unsigned)cdiv(count, 256)), dim3(256), 0, stream>>>(tensors, count);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return (int)e;
    }
    const AdamScalars h{lr, beta1, beta2, eps, weight_decay, maximize ? 1 : 0};
    if (dtype == CT_BF16)
        adamw_chunks<CT_BF16><<<dim3((unsigned)n_chunks), dim3(kAdamThreads), 0, stream>>>(tensors, chunks,
                                                                                          chunk_elems, h);
    else
        adamw_chunks<CT_F32><<<dim3((unsigned)n_chunks), dim3(kAdamThreads), 0, stream>>>(tensors, chunks,
                                                                                         chunk_elems, h);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : (int)e;
}
