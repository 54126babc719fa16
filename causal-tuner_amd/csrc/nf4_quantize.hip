// NF4 quantizer on gfx950: the state bitsandbytes' quantize_4bit(quant_type="nf4",
// compress_statistics=True) gives the reference at modeling/lora.py:50-55 (Params4bit ->
// QuantState), restated from its published blockwise algorithm:
//
//   1. absmax[g] = max |w| over first-level block g (blocksize elements, zero-padded tail);
//   2. x = w * (1 / absmax[g]) in fp32; the NF4 code is the index of the first decision
//      midpoint >= x (15 midpoints between the 16 code values; a NaN, from an all-zero
//      block, takes code 15 and decodes to 0 * 1 = 0);
//   3. two codes per byte, element 2j in the high nibble (an odd count pads a zero nibble);
//   4. nested: offset = mean(absmax) (float64 sum, divided, rounded to fp32 once);
//      c = absmax - offset, blocks of 256: absmax2 = max |c|, and c * (1 / absmax2) is
//      coded against the 256-entry signed dynamic map by bitsandbytes' binary search
//      with the midpoint rule (dQuantize).
//
// Three launches: the first-level blocks (one lane per block), the offset (one
// workgroup, a fixed summation order), the second level (one workgroup per 256 blocks).
// Quantization runs once per weight load; the kernels favour simple, exact code.

#include "common.hpp"

namespace ct {
namespace {

constexpr int kQThreads = 256;

template <int IN>
__device__ __forceinline__ float load_value(const void *w, int64_t i) {
    if constexpr (IN == CT_BF16) return bf16_to_f32(static_cast<const uint16_t *>(w)[i]);
    else if constexpr (IN == CT_F16) return f16_to_f32(static_cast<const uint16_t *>(w)[i]);
    else return static_cast<const float *>(w)[i];
}

// searchsorted(midpoints, x, side="left") over the 15 sorted midpoints; NaN -> 15.
__device__ __forceinline__ uint32_t nf4_code_of(float x, const float *mid) {
    uint32_t c = 0;
#pragma unroll
    for (int i = 0; i < 15; ++i) c += !(mid[i] >= x);
    return c;
}

// First level: one lane per block. Eight-element groups (one 4-byte packed store) when the
// block and the element count allow it, single elements otherwise.
template <int IN>
__global__ __launch_bounds__(kQThreads) void nf4_quantize_blocks(const void *__restrict__ w, int64_t n, int blocksize,
                                                                const float *__restrict__ midpoints,
                                                                uint8_t *__restrict__ packed,
                                                                float *__restrict__ absmax) {
    __shared__ float mid[15];
    if (threadIdx.x < 15) mid[threadIdx.x] = midpoints[threadIdx.x];
    __syncthreads();
    const int64_t nb = cdiv(n, blocksize);
    const int64_t g = (int64_t)blockIdx.x * kQThreads + threadIdx.x;
    if (g >= nb) return;
    const int64_t e0 = g * blocksize;
    const int64_t e1 = e0 + blocksize < n ? e0 + blocksize : n;
    float m = 0.f;
    for (int64_t i = e0; i < e1; ++i) m = fmaxf(m, fabsf(load_value<IN>(w, i)));
    absmax[g] = m;
    const float r = 1.0f / m;  // IEEE division, as the reference's fp32 reciprocal
    if ((blocksize & 7) == 0 && (n & 7) == 0) {
        for (int64_t i = e0; i < e1; i += 8) {
            uint32_t word = 0;
#pragma unroll
            for (int j = 0; j < 8; j += 2) {
                const uint32_t hi = nf4_code_of(load_value<IN>(w, i + j) * r, mid);
                const uint32_t lo = nf4_code_of(load_value<IN>(w, i + j + 1) * r, mid);
                word |= ((hi << 4) | lo) << (4 * j);
            }
            *reinterpret_cast<uint32_t *>(packed + (i >> 1)) = word;
        }
    } else {
        for (int64_t i = e0; i < e1; i += 2) {  // blocks start at even elements
            const uint32_t hi = nf4_code_of(load_value<IN>(w, i) * r, mid);
            const uint32_t lo = i + 1 < e1 ? nf4_code_of(load_value<IN>(w, i + 1) * r, mid) : 0u;
            packed[i >> 1] = (uint8_t)((hi << 4) | lo);
        }
    }
}

// offset = fp32(sum(absmax) / nb) with the sum in float64: each thread adds a strided
// subset in index order, then a fixed pairwise tree over the 1024 partial sums.
__global__ __launch_bounds__(1024) void nf4_quantize_offset(const float *__restrict__ absmax, int64_t nb,
                                                           float *__restrict__ offset) {
    __shared__ double part[1024];
    double s = 0.0;
    for (int64_t i = threadIdx.x; i < nb; i += 1024) s += (double)absmax[i];
    part[threadIdx.x] = s;
    __syncthreads();
    for (int h = 512; h > 0; h >>= 1) {
        if ((int)threadIdx.x < h) part[threadIdx.x] += part[threadIdx.x + h];
        __syncthreads();
    }
    if (threadIdx.x == 0) *offset = (float)(part[0] / (double)nb);
}

// bitsandbytes dQuantize: binary search over the sorted 256-entry map, then the midpoint
// rule against the neighbour on the side x lies.
__device__ __forceinline__ uint32_t dynamic_code(float x, const float *code) {
    int pivot = 127, upper_pivot = 255, lower_pivot = 0;
    float lower = -1.0f, upper = 1.0f;
    float val = code[pivot];
    for (int step = 64; step > 0; step >>= 1) {
        if (x > val) {
            lower_pivot = pivot;
            lower = val;
            pivot += step;
        } else {
            upper_pivot = pivot;
            upper = val;
            pivot -= step;
        }
        val = code[pivot];
    }
    if (upper_pivot == 255) upper = code[255];
    if (lower_pivot == 0) lower = code[0];
    if (x > val) return (uint32_t)(x > (upper + val) * 0.5f ? upper_pivot : pivot);
    return (uint32_t)(x < (lower + val) * 0.5f ? lower_pivot : pivot);
}

// Second level: one workgroup per 256 first-level blocks (zero-padded past nb).
__global__ __launch_bounds__(256) void nf4_quantize_nested(const float *__restrict__ absmax, int64_t nb,
                                                          const float *__restrict__ offset,
                                                          const float *__restrict__ code2,
                                                          uint8_t *__restrict__ qabs,
                                                          float *__restrict__ absmax2) {
    __shared__ float lcode[256];
    __shared__ float red[256];
    const int tid = threadIdx.x;
    lcode[tid] = code2[tid];
    const int64_t g = (int64_t)blockIdx.x * 256 + tid;
    const float c = g < nb ? absmax[g] - *offset : 0.f;
    red[tid] = fabsf(c);
    __syncthreads();
    for (int h = 128; h > 0; h >>= 1) {
        if (tid < h) red[tid] = fmaxf(red[tid], red[tid + h]);
        __syncthreads();
    }
    const float m = red[0];
    if (tid == 0) absmax2[blockIdx.x] = m;
    if (g < nb) qabs[g] = (uint8_t)dynamic_code(c * (1.0f / m), lcode);
}

template <int IN>
hipError_t launch_quantize(const void *w, int64_t n, int blocksize, int nested, const float *midpoints,
                           const float *code2, uint8_t *packed, void *absmax, float *absmax2, float *offset,
                           float *scratch, hipStream_t stream) {
    const int64_t nb = cdiv(n, blocksize);
    float *first = nested ? scratch : static_cast<float *>(absmax);
    nf4_quantize_blocks<IN><<<dim3((unsigned)cdiv(nb, kQThreads)), dim3(kQThreads), 0, stream>>>(
        w, n, blocksize, midpoints, packed, first);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || !nested) return e;
    nf4_quantize_offset<<<dim3(1), dim3(1024), 0, stream>>>(first, nb, offset);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    nf4_quantize_nested<<<dim3((unsigned)cdiv(nb, 256)), dim3(256), 0, stream>>>(
        first, nb, offset, code2, static_cast<uint8_t *>(absmax), absmax2);
    return hipGetLastError();
}

}  // namespace
}  // namespace ct

using namespace ct;

extern "C" int64_t ct_nf4_quantize_workspace(int64_t n, int32_t blocksize, int32_t nested) {
    if (n <= 0 || blocksize < 2 || !nested) return 0;
    return cdiv(n, blocksize) * (int64_t)sizeof(float);
}

extern "C" int ct_nf4_quantize(const void *w, int32_t w_dtype, int64_t n, int32_t blocksize, int32_t nested,
                               const float *midpoints, const float *code2, uint8_t *packed, void *absmax,
                               float *absmax2, float *offset, void *workspace, int64_t workspace_bytes,
                               hipStream_t stream) {
    if (n < 0) return -CT_EINVAL_SHAPE;
    if (blocksize < 2 || (blocksize & (blocksize - 1))) return -CT_EINVAL_SHAPE;
    if (w_dtype != CT_BF16 && w_dtype != CT_F16 && w_dtype != CT_F32) return -CT_EINVAL_DTYPE;
    if (n == 0) return 0;
    if (!w || !midpoints || !packed || !absmax) return -CT_EINVAL_POINTER;
    if (nested && (!code2 || !absmax2 || !offset)) return -CT_EINVAL_POINTER;
    if ((reinterpret_cast<uintptr_t>(packed) & 3) != 0) return -CT_EINVAL_POINTER;
    if (nested && (!workspace || workspace_bytes < ct_nf4_quantize_workspace(n, blocksize, nested)))
        return -CT_EINVAL_WORKSPACE;
    float *scratch = static_cast<float *>(workspace);
    hipError_t e;
    switch (w_dtype) {
        case CT_BF16:
            e = launch_quantize<CT_BF16>(w, n, blocksize, nested, midpoints, code2, packed, absmax, absmax2, offset,
                                         scratch, stream);
            break;
        case CT_F16:
            e = launch_quantize<CT_F16>(w, n, blocksize, nested, midpoints, code2, packed, absmax, absmax2, offset,
                                        scratch, stream);
            break;
        default:
            e = launch_quantize<CT_F32>(w, n, blocksize, nested, midpoints, code2, packed, absmax, absmax2, offset,
                                        scratch, stream);
            break;
    }
    return e == hipSuccess ? 0 : (int)e;
}

extern "C" int ct_quantize_blockwise(const float *values, int64_t n, const float *offset, const float *code2,
                                     uint8_t *codes, float *absmax2, hipStream_t stream) {
    if (n < 0) return -CT_EINVAL_SHAPE;
    if (n == 0) return 0;
    if (!values || !offset || !code2 || !codes || !absmax2) return -CT_EINVAL_POINTER;
    nf4_quantize_nested<<<dim3((unsigned)cdiv(n, 256)), dim3(256), 0, stream>>>(values, n, offset, code2, codes,
                                                                                 absmax2);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : (int)e;
}
