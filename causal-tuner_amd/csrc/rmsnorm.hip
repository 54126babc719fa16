// Row-wise RMS normalization on gfx950 (the reference's kernels/core_cuda.py:29-130:
// _rms_forward, _rms_backward, _rms_weight_reduce behind RMS), with its rounding points:
//
//   forward   inverse = 1 / sqrt(sum(x^2) / width + eps)          (fp32, per row)
//             y = T(T(x * inverse) * T(w))                         T = round to x's dtype
//   backward  g = T(go * T(w))
//             from x:      gx = inverse * (g - x * (inverse^2 * sum(g * x) / width))
//             from output: n = y / T(w),  gx = inverse * (g - n * (sum(g * n) / width))
//             dw = sum over rows of go * T(x * inverse)            (fp32, rounded to w's dtype)
//
// One wave per row for the row passes (wave-level shuffle reduction, fixed order; 16-byte
// loads with the row kept in registers for 16-bit tensors up to 4096 wide); the
// weight gradient is summed over fixed row groups (one lane per column and group, rows in
// order) and then over the groups in order, so every result is reproducible bit for bit.
// The row sums' order differs from the reference's Triton reduction, and the reciprocal
// square root is an IEEE division of an IEEE square root: results agree with the
// reference to the rounding of the stored dtype, not bit for bit.

#include <initializer_list>

#include "common.hpp"

namespace ct {
namespace {

constexpr int kRowsPerBlock = 4;  // one wave per row, four waves per workgroup

template <int DT>
__device__ __forceinline__ float load_as_f32(const void *p, int64_t i) {
    if constexpr (DT == CT_BF16) return bf16_to_f32(static_cast<const uint16_t *>(p)[i]);
    else if constexpr (DT == CT_F16) return f16_to_f32(static_cast<const uint16_t *>(p)[i]);
    else return static_cast<const float *>(p)[i];
}

template <int DT>
__device__ __forceinline__ void store_from_f32(void *p, int64_t i, float v) {
    if constexpr (DT == CT_BF16) static_cast<uint16_t *>(p)[i] = bf16_bits(v);
    else if constexpr (DT == CT_F16) static_cast<uint16_t *>(p)[i] = f16_bits(v);
    else static_cast<float *>(p)[i] = v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

template <int XT, int WT>
__global__ __launch_bounds__(64 * kRowsPerBlock) void rms_forward(const void *__restrict__ x, const void *__restrict__ w,
                                                                 void *__restrict__ y, float *__restrict__ rstd,
                                                                 int64_t rows, int64_t width, float eps) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    if (row >= rows) return;  // wave-uniform
    const int64_t base = row * width;
    float s = 0.f;
    for (int64_t c = lane; c < width; c += 64) {
        const float v = load_as_f32<XT>(x, base + c);
        s += v * v;
    }
    s = wave_sum(s);
    const float inverse = 1.0f / sqrtf(s / (float)width + eps);
    for (int64_t c = lane; c < width; c += 64) {
        const float normalized = round_to_storage<XT>(load_as_f32<XT>(x, base + c) * inverse);
        const float weight = round_to_storage<XT>(load_as_f32<WT>(w, c));
        store_from_f32<XT>(y, base + c, normalized * weight);
    }
    if (lane == 0) rstd[row] = inverse;
}

// Input gradient, one wave per row. gx may alias go: each lane reads go[c] again before
// writing gx[c] at the same index.
template <int XT, int WT, bool FROM_OUTPUT>
__global__ __launch_bounds__(64 * kRowsPerBlock) void rms_input_grad(const void *__restrict__ x,
                                                                    const void *__restrict__ w,
                                                                    const float *__restrict__ rstd, const void *go,
                                                                    void *gx, int64_t rows, int64_t width) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int64_t base = row * width;
    const float inverse = rstd[row];
    const auto operand = [&](int64_t c, float weight) {
        const float v = load_as_f32<XT>(x, base + c);
        return FROM_OUTPUT ? v / weight : v;
    };
    float s = 0.f;
    for (int64_t c = lane; c < width; c += 64) {
        const float weight = round_to_storage<XT>(load_as_f32<WT>(w, c));
        const float g = round_to_storage<XT>(load_as_f32<XT>(go, base + c) * weight);
        s += g * operand(c, weight);
    }
    const float projection = wave_sum(s) / (float)width;
    const float factor = FROM_OUTPUT ? projection : inverse * inverse * projection;
    for (int64_t c = lane; c < width; c += 64) {
        const float weight = round_to_storage<XT>(load_as_f32<WT>(w, c));
        const float g = round_to_storage<XT>(load_as_f32<XT>(go, base + c) * weight);
        store_from_f32<XT>(gx, base + c, inverse * (g - operand(c, weight) * factor));
    }
}

// ---------------------------------------------------------------- 16-byte row passes
// 16-bit activations and weights, width a multiple of 8 up to 64 * 8 * kVecChunks: lane l
// of the row's wave holds elements 512 j + 8 l .. + 7 of chunk j, loaded once as 16 bytes
// and kept in registers for the second pass (the row is read from HBM once).
constexpr int kVecChunks = 8;

template <int DT>
__device__ __forceinline__ float half_to_f32(uint32_t word, int hi) {
    const uint16_t h = (uint16_t)(hi ? word >> 16 : word & 0xffffu);
    return DT == CT_BF16 ? bf16_to_f32(h) : f16_to_f32(h);
}
template <int DT>
__device__ __forceinline__ float vec_elem(const uint4 &q, int e) {
    const uint32_t w = e < 2 ? q.x : e < 4 ? q.y : e < 6 ? q.z : q.w;
    return half_to_f32<DT>(w, e & 1);
}
template <int DT>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    if constexpr (DT == CT_BF16) return pack_bf16x2(lo, hi);
    else return (uint32_t)f16_bits(lo) | ((uint32_t)f16_bits(hi) << 16);
}

template <int XT, int WT>
__global__ __launch_bounds__(64 * kRowsPerBlock) void rms_forward_vec(const void *__restrict__ x,
                                                                     const void *__restrict__ w,
                                                                     void *__restrict__ y, float *__restrict__ rstd,
                                                                     int64_t rows, int64_t width, float eps) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    if (row >= rows) return;  // wave-uniform
    const uint4 *xr = reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(x) + row * width);
    const int n = (int)(width / 8);  // 16-byte groups in the row
    uint4 v[kVecChunks];
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < kVecChunks; ++j) {
        const int g = j * 64 + lane;
        v[j] = g < n ? xr[g] : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < kVecChunks; ++j)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float t = vec_elem<XT>(v[j], e);
            s += t * t;
        }
    s = wave_sum(s);
    const float inverse = 1.0f / sqrtf(s / (float)width + eps);
    const uint4 *wr = reinterpret_cast<const uint4 *>(w);
    uint4 *yr = reinterpret_cast<uint4 *>(static_cast<uint16_t *>(y) + row * width);
#pragma unroll
    for (int j = 0; j < kVecChunks; ++j) {
        const int g = j * 64 + lane;
        if (g >= n) continue;
        const uint4 wq = wr[g];
        uint32_t out[4];
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            float o[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const float normalized = round_to_storage<XT>(vec_elem<XT>(v[j], e + h) * inverse);
                const float weight = round_to_storage<XT>(vec_elem<WT>(wq, e + h));
                o[h] = normalized * weight;
            }
            out[e / 2] = pack2<XT>(o[0], o[1]);
        }
        yr[g] = make_uint4(out[0], out[1], out[2], out[3]);
    }
    if (lane == 0) rstd[row] = inverse;
}

// Input gradient on 16-byte groups; gx may alias go (each lane rewrites only the groups it
// read).
template <int XT, int WT, bool FROM_OUTPUT>
__global__ __launch_bounds__(64 * kRowsPerBlock) void rms_input_grad_vec(const void *__restrict__ x,
                                                                        const void *__restrict__ w,
                                                                        const float *__restrict__ rstd,
                                                                        const void *go, void *gx, int64_t rows,
                                                                        int64_t width) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int n = (int)(width / 8);
    const uint4 *xr = reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(x) + row * width);
    const uint4 *gr = reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(go) + row * width);
    const uint4 *wr = reinterpret_cast<const uint4 *>(w);
    const float inverse = rstd[row];
    uint4 xv[kVecChunks], gv[kVecChunks], wv[kVecChunks];
#pragma unroll
    for (int j = 0; j < kVecChunks; ++j) {
        const int g = j * 64 + lane;
        const bool ok = g < n;
        xv[j] = ok ? xr[g] : make_uint4(0, 0, 0, 0);
        gv[j] = ok ? gr[g] : make_uint4(0, 0, 0, 0);
        wv[j] = ok ? wr[g] : make_uint4(0, 0, 0, 0);
    }
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < kVecChunks; ++j) {
        if (j * 64 + lane >= n) continue;  // past the row (zero weights would divide 0 by 0)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float weight = round_to_storage<XT>(vec_elem<WT>(wv[j], e));
            const float g = round_to_storage<XT>(vec_elem<XT>(gv[j], e) * weight);
            const float v = vec_elem<XT>(xv[j], e);
            s += g * (FROM_OUTPUT ? v / weight : v);
        }
    }
    const float projection = wave_sum(s) / (float)width;
    const float factor = FROM_OUTPUT ? projection : inverse * inverse * projection;
    uint4 *dr = reinterpret_cast<uint4 *>(static_cast<uint16_t *>(gx) + row * width);
#pragma unroll
    for (int j = 0; j < kVecChunks; ++j) {
        const int g = j * 64 + lane;
        if (g >= n) continue;
        uint32_t out[4];
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            float o[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const float weight = round_to_storage<XT>(vec_elem<WT>(wv[j], e + h));
                const float gg = round_to_storage<XT>(vec_elem<XT>(gv[j], e + h) * weight);
                const float v = vec_elem<XT>(xv[j], e + h);
                const float operand = FROM_OUTPUT ? v / weight : v;
                o[h] = inverse * (gg - operand * factor);
            }
            out[e / 2] = pack2<XT>(o[0], o[1]);
        }
        dr[g] = make_uint4(out[0], out[1], out[2], out[3]);
    }
}

// Weight-gradient partials: partial[group][c] = sum over the group's rows, in order, of
// go * T(x * inverse).
template <int XT>
__global__ __launch_bounds__(256) void rms_weight_partials(const void *__restrict__ x, const float *__restrict__ rstd,
                                                          const void *__restrict__ go, float *__restrict__ partial,
                                                          int64_t rows, int64_t width, int64_t rows_per_group) {
    const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t group = blockIdx.y;
    if (c >= width) return;
    const int64_t r0 = group * rows_per_group;
    const int64_t r1 = r0 + rows_per_group < rows ? r0 + rows_per_group : rows;
    float s = 0.f;
    for (int64_t r = r0; r < r1; ++r)
        s += load_as_f32<XT>(go, r * width + c) * round_to_storage<XT>(load_as_f32<XT>(x, r * width + c) * rstd[r]);
    partial[group * width + c] = s;
}

template <int WT>
__global__ __launch_bounds__(256) void rms_weight_reduce(const float *__restrict__ partial, int64_t groups,
                                                        int64_t width, void *__restrict__ dw) {
    const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (c >= width) return;
    float s = 0.f;
    for (int64_t g = 0; g < groups; ++g) s += partial[g * width + c];
    store_from_f32<WT>(dw, c, s);
}

int device_cus() {
    int device = 0, cus = 256;
    if (hipGetDevice(&device) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess)
        cus = 256;
    return cus;
}

// Row groups of the weight gradient (the reference's rule, core_cuda.py:113-115): at most
// four per CU, whole rows each.
void weight_groups(int64_t rows, int64_t *groups, int64_t *rows_per_group) {
    int64_t g = 4 * (int64_t)device_cus();
    if (g > rows) g = rows;
    const int64_t per = g > 0 ? cdiv(rows, g) : 1;
    *rows_per_group = per;
    *groups = per > 0 ? cdiv(rows, per) : 0;
}

bool valid(int d) { return d == CT_F32 || d == CT_F16 || d == CT_BF16; }

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// The 16-byte row kernels: 16-bit activations and weights, width a multiple of 8 and at
// most 64 * 8 * kVecChunks, every row pointer 16-byte aligned.
template <int XT, int WT>
constexpr bool kVecTypes = (XT == CT_BF16 || XT == CT_F16) && (WT == CT_BF16 || WT == CT_F16);

bool vec_rows(int64_t width, std::initializer_list<const void *> ptrs) {
    if (width % 8 || width > 64 * 8 * kVecChunks) return false;
    for (const void *p : ptrs)
        if (p && !aligned16(p)) return false;
    return true;
}

template <int XT, int WT>
hipError_t forward_typed(const void *x, const void *w, void *y, float *rstd, int64_t rows, int64_t width, float eps,
                         hipStream_t s) {
    const dim3 grid((unsigned)cdiv(rows, kRowsPerBlock)), block(64 * kRowsPerBlock);
    if constexpr (kVecTypes<XT, WT>) {
        if (vec_rows(width, {x, w, y})) {
            rms_forward_vec<XT, WT><<<grid, block, 0, s>>>(x, w, y, rstd, rows, width, eps);
            return hipGetLastError();
        }
    }
    rms_forward<XT, WT><<<grid, block, 0, s>>>(x, w, y, rstd, rows, width, eps);
    return hipGetLastError();
}

template <int XT, int WT>
hipError_t backward_typed(const void *x, const void *w, const float *rstd, const void *go, void *gx, void *dw,
                          int64_t rows, int64_t width, int from_output, float *partial, int64_t groups,
                          int64_t rows_per_group, hipStream_t s) {
    if (gx) {
        const dim3 grid((unsigned)cdiv(rows, kRowsPerBlock)), block(64 * kRowsPerBlock);
        bool done = false;
        if constexpr (kVecTypes<XT, WT>) {
            if (vec_rows(width, {x, w, go, gx})) {
                if (from_output) rms_input_grad_vec<XT, WT, true><<<grid, block, 0, s>>>(x, w, rstd, go, gx, rows, width);
                else rms_input_grad_vec<XT, WT, false><<<grid, block, 0, s>>>(x, w, rstd, go, gx, rows, width);
                done = true;
            }
        }
        if (!done && from_output) rms_input_grad<XT, WT, true><<<grid, block, 0, s>>>(x, w, rstd, go, gx, rows, width);
        else if (!done) rms_input_grad<XT, WT, false><<<grid, block, 0, s>>>(x, w, rstd, go, gx, rows, width);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    if (!dw) return hipSuccess;
    if (groups > 0) {
        rms_weight_partials<XT><<<dim3((unsigned)cdiv(width, 256), (unsigned)groups), dim3(256), 0, s>>>(
            x, rstd, go, partial, rows, width, rows_per_group);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    rms_weight_reduce<WT><<<dim3((unsigned)cdiv(width, 256)), dim3(256), 0, s>>>(partial, groups, width, dw);
    return hipGetLastError();
}

}  // namespace
}  // namespace ct

using namespace ct;

#define CT_RMS_DISPATCH(FN, XT, WT, ...)                                                        \
    [&]() -> hipError_t {                                                                      \
        switch ((XT) * 4 + (WT)) {                                                             \
            case CT_BF16 * 4 + CT_BF16: return FN<CT_BF16, CT_BF16>(__VA_ARGS__);              \
            case CT_BF16 * 4 + CT_F32: return FN<CT_BF16, CT_F32>(__VA_ARGS__);                \
            case CT_BF16 * 4 + CT_F16: return FN<CT_BF16, CT_F16>(__VA_ARGS__);                \
            case CT_F16 * 4 + CT_F16: return FN<CT_F16, CT_F16>(__VA_ARGS__);                  \
            case CT_F16 * 4 + CT_F32: return FN<CT_F16, CT_F32>(__VA_ARGS__);                  \
            case CT_F16 * 4 + CT_BF16: return FN<CT_F16, CT_BF16>(__VA_ARGS__);                \
            case CT_F32 * 4 + CT_F32: return FN<CT_F32, CT_F32>(__VA_ARGS__);                  \
            case CT_F32 * 4 + CT_BF16: return FN<CT_F32, CT_BF16>(__VA_ARGS__);                \
            default: return FN<CT_F32, CT_F16>(__VA_ARGS__);                                   \
        }                                                                                      \
    }()

extern "C" int ct_rms_forward(const void *x, int32_t x_dtype, const void *w, int32_t w_dtype, void *y, float *rstd,
                              int64_t rows, int64_t width, float eps, hipStream_t stream) {
    if (rows < 0 || width < 0) return -CT_EINVAL_SHAPE;
    if (!valid(x_dtype) || !valid(w_dtype)) return -CT_EINVAL_DTYPE;
    if (rows == 0) return 0;
    if (width == 0) return -CT_EINVAL_SHAPE;
    if (!x || !w || !y || !rstd) return -CT_EINVAL_POINTER;
    const hipError_t e = CT_RMS_DISPATCH(forward_typed, x_dtype, w_dtype, x, w, y, rstd, rows, width, eps, stream);
    return e == hipSuccess ? 0 : (int)e;
}

extern "C" int64_t ct_rms_backward_workspace(int64_t rows, int64_t width, int32_t weight_grad) {
    if (!weight_grad || rows <= 0 || width <= 0) return 0;
    int64_t groups, per;
    weight_groups(rows, &groups, &per);
    return groups * width * (int64_t)sizeof(float);
}

extern "C" int ct_rms_backward(const void *x, int32_t x_dtype, const void *w, int32_t w_dtype, const float *rstd,
                               const void *go, void *gx, void *dw, int64_t rows, int64_t width, int32_t from_output,
                               void *workspace, int64_t workspace_bytes, hipStream_t stream) {
    if (rows < 0 || width < 0) return -CT_EINVAL_SHAPE;
    if (!valid(x_dtype) || !valid(w_dtype)) return -CT_EINVAL_DTYPE;
    if (width == 0) return rows == 0 ? 0 : -CT_EINVAL_SHAPE;
    if (!gx && !dw) return 0;
    if (!w || (rows > 0 && (!x || !rstd || !go))) return -CT_EINVAL_POINTER;
    if (dw && from_output) return -CT_EINVAL_SHAPE;  // the weight gradient needs x itself
    int64_t groups = 0, per = 1;
    if (dw && rows > 0) weight_groups(rows, &groups, &per);
    if (dw && rows > 0 && (!workspace || workspace_bytes < groups * width * (int64_t)sizeof(float)))
        return -CT_EINVAL_WORKSPACE;
    if (rows == 0) gx = nullptr;  // nothing to write; dw below is then all zeros
    const hipError_t e = CT_RMS_DISPATCH(backward_typed, x_dtype, w_dtype, x, w, rstd, go, gx, dw, rows, width,
                                         from_output, static_cast<float *>(workspace), groups, per, stream);
    return e == hipSuccess ? 0 : (int)e;
}
