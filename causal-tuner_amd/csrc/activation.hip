// SiLU-multiply of the LoRA MLP for gfx950: the MI355X replacement of the reference's
// Triton kernel `_activation` (kernels/mlp_cuda.py:10-35).
//
// Per element, in fp32 (kernels/mlp_cuda.py:13-25):
//   sig  = 1 / (1 + exp(-g))
//   act  = dtype(g * sig)                          rounded to the tensor type first
//   forward      h  = act * u
//   backward     pg = dtype(grad * u)              rounded
//                dg = pg * (sig * (1 + g * (1 - sig)))
//                du = grad * act
// with every output rounded once to the tensor type. In the reference's backward call
// (mlp_cuda.py:133) the outputs alias the inputs (dg -> gate, du -> up, hidden -> grad);
// each element is read completely before any of its outputs is written, so that is safe.
// Elementwise and HBM-bound: 8 elements per lane per step with 16-byte accesses.

#include "epilogue.hpp"

namespace ct {
namespace {

template <int T>
__device__ __forceinline__ float load_t(const void *p, int64_t i) {
    if constexpr (T == CT_BF16) return bf16_to_f32(static_cast<const uint16_t *>(p)[i]);
    else return static_cast<const float *>(p)[i];
}

template <int T>
__device__ __forceinline__ void store_t(void *p, int64_t i, float v) {
    if constexpr (T == CT_BF16) static_cast<uint16_t *>(p)[i] = bf16_bits(v);
    else static_cast<float *>(p)[i] = v;
}

template <int T, bool BACKWARD, bool RECONSTRUCT>
__device__ __forceinline__ void element(const void *gate, const void *up, void *h, void *dg, void *du, int64_t i) {
    const float g = load_t<T>(gate, i), u = load_t<T>(up, i);
    if constexpr (BACKWARD) {
        float dgate, dup, hidden;
        silu_backward<T>(g, u, load_t<T>(h, i), dgate, dup, hidden);
        store_t<T>(dg, i, dgate);
        store_t<T>(du, i, dup);
        if constexpr (RECONSTRUCT) store_t<T>(h, i, hidden);
    } else {
        store_t<T>(h, i, silu_forward<T>(g, u));
    }
}

// bf16, 16-byte aligned, n % 8 == 0: one 16-byte load or store per operand per lane.
template <bool BACKWARD, bool RECONSTRUCT>
__global__ __launch_bounds__(256) void silu_multiply_vec(const uint4 *gate, const uint4 *up, uint4 *h, uint4 *dg,
                                                         uint4 *du, int64_t chunks) {
    const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (c >= chunks) return;
    const uint4 gv = gate[c], uv = up[c];
    uint4 hv = make_uint4(0, 0, 0, 0);
    if constexpr (BACKWARD) hv = h[c];
    const uint16_t *g16 = reinterpret_cast<const uint16_t *>(&gv);
    const uint16_t *u16 = reinterpret_cast<const uint16_t *>(&uv);
    const uint16_t *h16 = reinterpret_cast<const uint16_t *>(&hv);
    float o_dg[8], o_du[8], o_h[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const float g = bf16_to_f32(g16[j]), u = bf16_to_f32(u16[j]);
        if constexpr (BACKWARD) silu_backward<CT_BF16>(g, u, bf16_to_f32(h16[j]), o_dg[j], o_du[j], o_h[j]);
        else o_h[j] = silu_forward<CT_BF16>(g, u);
    }
    auto pack = [](const float (&v)[8]) {
        return make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                          pack_bf16x2(v[6], v[7]));
    };
    if constexpr (BACKWARD) {
        dg[c] = pack(o_dg);
        du[c] = pack(o_du);
    }
    if constexpr (RECONSTRUCT) h[c] = pack(o_h);
}

template <int T, bool BACKWARD, bool RECONSTRUCT>
__global__ __launch_bounds__(256) void silu_multiply_kernel(const void *gate, const void *up, void *h, void *dg,
                                                            void *du, int64_t n) {
    const int64_t base = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
    if (base + 8 <= n) {
#pragma unroll
        for (int j = 0; j < 8; ++j) element<T, BACKWARD, RECONSTRUCT>(gate, up, h, dg, du, base + j);
    } else {
        for (int64_t i = base; i < n; ++i) element<T, BACKWARD, RECONSTRUCT>(gate, up, h, dg, du, i);
    }
}

bool aligned16(const void *q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; }

template <int T>
hipError_t launch(const void *gate, const void *up, void *h, void *dg, void *du, int64_t n, int backward,
                  int reconstruct, hipStream_t s) {
    const dim3 grid((unsigned)cdiv(n, 256 * 8)), block(256);
    if (T == CT_BF16 && n % 8 == 0 && aligned16(gate) && aligned16(up) && aligned16(h) &&
        (!backward || (aligned16(dg) && aligned16(du)))) {
        const int64_t chunks = n / 8;
        auto g = static_cast<const uint4 *>(gate);
        auto u = static_cast<const uint4 *>(up);
        auto hh = static_cast<uint4 *>(h);
        auto a = static_cast<uint4 *>(dg);
        auto b = static_cast<uint4 *>(du);
        if (backward && reconstruct) silu_multiply_vec<true, true><<<grid, block, 0, s>>>(g, u, hh, a, b, chunks);
        else if (backward) silu_multiply_vec<true, false><<<grid, block, 0, s>>>(g, u, hh, a, b, chunks);
        else silu_multiply_vec<false, true><<<grid, block, 0, s>>>(g, u, hh, a, b, chunks);
        return hipGetLastError();
    }
    if (backward && reconstruct) silu_multiply_kernel<T, true, true><<<grid, block, 0, s>>>(gate, up, h, dg, du, n);
    else if (backward) silu_multiply_kernel<T, true, false><<<grid, block, 0, s>>>(gate, up, h, dg, du, n);
    else silu_multiply_kernel<T, false, true><<<grid, block, 0, s>>>(gate, up, h, dg, du, n);
    return hipGetLastError();
}

}  // namespace

// h = bf16(silu(gate)) * up over n contiguous bf16 elements with silu_multiply_vec: the
// pass after a GEMM whose SiLU step runs outside it (the product in `up`), with the kernel
// and the bits of ct_silu_multiply. Needs n % 8 == 0 and 16-byte aligned operands.
hipError_t silu_forward_flat(const uint16_t *gate, const uint16_t *up, uint16_t *h, int64_t n, hipStream_t s) {
    if (n % 8 || !aligned16(gate) || !aligned16(up) || !aligned16(h)) return hipErrorInvalidValue;
    const int64_t chunks = n / 8;
    silu_multiply_vec<false, true><<<dim3((unsigned)cdiv(chunks, 256)), dim3(256), 0, s>>>(
        reinterpret_cast<const uint4 *>(gate), reinterpret_cast<const uint4 *>(up), reinterpret_cast<uint4 *>(h),
        nullptr, nullptr, chunks);
    return hipGetLastError();
}

// The backward twin: reads gate, up and the upstream gradient in h, writes dgate, dup and
// the reconstructed h over it (ct_silu_multiply's backward kernel and bits). The outputs
// may alias gate and up (each lane reads its chunk before writing it).
hipError_t silu_backward_flat(const uint16_t *gate, const uint16_t *up, uint16_t *h, uint16_t *dg, uint16_t *du,
                              int64_t n, hipStream_t s) {
    if (n % 8 || !aligned16(gate) || !aligned16(up) || !aligned16(h) || !aligned16(dg) || !aligned16(du))
        return hipErrorInvalidValue;
    const int64_t chunks = n / 8;
    silu_multiply_vec<true, true><<<dim3((unsigned)cdiv(chunks, 256)), dim3(256), 0, s>>>(
        reinterpret_cast<const uint4 *>(gate), reinterpret_cast<const uint4 *>(up), reinterpret_cast<uint4 *>(h),
        reinterpret_cast<uint4 *>(dg), reinterpret_cast<uint4 *>(du), chunks);
    return hipGetLastError();
}

}  // namespace ct

extern "C" int ct_silu_multiply(const void *gate, const void *up, void *h, void *dgate, void *dup, int64_t n,
                                int32_t backward, int32_t reconstruct, int32_t dtype, hipStream_t stream) {
    using namespace ct;
    if (n < 0) return -CT_EINVAL_SHAPE;
    if (dtype != CT_BF16 && dtype != CT_F32) return -CT_EINVAL_DTYPE;
    if (!backward && !reconstruct) return 0;
    if (n == 0) return 0;
    if (!gate || !up || !h || (backward && (!dgate || !dup))) return -CT_EINVAL_POINTER;
    const hipError_t e = dtype == CT_BF16 ? launch<CT_BF16>(gate, up, h, dgate, dup, n, backward, reconstruct, stream)
                                          : launch<CT_F32>(gate, up, h, dgate, dup, n, backward, reconstruct, stream);
    return e == hipSuccess ? 0 : (int)e;
}
