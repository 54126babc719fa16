// Shared device helpers for the gfx950 kernels: element types, rounding, MFMA fragments.
// Every translation unit is compiled with -ffp-contract=off, so `a * b + c` is a multiply
// and a separately rounded add, as the reference's NF4 decoder requires
// (kernels/nf4_cuda.py:42 launches with enable_fp_fusion=False).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/causal_tuner_hip.h"

namespace ct {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4;

constexpr int kWave = 64;

// ---------------------------------------------------------------- rounding to storage types
// Pins v in a VGPR as an fp32 value. Without it the backend folds `fp32 multiply ->
// half cast` into one v_fma_mixlo_f16 (a single rounding of the exact product), even with
// contraction off; the reference rounds the product to fp32 first and narrows after.
__device__ __forceinline__ float as_f32(float v) {
    asm volatile("" : "+v"(v));
    return v;
}

// fp32 -> bf16 bits, round to nearest even. On gfx950 the cast lowers to v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint16_t bf16_bits(float v) {
    __bf16 h = (__bf16)v;
    return __builtin_bit_cast(uint16_t, h);
}
// Two values -> one dword of bf16 (lo in the low half), as one v_cvt_pk_bf16_f32: the
// scalar form converts each value separately and re-packs them with a shift and an OR.
typedef __bf16 bf16x2_v __attribute__((ext_vector_type(2)));
typedef float f32x2_v __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    const f32x2_v f = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2_v));
}
__device__ __forceinline__ float bf16_to_f32(uint16_t bits) {
    return __builtin_bit_cast(float, (uint32_t)bits << 16);
}
__device__ __forceinline__ uint16_t f16_bits(float v) {
    _Float16 h = (_Float16)as_f32(v);
    return __builtin_bit_cast(uint16_t, h);
}
__device__ __forceinline__ float f16_to_f32(uint16_t bits) {
    return (float)__builtin_bit_cast(_Float16, bits);
}

// Round v to `storage` (the dtype the reference casts decoded values to), returning the
// rounded value widened back to fp32 (exact).
template <int STORAGE>
__device__ __forceinline__ float round_to_storage(float v) {
    if constexpr (STORAGE == CT_BF16) return bf16_to_f32(bf16_bits(v));
    else if constexpr (STORAGE == CT_F16) return f16_to_f32(f16_bits(v));
    else return v;
}

// ---------------------------------------------------------------- 8x8 16-bit transpose
// in[i] holds row i (8 values, two per dword, element 2p in the low half of dword p).
// out[j] receives column j: element i of out[j] = element j of in[i].
__device__ __forceinline__ void transpose8x8_b16(const uint4 (&in)[8], uint4 (&out)[8]) {
    const uint32_t *s = reinterpret_cast<const uint32_t *>(in);
    uint32_t *d = reinterpret_cast<uint32_t *>(out);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            // rows 2p (low half) and 2p+1 (high half) of column j
            uint32_t lo_row = s[(2 * p) * 4 + (j >> 1)];
            uint32_t hi_row = s[(2 * p + 1) * 4 + (j >> 1)];
            // v_perm_b32: selector bytes 0-3 pick from the second operand, 4-7 from the first.
            uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
            d[j * 4 + p] = __builtin_amdgcn_perm(hi_row, lo_row, sel);
        }
    }
}

// ---------------------------------------------------------------- MFMA 16x16x32 bf16
// v_mfma_f32_16x16x32_bf16. Lane l supplies A[l%16][8*(l/16) .. +7] and
// B[8*(l/16) .. +7][l%16]; it receives D[4*(l/16) + i][l%16] for i = 0..3.
__device__ __forceinline__ f32x4 mfma16x16x32(const uint4 &a, const uint4 &b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

__host__ __device__ constexpr int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace ct
