// Elementwise steps that follow a projection GEMM on the path: the SiLU-multiply of the
// MLP (reference kernels/mlp_cuda.py:10-35), its backward, the o/down-proj residual add
// (kernels/linear.py:90-91) and the partial GPT-J rotation of q/k (kernels/core_cuda.py:
// 133-189). The same device functions serve the fused GEMM epilogue (gemm.hip), the
// standalone fallback over a finished output (ct_apply_epilogue's kernel) and the
// standalone SiLU / RoPE kernels (activation.hip, rope.hip), so every route gives
// bit-identical values. Every function takes y, the GEMM output already rounded to bf16,
// as the reference stores it before the elementwise step.
#pragma once

#include "common.hpp"

namespace ct {

// ---------------------------------------------------------------- SiLU x up (fp32 math)
//   sig = 1 / (1 + exp(-g)), act = T(g * sig)          (T: round to the tensor type)
//   forward  h  = act * u
//   backward pg = T(grad * u), dg = pg * (sig * (1 + g * (1 - sig))), du = grad * act
template <int T>
__device__ __forceinline__ float silu_round(float v) {
    if constexpr (T == CT_BF16) return bf16_to_f32(bf16_bits(v));
    else return v;
}
template <int T>
__device__ __forceinline__ float silu_forward(float g, float u) {
    const float sig = 1.f / (1.f + expf(-g));
    const float act = silu_round<T>(g * sig);
    return act * u;
}
template <int T>
__device__ __forceinline__ void silu_backward(float g, float u, float grad, float &dg, float &du, float &h) {
    const float sig = 1.f / (1.f + expf(-g));
    const float act = silu_round<T>(g * sig);
    const float pg = silu_round<T>(grad * u);
    dg = pg * (sig * (1.f + g * (1.f - sig)));
    du = grad * act;
    h = act * u;
}

// ---------------------------------------------------------------- GPT-J pair rotation
// e' = T(T(e c) - T(o s)), o' = T(T(o c) + T(e s)), every product rounded to the tensor
// type first; the caller negates s for the inverse rotation. Returns the unrounded sums
// (the store rounds them).
template <int T>
__device__ __forceinline__ void rope_pair(float e, float o, float c, float s, float &e2, float &o2) {
    const float ec = round_to_storage<T>(e * c), os = round_to_storage<T>(o * s);
    const float oc = round_to_storage<T>(o * c), es = round_to_storage<T>(e * s);
    e2 = ec - os;
    o2 = oc + es;
}

template <int T>
__device__ __forceinline__ float load_typed(const void *p, int64_t i) {
    if constexpr (T == CT_BF16) return bf16_to_f32(static_cast<const uint16_t *>(p)[i]);
    else if constexpr (T == CT_F16) return f16_to_f32(static_cast<const uint16_t *>(p)[i]);
    else return static_cast<const float *>(p)[i];
}

__device__ __forceinline__ float load_trig(const void *p, int64_t i, int dtype) {
    if (dtype == CT_BF16) return load_typed<CT_BF16>(p, i);
    if (dtype == CT_F16) return load_typed<CT_F16>(p, i);
    return load_typed<CT_F32>(p, i);
}

// ---------------------------------------------------------------- bf16 GEMM epilogue
// The device view of ct_epilogue for bf16 outputs; row/col index the GEMM output.
struct EpiParams {
    int kind;        // CT_EPI_*
    int trig_dtype;  // ROPE
    const uint16_t *in0, *in1;
    int64_t ld_in0, ld_in1;
    uint16_t *out0, *out1;
    int64_t ld_out0, ld_out1;
    const void *cosine, *sine;  // ROPE: [rows, half] of trig_dtype
    int64_t head_dim, half;
    int vec;       // every side matrix 16-byte aligned with a row pitch of a multiple of 8
    int rope_vec;  // ROPE: head_dim % 8 == 0, half % 4 == 0 and the tables aligned for 4-value loads
};

// count (<= N) consecutive bf16 values from p as packed pairs (element 2j in the low half
// of w[j]); one 16-byte access for a full group of 8 when `vec` says p is 16-byte aligned.
template <int N>
__device__ __forceinline__ void load_bf16_pairs(const uint16_t *p, int count, int vec, uint32_t (&w)[N / 2]) {
    if constexpr (N == 8) {
        if (vec && count == 8) {
            const uint4 q = *reinterpret_cast<const uint4 *>(p);
            w[0] = q.x, w[1] = q.y, w[2] = q.z, w[3] = q.w;
            return;
        }
    }
#pragma unroll
    for (int j = 0; j < N / 2; ++j) {
        const uint32_t lo = 2 * j < count ? p[2 * j] : 0u, hi = 2 * j + 1 < count ? p[2 * j + 1] : 0u;
        w[j] = lo | (hi << 16);
    }
}

__device__ __forceinline__ float pair_value(const uint32_t w, int half) {
    return bf16_to_f32((uint16_t)(half ? w >> 16 : w & 0xffffu));
}

template <int N>
__device__ __forceinline__ void load_bf16_run(const uint16_t *p, int count, int vec, float (&v)[N]) {
    uint32_t w[N / 2];
    load_bf16_pairs<N>(p, count, vec, w);
#pragma unroll
    for (int j = 0; j < N; ++j) v[j] = pair_value(w[j / 2], j & 1);
}

template <int N>
__device__ __forceinline__ void store_bf16_run(uint16_t *p, int count, int vec, const float (&v)[N]) {
    if constexpr (N == 8) {
        if (vec && count == 8) {
            *reinterpret_cast<uint4 *>(p) = make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]),
                                                       pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7]));
            return;
        }
    }
#pragma unroll
    for (int j = 0; j < N; ++j)
        if (j < count) p[j] = bf16_bits(v[j]);
}

// Rotary pair of output column col + j (j even): its index inside the head, or -1 when
// the pair passes through. Columns stay below 2^31 (checked on the host).
__device__ __forceinline__ int rope_pair_index(const EpiParams &e, int64_t col, int j) {
    const int pair = (int)((uint32_t)(col + j) % (uint32_t)e.head_dim) / 2;
    return pair < e.half ? pair : -1;
}

// The side inputs of one run of N output columns of one row, read ahead of the step:
// in0 / in1 as packed bf16 pairs, or (ROPE) the float bits of each pair's cosine / sine.
template <int N>
struct EpiSide {
    uint32_t a[N / 2], b[N / 2];
};

template <int KIND, int N>
__device__ __forceinline__ void epilogue_load(const EpiParams &e, int64_t row, int64_t col, int count,
                                              EpiSide<N> &s) {
    if constexpr (KIND == CT_EPI_RESIDUAL || KIND == CT_EPI_SILU) {
        load_bf16_pairs<N>(e.in0 + row * e.ld_in0 + col, count, e.vec, s.a);
    } else if constexpr (KIND == CT_EPI_DSILU) {
        load_bf16_pairs<N>(e.in0 + row * e.ld_in0 + col, count, e.vec, s.a);
        load_bf16_pairs<N>(e.in1 + row * e.ld_in1 + col, count, e.vec, s.b);
    } else if constexpr (KIND == CT_EPI_ROPE) {
        if constexpr (N == 8) {
            if (e.rope_vec && count == 8) {
                // the run's 4 pairs sit in one head and either all rotate or none does
                const int pair = rope_pair_index(e, col, 0);
                if (pair < 0) return;
                const int64_t t = row * e.half + pair;
                if (e.trig_dtype == CT_F32) {
                    const uint4 c = *reinterpret_cast<const uint4 *>(static_cast<const float *>(e.cosine) + t);
                    const uint4 q = *reinterpret_cast<const uint4 *>(static_cast<const float *>(e.sine) + t);
                    s.a[0] = c.x, s.a[1] = c.y, s.a[2] = c.z, s.a[3] = c.w;
                    s.b[0] = q.x, s.b[1] = q.y, s.b[2] = q.z, s.b[3] = q.w;
                } else {
                    const uint2 c = *reinterpret_cast<const uint2 *>(static_cast<const uint16_t *>(e.cosine) + t);
                    const uint2 q = *reinterpret_cast<const uint2 *>(static_cast<const uint16_t *>(e.sine) + t);
                    const uint32_t cw[2] = {c.x, c.y}, sw[2] = {q.x, q.y};
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const uint16_t cb = (uint16_t)(j & 1 ? cw[j / 2] >> 16 : cw[j / 2] & 0xffffu);
                        const uint16_t sb = (uint16_t)(j & 1 ? sw[j / 2] >> 16 : sw[j / 2] & 0xffffu);
                        s.a[j] = __float_as_uint(e.trig_dtype == CT_BF16 ? bf16_to_f32(cb) : f16_to_f32(cb));
                        s.b[j] = __float_as_uint(e.trig_dtype == CT_BF16 ? bf16_to_f32(sb) : f16_to_f32(sb));
                    }
                }
                return;
            }
        }
#pragma unroll
        for (int j = 0; j + 1 < N; j += 2) {
            const int pair = j < count ? rope_pair_index(e, col, j) : -1;
            if (pair < 0) continue;
            const int64_t t = row * e.half + pair;
            s.a[j / 2] = __float_as_uint(load_trig(e.cosine, t, e.trig_dtype));
            s.b[j / 2] = __float_as_uint(load_trig(e.sine, t, e.trig_dtype));
        }
    }
}

// Applies the step to `count` consecutive columns col.. of one row: y[j] holds the GEMM
// output rounded to bf16 and `s` the run's side inputs (epilogue_load); side outputs are
// stored here, the main output's new values are returned in y (the caller rounds and
// stores them). count is even for ROPE (pairs never straddle: head_dim and the column
// start are even).
template <int KIND, int N>
__device__ __forceinline__ void epilogue_apply(const EpiParams &e, int64_t row, int64_t col, int count,
                                               const EpiSide<N> &s, float (&y)[N]) {
    if constexpr (KIND == CT_EPI_RESIDUAL) {
#pragma unroll
        for (int j = 0; j < N; ++j) y[j] = y[j] + pair_value(s.a[j / 2], j & 1);
    } else if constexpr (KIND == CT_EPI_SILU) {
        if (e.out0) store_bf16_run<N>(e.out0 + row * e.ld_out0 + col, count, e.vec, y);
#pragma unroll
        for (int j = 0; j < N; ++j) y[j] = silu_forward<CT_BF16>(pair_value(s.a[j / 2], j & 1), y[j]);
    } else if constexpr (KIND == CT_EPI_DSILU) {
        // out0/out1 may be in0/in1: every value was read (epilogue_load) before this lane
        // writes it
        float dg[N], du[N];
#pragma unroll
        for (int j = 0; j < N; ++j)
            silu_backward<CT_BF16>(pair_value(s.a[j / 2], j & 1), pair_value(s.b[j / 2], j & 1), y[j], dg[j], du[j],
                                   y[j]);
        store_bf16_run<N>(e.out0 + row * e.ld_out0 + col, count, e.vec, dg);
        store_bf16_run<N>(e.out1 + row * e.ld_out1 + col, count, e.vec, du);
    } else if constexpr (KIND == CT_EPI_ROPE) {
        if constexpr (N == 8) {
            if (e.rope_vec && count == 8) {
                if (rope_pair_index(e, col, 0) < 0) return;
#pragma unroll
                for (int j = 0; j < N; j += 2) {
                    float e2, o2;
                    rope_pair<CT_BF16>(y[j], y[j + 1], __uint_as_float(s.a[j / 2]), __uint_as_float(s.b[j / 2]), e2,
                                       o2);
                    y[j] = e2;
                    y[j + 1] = o2;
                }
                return;
            }
        }
#pragma unroll
        for (int j = 0; j + 1 < N; j += 2) {
            if (j >= count || rope_pair_index(e, col, j) < 0) continue;
            float e2, o2;
            rope_pair<CT_BF16>(y[j], y[j + 1], __uint_as_float(s.a[j / 2]), __uint_as_float(s.b[j / 2]), e2, o2);
            y[j] = e2;
            y[j + 1] = o2;
        }
    }
}

template <int KIND, int N>
__device__ __forceinline__ void epilogue_values_k(const EpiParams &e, int64_t row, int64_t col, int count,
                                                  float (&y)[N]) {
    EpiSide<N> s;
    epilogue_load<KIND, N>(e, row, col, count, s);
    epilogue_apply<KIND, N>(e, row, col, count, s, y);
}

template <int N>
__device__ __forceinline__ void epilogue_values(const EpiParams &e, int64_t row, int64_t col, int count,
                                                float (&y)[N]) {
    switch (e.kind) {
        case CT_EPI_RESIDUAL: epilogue_values_k<CT_EPI_RESIDUAL, N>(e, row, col, count, y); break;
        case CT_EPI_SILU: epilogue_values_k<CT_EPI_SILU, N>(e, row, col, count, y); break;
        case CT_EPI_DSILU: epilogue_values_k<CT_EPI_DSILU, N>(e, row, col, count, y); break;
        case CT_EPI_ROPE: epilogue_values_k<CT_EPI_ROPE, N>(e, row, col, count, y); break;
        default: break;
    }
}

// Launches the standalone form over a finished bf16 product src [m, n] (row pitch ldsrc),
// writing the step's main output to dst (may be src), 8 columns per lane: the pass for GEMM
// routes that do not fuse the step.
hipError_t epilogue_run(const EpiParams &e, const uint16_t *src, int64_t ldsrc, uint16_t *dst, int64_t lddst, int64_t m,
                        int64_t n, hipStream_t stream);

}  // namespace ct
