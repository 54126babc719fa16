// Partial GPT-J rotary embedding for gfx950: the MI355X replacement of the reference's
// Triton kernels `_rotate_pair`, `_rope` and `_owned_qk_rope` (kernels/core_cuda.py:133-189)
// behind `PartialRoPE`, `inverse_rope_tile` and `rotate_owned_qk` (core_cuda.py:192-229).
//
// Layout: x [tokens, heads, head_dim] with ldx elements between tokens (heads * head_dim
// when contiguous), y likewise with ldy; cosine and sine [tokens, half] contiguous,
// half <= head_dim / 2. Channel pairs (2c, 2c+1) with c < half rotate, the rest pass
// through. Per pair, in fp32 with every product rounded to the tensor type first
// (core_cuda.py:136-142, launched without FMA contraction):
//   ec = T(e c), os = T(o s), oc = T(o c), es = T(e s)
//   e' = T(ec - os), o' = T(oc + es)
// The inverse rotation negates the sine. HBM-bound elementwise work: one lane per pair.

#include "epilogue.hpp"

namespace ct {
namespace {

template <int T>
__device__ __forceinline__ float load_t(const void *p, int64_t i) {
    if constexpr (T == CT_BF16) return bf16_to_f32(static_cast<const uint16_t *>(p)[i]);
    else if constexpr (T == CT_F16) return f16_to_f32(static_cast<const uint16_t *>(p)[i]);
    else return static_cast<const float *>(p)[i];
}

template <int T>
__device__ __forceinline__ void store_t(void *p, int64_t i, float v) {
    if constexpr (T == CT_BF16) static_cast<uint16_t *>(p)[i] = bf16_bits(v);
    else if constexpr (T == CT_F16) static_cast<uint16_t *>(p)[i] = f16_bits(v);
    else static_cast<float *>(p)[i] = v;
}

template <int T, int TC, bool INVERSE>
__device__ __forceinline__ void rotate_pair(const void *x, int64_t xi, void *y, int64_t yi, float c, float s) {
    const float e = load_t<T>(x, xi), o = load_t<T>(x, xi + 1);
    if constexpr (INVERSE) s = -s;
    float e2, o2;
    rope_pair<T>(e, o, c, s, e2, o2);
    store_t<T>(y, yi, e2);
    store_t<T>(y, yi + 1, o2);
}

// Every pair of x -> y (y may be x): rotated channels rotate, the others are copied.
template <int T, int TC, bool INVERSE>
__global__ __launch_bounds__(256) void rope_all(const void *x, void *y, const void *cosine, const void *sine,
                                                int64_t pairs, int64_t heads, int64_t dim2, int64_t half, int64_t ldx,
                                                int64_t ldy) {
    const int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (p >= pairs) return;
    const int64_t per = heads * dim2;  // pairs per token
    const int64_t token = p / per, within = p - token * per;
    const int64_t channel = within % dim2;
    const int64_t xi = token * ldx + 2 * within, yi = token * ldy + 2 * within;
    if (channel < half) {
        const int64_t t = token * half + channel;
        rotate_pair<T, TC, INVERSE>(x, xi, y, yi, load_t<TC>(cosine, t), load_t<TC>(sine, t));
    } else if (x != y) {
        store_t<T>(y, yi, load_t<T>(x, xi));
        store_t<T>(y, yi + 1, load_t<T>(x, xi + 1));
    }
}

// In place, rotated channels only (the owned q/k outputs of a projection group).
template <int T, int TC, bool INVERSE>
__global__ __launch_bounds__(256) void rope_rotated(void *x, const void *cosine, const void *sine, int64_t pairs,
                                                    int64_t heads, int64_t dim2, int64_t half, int64_t ldx) {
    const int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x;  // over tokens x heads x half
    if (p >= pairs) return;
    const int64_t channel = p % half;
    const int64_t th = p / half;  // token * heads + head
    const int64_t token = th / heads, head = th - token * heads;
    const int64_t t = token * half + channel;
    const int64_t xi = token * ldx + 2 * (head * dim2 + channel);
    rotate_pair<T, TC, INVERSE>(x, xi, x, xi, load_t<TC>(cosine, t), load_t<TC>(sine, t));
}

template <int T, int TC, bool INVERSE>
hipError_t launch(const void *x, void *y, const void *cosine, const void *sine, int64_t tokens, int64_t heads,
                  int64_t head_dim, int64_t half, bool rotated_only, int64_t ldx, int64_t ldy, hipStream_t s) {
    const int64_t dim2 = head_dim / 2;
    const int64_t pairs = rotated_only ? tokens * heads * half : tokens * heads * dim2;
    if (pairs == 0) return hipSuccess;
    const dim3 grid((unsigned)cdiv(pairs, 256)), block(256);
    if (rotated_only)
        rope_rotated<T, TC, INVERSE><<<grid, block, 0, s>>>(y, cosine, sine, pairs, heads, dim2, half, ldy);
    else
        rope_all<T, TC, INVERSE><<<grid, block, 0, s>>>(x, y, cosine, sine, pairs, heads, dim2, half, ldx, ldy);
    return hipGetLastError();
}

template <int T, int TC>
hipError_t launch_dir(const void *x, void *y, const void *cosine, const void *sine, int64_t tokens, int64_t heads,
                      int64_t head_dim, int64_t half, bool inverse, bool rotated_only, int64_t ldx, int64_t ldy,
                      hipStream_t s) {
    return inverse ? launch<T, TC, true>(x, y, cosine, sine, tokens, heads, head_dim, half, rotated_only, ldx, ldy, s)
                   : launch<T, TC, false>(x, y, cosine, sine, tokens, heads, head_dim, half, rotated_only, ldx, ldy,
                                          s);
}

template <int T>
hipError_t launch_trig(const void *x, void *y, const void *cosine, const void *sine, int64_t tokens, int64_t heads,
                       int64_t head_dim, int64_t half, bool inverse, bool rotated_only, int trig, int64_t ldx,
                       int64_t ldy, hipStream_t s) {
    switch (trig) {
        case CT_BF16: return launch_dir<T, CT_BF16>(x, y, cosine, sine, tokens, heads, head_dim, half, inverse,
                                                    rotated_only, ldx, ldy, s);
        case CT_F16: return launch_dir<T, CT_F16>(x, y, cosine, sine, tokens, heads, head_dim, half, inverse,
                                                  rotated_only, ldx, ldy, s);
        default: return launch_dir<T, CT_F32>(x, y, cosine, sine, tokens, heads, head_dim, half, inverse,
                                              rotated_only, ldx, ldy, s);
    }
}

bool known_dtype(int d) { return d == CT_F32 || d == CT_F16 || d == CT_BF16; }

}  // namespace
}  // namespace ct

extern "C" int ct_rope(const void *x, void *y, const void *cosine, const void *sine, int64_t tokens, int64_t heads,
                       int64_t head_dim, int64_t half, int64_t ldx, int64_t ldy, int32_t inverse,
                       int32_t rotated_only, int32_t dtype, int32_t trig_dtype, hipStream_t stream) {
    using namespace ct;
    if (tokens < 0 || heads < 0 || head_dim <= 0 || head_dim % 2 || half < 0 || half > head_dim / 2)
        return -CT_EINVAL_SHAPE;
    if (ldx == 0) ldx = heads * head_dim;
    if (ldy == 0) ldy = heads * head_dim;
    if (ldx < heads * head_dim || ldy < heads * head_dim) return -CT_EINVAL_SHAPE;
    if (x == y && ldx != ldy) return -CT_EINVAL_LAYOUT;
    if (!known_dtype(dtype) || !known_dtype(trig_dtype)) return -CT_EINVAL_DTYPE;
    if (tokens == 0 || heads == 0) return 0;
    if (!x || !y || (half > 0 && (!cosine || !sine))) return -CT_EINVAL_POINTER;
    if (rotated_only && x != y) return -CT_EINVAL_LAYOUT;  // rotated-only runs in place
    if (rotated_only && half == 0) return 0;
    hipError_t e;
    switch (dtype) {
        case CT_BF16:
            e = launch_trig<CT_BF16>(x, y, cosine, sine, tokens, heads, head_dim, half, inverse, rotated_only,
                                     trig_dtype, ldx, ldy, stream);
            break;
        case CT_F16:
            e = launch_trig<CT_F16>(x, y, cosine, sine, tokens, heads, head_dim, half, inverse, rotated_only,
                                    trig_dtype, ldx, ldy, stream);
            break;
        default:
            e = launch_trig<CT_F32>(x, y, cosine, sine, tokens, heads, head_dim, half, inverse, rotated_only,
                                    trig_dtype, ldx, ldy, stream);
    }
    return e == hipSuccess ? 0 : (int)e;
}
