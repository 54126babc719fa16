// float32 GEMM for the projection operators' float32 compute dtype: the reference runs its
// projections through torch.mm / addmm in whatever compute dtype the model uses
// (kernels/linear.py:16-44, with TF32 off in train.py:80-82), so a float32 model needs
// every product of forward_linear, input_gradient and parameter_gradients in full fp32.
//
//   C[m, n] = op(A)[m, k] op(B)[k, n] (+ C when beta) (+ bias[n])
//
// op(A) is A stored [m, k] (trans_a = 0) or [k, m] (trans_a = 1); op(B) is B stored [k, n]
// (trans_b = 0) or [n, k] (trans_b = 1); leading dimensions are the stored row pitches.
// With beta = 0 the destination is never read (garbage or NaN there is ignored).
//
// Design: v_mfma_f32_16x16x4_f32 (full fp32 products and sums; no TF32 or reduced-
// precision step), 128 x 128 output tiles of 4 waves (2 x 2 of 64 x 64), BK = 16, both
// operands staged k-major in LDS (rows padded by 16 floats so the four k rows a wave
// reads at once fall in distinct banks), the next k-slice loaded into registers while the
// current one is multiplied. Every output element is one in-order reduction over k by one
// lane, so results are deterministic and independent of the grid.

#include "common.hpp"

namespace ct {
namespace {

constexpr int kBM = 128, kBN = 128, kBK = 16, kPad = 16, kThreadsF32 = 256;
constexpr int kRow = kBM + kPad;  // floats per k row of a staged tile (kBM == kBN)

__device__ __forceinline__ f32x4 mfma_f32(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

struct F32Args {
    const float *a, *b, *bias;
    float *c;
    int64_t lda, ldb, ldc, m, n, k;
    int trans_a, trans_b, beta, vec_a, vec_b;
};

// One operand's k-slice [k0, k0 + 16) of the tile rows [r0, r0 + 128) into registers:
// eight values per thread. `rows_fast` says the stored matrix is contiguous along the tile
// rows (m of A when trans_a, n of B when !trans_b); otherwise it is contiguous along k.
struct Slice {
    float v[8];
};

__device__ __forceinline__ void load_slice(const float *p, int64_t ld, bool rows_fast, bool vec, int64_t r0,
                                           int64_t rows, int64_t k0, int64_t kdim, int tid, Slice &s) {
    if (rows_fast) {
        // stored [k, rows]: thread t covers k row (t / 32) * 2 + h, rows 4 (t % 32) .. +3
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int kk = (tid / 32) * 2 + h, rr = (tid % 32) * 4;
            const int64_t kg = k0 + kk, rg = r0 + rr;
            if (vec && kg < kdim && rg + 3 < rows) {
                const f32x4 q = *reinterpret_cast<const f32x4 *>(p + kg * ld + rg);
                s.v[4 * h + 0] = q[0], s.v[4 * h + 1] = q[1], s.v[4 * h + 2] = q[2], s.v[4 * h + 3] = q[3];
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) s.v[4 * h + j] = (kg < kdim && rg + j < rows) ? p[kg * ld + rg + j] : 0.f;
            }
        }
    } else {
        // stored [rows, k]: thread t covers row (t / 4) + 64 h, k 4 (t % 4) .. +3
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int rr = tid / 4 + 64 * h, kk = (tid % 4) * 4;
            const int64_t kg = k0 + kk, rg = r0 + rr;
            if (vec && rg < rows && kg + 3 < kdim) {
                const f32x4 q = *reinterpret_cast<const f32x4 *>(p + rg * ld + kg);
                s.v[4 * h + 0] = q[0], s.v[4 * h + 1] = q[1], s.v[4 * h + 2] = q[2], s.v[4 * h + 3] = q[3];
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) s.v[4 * h + j] = (rg < rows && kg + j < kdim) ? p[rg * ld + kg + j] : 0.f;
            }
        }
    }
}

// Registers -> the k-major LDS tile t[k][row].
__device__ __forceinline__ void store_slice(float *t, bool rows_fast, int tid, const Slice &s) {
    if (rows_fast) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int kk = (tid / 32) * 2 + h, rr = (tid % 32) * 4;
            *reinterpret_cast<f32x4 *>(t + kk * kRow + rr) =
                f32x4{s.v[4 * h], s.v[4 * h + 1], s.v[4 * h + 2], s.v[4 * h + 3]};
        }
    } else {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int rr = tid / 4 + 64 * h, kk = (tid % 4) * 4;
#pragma unroll
            for (int j = 0; j < 4; ++j) t[(kk + j) * kRow + rr] = s.v[4 * h + j];
        }
    }
}

__global__ __launch_bounds__(kThreadsF32) void gemm_f32(const F32Args g) {
    __shared__ float sa[2][kBK * kRow];
    __shared__ float sb[2][kBK * kRow];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t tiles_n = (g.n + kBN - 1) / kBN;
    const int64_t m0 = (int64_t)(blockIdx.x / tiles_n) * kBM, n0 = (int64_t)(blockIdx.x % tiles_n) * kBN;
    const int wm = (wave & 1) * 64, wn = (wave >> 1) * 64;
    const bool a_rows_fast = g.trans_a != 0, b_rows_fast = g.trans_b == 0;

    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int64_t steps = (g.k + kBK - 1) / kBK;
    Slice la, lb;
    if (steps > 0) {
        load_slice(g.a, g.lda, a_rows_fast, g.vec_a, m0, g.m, 0, g.k, tid, la);
        load_slice(g.b, g.ldb, b_rows_fast, g.vec_b, n0, g.n, 0, g.k, tid, lb);
        store_slice(sa[0], a_rows_fast, tid, la);
        store_slice(sb[0], b_rows_fast, tid, lb);
    }
    __syncthreads();
    for (int64_t s = 0; s < steps; ++s) {
        const int cur = (int)(s & 1);
        const bool more = s + 1 < steps;
        if (more) {
            load_slice(g.a, g.lda, a_rows_fast, g.vec_a, m0, g.m, (s + 1) * kBK, g.k, tid, la);
            load_slice(g.b, g.ldb, b_rows_fast, g.vec_b, n0, g.n, (s + 1) * kBK, g.k, tid, lb);
        }
        const float *ta = sa[cur], *tb = sb[cur];
#pragma unroll
        for (int kk = 0; kk < kBK; kk += 4) {
            const int kr = kk + lane / 16;
            float af[4], bf[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) af[i] = ta[kr * kRow + wm + i * 16 + (lane & 15)];
#pragma unroll
            for (int j = 0; j < 4; ++j) bf[j] = tb[kr * kRow + wn + j * 16 + (lane & 15)];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = mfma_f32(af[i], bf[j], acc[i][j]);
        }
        if (more) {
            store_slice(sa[cur ^ 1], a_rows_fast, tid, la);
            store_slice(sb[cur ^ 1], b_rows_fast, tid, lb);
        }
        __syncthreads();
    }

    // lane l holds rows 4 (l / 16) + e of each 16-row block and column l % 16
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int64_t col = n0 + wn + j * 16 + (lane & 15);
        if (col >= g.n) continue;
        const float bias = g.bias ? g.bias[col] : 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int64_t row = m0 + wm + i * 16 + (lane >> 4) * 4 + e;
                if (row >= g.m) continue;
                float *c = g.c + row * g.ldc + col;
                const float v = acc[i][j][e] + bias;
                *c = g.beta ? *c + v : v;
            }
    }
}

}  // namespace
}  // namespace ct

extern "C" int ct_gemm_f32(const float *a, int64_t lda, int32_t trans_a, const float *b, int64_t ldb, int32_t trans_b,
                           float *c, int64_t ldc, int32_t beta, const float *bias, int64_t m, int64_t n, int64_t k,
                           hipStream_t stream) {
    using namespace ct;
    if (m < 0 || n < 0 || k < 0) return -CT_EINVAL_SHAPE;
    if (m == 0 || n == 0) return 0;
    if (!c || (k > 0 && (!a || !b))) return -CT_EINVAL_POINTER;
    const int64_t arows = trans_a ? k : m, acols = trans_a ? m : k;
    const int64_t brows = trans_b ? n : k, bcols = trans_b ? k : n;
    if (ldc < n || (k > 0 && (lda < acols || ldb < bcols)) || arows < 0 || brows < 0) return -CT_EINVAL_SHAPE;
    F32Args g{};
    g.a = a, g.b = b, g.bias = bias, g.c = c;
    g.lda = lda, g.ldb = ldb, g.ldc = ldc, g.m = m, g.n = n, g.k = k;
    g.trans_a = trans_a != 0, g.trans_b = trans_b != 0, g.beta = beta != 0;
    g.vec_a = reinterpret_cast<uintptr_t>(a) % 16 == 0 && lda % 4 == 0;
    g.vec_b = reinterpret_cast<uintptr_t>(b) % 16 == 0 && ldb % 4 == 0;
    const int64_t tiles = ((m + kBM - 1) / kBM) * ((n + kBN - 1) / kBN);
    if (tiles > 0x7fffffff) return -CT_EINVAL_SHAPE;
    gemm_f32<<<dim3((unsigned)tiles), dim3(kThreadsF32), 0, stream>>>(g);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : (int)e;  // a positive HIP error code
}
