// bf16 MFMA GEMMs for the NF4-LoRA projection path on gfx950.
//
// One kernel template serves every contraction of the reference's operator layer
// (kernels/linear.py:27-44): C[m,n] = sum over one or two K segments of A(m,k) B(k,n),
// with fp32 accumulation in v_mfma_f32_16x16x32_bf16 and a fused epilogue (bias, beta
// accumulation, bf16 or fp32 output, or fp32 split partials).
//
// Two segments implement the rank-r LoRA terms as extra reduction columns:
//   forward  out = [x | xa] [w | b]^T      (segment 0: k columns, segment 1: r columns)
//   backward dx  = [dy | low] [w ; a]      (segment 0: n rows,    segment 1: r rows)
// so the low-rank epilogue costs no extra pass over the output.
//
// Operand staging: each k-tile of both operands is written into LDS as [rows][64] bf16
// with the reduction dimension contiguous, in 16-byte chunks whose position within a
// 128-byte row is XORed with a row-dependent swizzle (conflict-free ds_read_b128 for the
// MFMA fragment reads). A source whose reduction dimension is contiguous in HBM is copied
// chunk by chunk; a source whose output dimension is contiguous ("k-strided") is loaded
// as 8x8 blocks of 16-byte rows and transposed in registers with v_perm_b32.
//
// Fragment mapping: lane l of a wave reads A rows wm0 + 16 f + l%16 and B rows
// wn0 + (l%16) FN + f for fragment f, so each lane's accumulators for a fixed output row
// cover FN consecutive columns and the epilogue writes FN-element vectors.

#include "common.hpp"

namespace ct {

int validate_nf4(const ct_nf4_weight *w);

namespace {

constexpr int kBK = 64;       // reduction columns per k-tile (8 chunks of 8 bf16)
constexpr int kThreads = 256; // 4 wavefronts per workgroup
enum { SRC_KC = 0, SRC_KS = 1 };

struct Segment {
    const uint16_t *a;  // bf16 bits
    const uint16_t *b;
    int64_t lda, ldb;
    int64_t k;          // reduction extent of this segment
};

struct GemmParams {
    Segment seg[2];
    int nseg;
    int64_t m, n;
    void *c;
    int64_t ldc;
    int64_t split_stride;     // elements between split partial outputs (blockIdx.z)
    int64_t tiles_per_split;  // k-tiles handled by one blockIdx.z
    const uint16_t *bias;     // bf16 [n] or null
    int beta;                 // add the existing C
};

__device__ __forceinline__ uint4 zero4() { return make_uint4(0, 0, 0, 0); }

// ------------------------------------------------------------------ operand tile loader
// ROWS: output-dimension extent of the tile. SWZ_DIV: rows that share one swizzle value
// (1 for A; FN for B, whose fragment rows are strided by FN).
template <int ROWS, int SRC, bool VEC, int SWZ_DIV>
struct Loader {
    static constexpr int kKcPerThread = (ROWS * 8 + kThreads - 1) / kThreads;
    static constexpr int kRegs = SRC == SRC_KC ? kKcPerThread : 8;
    uint4 r[kRegs];

    __device__ __forceinline__ static int slot(int row, int chunk) {
        return row * 8 + (chunk ^ ((row / SWZ_DIV) & 7));
    }

    // Source element (row, k) lives at p[row * ld + k] (KC) or p[k * ld + row] (KS).
    __device__ __forceinline__ void load(const uint16_t *p, int64_t ld, int64_t rows, int64_t kext,
                                         int64_t r0, int64_t k0, int tid) {
        if constexpr (SRC == SRC_KC) {
#pragma unroll
            for (int i = 0; i < kKcPerThread; ++i) {
                const int id = tid + i * kThreads;
                if (id >= ROWS * 8) break;
                const int64_t row = r0 + (id >> 3);
                const int64_t k = k0 + (id & 7) * 8;
                if constexpr (VEC) {
                    r[i] = (row < rows && k < kext) ? *reinterpret_cast<const uint4 *>(p + row * ld + k)
                                                    : zero4();
                } else {
                    uint16_t e[8];
#pragma unroll
                    for (int j = 0; j < 8; ++j)
                        e[j] = (row < rows && k + j < kext) ? p[row * ld + k + j] : uint16_t(0);
                    r[i] = __builtin_bit_cast(uint4, e);
                }
            }
        } else {
            // 8x8 block: k-chunk c = tid % 8, row block rb = tid / 8 (ROWS/8 row blocks).
            if (tid >= ROWS) return;
            const int64_t row = r0 + (tid >> 3) * 8;
            const int64_t kb = k0 + (tid & 7) * 8;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int64_t k = kb + i;
                if constexpr (VEC) {
                    r[i] = (k < kext && row < rows) ? *reinterpret_cast<const uint4 *>(p + k * ld + row)
                                                    : zero4();
                } else {
                    uint16_t e[8];
#pragma unroll
                    for (int j = 0; j < 8; ++j)
                        e[j] = (k < kext && row + j < rows) ? p[k * ld + row + j] : uint16_t(0);
                    r[i] = __builtin_bit_cast(uint4, e);
                }
            }
        }
    }

    __device__ __forceinline__ void store(uint4 *lds, int tid) const {
        if constexpr (SRC == SRC_KC) {
#pragma unroll
            for (int i = 0; i < kKcPerThread; ++i) {
                const int id = tid + i * kThreads;
                if (id >= ROWS * 8) break;
                lds[slot(id >> 3, id & 7)] = r[i];
            }
        } else {
            if (tid >= ROWS) return;
            uint4 t[8];
            transpose8x8_b16(r, t);
            const int row = (tid >> 3) * 8;
            const int chunk = tid & 7;
#pragma unroll
            for (int j = 0; j < 8; ++j) lds[slot(row + j, chunk)] = t[j];
        }
    }
};

// ------------------------------------------------------------------------- the kernel
template <int BM, int BN, int WAVES_M, int A_SRC, int B_SRC, bool VEC, int OUT>
__global__ __launch_bounds__(kThreads) void gemm_kernel(const GemmParams p) {
    constexpr int WAVES_N = 4 / WAVES_M;
    constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;  // wave tile
    constexpr int FM = WM / 16, FN = WN / 16;             // 16x16 fragments per wave
    using LA = Loader<BM, A_SRC, VEC, 1>;
    using LB = Loader<BN, B_SRC, VEC, FN>;

    __shared__ uint4 lds[2][(BM + BN) * 8];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm0 = (wave % WAVES_M) * WM, wn0 = (wave / WAVES_M) * WN;
    const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;

    const int64_t t0 = cdiv(p.seg[0].k, kBK);
    const int64_t total = t0 + (p.nseg > 1 ? cdiv(p.seg[1].k, kBK) : 0);
    const int64_t tbeg = (int64_t)blockIdx.z * p.tiles_per_split;
    const int64_t tend = tbeg + p.tiles_per_split < total ? tbeg + p.tiles_per_split : total;

    LA la;
    LB lb;
    auto fetch = [&](int64_t t) {
        const int s = t < t0 ? 0 : 1;
        const int64_t k0 = (s == 0 ? t : t - t0) * kBK;
        const Segment &g = p.seg[s];
        la.load(g.a, g.lda, p.m, g.k, m0, k0, tid);
        lb.load(g.b, g.ldb, p.n, g.k, n0, k0, tid);
    };

    f32x4 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    if (tbeg < tend) {
        fetch(tbeg);
        la.store(lds[0], tid);
        lb.store(lds[0] + BM * 8, tid);
        __syncthreads();
        for (int64_t t = tbeg; t < tend; ++t) {
            const int buf = (int)((t - tbeg) & 1);
            if (t + 1 < tend) fetch(t + 1);
            const uint4 *sa = lds[buf];
            const uint4 *sb = lds[buf] + BM * 8;
#pragma unroll
            for (int ks = 0; ks < kBK / 32; ++ks) {
                const int chunk = ks * 4 + (lane >> 4);
                uint4 af[FM], bf[FN];
#pragma unroll
                for (int i = 0; i < FM; ++i) af[i] = sa[LA::slot(wm0 + i * 16 + (lane & 15), chunk)];
#pragma unroll
                for (int j = 0; j < FN; ++j) bf[j] = sb[LB::slot(wn0 + (lane & 15) * FN + j, chunk)];
#pragma unroll
                for (int i = 0; i < FM; ++i)
#pragma unroll
                    for (int j = 0; j < FN; ++j) acc[i][j] = mfma16x16x32(af[i], bf[j], acc[i][j]);
            }
            if (t + 1 < tend) {
                la.store(lds[buf ^ 1], tid);
                lb.store(lds[buf ^ 1] + BM * 8, tid);
            }
            __syncthreads();
        }
    }

    // ------------------------------------------------------------------ epilogue
    const int64_t col = n0 + wn0 + (lane & 15) * FN;
    float bias[FN];
#pragma unroll
    for (int j = 0; j < FN; ++j)
        bias[j] = (p.bias && col + j < p.n) ? bf16_to_f32(p.bias[col + j]) : 0.f;
    const bool full = col + FN <= p.n;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int64_t row = m0 + wm0 + i * 16 + (lane >> 4) * 4 + e;
            if (row >= p.m) continue;
            float v[FN];
#pragma unroll
            for (int j = 0; j < FN; ++j) v[j] = acc[i][j][e] + bias[j];
            if constexpr (OUT == CT_F32) {
                float *c = static_cast<float *>(p.c) + (int64_t)blockIdx.z * p.split_stride + row * p.ldc + col;
#pragma unroll
                for (int j = 0; j < FN; ++j) {
                    if (!full && col + j >= p.n) break;
                    c[j] = p.beta ? v[j] + c[j] : v[j];
                }
            } else {
                uint16_t *c = static_cast<uint16_t *>(p.c) + row * p.ldc + col;
                if (p.beta) {
#pragma unroll
                    for (int j = 0; j < FN; ++j)
                        if (full || col + j < p.n) v[j] = v[j] + bf16_to_f32(c[j]);
                }
                if (VEC && full && FN == 4) {
                    uint2 w;
                    w.x = pack_bf16x2(v[0], v[1]);
                    w.y = pack_bf16x2(v[2], v[3]);
                    *reinterpret_cast<uint2 *>(c) = w;
                } else {
#pragma unroll
                    for (int j = 0; j < FN; ++j) {
                        if (!full && col + j >= p.n) break;
                        c[j] = bf16_bits(v[j]);
                    }
                }
            }
        }
    }
}

// Deterministic reduction of fp32 split partials: out = sum_z ws[z] (+ out), in z order.
template <int OUT>
__global__ __launch_bounds__(256) void reduce_splits(const float *__restrict__ ws, int splits, int64_t stride,
                                                     int64_t rows, int64_t cols, void *out, int64_t ldo,
                                                     int add) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= rows * cols) return;
    const int64_t r = i / cols, c = i % cols;
    float s = ws[i];
    for (int z = 1; z < splits; ++z) s += ws[z * stride + i];
    if constexpr (OUT == CT_F32) {
        float *o = static_cast<float *>(out) + r * ldo + c;
        *o = add ? s + *o : s;
    } else {
        uint16_t *o = static_cast<uint16_t *>(out) + r * ldo + c;
        *o = bf16_bits(add ? s + bf16_to_f32(*o) : s);
    }
}

// ------------------------------------------------------------------------ host side
struct Problem {
    GemmParams p;
    int a_src, b_src;
    int out;      // CT_BF16 or CT_F32
    bool vec;
    int splits;
};

bool aligned16(const void *q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; }

// Vector (16-byte) operand access needs aligned bases, leading dimensions that are
// multiples of 8 elements, and 8-multiple extents along each contiguous dimension.
bool vec_ok(const Problem &pr) {
    const GemmParams &p = pr.p;
    for (int s = 0; s < p.nseg; ++s) {
        const Segment &g = p.seg[s];
        if (!aligned16(g.a) || !aligned16(g.b) || g.lda % 8 || g.ldb % 8) return false;
        if (g.k % 8) return false;
        if (pr.a_src == SRC_KS && p.m % 8) return false;
        if (pr.b_src == SRC_KS && p.n % 8) return false;
    }
    if (pr.out == CT_BF16 && (!aligned16(p.c) || p.ldc % 8)) return false;
    return true;
}

template <int BM, int BN, int WAVES_M, int A_SRC, int B_SRC, bool VEC, int OUT>
hipError_t launch_cfg(const GemmParams &p, int splits, hipStream_t s) {
    dim3 grid((unsigned)cdiv(p.n, BN), (unsigned)cdiv(p.m, BM), (unsigned)splits);
    gemm_kernel<BM, BN, WAVES_M, A_SRC, B_SRC, VEC, OUT><<<grid, dim3(kThreads), 0, s>>>(p);
    return hipGetLastError();
}

template <int A_SRC, int B_SRC, bool VEC, int OUT>
hipError_t launch_tiles(const GemmParams &p, int splits, bool small, hipStream_t s) {
    if (small) return launch_cfg<64, 64, 2, A_SRC, B_SRC, VEC, OUT>(p, splits, s);
    return launch_cfg<128, 128, 2, A_SRC, B_SRC, VEC, OUT>(p, splits, s);
}

template <int A_SRC, int B_SRC>
hipError_t launch_layout(const GemmParams &p, int splits, bool small, bool vec, int out, hipStream_t s) {
    if (vec) {
        return out == CT_F32 ? launch_tiles<A_SRC, B_SRC, true, CT_F32>(p, splits, small, s)
                             : launch_tiles<A_SRC, B_SRC, true, CT_BF16>(p, splits, small, s);
    }
    return out == CT_F32 ? launch_tiles<A_SRC, B_SRC, false, CT_F32>(p, splits, small, s)
                         : launch_tiles<A_SRC, B_SRC, false, CT_BF16>(p, splits, small, s);
}

int64_t total_tiles(const GemmParams &p) {
    return cdiv(p.seg[0].k, kBK) + (p.nseg > 1 ? cdiv(p.seg[1].k, kBK) : 0);
}

// Small problems (fewer than ~2 waves of 128x128 tiles over 256 CUs) use 64x64 tiles.
bool use_small_tiles(int64_t m, int64_t n) { return cdiv(m, 128) * cdiv(n, 128) < 512; }

hipError_t run(Problem &pr, hipStream_t s) {
    GemmParams &p = pr.p;
    if (p.m == 0 || p.n == 0) return hipSuccess;
    const bool small = use_small_tiles(p.m, p.n);
    const int64_t tiles = total_tiles(p);
    p.tiles_per_split = cdiv(tiles > 0 ? tiles : 1, pr.splits);
    const int a = pr.a_src, b = pr.b_src;
    if (a == SRC_KC && b == SRC_KC) return launch_layout<SRC_KC, SRC_KC>(p, pr.splits, small, pr.vec, pr.out, s);
    if (a == SRC_KC && b == SRC_KS) return launch_layout<SRC_KC, SRC_KS>(p, pr.splits, small, pr.vec, pr.out, s);
    if (a == SRC_KS && b == SRC_KS) return launch_layout<SRC_KS, SRC_KS>(p, pr.splits, small, pr.vec, pr.out, s);
    return launch_layout<SRC_KS, SRC_KC>(p, pr.splits, small, pr.vec, pr.out, s);
}

// Split count for a reduction-heavy GEMM with a small output (dA, dB): enough
// workgroups to cover the 256 CUs about twice, at least 4 k-tiles per split.
int choose_splits(int64_t m, int64_t n, int64_t kred) {
    const int64_t tiles_out = use_small_tiles(m, n) ? cdiv(m, 64) * cdiv(n, 64) : cdiv(m, 128) * cdiv(n, 128);
    const int64_t ktiles = cdiv(kred, kBK);
    int64_t s = cdiv(512, tiles_out > 0 ? tiles_out : 1);
    const int64_t cap = ktiles / 4 > 1 ? ktiles / 4 : 1;
    if (s > cap) s = cap;
    if (s > 32) s = 32;
    return (int)(s < 1 ? 1 : s);
}

int64_t split_workspace_bytes(int64_t m, int64_t n, int64_t kred) {
    const int s = choose_splits(m, n, kred);
    return s > 1 ? (int64_t)s * m * n * (int64_t)sizeof(float) : 0;
}

// out (fp32 or bf16) = sum_k A B (+ out) through split partials in ws when profitable.
hipError_t run_reduction(Problem pr, void *out, int64_t ldo, int add, void *ws, int64_t ws_bytes,
                         hipStream_t s, int *status) {
    GemmParams &p = pr.p;
    const int64_t kred = p.seg[0].k;
    const int splits = choose_splits(p.m, p.n, kred);
    *status = 0;
    if (splits <= 1) {
        pr.splits = 1;
        p.c = out;
        p.ldc = ldo;
        p.beta = add;
        return run(pr, s);
    }
    const int64_t need = (int64_t)splits * p.m * p.n * (int64_t)sizeof(float);
    if (!ws || ws_bytes < need) {
        *status = -CT_EINVAL_WORKSPACE;
        return hipSuccess;
    }
    const int final_out = pr.out;
    pr.splits = splits;
    pr.out = CT_F32;
    p.c = ws;
    p.ldc = p.n;
    p.split_stride = p.m * p.n;
    p.beta = 0;
    p.bias = nullptr;
    hipError_t e = run(pr, s);
    if (e != hipSuccess) return e;
    const int64_t count = p.m * p.n;
    const unsigned grid = (unsigned)cdiv(count, 256);
    if (final_out == CT_F32)
        reduce_splits<CT_F32><<<grid, 256, 0, s>>>(static_cast<float *>(ws), splits, p.split_stride, p.m, p.n,
                                                   out, ldo, add);
    else
        reduce_splits<CT_BF16><<<grid, 256, 0, s>>>(static_cast<float *>(ws), splits, p.split_stride, p.m,
                                                    p.n, out, ldo, add);
    return hipGetLastError();
}

int to_status(hipError_t e) { return e == hipSuccess ? 0 : (int)e; }

}  // namespace
}  // namespace ct

using namespace ct;

extern "C" int ct_abi_version(void) { return 1; }

extern "C" const char *ct_status_string(int status) {
    switch (status) {
        case 0: return "success";
        case -CT_EINVAL_POINTER: return "invalid argument: null or misaligned pointer";
        case -CT_EINVAL_SHAPE: return "invalid argument: size or leading dimension out of range";
        case -CT_EINVAL_DTYPE: return "invalid argument: unsupported element type";
        case -CT_EINVAL_BLOCKSIZE: return "invalid argument: unsupported NF4 block size";
        case -CT_EINVAL_WORKSPACE: return "invalid argument: workspace missing or too small";
        default: return status > 0 ? hipGetErrorString((hipError_t)status) : "unknown status";
    }
}

extern "C" int ct_gemm(const void *a, int64_t lda, int32_t trans_a, const void *b, int64_t ldb, int32_t trans_b,
                       void *c, int64_t ldc, int32_t c_dtype, const void *bias, int32_t beta, int64_t m, int64_t n,
                       int64_t k, hipStream_t stream) {
    if (m < 0 || n < 0 || k < 0) return -CT_EINVAL_SHAPE;
    if (c_dtype != CT_BF16 && c_dtype != CT_F32) return -CT_EINVAL_DTYPE;
    if (m == 0 || n == 0) return 0;
    if (!c || (k > 0 && (!a || !b))) return -CT_EINVAL_POINTER;
    if (ldc < n || lda < (trans_a ? m : k) || ldb < (trans_b ? k : n)) return -CT_EINVAL_SHAPE;
    Problem pr{};
    pr.p.seg[0] = Segment{static_cast<const uint16_t *>(a), static_cast<const uint16_t *>(b), lda, ldb, k};
    pr.p.nseg = 1;
    pr.p.m = m;
    pr.p.n = n;
    pr.p.c = c;
    pr.p.ldc = ldc;
    pr.p.bias = static_cast<const uint16_t *>(bias);
    pr.p.beta = beta;
    pr.a_src = trans_a ? SRC_KS : SRC_KC;
    pr.b_src = trans_b ? SRC_KC : SRC_KS;
    pr.out = c_dtype;
    pr.splits = 1;
    pr.vec = vec_ok(pr);
    return to_status(run(pr, stream));
}

extern "C" int ct_forward_linear(const void *x, int64_t ldx, const void *w_dense, const ct_nf4_weight *w_nf4,
                                 const void *a, const void *b, const void *bias, void *out, int64_t ldo, void *xa,
                                 int64_t m, int64_t n, int64_t k, int64_t r, hipStream_t stream) {
    if (m < 0 || n < 0 || k < 0 || r < 0) return -CT_EINVAL_SHAPE;
    if (m == 0 || n == 0) return 0;
    if (w_nf4) return -CT_EINVAL_POINTER;  // the fused NF4 operand is not built into this entry yet
    if (!x || !w_dense || !out || (r > 0 && (!a || !b || !xa))) return -CT_EINVAL_POINTER;
    if (ldx < k || ldo < n) return -CT_EINVAL_SHAPE;
    int st;
    if (r > 0) {
        // xa = x a^T  (NT, bf16 out)
        st = ct_gemm(x, ldx, 0, a, k, 1, xa, r, CT_BF16, nullptr, 0, m, r, k, stream);
        if (st) return st;
    }
    Problem pr{};
    pr.p.seg[0] = Segment{static_cast<const uint16_t *>(x), static_cast<const uint16_t *>(w_dense), ldx, k, k};
    pr.p.seg[1] = Segment{static_cast<const uint16_t *>(xa), static_cast<const uint16_t *>(b), r, r, r};
    pr.p.nseg = r > 0 ? 2 : 1;
    pr.p.m = m;
    pr.p.n = n;
    pr.p.c = out;
    pr.p.ldc = ldo;
    pr.p.bias = static_cast<const uint16_t *>(bias);
    pr.p.beta = 0;
    pr.a_src = SRC_KC;
    pr.b_src = SRC_KC;
    pr.out = CT_BF16;
    pr.splits = 1;
    pr.vec = vec_ok(pr);
    return to_status(run(pr, stream));
}

extern "C" int ct_input_gradient(const void *dy, int64_t lddy, const void *w_dense, const ct_nf4_weight *w_nf4,
                                 const void *a, const void *b, void *dx, int64_t lddx, void *low, int64_t m,
                                 int64_t n, int64_t k, int64_t r, int32_t add, hipStream_t stream) {
    if (m < 0 || n < 0 || k < 0 || r < 0) return -CT_EINVAL_SHAPE;
    if (m == 0 || k == 0) return 0;
    if (w_nf4) return -CT_EINVAL_POINTER;
    if (!dy || !w_dense || !dx || (r > 0 && (!a || !b || !low))) return -CT_EINVAL_POINTER;
    if (lddy < n || lddx < k) return -CT_EINVAL_SHAPE;
    int st;
    if (r > 0) {
        // low = dy b  (NN, bf16 out)
        st = ct_gemm(dy, lddy, 0, b, r, 0, low, r, CT_BF16, nullptr, 0, m, r, n, stream);
        if (st) return st;
    }
    Problem pr{};
    pr.p.seg[0] = Segment{static_cast<const uint16_t *>(dy), static_cast<const uint16_t *>(w_dense), lddy, k, n};
    pr.p.seg[1] = Segment{static_cast<const uint16_t *>(low), static_cast<const uint16_t *>(a), r, k, r};
    pr.p.nseg = r > 0 ? 2 : 1;
    pr.p.m = m;
    pr.p.n = k;
    pr.p.c = dx;
    pr.p.ldc = lddx;
    pr.p.beta = add;
    pr.a_src = SRC_KC;
    pr.b_src = SRC_KS;
    pr.out = CT_BF16;
    pr.splits = 1;
    pr.vec = vec_ok(pr);
    return to_status(run(pr, stream));
}

extern "C" int64_t ct_accumulate_workspace(int64_t p, int64_t q, int64_t j) {
    if (p <= 0 || q <= 0 || j <= 0) return 0;
    return split_workspace_bytes(p, q, j);
}

extern "C" int ct_accumulate(float *out, int64_t ldo, const void *left, int64_t ldl, int32_t trans_l,
                             const void *right, int64_t ldr, int32_t trans_r, int64_t p, int64_t q, int64_t j,
                             int32_t add, void *workspace, int64_t workspace_bytes, hipStream_t stream) {
    if (p < 0 || q < 0 || j < 0) return -CT_EINVAL_SHAPE;
    if (p == 0 || q == 0) return 0;
    if (!out || (j > 0 && (!left || !right))) return -CT_EINVAL_POINTER;
    if (ldo < q || ldl < (trans_l ? p : j) || ldr < (trans_r ? j : q)) return -CT_EINVAL_SHAPE;
    Problem pr{};
    pr.p.seg[0] = Segment{static_cast<const uint16_t *>(left), static_cast<const uint16_t *>(right), ldl, ldr, j};
    pr.p.nseg = 1;
    pr.p.m = p;
    pr.p.n = q;
    pr.a_src = trans_l ? SRC_KS : SRC_KC;
    pr.b_src = trans_r ? SRC_KC : SRC_KS;
    pr.out = CT_F32;
    pr.vec = vec_ok(pr);
    int st = 0;
    hipError_t e = run_reduction(pr, out, ldo, add, workspace, workspace_bytes, stream, &st);
    return st ? st : to_status(e);
}

extern "C" int64_t ct_parameter_gradients_workspace(int64_t m, int64_t n, int64_t k, int64_t r) {
    if (m <= 0 || r <= 0) return 0;
    const int64_t a = k > 0 ? split_workspace_bytes(r, k, m) : 0;
    const int64_t b = n > 0 ? split_workspace_bytes(n, r, m) : 0;
    return a > b ? a : b;  // dA and dB run in sequence on one stream and share the buffer
}

extern "C" int ct_parameter_gradients(const void *x, int64_t ldx, const void *dy, int64_t lddy, const void *low,
                                      const void *xa, float *da, float *db, int64_t m, int64_t n, int64_t k,
                                      int64_t r, int32_t add, void *workspace, int64_t workspace_bytes,
                                      hipStream_t stream) {
    if (m < 0 || n < 0 || k < 0 || r < 0) return -CT_EINVAL_SHAPE;
    if (r == 0) return 0;
    if (!da || !db) return -CT_EINVAL_POINTER;
    // da[r, k] = low^T x : L(p=i, j=row) = low[row*r + i]  -> trans_l; R(j=row, q) = x[row*ldx + q]
    int st = ct_accumulate(da, k, low, r, 1, x, ldx, 0, r, k, m, add, workspace, workspace_bytes, stream);
    if (st) return st;
    // db[n, r] = dy^T xa : L(p=col, j=row) = dy[row*lddy + col] -> trans_l; R(j=row, q) = xa[row*r + q]
    return ct_accumulate(db, r, dy, lddy, 1, xa, r, 0, n, r, m, add, workspace, workspace_bytes, stream);
}
