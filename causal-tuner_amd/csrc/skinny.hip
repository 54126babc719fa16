// Few-row projection GEMMs for gfx950: the small-batch regime of the NF4-LoRA path
// (M in {16, 64, 256}), where streaming the packed weight from
// HBM, not MFMA, bounds the time.
//
// C[m, n] = sum over one or two reduction segments of A(m, k) B(k, n), m <= 64, A the
// activations (bf16, reduction-contiguous: x, dy, xa, low) and B any operand source:
// packed NF4 rows (forward), packed NF4 used transposed (dx), dense bf16 rows (b in the
// forward, a in xa = x a^T), dense bf16 transposed (a in dx, b in low = dy b).
//
// Work split: a workgroup of 8 waves owns 16*NB output columns and all m rows; the 8
// waves split the reduction into contiguous ranges of 128-element k-blocks, so every
// wave streams its own slice of the weight with several loads in flight. Inside a wave,
// v_mfma_f32_16x16x32_bf16 does the reduction across lanes; the 8 partial [m, 16*NB]
// sums meet in LDS and are added in wave order 0..7 (deterministic).
//
// Fragment order: in a k-block, lane (g = lane / 16, c = lane % 16) owns reduction
// elements kb + 32 g + [0, 32); MFMA step s (0..3) uses elements 8 s .. 8 s + 7 of them.
// A and B follow the same order, so their products pair up, and each lane reads 64
// contiguous bytes of an activation row or 16 contiguous bytes of a packed NF4 row with
// one load per 16 bytes. Transposed sources (reduction along memory rows) are decoded or
// transposed through a wave-private LDS tile [16*NB columns][128 + 8] (the padding
// spreads columns over banks); no workgroup barrier is needed for them.

#include <cstdlib>

#include "gemm_common.hpp"

namespace ct {
namespace {

constexpr int kSkWaves = 8;
constexpr int kSkThreads = 64 * kSkWaves;
constexpr int kKB = 128;             // reduction elements per k-block
constexpr int kPitch = kKB + 8;      // bf16 elements per column of a transposed tile

constexpr bool transposed_src(int s) { return s == SRC_KS || s == SRC_NF4T; }

// Loads of one k-block of one segment, held in registers between issue and use.
template <int SRC, int MB, int NB>
struct SkStage;

// Activations: MB row blocks of 16, four 16-byte loads (64 contiguous bytes) per lane each.
template <int MB>
struct SkA {
    uint4 f[MB][4];
    __device__ __forceinline__ void load(const __amdgpu_buffer_rsrc_t &r, int64_t ld, int kext, int kb, int g,
                                         int c) {
        const int k = kb * kKB + 32 * g;
#pragma unroll
        for (int mi = 0; mi < MB; ++mi) {
            const uint32_t base = (uint32_t)(((16 * mi + c) * ld + k) * 2);
#pragma unroll
            for (int s = 0; s < 4; ++s) f[mi][s] = buf_load16(r, k + 8 * s < kext ? base + 16 * s : kOOB);
        }
    }
};

// Dense rows (reduction-contiguous): like the activations, one column per lane.
template <int MB, int NB>
struct SkStage<SRC_KC, MB, NB> {
    uint4 f[NB][4];
    __amdgpu_buffer_rsrc_t r;
    int64_t ld;
    int64_t n0;
    int kext;
    __device__ __forceinline__ void init(const Operand &o, int64_t n, int64_t n0_, int64_t kext_) {
        r = make_rsrc(o.p, n * o.ld * 2);
        ld = o.ld;
        n0 = n0_;
        kext = (int)kext_;
    }
    __device__ __forceinline__ void load(int kb, int g, int c, int) {
        const int k = kb * kKB + 32 * g;
#pragma unroll
        for (int nj = 0; nj < NB; ++nj) {
            const uint32_t base = (uint32_t)(((n0 + 16 * nj + c) * ld + k) * 2);
#pragma unroll
            for (int s = 0; s < 4; ++s) f[nj][s] = buf_load16(r, k + 8 * s < kext ? base + 16 * s : kOOB);
        }
    }
    __device__ __forceinline__ void frags(uint4 (&b)[NB][4], char *, const float *, const float *, float, int,
                                          int) const {
#pragma unroll
        for (int nj = 0; nj < NB; ++nj)
#pragma unroll
            for (int s = 0; s < 4; ++s) b[nj][s] = f[nj][s];
    }
};

// Packed NF4 rows (forward): 16 bytes = 32 elements of one block per lane and column block.
template <int MB, int NB>
struct SkStage<SRC_NF4, MB, NB> {
    uint4 q[NB];
    uint32_t qa[NB];
    float a2[NB];
    bool ok[NB];
    __amdgpu_buffer_rsrc_t rq, ra, r2;
    int64_t n, n0;
    uint32_t ld;
    int kext, lb, lb2;
    __device__ __forceinline__ void init(const Operand &o, int64_t n_, int64_t n0_, int64_t kext_) {
        n = n_;
        n0 = n0_;
        ld = (uint32_t)o.ld;
        kext = (int)kext_;
        lb = o.lb;
        lb2 = o.lb2;
        const int64_t numel = n * o.ld;
        rq = make_rsrc(o.p, (numel + 1) / 2);
        const int64_t nb = (numel + (int64_t{1} << lb) - 1) >> lb;
        ra = make_rsrc(o.absmax, nb);
        r2 = make_rsrc(o.absmax2, ((nb + (int64_t{1} << lb2) - 1) >> lb2) * 4);
    }
    __device__ __forceinline__ void load(int kb, int g, int c, int) {
        const int k = kb * kKB + 32 * g;
#pragma unroll
        for (int nj = 0; nj < NB; ++nj) {
            const int64_t col = n0 + 16 * nj + c;
            ok[nj] = col < n && k < kext;
            const uint32_t e = (uint32_t)(col * ld + k);
            const uint32_t gb = e >> lb;
            q[nj] = buf_load16(rq, ok[nj] ? e >> 1 : kOOB);
            qa[nj] = buf_load1(ra, ok[nj] ? gb : kOOB);
            a2[nj] = __builtin_bit_cast(float, buf_load4(r2, ok[nj] ? (gb >> lb2) * 4 : kOOB));
        }
    }
    __device__ __forceinline__ void frags(uint4 (&b)[NB][4], char *, const float *lcode, const float *lcode2,
                                          float offset, int, int) const {
#pragma unroll
        for (int nj = 0; nj < NB; ++nj) {
            const float decoded = lcode2[qa[nj] & 255u] * a2[nj] + offset;  // read unconditionally: no branch
            const float s = ok[nj] ? decoded : 0.f;
            b[nj][0] = nf4_decode8(q[nj].x, s, lcode);
            b[nj][1] = nf4_decode8(q[nj].y, s, lcode);
            b[nj][2] = nf4_decode8(q[nj].z, s, lcode);
            b[nj][3] = nf4_decode8(q[nj].w, s, lcode);
        }
    }
};

// Units of 8 reduction rows x 8 columns for the transposed sources: the tile has 16 row
// groups x 2*NB column groups; each lane takes kUnits of them (lanes repeat units when
// there are fewer units than lanes).
template <int NB>
struct SkUnits {
    static constexpr int kCount = 16 * 2 * NB;
    static constexpr int kPer = (kCount + 63) / 64;
    __device__ __forceinline__ static void unit(int lane, int t, int &rg, int &cg) {
        // column groups fastest: one load instruction covers 64 / (2 NB) rows x 16 NB bytes
        const int u = (lane + 64 * t) % kCount;
        cg = u % (2 * NB);
        rg = u / (2 * NB);
    }
};

__device__ __forceinline__ void store_column(char *tile, int col, int row, uint4 v) {
    *reinterpret_cast<uint4 *>(tile + (col * kPitch + row) * 2) = v;
}

__device__ __forceinline__ uint4 read_column(const char *tile, int col, int row) {
    return *reinterpret_cast<const uint4 *>(tile + (col * kPitch + row) * 2);
}

template <int NB>
__device__ __forceinline__ void tile_frags(uint4 (&b)[NB][4], const char *tile, int g, int c) {
#pragma unroll
    for (int nj = 0; nj < NB; ++nj)
#pragma unroll
        for (int s = 0; s < 4; ++s) b[nj][s] = read_column(tile, 16 * nj + c, 32 * g + 8 * s);
}

// Dense bf16, reduction along memory rows: 8 rows x 16 bytes per unit, transposed in
// registers into 8 column chunks.
template <int MB, int NB>
struct SkStage<SRC_KS, MB, NB> {
    using U = SkUnits<NB>;
    uint4 v[U::kPer][8];
    __amdgpu_buffer_rsrc_t r;
    int64_t ld, n, n0;
    int kext;
    __device__ __forceinline__ void init(const Operand &o, int64_t n_, int64_t n0_, int64_t kext_) {
        ld = o.ld;
        n = n_;
        n0 = n0_;
        kext = (int)kext_;
        r = make_rsrc(o.p, kext_ > 0 ? ((kext_ - 1) * o.ld + n_) * 2 : 0);
    }
    __device__ __forceinline__ void load(int kb, int, int, int lane) {
#pragma unroll
        for (int t = 0; t < U::kPer; ++t) {
            int rg, cg;
            U::unit(lane, t, rg, cg);
            const int64_t col = n0 + 8 * cg;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int row = kb * kKB + 8 * rg + i;
                v[t][i] = buf_load16(r, (row < kext && col < n) ? (uint32_t)((row * ld + col) * 2) : kOOB);
            }
        }
    }
    __device__ __forceinline__ void frags(uint4 (&b)[NB][4], char *tile, const float *, const float *, float,
                                          int g, int c) const {
        const int lane = 16 * g + c;
#pragma unroll
        for (int t = 0; t < U::kPer; ++t) {
            int rg, cg;
            U::unit(lane, t, rg, cg);
            uint4 tr[8];
            transpose8x8_b16(v[t], tr);
#pragma unroll
            for (int j = 0; j < 8; ++j) store_column(tile, 8 * cg + j, 8 * rg, tr[j]);
        }
        __builtin_amdgcn_wave_barrier();  // one wave's LDS operations complete in order
        tile_frags<NB>(b, tile, g, c);
    }
};

// Packed NF4 used transposed (dx = dy w): units of 8 weight rows x 16 weight columns (one
// 8-byte load and one block scale per row), 16 row groups x NB column groups per tile,
// column groups fastest across lanes.
template <int NB>
struct SkUnitsT {
    static constexpr int kCount = 16 * NB;
    static constexpr int kPer = (kCount + 63) / 64;
    __device__ __forceinline__ static void unit(int lane, int t, int &rg, int &cg) {
        const int u = (lane + 64 * t) % kCount;
        cg = u % NB;
        rg = u / NB;
    }
};

template <int MB, int NB>
struct SkStage<SRC_NF4T, MB, NB> {
    using U = SkUnitsT<NB>;
    uint2 d[U::kPer][8];
    uint32_t qa[U::kPer][8];
    float a2[U::kPer][8];
    bool ok[U::kPer][8];
    __amdgpu_buffer_rsrc_t rq, ra, r2;
    int64_t n, n0;
    uint32_t ld;
    int kext, lb, lb2;
    __device__ __forceinline__ void init(const Operand &o, int64_t n_, int64_t n0_, int64_t kext_) {
        n = n_;
        n0 = n0_;
        ld = (uint32_t)o.ld;
        kext = (int)kext_;
        lb = o.lb;
        lb2 = o.lb2;
        const int64_t numel = kext_ * o.ld;  // weight rows x weight columns
        rq = make_rsrc(o.p, (numel + 1) / 2);
        const int64_t nb = (numel + (int64_t{1} << lb) - 1) >> lb;
        ra = make_rsrc(o.absmax, nb);
        r2 = make_rsrc(o.absmax2, ((nb + (int64_t{1} << lb2) - 1) >> lb2) * 4);
    }
    __device__ __forceinline__ void load(int kb, int, int, int lane) {
#pragma unroll
        for (int t = 0; t < U::kPer; ++t) {
            int rg, cg;
            U::unit(lane, t, rg, cg);
            const int64_t col = n0 + 16 * cg;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int row = kb * kKB + 8 * rg + i;
                ok[t][i] = row < kext && col < n;
                const uint32_t e = (uint32_t)(row * (int64_t)ld + col);
                const uint32_t gb = e >> lb;
                const uint32_t off = ok[t][i] ? e >> 1 : kOOB;
                d[t][i] = make_uint2(buf_load4(rq, off), buf_load4(rq, off + 4));
                qa[t][i] = buf_load1(ra, ok[t][i] ? gb : kOOB);
                a2[t][i] = __builtin_bit_cast(float, buf_load4(r2, ok[t][i] ? (gb >> lb2) * 4 : kOOB));
            }
        }
    }
    __device__ __forceinline__ void frags(uint4 (&b)[NB][4], char *tile, const float *lcode, const float *lcode2,
                                          float offset, int g, int c) const {
        const int lane = 16 * g + c;
#pragma unroll
        for (int t = 0; t < U::kPer; ++t) {
            int rg, cg;
            U::unit(lane, t, rg, cg);
            float s[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float decoded = lcode2[qa[t][i] & 255u] * a2[t][i] + offset;
                s[i] = ok[t][i] ? decoded : 0.f;
            }
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                // column j of the unit: element j of each row's 8 bytes (high nibble first)
                const int shift = (j & 1) ? 8 * ((j >> 1) & 3) : 8 * ((j >> 1) & 3) + 4;
                float v[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) v[i] = lcode[(((j < 8) ? d[t][i].x : d[t][i].y) >> shift) & 15u] * s[i];
                store_column(tile, 16 * cg + j, 8 * rg,
                             make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                                        pack_bf16x2(v[6], v[7])));
            }
        }
        __builtin_amdgcn_wave_barrier();
        tile_frags<NB>(b, tile, g, c);
    }
};

// k-blocks in flight while one is computed: two for the row-streaming sources with few
// rows (their register stages are small and HBM latency dominates), one otherwise.
template <int SB, int MB, int NB>
constexpr int sk_depth() {
    return (!transposed_src(SB) && MB * NB <= 2) ? 2 : 1;
}

// One segment: this wave's contiguous range of k-blocks, loads one or two blocks ahead.
template <int SB, int MB, int NB>
__device__ __forceinline__ void sk_segment(const Segment &sg, int64_t m, int64_t n, int64_t n0, int wave, int lane,
                                           f32x4 (&acc)[MB][NB], char *tile, const float *lcode,
                                           const float *lcode2) {
    // This workgroup's share of the k-blocks (split `blockIdx.y` of `gridDim.y`), then this
    // wave's contiguous part of it.
    const int nkb = (int)cdiv(sg.k, kKB);
    const int split = blockIdx.y, splits = gridDim.y;
    const int s0 = split * nkb / splits, s1 = (split + 1) * nkb / splits;
    const int kb0 = s0 + wave * (s1 - s0) / kSkWaves, kb1 = s0 + (wave + 1) * (s1 - s0) / kSkWaves;
    if (kb0 >= kb1) return;  // wave-uniform; nothing below synchronises across waves
    const int g = lane >> 4, c = lane & 15;
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(sg.a.p, m * sg.a.ld * 2);
    const float offset = is_nf4_src(SB) ? *sg.b.offset : 0.f;
    SkStage<SB, MB, NB> st;
    st.init(sg.b, n, n0, sg.k);
    const auto compute = [&](const SkA<MB> &a, const SkStage<SB, MB, NB> &stage) {
        uint4 b[NB][4];
        stage.frags(b, tile, lcode, lcode2, offset, g, c);
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int mi = 0; mi < MB; ++mi)
#pragma unroll
                for (int nj = 0; nj < NB; ++nj) acc[mi][nj] = mfma16x16x32(a.f[mi][s], b[nj][s], acc[mi][nj]);
    };
    const auto fetch = [&](SkA<MB> &a, SkStage<SB, MB, NB> &stage, int kb) {
        if (kb < kb1) {  // wave-uniform
            a.load(ra, sg.a.ld, (int)sg.k, kb, g, c);
            stage.load(kb, g, c, lane);
        }
    };
    if constexpr (sk_depth<SB, MB, NB>() == 2) {
        // Two k-blocks in flight: three register stages in rotation, the loop unrolled by
        // three so every stage keeps its registers.
        SkA<MB> a0, a1, a2;
        SkStage<SB, MB, NB> s0 = st, s1 = st, s2 = st;
        fetch(a0, s0, kb0);
        fetch(a1, s1, kb0 + 1);
        for (int kb = kb0; kb < kb1; kb += 3) {
            fetch(a2, s2, kb + 2);
            compute(a0, s0);
            if (kb + 1 >= kb1) break;
            fetch(a0, s0, kb + 3);
            compute(a1, s1);
            if (kb + 2 >= kb1) break;
            fetch(a1, s1, kb + 4);
            compute(a2, s2);
        }
    } else {
        SkA<MB> a;
        a.load(ra, sg.a.ld, (int)sg.k, kb0, g, c);
        st.load(kb0, g, c, lane);
        for (int kb = kb0; kb < kb1; ++kb) {
            SkA<MB> an = a;
            SkStage<SB, MB, NB> sn = st;
            fetch(an, sn, kb + 1);
            compute(a, st);
            a = an;
            st = sn;
        }
    }
}

template <int SB0, int SB1, int MB, int NB>
__global__ __launch_bounds__(kSkThreads) void skinny_kernel(const GemmParams p) {
    constexpr int kCols = 16 * NB, kRows = 16 * MB;
    constexpr bool kTransposed = transposed_src(SB0) || transposed_src(SB1);
    constexpr bool kNF4 = is_nf4_src(SB0) || is_nf4_src(SB1);
    constexpr int kTileBytes = kTransposed ? kCols * kPitch * 2 : 0;
    constexpr int kPartBytes = kRows * kCols * 4;
    constexpr int kWaveBytes = kTileBytes > kPartBytes ? kTileBytes : kPartBytes;
    __shared__ __attribute__((aligned(16))) char smem[kSkWaves * kWaveBytes];
    __shared__ float lcode[kNF4 ? 16 : 1];
    __shared__ float lcode2[kNF4 ? 256 : 1];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t n0 = (int64_t)blockIdx.x * kCols;
    if constexpr (kNF4) {
        if (tid < 16) lcode[tid] = p.code[tid];
        if (p.code2 && tid < 256) lcode2[tid] = p.code2[tid];
        __syncthreads();
    }
    f32x4 acc[MB][NB];
#pragma unroll
    for (int mi = 0; mi < MB; ++mi)
#pragma unroll
        for (int nj = 0; nj < NB; ++nj) acc[mi][nj] = f32x4{0.f, 0.f, 0.f, 0.f};

    char *mine = smem + wave * kWaveBytes;
    sk_segment<SB0, MB, NB>(p.seg[0], p.m, p.n, n0, wave, lane, acc, mine, lcode, lcode2);
    if (p.nseg > 1) sk_segment<SB1, MB, NB>(p.seg[1], p.m, p.n, n0, wave, lane, acc, mine, lcode, lcode2);

    // Partial sums of the 8 waves meet in LDS (reusing the tiles) and add in wave order.
    __syncthreads();
    float *part = reinterpret_cast<float *>(mine);
    const int g = lane >> 4, c = lane & 15;
#pragma unroll
    for (int mi = 0; mi < MB; ++mi)
#pragma unroll
        for (int nj = 0; nj < NB; ++nj)
#pragma unroll
            for (int i = 0; i < 4; ++i) part[(16 * mi + 4 * g + i) * kCols + 16 * nj + c] = acc[mi][nj][i];
    __syncthreads();
    for (int e = tid; e < kRows * kCols; e += kSkThreads) {
        const int row = e / kCols, col = e % kCols;
        const int64_t gc = n0 + col;
        if (row >= p.m || gc >= p.n) continue;
        float s = 0.f;
#pragma unroll
        for (int w = 0; w < kSkWaves; ++w) s += reinterpret_cast<const float *>(smem + w * kWaveBytes)[e];
        if (gridDim.y > 1) {
            // split partial: fp32 [split][m][n] in the caller's workspace (p.split_ws)
            p.split_ws[(int64_t)blockIdx.y * p.split_stride + row * p.n + gc] = s;
            continue;
        }
        if (p.bias) s += bf16_to_f32(p.bias[gc]);
        uint16_t *out = static_cast<uint16_t *>(p.c) + row * p.ldc + gc;
        if (p.beta) s += bf16_to_f32(*out);
        *out = bf16_bits(s);
    }
}

// Sum of the split partials in split order, then bias and beta, rounded once to bf16.
__global__ __launch_bounds__(256) void skinny_reduce(const GemmParams p, int splits) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= p.m * p.n) return;
    const int64_t row = i / p.n, col = i % p.n;
    float s = p.split_ws[i];
    for (int z = 1; z < splits; ++z) s += p.split_ws[z * p.split_stride + i];
    if (p.bias) s += bf16_to_f32(p.bias[col]);
    uint16_t *out = static_cast<uint16_t *>(p.c) + row * p.ldc + col;
    if (p.beta) s += bf16_to_f32(*out);
    *out = bf16_bits(s);
}

// Shape of a few-row launch: columns per workgroup (16 NB) and reduction splits.
struct SkShape {
    int nb, splits;
};

SkShape sk_shape(const GemmParams &p, bool transposed, int64_t ws_floats) {
    const int mb = p.m <= 16 ? 1 : (p.m <= 32 ? 2 : 4);
    // Transposed sources keep all 64 lanes busy only with 64-column tiles; the others take
    // the widest tile that still leaves ~128 workgroups before splitting the reduction.
    int nb;
    if (transposed) nb = mb <= 2 ? 4 : 2;
    else nb = (mb <= 2 && cdiv(p.n, 64) >= 128) ? 4 : (cdiv(p.n, 32) >= 128 ? 2 : 1);
#ifdef CT_TUNING
    if (const char *env = getenv(transposed ? "CT_SKNB_T" : "CT_SKNB")) nb = atoi(env);
#endif
    const int64_t wgs = cdiv(p.n, 16 * nb);
    int64_t nkb = 0;
    for (int s = 0; s < p.nseg; ++s) nkb = nkb > cdiv(p.seg[s].k, kKB) ? nkb : cdiv(p.seg[s].k, kKB);
    // About one 8-wave workgroup per CU; each wave keeps >= 4 k-blocks (>= 1 when the output
    // is too narrow to fill the GPU otherwise), so per-workgroup set-up stays amortised.
    int64_t splits = cdiv(256, wgs);
    const int64_t per_wave = wgs >= 64 ? 4 : 1;
    int64_t cap = nkb / (kSkWaves * per_wave);
    if (cap < 1) cap = 1;
    if (splits > cap) splits = cap;
    if (splits > 64) splits = 64;
    if (splits < 1) splits = 1;
    if (splits > 1 && ws_floats >= 0 && splits * p.m * p.n > ws_floats) splits = 1;
    return SkShape{nb, (int)splits};
}

template <int SB0, int SB1, int MB, int NB>
hipError_t launch_shape(const GemmParams &p, int splits, hipStream_t stream) {
    const dim3 grid((unsigned)cdiv(p.n, 16 * NB), (unsigned)splits);
    skinny_kernel<SB0, SB1, MB, NB><<<grid, dim3(kSkThreads), 0, stream>>>(p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || splits == 1) return e;
    skinny_reduce<<<dim3((unsigned)cdiv(p.m * p.n, 256)), dim3(256), 0, stream>>>(p, splits);
    return hipGetLastError();
}

template <int SB0, int SB1, int MB>
hipError_t launch_nb(const GemmParams &p, const SkShape &sh, hipStream_t stream) {
    if constexpr (MB <= 2) {
        if (sh.nb == 4) return launch_shape<SB0, SB1, MB, 4>(p, sh.splits, stream);
    }
    if (sh.nb == 2) return launch_shape<SB0, SB1, MB, 2>(p, sh.splits, stream);
    return launch_shape<SB0, SB1, MB, 1>(p, sh.splits, stream);
}

template <int SB0, int SB1>
hipError_t launch_mb(const GemmParams &p, const SkShape &sh, hipStream_t stream) {
    if (p.m <= 16) return launch_nb<SB0, SB1, 1>(p, sh, stream);
    if (p.m <= 32) return launch_nb<SB0, SB1, 2>(p, sh, stream);
    return launch_nb<SB0, SB1, 4>(p, sh, stream);
}

bool aligned16(const void *q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; }

}  // namespace

bool skinny_supported(const GemmParams &p, const int src_a[2], const int src_b[2], int out_dtype) {
    if (out_dtype != CT_BF16 || p.m < 1 || p.m > 64 || p.n < 1) return false;
    constexpr int64_t kLimit = int64_t{1} << 31;
    for (int s = 0; s < p.nseg; ++s) {
        const Segment &g = p.seg[s];
        if (src_a[s] != SRC_KC || !aligned16(g.a.p) || g.a.ld % 8 || g.k % 8) return false;
        if (p.m * g.a.ld * 2 >= kLimit) return false;
        switch (src_b[s]) {
            case SRC_KC:
                if (!aligned16(g.b.p) || g.b.ld % 8 || p.n * g.b.ld * 2 >= kLimit) return false;
                break;
            case SRC_KS:
                if (!aligned16(g.b.p) || g.b.ld % 8 || p.n % 8 || g.k * g.b.ld * 2 >= kLimit) return false;
                break;
            case SRC_NF4:
                if (!g.b.nested || g.b.ld % 32 || g.b.lb < 5 || p.n * g.b.ld >= kLimit) return false;
                break;
            case SRC_NF4T:
                // 8-byte row loads: 16 columns per unit, inside one first-level block
                if (!g.b.nested || g.b.ld % 16 || g.b.lb < 4 || p.n % 16 || g.k * g.b.ld >= kLimit) return false;
                break;
            default:
                return false;
        }
    }
    return true;
}

int64_t skinny_workspace_bytes(const GemmParams &p, const int src_b[2]) {
    const bool transposed = transposed_src(src_b[0]) || (p.nseg > 1 && transposed_src(src_b[1]));
    const SkShape sh = sk_shape(p, transposed, -1);
    return sh.splits > 1 ? (int64_t)sh.splits * p.m * p.n * 4 : 0;
}

hipError_t skinny_run(GemmParams p, const int src_b[2], void *ws, int64_t ws_bytes, hipStream_t stream) {
    const int b0 = src_b[0], b1 = p.nseg > 1 ? src_b[1] : src_b[0];
    const bool transposed = transposed_src(b0) || transposed_src(b1);
    const SkShape sh = sk_shape(p, transposed, ws ? ws_bytes / 4 : 0);
    p.split_ws = static_cast<float *>(ws);
    p.split_stride = p.m * p.n;
    if (b0 == SRC_NF4 && b1 == SRC_KC) return launch_mb<SRC_NF4, SRC_KC>(p, sh, stream);
    if (b0 == SRC_NF4T && b1 == SRC_KS) return launch_mb<SRC_NF4T, SRC_KS>(p, sh, stream);
    if (b0 == SRC_KC && b1 == SRC_KC) return launch_mb<SRC_KC, SRC_KC>(p, sh, stream);
    if (b0 == SRC_KS && b1 == SRC_KS) return launch_mb<SRC_KS, SRC_KS>(p, sh, stream);
    return hipErrorNotSupported;
}

}  // namespace ct
