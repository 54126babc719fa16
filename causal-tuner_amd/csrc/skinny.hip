// Few-row projection GEMMs for gfx950: the small-batch regime of the NF4-LoRA path
// (M in {16, 64}), where streaming the packed weight from HBM
// and decoding it, not MFMA, bound the time.
//
// C[m, n] = sum over one or two reduction segments of A(m, k) B(k, n), m <= 64, A the
// activations (bf16, reduction-contiguous: x, dy, xa, low) and B one of
//   rows    B(k, n) = W[n][k]: packed NF4 rows (forward x w^T) or dense bf16 rows
//           (b in the forward, a in xa = x a^T) -- the "rows" kernel;
//   columns B(k, n) = W[k][n]: packed NF4 used transposed (dx = dy w) or dense bf16
//           (a in dx, b in low = dy b) -- the "columns" kernel.
// Both use v_mfma_f32_16x16x32_bf16 with the activations as the A operand: lane
// (g = lane / 16, c = lane % 16) supplies A rows c and reduction slots 8 g .. 8 g + 7,
// and the B operand for output column c at the same slots. Which reduction index sits
// in which slot is free as long as A and B agree, and each kernel picks the assignment
// that lets a lane load long contiguous runs of the weight:
//
// rows kernel: a step is 128 reduction elements; lane (g, c) holds elements
//   32 g .. 32 g + 31 of weight row c (16 packed bytes = one NF4 block part, or 64 dense
//   bytes), MFMA s (0..3) uses elements 8 s .. 8 s + 7 of them. A workgroup of four
//   waves owns 64 NB weight rows (16 NB per wave); the activation tile of a step is
//   staged once per workgroup in LDS (double buffered, one barrier per step) and the
//   weight is prefetched into registers several steps ahead.
// columns kernel: a step is 32 weight rows; lane (g, c) holds rows 8 g .. 8 g + 7 and
//   the 8 columns 8 c .. 8 c + 7 of each (one packed dword per row, or 16 dense bytes),
//   i.e. an 8 x 8 block already transposed for the MFMA: MFMA t (0..7) takes column
//   8 c + t of its eight rows, so its output column c is weight column 8 c + t. A
//   workgroup owns 128 columns; its four waves split the rows and add their partial
//   sums in LDS in a fixed order. The NF4 block scale of a (row, 64-column span) is
//   decoded by one lane and fetched by the seven others with ds_bpermute.
//
// Longer reductions are split across workgroups (blockIdx.y); the fp32 partials go to
// the caller's workspace and skinny_reduce adds them in split order. Results depend
// only on the shapes, never on the operand kinds, so a packed NF4 weight and the bf16
// weight that `materialize` decodes from it give bit-identical products.

#include <cstdlib>

#include "gemm_common.hpp"

namespace ct {
namespace {

constexpr int kSkThreads = 256;  // four waves
constexpr int kRStep = 128;      // rows kernel: reduction elements per step
constexpr int kTStep = 32;       // columns kernel: weight rows per step
constexpr int kTCols = 128;      // columns kernel: output columns per workgroup

constexpr bool column_src(int s) { return s == SRC_KS || s == SRC_NF4T; }

// Workgroups resident per CU: the waves per SIMD each kernel is compiled for (its
// __launch_bounds__), since a four-wave workgroup puts one wave on each SIMD. The 4-row-
// block rows kernel fits 3 (166 VGPRs with its unordered decode; measured on MI355X at 64
// rows: the 24576-long forward 65 -> 61 us with 8 splits of 96 column blocks).
constexpr int kCUs = 256;
constexpr int rows_per_cu(int) { return 3; }
constexpr int cols_per_cu(int mb) { return mb == 1 ? 3 : (mb == 2 ? 2 : 1); }

// Code book lookup by byte offset (4 x nibble), so the nibble needs no separate shift.
__device__ __forceinline__ float code_at(const float *lcode, uint32_t byte_off) {
    return *reinterpret_cast<const float *>(reinterpret_cast<const char *>(lcode) + byte_off);
}
// 4 x (high nibble) and 4 x (low nibble) of each byte of a packed dword. The values are
// pinned in registers so each lookup offset then costs one byte extract (the compiler
// would otherwise fold the mask into every extract: a shift and an AND per element).
// The columns kernel pins with a volatile statement, which also keeps each dword's decode
// in program order; the rows kernel's decode (decode_dword) pins without it, so the
// compiler may interleave the decodes of a step (measured on MI355X at 64 rows: the
// 6144 x 24576 forward 70 -> 64 us; the columns kernel is 2-7% slower unordered).
__device__ __forceinline__ uint32_t pinned(uint32_t v) {
    asm volatile("" : "+v"(v));
    return v;
}
__device__ __forceinline__ uint32_t pinned_unordered(uint32_t v) {
    asm("" : "+v"(v));
    return v;
}
__device__ __forceinline__ uint32_t hi_offsets(uint32_t d) { return pinned((d >> 2) & 0x3C3C3C3Cu); }
__device__ __forceinline__ uint32_t lo_offsets(uint32_t d) { return pinned((d << 2) & 0x3C3C3C3Cu); }

// Eight elements of one packed dword times s (element 2b from the high nibble of byte b),
// the reference's decoding rule, as bf16 pairs.
__device__ __forceinline__ uint4 decode_dword(uint32_t d, float s, const float *lcode) {
    const uint32_t hi = pinned_unordered((d >> 2) & 0x3C3C3C3Cu), lo = pinned_unordered((d << 2) & 0x3C3C3C3Cu);
    float v[8];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        v[2 * b] = code_at(lcode, (hi >> (8 * b)) & 0xFFu) * s;
        v[2 * b + 1] = code_at(lcode, (lo >> (8 * b)) & 0xFFu) * s;
    }
    return make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                      pack_bf16x2(v[6], v[7]));
}

// Block scale of a nested NF4 state: code2[qa] * absmax2 + offset (two roundings).
__device__ __forceinline__ float nested_scale(uint32_t qa, float a2, float offset, const float *lcode2) {
    return lcode2[qa & 255u] * a2 + offset;
}

struct NF4Rsrc {
    __amdgpu_buffer_rsrc_t q, a, a2;
    int lb, lb2;
    float offset;
    __device__ __forceinline__ void init(const Operand &o, int64_t numel) {
        q = make_rsrc(o.p, (numel + 1) / 2);
        lb = o.lb;
        lb2 = o.lb2;
        const int64_t nb = (numel + (int64_t{1} << lb) - 1) >> lb;
        a = make_rsrc(o.absmax, nb);
        a2 = make_rsrc(o.absmax2, ((nb + (int64_t{1} << lb2) - 1) >> lb2) * 4);
        offset = *o.offset;
    }
};

// ================================================================= rows kernel
// Weight registers of one step: NF4 rows (16 bytes and the block's scale codes per
// column block) or dense rows (64 bytes per column block).
template <int SRC, int NB>
struct RWeight;

template <int NB>
struct RWeight<SRC_NF4, NB> {
    static constexpr int kDepth = 3;  // steps in flight ahead of the one computed
    uint4 q[NB];
    uint32_t qa[NB];
    float a2[NB];
};

template <int NB>
struct RWeight<SRC_KC, NB> {
    static constexpr int kDepth = 1;
    uint4 v[NB][4];
};

// Activations of a step: loaded once per workgroup into LDS (one barrier per step), or
// (direct) each wave loads its own MFMA fragments, 64 bytes of a row per lane and block,
// one step ahead with no barriers. Measured on MI355X with 6144 x 24576 weights, the
// shared tile is faster at every row count: direct loads quadruple the L2 traffic of
// the activations.
template <int MB>
constexpr bool rows_direct() {
    return false;
}

// One segment of the rows kernel over steps [s0, s1) of its reduction. Loads past the
// last step are issued too, pointed out of range (they return zeros): with no branch
// around them the compiler counts outstanding loads exactly and waits only for the
// step being computed. Weight values read past the reduction end (or past the last
// row) are finite and meet zero activations, so only the activation loads check k.
template <int SRC, int MB, int NB>
__device__ __forceinline__ void rows_segment(const Segment &sg, int64_t m, int64_t n, int64_t n0w, int s0, int s1,
                                             f32x4 (&acc)[MB][NB], uint4 *abuf, const float *lcode,
                                             const float *lcode2) {
    constexpr int D = RWeight<SRC, NB>::kDepth;
    constexpr bool kDirect = rows_direct<MB>();
    static_assert((D + 1) % 2 == 0, "the activation ring alternates with the step parity");
    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, c = lane & 15;
    const int nsteps = s1 - s0;
    const int kext = (int)sg.k;
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(sg.a.p, m * sg.a.ld * 2);
    // Direct: lane (g, c) reads row 16 mi + c at k0 + 32 g + 8 s. LDS: thread tid loads
    // unit tid + 256 j of the [16 MB rows][16 chunks] tile, chunk q of row r stored at
    // unit 16 r + (q ^ (r mod 16)) so the fragment reads are conflict-free.
    uint32_t a_off[MB];
    int a_k[MB], a_slot[MB];
#pragma unroll
    for (int j = 0; j < MB; ++j) {
        const int r = kDirect ? 16 * j + c : (tid + kSkThreads * j) >> 4;
        const int q = kDirect ? 4 * g : (tid + kSkThreads * j) & 15;
        a_k[j] = 8 * q;
        a_off[j] = r < m ? (uint32_t)((r * sg.a.ld + 8 * q) * 2) : kOOB;
        a_slot[j] = 16 * r + (q ^ (r & 15));
    }
    // Weight side: row n0w + 16 nj + c, elements 32 g .. 32 g + 31 of each step.
    NF4Rsrc wr;
    __amdgpu_buffer_rsrc_t rb;
    if constexpr (SRC == SRC_NF4) wr.init(sg.b, n * sg.b.ld);
    else rb = make_rsrc(sg.b.p, n * sg.b.ld * 2);
    uint32_t w_el[NB];  // element index of the lane's first weight element at k = 0
#pragma unroll
    for (int nj = 0; nj < NB; ++nj) w_el[nj] = (uint32_t)((n0w + 16 * nj + c) * sg.b.ld + 32 * g);

    RWeight<SRC, NB> w[D + 1];
    uint4 ad[kDirect ? 2 : 1][MB][kDirect ? 4 : 1];  // direct: fragments, two steps in rotation
    uint4 al[kDirect ? 1 : D + 1][MB];               // LDS mode: this thread's share of a tile

    const auto fetch_w = [&](RWeight<SRC, NB> &st, int t) {
        const int k0 = t < nsteps ? (s0 + t) * kRStep : kext;
#pragma unroll
        for (int nj = 0; nj < NB; ++nj) {
            if constexpr (SRC == SRC_NF4) {
                const uint32_t e = w_el[nj] + (uint32_t)k0;
                const uint32_t blk = e >> wr.lb;
                st.q[nj] = buf_load16(wr.q, e >> 1);
                st.qa[nj] = buf_load1(wr.a, blk);
                st.a2[nj] = __builtin_bit_cast(float, buf_load4(wr.a2, (blk >> wr.lb2) * 4));
            } else {
                const uint32_t base = (w_el[nj] + (uint32_t)k0) * 2;
                const int k = k0 + 32 * g;
                // dense rows may hold anything past the reduction end: zeros there
#pragma unroll
                for (int s = 0; s < 4; ++s) st.v[nj][s] = buf_load16(rb, k + 8 * s < kext ? base + 16 * s : kOOB);
            }
        }
    };
    const auto a_at = [&](int j, int k0, int s) {
        return (a_off[j] != kOOB && k0 + a_k[j] + 8 * s < kext) ? a_off[j] + 2 * k0 + 16 * s : kOOB;
    };
    const auto fetch_direct = [&](uint4 (&dst)[MB][kDirect ? 4 : 1], int t) {
        const int k0 = t < nsteps ? (s0 + t) * kRStep : kext;
#pragma unroll
        for (int mi = 0; mi < MB; ++mi)
#pragma unroll
            for (int s = 0; s < (kDirect ? 4 : 1); ++s) dst[mi][s] = buf_load16(ra, a_at(mi, k0, s));
    };
    const auto fetch_share = [&](uint4 (&dst)[MB], int t) {
        const int k0 = t < nsteps ? (s0 + t) * kRStep : kext;
#pragma unroll
        for (int j = 0; j < MB; ++j) dst[j] = buf_load16(ra, a_at(j, k0, 0));
    };
    const auto stage_a = [&](const uint4 (&src)[MB], int t) {
        uint4 *dst = abuf + (t & 1) * (MB * kSkThreads);
#pragma unroll
        for (int j = 0; j < MB; ++j) dst[a_slot[j]] = src[j];
    };
    const auto compute = [&](const RWeight<SRC, NB> &st, const uint4 (&af)[MB][4]) {
#pragma unroll
        for (int nj = 0; nj < NB; ++nj) {
            uint4 b[4];
            if constexpr (SRC == SRC_NF4) {
                const float sc = nested_scale(st.qa[nj], st.a2[nj], wr.offset, lcode2);
                b[0] = decode_dword(st.q[nj].x, sc, lcode);
                b[1] = decode_dword(st.q[nj].y, sc, lcode);
                b[2] = decode_dword(st.q[nj].z, sc, lcode);
                b[3] = decode_dword(st.q[nj].w, sc, lcode);
            } else {
#pragma unroll
                for (int s = 0; s < 4; ++s) b[s] = st.v[nj][s];
            }
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int mi = 0; mi < MB; ++mi) acc[mi][nj] = mfma16x16x32(af[mi][s], b[s], acc[mi][nj]);
        }
    };
    const auto lds_frags = [&](uint4 (&af)[MB][4], int t) {
        const uint4 *src = abuf + (t & 1) * (MB * kSkThreads);
#pragma unroll
        for (int mi = 0; mi < MB; ++mi)
#pragma unroll
            for (int s = 0; s < 4; ++s) af[mi][s] = src[16 * (16 * mi + c) + ((4 * g + s) ^ c)];
    };

    // Ring of D + 1 weight stages; step t lives in stage t mod (D + 1). The loop is
    // unrolled by D + 1 so every stage index is a constant.
    if constexpr (kDirect) {
        fetch_direct(ad[0], 0);
#pragma unroll
        for (int j = 0; j < D; ++j) fetch_w(w[j], j);
        const auto body = [&](int t, int j) {
            fetch_direct(ad[(j + 1) & 1], t + 1);
            fetch_w(w[(j + D) % (D + 1)], t + D);
            compute(w[j], ad[j & 1]);
        };
        // Whole rounds of D + 1 steps, then the rest: no exit inside the main loop, so the
        // compiler's count of outstanding loads carries across iterations.
        int t0 = 0;
        for (; t0 + D + 1 <= nsteps; t0 += D + 1)
#pragma unroll
            for (int j = 0; j <= D; ++j) body(t0 + j, j);
#pragma unroll
        for (int j = 0; j < D; ++j)
            if (t0 + j < nsteps) body(t0 + j, j);
    } else {
        // Step t: fetch step t + D, compute step t from LDS buffer t mod 2, store the
        // activations of step t + 1 into the other buffer (last read in step t - 1,
        // before the previous barrier), barrier.
#pragma unroll
        for (int j = 0; j < D; ++j) {
            fetch_share(al[j], j);
            fetch_w(w[j], j);
        }
        stage_a(al[0], 0);
        __syncthreads();
        const auto body = [&](int t, int j) {
            fetch_share(al[(j + D) % (D + 1)], t + D);
            fetch_w(w[(j + D) % (D + 1)], t + D);
            uint4 af[MB][4];
            lds_frags(af, t);
            compute(w[j], af);
            stage_a(al[(j + 1) % (D + 1)], t + 1);  // zeros after the last step
            __syncthreads();
        };
        int t0 = 0;
        for (; t0 + D + 1 <= nsteps; t0 += D + 1)
#pragma unroll
            for (int j = 0; j <= D; ++j) body(t0 + j, j);
#pragma unroll
        for (int j = 0; j < D; ++j)
            if (t0 + j < nsteps) body(t0 + j, j);  // workgroup-uniform
    }
}

template <int SB0, int SB1, int MB, int NB>
__global__ __launch_bounds__(kSkThreads, rows_per_cu(MB)) void rows_kernel(const GemmParams p) {
    constexpr bool kNF4 = SB0 == SRC_NF4 || SB1 == SRC_NF4;
    __shared__ uint4 abuf[rows_direct<MB>() ? 1 : 2 * MB * kSkThreads];
    __shared__ float lcode[kNF4 ? 16 : 1];
    __shared__ float lcode2[kNF4 ? 256 : 1];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 4, c = lane & 15;
    if constexpr (kNF4) {
        if (tid < 16) lcode[tid] = p.code[tid];
        lcode2[tid] = p.code2[tid];
        __syncthreads();
    }
    const int64_t n0w = (int64_t)blockIdx.x * (64 * NB) + wave * (16 * NB);
    f32x4 acc[MB][NB];
#pragma unroll
    for (int mi = 0; mi < MB; ++mi)
#pragma unroll
        for (int nj = 0; nj < NB; ++nj) acc[mi][nj] = f32x4{0.f, 0.f, 0.f, 0.f};
    // This split's steps of the two segments taken end to end.
    const int st0 = (int)cdiv(p.seg[0].k, kRStep), st1 = p.nseg > 1 ? (int)cdiv(p.seg[1].k, kRStep) : 0;
    const int total = st0 + st1, split = blockIdx.y, splits = gridDim.y;
    const int b = (int)((int64_t)split * total / splits), e = (int)((int64_t)(split + 1) * total / splits);
    // (in LDS mode each segment ends with a barrier, so the second may restage the tile)
    if (b < st0) rows_segment<SB0, MB, NB>(p.seg[0], p.m, p.n, n0w, b, e < st0 ? e : st0, acc, abuf, lcode, lcode2);
    if (e > st0 && st1 > 0)
        rows_segment<SB1, MB, NB>(p.seg[1], p.m, p.n, n0w, (b > st0 ? b : st0) - st0, e - st0, acc, abuf, lcode,
                                  lcode2);

    // Lane (g, c) holds C[16 mi + 4 g + i][n0w + 16 nj + c].
#pragma unroll
    for (int nj = 0; nj < NB; ++nj) {
        const int64_t col = n0w + 16 * nj + c;
        if (col >= p.n) continue;
#pragma unroll
        for (int mi = 0; mi < MB; ++mi)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int64_t row = 16 * mi + 4 * g + i;
                if (row >= p.m) continue;
                float s = acc[mi][nj][i];
                if (splits > 1) {
                    p.split_ws[(int64_t)split * p.split_stride + row * p.n + col] = s;
                    continue;
                }
                if (p.bias) s += bf16_to_f32(p.bias[col]);
                uint16_t *out = static_cast<uint16_t *>(p.c) + row * p.ldc + col;
                if (p.beta) s += bf16_to_f32(*out);
                *out = bf16_bits(s);
            }
    }
}

// ================================================================= columns kernel
template <int SRC, int MB, bool SHARED>
struct TWeight;

// NF4 used transposed: one packed dword (8 columns) per row; the scale codes of one
// (row, column span) per lane with SHARED, of all eight rows without.
template <int MB, bool SHARED>
struct TWeight<SRC_NF4T, MB, SHARED> {
    // 4 row blocks: two stages ahead (156 VGPRs beside the 256 AGPRs of accumulators;
    // measured at 64 rows: dx 67 -> 62 us and 76 -> 71 us on the C5 shapes)
    static constexpr int kDepth = MB == 1 ? 3 : 2;
    static constexpr int kScales = SHARED ? 1 : 8;
    uint32_t d[8];
    uint32_t qa[kScales];
    float a2[kScales];
};

template <int MB, bool SHARED>
struct TWeight<SRC_KS, MB, SHARED> {
    static constexpr int kDepth = 0;  // loaded and used in the same step: few registers
    uint4 v[8];
};

template <int SRC, int MB, bool SHARED>
struct TStage {
    uint4 a[MB];
    TWeight<SRC, MB, SHARED> w;
};

// One segment of the columns kernel: this wave's steps [s0, s1) (32 weight rows each).
template <int SRC, int MB, bool SHARED>
__device__ __forceinline__ void cols_segment(const Segment &sg, int64_t m, int64_t n, int64_t j0, int s0, int s1,
                                             f32x4 (&acc)[MB][8], const float *lcode, const float *lcode2) {
    constexpr int D = TWeight<SRC, MB, SHARED>::kDepth;
    const int lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15;
    const int nsteps = s1 - s0;
    if (nsteps <= 0) return;  // wave-uniform; nothing below synchronises across waves
    const int kext = (int)sg.k;  // weight rows
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(sg.a.p, m * sg.a.ld * 2);
    uint32_t a_off[MB];
#pragma unroll
    for (int mi = 0; mi < MB; ++mi)
        a_off[mi] = 16 * mi + c < m ? (uint32_t)(((16 * mi + c) * sg.a.ld + 8 * g) * 2) : kOOB;
    // Weight side: lane (g, c) reads columns j0 + 8 c .. + 7 of rows i0 + 8 g + e. Rows
    // past the reduction end are out of the buffer range (zeros), columns past n read
    // finite neighbours whose products land in discarded outputs, and the activations of
    // rows past the end are zero, so only the step offset is checked: once per step, on
    // a uniform value.
    const uint32_t ld = (uint32_t)sg.b.ld;
    const uint32_t lane_el = (uint32_t)(8 * g) * ld + (uint32_t)(j0 + 8 * c);
    NF4Rsrc wr;
    __amdgpu_buffer_rsrc_t rb;
    if constexpr (SRC == SRC_NF4T) wr.init(sg.b, (int64_t)kext * sg.b.ld);
    else rb = make_rsrc(sg.b.p, (int64_t)kext * sg.b.ld * 2);
    // With SHARED, lane (g, c) decodes the scale of row 8 g + (c mod 8) over its 64-column
    // span j0 + 64 (c / 8) (one block: blocks start every row and hold >= 64 elements); the
    // eight lanes (c & 8) | e of that span fetch it with ds_bpermute.
    const uint32_t own_el = (uint32_t)(8 * g + (c & 7)) * ld + (uint32_t)(j0 + 64 * (c >> 3));
    const int perm_base = (16 * g + (c & 8)) * 4;  // ds_bpermute byte address of lane (g, c & 8)
    const int64_t col = j0 + 8 * c;

    const auto fetch = [&](TStage<SRC, MB, SHARED> &st, int t) {
        // past the last step: everything out of range (zeros), no branch (see rows_segment)
        const bool live = t < nsteps;
        const int i0 = live ? (s0 + t) * kTStep : kext;
        // element offset of row i0, or one that puts every lane past the buffer end
        const uint32_t row0 = live ? (uint32_t)i0 * ld : 0x40000000u;
#pragma unroll
        for (int mi = 0; mi < MB; ++mi)
            st.a[mi] = buf_load16(ra, (a_off[mi] != kOOB && i0 + 8 * g < kext) ? a_off[mi] + 2 * i0 : kOOB);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t el = lane_el + row0 + (uint32_t)e * ld;
            if constexpr (SRC == SRC_NF4T) {
                st.w.d[e] = buf_load4(wr.q, el >> 1);
                if (!SHARED || e == 0) {
                    const uint32_t blk = (SHARED ? own_el + row0 : el) >> wr.lb;
                    st.w.qa[SHARED ? 0 : e] = buf_load1(wr.a, blk);
                    st.w.a2[SHARED ? 0 : e] = __builtin_bit_cast(float, buf_load4(wr.a2, (blk >> wr.lb2) * 4));
                }
            } else {
                st.w.v[e] = buf_load16(rb, el * 2);
            }
        }
    };
    const auto compute = [&](const TStage<SRC, MB, SHARED> &st, int) {
        const auto mma = [&](int t8, const uint4 &frag) {
#pragma unroll
            for (int mi = 0; mi < MB; ++mi) acc[mi][t8] = mfma16x16x32(st.a[mi], frag, acc[mi][t8]);
        };
        if constexpr (SRC == SRC_NF4T) {
            float sc[8];
            if constexpr (SHARED) {
                const int own = __builtin_bit_cast(int, nested_scale(st.w.qa[0], st.w.a2[0], wr.offset, lcode2));
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    sc[e] = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(perm_base + 4 * e, own));
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) sc[e] = nested_scale(st.w.qa[e], st.w.a2[e], wr.offset, lcode2);
            }
            uint32_t hi[8], lo[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                hi[e] = hi_offsets(st.w.d[e]);
                lo[e] = lo_offsets(st.w.d[e]);
            }
#pragma unroll
            for (int t8 = 0; t8 < 8; ++t8) {
                // column t8 of the lane's 8 columns: element t8 of each row's dword
                float v[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const uint32_t w = (t8 & 1) ? lo[e] : hi[e];
                    v[e] = code_at(lcode, (w >> (8 * (t8 >> 1))) & 0xFFu) * sc[e];
                }
                mma(t8, make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                                   pack_bf16x2(v[6], v[7])));
            }
        } else {
            uint4 frag[8];
            transpose8x8_b16(st.w.v, frag);
#pragma unroll
            for (int t8 = 0; t8 < 8; ++t8) mma(t8, frag[t8]);
        }
    };

    TStage<SRC, MB, SHARED> st[D + 1];
#pragma unroll
    for (int j = 0; j < D; ++j) fetch(st[j], j);
    const auto body = [&](int t, int j) {
        fetch(st[(j + D) % (D + 1)], t + D);
        compute(st[j], t);
    };
    int t0 = 0;  // whole rounds, then the rest (see rows_segment)
    for (; t0 + D + 1 <= nsteps; t0 += D + 1)
#pragma unroll
        for (int j = 0; j <= D; ++j) body(t0 + j, j);
#pragma unroll
    for (int j = 0; j < D; ++j)
        if (t0 + j < nsteps) body(t0 + j, j);
}

template <int SB0, int SB1, int MB, bool SHARED>
__global__ __launch_bounds__(kSkThreads, SHARED ? cols_per_cu(MB) : (MB == 1 ? 2 : cols_per_cu(MB))) void cols_kernel(const GemmParams p) {
    constexpr bool kNF4 = SB0 == SRC_NF4T || SB1 == SRC_NF4T;
    __shared__ __attribute__((aligned(16))) float red[16 * MB * kTCols];
    __shared__ float lcode[kNF4 ? 16 : 1];
    __shared__ float lcode2[kNF4 ? 256 : 1];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 4, c = lane & 15;
    if constexpr (kNF4) {
        if (tid < 16) lcode[tid] = p.code[tid];
        lcode2[tid] = p.code2[tid];
        __syncthreads();
    }
    // Column blocks 2q and 2q + 1 share every 128-byte line of a packed weight row (64
    // bytes each). Workgroups are dealt to the eight XCDs round-robin by their linear id,
    // so when the grid allows, ids x and x + 8 (one XCD) take blocks 2q and 2q + 1 and
    // that XCD's L2 serves the second half of each line instead of a second fetch.
    int bx = blockIdx.x;
    if ((gridDim.x & 15) == 0) bx = (bx & ~15) | ((bx & 7) << 1) | ((bx >> 3) & 1);
    const int64_t j0 = (int64_t)bx * kTCols;
    f32x4 acc[MB][8];
#pragma unroll
    for (int mi = 0; mi < MB; ++mi)
#pragma unroll
        for (int t = 0; t < 8; ++t) acc[mi][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    // The split's steps of both segments end to end, then this wave's quarter of them.
    const int st0 = (int)cdiv(p.seg[0].k, kTStep), st1 = p.nseg > 1 ? (int)cdiv(p.seg[1].k, kTStep) : 0;
    const int total = st0 + st1, split = blockIdx.y, splits = gridDim.y;
    const int b = (int)((int64_t)split * total / splits), e = (int)((int64_t)(split + 1) * total / splits);
    const int wb = b + (e - b) * wave / 4, we = b + (e - b) * (wave + 1) / 4;
    if (wb < st0) cols_segment<SB0, MB, SHARED>(p.seg[0], p.m, p.n, j0, wb, we < st0 ? we : st0, acc, lcode, lcode2);
    if (we > st0 && st1 > 0)
        cols_segment<SB1, MB, SHARED>(p.seg[1], p.m, p.n, j0, (wb > st0 ? wb : st0) - st0, we - st0, acc, lcode,
                                      lcode2);

    // Partial sums of the four waves: ((w3 + w2) + w1) + w0, through one LDS tile.
    // Lane (g, c) holds C[16 mi + 4 g + i][j0 + 8 c + t].
    for (int w = 3; w >= 1; --w) {
        if (wave == w) {
#pragma unroll
            for (int mi = 0; mi < MB; ++mi)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float4 *r = reinterpret_cast<float4 *>(red + (16 * mi + 4 * g + i) * kTCols + 8 * c);
                    float4 lo = make_float4(acc[mi][0][i], acc[mi][1][i], acc[mi][2][i], acc[mi][3][i]);
                    float4 hi = make_float4(acc[mi][4][i], acc[mi][5][i], acc[mi][6][i], acc[mi][7][i]);
                    if (w < 3) {
                        const float4 ol = r[0], oh = r[1];
                        lo = make_float4(ol.x + lo.x, ol.y + lo.y, ol.z + lo.z, ol.w + lo.w);
                        hi = make_float4(oh.x + hi.x, oh.y + hi.y, oh.z + hi.z, oh.w + hi.w);
                    }
                    r[0] = lo;
                    r[1] = hi;
                }
        }
        __syncthreads();
    }
    if (wave != 0) return;
    const int64_t col = j0 + 8 * c;
    if (col >= p.n) return;
#pragma unroll
    for (int mi = 0; mi < MB; ++mi)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int64_t row = 16 * mi + 4 * g + i;
            if (row >= p.m) continue;
            const float *r = red + (16 * mi + 4 * g + i) * kTCols + 8 * c;
            float s[8];
#pragma unroll
            for (int t = 0; t < 8; ++t) s[t] = r[t] + acc[mi][t][i];
            if (splits > 1) {
                float4 *dst = reinterpret_cast<float4 *>(p.split_ws + (int64_t)split * p.split_stride + row * p.n + col);
                dst[0] = make_float4(s[0], s[1], s[2], s[3]);
                dst[1] = make_float4(s[4], s[5], s[6], s[7]);
                continue;
            }
            uint16_t *out = static_cast<uint16_t *>(p.c) + row * p.ldc + col;
            uint32_t packed[4];
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                float lo = s[2 * h], hi = s[2 * h + 1];
                if (p.bias) {
                    lo += bf16_to_f32(p.bias[col + 2 * h]);
                    hi += bf16_to_f32(p.bias[col + 2 * h + 1]);
                }
                if (p.beta) {
                    lo += bf16_to_f32(out[2 * h]);
                    hi += bf16_to_f32(out[2 * h + 1]);
                }
                packed[h] = (uint32_t)bf16_bits(lo) | ((uint32_t)bf16_bits(hi) << 16);
            }
            if ((p.ldc & 7) == 0 && (reinterpret_cast<uintptr_t>(p.c) & 15) == 0)
                *reinterpret_cast<uint4 *>(out) = make_uint4(packed[0], packed[1], packed[2], packed[3]);
            else
#pragma unroll
                for (int h = 0; h < 4; ++h) {
                    out[2 * h] = (uint16_t)packed[h];
                    out[2 * h + 1] = (uint16_t)(packed[h] >> 16);
                }
        }
}

// Sum of the split partials in split order, then bias and beta, rounded once to bf16.
// Grid: (column blocks of 256, rows).
__global__ __launch_bounds__(256) void skinny_reduce(const GemmParams p, int splits) {
    const int64_t col = (int64_t)blockIdx.x * 256 + threadIdx.x, row = blockIdx.y;
    if (col >= p.n) return;
    const int64_t i = row * p.n + col;
    // Eight partials in flight at a time (written by other XCDs, they come from memory),
    // added in split order.
    float s = 0.f;
    for (int z0 = 0; z0 < splits; z0 += 8) {
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = z0 + j < splits ? p.split_ws[(z0 + j) * p.split_stride + i] : 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (z0 + j < splits) s = (z0 + j == 0) ? v[j] : s + v[j];
    }
    if (p.bias) s += bf16_to_f32(p.bias[col]);
    uint16_t *out = static_cast<uint16_t *>(p.c) + row * p.ldc + col;
    if (p.beta) s += bf16_to_f32(*out);
    *out = bf16_bits(s);
}

// ================================================================= host side
// Launch shape: column blocks per wave (rows kernel) and reduction splits. Only the
// shapes decide it, so every operand kind of one problem gets the same summation order.
struct SkShape {
    int mb, nb, splits;
};

SkShape sk_shape(const GemmParams &p, bool columns, int64_t ws_floats) {
    SkShape sh{};
    sh.mb = p.m <= 16 ? 1 : (p.m <= 32 ? 2 : 4);
    int64_t steps = 0, groups, target, min_steps;
    const int step = columns ? kTStep : kRStep;
    for (int s = 0; s < p.nseg; ++s) steps += cdiv(p.seg[s].k, step);
    if (columns) {
        sh.nb = 1;
        target = (int64_t)cols_per_cu(sh.mb) * kCUs;
        groups = cdiv(p.n, kTCols);
        min_steps = 4 * 4;  // four per wave
    } else {
        target = (int64_t)rows_per_cu(sh.mb) * kCUs;
        // two column blocks per wave when that still leaves a full round of workgroups
        sh.nb = sh.mb <= 2 && cdiv(p.n, 128) >= target ? 2 : 1;
        groups = cdiv(p.n, 64 * sh.nb);
        min_steps = 4;
    }
    // At most enough splits to fill the resident slots once when the columns alone do not
    // fill the GPU; below that, the count that spreads the work most evenly over the CUs:
    // the busiest CU holds ceil(s * groups / CUs) workgroups of 1/s of the reduction each,
    // so a count just past a whole round costs a second round (measured on MI355X at 64
    // rows: the 6144-wide dx 102.7 -> 65.5 us with 5 splits instead of 6, the 24576-long
    // forward 83.2 -> 67.3 us with 5 instead of 6; at 16 rows the counts are unchanged).
    int64_t limit = groups >= target ? 1 : cdiv(target, groups);
    const int64_t cap = steps / min_steps > 1 ? steps / min_steps : 1;
    if (limit > cap) limit = cap;
    if (limit > 64) limit = 64;
    int64_t splits = 1, busiest = cdiv(groups, kCUs);  // busiest CU's load x splits
    for (int64_t s = 2; s <= limit; ++s) {
        const int64_t load = cdiv(s * groups, kCUs);
        if (load * splits < busiest * s) {  // load / s < busiest / splits
            splits = s;
            busiest = load;
        }
    }
    if (splits > 1 && ws_floats >= 0 && splits * p.m * p.n > ws_floats) splits = 1;
    sh.splits = (int)splits;
    return sh;
}

template <int SB0, int SB1, int MB, int NB>
hipError_t launch_rows(const GemmParams &p, int splits, hipStream_t stream) {
    const dim3 grid((unsigned)cdiv(p.n, 64 * NB), (unsigned)splits);
    rows_kernel<SB0, SB1, MB, NB><<<grid, dim3(kSkThreads), 0, stream>>>(p);
    return hipGetLastError();
}

template <int SB0, int SB1, int MB, bool SHARED>
hipError_t launch_cols(const GemmParams &p, int splits, hipStream_t stream) {
    const dim3 grid((unsigned)cdiv(p.n, kTCols), (unsigned)splits);
    cols_kernel<SB0, SB1, MB, SHARED><<<grid, dim3(kSkThreads), 0, stream>>>(p);
    return hipGetLastError();
}

template <int SB0, int SB1, int MB>
hipError_t launch_rows_nb(const GemmParams &p, const SkShape &sh, hipStream_t stream) {
    if constexpr (MB <= 2) {
        if (sh.nb >= 2) return launch_rows<SB0, SB1, MB, 2>(p, sh.splits, stream);
    }
    return launch_rows<SB0, SB1, MB, 1>(p, sh.splits, stream);
}

template <int SB0, int SB1>
hipError_t launch_rows_mb(const GemmParams &p, const SkShape &sh, hipStream_t stream) {
    if (sh.mb == 1) return launch_rows_nb<SB0, SB1, 1>(p, sh, stream);
    if (sh.mb == 2) return launch_rows_nb<SB0, SB1, 2>(p, sh, stream);
    return launch_rows_nb<SB0, SB1, 4>(p, sh, stream);
}

template <int SB0, int SB1, bool SHARED>
hipError_t launch_cols_mb(const GemmParams &p, const SkShape &sh, hipStream_t stream) {
    if (sh.mb == 1) return launch_cols<SB0, SB1, 1, SHARED>(p, sh.splits, stream);
    if (sh.mb == 2) return launch_cols<SB0, SB1, 2, SHARED>(p, sh.splits, stream);
    return launch_cols<SB0, SB1, 4, SHARED>(p, sh.splits, stream);
}

bool aligned16(const void *q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; }

// A packed weight whose block scales the columns kernel may share across eight lanes:
// blocks of at least 64 elements that start every row (a 64-column span aligned to 64
// then lies inside one block).
bool scales_shared(const Operand &o) { return o.lb >= 6 && o.ld % (int64_t{1} << o.lb) == 0; }

}  // namespace

bool skinny_supported(const GemmParams &p, const int src_a[2], const int src_b[2], int out_dtype) {
    if (out_dtype != CT_BF16 || p.m < 1 || p.m > 64 || p.n < 1) return false;
    constexpr int64_t kLimit = int64_t{1} << 31;
    const bool columns = column_src(src_b[0]);
    for (int s = 0; s < p.nseg; ++s) {
        const Segment &g = p.seg[s];
        if (column_src(src_b[s]) != columns) return false;
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
                // 16-byte row loads: 32 elements inside one first-level block
                if (!g.b.nested || g.b.ld % 32 || g.b.lb < 5 || p.n * g.b.ld >= kLimit) return false;
                break;
            case SRC_NF4T:
                // 4-byte row loads: 8 columns inside one first-level block
                if (!g.b.nested || g.b.ld % 8 || g.b.lb < 3 || p.n % 8 || g.k * g.b.ld >= kLimit) return false;
                break;
            default:
                return false;
        }
    }
    return true;
}

int64_t skinny_workspace_bytes(const GemmParams &p, const int src_b[2]) {
    const SkShape sh = sk_shape(p, column_src(src_b[0]), -1);
    return sh.splits > 1 ? (int64_t)sh.splits * p.m * p.n * 4 : 0;
}

hipError_t skinny_run(GemmParams p, const int src_b[2], void *ws, int64_t ws_bytes, hipStream_t stream) {
    const int b0 = src_b[0], b1 = p.nseg > 1 ? src_b[1] : src_b[0];
    const bool columns = column_src(b0);
    // The partials are written with 16-byte stores: a misaligned workspace counts as none
    // (no split), as the many-row paths treat it.
    const SkShape sh = sk_shape(p, columns, (ws && aligned16(ws)) ? ws_bytes / 4 : 0);
    p.split_ws = static_cast<float *>(ws);
    p.split_stride = p.m * p.n;
    hipError_t e = hipErrorNotSupported;
    if (b0 == SRC_NF4 && b1 == SRC_KC) e = launch_rows_mb<SRC_NF4, SRC_KC>(p, sh, stream);
    else if (b0 == SRC_KC && b1 == SRC_KC) e = launch_rows_mb<SRC_KC, SRC_KC>(p, sh, stream);
    else if (b0 == SRC_NF4T && b1 == SRC_KS) {
        e = scales_shared(p.seg[0].b) ? launch_cols_mb<SRC_NF4T, SRC_KS, true>(p, sh, stream)
                                       : launch_cols_mb<SRC_NF4T, SRC_KS, false>(p, sh, stream);
    } else if (b0 == SRC_KS && b1 == SRC_KS)
        e = launch_cols_mb<SRC_KS, SRC_KS, true>(p, sh, stream);
    if (e != hipSuccess || sh.splits == 1) return e;
    skinny_reduce<<<dim3((unsigned)cdiv(p.n, 256), (unsigned)p.m), dim3(256), 0, stream>>>(p, sh.splits);
    return hipGetLastError();
}

}  // namespace ct
