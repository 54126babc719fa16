// bf16 MFMA GEMMs for the NF4-LoRA projection path on gfx950.
//
// One kernel template serves every contraction of the reference's operator layer
// (kernels/linear.py:27-44): C[m,n] = sum over one or two reduction segments of
// A(m,k) B(k,n), fp32 accumulation in v_mfma_f32_16x16x32_bf16, and a fused epilogue
// (bias, beta accumulation, bf16 or fp32 output, or fp32 split partials).
//
// Two segments carry the rank-r LoRA terms as extra reduction columns:
//   forward  out = [x | xa] [w | b]^T      (segment 0: k columns, segment 1: r columns)
//   backward dx  = [dy | low] [w ; a]      (segment 0: n rows,    segment 1: r rows)
// so the low-rank term costs no extra pass over the output.
//
// Operand sources (how a k-tile reaches LDS):
//   KC    bf16, reduction dimension contiguous: 16-byte chunks copied as they are;
//   KS    bf16, output dimension contiguous: 8x8 blocks transposed in registers (v_perm);
//   NF4   packed NF4 weight [rows, cols] used with its columns as the reduction
//         dimension (forward: x w^T): 16 packed bytes per lane decode into 32 bf16;
//   NF4T  the same weight used with its rows as the reduction dimension (dx = dy w):
//         8 rows x 8 columns per lane, decoded straight into the transposed layout.
// NF4 decoding follows the reference's rule exactly (kernels/nf4_cuda.py:16-29): the
// block scale is code2[q] * absmax2 + offset (fp32 multiply, separately rounded add), the
// value is code[nibble] * scale in fp32, rounded once to bf16; so a fused contraction sees
// bit-for-bit the weight that the standalone decoder materialises.
//
// LDS holds each k-tile as [rows][64] bf16 (reduction contiguous) in 16-byte chunks whose
// position in the 128-byte row is XORed with a row-dependent swizzle, so the MFMA fragment
// reads (ds_read_b128) and the loader writes are free of bank conflicts. Tiles are double
// buffered: the next tile's global loads are in flight while the current one feeds MFMA.
//
// Tile shapes: 256x256 (gemm_big8: 8 waves of 64x128, two per SIMD; the generic runner's
// gemm_big: 4 waves of 128x128), 128x128 and 64x64 (4 waves).
// Workgroup ids are remapped so each of the 8 XCDs walks a contiguous, M-grouped range of
// output tiles: the workgroups that share an L2 also share A and B panels.

#include <cstdlib>

#include "gemm_common.hpp"
#include "profile.hpp"

namespace ct {

int validate_nf4(const ct_nf4_weight *w);
bool nf4_transposable(const ct_nf4_weight *w);
hipError_t nf4_dequant_transposed(const ct_nf4_weight *w, void *out, hipStream_t stream, int64_t ldo = 0);

namespace {

constexpr int kBK = 64;        // reduction columns per k-tile (8 chunks of 8 bf16)
constexpr int kThreads = 256;  // 4 wavefronts per workgroup
constexpr int kXcds = 8;       // MI355X dispatches workgroups round-robin over 8 XCDs
constexpr int kGroupM = 4;     // m-tiles per group in the L2-friendly tile order (4: measured best of 2-32)


// ------------------------------------------------------------------ operand tile loaders
// ROWS: output-dimension extent of the tile. FRAG: output columns per lane of the MFMA
// fragments that read the tile (1 for the A side, FN for the B side); tile row n is
// stored at LDS row frag_row<FRAG>(n).
// load() issues the global reads of k-tile k0 into registers; store() writes the tile to
// LDS (decoding NF4 on the way).
template <int SRC, int ROWS, bool VEC, int FRAG>
struct Loader;

template <int ROWS, bool VEC, int FRAG>
struct Loader<SRC_KC, ROWS, VEC, FRAG> {
    static constexpr int kPer = (ROWS * 8 + kThreads - 1) / kThreads;
    uint4 r[kPer];
    __device__ __forceinline__ void load(const Operand &o, int64_t rows, int64_t kext, int64_t r0, int64_t k0,
                                         int tid) {
        const uint16_t *p = static_cast<const uint16_t *>(o.p);
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int id = tid + i * kThreads;
            if (id >= ROWS * 8) break;
            const int64_t row = r0 + (id >> 3);
            const int64_t k = k0 + (id & 7) * 8;
            if constexpr (VEC) {
                r[i] = (row < rows && k < kext) ? *reinterpret_cast<const uint4 *>(p + row * o.ld + k) : zero4();
            } else {
                uint16_t e[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) e[j] = (row < rows && k + j < kext) ? p[row * o.ld + k + j] : uint16_t(0);
                r[i] = __builtin_bit_cast(uint4, e);
            }
        }
    }
    __device__ __forceinline__ void store(uint4 *lds, int tid, const float *, const float *) const {
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int id = tid + i * kThreads;
            if (id >= ROWS * 8) break;
            lds[slot(frag_row<FRAG>(id >> 3), id & 7)] = r[i];
        }
    }
};

template <int ROWS, bool VEC, int FRAG>
struct Loader<SRC_KS, ROWS, VEC, FRAG> {
    // ROWS/8 row blocks x 8 k-chunks = ROWS blocks of 8x8, at most one per lane.
    uint4 r[8];
    __device__ __forceinline__ void load(const Operand &o, int64_t rows, int64_t kext, int64_t r0, int64_t k0,
                                         int tid) {
        if (tid >= ROWS) return;
        const uint16_t *p = static_cast<const uint16_t *>(o.p);
        const int64_t row = r0 + (tid % (ROWS / 8)) * 8;
        const int64_t kb = k0 + (tid / (ROWS / 8)) * 8;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int64_t k = kb + i;
            if constexpr (VEC) {
                r[i] = (k < kext && row < rows) ? *reinterpret_cast<const uint4 *>(p + k * o.ld + row) : zero4();
            } else {
                uint16_t e[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) e[j] = (k < kext && row + j < rows) ? p[k * o.ld + row + j] : uint16_t(0);
                r[i] = __builtin_bit_cast(uint4, e);
            }
        }
    }
    __device__ __forceinline__ void store(uint4 *lds, int tid, const float *, const float *) const {
        if (tid >= ROWS) return;
        uint4 t[8];
        transpose8x8_b16(r, t);
        const int row = (tid % (ROWS / 8)) * 8;
        const int chunk = tid / (ROWS / 8);
#pragma unroll
        for (int j = 0; j < 8; ++j) lds[slot(frag_row<FRAG>(row + j), chunk)] = t[j];
    }
};

// NF4 weight [rows][cols], reduction along cols (forward: x w^T). One unit = 32 elements
// of one row: 16 packed bytes inside one first-level block (blocksize >= 32, cols % 32 == 0).
// load() fetches the packed bytes and the block's scale code; store() decodes.
template <int ROWS, bool VEC, int FRAG>
struct Loader<SRC_NF4, ROWS, VEC, FRAG> {
    static constexpr int kUnits = ROWS * 2;
    static constexpr int kPer = (kUnits + kThreads - 1) / kThreads;
    uint4 q[kPer];
    float a2[kPer];     // nested: absmax2 of the block's group; plain: the block scale
    uint32_t qa[kPer];  // nested: the block's u8 scale code; 256 marks an empty unit
    __device__ __forceinline__ void load(const Operand &o, int64_t rows, int64_t kext, int64_t r0, int64_t k0,
                                         int tid) {
        const uint8_t *packed = static_cast<const uint8_t *>(o.p);
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int id = tid + i * kThreads;
            if (id >= kUnits) break;
            const int64_t row = r0 + (id >> 1);
            const int64_t k = k0 + (id & 1) * 32;
            if (row < rows && k < kext) {
                const int64_t e = row * o.ld + k;
                const int64_t g = e >> o.lb;
                q[i] = *reinterpret_cast<const uint4 *>(packed + (e >> 1));
                if (o.nested) {
                    qa[i] = static_cast<const uint8_t *>(o.absmax)[g];
                    a2[i] = o.absmax2[g >> o.lb2];
                } else {
                    qa[i] = 0;
                    a2[i] = static_cast<const float *>(o.absmax)[g];
                }
            } else {
                q[i] = zero4();
                qa[i] = 256;
                a2[i] = 0.f;
            }
        }
    }
    __device__ __forceinline__ void store(uint4 *lds, int tid, const float *lcode, const float *lcode2,
                                          int nested, float offset) const {
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int id = tid + i * kThreads;
            if (id >= kUnits) break;
            float s = a2[i];
            if (nested) s = qa[i] < 256 ? lcode2[qa[i]] * a2[i] + offset : 0.f;
            const int row = id >> 1, c0 = (id & 1) * 4;
            lds[slot(frag_row<FRAG>(row), c0 + 0)] = nf4_decode8(q[i].x, s, lcode);
            lds[slot(frag_row<FRAG>(row), c0 + 1)] = nf4_decode8(q[i].y, s, lcode);
            lds[slot(frag_row<FRAG>(row), c0 + 2)] = nf4_decode8(q[i].z, s, lcode);
            lds[slot(frag_row<FRAG>(row), c0 + 3)] = nf4_decode8(q[i].w, s, lcode);
        }
    }
};

// NF4 weight [rows][cols], reduction along rows (the transposed use in dx = dy w). One
// unit = 8 weight rows x 8 weight columns (one packed dword per row), at most one per lane;
// the decoded values are written straight into the reduction-contiguous LDS layout.
template <int ROWS, bool VEC, int FRAG>
struct Loader<SRC_NF4T, ROWS, VEC, FRAG> {
    static constexpr int kCB = ROWS / 8;  // 8-column blocks across the tile
    uint32_t d[8];
    float a2[8];
    uint32_t qa[8];
    __device__ __forceinline__ void load(const Operand &o, int64_t rows, int64_t kext, int64_t r0, int64_t k0,
                                         int tid) {
        if (tid >= 8 * kCB) return;
        const uint8_t *packed = static_cast<const uint8_t *>(o.p);
        const int64_t col = r0 + (tid % kCB) * 8;
        const int64_t wrow0 = k0 + (tid / kCB) * 8;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int64_t wrow = wrow0 + i;
            if (wrow < kext && col < rows) {
                const int64_t e = wrow * o.ld + col;
                const int64_t g = e >> o.lb;
                d[i] = *reinterpret_cast<const uint32_t *>(packed + (e >> 1));
                if (o.nested) {
                    qa[i] = static_cast<const uint8_t *>(o.absmax)[g];
                    a2[i] = o.absmax2[g >> o.lb2];
                } else {
                    qa[i] = 0;
                    a2[i] = static_cast<const float *>(o.absmax)[g];
                }
            } else {
                d[i] = 0;
                qa[i] = 256;
                a2[i] = 0.f;
            }
        }
    }
    __device__ __forceinline__ void store(uint4 *lds, int tid, const float *lcode, const float *lcode2,
                                          int nested, float offset) const {
        if (tid >= 8 * kCB) return;
        float s[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            s[i] = a2[i];
            if (nested) s[i] = qa[i] < 256 ? lcode2[qa[i]] * a2[i] + offset : 0.f;
        }
        const int col = (tid % kCB) * 8;
        const int chunk = tid / kCB;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            // column j of the 8x8 unit: element j of each row's dword (high nibble first)
            const int shift = (j & 1) ? 8 * (j >> 1) : 8 * (j >> 1) + 4;
            float v[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = lcode[(d[i] >> shift) & 15u] * s[i];
            lds[slot(frag_row<FRAG>(col + j), chunk)] = make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]),
                                                            pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7]));
        }
    }
};

// Dense loaders ignore the NF4 tables.
template <int SRC>
constexpr bool is_nf4() { return SRC == SRC_NF4 || SRC == SRC_NF4T; }

template <class L, int SRC>
__device__ __forceinline__ void store_tile(const L &l, uint4 *lds, int tid, const float *lcode,
                                           const float *lcode2, int nested, float offset) {
    if constexpr (is_nf4<SRC>()) l.store(lds, tid, lcode, lcode2, nested, offset);
    else l.store(lds, tid, lcode, lcode2);
}

// ------------------------------------------------------------------ one reduction segment
template <int BM, int BN, int SA, int SB, bool VEC>
struct SegmentRunner {
    static constexpr int WM = BM / 2, WN = BN / 2;  // 2 x 2 waves
    static constexpr int FM = WM / 16, FN = WN / 16;

    __device__ __forceinline__ static void run(const Segment &sg, int64_t m, int64_t n, int64_t m0, int64_t n0,
                                               int64_t tbeg, int64_t tend, f32x4 (&acc)[FM][FN], uint4 *lds0,
                                               uint4 *lds1, const float *lcode, const float *lcode2, int tid,
                                               int wm0, int wn0) {
        if (tbeg >= tend) return;
        const int lane = tid & 63;
        Loader<SA, BM, VEC, 1> la;
        Loader<SB, BN, VEC, FN> lb;
        const float off_a = (is_nf4<SA>() && sg.a.nested) ? *sg.a.offset : 0.f;
        const float off_b = (is_nf4<SB>() && sg.b.nested) ? *sg.b.offset : 0.f;
        la.load(sg.a, m, sg.k, m0, tbeg * kBK, tid);
        lb.load(sg.b, n, sg.k, n0, tbeg * kBK, tid);
        __syncthreads();  // every wave is done with the buffers of a previous segment
        store_tile<decltype(la), SA>(la, lds0, tid, lcode, lcode2, sg.a.nested, off_a);
        store_tile<decltype(lb), SB>(lb, lds0 + BM * 8, tid, lcode, lcode2, sg.b.nested, off_b);
        __syncthreads();
        for (int64_t t = tbeg; t < tend; ++t) {
            const int buf = (int)((t - tbeg) & 1);
            const bool more = t + 1 < tend;
            if (more) {
                la.load(sg.a, m, sg.k, m0, (t + 1) * kBK, tid);
                lb.load(sg.b, n, sg.k, n0, (t + 1) * kBK, tid);
            }
            const uint4 *sa = buf ? lds1 : lds0;
            const uint4 *sb = sa + BM * 8;
#pragma unroll
            for (int ks = 0; ks < kBK / 32; ++ks) {
                const int chunk = ks * 4 + (lane >> 4);
                uint4 af[FM], bf[FN];
#pragma unroll
                for (int i = 0; i < FM; ++i) af[i] = sa[slot(wm0 + i * 16 + (lane & 15), chunk)];
#pragma unroll
                for (int j = 0; j < FN; ++j) bf[j] = sb[slot(wn0 + j * 16 + (lane & 15), chunk)];
#pragma unroll
                for (int i = 0; i < FM; ++i)
#pragma unroll
                    for (int j = 0; j < FN; ++j) acc[i][j] = mfma16x16x32(af[i], bf[j], acc[i][j]);
            }
            __builtin_amdgcn_sched_barrier(0);  // keep the next tile's stores after the MFMA block
            if (more) {
                uint4 *next = buf ? lds0 : lds1;
                store_tile<decltype(la), SA>(la, next, tid, lcode, lcode2, sg.a.nested, off_a);
                store_tile<decltype(lb), SB>(lb, next + BM * 8, tid, lcode, lcode2, sg.b.nested, off_b);
            }
            __syncthreads();
        }
    }
};

// ------------------------------------------------------------------ fast segment runner
// Used when every dense operand is 16-byte aligned with 8-element leading dimensions and
// every operand spans less than 2 GiB (32-bit buffer offsets). All global reads are raw
// buffer loads: the hardware range check returns zeros past num_records, and an invalid
// lane is pointed past the range, so the k-loop body has no branches and the compiler can
// interleave loads, LDS traffic, NF4 decoding and MFMA within one basic block.
template <int SRC, int ROWS, int FRAG, int THREADS>
struct Fast;

// KC: each wave instruction moves 64 x 16 bytes = 8 tile rows x 8 chunks; lane l owns slot
// base + l (row l/8, physical chunk l%8), so it fetches the global chunk that the swizzle
// maps to that physical position. The chunk goes global -> VGPR -> ds_write: measured on
// MI355X at M=8192 this beat loading straight into LDS (buffer_load ... lds) by 5-20%, as
// the LDS form needs an M0 write per wave instruction and must complete before the barrier
// that publishes the stage, while register staging lets the loads run across it.
template <int ROWS, int FRAG, int THREADS>
struct Fast<SRC_KC, ROWS, FRAG, THREADS> {
    static constexpr int kWaves = THREADS / 64;
    static constexpr int kInstr = ROWS / (8 * kWaves);
    static constexpr int kVmem = kInstr, kWrites = kInstr;  // per tile, per lane
    static_assert(kInstr >= 1, "tile too small for the workgroup");
    __amdgpu_buffer_rsrc_t r;
    uint32_t off[kInstr];  // byte offset of the lane's chunk at k0 = 0
    int kc[kInstr];        // the lane's first reduction column within the tile
    int kext;              // reduction extent (< 2^31: fast_ok bounds every operand)
    int wave;
    __device__ __forceinline__ void init(const Operand &o, int64_t rows, int64_t kext_, int64_t r0, int tid) {
        const uint16_t *p = static_cast<const uint16_t *>(o.p) + r0 * o.ld;
        const int64_t live = rows - r0 < ROWS ? rows - r0 : ROWS;
        r = make_rsrc(p, live * o.ld * 2);
        kext = (int)kext_;
        wave = tid >> 6;
        const int lane = tid & 63;
#pragma unroll
        for (int i = 0; i < kInstr; ++i) {
            int srow, c;
            slot_coords((wave * kInstr + i) * 64 + lane, srow, c);
            const int row = frag_row_inv<FRAG>(srow);
            kc[i] = c * 8;
            off[i] = (uint32_t)((row * o.ld + c * 8) * 2);
        }
    }
    uint4 v[kInstr];
    __device__ __forceinline__ void issue(uint4 *, int64_t k0) {
#pragma unroll
        for (int i = 0; i < kInstr; ++i) {
            const uint32_t o = ((int)k0 + kc[i] < kext) ? off[i] + (uint32_t)(k0 * 2) : kOOB;
            v[i] = buf_load16(r, o);
        }
    }
    __device__ __forceinline__ void commit(uint4 *stage, const float *, const float *, float) const {
        const int lane = threadIdx.x & 63;
#pragma unroll
        for (int i = 0; i < kInstr; ++i) stage[(wave * kInstr + i) * 64 + lane] = v[i];
    }
};

// Store R bf16 values (R/2 dwords) at byte offset `byte` of the stage.
template <int R>
__device__ __forceinline__ void store_part(uint4 *stage, int byte, const uint32_t (&w)[R / 2]) {
    char *b = reinterpret_cast<char *>(stage) + byte;
    if constexpr (R == 8) *reinterpret_cast<uint4 *>(b) = make_uint4(w[0], w[1], w[2], w[3]);
    else if constexpr (R == 4) *reinterpret_cast<uint2 *>(b) = make_uint2(w[0], w[1]);
    else *reinterpret_cast<uint32_t *>(b) = w[0];
}

// KS: 8x8 blocks (8 reduction rows x 8 output rows), split over LPB lanes that take
// R = 8 / LPB reduction rows each; transposed in registers, R values per LDS write.
// Adjacent lanes take the parts of one block, the next lanes its neighbours along the
// reduction (the 8 chunks of one LDS row), then the next 8 output rows: each store
// instruction then fills whole 256-byte lines instead of piling 16 lanes onto the same
// banks (rows 8 apart share a swizzle position).
template <int ROWS, int FRAG, int THREADS>
struct Fast<SRC_KS, ROWS, FRAG, THREADS> {
    static constexpr int kLPB = THREADS / ROWS;
    static constexpr int R = 8 / kLPB;
    static constexpr int kVmem = R, kWrites = 8;
    static_assert(kLPB >= 1 && kLPB <= 4, "unsupported tile / workgroup ratio");
    __amdgpu_buffer_rsrc_t r;
    uint32_t off0, pitch;
    int col, chunk, h;
    bool valid;
    uint4 v[R];
    __device__ __forceinline__ void init(const Operand &o, int64_t rows, int64_t kext, int64_t r0, int tid) {
        const int b = tid / kLPB;
        h = tid % kLPB;
        col = (b >> 3) * 8;
        chunk = b & 7;
        const uint16_t *p = static_cast<const uint16_t *>(o.p) + r0;
        r = make_rsrc(p, kext > 0 ? ((kext - 1) * o.ld + (rows - r0)) * 2 : 0);
        valid = r0 + col < rows;
        pitch = (uint32_t)(o.ld * 2);
        off0 = (uint32_t)(((chunk * 8 + h * R) * o.ld + col) * 2);
    }
    __device__ __forceinline__ void issue(uint4 *, int64_t k0) {
        const uint32_t base = off0 + (uint32_t)(k0 * pitch);
#pragma unroll
        for (int i = 0; i < R; ++i) v[i] = buf_load16(r, valid ? base + i * pitch : kOOB);
    }
    __device__ __forceinline__ void commit(uint4 *stage, const float *, const float *, float) const {
        const uint32_t *d = reinterpret_cast<const uint32_t *>(v);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            uint32_t w[R / 2];
#pragma unroll
            for (int q = 0; q < R / 2; ++q) w[q] = pick16(d[(2 * q + 1) * 4 + (j >> 1)], d[(2 * q) * 4 + (j >> 1)], j & 1);
            store_part<R>(stage, slot(frag_row<FRAG>(col + j), chunk) * 16 + h * R * 2, w);
        }
    }
};

// KT: 16-byte chunks of the operand's reduction rows, stored as loaded (k-major, swizzled
// segments); consecutive lanes take consecutive chunks of one row, and a lane's chunks sit
// in rows k, k + RS, k + 2 RS, ... (RS = rows per pass), which share one swizzle, so their
// global and LDS addresses differ by constants.
template <int ROWS, int FRAG, int THREADS>
struct Fast<SRC_KT, ROWS, FRAG, THREADS> {
    static constexpr int kRowChunks = ROWS / 8;
    static constexpr int kPer = 64 * kRowChunks / THREADS;
    static constexpr int kRowStep = THREADS / kRowChunks;  // rows covered by one pass of the lanes
    static constexpr int kVmem = kPer, kWrites = kPer;
    static_assert(kPer * THREADS == 64 * kRowChunks && THREADS % kRowChunks == 0 && kRowStep % 16 == 0 &&
                      ROWS >= 128, "unsupported KT tile");
    __amdgpu_buffer_rsrc_t r;
    uint32_t off0, pitch;
    int k_first, byte0, kext;
    bool ok;
    uint4 v[kPer];
    __device__ __forceinline__ void init(const Operand &o, int64_t rows, int64_t kext_, int64_t r0, int tid) {
        const uint16_t *p = static_cast<const uint16_t *>(o.p) + r0;
        r = make_rsrc(p, kext_ > 0 ? ((kext_ - 1) * o.ld + (rows - r0)) * 2 : 0);
        kext = (int)kext_;
        pitch = (uint32_t)(o.ld * 2);
        const int cc = tid % kRowChunks;
        k_first = tid / kRowChunks;
        ok = r0 + 8 * cc < rows;
        off0 = (uint32_t)(k_first * o.ld + 8 * cc) * 2;
        byte0 = kt_byte<ROWS>(k_first, 8 * cc);
    }
    __device__ __forceinline__ void issue(uint4 *, int64_t k0) {
        const uint32_t base = off0 + (uint32_t)k0 * pitch;
#pragma unroll
        for (int i = 0; i < kPer; ++i)
            v[i] = buf_load16(r, (ok && (int)k0 + k_first + i * kRowStep < kext) ? base + i * kRowStep * pitch : kOOB);
    }
    __device__ __forceinline__ void commit(uint4 *stage, const float *, const float *, float) const {
        char *b = reinterpret_cast<char *>(stage) + byte0;
#pragma unroll
        for (int i = 0; i < kPer; ++i) *reinterpret_cast<uint4 *>(b + i * kRowStep * (ROWS * 2)) = v[i];
    }
};

// NF4 (nested), reduction along the weight's columns: units of 32 elements of one row.
template <int ROWS, int FRAG, int THREADS>
struct Fast<SRC_NF4, ROWS, FRAG, THREADS> {
    static constexpr int kUnits = ROWS * 2;
    static constexpr int kPer = (kUnits + THREADS - 1) / THREADS;
    static constexpr int kVmem = 3 * kPer, kWrites = 4 * kPer;
    __amdgpu_buffer_rsrc_t rq, ra, r2;
    uint32_t e0[kPer];  // element index of the unit at k0 = 0 (whole weight)
    int row[kPer], half[kPer];
    int kext;
    int lb, lb2;
    uint4 q[kPer];
    uint32_t qa[kPer];
    float a2[kPer];
    bool ok[kPer];
    __device__ __forceinline__ void init(const Operand &o, int64_t rows, int64_t kext_, int64_t r0, int tid) {
        kext = (int)kext_;
        lb = o.lb;
        lb2 = o.lb2;
        const int64_t n = rows * o.ld;
        rq = make_rsrc(o.p, (n + 1) / 2);
        const int64_t nb = (n + (int64_t{1} << lb) - 1) >> lb;
        ra = make_rsrc(o.absmax, nb);
        r2 = make_rsrc(o.absmax2, ((nb + (int64_t{1} << lb2) - 1) >> lb2) * 4);
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int u = (tid + i * THREADS) % kUnits;
            row[i] = u >> 1;
            half[i] = u & 1;
            const int64_t gr = r0 + row[i];
            e0[i] = gr < rows ? (uint32_t)(gr * o.ld + half[i] * 32) : 0xffffffffu;
        }
    }
    __device__ __forceinline__ void issue(uint4 *, int64_t k0) {
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            ok[i] = e0[i] != 0xffffffffu && (int)k0 + half[i] * 32 < kext;
            const uint32_t e = e0[i] + (uint32_t)k0;
            const uint32_t g = e >> lb;
            q[i] = buf_load16(rq, ok[i] ? e >> 1 : kOOB);
            qa[i] = buf_load1(ra, ok[i] ? g : kOOB);
            a2[i] = __builtin_bit_cast(float, buf_load4(r2, ok[i] ? (g >> lb2) * 4 : kOOB));
        }
    }
    __device__ __forceinline__ void commit(uint4 *stage, const float *lcode, const float *lcode2,
                                           float offset) const {
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const float decoded = lcode2[qa[i] & 255u] * a2[i] + offset;  // read unconditionally: no branch
            const float s = ok[i] ? decoded : 0.f;
            const int c0 = half[i] * 4;
            stage[slot(frag_row<FRAG>(row[i]), c0 + 0)] = nf4_decode8(q[i].x, s, lcode);
            stage[slot(frag_row<FRAG>(row[i]), c0 + 1)] = nf4_decode8(q[i].y, s, lcode);
            stage[slot(frag_row<FRAG>(row[i]), c0 + 2)] = nf4_decode8(q[i].z, s, lcode);
            stage[slot(frag_row<FRAG>(row[i]), c0 + 3)] = nf4_decode8(q[i].w, s, lcode);
        }
    }
};

// NF4 (nested), reduction along the weight's rows: units of 8 weight rows x 8 columns,
// split over LPB lanes that take R = 8 / LPB weight rows each.
template <int ROWS, int FRAG, int THREADS>
struct Fast<SRC_NF4T, ROWS, FRAG, THREADS> {
    static constexpr int kLPB = THREADS / ROWS;
    static constexpr int R = 8 / kLPB;
    static constexpr int kVmem = 3 * R, kWrites = 8;
    static_assert(kLPB >= 1 && kLPB <= 4, "unsupported tile / workgroup ratio");
    __amdgpu_buffer_rsrc_t rq, ra, r2;
    uint32_t e0;  // element index of (weight row chunk*8 + h*R, column r0 + col) at k0 = 0
    uint32_t ld;
    int col, chunk, h, row0;
    bool colok;
    int kext;
    int lb, lb2;
    uint32_t d[R], qa[R];
    float a2[R];
    bool ok[R];
    __device__ __forceinline__ void init(const Operand &o, int64_t rows, int64_t kext_, int64_t r0, int tid) {
        kext = (int)kext_;
        lb = o.lb;
        lb2 = o.lb2;
        const int64_t n = kext_ * o.ld;  // weight rows x weight columns
        rq = make_rsrc(o.p, (n + 1) / 2);
        const int64_t nb = (n + (int64_t{1} << lb) - 1) >> lb;
        ra = make_rsrc(o.absmax, nb);
        r2 = make_rsrc(o.absmax2, ((nb + (int64_t{1} << lb2) - 1) >> lb2) * 4);
        const int b = tid / kLPB;  // lane order as in the KS loader
        h = tid % kLPB;
        col = (b >> 3) * 8;
        chunk = b & 7;
        row0 = chunk * 8 + h * R;
        colok = r0 + col < rows;
        ld = (uint32_t)o.ld;
        e0 = (uint32_t)(row0 * o.ld + r0 + col);
    }
    __device__ __forceinline__ void issue(uint4 *, int64_t k0) {
#pragma unroll
        for (int i = 0; i < R; ++i) {
            ok[i] = colok && (int)k0 + row0 + i < kext;
            const uint32_t e = e0 + (uint32_t)(k0 + i) * ld;
            const uint32_t g = e >> lb;
            d[i] = buf_load4(rq, ok[i] ? e >> 1 : kOOB);
            qa[i] = buf_load1(ra, ok[i] ? g : kOOB);
            a2[i] = __builtin_bit_cast(float, buf_load4(r2, ok[i] ? (g >> lb2) * 4 : kOOB));
        }
    }
    __device__ __forceinline__ void commit(uint4 *stage, const float *lcode, const float *lcode2,
                                           float offset) const {
        float s[R];
#pragma unroll
        for (int i = 0; i < R; ++i) {
            const float decoded = lcode2[qa[i] & 255u] * a2[i] + offset;  // read unconditionally: no branch
            s[i] = ok[i] ? decoded : 0.f;
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int shift = (j & 1) ? 8 * (j >> 1) : 8 * (j >> 1) + 4;
            uint32_t w[R / 2];
#pragma unroll
            for (int q = 0; q < R / 2; ++q)
                w[q] = pack_bf16x2(lcode[(d[2 * q] >> shift) & 15u] * s[2 * q],
                                   lcode[(d[2 * q + 1] >> shift) & 15u] * s[2 * q + 1]);
            store_part<R>(stage, slot(frag_row<FRAG>(col + j), chunk) * 16 + h * R * 2, w);
        }
    }
};

#ifndef CT_PV
#define CT_PV 2
#endif
// Instruction-group order for one k-step of FastRunner (LLVM's sched_group_barrier masks:
// 0x8 MFMA, 0x20 VMEM read, 0x100 DS read, 0x200 DS write). The A fragments and the first
// column's B fragments are read first; after that every column's MFMAs carry the next
// column's B reads and a share of the stage writes and global loads for later tiles.
template <int FM, int FN, int KS, class LA, class LB>
struct SchedPattern {
    static constexpr int kW = LA::kWrites + LB::kWrites, kV = LA::kVmem + LB::kVmem;
    static constexpr int kWper = (kW + FN - 1) / FN, kVper = (kV + FN - 1) / FN;
    template <int J>
    __device__ __forceinline__ static void column() {
        if constexpr (J < FN) {
            constexpr int w = kW - J * kWper < kWper ? (kW - J * kWper > 0 ? kW - J * kWper : 0) : kWper;
            constexpr int v = kV - J * kVper < kVper ? (kV - J * kVper > 0 ? kV - J * kVper : 0) : kVper;
            constexpr int mf = FM * KS;
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            if constexpr (J + 1 < FN) __builtin_amdgcn_sched_group_barrier(0x100, KS, 0);
            if constexpr (w > 0) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x200, w, 0);
            }
            if constexpr (v > 0) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x020, v, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, mf - 1 - (w > 0) - (v > 0), 0);
            column<J + 1>();
        }
    }
    __device__ __forceinline__ static void emit() {
        __builtin_amdgcn_sched_group_barrier(0x100, KS * FM + KS, 0);
        column<0>();
    }
};

template <int BM, int BN, int SA, int SB, int WAVES_M, int WAVES_N>
struct FastRunner {
    static constexpr int THREADS = 64 * WAVES_M * WAVES_N;
    static constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
    static constexpr int FM = WM / 16, FN = WN / 16;
    static constexpr int KS = kBK / 32;
    using LA = Fast<SA, BM, 1, THREADS>;
    using LB = Fast<SB, BN, FN, THREADS>;

    // One k-step: MFMAs over stage `cur` while the registers' tile goes into stage `nxt`
    // and the loads of the tile after it are issued. The two stages are distinct LDS
    // arrays, so the compiler knows the stage writes never alias the fragment reads and
    // can interleave them with the MFMAs.
    __device__ __forceinline__ static void step(LA &la, LB &lb, const uint4 *cur, uint4 *nxt, int64_t knext,
                                                f32x4 (&acc)[FM][FN], const float *lcode, const float *lcode2,
                                                float off_a, float off_b, int lane, int wm0, int wn0) {
        uint4 af[KS][FM];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
            for (int i = 0; i < FM; ++i) {
                if constexpr (SA == SRC_KT) af[ks][i] = kt_fragment<BM>(cur, wm0 + i * 16, ks * 32, lane);
                else af[ks][i] = cur[slot(wm0 + i * 16 + (lane & 15), ks * 4 + (lane >> 4))];
            }
        la.commit(nxt, lcode, lcode2, off_a);
        lb.commit(nxt + BM * 8, lcode, lcode2, off_b);
        la.issue(nxt, knext);
        lb.issue(nxt + BM * 8, knext);
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            uint4 bf[KS];
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                if constexpr (SB == SRC_KT) bf[ks] = kt_fragment<BN>(cur + BM * 8, wn0 + j * 16, ks * 32, lane);
                else bf[ks] = cur[BM * 8 + slot(wn0 + j * 16 + (lane & 15), ks * 4 + (lane >> 4))];
            }
#pragma unroll
            for (int ks = 0; ks < KS; ++ks)
#pragma unroll
                for (int i = 0; i < FM; ++i) acc[i][j] = mfma16x16x32(af[ks][i], bf[ks], acc[i][j]);
        }
#if CT_PV == 2
        SchedPattern<FM, FN, KS, LA, LB>::emit();
#endif
        __syncthreads();
    }

    __device__ __forceinline__ static void run(const Segment &sg, int64_t m, int64_t n, int64_t m0, int64_t n0,
                                               int64_t tbeg, int64_t tend, f32x4 (&acc)[FM][FN], uint4 *lds0,
                                               uint4 *lds1, const float *lcode, const float *lcode2, int tid,
                                               int wm0, int wn0) {
        if (tbeg >= tend) return;
        const int lane = tid & 63;
        LA la;
        LB lb;
        la.init(sg.a, m, sg.k, m0, tid);
        lb.init(sg.b, n, sg.k, n0, tid);
        const float off_a = is_nf4<SA>() ? *sg.a.offset : 0.f;
        const float off_b = is_nf4<SB>() ? *sg.b.offset : 0.f;
        __syncthreads();  // every wave is done with the buffers of a previous segment
        la.issue(lds0, tbeg * kBK);
        lb.issue(lds0 + BM * 8, tbeg * kBK);
        la.commit(lds0, lcode, lcode2, off_a);
        lb.commit(lds0 + BM * 8, lcode, lcode2, off_b);
        la.issue(lds1, (tbeg + 1) * kBK);
        lb.issue(lds1 + BM * 8, (tbeg + 1) * kBK);
        __syncthreads();
        // Step t reads stage (t - tbeg) % 2, which holds tile t; the registers hold tile t+1.
        // Tiles past the end are masked to zeros and never consumed.
        int64_t t = tbeg;
        for (; t + 1 < tend; t += 2) {
            step(la, lb, lds0, lds1, (t + 2) * kBK, acc, lcode, lcode2, off_a, off_b, lane, wm0, wn0);
            step(la, lb, lds1, lds0, (t + 3) * kBK, acc, lcode, lcode2, off_a, off_b, lane, wm0, wn0);
        }
        if (t < tend) step(la, lb, lds0, lds1, (t + 2) * kBK, acc, lcode, lcode2, off_a, off_b, lane, wm0, wn0);
    }
};

// ------------------------------------------------------------------------- the kernel body

// The elementwise step (epilogue.hpp) over a bf16 output tile staged in LDS: rows
// [0, BM/2) in lo, [BM/2, BM) in hi, BN values per row. The workgroup walks the tile in
// 16-byte runs, consecutive threads along a row, so every side input and output access is
// coalesced; each thread reads the side inputs of U runs before it applies and stores any.
template <int KIND, int BM, int BN, int THREADS, bool VEC>
__device__ __forceinline__ void epilogue_tile(const GemmParams &p, const uint16_t *lo, const uint16_t *hi, int tid,
                                              int64_t m0, int64_t n0, int64_t ncols, uint16_t *c) {
    constexpr int kRuns = BM * (BN / 8), kPer = kRuns / THREADS, U = kPer < 8 ? kPer : 8;
    static_assert(kRuns % (THREADS * U) == 0, "whole batches of runs");
    for (int base = tid; base < kRuns; base += THREADS * U) {
        EpiSide<8> side[U];
        float y[U][8];
        int64_t row[U], col[U];
        int count[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int run = base + u * THREADS, lr = run / (BN / 8), lc = (run % (BN / 8)) * 8;
            row[u] = m0 + lr;
            col[u] = n0 + lc;
            count[u] = (row[u] < p.m && col[u] < ncols) ? (ncols - col[u] < 8 ? (int)(ncols - col[u]) : 8) : 0;
            if (count[u] <= 0) continue;
            epilogue_load<KIND, 8>(p.epi, row[u], col[u], count[u], side[u]);
            const uint16_t *src = (lr < BM / 2 ? lo + lr * BN : hi + (lr - BM / 2) * BN) + lc;
            const uint4 q = *reinterpret_cast<const uint4 *>(src);
            const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
            for (int j = 0; j < 8; ++j) y[u][j] = pair_value(w[j / 2], j & 1);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (count[u] <= 0) continue;
            epilogue_apply<KIND, 8>(p.epi, row[u], col[u], count[u], side[u], y[u]);
            uint16_t *out = c + row[u] * p.ldc + col[u];
            if (VEC && count[u] == 8) {
                *reinterpret_cast<uint4 *>(out) = make_uint4(pack_bf16x2(y[u][0], y[u][1]), pack_bf16x2(y[u][2], y[u][3]),
                                                             pack_bf16x2(y[u][4], y[u][5]), pack_bf16x2(y[u][6], y[u][7]));
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    if (j < count[u]) out[j] = bf16_bits(y[u][j]);
            }
        }
    }
}

template <int BM, int BN, int A0, int B0, int A1, int B1, int MODE, int OUT, int WAVES_M = 2, int WAVES_N = 2>
__device__ __forceinline__ void gemm_body(const GemmParams &p) {
    constexpr bool VEC = MODE != 0;
    constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
    constexpr int FM = WM / 16, FN = WN / 16;
    static_assert(MODE == 2 || (WAVES_M == 2 && WAVES_N == 2), "the generic runner uses 4 waves");
    constexpr bool kNF4 = is_nf4<A0>() || is_nf4<B0>() || is_nf4<A1>() || is_nf4<B1>();
    __shared__ uint4 lds0[(BM + BN) * 8];
    __shared__ uint4 lds1[(BM + BN) * 8];
    __shared__ float lcode[kNF4 ? 16 : 1];
    __shared__ float lcode2[kNF4 ? 256 : 1];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm0 = (wave % WAVES_M) * WM, wn0 = (wave / WAVES_M) * WN;

    // Tile order: contiguous ranges per XCD, M-grouped inside a range.
    const int tiles = p.tiles_m * p.tiles_n;
    const int pid = blockIdx.x;
    const int xcd = pid % kXcds, local = pid / kXcds;
    const int per = (tiles + kXcds - 1) / kXcds;
    const int tall = tiles % kXcds == 0 ? kXcds : tiles % kXcds;
    const int rid = xcd < tall ? xcd * per + local : tall * per + (xcd - tall) * (per - 1) + local;
    const int group = rid / (kGroupM * p.tiles_n);
    const int first_m = group * kGroupM;
    const int gsize = p.tiles_m - first_m < kGroupM ? p.tiles_m - first_m : kGroupM;
    const int tm = first_m + (rid % (kGroupM * p.tiles_n)) % gsize;
    const int tn = (rid % (kGroupM * p.tiles_n)) / gsize;
    const int64_t m0 = (int64_t)tm * BM;
    // Grouped products: the tile's operands, its column offset inside them and its column
    // count; `out_shift` moves its output columns past group 0.
    constexpr bool kGrouped = OUT == CT_F32 && (A0 == SRC_KS || A0 == SRC_KT) &&
                              (B0 == SRC_KS || B0 == SRC_KT);  // the parameter gradients
    const bool second = kGrouped && p.group_tiles > 0 && tn >= p.group_tiles;
    // Copied by a branch on the (uniform) condition: a reference chosen by a select would
    // move the kernel argument to private memory and make every descriptor built from it
    // look divergent (a readfirstlane loop around each buffer load).
    Segment sg0;
    if (second) sg0 = p.seg[1];
    else sg0 = p.seg[0];
    const int64_t n0 = (int64_t)(second ? tn - p.group_tiles : tn) * BN;
    const int64_t ncols = second ? p.n1 : p.n;
    // The second of two side-by-side projections (ct_group_forward): its own output matrix
    // and its columns of the stacked xa. Chosen by branches on the uniform condition (see
    // sg0 above).
    const bool alt = p.alt_col > 0 && n0 >= p.alt_col;
    void *cout = p.c;
    int64_t ldc = p.ldc;
    int64_t out_shift = second ? (int64_t)p.group_tiles * BN : 0;
    // bias element of output column col: bias_p[col + bias_shift]
    const uint16_t *bias_p = p.bias;
    int64_t bias_shift = 0;
    Segment sg1;
    if (alt) {
        sg1 = p.seg[1];
        sg1.a.p = static_cast<const uint16_t *>(sg1.a.p) + p.alt_a1;
        cout = p.c_alt;
        ldc = p.ldc_alt;
        out_shift = -p.alt_col;
        bias_p = p.bias_alt;
        bias_shift = -p.alt_col;
    } else {
        sg1 = p.seg[1];
    }

    if constexpr (kNF4) {
        if (tid < 16) lcode[tid] = p.code[tid];
        if (p.code2 && tid < 256) lcode2[tid] = p.code2[tid];
        // made visible by the barrier that precedes the first tile store
    }

    f32x4 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int64_t t0 = cdiv(sg0.k, kBK);
    const int64_t t1 = p.nseg > 1 ? cdiv(p.seg[1].k, kBK) : 0;
    const int64_t tbeg = (int64_t)blockIdx.z * p.tiles_per_split;
    const int64_t tend = tbeg + p.tiles_per_split < t0 + t1 ? tbeg + p.tiles_per_split : t0 + t1;
    {
        const int64_t b = tbeg, e = tend < t0 ? tend : t0;
        if constexpr (MODE == 2)
            FastRunner<BM, BN, A0, B0, WAVES_M, WAVES_N>::run(sg0, p.m, ncols, m0, n0, b, e, acc, lds0, lds1,
                                                              lcode, lcode2, tid, wm0, wn0);
        else
            SegmentRunner<BM, BN, A0, B0, VEC>::run(sg0, p.m, ncols, m0, n0, b, e, acc, lds0, lds1, lcode,
                                                    lcode2, tid, wm0, wn0);
    }
    if (t1 > 0) {
        const int64_t b = tbeg > t0 ? tbeg - t0 : 0, e = tend - t0;
        if constexpr (MODE == 2)
            FastRunner<BM, BN, A1, B1, WAVES_M, WAVES_N>::run(sg1, p.m, p.n, m0, n0, b, e, acc, lds0, lds1,
                                                              lcode, lcode2, tid, wm0, wn0);
        else
            SegmentRunner<BM, BN, A1, B1, VEC>::run(sg1, p.m, p.n, m0, n0, b, e, acc, lds0, lds1, lcode,
                                                    lcode2, tid, wm0, wn0);
    }

    // ------------------------------------------------------------------ epilogue
    if constexpr (B0 == SRC_KT) {
        // KT B fragments leave lane l with columns wn0 + 16 j + (l % 16): element stores.
#pragma unroll
        for (int i = 0; i < FM; ++i) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int64_t row = m0 + wm0 + i * 16 + (lane >> 4) * 4 + e;
                if (row >= p.m) continue;
#pragma unroll
                for (int j = 0; j < FN; ++j) {
                    const int64_t col = n0 + wn0 + 16 * j + (lane & 15);
                    if (col >= ncols) continue;
                    const float bias = bias_p ? bf16_to_f32(bias_p[col + bias_shift]) : 0.f;
                    const float v = acc[i][j][e] + bias;
                    if constexpr (OUT == CT_F32) {
                        float *c = (second && p.c1) ? p.c1 + col * p.ldc1 + row
                                                    : static_cast<float *>(p.c) + (int64_t)blockIdx.z * p.split_stride +
                                                          row * p.ldc + out_shift + col;
                        *c = p.beta ? v + *c : v;
                    } else {
                        uint16_t *c = static_cast<uint16_t *>(p.c) + row * p.ldc + out_shift + col;
                        *c = bf16_bits(p.beta ? v + bf16_to_f32(*c) : v);
                    }
                }
            }
        }
        return;
    }
    // Lane l holds rows wm0 + 16 i + 4 (l / 16) + e and columns wn0 + FN (l % 16) + j.
    const int64_t col = n0 + wn0 + (lane & 15) * FN;
    float bias[FN];
#pragma unroll
    for (int j = 0; j < FN; ++j)
        bias[j] = (bias_p && col + j < ncols) ? bf16_to_f32(bias_p[col + j + bias_shift]) : 0.f;
    const bool full = col + FN <= ncols;
    if constexpr (OUT == CT_BF16) {
        if (p.epi.kind != CT_EPI_NONE && !p.beta) {
            // Stage the rounded tile in LDS (the operand buffers are free once every wave
            // has left the main loop), then run the step over it in coalesced runs.
            static_assert((BM + BN) * 8 * 16 >= BM * BN, "half a bf16 tile fits one operand buffer");
            static_assert(WM <= BM / 2 && (BM / 2) % WM == 0, "a wave's rows stay inside one half");
            __syncthreads();
            uint16_t *lo = reinterpret_cast<uint16_t *>(lds0), *hi = reinterpret_cast<uint16_t *>(lds1);
            uint16_t *mine = wm0 < BM / 2 ? lo : hi;
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int lr = (wm0 % (BM / 2)) + i * 16 + (lane >> 4) * 4 + e;
                    uint32_t w[FN / 2];
#pragma unroll
                    for (int j = 0; j < FN / 2; ++j)
                        w[j] = pack_bf16x2(acc[i][2 * j][e] + bias[2 * j], acc[i][2 * j + 1][e] + bias[2 * j + 1]);
                    uint16_t *dst = mine + lr * BN + wn0 + (lane & 15) * FN;
                    if constexpr (FN == 8) *reinterpret_cast<uint4 *>(dst) = make_uint4(w[0], w[1], w[2], w[3]);
                    else if constexpr (FN == 4) *reinterpret_cast<uint2 *>(dst) = make_uint2(w[0], w[1]);
                    else *reinterpret_cast<uint32_t *>(dst) = w[0];
                }
            __syncthreads();
            constexpr int kThreadsWg = WAVES_M * WAVES_N * 64;
            uint16_t *c = static_cast<uint16_t *>(p.c) + out_shift;
            switch (p.epi.kind) {
                case CT_EPI_RESIDUAL:
                    epilogue_tile<CT_EPI_RESIDUAL, BM, BN, kThreadsWg, VEC>(p, lo, hi, tid, m0, n0, ncols, c);
                    break;
                case CT_EPI_SILU:
                    epilogue_tile<CT_EPI_SILU, BM, BN, kThreadsWg, VEC>(p, lo, hi, tid, m0, n0, ncols, c);
                    break;
                case CT_EPI_DSILU:
                    epilogue_tile<CT_EPI_DSILU, BM, BN, kThreadsWg, VEC>(p, lo, hi, tid, m0, n0, ncols, c);
                    break;
                case CT_EPI_ROPE:
                    epilogue_tile<CT_EPI_ROPE, BM, BN, kThreadsWg, VEC>(p, lo, hi, tid, m0, n0, ncols, c);
                    break;
                default:
                    break;
            }
            return;
        }
    }
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
                float *c = static_cast<float *>(cout) + (int64_t)blockIdx.z * p.split_stride + row * ldc +
                           out_shift + col;
                if (VEC && full && FN % 4 == 0) {
#pragma unroll
                    for (int j = 0; j < FN; j += 4) {
                        f32x4 w = {v[j], v[j + 1], v[j + 2], v[j + 3]};
                        if (p.beta) w += *reinterpret_cast<const f32x4 *>(c + j);
                        *reinterpret_cast<f32x4 *>(c + j) = w;
                    }
                } else {
#pragma unroll
                    for (int j = 0; j < FN; ++j) {
                        if (!full && col + j >= ncols) break;
                        c[j] = p.beta ? v[j] + c[j] : v[j];
                    }
                }
            } else {
                uint16_t *c = static_cast<uint16_t *>(cout) + row * ldc + out_shift + col;
                if (p.beta) {
                    if (VEC && full && (FN == 8 || FN == 4)) {
                        // one 16- or 8-byte read of the FN existing values
                        uint32_t w[FN / 2];
                        if constexpr (FN == 8) {
                            const uint4 q = *reinterpret_cast<const uint4 *>(c);
                            w[0] = q.x, w[1] = q.y, w[2] = q.z, w[3] = q.w;
                        } else {
                            const uint2 q = *reinterpret_cast<const uint2 *>(c);
                            w[0] = q.x, w[1] = q.y;
                        }
#pragma unroll
                        for (int j = 0; j < FN; ++j)
                            v[j] = v[j] + bf16_to_f32((uint16_t)(j & 1 ? w[j / 2] >> 16 : w[j / 2] & 0xffffu));
                    } else {
#pragma unroll
                        for (int j = 0; j < FN; ++j)
                            if (full || col + j < ncols) v[j] = v[j] + bf16_to_f32(c[j]);
                    }
                }
                if (VEC && full && FN >= 2) {
                    uint32_t w[FN / 2];
#pragma unroll
                    for (int j = 0; j < FN / 2; ++j) w[j] = pack_bf16x2(v[2 * j], v[2 * j + 1]);
                    if constexpr (FN == 8) *reinterpret_cast<uint4 *>(c) = make_uint4(w[0], w[1], w[2], w[3]);
                    else if constexpr (FN == 4) *reinterpret_cast<uint2 *>(c) = make_uint2(w[0], w[1]);
                    else *reinterpret_cast<uint32_t *>(c) = w[0];
                } else {
#pragma unroll
                    for (int j = 0; j < FN; ++j) {
                        if (!full && col + j >= ncols) break;
                        c[j] = bf16_bits(v[j]);
                    }
                }
            }
        }
    }
}

// 256x256 tiles: one workgroup per CU, 512 registers per lane (accumulators in AGPRs).
template <int A0, int B0, int A1, int B1, int MODE, int OUT>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1))) void gemm_big(
    const GemmParams p) {
    gemm_body<256, 256, A0, B0, A1, B1, MODE, OUT>(p);
}

template <int BM, int BN, int A0, int B0, int A1, int B1, int MODE, int OUT>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2))) void gemm_small(const GemmParams p) {
    gemm_body<BM, BN, A0, B0, A1, B1, MODE, OUT>(p);
}

// 256x256 tiles, 8 waves (two per SIMD) of 64x128: each wave's accumulators fit in 128
// registers, and the second wave on a SIMD issues MFMA while the first waits on LDS or
// the barrier. Fast operand path only.
template <int A0, int B0, int A1, int B1, int OUT>
__global__ __launch_bounds__(512) void gemm_big8(const GemmParams p) {
    gemm_body<256, 256, A0, B0, A1, B1, 2, OUT, 4, 2>(p);
}

// Deterministic reduction of fp32 split partials: out = sum_z ws[z] (+ bias) (+ out), in
// z order. Grid: (column blocks of 256, rows); eight partials in flight per thread (they
// were written by other XCDs and come from memory).
template <int OUT>
__global__ __launch_bounds__(256) void reduce_splits(const float *__restrict__ ws, int splits, int64_t stride,
                                                     int64_t rows, int64_t cols, void *out, int64_t ldo, int add,
                                                     const uint16_t *__restrict__ bias) {
    const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x, r = blockIdx.y;
    if (c >= cols) return;
    const int64_t i = r * cols + c;
    float s = 0.f;
    for (int z0 = 0; z0 < splits; z0 += 8) {
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = z0 + j < splits ? ws[(z0 + j) * stride + i] : 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (z0 + j < splits) s = (z0 + j == 0) ? v[j] : s + v[j];
    }
    if (bias) s += bf16_to_f32(bias[c]);
    if constexpr (OUT == CT_F32) {
        float *o = static_cast<float *>(out) + r * ldo + c;
        *o = add ? s + *o : s;
    } else {
        uint16_t *o = static_cast<uint16_t *>(out) + r * ldo + c;
        *o = bf16_bits(add ? s + bf16_to_f32(*o) : s);
    }
}

// reduce_splits with 16-byte accesses, eight columns per thread, the same sums in the same
// order (identical results). Needs cols % 8 == 0, 16-byte aligned partials, output and
// bias, and ldo % 8 == 0. Grid: (column blocks of 2048, rows).
// With `res` (bf16 output only, add = 0): the residual step of the projection epilogue,
// out = bf16(bf16(sum) + res), the reference's add_ on the stored output
// (kernels/linear.py:90-91, kernels/mlp_cuda.py:80), fused into the reduction.
template <int OUT>
__global__ __launch_bounds__(256) void reduce_splits_vec(const float *__restrict__ ws, int splits, int64_t stride,
                                                         int64_t rows, int64_t cols, void *out, int64_t ldo, int add,
                                                         const uint16_t *__restrict__ bias,
                                                         const uint16_t *__restrict__ res = nullptr,
                                                         int64_t ldres = 0) {
    const int64_t c = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8, r = blockIdx.y;
    if (c >= cols) return;
    const float *src = ws + r * cols + c;
    float s[8];
    for (int z0 = 0; z0 < splits; z0 += 4) {
        float4 v[4][2];
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (z0 + j < splits) {
                const float4 *q = reinterpret_cast<const float4 *>(src + (z0 + j) * stride);
                v[j][0] = q[0];
                v[j][1] = q[1];
            }
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (z0 + j < splits) {
                const float x[8] = {v[j][0].x, v[j][0].y, v[j][0].z, v[j][0].w,
                                    v[j][1].x, v[j][1].y, v[j][1].z, v[j][1].w};
#pragma unroll
                for (int e = 0; e < 8; ++e) s[e] = (z0 + j == 0) ? x[e] : s[e] + x[e];
            }
    }
    if (bias) {
        const uint4 b = *reinterpret_cast<const uint4 *>(bias + c);
        const uint32_t w[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) s[e] += bf16_to_f32((uint16_t)(w[e / 2] >> (16 * (e & 1))));
    }
    if constexpr (OUT == CT_F32) {
        float4 *o = reinterpret_cast<float4 *>(static_cast<float *>(out) + r * ldo + c);
        float4 lo = make_float4(s[0], s[1], s[2], s[3]), hi = make_float4(s[4], s[5], s[6], s[7]);
        if (add) {
            const float4 a0 = o[0], a1 = o[1];
            lo = make_float4(s[0] + a0.x, s[1] + a0.y, s[2] + a0.z, s[3] + a0.w);
            hi = make_float4(s[4] + a1.x, s[5] + a1.y, s[6] + a1.z, s[7] + a1.w);
        }
        o[0] = lo;
        o[1] = hi;
    } else {
        uint4 *o = reinterpret_cast<uint4 *>(static_cast<uint16_t *>(out) + r * ldo + c);
        if (add) {
            const uint4 q = *o;
            const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) s[e] = s[e] + bf16_to_f32((uint16_t)(w[e / 2] >> (16 * (e & 1))));
        }
        if (res) {
            const uint4 q = *reinterpret_cast<const uint4 *>(res + r * ldres + c);
            const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
            for (int e = 0; e < 8; ++e)
                s[e] = bf16_to_f32(bf16_bits(s[e])) + bf16_to_f32((uint16_t)(w[e / 2] >> (16 * (e & 1))));
        }
        *o = make_uint4(pack_bf16x2(s[0], s[1]), pack_bf16x2(s[2], s[3]), pack_bf16x2(s[4], s[5]),
                        pack_bf16x2(s[6], s[7]));
    }
}

// A fill kernel rather than hipMemsetAsync, so the call stays safe inside graph capture.
__global__ __launch_bounds__(256) void fill_zero(float *p, int64_t count) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < count) p[i] = 0.f;
}

// Sums the split partials of the grouped parameter-gradient GEMM, ws[z][i][c] with
// c < width, in split order: columns below `gcols` are da[i][c] (c < k), the rest are
// db[c - gcols][i] (< n), i.e. dB^T is written transposed.
// Grid: (column blocks of 256, rows r); eight partials in flight per thread.
__global__ __launch_bounds__(256) void reduce_param(const float *__restrict__ ws, int splits, int64_t stride,
                                                    int64_t r, int64_t width, int64_t gcols, int64_t k,
                                                    int64_t n, float *da, float *db, int add) {
    const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x, i = blockIdx.y;
    if (c >= width) return;
    float *o;
    if (c < gcols) {
        if (c >= k) return;
        o = da + i * k + c;
    } else {
        if (c - gcols >= n) return;
        o = db + (c - gcols) * r + i;
    }
    const int64_t idx = i * width + c;
    float s = 0.f;
    for (int z0 = 0; z0 < splits; z0 += 8) {
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = z0 + j < splits ? ws[(z0 + j) * stride + idx] : 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (z0 + j < splits) s = (z0 + j == 0) ? v[j] : s + v[j];
    }
    *o = add ? s + *o : s;
}

// reduce_param over 32 x 64 tiles (rows i, columns c) with 16-byte accesses and the same
// sums in the same order (identical results): a dA tile is written row by row; a dB^T tile
// goes through LDS so that dB [n, r] is written along r, 32 contiguous floats per column
// (the per-element kernel writes it with a stride of r floats). Needs width, k and r
// multiples of 8, gcols a multiple of 64, and 16-byte aligned partials, da and db.
// Grid: (cdiv(width, 64), cdiv(r, 32)).
__global__ __launch_bounds__(256) void reduce_param_tiled(const float *__restrict__ ws, int splits, int64_t stride,
                                                          int64_t r, int64_t width, int64_t gcols, int64_t k,
                                                          int64_t n, float *da, float *db, int add) {
    __shared__ float tile[64][33];
    const int t = threadIdx.x, li = t >> 3, lc = (t & 7) * 8;
    const int64_t i0 = (int64_t)blockIdx.y * 32, c0 = (int64_t)blockIdx.x * 64;
    const int64_t i = i0 + li, c = c0 + lc;
    float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (i < r && c < width) {
        const float *src = ws + i * width + c;
        for (int z0 = 0; z0 < splits; z0 += 4) {
            float4 v[4][2];
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (z0 + j < splits) {
                    const float4 *q = reinterpret_cast<const float4 *>(src + (z0 + j) * stride);
                    v[j][0] = q[0];
                    v[j][1] = q[1];
                }
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (z0 + j < splits) {
                    const float x[8] = {v[j][0].x, v[j][0].y, v[j][0].z, v[j][0].w,
                                        v[j][1].x, v[j][1].y, v[j][1].z, v[j][1].w};
#pragma unroll
                    for (int e = 0; e < 8; ++e) s[e] = (z0 + j == 0) ? x[e] : s[e] + x[e];
                }
        }
    }
    if (c0 < gcols) {  // the whole tile is dA (gcols is a multiple of 64)
        if (i >= r || c >= k) return;
        float4 *o = reinterpret_cast<float4 *>(da + i * k + c);
        float4 lo = make_float4(s[0], s[1], s[2], s[3]), hi = make_float4(s[4], s[5], s[6], s[7]);
        if (add) {
            const float4 a0 = o[0], a1 = o[1];
            lo = make_float4(s[0] + a0.x, s[1] + a0.y, s[2] + a0.z, s[3] + a0.w);
            hi = make_float4(s[4] + a1.x, s[5] + a1.y, s[6] + a1.z, s[7] + a1.w);
        }
        o[0] = lo;
        o[1] = hi;
        return;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) tile[lc + e][li] = s[e];
    __syncthreads();
    const int cc = t >> 2, ig = (t & 3) * 8;
    const int64_t col = c0 - gcols + cc, row = i0 + ig;
    if (col >= n || row >= r) return;
    float y[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) y[e] = tile[cc][ig + e];
    float4 *o = reinterpret_cast<float4 *>(db + col * r + row);
    float4 lo = make_float4(y[0], y[1], y[2], y[3]), hi = make_float4(y[4], y[5], y[6], y[7]);
    if (add) {
        const float4 a0 = o[0], a1 = o[1];
        lo = make_float4(y[0] + a0.x, y[1] + a0.y, y[2] + a0.z, y[3] + a0.w);
        hi = make_float4(y[4] + a1.x, y[5] + a1.y, y[6] + a1.z, y[7] + a1.w);
    }
    o[0] = lo;
    o[1] = hi;
}

// ------------------------------------------------------------------------ host side
enum Tile { TILE_256 = 0, TILE_128 = 1, TILE_64 = 2 };
constexpr int kTileEdge[3] = {256, 128, 64};

#ifndef CT_MATERIALIZE_ROWS
#define CT_MATERIALIZE_ROWS 512
#endif
// An NF4 base weight is decoded inside the GEMM's operand loader only while the rows are
// few: each 256-row tile decodes its slice of the weight again, and from kMaterializeRows
// rows on one ct_nf4_dequant pass into the workspace (the reference's materialize) plus
// the dense GEMM is faster. Both give identical results.
constexpr int64_t kMaterializeRows = CT_MATERIALIZE_ROWS;
// Reductions at least this long keep the split route from kMaterializeRows rows on.
constexpr int64_t kLongReduction = 8192;
// Rows between the few-row kernels (m <= 64) and kMaterializeRows, and more rows with a
// reduction of at least kLongReduction: the output leaves the 256 x 256 grid short of one
// round, so the fast runner splits the reduction and the fp32 partials are added in split
// order (with bias and beta) by reduce_splits. Past kMaterializeRows the alternative is
// the 128 x 128 or 64 x 64 grid over the whole reduction, which runs at half the rate or
// less (measured on MI355X at 512-4096 rows and 12288-49152 reductions: 1.2-2.8x slower
// than the split; 6-9% slower at 2048-4096 rows, 2048 columns and 8448); shorter
// reductions there pay too much for the partials' traffic (2048: 25% slower split). The
// split count depends only on the shapes.
int mid_splits(int64_t m, int64_t n, int64_t ktot) {
    if (m <= 64 || n <= 0) return 1;
    const int64_t tiles = cdiv(m, 256) * cdiv(n, 256);
    if (m >= kMaterializeRows && (ktot < kLongReduction || tiles >= 256)) return 1;
    // One round of the one-per-CU 256 x 256 workgroups: a partial second round would
    // take as long as the first.
    int64_t s = 256 / tiles;
    const int64_t cap = cdiv(ktot, kBK) / 8;  // at least 8 k-tiles per split
    if (s > cap) s = cap;
    if (s > 32) s = 32;
    return (int)(s < 1 ? 1 : s);
}

struct Problem {
    GemmParams p;
    int src[4];   // A0, B0, A1, B1
    int out;      // CT_BF16 or CT_F32
    bool vec;
    int splits;
    int tile;     // forced tile, or -1 to choose
    void *ws;     // caller's workspace for few-row split reductions (may be null)
    int64_t ws_bytes;
};

// Byte extent of a dense operand whose output-dimension extent is `rows`.
int64_t dense_extent(const Operand &o, int src, int64_t rows, int64_t k) {
    return (src == SRC_KS || src == SRC_KT) ? ((k > 0 ? k - 1 : 0) * o.ld + rows) * 2 : rows * o.ld * 2;
}

bool aligned16(const void *q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; }
constexpr bool is_nf4_host(int src) { return src == SRC_NF4 || src == SRC_NF4T; }

// Vector (16-byte) operand access needs aligned bases, leading dimensions that are
// multiples of 8 elements, and 8-multiple extents along each contiguous dimension.
// Segments the kernels read: both for a two-segment contraction or a grouped launch.
int operand_segments(const GemmParams &p) { return p.group_tiles > 0 ? 2 : p.nseg; }
// Columns of segment s's B operand.
int64_t segment_cols(const GemmParams &p, int s) { return (p.group_tiles > 0 && s == 1) ? p.n1 : p.n; }

bool vec_ok(const Problem &pr) {
    const GemmParams &p = pr.p;
    for (int s = 0; s < operand_segments(p); ++s) {
        const Segment &g = p.seg[s];
        const int sa = pr.src[2 * s], sb = pr.src[2 * s + 1];
        if (g.k % 8) return false;
        if (!is_nf4_host(sa) && (!aligned16(g.a.p) || g.a.ld % 8)) return false;
        if (!is_nf4_host(sb) && (!aligned16(g.b.p) || g.b.ld % 8)) return false;
        if ((sa == SRC_KS || sa == SRC_KT) && p.m % 8) return false;
        if ((sb == SRC_KS || sb == SRC_KT) && segment_cols(p, s) % 8) return false;
    }
    if (!aligned16(p.c) || p.ldc % 8) return false;
    return true;
}

// The fast runner: 16-byte operand access (vec_ok), 32-bit buffer offsets, nested NF4.
bool fast_ok(const Problem &pr) {
    if (!pr.vec) return false;
    const GemmParams &p = pr.p;
    constexpr int64_t kLimit = int64_t{1} << 31;
    for (int s = 0; s < operand_segments(p); ++s) {
        const Segment &g = p.seg[s];
        const int src[2] = {pr.src[2 * s], pr.src[2 * s + 1]};
        const Operand *op[2] = {&g.a, &g.b};
        const int64_t rows[2] = {p.m, segment_cols(p, s)};
        for (int i = 0; i < 2; ++i) {
            if (is_nf4_host(src[i])) {
                const int64_t n = (src[i] == SRC_NF4 ? rows[i] : g.k) * op[i]->ld;
                if (!op[i]->nested || n >= kLimit) return false;
            } else if (dense_extent(*op[i], src[i], rows[i], g.k) >= kLimit) {
                return false;
            }
        }
    }
    return true;
}

// Largest tile that still yields about one workgroup per CU (256 CUs).
int choose_tile(int64_t m, int64_t n, int splits) {
    for (int t = TILE_256; t < TILE_64; ++t) {
        const int64_t e = kTileEdge[t];
        if (cdiv(m, e) * cdiv(n, e) * splits >= 256) return t;
    }
    return TILE_64;
}

template <int A0, int B0, int A1, int B1, int MODE, int OUT>
hipError_t launch_cfg(const GemmParams &p0, int tile, int splits, hipStream_t s) {
    GemmParams p = p0;
    const int e = kTileEdge[tile];
    p.tiles_m = (int)cdiv(p.m, e);
    p.tiles_n = (int)(p.group_tiles > 0 ? p.group_tiles + cdiv(p.n1, e) : cdiv(p.n, e));
    dim3 grid((unsigned)(p.tiles_m * p.tiles_n), 1, (unsigned)splits);
    if (tile == TILE_256 && MODE == 2) gemm_big8<A0, B0, A1, B1, OUT><<<grid, dim3(512), 0, s>>>(p);
    else if (tile == TILE_256) gemm_big<A0, B0, A1, B1, MODE, OUT><<<grid, dim3(kThreads), 0, s>>>(p);
    else if (tile == TILE_128) gemm_small<128, 128, A0, B0, A1, B1, MODE, OUT><<<grid, dim3(kThreads), 0, s>>>(p);
    else gemm_small<64, 64, A0, B0, A1, B1, MODE, OUT><<<grid, dim3(kThreads), 0, s>>>(p);
    return hipGetLastError();
}

// One fixed tile on the fast runner (operand sources the generic runner does not have).
template <int A0, int B0, int A1, int B1, int OUT, int TILE>
hipError_t launch_cfg_fast(const GemmParams &p0, int splits, hipStream_t s) {
    GemmParams p = p0;
    constexpr int e = TILE == TILE_256 ? 256 : 128;
    p.tiles_m = (int)cdiv(p.m, e);
    p.tiles_n = (int)(p.group_tiles > 0 ? p.group_tiles + cdiv(p.n1, e) : cdiv(p.n, e));
    dim3 grid((unsigned)(p.tiles_m * p.tiles_n), 1, (unsigned)splits);
    if constexpr (TILE == TILE_256) gemm_big8<A0, B0, A1, B1, OUT><<<grid, dim3(512), 0, s>>>(p);
    else gemm_small<128, 128, A0, B0, A1, B1, 2, OUT><<<grid, dim3(kThreads), 0, s>>>(p);
    return hipGetLastError();
}

template <int A0, int B0, int A1, int B1, int OUT>
hipError_t launch_mode(const Problem &pr, int tile, hipStream_t s) {
    if (fast_ok(pr)) return launch_cfg<A0, B0, A1, B1, 2, OUT>(pr.p, tile, pr.splits, s);
    if (pr.vec) return launch_cfg<A0, B0, A1, B1, 1, OUT>(pr.p, tile, pr.splits, s);
    return launch_cfg<A0, B0, A1, B1, 0, OUT>(pr.p, tile, pr.splits, s);
}

template <int A0, int B0, int A1, int B1>
hipError_t launch_vec_out(const Problem &pr, int tile, hipStream_t s) {
    return pr.out == CT_F32 ? launch_mode<A0, B0, A1, B1, CT_F32>(pr, tile, s)
                            : launch_mode<A0, B0, A1, B1, CT_BF16>(pr, tile, s);
}

int64_t total_tiles(const GemmParams &p) {
    return cdiv(p.seg[0].k, kBK) + (p.nseg > 1 ? cdiv(p.seg[1].k, kBK) : 0);
}

#define CT_LAYOUT(a0, b0, a1, b1) \
    (((a0) << 12) | ((b0) << 8) | ((a1) << 4) | (b1))

// out (+)= sum of the fp32 split partials in ws (+ bias), in split order: 16-byte accesses
// where the layout allows them (the same sums either way).
bool reduce_vec_ok(const float *ws, int64_t cols, const void *out, int64_t ldo, const uint16_t *bias) {
    return cols % 8 == 0 && ldo % 8 == 0 && aligned16(ws) && aligned16(out) && (!bias || aligned16(bias));
}

template <int OUT>
hipError_t launch_reduce(const float *ws, int splits, int64_t stride, int64_t rows, int64_t cols, void *out,
                         int64_t ldo, int add, const uint16_t *bias, hipStream_t s, const uint16_t *res = nullptr,
                         int64_t ldres = 0) {
    if (res && !reduce_vec_ok(ws, cols, out, ldo, bias)) return hipErrorInvalidValue;
    if (reduce_vec_ok(ws, cols, out, ldo, bias))
        reduce_splits_vec<OUT><<<dim3((unsigned)cdiv(cols, 2048), (unsigned)rows), 256, 0, s>>>(
            ws, splits, stride, rows, cols, out, ldo, add, bias, res, ldres);
    else
        reduce_splits<OUT><<<dim3((unsigned)cdiv(cols, 256), (unsigned)rows), 256, 0, s>>>(ws, splits, stride, rows,
                                                                                          cols, out, ldo, add, bias);
    return hipGetLastError();
}

// Split count of the split route (fp32 split partials of the 256 x 256 runner, then a
// reduction; the shapes mid_splits takes), or 1 when the problem does not take it.
int mid_split_route(const Problem &pr) {
    const GemmParams &p = pr.p;
    if (pr.splits != 1 || pr.out != CT_BF16 || p.group_tiles != 0 || p.m <= 64) return 1;
    const int splits = mid_splits(p.m, p.n, p.seg[0].k + (p.nseg > 1 ? p.seg[1].k : 0));
    const int64_t need = (int64_t)splits * p.m * p.n * 4;
    return (splits > 1 && fast_ok(pr) && pr.ws && pr.ws_bytes >= need && aligned16(pr.ws) && p.n % 8 == 0) ? splits
                                                                                                           : 1;
}

// Whether the problem's epilogue runs inside the GEMM (epilogue_tile over the LDS-staged
// output tile) rather than as a pass over the finished output. The split and few-row
// routes always pass afterwards. So do the SiLU steps on 256 x 256 tiles: one workgroup
// fills a CU there, so their two or three extra tensor streams would run with the MFMA
// units idle, after every tile at once (measured slower than the separate pass at 4096 x
// 8192), while the 128 x 128 tiles run two workgroups per CU and overlap one's step with
// the other's products.
// The residual step on the split route rides in the split reduction (reduce_splits_vec),
// which reads the partials and writes the output anyway: measured on MI355X, the pass after
// the reduction cost more than a separate add (C4's down projection, 4096 x 2048 over 8448).
bool residual_in_reduction(const Problem &pr) {
    const GemmParams &p = pr.p;
    return p.epi.kind == CT_EPI_RESIDUAL && !p.beta && p.epi.vec && p.epi.in0 && mid_split_route(pr) > 1 &&
           aligned16(p.c) && p.ldc % 8 == 0 && (!p.bias || aligned16(p.bias));
}

bool epilogue_fused(const Problem &pr) {
    const GemmParams &p = pr.p;
    if (residual_in_reduction(pr)) return true;
    if (mid_split_route(pr) > 1) return false;
    if (pr.splits == 1 && pr.out == CT_BF16 && p.m <= 64) {
        const int sa[2] = {pr.src[0], p.nseg > 1 ? pr.src[2] : pr.src[0]};
        const int sb[2] = {pr.src[1], p.nseg > 1 ? pr.src[3] : pr.src[1]};
        if (skinny_supported(p, sa, sb, pr.out)) return false;
    }
    const int tile = pr.tile >= 0 ? pr.tile : choose_tile(p.m, p.n, pr.splits);
    return !(tile == TILE_256 && (p.epi.kind == CT_EPI_SILU || p.epi.kind == CT_EPI_DSILU));
}

// A 256 x 256 grid whose last round holds at most half of the 256 CUs' workgroups (C3's
// dx of down: 32 x 43 tiles, 5 rounds and 96 tiles) splits its output columns: the first
// `head` (a multiple of 256) give whole rounds, the rest (at most 128 tiles' worth) run as
// a second launch of 128 x 128 tiles, two per CU. Dense bf16 operands with plain bf16
// output only: the B operands and the output are offset by `head` columns.
bool column_split(const Problem &pr, int64_t *head) {
    const GemmParams &p = pr.p;
    if (pr.splits != 1 || pr.out != CT_BF16 || p.group_tiles > 0 || p.alt_col > 0 || p.epi.kind != CT_EPI_NONE)
        return false;
    for (int s = 0; s < p.nseg; ++s) {
        const int a = pr.src[2 * s], b = pr.src[2 * s + 1];
        if (a != SRC_KC || (b != SRC_KC && b != SRC_KS)) return false;
    }
    const int64_t tm = cdiv(p.m, 256), tn = cdiv(p.n, 256);
    const int64_t rem = (tm * tn) % 256;
    if (rem == 0 || rem > 128 || tn < 2) return false;
    int64_t lead = tn - 1;
    while (lead > 0 && (tm * lead) % 256) --lead;
    if (lead <= 0 || tm * (tn - lead) > 128) return false;
    *head = lead * 256;
    return true;
}

hipError_t run(Problem &pr, hipStream_t s) {
    GemmParams &p = pr.p;
    if (p.m == 0 || p.n == 0) return hipSuccess;
    if (p.nseg == 1) {
        pr.src[2] = pr.src[0];
        pr.src[3] = pr.src[1];
    }
    if (p.epi.kind != CT_EPI_NONE && !epilogue_fused(pr)) {
        // The product alone, then the step over it. A SiLU step that keeps the raw product
        // has the GEMM write it straight to the kept buffer, which the pass then reads.
        Problem q = pr;
        EpiParams post = p.epi;
        q.p.epi.kind = CT_EPI_NONE;
        void *src = p.c;
        int64_t ldsrc = p.ldc;
        if (post.kind == CT_EPI_SILU && post.out0) {
            src = post.out0;
            ldsrc = post.ld_out0;
            q.p.c = post.out0;
            q.p.ldc = post.ld_out0;
            q.vec = vec_ok(q);
            post.out0 = nullptr;
        }
        const hipError_t e = run(q, s);
        if (e != hipSuccess) return e;
        return epilogue_run(post, static_cast<const uint16_t *>(src), ldsrc, static_cast<uint16_t *>(p.c), p.ldc, p.m,
                            p.n, s);
    }
    if (const int splits = mid_split_route(pr); splits > 1) {
        Problem q = pr;
        q.splits = splits;
        q.out = CT_F32;
        // Up to 128 rows, dense operands run the split on 128 x 128 tiles (two workgroups
        // per CU, none of the 256-row tile's padding rows): the same splits and sums, 9-14%
        // faster for the loss's d hidden at 65-128 rows (measured on MI355X). NF4 operands
        // keep the 256 x 256 runner, the only one with a fused NF4 loader for fp32 partials.
        const bool packed = is_nf4_host(pr.src[0]) || is_nf4_host(pr.src[1]) || is_nf4_host(pr.src[2]) ||
                            is_nf4_host(pr.src[3]);
        q.tile = (p.m <= 128 && !packed) ? TILE_128 : TILE_256;
        q.ws = nullptr;
        q.ws_bytes = 0;
        q.p.c = pr.ws;
        q.p.ldc = p.n;
        q.p.split_stride = p.m * p.n;
        q.p.beta = 0;
        q.p.bias = nullptr;
        q.p.epi.kind = CT_EPI_NONE;  // a residual step is applied by the reduction below
        const hipError_t e = run(q, s);
        if (e != hipSuccess) return e;
        const bool res = p.epi.kind == CT_EPI_RESIDUAL;
        return launch_reduce<CT_BF16>(static_cast<const float *>(pr.ws), splits, p.m * p.n, p.m, p.n, p.c, p.ldc,
                                      p.beta, p.bias, s, res ? p.epi.in0 : nullptr, res ? p.epi.ld_in0 : 0);
    }
    if (pr.splits == 1 && pr.out == CT_BF16 && p.m <= 64) {
        // Few rows: the workgroup streams the weight with its 8 waves splitting the reduction.
        const int sa[2] = {pr.src[0], pr.src[2]}, sb[2] = {pr.src[1], pr.src[3]};
        if (skinny_supported(p, sa, sb, pr.out)) {
            const hipError_t e = skinny_run(p, sb, pr.ws, pr.ws_bytes, s);
            if (e != hipErrorNotSupported) return e;
        }
    }
    const int tile = pr.tile >= 0 ? pr.tile : choose_tile(p.m, p.n, pr.splits);
    if (pr.tile < 0 && tile == TILE_256) {
        int64_t head = 0;
        if (column_split(pr, &head)) {
            // The leading columns on 256 x 256 tiles in whole rounds, the rest on the tile
            // their own width takes: the same per-element sums either way.
            Problem lead = pr, rest = pr;
            lead.p.n = head;
            lead.tile = TILE_256;
            rest.p.n = p.n - head;
            rest.p.c = static_cast<uint16_t *>(p.c) + head;
            rest.ws = nullptr;  // unsplit, as the whole grid would run
            rest.ws_bytes = 0;
            if (p.bias) rest.p.bias = p.bias + head;
            for (int g = 0; g < p.nseg; ++g) {
                Operand &b = rest.p.seg[g].b;
                b.p = static_cast<const uint16_t *>(b.p) + (pr.src[2 * g + 1] == SRC_KC ? head * b.ld : head);
            }
            const hipError_t e = run(lead, s);
            return e != hipSuccess ? e : run(rest, s);
        }
    }
    const int64_t tiles = total_tiles(p);
    p.tiles_per_split = cdiv(tiles > 0 ? tiles : 1, pr.splits);
    const bool nf4 = is_nf4_host(pr.src[0]) || is_nf4_host(pr.src[1]);
    // NF4 operands with fp32 output: split partials of the fast 256 x 256 runner only.
    if (nf4 && pr.out != CT_BF16 && !(pr.out == CT_F32 && tile == TILE_256 && fast_ok(pr)))
        return hipErrorInvalidValue;
    switch (CT_LAYOUT(pr.src[0], pr.src[1], pr.src[2], pr.src[3])) {
        case CT_LAYOUT(SRC_KC, SRC_KC, SRC_KC, SRC_KC):
            return launch_vec_out<SRC_KC, SRC_KC, SRC_KC, SRC_KC>(pr, tile, s);
        case CT_LAYOUT(SRC_KC, SRC_KS, SRC_KC, SRC_KS):
            return launch_vec_out<SRC_KC, SRC_KS, SRC_KC, SRC_KS>(pr, tile, s);
        case CT_LAYOUT(SRC_KC, SRC_KC, SRC_KC, SRC_KS):  // dx on the transposed decode
            return launch_vec_out<SRC_KC, SRC_KC, SRC_KC, SRC_KS>(pr, tile, s);
        case CT_LAYOUT(SRC_KS, SRC_KS, SRC_KS, SRC_KS):
            return launch_vec_out<SRC_KS, SRC_KS, SRC_KS, SRC_KS>(pr, tile, s);
        case CT_LAYOUT(SRC_KS, SRC_KC, SRC_KS, SRC_KC):
            return launch_vec_out<SRC_KS, SRC_KC, SRC_KS, SRC_KC>(pr, tile, s);
        case CT_LAYOUT(SRC_KT, SRC_KT, SRC_KT, SRC_KT):
            // Fast runner only, fp32 output, tiles of at least 128 (the parameter gradients).
            if (!fast_ok(pr) || pr.out != CT_F32 || tile == TILE_64) return hipErrorInvalidValue;
            if (tile == TILE_256)
                return launch_cfg_fast<SRC_KT, SRC_KT, SRC_KT, SRC_KT, CT_F32, TILE_256>(pr.p, pr.splits, s);
            return launch_cfg_fast<SRC_KT, SRC_KT, SRC_KT, SRC_KT, CT_F32, TILE_128>(pr.p, pr.splits, s);
        // NF4 loaders keep their own alignment (checked by nf4_fusable); VEC covers the
        // dense operands and the output.
        case CT_LAYOUT(SRC_KC, SRC_NF4, SRC_KC, SRC_KC):
            if (pr.out == CT_F32)
                return launch_cfg_fast<SRC_KC, SRC_NF4, SRC_KC, SRC_KC, CT_F32, TILE_256>(pr.p, pr.splits, s);
            return launch_mode<SRC_KC, SRC_NF4, SRC_KC, SRC_KC, CT_BF16>(pr, tile, s);
        case CT_LAYOUT(SRC_KC, SRC_NF4T, SRC_KC, SRC_KS):
            if (pr.out == CT_F32)
                return launch_cfg_fast<SRC_KC, SRC_NF4T, SRC_KC, SRC_KS, CT_F32, TILE_256>(pr.p, pr.splits, s);
            return launch_mode<SRC_KC, SRC_NF4T, SRC_KC, SRC_KS, CT_BF16>(pr, tile, s);
        default:
            return hipErrorInvalidValue;
    }
}

// Tile and split count for a reduction-heavy GEMM with a small output (dA, dB): enough
// workgroups for about one per CU, at least 8 k-tiles per split, at most 32 splits.
void choose_reduction(int64_t m, int64_t n, int64_t kred, int *tile, int *splits) {
    *tile = (m >= 128 && n >= 128) ? TILE_128 : TILE_64;
    const int64_t e = kTileEdge[*tile];
    const int64_t tiles_out = cdiv(m, e) * cdiv(n, e);
    const int64_t ktiles = cdiv(kred, kBK);
    int64_t s = cdiv(256, tiles_out > 0 ? tiles_out : 1);
    const int64_t cap = ktiles / 8 > 1 ? ktiles / 8 : 1;
    if (s > cap) s = cap;
    if (s > 32) s = 32;
    *splits = (int)(s < 1 ? 1 : s);
}

int64_t split_workspace_bytes(int64_t m, int64_t n, int64_t kred) {
    int tile, s;
    choose_reduction(m, n, kred, &tile, &s);
    return s > 1 ? (int64_t)s * m * n * (int64_t)sizeof(float) : 0;
}

// out (fp32 or bf16) = sum_k A B (+ out), through fixed-order split partials in ws when
// the output alone cannot fill the GPU.
hipError_t run_reduction(Problem pr, void *out, int64_t ldo, int add, void *ws, int64_t ws_bytes,
                         hipStream_t s, int *status) {
    GemmParams &p = pr.p;
    const int64_t kred = p.seg[0].k;
    int tile = pr.tile, splits = pr.splits;
    if (tile < 0 || splits < 1) choose_reduction(p.m, p.n, kred, &tile, &splits);
    *status = 0;
    pr.tile = tile;
    if (splits <= 1) {
        pr.splits = 1;
        p.c = out;
        p.ldc = ldo;
        p.beta = add;
        pr.vec = pr.vec && aligned16(out) && ldo % 8 == 0;
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
    pr.vec = pr.vec && aligned16(ws) && p.n % 8 == 0;
    hipError_t e = run(pr, s);
    if (e != hipSuccess) return e;
    if (final_out == CT_F32)
        return launch_reduce<CT_F32>(static_cast<float *>(ws), splits, p.split_stride, p.m, p.n, out, ldo, add,
                                     nullptr, s);
    return launch_reduce<CT_BF16>(static_cast<float *>(ws), splits, p.split_stride, p.m, p.n, out, ldo, add, nullptr,
                                  s);
}

int to_status(hipError_t e) { return e == hipSuccess ? 0 : (int)e; }

// Workspace a problem can use for split partials: few rows (the skinny kernels) or the
// split route (mid_splits). Only the shapes and source kinds matter, so the operands need
// not exist yet.
int64_t problem_workspace(int64_t m, int64_t n, const int64_t k[2], int nseg, const int src_b[2]) {
    if (m > 64) {
        const int s = mid_splits(m, n, k[0] + (nseg > 1 ? k[1] : 0));
        return s > 1 ? (int64_t)s * m * n * 4 : 0;
    }
    if (m < 1 || n < 1) return 0;
    GemmParams p{};
    p.m = m;
    p.n = n;
    p.nseg = nseg;
    for (int s = 0; s < nseg; ++s) p.seg[s].k = k[s];
    return skinny_workspace_bytes(p, src_b);
}

int log2_of(int64_t v) {
    if (v <= 0 || (v & (v - 1))) return -1;
    int l = 0;
    while ((int64_t{1} << l) < v) ++l;
    return l;
}

Operand dense(const void *p, int64_t ld) {
    Operand o{};
    o.p = p;
    o.ld = ld;
    return o;
}

Operand nf4_operand(const ct_nf4_weight *w) {
    Operand o{};
    o.p = w->packed;
    o.ld = w->cols;
    o.absmax = w->absmax;
    o.absmax2 = w->absmax2;
    o.offset = w->offset;
    o.lb = log2_of(w->blocksize);
    o.lb2 = w->nested ? log2_of(w->blocksize2) : 0;
    o.nested = w->nested;
    return o;
}

// Conditions of the fused NF4 operand loaders: one first-level block per 32-element unit,
// 16-byte aligned packed rows, and a storage type whose rounding to bf16 is a single step.
bool nf4_fusable(const ct_nf4_weight *w) {
    if (validate_nf4(w) != 0) return false;
    if (w->storage_dtype != CT_BF16 && w->storage_dtype != CT_F32) return false;
    if (w->blocksize < 32 || w->cols % 32 != 0) return false;
    return aligned16(w->packed);
}

}  // namespace
}  // namespace ct

using namespace ct;

extern "C" int ct_abi_version(void) { return 13; }

extern "C" const char *ct_status_string(int status) {
    switch (status) {
        case 0: return "success";
        case -CT_EINVAL_POINTER: return "invalid argument: null or misaligned pointer";
        case -CT_EINVAL_SHAPE: return "invalid argument: size or leading dimension out of range";
        case -CT_EINVAL_DTYPE: return "invalid argument: unsupported element type";
        case -CT_EINVAL_BLOCKSIZE: return "invalid argument: unsupported NF4 block size";
        case -CT_EINVAL_WORKSPACE: return "invalid argument: workspace missing or too small";
        case -CT_EINVAL_LAYOUT: return "invalid argument: NF4 weight layout not supported by the fused path";
        default: return status > 0 ? hipGetErrorString((hipError_t)status) : "unknown status";
    }
}

extern "C" int ct_nf4_fused_supported(const ct_nf4_weight *w) { return nf4_fusable(w) ? 1 : 0; }

namespace ct {
namespace {
// Rank-r products (narrow outputs: r columns, or up to 1024 for a group's stacked factors;
// many rows; a reduction of at least 4096): when 128 x 128 tiles give less than one
// workgroup per CU, the reduction is split 2 to 4 ways (about 512 workgroups, two per CU).
// Measured on MI355X: at 8192 rows and 256 columns 20-25% faster than 64-wide tiles for
// reductions of 11008, at 4096 rows 27-40% faster for 8192. Over 2048 the unsplit 64 x 64
// grid is faster (4096 rows: 12.5 against 20.3 us at 256 columns, 24.9 against 30.7 at
// 768, 18.7 against 25.4 at 512).
bool lowrank_split(int64_t m, int64_t n, int64_t k, int *tile, int *splits) {
    if (n > 1024 || m < 4096 || k < 4096) return false;
    const int64_t tiles = cdiv(m, 128) * cdiv(n, 128);
    if (tiles >= 256) return false;
    int64_t s = 512 / tiles;
    *tile = TILE_128;
    *splits = (int)(s < 2 ? 2 : (s > 4 ? 4 : s));
    return true;
}
}  // namespace
}  // namespace ct

extern "C" int64_t ct_gemm_workspace(int64_t m, int64_t n, int64_t k, int32_t trans_a, int32_t trans_b,
                                     int32_t c_dtype) {
    if (trans_a || c_dtype != CT_BF16) return 0;
    int tile, splits;
    if (lowrank_split(m, n, k, &tile, &splits)) return (int64_t)splits * m * n * 4;
    const int64_t ks[2] = {k, 0};
    const int sb[2] = {trans_b ? SRC_KC : SRC_KS, trans_b ? SRC_KC : SRC_KS};
    return problem_workspace(m, n, ks, 1, sb);
}

extern "C" int ct_gemm(const void *a, int64_t lda, int32_t trans_a, const void *b, int64_t ldb, int32_t trans_b,
                       void *c, int64_t ldc, int32_t c_dtype, const void *bias, int32_t beta, int64_t m, int64_t n,
                       int64_t k, void *workspace, int64_t workspace_bytes, hipStream_t stream) {
    if (m < 0 || n < 0 || k < 0) return -CT_EINVAL_SHAPE;
    if (c_dtype != CT_BF16 && c_dtype != CT_F32) return -CT_EINVAL_DTYPE;
    if (m == 0 || n == 0) return 0;
    if (!c || (k > 0 && (!a || !b))) return -CT_EINVAL_POINTER;
    if (ldc < n || lda < (trans_a ? m : k) || ldb < (trans_b ? k : n)) return -CT_EINVAL_SHAPE;
    Problem pr{};
    pr.p.seg[0].a = dense(a, lda);
    pr.p.seg[0].b = dense(b, ldb);
    pr.p.seg[0].k = k;
    pr.p.nseg = 1;
    pr.p.m = m;
    pr.p.n = n;
    pr.p.c = c;
    pr.p.ldc = ldc;
    pr.p.bias = static_cast<const uint16_t *>(bias);
    pr.p.beta = beta;
    pr.src[0] = trans_a ? SRC_KS : SRC_KC;
    pr.src[1] = trans_b ? SRC_KC : SRC_KS;
    pr.out = c_dtype;
    pr.splits = 1;
    pr.tile = -1;
    pr.ws = workspace;
    pr.ws_bytes = workspace ? workspace_bytes : 0;
    pr.vec = vec_ok(pr);
    int tile, splits;
    if (!bias && c_dtype == CT_BF16 && !trans_a && lowrank_split(m, n, k, &tile, &splits) && workspace &&
        workspace_bytes >= (int64_t)splits * m * n * 4) {
        pr.tile = tile;
        pr.splits = splits;
        int status = 0;
        const hipError_t e = run_reduction(pr, c, ldc, beta, workspace, workspace_bytes, stream, &status);
        return status ? status : to_status(e);
    }
    return to_status(run(pr, stream));
}

namespace ct {
namespace {
// dx decodes its weight first from fewer rows than the forward: its loader, which decodes
// the packed weight into the transposed layout, is the slower of the two fused loaders,
// and once the rows need a second 256-row tile (which decodes every weight slice again)
// the transposed decode plus the dense kernel is faster (measured on MI355X at C5's
// shapes: 257 rows 314 -> 275 and 454 -> 290 us, 384 rows 318 -> 284 and 454 -> 305 us;
// at 256 rows the fused loader stays faster, 198 against 233 us). The forward's fused
// loader keeps up to kMaterializeRows (from 257 rows the two orders are within 7% either
// way, one shape each). Both orders give the same results.
constexpr int64_t kMaterializeRowsDx = 257;
// Also decoded first: a weight without double quantization (the fast runner's NF4 loader
// needs the nested state) in a problem that splits its reduction, so that it takes the
// same kernel and summation order as the bf16 weight it decodes to.
bool materialize_nf4(const ct_nf4_weight *w, int64_t m, int64_t n_out, int64_t ktot, int64_t from) {
    return w && (m >= from || (!w->nested && mid_splits(m, n_out, ktot) > 1));
}
// Workspace queries: nf4 is 0 (bf16 weight), 1 (NF4, double-quantized) or 2 (NF4, plain).
bool materialize_kind(int32_t nf4, int64_t m, int64_t n_out, int64_t ktot, int64_t from) {
    return nf4 && (m >= from || (nf4 == 2 && mid_splits(m, n_out, ktot) > 1));
}
int64_t weight_bytes(int64_t n, int64_t k) { return (n * k * 2 + 255) & ~int64_t{255}; }

// Splits the workspace into the materialized bf16 weight and the remainder.
int take_weight(void *&workspace, int64_t &workspace_bytes, int64_t n, int64_t k, void *&wbuf) {
    const int64_t need = weight_bytes(n, k);
    if (!workspace || workspace_bytes < need) return -CT_EINVAL_WORKSPACE;
    wbuf = workspace;
    workspace = static_cast<char *>(workspace) + need;
    workspace_bytes -= need;
    return 0;
}
}  // namespace
}  // namespace ct

namespace ct {
namespace {
// The device view of a caller's epilogue, checked on the host; kind CT_EPI_NONE for null.
int epilogue_params(const ct_epilogue *e, int64_t n, EpiParams *out) {
    *out = EpiParams{};
    if (!e || e->kind == CT_EPI_NONE) return 0;
    switch (e->kind) {
        case CT_EPI_RESIDUAL:
            if (!e->in0) return -CT_EINVAL_POINTER;
            if (e->ld_in0 < n) return -CT_EINVAL_SHAPE;
            break;
        case CT_EPI_SILU:
            if (!e->in0) return -CT_EINVAL_POINTER;
            if (e->ld_in0 < n || (e->out0 && e->ld_out0 < n)) return -CT_EINVAL_SHAPE;
            break;
        case CT_EPI_DSILU:
            if (!e->in0 || !e->in1 || !e->out0 || !e->out1) return -CT_EINVAL_POINTER;
            if (e->ld_in0 < n || e->ld_in1 < n || e->ld_out0 < n || e->ld_out1 < n) return -CT_EINVAL_SHAPE;
            break;
        case CT_EPI_ROPE:
            if (e->head_dim <= 0 || e->head_dim % 2 || n % e->head_dim || e->half < 0 || e->half > e->head_dim / 2 ||
                n >= (int64_t{1} << 31))
                return -CT_EINVAL_SHAPE;
            if (e->half > 0 && (!e->cosine || !e->sine)) return -CT_EINVAL_POINTER;
            if (e->trig_dtype != CT_F32 && e->trig_dtype != CT_F16 && e->trig_dtype != CT_BF16)
                return -CT_EINVAL_DTYPE;
            break;
        default:
            return -CT_EINVAL_LAYOUT;
    }
    out->kind = e->kind;
    out->trig_dtype = e->trig_dtype;
    out->in0 = static_cast<const uint16_t *>(e->in0);
    out->in1 = static_cast<const uint16_t *>(e->in1);
    out->ld_in0 = e->ld_in0;
    out->ld_in1 = e->ld_in1;
    out->out0 = static_cast<uint16_t *>(e->out0);
    out->out1 = static_cast<uint16_t *>(e->out1);
    out->ld_out0 = e->ld_out0;
    out->ld_out1 = e->ld_out1;
    out->cosine = e->cosine;
    out->sine = e->sine;
    out->head_dim = e->head_dim;
    out->half = e->half;
    bool vec = true;
    const void *side[4] = {e->in0, e->in1, e->out0, e->out1};
    const int64_t ld[4] = {e->ld_in0, e->ld_in1, e->ld_out0, e->ld_out1};
    for (int i = 0; i < 4; ++i)
        if (side[i] && (reinterpret_cast<uintptr_t>(side[i]) % 16 || ld[i] % 8)) vec = false;
    out->vec = vec;
    if (e->kind == CT_EPI_ROPE) {
        const int64_t unit = e->trig_dtype == CT_F32 ? 16 : 8;  // 4 table values
        out->rope_vec = e->head_dim % 8 == 0 && e->half % 4 == 0 &&
                        reinterpret_cast<uintptr_t>(e->cosine) % unit == 0 &&
                        reinterpret_cast<uintptr_t>(e->sine) % unit == 0;
    }
    return 0;
}
}  // namespace
}  // namespace ct

extern "C" int64_t ct_forward_linear_workspace(int64_t m, int64_t n, int64_t k, int64_t r, int32_t nf4) {
    const int64_t inner = ct_gemm_workspace(m, r, k, 0, 1, CT_BF16);
    const int64_t ks[2] = {k, r};
    const int sb[2] = {SRC_NF4, SRC_KC};  // the dense weight (KC) has the same split shape
    const int64_t main = problem_workspace(m, n, ks, r > 0 ? 2 : 1, sb);
    const int64_t rest = inner > main ? inner : main;  // the two launches run in order on one stream
    return materialize_kind(nf4, m, n, k + r, kMaterializeRows) ? weight_bytes(n, k) + rest : rest;
}

extern "C" int ct_forward_linear(const void *x, int64_t ldx, const void *w_dense, const ct_nf4_weight *w_nf4,
                                 const void *a, const void *b, const void *bias, void *out, int64_t ldo, void *xa,
                                 int64_t ldxa, int32_t xa_given, int64_t m, int64_t n, int64_t k, int64_t r,
                                 const ct_epilogue *epilogue, void *workspace, int64_t workspace_bytes,
                                 hipStream_t stream) {
    if (m < 0 || n < 0 || k < 0 || r < 0) return -CT_EINVAL_SHAPE;
    if (m == 0 || n == 0) return 0;
    EpiParams epi;
    if (const int st = epilogue_params(epilogue, n, &epi)) return st;
    if (!x || !out || (!w_dense == !w_nf4) || (r > 0 && (!b || !xa || (!xa_given && !a)))) return -CT_EINVAL_POINTER;
    if (ldx < k || ldo < n || (r > 0 && ldxa < r)) return -CT_EINVAL_SHAPE;
    if (w_nf4) {
        const int st = validate_nf4(w_nf4);
        if (st) return st;
        if (w_nf4->rows != n || w_nf4->cols != k) return -CT_EINVAL_SHAPE;
        if (materialize_nf4(w_nf4, m, n, k + r, kMaterializeRows)) {
            void *wbuf = nullptr;
            const int ws = take_weight(workspace, workspace_bytes, n, k, wbuf);
            if (ws) return ws;
            const int dq = ct_nf4_dequant(w_nf4, wbuf, CT_BF16, stream);
            if (dq) return dq;
            w_dense = wbuf;
            w_nf4 = nullptr;
        } else if (!nf4_fusable(w_nf4)) {
            return -CT_EINVAL_LAYOUT;
        }
    }
    if (r > 0 && !xa_given) {
        // xa = x a^T  (NT, bf16 out)
        const int slot = profile_open(CT_PROF_LOWRANK, stream);
        const int st = ct_gemm(x, ldx, 0, a, k, 1, xa, ldxa, CT_BF16, nullptr, 0, m, r, k, workspace,
                               workspace_bytes, stream);
        profile_close(slot, stream, 2.0 * m * r * k);
        if (st) return st;
    }
    Problem pr{};
    pr.p.seg[0].a = dense(x, ldx);
    pr.p.seg[0].b = w_nf4 ? nf4_operand(w_nf4) : dense(w_dense, k);
    pr.p.seg[0].k = k;
    pr.p.seg[1].a = dense(xa, ldxa);
    pr.p.seg[1].b = dense(b, r);
    pr.p.seg[1].k = r;
    pr.p.nseg = r > 0 ? 2 : 1;
    pr.p.m = m;
    pr.p.n = n;
    pr.p.c = out;
    pr.p.ldc = ldo;
    pr.p.bias = static_cast<const uint16_t *>(bias);
    pr.p.beta = 0;
    pr.p.epi = epi;
    pr.p.code = w_nf4 ? w_nf4->code : nullptr;
    pr.p.code2 = (w_nf4 && w_nf4->nested) ? w_nf4->code2 : nullptr;
    pr.src[0] = SRC_KC;
    pr.src[1] = w_nf4 ? SRC_NF4 : SRC_KC;
    pr.src[2] = SRC_KC;
    pr.src[3] = SRC_KC;
    pr.out = CT_BF16;
    pr.splits = 1;
    pr.tile = -1;
    pr.ws = workspace;
    pr.ws_bytes = workspace ? workspace_bytes : 0;
    pr.vec = vec_ok(pr);
    const int slot = profile_open(CT_PROF_FWD_GEMM, stream);
    const hipError_t e = run(pr, stream);
    profile_close(slot, stream, 2.0 * m * n * (double)(k + r));
    return to_status(e);
}

extern "C" int64_t ct_group_forward_workspace(int64_t m, int32_t count, const int64_t *n, int64_t k, int64_t r) {
    if (m <= 0 || k <= 0 || count != 2 || !n || n[0] <= 0 || n[1] <= 0) return 0;
    return weight_bytes(n[0] + n[1], k);
}

extern "C" int ct_group_forward(const void *x, int64_t ldx, int32_t count, const int64_t *n,
                                const void *const *w_dense, const ct_nf4_weight *const *w_nf4, const void *b_stack,
                                const void *xa, int64_t ldxa, const void *const *bias, void *const *out,
                                const int64_t *ldo, int64_t m, int64_t k, int64_t r, void *workspace,
                                int64_t workspace_bytes, hipStream_t stream) {
    if (count != 2 || !n || !out || !ldo) return -CT_EINVAL_SHAPE;
    if (m < 0 || k < 0 || r < 0 || n[0] <= 0 || n[1] <= 0) return -CT_EINVAL_SHAPE;
    if (m == 0) return 0;
    // the second projection starts on a tile boundary (of the 64 x 64 tiles at least)
    if (n[0] % 64 || k % 8 || (r > 0 && ldxa < 2 * r)) return -CT_EINVAL_SHAPE;
    // The few-row kernels do not take the column switch: the caller runs the projections
    // one by one (refused before any work is queued).
    if (m <= 64) return -CT_EINVAL_SHAPE;
    if (!x || !out[0] || !out[1] || (r > 0 && (!xa || !b_stack))) return -CT_EINVAL_POINTER;
    if (ldx < k || ldo[0] < n[0] || ldo[1] < n[1]) return -CT_EINVAL_SHAPE;
    if (k == 0) return -CT_EINVAL_SHAPE;
    const int64_t nt = n[0] + n[1];
    for (int i = 0; i < 2; ++i) {
        const void *wd = w_dense ? w_dense[i] : nullptr;
        const ct_nf4_weight *wq = w_nf4 ? w_nf4[i] : nullptr;
        if (!wd == !wq) return -CT_EINVAL_POINTER;
        if (wq) {
            if (const int st = validate_nf4(wq)) return st;
            if (wq->rows != n[i] || wq->cols != k) return -CT_EINVAL_SHAPE;
        }
    }
    // [w_1; w_2] decoded (or copied) row by row into the workspace: one [n_total, k] operand
    void *wbuf = nullptr;
    if (const int st = take_weight(workspace, workspace_bytes, nt, k, wbuf)) return st;
    for (int i = 0; i < 2; ++i) {
        uint16_t *dst = static_cast<uint16_t *>(wbuf) + (i ? n[0] * k : 0);
        if (w_nf4 && w_nf4[i]) {
            if (const int st = ct_nf4_dequant(w_nf4[i], dst, CT_BF16, stream)) return st;
        } else {
            const hipError_t e = hipMemcpyAsync(dst, w_dense[i], (size_t)(n[i] * k * 2), hipMemcpyDeviceToDevice,
                                                stream);
            if (e != hipSuccess) return to_status(e);
        }
    }
    Problem pr{};
    pr.p.seg[0].a = dense(x, ldx);
    pr.p.seg[0].b = dense(wbuf, k);
    pr.p.seg[0].k = k;
    pr.p.seg[1].a = dense(xa, ldxa);
    pr.p.seg[1].b = dense(b_stack, r);
    pr.p.seg[1].k = r;
    pr.p.nseg = r > 0 ? 2 : 1;
    pr.p.m = m;
    pr.p.n = nt;
    pr.p.c = out[0];
    pr.p.ldc = ldo[0];
    pr.p.alt_col = n[0];
    pr.p.alt_a1 = r;
    pr.p.c_alt = out[1];
    pr.p.ldc_alt = ldo[1];
    pr.p.bias = bias ? static_cast<const uint16_t *>(bias[0]) : nullptr;
    pr.p.bias_alt = bias ? static_cast<const uint16_t *>(bias[1]) : nullptr;
    pr.src[0] = pr.src[1] = pr.src[2] = pr.src[3] = SRC_KC;
    pr.out = CT_BF16;
    pr.splits = 1;
    // The tile the whole output would take, or the largest smaller one on whose edge the
    // second projection starts.
    int tile = choose_tile(m, nt, 1);
    while (tile < TILE_64 && n[0] % kTileEdge[tile]) ++tile;
    pr.tile = tile;
    // Without a workspace the split route is not taken: the tiled kernels only.
    pr.ws = nullptr;
    pr.ws_bytes = 0;
    pr.vec = vec_ok(pr) && aligned16(out[1]) && ldo[1] % 8 == 0;
    const int slot = profile_open(CT_PROF_FWD_GEMM, stream);
    const hipError_t e = run(pr, stream);
    profile_close(slot, stream, 2.0 * m * nt * (double)(k + r));
    return to_status(e);
}

extern "C" int64_t ct_input_gradient_workspace(int64_t m, int64_t n, int64_t k, int64_t r, int32_t nf4) {
    const int64_t inner = ct_gemm_workspace(m, r, n, 0, 0, CT_BF16);
    const int64_t ks[2] = {n, r};
    const int sb[2] = {SRC_NF4T, SRC_KS};
    const int64_t main = problem_workspace(m, k, ks, r > 0 ? 2 : 1, sb);
    const int64_t rest = inner > main ? inner : main;
    // Many rows: the decoded weight (transposed) comes first.
    return materialize_kind(nf4, m, k, n + r, kMaterializeRowsDx) ? weight_bytes(n, k) + rest : rest;
}

extern "C" int ct_input_gradient(const void *dy, int64_t lddy, const void *w_dense, const ct_nf4_weight *w_nf4,
                                 const void *a, const void *b, void *dx, int64_t lddx, void *low, int64_t m,
                                 int64_t n, int64_t k, int64_t r, int32_t add, const ct_epilogue *epilogue,
                                 void *workspace, int64_t workspace_bytes, hipStream_t stream) {
    if (m < 0 || n < 0 || k < 0 || r < 0) return -CT_EINVAL_SHAPE;
    if (m == 0 || k == 0) return 0;
    EpiParams epi;
    if (const int st = epilogue_params(epilogue, k, &epi)) return st;
    if (epi.kind != CT_EPI_NONE && add) return -CT_EINVAL_LAYOUT;
    if (!dy || !dx || (!w_dense == !w_nf4) || (r > 0 && (!a || !b || !low))) return -CT_EINVAL_POINTER;
    if (lddy < n || lddx < k) return -CT_EINVAL_SHAPE;
    const void *w_trans = nullptr;  // w^T [k, n] in the workspace
    if (w_nf4) {
        const int st = validate_nf4(w_nf4);
        if (st) return st;
        if (w_nf4->rows != n || w_nf4->cols != k) return -CT_EINVAL_SHAPE;
        if (materialize_nf4(w_nf4, m, k, n + r, kMaterializeRowsDx)) {
            void *wbuf = nullptr;
            const int ws = take_weight(workspace, workspace_bytes, n, k, wbuf);
            if (ws) return ws;
            if (nf4_transposable(w_nf4)) {
                // Decode w^T [k, n]: the main segment then runs reduction-contiguous on both
                // operands, on the forward GEMM's kernel; a [r, k] enters the short second
                // segment through the transposing loader.
                const hipError_t dq = nf4_dequant_transposed(w_nf4, wbuf, stream);
                if (dq != hipSuccess) return to_status(dq);
                w_trans = wbuf;
            } else {
                const int dq = ct_nf4_dequant(w_nf4, wbuf, CT_BF16, stream);
                if (dq) return dq;
                w_dense = wbuf;
            }
            w_nf4 = nullptr;
        } else if (!nf4_fusable(w_nf4)) {
            return -CT_EINVAL_LAYOUT;
        }
    }
    if (r > 0) {
        // low = dy b  (NN, bf16 out)
        const int slot = profile_open(CT_PROF_LOWRANK, stream);
        const int st = ct_gemm(dy, lddy, 0, b, r, 0, low, r, CT_BF16, nullptr, 0, m, r, n, workspace,
                               workspace_bytes, stream);
        profile_close(slot, stream, 2.0 * m * r * n);
        if (st) return st;
    }
    Problem pr{};
    pr.p.seg[0].a = dense(dy, lddy);
    pr.p.seg[0].b = w_nf4 ? nf4_operand(w_nf4) : (w_trans ? dense(w_trans, n) : dense(w_dense, k));
    pr.p.seg[0].k = n;
    pr.p.seg[1].a = dense(low, r);
    pr.p.seg[1].b = dense(a, k);
    pr.p.seg[1].k = r;
    pr.p.nseg = r > 0 ? 2 : 1;
    pr.p.m = m;
    pr.p.n = k;
    pr.p.c = dx;
    pr.p.ldc = lddx;
    pr.p.beta = add;
    pr.p.epi = epi;
    pr.p.code = w_nf4 ? w_nf4->code : nullptr;
    pr.p.code2 = (w_nf4 && w_nf4->nested) ? w_nf4->code2 : nullptr;
    pr.src[0] = SRC_KC;
    pr.src[1] = w_nf4 ? SRC_NF4T : (w_trans ? SRC_KC : SRC_KS);
    pr.src[2] = SRC_KC;
    pr.src[3] = SRC_KS;
    pr.out = CT_BF16;
    pr.splits = 1;
    pr.tile = -1;
    pr.ws = workspace;
    pr.ws_bytes = workspace ? workspace_bytes : 0;
    pr.vec = vec_ok(pr);
    const int slot = profile_open(CT_PROF_DX_GEMM, stream);
    const hipError_t e = run(pr, stream);
    profile_close(slot, stream, 2.0 * m * k * (double)(n + r));
    return to_status(e);
}

namespace ct {
namespace {
// out[c][r] = in[r][c] for a bf16 [rows, cols] matrix (pitches ldin, ldo): 64 x 64 tiles
// through LDS, the padded row keeping the column reads free of bank conflicts.
__global__ __launch_bounds__(256) void transpose_bf16(const uint16_t *__restrict__ in, int64_t ldin, int64_t rows,
                                                      int64_t cols, uint16_t *__restrict__ out, int64_t ldo) {
    __shared__ uint16_t tile[64][66];
    const int64_t r0 = (int64_t)blockIdx.y * 64, c0 = (int64_t)blockIdx.x * 64;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    for (int i = ty; i < 64; i += 4)
        if (r0 + i < rows && c0 + tx < cols) tile[i][tx] = in[(r0 + i) * ldin + c0 + tx];
    __syncthreads();
    for (int i = ty; i < 64; i += 4)
        if (c0 + i < cols && r0 + tx < rows) out[(c0 + i) * ldo + r0 + tx] = tile[tx][i];
}

// Reduction widths of a projection group's dx: n_total (the side-by-side upstream
// gradients) and r_total (the stacked ranks), or -1 for an invalid description.
int group_widths(int32_t count, const int64_t *n, const int64_t *r, int64_t *n_total, int64_t *r_total) {
    if (count < 1 || count > CT_GROUP_MAX || !n || !r) return -1;
    *n_total = *r_total = 0;
    for (int i = 0; i < count; ++i) {
        if (n[i] <= 0 || r[i] < 0) return -1;
        *n_total += n[i];
        *r_total += r[i];
    }
    return 0;
}
}  // namespace
}  // namespace ct

extern "C" int64_t ct_group_input_gradient_workspace(int64_t m, int32_t count, const int64_t *n, const int64_t *r,
                                                     int64_t k) {
    int64_t nt, rt;
    if (m <= 0 || k <= 0 || group_widths(count, n, r, &nt, &rt)) return 0;
    int64_t low = 0;
    for (int i = 0; i < count; ++i) {
        const int64_t w = r[i] > 0 ? ct_gemm_workspace(m, r[i], n[i], 0, 0, CT_BF16) : 0;
        low = w > low ? w : low;
    }
    const int64_t ks[2] = {nt, rt};
    const int sb[2] = {SRC_KC, SRC_KS};
    const int64_t main = problem_workspace(m, k, ks, rt > 0 ? 2 : 1, sb);
    return weight_bytes(nt, k) + (low > main ? low : main);
}

extern "C" int ct_group_input_gradient(const void *dy, int64_t lddy, int32_t count, const int64_t *n,
                                       const int64_t *r, const void *const *w_dense,
                                       const ct_nf4_weight *const *w_nf4, const void *a_stack, const void *const *b,
                                       void *dx, int64_t lddx, void *low, int64_t ldlow, int64_t m, int64_t k,
                                       int32_t add, void *workspace, int64_t workspace_bytes, hipStream_t stream) {
    int64_t nt, rt;
    if (m < 0 || k < 0 || group_widths(count, n, r, &nt, &rt)) return -CT_EINVAL_SHAPE;
    if (m == 0 || k == 0) return 0;
    if (!dy || !dx || (rt > 0 && (!a_stack || !low || !b))) return -CT_EINVAL_POINTER;
    if (lddy < nt || lddx < k || (rt > 0 && ldlow < rt)) return -CT_EINVAL_SHAPE;
    // Every projection's w^T goes side by side into the workspace: [k, n_total], 16-byte
    // aligned columns, so the whole group's base product is one reduction-contiguous operand.
    if (nt % 8) return -CT_EINVAL_SHAPE;
    for (int i = 0; i < count; ++i) {
        const void *wd = w_dense ? w_dense[i] : nullptr;
        const ct_nf4_weight *wq = w_nf4 ? w_nf4[i] : nullptr;
        if (!wd == !wq || n[i] % 8 || (r[i] > 0 && !b[i])) return -CT_EINVAL_POINTER;
        if (wq) {
            if (const int st = validate_nf4(wq)) return st;
            if (wq->rows != n[i] || wq->cols != k) return -CT_EINVAL_SHAPE;
            if (!nf4_transposable(wq)) return -CT_EINVAL_LAYOUT;
        }
    }
    void *wbuf = nullptr;
    if (const int st = take_weight(workspace, workspace_bytes, nt, k, wbuf)) return st;
    int64_t col = 0;
    for (int i = 0; i < count; ++i) {
        uint16_t *dst = static_cast<uint16_t *>(wbuf) + col;
        hipError_t e;
        if (w_nf4 && w_nf4[i]) {
            e = nf4_dequant_transposed(w_nf4[i], dst, stream, nt);
        } else {
            transpose_bf16<<<dim3((unsigned)cdiv(k, 64), (unsigned)cdiv(n[i], 64)), 256, 0, stream>>>(
                static_cast<const uint16_t *>(w_dense[i]), k, n[i], k, dst, nt);
            e = hipGetLastError();
        }
        if (e != hipSuccess) return to_status(e);
        col += n[i];
    }
    // low_i = dy_i b_i into low's columns
    col = 0;
    int64_t rcol = 0;
    for (int i = 0; i < count; ++i) {
        if (r[i] > 0) {
            const int slot = profile_open(CT_PROF_LOWRANK, stream);
            const int st = ct_gemm(static_cast<const uint16_t *>(dy) + col, lddy, 0, b[i], r[i], 0,
                                   static_cast<uint16_t *>(low) + rcol, ldlow, CT_BF16, nullptr, 0, m, r[i], n[i],
                                   workspace, workspace_bytes, stream);
            profile_close(slot, stream, 2.0 * m * r[i] * n[i]);
            if (st) return st;
        }
        col += n[i];
        rcol += r[i];
    }
    // dx (+)= [dy | low] [W^T ; a_stack]: one contraction over n_total + r_total columns
    Problem pr{};
    pr.p.seg[0].a = dense(dy, lddy);
    pr.p.seg[0].b = dense(wbuf, nt);
    pr.p.seg[0].k = nt;
    pr.p.seg[1].a = dense(low, ldlow);
    pr.p.seg[1].b = dense(a_stack, k);
    pr.p.seg[1].k = rt;
    pr.p.nseg = rt > 0 ? 2 : 1;
    pr.p.m = m;
    pr.p.n = k;
    pr.p.c = dx;
    pr.p.ldc = lddx;
    pr.p.beta = add;
    pr.src[0] = SRC_KC;
    pr.src[1] = SRC_KC;
    pr.src[2] = SRC_KC;
    pr.src[3] = SRC_KS;
    pr.out = CT_BF16;
    pr.splits = 1;
    pr.tile = -1;
    pr.ws = workspace;
    pr.ws_bytes = workspace ? workspace_bytes : 0;
    pr.vec = vec_ok(pr);
    const int slot = profile_open(CT_PROF_DX_GEMM, stream);
    const hipError_t e = run(pr, stream);
    profile_close(slot, stream, 2.0 * m * k * (double)(nt + rt));
    return to_status(e);
}

// The workspace of ct_group_input_gradient_lead: w_0^T [k, n_0], then the tail's B operand
// [w_1; ...; w_{count-1}; a_stack] [n_tail + r_total, k], then the larger of the low-rank
// products' and the contraction's split partials.
extern "C" int64_t ct_group_input_gradient_lead_workspace(int64_t m, int32_t count, const int64_t *n,
                                                          const int64_t *r, int64_t k) {
    int64_t nt, rt;
    if (m <= 0 || k <= 0 || group_widths(count, n, r, &nt, &rt)) return 0;
    int64_t low = 0;
    for (int i = 0; i < count; ++i) {
        const int64_t w = r[i] > 0 ? ct_gemm_workspace(m, r[i], n[i], 0, 0, CT_BF16) : 0;
        low = w > low ? w : low;
    }
    const int64_t ks[2] = {n[0], nt - n[0] + rt};
    const int sb[2] = {SRC_KC, SRC_KS};
    const int64_t main = problem_workspace(m, k, ks, ks[1] > 0 ? 2 : 1, sb);
    return weight_bytes(n[0], k) + weight_bytes(nt - n[0] + rt, k) + (low > main ? low : main);
}

extern "C" int ct_group_input_gradient_lead(const void *dy0, int64_t lddy0, void *tail, int64_t ldtail,
                                            int32_t count, const int64_t *n, const int64_t *r,
                                            const void *const *w_dense, const ct_nf4_weight *const *w_nf4,
                                            const void *a_stack, const void *const *b, void *dx, int64_t lddx,
                                            int64_t m, int64_t k, int32_t add, void *workspace,
                                            int64_t workspace_bytes, hipStream_t stream) {
    int64_t nt, rt;
    if (m < 0 || k < 0 || group_widths(count, n, r, &nt, &rt)) return -CT_EINVAL_SHAPE;
    if (m == 0 || k == 0) return 0;
    const int64_t n0 = n[0], ntail = nt - n0, kt = ntail + rt;  // the tail's reduction
    if (!dy0 || !dx || (kt > 0 && !tail) || (rt > 0 && (!a_stack || !b))) return -CT_EINVAL_POINTER;
    if (lddy0 < n0 || lddx < k || (kt > 0 && ldtail < kt)) return -CT_EINVAL_SHAPE;
    for (int i = 0; i < count; ++i) {
        const void *wd = w_dense ? w_dense[i] : nullptr;
        const ct_nf4_weight *wq = w_nf4 ? w_nf4[i] : nullptr;
        if (n[i] % 8) return -CT_EINVAL_SHAPE;  // 16-byte aligned column blocks
        if (!wd == !wq || (r[i] > 0 && !b[i])) return -CT_EINVAL_POINTER;
        if (wq) {
            if (const int st = validate_nf4(wq)) return st;
            if (wq->rows != n[i] || wq->cols != k) return -CT_EINVAL_SHAPE;
            if (i == 0 && !nf4_transposable(wq)) return -CT_EINVAL_LAYOUT;
        }
    }
    void *w0buf = nullptr, *wtail = nullptr;
    if (const int st = take_weight(workspace, workspace_bytes, n0, k, w0buf)) return st;
    if (kt > 0)
        if (const int st = take_weight(workspace, workspace_bytes, kt, k, wtail)) return st;
    // w_0^T [k, n_0] for the first projection's reduction-contiguous segment
    if (w_nf4 && w_nf4[0]) {
        if (const hipError_t e = nf4_dequant_transposed(w_nf4[0], w0buf, stream, n0); e != hipSuccess)
            return to_status(e);
    } else {
        transpose_bf16<<<dim3((unsigned)cdiv(k, 64), (unsigned)cdiv(n0, 64)), 256, 0, stream>>>(
            static_cast<const uint16_t *>(w_dense[0]), k, n0, k, static_cast<uint16_t *>(w0buf), n0);
        if (const hipError_t e = hipGetLastError(); e != hipSuccess) return to_status(e);
    }
    // The tail's B operand, rows of its reduction: w_1 .. w_{count-1} in their own layout
    // (w_i [n_i, k]: row j of w_i multiplies column j of dy_i), then a_stack.
    int64_t row = 0;
    for (int i = 1; i < count; ++i) {
        uint16_t *dst = static_cast<uint16_t *>(wtail) + row * k;
        if (w_nf4 && w_nf4[i]) {
            if (const int st = ct_nf4_dequant(w_nf4[i], dst, CT_BF16, stream)) return st;
        } else {
            const hipError_t e = hipMemcpyAsync(dst, w_dense[i], (size_t)(n[i] * k * 2), hipMemcpyDeviceToDevice,
                                                stream);
            if (e != hipSuccess) return to_status(e);
        }
        row += n[i];
    }
    if (rt > 0) {
        const hipError_t e = hipMemcpyAsync(static_cast<uint16_t *>(wtail) + ntail * k, a_stack, (size_t)(rt * k * 2),
                                            hipMemcpyDeviceToDevice, stream);
        if (e != hipSuccess) return to_status(e);
    }
    // low_i = dy_i b_i into the tail's columns after the upstream gradients
    int64_t col = 0, rcol = ntail;
    for (int i = 0; i < count; ++i) {
        if (r[i] > 0) {
            const void *a = i == 0 ? dy0 : static_cast<const void *>(static_cast<const uint16_t *>(tail) + col);
            const int slot = profile_open(CT_PROF_LOWRANK, stream);
            const int st = ct_gemm(a, i == 0 ? lddy0 : ldtail, 0, b[i], r[i], 0, static_cast<uint16_t *>(tail) + rcol,
                                   ldtail, CT_BF16, nullptr, 0, m, r[i], n[i], workspace, workspace_bytes, stream);
            profile_close(slot, stream, 2.0 * m * r[i] * n[i]);
            if (st) return st;
        }
        if (i > 0) col += n[i];
        rcol += r[i];
    }
    // dx (+)= dy_0 w_0^T-segment + tail [w_1; ...; a_stack]: one contraction, rounded once
    Problem pr{};
    pr.p.seg[0].a = dense(dy0, lddy0);
    pr.p.seg[0].b = dense(w0buf, n0);
    pr.p.seg[0].k = n0;
    pr.p.seg[1].a = dense(tail, ldtail);
    pr.p.seg[1].b = dense(wtail, k);
    pr.p.seg[1].k = kt;
    pr.p.nseg = kt > 0 ? 2 : 1;
    pr.p.m = m;
    pr.p.n = k;
    pr.p.c = dx;
    pr.p.ldc = lddx;
    pr.p.beta = add;
    pr.src[0] = SRC_KC;
    pr.src[1] = SRC_KC;
    pr.src[2] = SRC_KC;
    pr.src[3] = SRC_KS;
    pr.out = CT_BF16;
    pr.splits = 1;
    pr.tile = -1;
    pr.ws = workspace;
    pr.ws_bytes = workspace ? workspace_bytes : 0;
    pr.vec = vec_ok(pr);
    const int slot = profile_open(CT_PROF_DX_GEMM, stream);
    const hipError_t e = run(pr, stream);
    profile_close(slot, stream, 2.0 * m * k * (double)(nt + rt));
    return to_status(e);
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
    pr.p.seg[0].a = dense(left, ldl);
    pr.p.seg[0].b = dense(right, ldr);
    pr.p.seg[0].k = j;
    pr.p.nseg = 1;
    pr.p.m = p;
    pr.p.n = q;
    pr.p.c = out;
    pr.p.ldc = ldo;
    pr.src[0] = trans_l ? SRC_KS : SRC_KC;
    pr.src[1] = trans_r ? SRC_KC : SRC_KS;
    pr.out = CT_F32;
    pr.tile = -1;
    pr.vec = vec_ok(pr);
    int st = 0;
    hipError_t e = run_reduction(pr, out, ldo, add, workspace, workspace_bytes, stream, &st);
    return st ? st : to_status(e);
}

namespace ct {
namespace {
// One launch computes dA = low^T x ([r, k]) and dB^T = xa^T dy ([r, n]) side by side: the
// output is r rows by gt * e + n columns (gt column tiles for dA), the token reduction is
// split so that the grid holds about one workgroup per CU, and reduce_param sums the
// splits in order (bit-identical across calls) and writes dB transposed.
struct ParamPlan {
    int tile, splits, gt;
    int64_t width;
};
ParamPlan param_plan(int64_t m, int64_t n, int64_t k, int64_t r) {
    ParamPlan pl{};
    pl.tile = r > 128 ? TILE_256 : (r > 64 ? TILE_128 : TILE_64);
    if (r <= 64 && m <= 512) {
        // Ranks up to 64 over at most 512 tokens (8 k-tiles): one 128 x 128 grid writes dA
        // and dB^T directly, one launch instead of the 64 x 64 grid and the pass that writes
        // dB transposed (C1, 512 tokens, 1024 x 1024 at rank 16: 157 -> 153 us per projection
        // step on the host, the GPU's share 1.5 us longer; measured on MI355X).
        pl.tile = TILE_128;
        pl.gt = (int)cdiv(k, 128);
        pl.width = pl.gt * 128 + n;
        pl.splits = 1;
        return pl;
    }
    if (pl.tile != TILE_64 && m <= 2048) {
        // Few tokens: the reduction is short and writing the fp32 outputs dominates, so
        // smaller tiles spread them over more workgroups (two per CU at 128 x 128) and no
        // split partials are written (measured at 16-1024 tokens: 36 -> 21 us at C5's
        // 6144 x 24576, 33 -> 8.4 us at C1's 1024 x 1024, rank 256).
        const int64_t tiles128 = cdiv(r, 128) * (cdiv(k, 128) + cdiv(n, 128));
        pl.tile = tiles128 >= 128 ? TILE_128 : TILE_64;
        const int64_t e = kTileEdge[pl.tile];
        pl.gt = (int)cdiv(k, e);
        pl.width = pl.gt * e + n;
        pl.splits = 1;
        return pl;
    }
    // Outputs that give the 256 x 256 grid fewer than 32 tiles would need more than 8
    // splits to fill the GPU: 128 x 128 tiles fill it with fewer, shorter partials
    // (measured on MI355X: 2048 x 2048 at 4096 tokens 41.5 -> 30.9 us, the k/v projections'
    // 2048 x 128 at 4096 tokens 35.2 -> 23.3 us, 4096 x 128 at 8192 53.5 -> 47.6 us).
    if (pl.tile == TILE_256 && cdiv(r, 256) * (cdiv(k, 256) + cdiv(n, 256)) < 32) pl.tile = TILE_128;
    const int64_t e = kTileEdge[pl.tile];
    pl.gt = (int)cdiv(k, e);
    pl.width = pl.gt * e + n;
    const int64_t tiles = cdiv(r, e) * (pl.gt + cdiv(n, e));
    const int64_t ktiles = cdiv(m, kBK);
    // At most 8 splits: beyond that the partial sums' traffic costs more than the extra
    // workgroups gain (measured on MI355X at 8192 tokens). At most one workgroup per CU:
    // 128 x 128 tiles run two per CU, and a count just past 256 leaves some CUs with two
    // and the rest with one.
    int64_t s = 256 / (tiles > 0 ? tiles : 1);
    const int64_t cap = ktiles / 8 > 1 ? ktiles / 8 : 1;
    if (s > cap) s = cap;
    if (s > 8) s = 8;
    pl.splits = (int)(s < 1 ? 1 : s);
    return pl;
}
int64_t param_workspace(const ParamPlan &pl, int64_t r) { return (int64_t)pl.splits * r * pl.width * 4; }
}  // namespace
}  // namespace ct

extern "C" int64_t ct_parameter_gradients_workspace(int64_t m, int64_t n, int64_t k, int64_t r) {
    if (m <= 0 || r <= 0 || (n <= 0 && k <= 0)) return 0;
    return param_workspace(param_plan(m, n, k, r), r);
}

extern "C" int ct_parameter_gradients(const void *x, int64_t ldx, const void *dy, int64_t lddy, const void *low,
                                      int64_t ldlow, const void *xa, int64_t ldxa, float *da, float *db, int64_t m,
                                      int64_t n, int64_t k, int64_t r, int32_t add, void *workspace,
                                      int64_t workspace_bytes, hipStream_t stream) {
    if (m < 0 || n < 0 || k < 0 || r < 0) return -CT_EINVAL_SHAPE;
    if (r == 0 || (n == 0 && k == 0)) return 0;
    if ((k > 0 && !da) || (n > 0 && !db)) return -CT_EINVAL_POINTER;
    if (m == 0) {  // empty reduction: zero gradients (or unchanged with add)
        if (add) return 0;
        if (k) fill_zero<<<(unsigned)cdiv(r * k, 256), 256, 0, stream>>>(da, r * k);
        if (n) fill_zero<<<(unsigned)cdiv(n * r, 256), 256, 0, stream>>>(db, n * r);
        return to_status(hipGetLastError());
    }
    if ((k > 0 && (!x || !low)) || (n > 0 && (!dy || !xa))) return -CT_EINVAL_POINTER;
    if (ldx < k || lddy < n || ldlow < r || ldxa < r) return -CT_EINVAL_SHAPE;
    const ParamPlan pl = param_plan(m, n, k, r);
    if (!workspace || workspace_bytes < param_workspace(pl, r)) return -CT_EINVAL_WORKSPACE;
    const int slot = profile_open(CT_PROF_PARAM, stream);
    Problem pr{};
    // Group 0 (dA): A(i, t) = low[t][i], B(q, t) = x[t][q]; group 1 (dB^T): xa and dy.
    Segment dA{dense(low, ldlow), dense(x, ldx), m}, dB{dense(xa, ldxa), dense(dy, lddy), m};
    if (k > 0 && n > 0) {
        pr.p.seg[0] = dA;
        pr.p.seg[1] = dB;
        pr.p.n = k;
        pr.p.n1 = n;
        pr.p.group_tiles = pl.gt;
    } else {
        pr.p.seg[0] = k > 0 ? dA : dB;
        pr.p.n = k > 0 ? k : n;
    }
    pr.p.nseg = 1;
    pr.p.m = r;
    pr.p.c = workspace;
    pr.p.ldc = pl.width;
    pr.p.split_stride = r * pl.width;
    // One split on the KT path: the kernel writes dA and dB (transposed) itself.
    const bool direct = pl.splits == 1 && k > 0 && n > 0;
    // Both operands are token-major. On the fast path they enter LDS as loaded (KT) and the
    // MFMA fragments come from transpose reads; otherwise the registers transpose them (KS).
    pr.src[0] = pr.src[1] = pr.src[2] = pr.src[3] = SRC_KT;
    pr.out = CT_F32;
    pr.splits = pl.splits;
    pr.tile = pl.tile;
    pr.vec = vec_ok(pr);
    if (pl.tile == TILE_64 || !fast_ok(pr)) {
        pr.src[0] = pr.src[1] = pr.src[2] = pr.src[3] = SRC_KS;
        pr.vec = vec_ok(pr);
    }
    if (direct && pr.src[0] == SRC_KT) {
        pr.p.c = da;
        pr.p.ldc = k;
        pr.p.beta = add;
        pr.p.c1 = db;
        pr.p.ldc1 = r;
        const hipError_t e = run(pr, stream);
        profile_close(slot, stream, 2.0 * m * r * (double)(k + n));
        return to_status(e);
    }
    hipError_t e = run(pr, stream);
    if (e == hipSuccess) {
        const int64_t gcols = k > 0 ? (int64_t)pl.gt * kTileEdge[pl.tile] : 0;
        if (pl.width % 8 == 0 && k % 8 == 0 && r % 8 == 0 && gcols % 64 == 0 && aligned16(workspace) &&
            (k == 0 || aligned16(da)) && (n == 0 || aligned16(db)))
            reduce_param_tiled<<<dim3((unsigned)cdiv(pl.width, 64), (unsigned)cdiv(r, 32)), 256, 0, stream>>>(
                static_cast<const float *>(workspace), pl.splits, r * pl.width, r, pl.width, gcols, k, n, da, db, add);
        else
            reduce_param<<<dim3((unsigned)cdiv(pl.width, 256), (unsigned)r), 256, 0, stream>>>(
                static_cast<const float *>(workspace), pl.splits, r * pl.width, r, pl.width, gcols, k, n, da, db, add);
        e = hipGetLastError();
    }
    profile_close(slot, stream, 2.0 * m * r * (double)(k + n));
    return to_status(e);
}
