// Operand descriptors and device helpers shared by the projection GEMM kernels
// (gemm.hip: tiled MFMA GEMMs; skinny.hip: few-row GEMMs).
#pragma once

#include "common.hpp"
#include "epilogue.hpp"

namespace ct {

// Operand sources: KC reduction-contiguous bf16; KS output-contiguous bf16 transposed in
// registers on its way to LDS; NF4/NF4T packed weights; KT output-contiguous bf16 stored
// in LDS as loaded (one LDS row per reduction index) and transposed by the fragment reads.
enum Src { SRC_KC = 0, SRC_KS = 1, SRC_NF4 = 2, SRC_NF4T = 3, SRC_KT = 4 };

struct Operand {
    const void *p;        // bf16 elements, or packed NF4 bytes
    int64_t ld;           // bf16: row pitch in elements; NF4: columns of the dense weight
    const void *absmax;   // NF4: u8 codes (nested) or f32 scales
    const float *absmax2; // NF4 nested: second-level scales
    const float *offset;  // NF4 nested: scalar offset
    int32_t lb, lb2;      // NF4: log2 of the first- and second-level block sizes
    int32_t nested;
};

struct Segment {
    Operand a, b;
    int64_t k;  // reduction extent
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
    int tiles_m, tiles_n;
    const float *code;        // NF4 code book [16]
    const float *code2;       // NF4 second-level code book [256]
    float *split_ws;          // few-row kernels: fp32 split partials [splits][m][n]
    // Grouped mode (group_tiles > 0, nseg == 1): column tiles tn >= group_tiles compute a
    // second, independent product seg[1] with n1 columns, stored from output column
    // group_tiles * BN on.
    int group_tiles;
    int64_t n1;
    // Grouped mode with one split: group 1 is written transposed to c1 (element (i, c) at
    // c1[c * ldc1 + i]) instead of next to group 0.
    float *c1;
    int64_t ldc1;
    // Elementwise step on a bf16 output (kind CT_EPI_NONE: none).
    EpiParams epi;
    // Two projections side by side (ct_group_forward; alt_col > 0, a multiple of the
    // launch's tile edge): output columns from alt_col on belong to the second one, whose
    // rank-r term reads segment 1's A operand alt_a1 elements further along its rows, whose
    // bias is bias_alt (bf16 [n - alt_col] or null) and whose output goes to c_alt (ldc_alt)
    // from its column 0. No elementwise step.
    int64_t alt_col;
    int64_t alt_a1;
    void *c_alt;
    int64_t ldc_alt;
    const uint16_t *bias_alt;
};

// ------------------------------------------------------------------ LDS layout and NF4 decode
__device__ __forceinline__ uint4 zero4() { return make_uint4(0, 0, 0, 0); }

// LDS slot (16-byte unit) of chunk `chunk` (0..7) of LDS row `row`. Rows are 128 bytes,
// so a 256-byte line of 16 units holds rows 2L and 2L+1; inside line L the unit index
// (row & 1) * 8 + chunk is XORed with line_swizzle(L) = 2 (L mod 8).
//
// gfx950 serves a ds_read_b128 in four groups of 16 lanes, {0-7, 24-31}, {8-15, 16-23},
// {32-39, 56-63} and {40-47, 48-55}, over 64 four-byte banks, i.e. the 16 units of a
// 256-byte line (measured on MI355X with exec-masked probes: bank = unit mod 16, no
// address hash). A group is conflict-free when its 16 lanes hit 16 distinct units mod 16.
// Every MFMA fragment read takes LDS rows R0 + (l mod 16), R0 a multiple of 16, at chunk
// 4 ks + l / 16; with this swizzle all of them are conflict-free, and since the swizzle
// depends only on l, the fragments of one lane differ by immediate offsets. (A per-row
// XOR of the chunk alone leaves these reads two-way conflicted, halving LDS throughput.)
__device__ __forceinline__ int line_swizzle(int line) { return (line & 7) << 1; }
__device__ __forceinline__ int slot(int row, int chunk) {
    const int line = row >> 1;
    return (line << 4) + ((((row & 1) << 3) | chunk) ^ line_swizzle(line));
}
// Inverse of slot(): the LDS row and chunk stored in unit `s`.
__device__ __forceinline__ void slot_coords(int s, int &row, int &chunk) {
    const int line = s >> 4;
    const int w = (s & 15) ^ line_swizzle(line);
    row = (line << 1) | (w >> 3);
    chunk = w & 7;
}
// LDS row of tile row n for a side whose MFMA fragments give each lane FRAG consecutive
// output columns (lane m of a 16 x (16 FRAG) wave tile holds columns FRAG m .. FRAG m +
// FRAG - 1, so its epilogue stores are contiguous): column FRAG m + j goes to LDS row
// 16 j + m of the wave's block, so fragment j reads 16 consecutive LDS rows. FRAG = 1 is
// the identity.
template <int FRAG>
__device__ __forceinline__ int frag_row(int n) {
    if constexpr (FRAG == 1) return n;
    constexpr int W = 16 * FRAG;
    return (n & ~(W - 1)) | ((n % FRAG) << 4) | ((n % W) / FRAG);
}
template <int FRAG>
__device__ __forceinline__ int frag_row_inv(int s) {
    if constexpr (FRAG == 1) return s;
    constexpr int W = 16 * FRAG;
    return (s & ~(W - 1)) | ((s & 15) * FRAG) | ((s % W) >> 4);
}

// KT tiles: LDS row k holds the COLS output-side elements of reduction index k (COLS * 2
// bytes), its 32-byte segments XORed with kt_swizzle(k). A fragment read (two
// ds_read_b64_tr_b16) has its lanes address rows k0 + 8 (l / 16) + (l % 16) / 4 at
// 32-byte segment columns; under this swizzle those reads are conflict-free (measured on
// MI355X: 117 B/clk per CU, the rate of linear 8-byte reads).
__device__ __forceinline__ int kt_swizzle(int k) { return (k & 3) | (((k >> 3) & 1) << 2); }
template <int COLS>
__device__ __forceinline__ int kt_byte(int k, int e) {
    static_assert(COLS >= 128, "KT tiles need at least 8 segments per row");
    return k * (COLS * 2) + (((e >> 4) ^ kt_swizzle(k)) << 5) + ((e & 15) << 1);
}
typedef short kt_v4s __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) kt_v4s lds_kt_v4s;
// The MFMA operand of 16 output-side elements c0 .. c0+15 and reduction indices
// k0 + 8 (l / 16) + 0..7 from a KT tile: lane i of each 16-lane group receives element
// c0 + i at 4 consecutive k per transpose read.
// k0 must be a multiple of 32: the swizzle of rows k0 + lk (+ 4) then depends on the lane
// alone, so the k0 and second-read parts of the address are immediate offsets.
template <int COLS>
__device__ __forceinline__ uint4 kt_fragment(const uint4 *tile, int c0, int k0, int lane) {
    const int g = lane >> 4, j = lane & 15;
    const int lk = 8 * g + (j >> 2);
    const int base = lk * (COLS * 2) + (((c0 >> 4) ^ kt_swizzle(lk)) << 5) + ((j & 3) << 3);
    const __attribute__((address_space(3))) char *b =
        (const __attribute__((address_space(3))) char *)tile + k0 * (COLS * 2) + base;
    const kt_v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_kt_v4s *)b);
    const kt_v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_kt_v4s *)(b + 4 * (COLS * 2)));
    const uint2 l2 = __builtin_bit_cast(uint2, lo), h2 = __builtin_bit_cast(uint2, hi);
    return make_uint4(l2.x, l2.y, h2.x, h2.y);
}

// Eight nibbles of one packed dword -> eight bf16 (element 2j from the high nibble of byte j).
__device__ __forceinline__ uint4 nf4_decode8(uint32_t d, float s, const float *lds_code) {
    float v[8];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        v[2 * b] = lds_code[(d >> (8 * b + 4)) & 15u] * s;
        v[2 * b + 1] = lds_code[(d >> (8 * b)) & 15u] * s;
    }
    return make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                      pack_bf16x2(v[6], v[7]));
}

// ------------------------------------------------------------------ buffer loads
// Raw buffer loads: the hardware range check returns zeros past num_records, and an
// invalid lane is pointed past the range, so loops over k need no branches.
constexpr uint32_t kOOB = 0x80000000u;  // a byte offset beyond every buffer range used here

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, int64_t bytes) {
    const int64_t clamped = bytes < 0 ? 0 : (bytes > 0x7fffffff ? 0x7fffffff : bytes);
    // 0x00020000: the raw 32-bit data format word used for gfx9 buffer descriptors.
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)clamped, 0x00020000);
}

__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
__device__ __forceinline__ uint32_t buf_load4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}
__device__ __forceinline__ uint32_t buf_load1(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b8(r, off, 0, 0);
}

// Pack elements (half h) of dwords lo and hi into one dword: lo's in the low half.
__device__ __forceinline__ uint32_t pick16(uint32_t hi, uint32_t lo, int h) {
    return __builtin_amdgcn_perm(hi, lo, h ? 0x07060302u : 0x05040100u);
}

constexpr bool is_nf4_src(int src) { return src == SRC_NF4 || src == SRC_NF4T; }

// Few-row GEMMs (skinny.hip): C[m, n] for m <= 64 with activation operands A (reduction-
// contiguous bf16) and B of any source. Returns hipErrorNotSupported when the problem is
// outside what the skinny kernels take (the caller then uses the tiled kernels).
// With `ws` (fp32, ws_bytes) the reduction may be split across workgroups (partials summed
// in split order); skinny_workspace_bytes() is the size that allows the preferred split.
hipError_t skinny_run(GemmParams p, const int src_b[2], void *ws, int64_t ws_bytes, hipStream_t stream);
int64_t skinny_workspace_bytes(const GemmParams &p, const int src_b[2]);
bool skinny_supported(const GemmParams &p, const int src_a[2], const int src_b[2], int out_dtype);

}  // namespace ct
