// Standalone NF4 dequantization for gfx950: the MI355X replacement of the reference's
// single-launch Triton decoder (kernels/nf4_cuda.py:9-43, `_decode` + `dequantize_nf4`).
//
// Decoding rule (kernels/nf4_cuda.py:16-29), for element e of a weight with N elements:
//   g      = e / blocksize                                         first-level block
//   s[g]   = code2[absmax[g]] * absmax2[g / blocksize2] + offset   nested (fp32 mul, then add)
//          = absmax[g]                                             otherwise
//   byte   = packed[e / 2];  nibble = e even ? byte >> 4 : byte & 15
//   out[e] = out_dtype(storage_dtype(code[nibble] * s[g]))
//
// The vector kernel moves 8 elements per lane per step: a 4-byte load of packed nibbles
// and one 16-byte store (two for fp32 output), each coalesced across the wavefront. The
// 16-entry code book and the 256-entry second-level code book sit in LDS, so every lookup
// is an LDS read whose 16 (resp. 256) fp32 entries occupy distinct banks.

#include "common.hpp"
#include "profile.hpp"

namespace ct {
namespace {

constexpr int kDequantThreads = 256;
constexpr int kChunksPerThread = 4;  // 8-element chunks per lane per launch slot

template <int STORAGE, int OUT>
__device__ __forceinline__ uint32_t encode_pair(float v0, float v1) {
    // Two decoded values -> one 32-bit word of a 16-bit output type, element v0 first. The
    // intermediate rounding to the storage type is skipped when it cannot change the result
    // (same type, or fp32 storage).
    constexpr bool direct = STORAGE == OUT || STORAGE == CT_F32;
    const float r0 = direct ? v0 : round_to_storage<STORAGE>(v0);
    const float r1 = direct ? v1 : round_to_storage<STORAGE>(v1);
    if constexpr (OUT == CT_BF16) return pack_bf16x2(r0, r1);
    else return (uint32_t)f16_bits(r0) | ((uint32_t)f16_bits(r1) << 16);
}

// Vector path: requires N % 8 == 0 and 8 | blocksize (every bitsandbytes block size).
template <bool NESTED, int STORAGE, int OUT>
__global__ __launch_bounds__(kDequantThreads) void nf4_dequant_vec(
    const uint32_t *__restrict__ packed, const void *__restrict__ absmax_ptr,
    const float *__restrict__ code, const float *__restrict__ code2,
    const float *__restrict__ absmax2, const float *__restrict__ offset_ptr,
    void *__restrict__ out, int64_t chunks, int log2_block, int log2_block2) {
    __shared__ float lds_code[16];
    __shared__ float lds_code2[NESTED ? 256 : 1];
    const int tid = threadIdx.x;
    if (tid < 16) lds_code[tid] = code[tid];
    if constexpr (NESTED) lds_code2[tid] = code2[tid];
    __syncthreads();

    float offset = 0.f;
    if constexpr (NESTED) offset = *offset_ptr;
    // Persistent grid (a few workgroups per CU, striding over the weight): measured on
    // MI355X it sustains ~8% more HBM bandwidth than one workgroup per 1024 chunks.
    for (int64_t base = (int64_t)blockIdx.x * (kDequantThreads * kChunksPerThread) + tid; base < chunks;
         base += (int64_t)gridDim.x * (kDequantThreads * kChunksPerThread)) {
    uint32_t word[kChunksPerThread];
    float scale[kChunksPerThread];
#pragma unroll
    for (int j = 0; j < kChunksPerThread; ++j) {
        const int64_t c = base + j * kDequantThreads;
        if (c < chunks) {
            word[j] = __builtin_nontemporal_load(packed + c);
            const int64_t g = (c << 3) >> log2_block;
            if constexpr (NESTED) {
                const uint8_t q = static_cast<const uint8_t *>(absmax_ptr)[g];
                const float decoded = lds_code2[q] * absmax2[g >> log2_block2];
                scale[j] = decoded + offset;  // separately rounded add (no contraction)
            } else {
                scale[j] = static_cast<const float *>(absmax_ptr)[g];
            }
        }
    }
#pragma unroll
    for (int j = 0; j < kChunksPerThread; ++j) {
        const int64_t c = base + j * kDequantThreads;
        if (c >= chunks) continue;
        const uint32_t d = word[j];
        const float s = scale[j];
        float v[8];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            // The products feed f16 conversions only through f16_bits(), which pins them.
            v[2 * b] = lds_code[(d >> (8 * b + 4)) & 15u] * s;
            v[2 * b + 1] = lds_code[(d >> (8 * b)) & 15u] * s;
        }
        if constexpr (OUT == CT_F32) {
            const f32x4 lo = {round_to_storage<STORAGE>(v[0]), round_to_storage<STORAGE>(v[1]),
                              round_to_storage<STORAGE>(v[2]), round_to_storage<STORAGE>(v[3])};
            const f32x4 hi = {round_to_storage<STORAGE>(v[4]), round_to_storage<STORAGE>(v[5]),
                              round_to_storage<STORAGE>(v[6]), round_to_storage<STORAGE>(v[7])};
            f32x4 *o = static_cast<f32x4 *>(out) + 2 * c;
            __builtin_nontemporal_store(lo, o);
            __builtin_nontemporal_store(hi, o + 1);
        } else {
            const u32x4 r = {encode_pair<STORAGE, OUT>(v[0], v[1]), encode_pair<STORAGE, OUT>(v[2], v[3]),
                             encode_pair<STORAGE, OUT>(v[4], v[5]), encode_pair<STORAGE, OUT>(v[6], v[7])};
            __builtin_nontemporal_store(r, static_cast<u32x4 *>(out) + c);
        }
    }
    }
}

// Exchange path (16-bit outputs; N % 32 == 0, blocksize >= 32, 16-byte aligned): each
// lane loads 16 packed bytes (32 elements, one block scale) with one coalesced load,
// decodes them into four 16-byte chunks, and the wave swaps chunks through LDS so that each
// of its four 16-byte store instructions covers 1 KiB of contiguous output. Loading 16
// bytes per lane and storing coalesced chunks is what this layout buys: measured on
// MI355X it moves ~6.3 TB/s, against ~5.5 TB/s for 4-byte loads and ~1.5-3 TB/s when
// each lane stores its own 64 contiguous bytes.
template <bool NESTED, int STORAGE, int OUT>
__global__ __launch_bounds__(kDequantThreads) void nf4_dequant_x(
    const u32x4 *__restrict__ packed, const void *__restrict__ absmax_ptr,
    const float *__restrict__ code, const float *__restrict__ code2,
    const float *__restrict__ absmax2, const float *__restrict__ offset_ptr,
    void *__restrict__ out, int64_t units, int unit_shift, int log2_block2) {
    __shared__ float lds_code[16];
    __shared__ float lds_code2[NESTED ? 256 : 1];
    __shared__ u32x4 exchange[kDequantThreads / 64][256];
    const int tid = threadIdx.x;
    if (tid < 16) lds_code[tid] = code[tid];
    if constexpr (NESTED) lds_code2[tid] = code2[tid];
    __syncthreads();

    const int lane = tid & 63, wave = tid >> 6;
    const int64_t ub = (int64_t)blockIdx.x * kDequantThreads + wave * 64;  // first unit of this wave
    const int64_t u = ub + lane;
    u32x4 w = {0, 0, 0, 0};
    float s = 0.f;
    if (u < units) {
        w = __builtin_nontemporal_load(packed + u);
        const int64_t g = u >> unit_shift;  // block of the unit's 32 elements
        if constexpr (NESTED) {
            const uint8_t q = static_cast<const uint8_t *>(absmax_ptr)[g];
            const float decoded = lds_code2[q] * absmax2[g >> log2_block2];
            s = decoded + *offset_ptr;  // separately rounded add (no contraction)
        } else {
            s = static_cast<const float *>(absmax_ptr)[g];
        }
    }
    u32x4 *x = exchange[wave];
    const uint32_t words[4] = {w[0], w[1], w[2], w[3]};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t d = words[q];
        float v[8];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            v[2 * b] = lds_code[(d >> (8 * b + 4)) & 15u] * s;
            v[2 * b + 1] = lds_code[(d >> (8 * b)) & 15u] * s;
        }
        x[lane * 4 + q] = u32x4{encode_pair<STORAGE, OUT>(v[0], v[1]), encode_pair<STORAGE, OUT>(v[2], v[3]),
                                encode_pair<STORAGE, OUT>(v[4], v[5]), encode_pair<STORAGE, OUT>(v[6], v[7])};
    }
    __builtin_amdgcn_wave_barrier();  // LDS operations of one wave complete in order
    const int64_t chunks = units * 4;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int64_t c = ub * 4 + q * 64 + lane;
        const u32x4 r = x[q * 64 + lane];
        if (c < chunks) __builtin_nontemporal_store(r, static_cast<u32x4 *>(out) + c);
    }
}

// General path: one lane per packed byte, any N (odd tails included).
template <bool NESTED, int STORAGE, int OUT>
__global__ __launch_bounds__(kDequantThreads) void nf4_dequant_any(
    const uint8_t *__restrict__ packed, const void *__restrict__ absmax_ptr,
    const float *__restrict__ code, const float *__restrict__ code2,
    const float *__restrict__ absmax2, const float *__restrict__ offset_ptr,
    void *__restrict__ out, int64_t n, int log2_block, int log2_block2) {
    const int64_t p = (int64_t)blockIdx.x * kDequantThreads + threadIdx.x;
    const int64_t bytes = (n + 1) >> 1;
    if (p >= bytes) return;
    const int64_t e = 2 * p;
    const int64_t g = e >> log2_block;  // 2p and 2p+1 share a block: blocksize is even
    float s;
    if constexpr (NESTED) {
        const uint8_t q = static_cast<const uint8_t *>(absmax_ptr)[g];
        const float decoded = code2[q] * absmax2[g >> log2_block2];
        s = decoded + *offset_ptr;
    } else {
        s = static_cast<const float *>(absmax_ptr)[g];
    }
    const uint8_t byte = packed[p];
    const float v[2] = {as_f32(code[byte >> 4] * s), as_f32(code[byte & 15] * s)};
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        if (e + i >= n) break;
        const float r = round_to_storage<STORAGE>(v[i]);
        if constexpr (OUT == CT_F32) static_cast<float *>(out)[e + i] = r;
        else if constexpr (OUT == CT_BF16) static_cast<uint16_t *>(out)[e + i] = bf16_bits(r);
        else static_cast<uint16_t *>(out)[e + i] = f16_bits(r);
    }
}

// Transposed decode for the dx GEMM: out[c][r] = bf16(W[r][c]) for a [rows, cols] weight
// (cols % 16 == 0, rows % 8 == 0, packed 8-byte aligned, blocksize >= 16). A workgroup
// decodes a 64-row x 128-column tile: lane (p, c) reads 8 packed bytes (16 elements, one
// block scale) of rows 2p and 2p+1, pairs the two rows' values into bf16x2 words and writes
// them to LDS as [column][row pair]; the tile then leaves as 128 output rows of 128
// contiguous bytes. The pair index is XORed with (column / 16 mod 4) * 8, which halves the
// bank conflicts of the 4-byte LDS stores and keeps each 16-byte read contiguous.
template <bool NESTED, int STORAGE>
__global__ __launch_bounds__(kDequantThreads) void nf4_dequant_t(
    const uint8_t *__restrict__ packed, const void *__restrict__ absmax_ptr, const float *__restrict__ code,
    const float *__restrict__ code2, const float *__restrict__ absmax2, const float *__restrict__ offset_ptr,
    uint16_t *__restrict__ out, int64_t rows, int64_t cols, int log2_block, int log2_block2, int64_t ldo) {
    __shared__ float lds_code[16];
    __shared__ float lds_code2[NESTED ? 256 : 1];
    __shared__ uint32_t tile[128][32];
    const int tid = threadIdx.x;
    if (tid < 16) lds_code[tid] = code[tid];
    if constexpr (NESTED) lds_code2[tid] = code2[tid];
    __syncthreads();

    const int64_t r0 = (int64_t)blockIdx.x * 64, c0 = (int64_t)blockIdx.y * 128;
    const int unit = tid & 7, pair = tid >> 3;
    const int64_t col = c0 + 16 * unit;
    float v[2][16];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int64_t row = r0 + 2 * pair + h;
        uint2 d = make_uint2(0, 0);
        float s = 0.f;
        if (row < rows && col < cols) {
            const int64_t e = row * cols + col;
            d = *reinterpret_cast<const uint2 *>(packed + (e >> 1));
            const int64_t g = e >> log2_block;
            if constexpr (NESTED) {
                const uint8_t q = static_cast<const uint8_t *>(absmax_ptr)[g];
                const float decoded = lds_code2[q] * absmax2[g >> log2_block2];
                s = decoded + *offset_ptr;  // separately rounded add (no contraction)
            } else {
                s = static_cast<const float *>(absmax_ptr)[g];
            }
        }
        const uint32_t words[2] = {d.x, d.y};
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            const uint32_t byte = (words[b >> 2] >> (8 * (b & 3))) & 255u;
            v[h][2 * b] = lds_code[byte >> 4] * s;
            v[h][2 * b + 1] = lds_code[byte & 15u] * s;
        }
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int k = 16 * unit + i;
        tile[k][pair ^ ((unit & 3) << 3)] = encode_pair<STORAGE, CT_BF16>(v[0][i], v[1][i]);
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int k = (tid >> 3) + 32 * j, chunk = tid & 7;
        const int64_t oc = c0 + k, orow = r0 + 8 * chunk;
        const u32x4 val = *reinterpret_cast<const u32x4 *>(&tile[k][(4 * chunk) ^ (((k >> 4) & 3) << 3)]);
        if (oc < cols && orow < rows)
            __builtin_nontemporal_store(val, reinterpret_cast<u32x4 *>(out + oc * ldo + orow));
    }
}

int log2_exact(int64_t v) {
    if (v <= 0 || (v & (v - 1))) return -1;
    int l = 0;
    while ((int64_t{1} << l) < v) ++l;
    return l;
}

template <bool NESTED, int STORAGE, int OUT>
hipError_t launch_dequant(const ct_nf4_weight *w, void *out, int64_t n, int lb, int lb2,
                          bool vec, hipStream_t stream) {
    const bool exchange = OUT != CT_F32 && vec && n % 32 == 0 && lb >= 5 &&
                          (reinterpret_cast<uintptr_t>(w->packed) % 16 == 0);
    if (exchange) {
        const int64_t units = n >> 5;
        const int64_t grid = cdiv(units, kDequantThreads);
        nf4_dequant_x<NESTED, STORAGE, OUT><<<dim3((unsigned)grid), dim3(kDequantThreads), 0, stream>>>(
            reinterpret_cast<const u32x4 *>(w->packed), w->absmax, w->code, w->code2, w->absmax2, w->offset, out,
            units, lb - 5, lb2);
    } else if (vec) {
        const int64_t chunks = n >> 3;
        const int64_t per_block = kDequantThreads * kChunksPerThread;
        int device = 0, cus = 256;
        if (hipGetDevice(&device) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess)
            cus = 256;
        const int64_t blocks = cdiv(chunks, per_block);
        const int64_t grid = blocks < 8 * (int64_t)cus ? blocks : 8 * (int64_t)cus;
        nf4_dequant_vec<NESTED, STORAGE, OUT><<<dim3((unsigned)grid), dim3(kDequantThreads), 0, stream>>>(
            reinterpret_cast<const uint32_t *>(w->packed), w->absmax, w->code, w->code2, w->absmax2,
            w->offset, out, chunks, lb, lb2);
    } else {
        const int64_t grid = cdiv((n + 1) >> 1, kDequantThreads);
        nf4_dequant_any<NESTED, STORAGE, OUT><<<dim3((unsigned)grid), dim3(kDequantThreads), 0, stream>>>(
            w->packed, w->absmax, w->code, w->code2, w->absmax2, w->offset, out, n, lb, lb2);
    }
    return hipGetLastError();
}

template <bool NESTED, int STORAGE>
hipError_t dispatch_out(const ct_nf4_weight *w, void *out, int out_dtype, int64_t n, int lb, int lb2,
                        bool vec, hipStream_t s) {
    switch (out_dtype) {
        case CT_BF16: return launch_dequant<NESTED, STORAGE, CT_BF16>(w, out, n, lb, lb2, vec, s);
        case CT_F16: return launch_dequant<NESTED, STORAGE, CT_F16>(w, out, n, lb, lb2, vec, s);
        default: return launch_dequant<NESTED, STORAGE, CT_F32>(w, out, n, lb, lb2, vec, s);
    }
}

template <bool NESTED>
hipError_t dispatch_storage(const ct_nf4_weight *w, void *out, int out_dtype, int64_t n, int lb, int lb2,
                            bool vec, hipStream_t s) {
    switch (w->storage_dtype) {
        case CT_BF16: return dispatch_out<NESTED, CT_BF16>(w, out, out_dtype, n, lb, lb2, vec, s);
        case CT_F16: return dispatch_out<NESTED, CT_F16>(w, out, out_dtype, n, lb, lb2, vec, s);
        default: return dispatch_out<NESTED, CT_F32>(w, out, out_dtype, n, lb, lb2, vec, s);
    }
}

bool valid_dtype(int d) { return d == CT_F32 || d == CT_F16 || d == CT_BF16; }

// Algorithmic HBM bytes of one decode: packed nibbles, first-level scales, second-level
// scales, the code books and the offset read once, and the output written once.
double dequant_bytes(const ct_nf4_weight *w, int64_t n, int out_dtype) {
    const int64_t nb = cdiv(n, w->blocksize);
    double bytes = (double)((n + 1) / 2) + 16 * 4;
    bytes += w->nested ? (double)nb + 4.0 * cdiv(nb, w->blocksize2) + 256 * 4 + 4 : 4.0 * nb;
    bytes += (double)n * (out_dtype == CT_F32 ? 4 : 2);
    return bytes;
}

template <bool NESTED>
hipError_t launch_transposed(const ct_nf4_weight *w, void *out, int64_t ldo, int lb, int lb2, hipStream_t stream) {
    const dim3 grid((unsigned)cdiv(w->rows, 64), (unsigned)cdiv(w->cols, 128));
    switch (w->storage_dtype) {
        case CT_BF16:
            nf4_dequant_t<NESTED, CT_BF16><<<grid, dim3(kDequantThreads), 0, stream>>>(
                w->packed, w->absmax, w->code, w->code2, w->absmax2, w->offset, static_cast<uint16_t *>(out),
                w->rows, w->cols, lb, lb2, ldo);
            break;
        case CT_F16:
            nf4_dequant_t<NESTED, CT_F16><<<grid, dim3(kDequantThreads), 0, stream>>>(
                w->packed, w->absmax, w->code, w->code2, w->absmax2, w->offset, static_cast<uint16_t *>(out),
                w->rows, w->cols, lb, lb2, ldo);
            break;
        default:
            nf4_dequant_t<NESTED, CT_F32><<<grid, dim3(kDequantThreads), 0, stream>>>(
                w->packed, w->absmax, w->code, w->code2, w->absmax2, w->offset, static_cast<uint16_t *>(out),
                w->rows, w->cols, lb, lb2, ldo);
    }
    return hipGetLastError();
}

}  // namespace

// Whether nf4_dequant_transposed takes this weight (validated by validate_nf4 first).
bool nf4_transposable(const ct_nf4_weight *w) {
    return w->cols % 16 == 0 && w->rows % 8 == 0 && w->blocksize >= 16 &&
           reinterpret_cast<uintptr_t>(w->packed) % 8 == 0 && cdiv(w->cols, 128) <= 65535;
}

// bf16 out[cols][ldo] = the transpose of the decoded weight (same values as
// ct_nf4_dequant with CT_BF16 output) in the first `rows` elements of each output row;
// out 16-byte aligned, ldo >= rows and a multiple of 8. Timed with the decoder family.
hipError_t nf4_dequant_transposed(const ct_nf4_weight *w, void *out, hipStream_t stream, int64_t ldo) {
    if (ldo <= 0) ldo = w->rows;
    if (ldo < w->rows || ldo % 8 || reinterpret_cast<uintptr_t>(out) % 16) return hipErrorInvalidValue;
    const int lb = log2_exact(w->blocksize);
    const int lb2 = w->nested ? log2_exact(w->blocksize2) : 0;
    const int slot = profile_open(CT_PROF_DEQUANT, stream);
    const hipError_t e = w->nested ? launch_transposed<true>(w, out, ldo, lb, lb2, stream)
                                   : launch_transposed<false>(w, out, ldo, lb, lb2, stream);
    profile_close(slot, stream, dequant_bytes(w, w->rows * w->cols, CT_BF16));
    return e;
}

// Host-side validation shared with the GEMM entry points.
int validate_nf4(const ct_nf4_weight *w) {
    if (!w || !w->packed || !w->absmax || !w->code) return -CT_EINVAL_POINTER;
    if (w->rows < 0 || w->cols < 0) return -CT_EINVAL_SHAPE;
    if (!valid_dtype(w->storage_dtype)) return -CT_EINVAL_DTYPE;
    if (log2_exact(w->blocksize) < 1) return -CT_EINVAL_BLOCKSIZE;
    if (w->nested) {
        if (!w->code2 || !w->absmax2 || !w->offset) return -CT_EINVAL_POINTER;
        if (log2_exact(w->blocksize2) < 0) return -CT_EINVAL_BLOCKSIZE;
    }
    return 0;
}

}  // namespace ct

extern "C" int ct_nf4_dequant(const ct_nf4_weight *w, void *out, int32_t out_dtype, hipStream_t stream) {
    using namespace ct;
    int st = validate_nf4(w);
    if (st) return st;
    if (!valid_dtype(out_dtype)) return -CT_EINVAL_DTYPE;
    const int64_t n = w->rows * w->cols;
    if (n == 0) return 0;
    if (!out) return -CT_EINVAL_POINTER;
    const int lb = log2_exact(w->blocksize);
    const int lb2 = w->nested ? log2_exact(w->blocksize2) : 0;
    const bool vec = (n % 8 == 0) && w->blocksize >= 8 &&
                     (reinterpret_cast<uintptr_t>(w->packed) % 4 == 0) &&
                     (reinterpret_cast<uintptr_t>(out) % 16 == 0);
    const int slot = profile_open(CT_PROF_DEQUANT, stream);
    hipError_t e = w->nested ? dispatch_storage<true>(w, out, out_dtype, n, lb, lb2, vec, stream)
                             : dispatch_storage<false>(w, out, out_dtype, n, lb, lb2, vec, stream);
    profile_close(slot, stream, dequant_bytes(w, n, out_dtype));
    return e == hipSuccess ? 0 : (int)e;
}
