// The standalone form of the projection epilogues (epilogue.hpp) over a finished bf16
// product: the pass after the GEMM routes that do not fuse the step (the few-row kernels,
// the split-reduction route, the SiLU steps on 256 x 256 tiles), with the same
// per-element code as the fused one.

#include "epilogue.hpp"

namespace ct {
namespace {

// One lane per 8 consecutive columns of one row (the last group of a row may be shorter);
// `vec`: src and dst are 16-byte aligned with pitches of a multiple of 8.
__global__ __launch_bounds__(256) void epilogue_rows(const EpiParams e, const uint16_t *src, int64_t ldsrc,
                                                     uint16_t *dst, int64_t lddst, int64_t m, int64_t n, int vec) {
    const int64_t groups = (n + 7) / 8;
    const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (g >= groups * m) return;
    const int64_t row = g / groups, col = (g % groups) * 8;
    const int count = n - col < 8 ? (int)(n - col) : 8;
    float y[8];
    load_bf16_run<8>(src + row * ldsrc + col, count, vec, y);
    epilogue_values<8>(e, row, col, count, y);
    store_bf16_run<8>(dst + row * lddst + col, count, vec, y);
}

}  // namespace

hipError_t epilogue_run(const EpiParams &e, const uint16_t *src, int64_t ldsrc, uint16_t *dst, int64_t lddst, int64_t m,
                        int64_t n, hipStream_t stream) {
    if (e.kind == CT_EPI_NONE || m <= 0 || n <= 0) return hipSuccess;
    const int64_t lanes = m * ((n + 7) / 8);
    const int vec = reinterpret_cast<uintptr_t>(src) % 16 == 0 && ldsrc % 8 == 0 &&
                    reinterpret_cast<uintptr_t>(dst) % 16 == 0 && lddst % 8 == 0;
    epilogue_rows<<<dim3((unsigned)cdiv(lanes, 256)), dim3(256), 0, stream>>>(e, src, ldsrc, dst, lddst, m, n, vec);
    return hipGetLastError();
}

}  // namespace ct
