// The standalone form of the projection epilogues (epilogue.hpp) over a finished bf16
// product: the pass after the GEMM routes that do not fuse the step (the few-row kernels,
// the split-reduction route, the SiLU steps on 256 x 256 tiles), with the same
// per-element code as the fused one.

#include "epilogue.hpp"

namespace ct {
namespace {

// One lane per 8 consecutive columns of a row (the last group of a row may be shorter):
// grid.x covers a row's column groups, grid.y strides over the rows (no index division).
// One instance per kind and access width keeps each kernel's registers to its own step.
// VEC: src and dst are 16-byte aligned with pitches of a multiple of 8.
template <int KIND, bool VEC>
__global__ __launch_bounds__(256) void epilogue_rows(const EpiParams e, const uint16_t *src, int64_t ldsrc,
                                                     uint16_t *dst, int64_t lddst, int64_t m, int64_t n) {
    const int64_t col = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
    if (col >= n) return;
    const int count = n - col < 8 ? (int)(n - col) : 8;
    for (int64_t row = blockIdx.y; row < m; row += gridDim.y) {
        float y[8];
        EpiSide<8> side;
        load_bf16_run<8>(src + row * ldsrc + col, count, VEC, y);
        epilogue_load<KIND, 8>(e, row, col, count, side);
        epilogue_apply<KIND, 8>(e, row, col, count, side, y);
        store_bf16_run<8>(dst + row * lddst + col, count, VEC, y);
    }
}

template <int KIND>
hipError_t launch_rows(const EpiParams &e, const uint16_t *src, int64_t ldsrc, uint16_t *dst, int64_t lddst, int64_t m,
                       int64_t n, bool vec, hipStream_t stream) {
    const int64_t groups = (n + 7) / 8;
    if (cdiv(groups, 256) > 0x7fffffff) return hipErrorInvalidValue;
    const dim3 grid((unsigned)cdiv(groups, 256), (unsigned)(m < 65535 ? m : 65535));
    if (vec) epilogue_rows<KIND, true><<<grid, dim3(256), 0, stream>>>(e, src, ldsrc, dst, lddst, m, n);
    else epilogue_rows<KIND, false><<<grid, dim3(256), 0, stream>>>(e, src, ldsrc, dst, lddst, m, n);
    return hipGetLastError();
}

}  // namespace

hipError_t silu_forward_flat(const uint16_t *gate, const uint16_t *up, uint16_t *h, int64_t n, hipStream_t s);
hipError_t silu_backward_flat(const uint16_t *gate, const uint16_t *up, uint16_t *h, uint16_t *dg, uint16_t *du,
                              int64_t n, hipStream_t s);

hipError_t epilogue_run(const EpiParams &e, const uint16_t *src, int64_t ldsrc, uint16_t *dst, int64_t lddst, int64_t m,
                        int64_t n, hipStream_t stream) {
    if (e.kind == CT_EPI_NONE || m <= 0 || n <= 0) return hipSuccess;
    const bool vec = reinterpret_cast<uintptr_t>(src) % 16 == 0 && ldsrc % 8 == 0 &&
                     reinterpret_cast<uintptr_t>(dst) % 16 == 0 && lddst % 8 == 0;
    // A SiLU step over whole contiguous matrices runs ct_silu_multiply's kernel (the same
    // per-element code): measured on MI355X, the row kernel below ran it slower than that
    // (the backward step over C4's 4096 x 8192 d hidden by 2.4 us).
    if (e.kind == CT_EPI_SILU && !e.out0 && vec && e.vec && ldsrc == n && lddst == n && e.ld_in0 == n &&
        (m * n) % 8 == 0)
        return silu_forward_flat(e.in0, src, dst, m * n, stream);
    if (e.kind == CT_EPI_DSILU && src == dst && vec && e.vec && ldsrc == n && e.ld_in0 == n && e.ld_in1 == n &&
        e.ld_out0 == n && e.ld_out1 == n && (m * n) % 8 == 0)
        return silu_backward_flat(e.in0, e.in1, dst, e.out0, e.out1, m * n, stream);
    switch (e.kind) {
        case CT_EPI_RESIDUAL: return launch_rows<CT_EPI_RESIDUAL>(e, src, ldsrc, dst, lddst, m, n, vec, stream);
        case CT_EPI_SILU: return launch_rows<CT_EPI_SILU>(e, src, ldsrc, dst, lddst, m, n, vec, stream);
        case CT_EPI_DSILU: return launch_rows<CT_EPI_DSILU>(e, src, ldsrc, dst, lddst, m, n, vec, stream);
        case CT_EPI_ROPE: return launch_rows<CT_EPI_ROPE>(e, src, ldsrc, dst, lddst, m, n, vec, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace ct
