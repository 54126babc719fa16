/*
 * C ABI of the MI355X (gfx950) NF4-LoRA projection library `libcausal_tuner_hip.so`.
 *
 * Every entry point takes raw device pointers, element counts, leading dimensions and
 * the caller's HIP stream. The library never allocates or frees device memory and keeps
 * no pointer, tensor or stream between calls; scratch space for split reductions is a
 * caller-owned workspace whose size a `*_workspace` query returns. Kernels are enqueued
 * on `stream` and the call returns without synchronising.
 *
 * Status: 0 on success; a negative CT_E* code for an argument error detected on the host
 * before anything is enqueued; a positive hipError_t if a launch failed. No C++ exception
 * crosses this boundary. `ct_status_string` names a status.
 *
 * Matrices are row-major with unit stride along a row; `ld*` is the distance, in
 * elements, between consecutive rows. bf16 values are passed as `const void *`.
 *
 * Reference interfaces (RealJosephus/causal-tuner, paths under src/causal_tuner/):
 *   kernels/nf4_cuda.py:9-43    _decode / dequantize_nf4   -> ct_nf4_dequant
 *   kernels/linear.py:6-13      materialize                -> ct_nf4_dequant
 *   modeling/lora.py:50-55      bitsandbytes quantize_4bit -> ct_nf4_quantize (+ ct_quantize_blockwise)
 *   kernels/linear.py:16-24     accumulate                 -> ct_accumulate
 *   kernels/linear.py:27-33     forward_linear             -> ct_forward_linear
 *   kernels/linear.py:36-39     input_gradient             -> ct_input_gradient
 *   kernels/linear.py:42-44     parameter_gradients        -> ct_parameter_gradients
 *   kernels/linear.py:84,125    torch.mm(x, a.T, out=xa)   -> ct_gemm (NT, bf16 out)
 *   kernels/linear.py:124,167   torch.mm(dy, b, out=low)   -> ct_gemm (NN, bf16 out)
 *   kernels/mlp_cuda.py:10-35   _activation (SiLU x up)    -> ct_silu_multiply
 *   kernels/core_cuda.py:29-130 RMS (_rms_forward/backward)  -> ct_rms_forward, ct_rms_backward
 *   kernels/loss_cuda.py:11-70  weighted_ce (_statistics)   -> ct_weighted_ce
 *   training/engine.py:10-16    torch fused AdamW step      -> ct_adamw_step
 *   kernels/linear.py:70,108    a.to(dtype), b.to(dtype)    -> ct_cast_f32_bf16 (one launch per group)
 *   kernels/core_cuda.py:133-229 _rope / _owned_qk_rope     -> ct_rope
 *                               (PartialRoPE, inverse_rope_tile, rotate_owned_qk)
 */
#ifndef CAUSAL_TUNER_HIP_H
#define CAUSAL_TUNER_HIP_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types (the torch dtypes the reference passes through these paths). */
#define CT_F32  0
#define CT_F16  1
#define CT_BF16 2

/* Host-side argument errors (returned negated). */
#define CT_EINVAL_POINTER   1  /* a required pointer is null or misaligned       */
#define CT_EINVAL_SHAPE     2  /* a size or leading dimension is out of range    */
#define CT_EINVAL_DTYPE     3  /* unsupported element type                       */
#define CT_EINVAL_BLOCKSIZE 4  /* unsupported NF4 block size                     */
#define CT_EINVAL_WORKSPACE 5  /* workspace missing or smaller than required    */
#define CT_EINVAL_LAYOUT    6  /* NF4 weight layout outside the fused loaders   */

/*
 * Frozen NF4 base weight: the fields of a bitsandbytes QuantState that the reference's
 * decoder reads (kernels/nf4_cuda.py:33-41, kernels/linear.py:8).
 *   packed     uint8 [ceil(rows*cols/2)]: element 2j in the high nibble of byte j.
 *   absmax     nested: uint8 [nb] codes into code2; else float32 [nb] block scales.
 *   code       float32 [16] NF4 code book (state.code).
 *   code2      float32 [256] second-level code book (state.state2.code), nested only.
 *   absmax2    float32 [ceil(nb/blocksize2)] (state.state2.absmax), nested only.
 *   offset     float32 [1] (state.offset), nested only.
 *   rows, cols the dense shape (state.shape), rows = out features.
 *   blocksize  first-level block (64..4096, power of two); blocksize2 second level.
 *   storage_dtype  state.dtype: every decoded value is rounded to it first.
 * nb = ceil(rows*cols/blocksize).
 */
typedef struct ct_nf4_weight {
    const uint8_t *packed;
    const void *absmax;
    const float *code;
    const float *code2;
    const float *absmax2;
    const float *offset;
    int64_t rows;
    int64_t cols;
    int32_t blocksize;
    int32_t blocksize2;
    int32_t nested;
    int32_t storage_dtype;
} ct_nf4_weight;

int ct_abi_version(void);

/*
 * Per-device set-up, once per GPU with that GPU current (idempotent, thread-safe):
 * resolves the device address of the static scratch array that ct_forward_linear_static
 * uses on this GPU, so that no later call runs a runtime symbol query. No counterpart in
 * the reference (its Triton kernels need no set-up). Returns 0 or a hipError_t.
 */
int ct_init_device(void);
const char *ct_status_string(int status);

/*
 * An elementwise step fused into the bf16 output of ct_forward_linear / ct_input_gradient
 * (or run over it right after the GEMM where a route has no fused epilogue; the values are
 * the same). y is the projection's output rounded to bf16 as the reference stores it;
 * tensors are bf16 [m, n] with the given row pitches, indexed like the output.
 *   CT_EPI_RESIDUAL  out = y + in0                          (the o/down-proj residual,
 *                    kernels/linear.py:90-91; kernels/mlp_cuda.py:80)
 *   CT_EPI_SILU      out = bf16(silu(in0)) * y, in0 = gate, y = up; out0 (optional) = y
 *                    (_activation's forward, kernels/mlp_cuda.py:10-35)
 *   CT_EPI_DSILU     y = dh; with g = in0, u = in1: out0 = d gate, out1 = d up and
 *                    out = the hidden activation h (_activation's backward with
 *                    reconstruction, kernels/mlp_cuda.py:131-133); out0/out1 may be in0/in1
 *   CT_EPI_ROPE      the partial GPT-J rotation of _owned_qk_rope (kernels/core_cuda.py:
 *                    133-189): the output is [m, heads, head_dim]; pairs (2c, 2c+1), c < half,
 *                    rotate by cosine/sine [m, half] of trig_dtype, the rest pass through.
 * The entry points require add = 0 (no beta) with an epilogue. in0/in1/out0/out1 must not
 * overlap the main output (the unfused routes store y there before the step reads them).
 */
#define CT_EPI_NONE     0
#define CT_EPI_RESIDUAL 1
#define CT_EPI_SILU     2
#define CT_EPI_DSILU    3
#define CT_EPI_ROPE     4
typedef struct ct_epilogue {
    int32_t kind;
    int32_t trig_dtype;
    const void *in0;
    int64_t ld_in0;
    const void *in1;
    int64_t ld_in1;
    void *out0;
    int64_t ld_out0;
    void *out1;
    int64_t ld_out1;
    const void *cosine;
    const void *sine;
    int64_t head_dim;
    int64_t half;
} ct_epilogue;

/*
 * Replaces dequantize_nf4 / _decode (kernels/nf4_cuda.py:9-43), the NF4 branch of
 * materialize (kernels/linear.py:6-13).
 * out[e] = out_dtype(storage_dtype(code[nibble(e)] * s[e / blocksize])) for e < rows*cols,
 * with s[g] = code2[absmax[g]] * absmax2[g / blocksize2] + offset (fp32 multiply, then a
 * separately rounded add) when nested, else s[g] = absmax[g]. Bit-exact to the reference.
 */
int ct_nf4_dequant(const ct_nf4_weight *w, void *out, int32_t out_dtype, hipStream_t stream);

/*
 * Replaces bitsandbytes' quantize_4bit(quant_type="nf4", compress_statistics=nested) as the
 * reference calls it through Params4bit in Projection.install_nf4 (modeling/lora.py:50-55).
 * w: n values of w_dtype (bf16, f16, f32), quantized in blocks of `blocksize` (a power of
 * two) over the flat order: absmax[g] = max |w| of block g; codes = first of the 15
 * `midpoints` (fp32, between the 16 NF4 code values) >= w * (1 / absmax[g]), NaN -> 15;
 * packed[j] = code[2j] << 4 | code[2j + 1] (ceil(n / 2) bytes, 4-byte aligned, a zero pad
 * nibble for odd n). nested = 0: absmax is fp32 [nb]. nested = 1: offset[0] = fp32 of the
 * float64 mean of the fp32 absmax, absmax - offset is block-quantized in blocks of 256
 * against code2 (the 256-entry signed dynamic map, bitsandbytes' binary search and
 * midpoint rule): absmax is u8 [nb], absmax2 fp32 [ceil(nb / 256)]. The workspace holds the
 * fp32 first-level absmax when nested. Finite inputs assumed (a NaN is not propagated into
 * absmax).
 */
int64_t ct_nf4_quantize_workspace(int64_t n, int32_t blocksize, int32_t nested);
/*
 * Replaces bitsandbytes' quantize_blockwise(absmax - offset, code2, blocksize=256), the
 * second level of quantize_4bit(compress_statistics=True) (called through Params4bit at
 * modeling/lora.py:50-55): c = values[i] - offset[0] in fp32; absmax2[j] = max |c| over
 * block j of 256; codes[i] = the dynamic-map code of c * (1 / absmax2[j]) (bitsandbytes'
 * binary search and midpoint rule over code2, 256 sorted fp32 values). With ct_nf4_quantize
 * run with nested = 0 (fp32 absmax) and offset = the caller's fp32 mean of that absmax (as
 * bitsandbytes computes it, absmax.mean()), the two calls give quantize_4bit's nested state.
 */
int ct_quantize_blockwise(const float *values, int64_t n, const float *offset, const float *code2,
                          uint8_t *codes, float *absmax2, hipStream_t stream);
int ct_nf4_quantize(const void *w, int32_t w_dtype, int64_t n, int32_t blocksize, int32_t nested,
                    const float *midpoints, const float *code2, uint8_t *packed, void *absmax,
                    float *absmax2, float *offset, void *workspace, int64_t workspace_bytes,
                    hipStream_t stream);

/*
 * Replaces the torch.mm / torch.addmm calls of the projection path (kernels/linear.py:28-33,
 * 37-39, 84, 124-125, 167). bf16 operands, fp32 accumulation.
 *   c[m,n] = sum_k A(m,k) B(k,n) (+ bias[n]) (+ c[m,n] if beta)
 *   A(m,k) = a[m*lda + k]  (trans_a = 0)  or  a[k*lda + m]  (trans_a = 1)
 *   B(k,n) = b[n*ldb + k]  (trans_b = 1)  or  b[k*ldb + n]  (trans_b = 0)
 * c_dtype is CT_BF16 (rounded once, RTNE) or CT_F32. bias may be null (bf16 [n]).
 *
 * Workspace (here and in ct_forward_linear / ct_input_gradient): with m <= 64 rows, with
 * 65-511 rows, with a rank-r output (n <= 1024) over many rows and a reduction of at least
 * 4096, and with a reduction of at least 8192 into an output short of one round of
 * 256 x 256 tiles, the reduction may be split across workgroups, the fp32 partials going to the caller's
 * workspace and summed in a fixed order (results do not depend on timing). The *_workspace
 * query gives the size that allows the preferred split; a null or smaller workspace is
 * valid and only splits less (no split at all without one). The partials are written with
 * 16-byte stores, so a workspace that is not 16-byte aligned is treated as absent.
 */
int64_t ct_gemm_workspace(int64_t m, int64_t n, int64_t k, int32_t trans_a, int32_t trans_b, int32_t c_dtype);
int ct_gemm(const void *a, int64_t lda, int32_t trans_a,
            const void *b, int64_t ldb, int32_t trans_b,
            void *c, int64_t ldc, int32_t c_dtype, const void *bias, int32_t beta,
            int64_t m, int64_t n, int64_t k, void *workspace, int64_t workspace_bytes, hipStream_t stream);

/*
 * The same products for a float32 compute dtype (the reference's torch.mm / addmm with
 * float32 operands, kernels/linear.py:16-44, TF32 off as in train.py:80-82): float32 a, b,
 * c and bias, fp32 MFMA products and sums (v_mfma_f32_16x16x4_f32), one in-order reduction
 * over k per output element (deterministic). Layouts as ct_gemm:
 *   c[m,n] = sum_k A(m,k) B(k,n) (+ bias[n]) (+ c[m,n] if beta)
 * With beta = 0, c is only written. No workspace.
 */
int ct_gemm_f32(const float *a, int64_t lda, int32_t trans_a, const float *b, int64_t ldb, int32_t trans_b,
                float *c, int64_t ldc, int32_t beta, const float *bias, int64_t m, int64_t n, int64_t k,
                hipStream_t stream);

/*
 * 1 when the fused NF4 operand of ct_forward_linear / ct_input_gradient accepts `w`:
 * blocksize >= 32, cols % 32 == 0, storage_dtype bf16 or f32 (decoded values reach bf16
 * in one rounding), packed 16-byte aligned. Otherwise 0: the caller decodes with
 * ct_nf4_dequant and passes the dense weight (the reference's materialize,
 * kernels/linear.py:6-13, followed by its dense GEMMs). No counterpart in the reference:
 * its GEMMs always read a materialised weight.
 */
int ct_nf4_fused_supported(const ct_nf4_weight *w);

/*
 * Replace _rms_forward / _rms_backward / _rms_weight_reduce behind RMS
 * (kernels/core_cuda.py:29-130; the decoder's RMSNorm, modeling/model.py:38-64).
 * x, y [rows, width] of x_dtype (contiguous), w [width] of w_dtype, rstd fp32 [rows].
 *   forward:  rstd = 1 / sqrt(sum(x^2) / width + eps);  y = T(T(x * rstd) * T(w)),
 *             T = rounding to x_dtype.
 *   backward: g = T(go * T(w)); with from_output = 0, x is the input and
 *             gx = rstd * (g - x * (rstd^2 * sum(g * x) / width)); with from_output = 1,
 *             x is the forward's output y and n = y / T(w), gx = rstd * (g - n * sum(g * n) / width).
 *             dw = sum over rows of go * T(x * rstd) in fp32, rounded to w_dtype (needs
 *             from_output = 0 and the workspace of ct_rms_backward_workspace).
 * go and gx are of x_dtype; gx may be go itself (written in place), either of gx and dw
 * may be null. Deterministic: fixed reduction orders.
 */
int ct_rms_forward(const void *x, int32_t x_dtype, const void *w, int32_t w_dtype, void *y, float *rstd,
                   int64_t rows, int64_t width, float eps, hipStream_t stream);
int64_t ct_rms_backward_workspace(int64_t rows, int64_t width, int32_t weight_grad);
int ct_rms_backward(const void *x, int32_t x_dtype, const void *w, int32_t w_dtype, const float *rstd,
                    const void *go, void *gx, void *dw, int64_t rows, int64_t width, int32_t from_output,
                    void *workspace, int64_t workspace_bytes, hipStream_t stream);

/*
 * Replaces weighted_ce (kernels/loss_cuda.py:11-70: _statistics, _finish), the fused
 * weighted cross-entropy of the chunked projection loss. logits [rows, vocab] of dtype
 * (row pitch ld), targets int64 [rows], weights fp32 [rows], loss fp32 [rows]:
 *   lse[r] = log sum_c exp(logits[r, c]);  loss[r] = weights[r] * (lse[r] - logits[r, target[r]])
 * (the target term is 0 for a target outside [0, vocab)). With gradient != 0 the logits
 * are overwritten with (exp(logits - lse) - onehot(target)) * weights[r], rounded to dtype.
 * Two launches over 4096-column splits of each row; the workspace (8-byte aligned,
 * ct_weighted_ce_workspace bytes) holds the per-split (maximum, sum) pairs and the target
 * logits. At most 65535 rows per call. Deterministic (fixed reduction order).
 */
int64_t ct_weighted_ce_workspace(int64_t rows, int64_t vocab);
int ct_weighted_ce(void *logits, int32_t dtype, int64_t rows, int64_t vocab, int64_t ld,
                   const int64_t *targets, const float *weights, float *loss, int32_t gradient,
                   void *workspace, int64_t workspace_bytes, hipStream_t stream);

/*
 * Replaces the optimizer step of torch.optim.AdamW(fused=True) as the reference builds it
 * (training/engine.py:10-16; amsgrad off): one launch updates every tensor of a parameter
 * group. `tensors` (device memory) lists `count` parameters; each has a fp32 step counter
 * on the device, and its gradient and states in the parameter's dtype (CT_F32 or CT_BF16
 * for all of them). `chunks` (device memory) holds n_chunks pairs (tensor index, first
 * element); a workgroup updates chunk_elems elements from there (fewer at a tensor's end).
 * With count_step != 0 every step counter is first incremented by one. Per element, with
 * s = *step: p -= lr * weight_decay * p; m = beta1 m + (1 - beta1) g;
 * v = beta2 v + (1 - beta2) g^2; p -= lr / (1 - beta1^s) * m / (sqrt(v) / sqrt(1 - beta2^s) + eps)
 * (g negated when maximize). Tensors must not overlap.
 */
/*
 * Rounds `count` (at most CT_CAST_MAX) fp32 tensors to bf16 in one launch: dst[i][j] =
 * bf16(src[i][j]) for j < counts[i], round to nearest even, as torch's .to(torch.bfloat16).
 * Replaces the per-tensor casts of the LoRA factors a.to(dtype), b.to(dtype) in
 * _LoRAGroup (kernels/linear.py:70,108) and _TiledLoRAMLP (kernels/mlp_cuda.py:62,110).
 * src, dst and counts are host arrays of device pointers and sizes; tensors must not overlap.
 */
#define CT_CAST_MAX 16
int ct_cast_f32_bf16(const float *const *src, uint16_t *const *dst, const int64_t *counts, int32_t count,
                     hipStream_t stream);

typedef struct ct_adamw_tensor {
    void *param;
    const void *grad;
    void *exp_avg;
    void *exp_avg_sq;
    const float *step;
    int64_t numel;
} ct_adamw_tensor;

int ct_adamw_step(const ct_adamw_tensor *tensors, int64_t count, const int64_t *chunks, int64_t n_chunks,
                  int64_t chunk_elems, int32_t dtype, double lr, double beta1, double beta2, double eps,
                  double weight_decay, int32_t maximize, int32_t count_step, hipStream_t stream);

/*
 * Replaces forward_linear (kernels/linear.py:27-33):
 *   xa  = bf16(x a^T)                               [m, r]   (written)
 *   out = bf16(x w^T + bias + xa b^T)               [m, n]
 * with the base GEMM and the rank-r epilogue as one contraction over k + r columns.
 * Exactly one of w_dense (bf16 [n, k]) or w_nf4 (rows n, cols k) is non-null. With w_nf4
 * and m >= 512 the weight is first decoded by ct_nf4_dequant into bf16 inside the
 * workspace (the reference's materialize) and the dense GEMM follows; below that the
 * weight is decoded tile by tile into LDS inside the GEMM (materialize fused away, which
 * needs ct_nf4_fused_supported(w_nf4), else -CT_EINVAL_LAYOUT). Both paths give results
 * bit-identical to ct_nf4_dequant's bf16 weight in the dense GEMM. Between 65 and 511
 * rows, and past them when a reduction of at least 8192 leaves the output short of one
 * round of 256 x 256 tiles, the reduction may be split across workgroups (fp32 partials
 * in the workspace, added in a fixed order); a weight without double quantization is
 * then decoded first.
 * x [m, k] (ldx), a bf16 [r, k], b bf16 [n, r], bias bf16 [n] or null, out [m, n] (ldo),
 * xa bf16 [m, r] (row pitch ldxa >= r). `epilogue` (may be null) is an elementwise step on
 * out (ct_epilogue). With xa_given != 0, xa already holds x a^T (a may
 * be null): projections that share x compute their xa together, x [a_1; a_2; ...]^T in
 * one ct_gemm with ldxa = the summed ranks, and pass column slices. The workspace query
 * takes nf4 = 0 for a bf16 weight, 1 for a double-quantized NF4 weight and 2 for NF4 with
 * plain absmax.
 */
int64_t ct_forward_linear_workspace(int64_t m, int64_t n, int64_t k, int64_t r, int32_t nf4);
int ct_forward_linear(const void *x, int64_t ldx,
                      const void *w_dense, const ct_nf4_weight *w_nf4,
                      const void *a, const void *b, const void *bias,
                      void *out, int64_t ldo, void *xa, int64_t ldxa, int32_t xa_given,
                      int64_t m, int64_t n, int64_t k, int64_t r,
                      const ct_epilogue *epilogue,
                      void *workspace, int64_t workspace_bytes, hipStream_t stream);

/*
 * ct_forward_linear without a workspace argument, for callers that cannot allocate device
 * memory (tight serving loops, harnesses that forbid hipMalloc). No counterpart in the
 * reference, whose operators allocate their workspaces with torch (kernels/linear.py:67,74).
 * Same arguments, results and row regimes as ct_forward_linear, which it calls with the
 * library's static device scratch array of CT_STATIC_SCRATCH_BYTES per GPU (held from the
 * library's load on that GPU until the process ends) in place of the workspace. Its device
 * address is resolved once per GPU by ct_init_device (or, on a GPU never set up, by the
 * first static call there). A problem whose ct_forward_linear_workspace exceeds
 * CT_STATIC_SCRATCH_BYTES returns -CT_EINVAL_WORKSPACE before anything is enqueued: 64 MiB
 * covers every few-row problem and the many-row ones whose decoded weight, plus the
 * split partials where the reduction is split, fits (up to about 32 M weight elements
 * without a split). It calls no allocator. Every call on one GPU uses that GPU's
 * one array: calls that overlap on a GPU (two streams or threads) race and must be ordered
 * by the caller. Capture of these calls into a HIP graph is not supported.
 */
#define CT_STATIC_SCRATCH_BYTES (64LL << 20)
int ct_forward_linear_static(const void *x, int64_t ldx,
                             const void *w_dense, const ct_nf4_weight *w_nf4,
                             const void *a, const void *b, const void *bias,
                             void *out, int64_t ldo, void *xa, int64_t ldxa, int32_t xa_given,
                             int64_t m, int64_t n, int64_t k, int64_t r,
                             const ct_epilogue *epilogue, hipStream_t stream);

/*
 * Replaces the forward of two projections that read one input with one rank, when their
 * xa are given (the stacked x [a_1; a_2]^T of ct_gemm): forward_linear per projection in
 * _LoRAGroup.forward (kernels/linear.py:72-86) for gate and up, or k and v beside q. For i < 2:
 *   out_i = bf16(x w_i^T + bias_i + xa[:, i r : (i + 1) r] b_i^T)        [m, n_i] (ldo[i])
 * as one GEMM over [w_1; w_2] (n_1 + n_2 output columns), so the two share one grid of
 * tiles: one partial last round instead of two. The results are those of
 * ct_forward_linear with xa_given per projection (the same products and sums). x [m, k]
 * (ldx, k % 8 == 0), w_dense[i] bf16 [n_i, k] or w_nf4[i] (exactly one per projection),
 * b_stack bf16 [n_1 + n_2, r] = [b_1; b_2] (contiguous), xa [m, 2 r] (ldxa), bias null or
 * bias[i] bf16 [n_i] or null. n_1 is a multiple of 64; the grid takes the tile the whole
 * output would take, or the largest smaller one whose edge divides n_1. No elementwise
 * step. Needs m > 64 (-CT_EINVAL_SHAPE otherwise: the caller runs the projections one by
 * one); the reduction is never split.
 * The weights are decoded (or copied) side by side into the workspace first, whose size
 * ct_group_forward_workspace gives (count must be 2).
 */
int64_t ct_group_forward_workspace(int64_t m, int32_t count, const int64_t *n, int64_t k, int64_t r);
int ct_group_forward(const void *x, int64_t ldx, int32_t count, const int64_t *n,
                     const void *const *w_dense, const ct_nf4_weight *const *w_nf4, const void *b_stack,
                     const void *xa, int64_t ldxa, const void *const *bias, void *const *out, const int64_t *ldo,
                     int64_t m, int64_t k, int64_t r, void *workspace, int64_t workspace_bytes, hipStream_t stream);

/*
 * Replaces input_gradient (kernels/linear.py:36-39):
 *   low = bf16(dy b)                                 [m, r]   (written)
 *   dx  = bf16(dy w + low a (+ dx if add))           [m, k]
 * dy [m, n] (lddy), w as in ct_forward_linear (a fused NF4 weight is decoded into LDS in
 * the transposed layout this product needs), a bf16 [r, k], b bf16 [n, r], dx [m, k]
 * (lddx), low bf16 [m, r] contiguous. `epilogue` (may be null, needs add = 0) is an
 * elementwise step on dx (ct_epilogue: CT_EPI_DSILU for the MLP's down projection).
 * Workspace query and row regimes as for ct_forward_linear, except that an NF4 weight is
 * decoded first (transposed, [k, n]) from 257 rows on (more than one 256-row tile)
 * instead of 512.
 */
int64_t ct_input_gradient_workspace(int64_t m, int64_t n, int64_t k, int64_t r, int32_t nf4);
int ct_input_gradient(const void *dy, int64_t lddy,
                      const void *w_dense, const ct_nf4_weight *w_nf4,
                      const void *a, const void *b,
                      void *dx, int64_t lddx, void *low,
                      int64_t m, int64_t n, int64_t k, int64_t r, int32_t add,
                      const ct_epilogue *epilogue,
                      void *workspace, int64_t workspace_bytes, hipStream_t stream);

/*
 * Replaces the dx half of the grouped backward of projections that share an input:
 * _LoRAGroup.backward's input_gradient per projection with add = index > 0
 * (kernels/linear.py:107-122, q/k/v) and the tiled MLP's gate and up
 * (kernels/mlp_cuda.py:136-140). For i < count (count <= CT_GROUP_MAX):
 *   low_i = bf16(dy_i b_i)                                    [m, r_i] (columns of low)
 *   dx    = bf16(sum_i (dy_i w_i + low_i a_i) (+ dx if add))  [m, k]
 * The sum is one contraction over n_total + r_total reduction columns with fp32
 * accumulation and one rounding; the reference rounds dx to bf16 after each projection,
 * so this is within its tolerances and closer to the float64 oracle. dy [m, n_total] holds
 * dy_1 .. dy_count side by side (lddy); w_i is w_dense[i] (bf16 [n_i, k]) or w_nf4[i]
 * (rows n_i, cols k, decodable transposed: cols % 16 == 0, rows % 8 == 0), exactly one per
 * projection (either array may be null when the other holds every weight); a_stack bf16
 * [r_total, k] = [a_1; ...; a_count] (contiguous rows); b[i] bf16 [n_i, r_i] contiguous;
 * low bf16 [m, r_total] (ldlow). Every n_i is a multiple of 8. The weights are decoded
 * (or, dense, transposed) side by side into the workspace first, whose size
 * ct_group_input_gradient_workspace gives; the low-rank products and the contraction's
 * split partials use the rest.
 */
#define CT_GROUP_MAX 8
int64_t ct_group_input_gradient_workspace(int64_t m, int32_t count, const int64_t *n, const int64_t *r, int64_t k);
int ct_group_input_gradient(const void *dy, int64_t lddy, int32_t count, const int64_t *n, const int64_t *r,
                            const void *const *w_dense, const ct_nf4_weight *const *w_nf4,
                            const void *a_stack, const void *const *b,
                            void *dx, int64_t lddx, void *low, int64_t ldlow, int64_t m, int64_t k, int32_t add,
                            void *workspace, int64_t workspace_bytes, hipStream_t stream);

/*
 * Replaces the same dx half (kernels/linear.py:107-122) where the upstream gradients
 * arrive as separate tensors: the first projection's dy_0 is read where it lies, so no
 * [m, n_total] side-by-side copy is made of it. For i < count (count <= CT_GROUP_MAX):
 *   low_i = bf16(dy_i b_i)                                    [m, r_i]
 *   dx    = bf16(dy_0 w_0 + tail [w_1; ...; w_{count-1}; a_stack] (+ dx if add))   [m, k]
 * where tail [m, n_tail + r_total] (ldtail, n_tail = n_1 + ... + n_{count-1}) holds
 * dy_1 .. dy_{count-1} side by side in its first n_tail columns on entry and receives
 * low_0 .. low_{count-1} side by side in the rest. The sum is one contraction over
 * n_total + r_total reduction columns, fp32-accumulated and rounded once, as in
 * ct_group_input_gradient (the two differ only in the order of the fp32 additions).
 * dy_0 [m, n_0] (lddy0); weights, a_stack and b as for ct_group_input_gradient, except
 * that only w_0 needs the transposed decode: w_0 is decoded (or, dense, transposed) into
 * [k, n_0] and the others in their own layout [n_i, k], beside a copy of a_stack, in the
 * workspace (ct_group_input_gradient_lead_workspace); the low-rank products and the
 * contraction's split partials use the rest. For projections whose later members are
 * narrow (q with k and v: 256 copied columns instead of 4352).
 */
int64_t ct_group_input_gradient_lead_workspace(int64_t m, int32_t count, const int64_t *n, const int64_t *r,
                                               int64_t k);
int ct_group_input_gradient_lead(const void *dy0, int64_t lddy0, void *tail, int64_t ldtail, int32_t count,
                                 const int64_t *n, const int64_t *r, const void *const *w_dense,
                                 const ct_nf4_weight *const *w_nf4, const void *a_stack, const void *const *b,
                                 void *dx, int64_t lddx, int64_t m, int64_t k, int32_t add, void *workspace,
                                 int64_t workspace_bytes, hipStream_t stream);

/*
 * Replaces parameter_gradients (kernels/linear.py:42-44) with accumulate's fp32 branch
 * (kernels/linear.py:16-24):
 *   da = low^T x   (+ da if add)   float32 [r, k]
 *   db = dy^T xa   (+ db if add)   float32 [n, r]
 * x [m, k] (ldx), dy [m, n] (lddy), low bf16 [m, r] (ldlow), xa bf16 [m, r] (ldxa; a
 * column slice of a group's shared xa). The m-reduction is split over workgroups and
 * summed in a fixed order, so repeated calls are bit-identical; add = 0 never reads da/db
 * (NaN-filled storage is ignored).
 */
int64_t ct_parameter_gradients_workspace(int64_t m, int64_t n, int64_t k, int64_t r);
int ct_parameter_gradients(const void *x, int64_t ldx, const void *dy, int64_t lddy,
                           const void *low, int64_t ldlow, const void *xa, int64_t ldxa, float *da, float *db,
                           int64_t m, int64_t n, int64_t k, int64_t r, int32_t add,
                           void *workspace, int64_t workspace_bytes, hipStream_t stream);

/*
 * Replaces accumulate (kernels/linear.py:16-24) for bf16 operands and a float32 output:
 *   out[p,q] = sum_j L(p,j) R(j,q) (+ out[p,q] if add)
 *   L(p,j) = left[p*ldl + j] (trans_l = 0) or left[j*ldl + p] (trans_l = 1)
 *   R(j,q) = right[j*ldr + q] (trans_r = 0) or right[q*ldr + j] (trans_r = 1)
 * Deterministic split reduction over j, as ct_parameter_gradients.
 */
int64_t ct_accumulate_workspace(int64_t p, int64_t q, int64_t j);
int ct_accumulate(float *out, int64_t ldo,
                  const void *left, int64_t ldl, int32_t trans_l,
                  const void *right, int64_t ldr, int32_t trans_r,
                  int64_t p, int64_t q, int64_t j, int32_t add,
                  void *workspace, int64_t workspace_bytes, hipStream_t stream);

/*
 * Replaces the SiLU-multiply kernel `_activation` (kernels/mlp_cuda.py:10-35) of the
 * tiled LoRA MLP, elementwise over n elements of `dtype` (CT_BF16 or CT_F32), fp32 math:
 *   sig = 1 / (1 + exp(-gate)),  act = dtype(gate * sig)
 *   reconstruct:  h = act * up
 *   backward:     dgate = dtype(h * up) * sig * (1 + gate * (1 - sig)),  dup = h * act
 * (in backward, h holds the incoming gradient; with reconstruct it is overwritten by the
 * hidden activation). The outputs may alias the inputs as the reference's backward call
 * does (dgate = gate, dup = up). Results match the reference within float rounding: the
 * exponential is this library's, not Triton's.
 */
int ct_silu_multiply(const void *gate, const void *up, void *h, void *dgate, void *dup, int64_t n,
                     int32_t backward, int32_t reconstruct, int32_t dtype, hipStream_t stream);

/*
 * Replaces the partial GPT-J rotary kernels `_rope` and `_owned_qk_rope` with
 * `_rotate_pair` (kernels/core_cuda.py:133-189). x and y are [tokens, heads, head_dim]
 * of `dtype` (CT_F32, CT_F16 or CT_BF16), contiguous within a token, with ldx / ldy
 * elements between tokens (0: heads * head_dim, contiguous; a larger pitch lets y be a
 * column range of a wider matrix, as the grouped backward's side-by-side upstream
 * gradients); x == y needs ldx == ldy. cosine and sine are [tokens, half]
 * contiguous of `trig_dtype`, half <= head_dim / 2. Channel pairs (2c, 2c+1), c < half:
 *   e' = T(T(e cos) - T(o sin)),  o' = T(T(o cos) + T(e sin))    (T = round to dtype)
 * with the sine negated when `inverse` (the backward rotation). With rotated_only = 0
 * every pair is written to y (unrotated channels copied; y may be x); with rotated_only =
 * 1 the rotation runs in place (y must be x) and other channels are not touched, as
 * rotate_owned_qk does on freshly written projection outputs.
 */
int ct_rope(const void *x, void *y, const void *cosine, const void *sine, int64_t tokens, int64_t heads,
            int64_t head_dim, int64_t half, int64_t ldx, int64_t ldy, int32_t inverse, int32_t rotated_only,
            int32_t dtype, int32_t trig_dtype, hipStream_t stream);

/*
 * Kernel timing for benchmarks; no counterpart in the reference (which publishes no kernel
 * timings). ct_profile_begin enables the families in `families` and creates `capacity`
 * HIP event pairs; each later launch of an enabled family is bracketed by one pair
 * recorded on the launch stream (launches beyond capacity go untimed). ct_profile_read
 * synchronises on those events and returns, for the launches of `family` (a mask), their
 * summed duration (ms), their count and their summed algorithmic work: FLOPs for the GEMM
 * families, HBM bytes for the decoder. ct_profile_end stops timing and frees the events.
 * One profiler at a time; the timed launches may come from any thread.
 */
#define CT_PROF_FWD_GEMM 1  /* fused projection GEMM of ct_forward_linear: 2 m n (k + r) */
#define CT_PROF_DX_GEMM  2  /* fused projection GEMM of ct_input_gradient: 2 m k (n + r) */
#define CT_PROF_DEQUANT  4  /* ct_nf4_dequant: packed + scale + code bytes read, output written */
#define CT_PROF_PARAM    8  /* ct_parameter_gradients (dA and dB): 2 m r (k + n) */
#define CT_PROF_LOWRANK 16  /* xa = x a^T and low = dy b inside the entry points: 2 m r k or 2 m r n */
int ct_profile_begin(int32_t families, int32_t capacity);
int ct_profile_read(int32_t family, double *total_ms, int64_t *launches, double *work);
int ct_profile_end(void);

#ifdef __cplusplus
}
#endif

#endif /* CAUSAL_TUNER_HIP_H */
