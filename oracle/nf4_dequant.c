/*
 * Plain-C NF4 decode. TEST INFRASTRUCTURE ONLY: the timed CPU baseline of bench.py and a
 * second restatement the tests compare with oracle/nf4.py.
 *
 * Follows the reference's decoder (kernels/nf4_cuda.py:13-29): per block g,
 *   s = code2[absmax[g]] * absmax2[g / blocksize2] + offset   (fp32 multiply, then add)
 * and out[e] = bf16_rtne(code[nibble(e)] * s), element 2j from the high nibble of byte j.
 * Built with -ffp-contract=off so no multiply-add is fused.
 */
#include <stdint.h>
#include <string.h>

static inline uint16_t bf16_rtne(float f) {
    uint32_t u;
    memcpy(&u, &f, sizeof u);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

/* Nested (double-quantized) bf16 decode of n elements; blocksize divides 2^k. */
void ct_oracle_nf4_dequant_bf16(const uint8_t *packed, const uint8_t *qabsmax, const float *code,
                                const float *code2, const float *absmax2, float offset, int64_t n,
                                int64_t blocksize, int64_t blocksize2, uint16_t *out) {
    const int64_t nb = (n + blocksize - 1) / blocksize;
#pragma omp parallel for schedule(static)
    for (int64_t g = 0; g < nb; ++g) {
        const float decoded = code2[qabsmax[g]] * absmax2[g / blocksize2];
        const float s = decoded + offset;
        const int64_t begin = g * blocksize;
        const int64_t end = begin + blocksize < n ? begin + blocksize : n;
        for (int64_t e = begin; e < end; ++e) {
            const uint8_t byte = packed[e >> 1];
            const uint8_t nib = (e & 1) ? (byte & 15u) : (byte >> 4);
            out[e] = bf16_rtne(code[nib] * s);
        }
    }
}

/* Sets the OpenMP team size of the decode (the bench's CPU baseline times several). */
void ct_oracle_set_threads(int threads) {
#ifdef _OPENMP
    extern void omp_set_num_threads(int);
    omp_set_num_threads(threads);
#else
    (void)threads;
#endif
}

int ct_oracle_threads(void) {
    int t = 1;
#pragma omp parallel
    {
#pragma omp single
        {
#ifdef _OPENMP
            extern int omp_get_num_threads(void);
            t = omp_get_num_threads();
#endif
        }
    }
    return t;
}
