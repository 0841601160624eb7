/* Test hooks of the MoE library (libmkmoe_testing.so, built beside libmkmoe.so): the
 * hardware converts and the scaled MFMA its kernels use, each run alone, and host builds of its
 * kernels' exact arithmetic, for the tests that pin them. They have no counterpart in the
 * reference and are not part of the drop-in surface (include/mkmoe.h, include/mkmoe_seam.h):
 * a caller of the MoE block needs none of them. Status codes and mkmoe_shape are mkmoe.h's. */
#ifndef MKMOE_TESTING_H
#define MKMOE_TESTING_H

#include <stdint.h>

#include "mkmoe.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Device decode of n bytes (device pointers): fp8[i] = e4m3 value of codes[i],
 * fp4[2i], fp4[2i + 1] = the e2m1 values of its low and high nibble, through
 * the same hardware converts the kernels use (for tests of those converts). */
int mkmoe_device_decode(const uint8_t* codes, float* fp8, float* fp4, int32_t n, void* stream);

/* Device sweep of the fp32 bit patterns [first, first + count) (inf and NaN skipped) through
 * the e4m3 convert the activation quantizers use, against the integer-step encoder of
 * mkmoe_numerics.h that the CPU oracle restates; adds the number of differing codes to *bad
 * and lowers *first_bad to the lowest differing pattern (device pointers the caller set). A
 * test hook with no counterpart in the reference, whose quantizer is torch's conversion
 * (check_ffn.py:104). MKMOE_ERR_ARG for count 0 or a range past 2^32. */
int mkmoe_device_e4m3_sweep(uint32_t first, uint32_t count, uint32_t* bad, uint32_t* first_bad, void* stream);

/* Device run of the scaled MFMA the MXFP4 option uses (v_mfma_scale_f32_16x16x128_f8f6f4,
 * C = 0), for its known-answer tests; no counterpart in the reference, which calls the
 * instruction through FlyDSL (common/mx.py:60-66). tiles waves, one 16x16x128 tile each: a
 * and b hold eight 32-bit words a lane ([tiles][64][8]; an e2m1 A (fmt_a 4) uses the first
 * four, an e4m3 A is fmt_a 0; B is e4m3), sa and sb one E8M0 code a lane ([tiles][64]), d
 * four floats a lane ([tiles][64][4]: C[m][n] in lane n + 16 (m / 4), element m % 4). */
int mkmoe_device_mfma_scaled(const void* a, const void* b, const void* sa, const void* sb, float* d,
                             int32_t fmt_a, int32_t tiles, void* stream);

/* Host builds of the kernels' exact arithmetic (no device needed): */
void mkmoe_host_e4m3_encode(const float* x, uint8_t* out, int64_t n);
void mkmoe_host_sigmoid(const float* x, float* out, int64_t n);
void mkmoe_host_sqrt_softplus(const float* x, float* out, int64_t n);
/* grouped top-k of one row of fp32 scores [E] with fp32 bias */
void mkmoe_host_topk(const mkmoe_shape* shape, const float* scores, const float* bias,
                     int32_t* ids, float* weights);

#ifdef __cplusplus
}
#endif
#endif /* MKMOE_TESTING_H */
