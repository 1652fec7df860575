/* W8A8 INT8 GEMM C ABI (attach library libp7_kernels.so), MI355X (gfx950) build.
 * Reference: include/int8_mma_gemm.h:14-39, attach/CONTRACT.md:10-16.
 *
 * Return values are hipError_t codes as int: 0 success, 1 (hipErrorInvalidValue, the
 * same value as cudaErrorInvalidValue) for bad arguments, other codes from the launch. */
#ifndef GLINT_INT8_MMA_GEMM_H
#define GLINT_INT8_MMA_GEMM_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif
struct ihipStream_t;

#define INT8_MMA_BLOCK 64

/* One bf16_to_int8_pin_v1 linear: q I8 [n_out, k_in] row-major, scale F32 [n_out * k_in / 64],
 * w[n, k] = q[n, k] * scale[n * (k_in / 64) + k / 64]. Reference: include/int8_mma_gemm.h:14-19. */
typedef struct {
    const int8_t *q;
    const float *scale;
    int n_out;
    int k_in;
} Int8MmaLinear;

/* Activation scratch: xq [m, k_in] bytes, sx [m, k_in / 64] floats. */
static inline size_t int8_mma_xq_bytes(int m, int k_in) { return (size_t)m * (size_t)k_in; }
static inline size_t int8_mma_sx_bytes(int m, int k_in) { return (size_t)m * (size_t)(k_in / INT8_MMA_BLOCK) * sizeof(float); }

/* y[m, n] = sum_kb ((float)ic_kb * sx[m, kb]) * sw[n, kb], ic_kb the exact int32 dot product of
 * the 64-wide K slice kb, kb ascending; x (BF16 bits [m, k_in]) is first quantized per (row,
 * 64-block): s = amax > 0 ? amax / 127 : 1, xq = clamp(rint(x / s), -127, 127) into xq/sx.
 * Requires k_in % 64 == 0, k_in >= 64, m >= 1, n_out >= 1; y is f32 [m, n_out].
 * Reference: include/int8_mma_gemm.h:21-30 (cuda/int8_mma_gemm.cu:11-155). */
int int8_mma_gemm(const void *x_bf16, Int8MmaLinear w, float *y, int m, int8_t *xq, float *sx,
                  struct ihipStream_t *stream);

/* Late plug, two passes: y = X (base)^T, then y += X (plug)^T with the same activation
 * quantization; the plug is a p7_plug_res4_v1 slice (plug_q4: ceil(n_out * k_in / 2) bytes,
 * element 2i in the low nibble, value nibble - 8; plug_scale: one f32 per 64 weights in the
 * base's block order) unpacked into plug_i8 (n_out * k_in bytes of caller scratch, 16-B
 * aligned). Each pass sums its kb terms as int8_mma_gemm does; the second adds into y.
 * Reference: include/int8_mma_gemm.h:41-47 (cuda/int8_mma_gemm.cu:157-181). */
int int8_mma_gemm_plug(const void *x_bf16, Int8MmaLinear w, const uint8_t *plug_q4, const float *plug_scale,
                       float *y, int m, int8_t *xq, float *sx, int8_t *plug_i8, struct ihipStream_t *stream);

/* Late plug in one kernel: per kb, acc = acc + ((float)ic * sx) * sw, then
 * acc = acc + ((float)ip * sx) * sp, ip the plug slice's dot product (nibbles unpacked in
 * LDS); no scratch. Reference: include/int8_mma_gemm.h:49-54 (cuda/int8_mma_gemm.cu:224-240). */
int int8_mma_gemm_plug_fused(const void *x_bf16, Int8MmaLinear w, const uint8_t *plug_q4,
                             const float *plug_scale, float *y, int m, int8_t *xq, float *sx,
                             struct ihipStream_t *stream);

/* Resolution: int8_mma_gemm (optionally plus a plug), plus the activation's quantization
 * residual r = x - (float)xq * sx re-quantized by the same rule into rq/sr (scratch the size
 * of xq/sx) and multiplied as further accumulating passes: y = xq W, += rq W, and with a plug
 * += xq P, += rq P. The three plug pointers are all NULL or all set.
 * Reference: include/int8_mma_gemm.h:56-61 (cuda/int8_mma_gemm.cu:183-222). */
int int8_mma_gemm_resolve(const void *x_bf16, Int8MmaLinear w, const uint8_t *plug_q4, const float *plug_scale,
                          float *y, int m, int8_t *xq, float *sx, int8_t *rq, float *sr, int8_t *plug_i8,
                          struct ihipStream_t *stream);

/* ---- Additive (no reference counterpart): the plain INT8 GEMM of the benchmark config. ----
 * C[m, n] = sum_k A[m, k] * B[n, k] in int32 (exact), A [M, K], B [N, K] row-major int8.
 * Requires K % 64 == 0. */
int glint_int8_gemm_i32(const int8_t *A, const int8_t *B, int32_t *C, int M, int N, int K,
                        struct ihipStream_t *stream);
/* Same product, output BF16 bits of RNE(((float)C[m, n] * sa[m]) * sb[n]). */
int glint_int8_gemm_scaled_bf16(const int8_t *A, const int8_t *B, const float *sa, const float *sb,
                                uint16_t *out_bf16, int M, int N, int K, struct ihipStream_t *stream);
#ifdef __cplusplus
}
#endif
#endif
