/* GLINT H-TILE GEMM / GEMV C ABI, MI355X (gfx950) build (exported by libglint_encode.so).
 *
 * y[M,N] = x[M,K] * W^T,  W[n,k] = GLINT_CELLS[hole][plug] * absmax[(n*K + k) / blocksize],
 * hole/plug packed along K (element i = n*K + k is nibble i & 1 of byte i >> 1).
 * x is BF16 bits [M, K] row-major. Any M, N >= 0, K >= 1, blocksize >= 1, and pointers
 * into larger (unaligned) buffers are accepted; aligned bs=64 shapes take the fast paths.
 */
#ifndef GLINT_HTILE_H_
#define GLINT_HTILE_H_
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif
struct ihipStream_t;

/* f32 output, f32 arithmetic (within 1e-5 * (1 + |ref|) of a float64 reference).
 * Enqueued on `stream`; y is overwritten. Returns 0, -1 for a null pointer,
 * -2 for blocksize <= 0 (or K < 1), -3 for a launch error.
 * Reference: include/glint_htile.h:11-14 (cuda/glint_htile.cu:165-180). */
int launch_glint_htile_s3_f32_stream(const uint8_t *d_hole, const uint8_t *d_plug, const float *d_absmax,
                                     const void *d_x_bf16, float *d_y,
                                     int M, int N, int K, int blocksize, struct ihipStream_t *stream);
/* Same on the null stream. Reference: include/glint_htile.h:16-19 (cuda/glint_htile.cu:181-187). */
int launch_glint_htile_s3_f32(const uint8_t *d_hole, const uint8_t *d_plug, const float *d_absmax,
                              const void *d_x_bf16, float *d_y, int M, int N, int K, int blocksize);

/* ---- Additive (no reference counterpart). ----
 * BF16 output with f32 accumulation: the decode GEMV (small M, HBM-bound) and the
 * prefill GEMM (larger M: BF16 MFMA on LDS-dequantized weight tiles). Contract: within
 * 1e-2 relative Frobenius error of an f32 GEMM on the expanded weights; results are
 * deterministic (split K adds its partial tiles in a fixed order).
 * At M > 1 the first call on a stream at a given size may allocate the stream's split-K
 * workspace (hipMalloc, at most 32 MiB, kept until exit); during graph capture it is not
 * grown and the GEMM runs unsplit. Same return codes. */
int launch_glint_htile_bf16_stream(const uint8_t *d_hole, const uint8_t *d_plug, const float *d_absmax,
                                   const void *d_x_bf16, uint16_t *d_y_bf16,
                                   int M, int N, int K, int blocksize, struct ihipStream_t *stream);
#ifdef __cplusplus
}
#endif
#endif
