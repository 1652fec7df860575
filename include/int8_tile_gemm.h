/* W8A16 tile GEMM over an INT8 pin linear (libp7_kernels.so), MI355X (gfx950) build.
 * Reference: include/int8_tile_gemm.h:1-29 (cuda/int8_tile_gemm.cu:169-180).
 *
 * The reference declares int8_tile_gemm_bf16 with C++ linkage and CUDA types
 * (__nv_bfloat16, cudaStream_t). This build exports it with C linkage and opaque
 * pointers: x is BF16 bits, the stream a hipStream_t. The return value is a hipError_t
 * code as int (0 success, 1 hipErrorInvalidValue, the same values as CUDA's). */
#ifndef GLINT_INT8_TILE_GEMM_H
#define GLINT_INT8_TILE_GEMM_H
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif
struct ihipStream_t;

#define INT8_PIN_BLOCK 64

/* One bf16_to_int8_pin_v1 linear resident on the device: q I8 [n_out, k_in] row-major,
 * scale F32 [ceil(n_out * k_in / 64)], w[i] = q[i] * scale[i / 64] over the flattened
 * index i (k_in need not be a multiple of 64). Reference: include/int8_tile_gemm.h:10-18. */
typedef struct {
    const int8_t *q;
    const float *scale;
    int n_out;
    int k_in;
} Int8PinLinear;

/* y[m, n] = sum_k x[m, k] * bf16(q[n, k] * scale), x BF16 [m, k_in] row-major, y f32
 * [m, n_out] row-major, fully overwritten. Each weight is rounded to BF16 (nearest even)
 * as a BF16 dequant of the pin would be; products accumulate in f32. Any m >= 0,
 * n_out >= 1, k_in >= 1 and any alignment; m == 0 launches nothing.
 * Before checking its arguments it returns, and clears, an error already pending on the
 * calling thread (hipGetLastError), without launching.
 * At m > 4 the first call on a stream may allocate the stream's split-K workspace
 * (hipMalloc, 128 MiB; at most two per stream, the second bound by graph captures, as in
 * glint_htile.h), kept until int8_tile_gemm_workspace_release; a capture on a stream with
 * no workspace runs unsplit. Results are deterministic.
 * Reference: include/int8_tile_gemm.h:20-27 (cuda/int8_tile_gemm.cu:169-180). */
int int8_tile_gemm_bf16(const void *x_bf16, Int8PinLinear w, float *y, int m, struct ihipStream_t *stream);
/* No reference counterpart. Free `stream`'s W8A16 split-K workspaces after waiting for the
 * stream (graphs captured on it before must not be replayed after). Not during capture.
 * Returns 0, or -1 if the stream is capturing or the runtime fails. */
int int8_tile_gemm_workspace_release(struct ihipStream_t *stream);

#ifdef __cplusplus
}
#endif
#endif
