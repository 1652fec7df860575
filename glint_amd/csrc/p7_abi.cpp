/* Attach-ABI version string and flat FFI entries of libp7_kernels.so.
 * Reference: cuda/p7_abi.c:3-11, attach/ABI_VERSION, cuda/p7_abi_selftest.cu:145-159. */
#include <stdint.h>
#include "int8_mma_gemm.h"
#include "p7_attach.h"

#define P7_API extern "C" __attribute__((visibility("default")))
#define P7_ABI_VERSION_STR "p7_attach_abi_v1"

P7_API const char *p7_abi_version(void) { return P7_ABI_VERSION_STR; }

P7_API int p7_int8_gemm_flat(const void *x_bf16, const void *q, const void *scale, int n_out, int k_in, void *y, int m,
                             void *xq, void *sx, void *stream) {
    Int8MmaLinear w = {(const int8_t *)q, (const float *)scale, n_out, k_in};
    return int8_mma_gemm(x_bf16, w, (float *)y, m, (int8_t *)xq, (float *)sx, (struct ihipStream_t *)stream);
}

P7_API int p7_int8_gemm_plug_flat(const void *x_bf16, const void *q, const void *scale, const void *plug_q4,
                                  const void *plug_scale, int n_out, int k_in, void *y, int m, void *xq, void *sx,
                                  void *stream) {
    Int8MmaLinear w = {(const int8_t *)q, (const float *)scale, n_out, k_in};
    return int8_mma_gemm_plug_fused(x_bf16, w, (const uint8_t *)plug_q4, (const float *)plug_scale, (float *)y, m,
                                    (int8_t *)xq, (float *)sx, (struct ihipStream_t *)stream);
}
