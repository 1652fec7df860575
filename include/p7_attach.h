/* Attach-ABI entry points of libp7_kernels.so that have no header in the reference.
 * Reference: attach/CONTRACT.md:10-16, cuda/p7_abi.c:3-11, cuda/p7_abi_selftest.cu:145-149. */
#ifndef GLINT_P7_ATTACH_H
#define GLINT_P7_ATTACH_H
#ifdef __cplusplus
extern "C" {
#endif
/* Returns "p7_attach_abi_v1" (attach/ABI_VERSION). */
const char *p7_abi_version(void);
/* Flat-argument int8_mma_gemm for FFI callers (no struct by value); returns the hipError_t code. */
int p7_int8_gemm_flat(const void *x_bf16, const void *q, const void *scale, int n_out, int k_in,
                      void *y, int m, void *xq, void *sx, void *stream);
#ifdef __cplusplus
}
#endif
#endif
