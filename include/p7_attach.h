/* Attach-ABI entry points of libp7_kernels.so that have no header in the reference.
 * Reference: attach/CONTRACT.md:10-22, cuda/p7_abi.c:3-11, cuda/p7_abi_selftest.cu:46-159. */
#ifndef GLINT_P7_ATTACH_H
#define GLINT_P7_ATTACH_H
#include <stddef.h>
#ifdef __cplusplus
extern "C" {
#endif
/* Returns "p7_attach_abi_v1" (attach/ABI_VERSION). */
const char *p7_abi_version(void);
/* Flat-argument int8_mma_gemm for FFI callers (no struct by value); returns the hipError_t code. */
int p7_int8_gemm_flat(const void *x_bf16, const void *q, const void *scale, int n_out, int k_in,
                      void *y, int m, void *xq, void *sx, void *stream);
/* Flat-argument int8_mma_gemm_plug_fused (base + p7_plug_res4_v1 slice in one kernel).
 * Reference: cuda/p7_abi_selftest.cu:152-159. */
int p7_int8_gemm_plug_flat(const void *x_bf16, const void *q, const void *scale, const void *plug_q4,
                           const void *plug_scale, int n_out, int k_in, void *y, int m, void *xq, void *sx,
                           void *stream);
/* The attach gate's self-test: 4-layer INT8 stack resident vs streamed through the plug
 * ring; 0 on pass, -1..-8 name the failed stage; msg gets a one-line report.
 * Reference: cuda/p7_abi_selftest.cu:46-142. */
int p7_abi_selftest(char *msg, size_t msg_n);
#ifdef __cplusplus
}
#endif
#endif
