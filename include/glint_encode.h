/* GLINT encode / expand C ABI (libglint_encode.so), MI355X (gfx950) build.
 *
 * Same symbols, argument meaning and return codes as the reference's
 * include/glint_encode.h, so ctypes and C callers bind unchanged. The stream type is
 * spelled `struct ihipStream_t *` (== hipStream_t); at the ABI level it is the same
 * opaque pointer the reference passes as cudaStream_t.
 *
 * Return codes: 0 ok; -1 bad argument, device allocation or host->device copy failed;
 * -2 table setup failed (never: the tables are compiled into the code object);
 * -3 kernel launch, synchronisation or device->host copy failed.
 * Pin layout: hole/plug are ceil(n/2) bytes, element 2e in the low nibble of byte e,
 * 2e+1 in the high nibble, a zero pad nibble for odd n; absmax is ceil(n/bs) f32.
 */
#ifndef GLINT_ENCODE_H_
#define GLINT_ENCODE_H_
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif
struct ihipStream_t;

/* Host pointers; synchronous; allocates device scratch per call.
 * Reference: include/glint_encode.h:11-13 (cuda/glint_encode.cu:182-204). */
int glint_encode_bf16_host(const uint16_t *w_bf16, int64_t n, int blocksize,
                           uint8_t *hole_packed, uint8_t *plug_packed, float *absmax);
/* Reference: include/glint_encode.h:14-16 (cuda/glint_encode.cu:169-181). */
int glint_encode_f32_host(const float *w, int64_t n, int blocksize,
                          uint8_t *hole_packed, uint8_t *plug_packed, float *absmax);
/* ceil(n / blocksize), 0 when blocksize <= 0. Reference: include/glint_encode.h:17. */
int glint_encode_n_absmax(int64_t n, int blocksize);
/* ceil(n / 2). Reference: include/glint_encode.h:18. */
int glint_encode_n_packed(int64_t n);
/* Host pointers; synchronous. Reference: include/glint_encode.h:20-22
 * (cuda/glint_encode.cu:205-246). */
int glint_expand_packed_to_f32_host(const uint8_t *hole_packed, const uint8_t *plug_packed,
                                    const float *absmax, int64_t n, int blocksize, float *out_f32);
/* Device pointers; enqueued on `stream`, no allocation, returns after the launch.
 * Reference: include/glint_encode.h:26-29 (cuda/glint_encode.cu:248-262). */
int glint_expand_packed_to_f32_device(const uint8_t *d_hole_packed, const uint8_t *d_plug_packed,
                                      const float *d_absmax, int64_t n, int blocksize,
                                      float *d_out_f32, struct ihipStream_t *stream);

/* ---- Additive entry points (no reference counterpart; nothing above changes). ---- */
/* Device-pointer encode, async on `stream`, no allocation. Same bytes as the host
 * variants. Returns -1 for a null pointer, blocksize <= 0 or n < 0, -3 on launch failure. */
int glint_encode_bf16_device(const uint16_t *d_w_bf16, int64_t n, int blocksize,
                             uint8_t *d_hole_packed, uint8_t *d_plug_packed, float *d_absmax,
                             struct ihipStream_t *stream);
int glint_encode_f32_device(const float *d_w, int64_t n, int blocksize,
                            uint8_t *d_hole_packed, uint8_t *d_plug_packed, float *d_absmax,
                            struct ihipStream_t *stream);
/* Unpin to BF16 on the GPU: the bits of RNE(f32 expand), NaN -> (u >> 16) | 0x40,
 * i.e. glint_unpin.py:25-32 computed on device. */
int glint_expand_packed_to_bf16_host(const uint8_t *hole_packed, const uint8_t *plug_packed,
                                     const float *absmax, int64_t n, int blocksize, uint16_t *out_bf16);
int glint_expand_packed_to_bf16_device(const uint8_t *d_hole_packed, const uint8_t *d_plug_packed,
                                       const float *d_absmax, int64_t n, int blocksize,
                                       uint16_t *d_out_bf16, struct ihipStream_t *stream);
#ifdef __cplusplus
}
#endif
#endif
