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

/* f32 output, f32 products and f32 sums (within 1e-5 * (1 + |ref|) of a float64 reference).
 * At M > 1 with blocksize 64, K % 64 == 0 and aligned pointers the products run on BF16
 * MFMA with each f32 weight split exactly into three BF16 planes (the sum differs from a
 * sequential f32 sum only in order); M = 1 is the f32 GEMV (K <= 32768; larger K takes
 * the MFMA route), other shapes a generic kernel. Enqueued on `stream`; y is overwritten
 * (with zeros when K <= 0: the empty sum, as in the reference). Returns 0, -1 for a null
 * pointer, -2 for blocksize <= 0, -3 for a launch error; M <= 0 or N <= 0 launches nothing
 * and returns 0. The MFMA route uses the stream's split-K workspace as
 * launch_glint_htile_bf16_stream does.
 * Reference: include/glint_htile.h:11-14 (cuda/glint_htile.cu:165-180). */
int launch_glint_htile_s3_f32_stream(const uint8_t *d_hole, const uint8_t *d_plug, const float *d_absmax,
                                     const void *d_x_bf16, float *d_y,
                                     int M, int N, int K, int blocksize, struct ihipStream_t *stream);
/* Same on the null stream. Reference: include/glint_htile.h:16-19 (cuda/glint_htile.cu:181-187). */
int launch_glint_htile_s3_f32(const uint8_t *d_hole, const uint8_t *d_plug, const float *d_absmax,
                              const void *d_x_bf16, float *d_y, int M, int N, int K, int blocksize);

/* ---- Additive (no reference counterpart). ----
 * BF16 output with f32 accumulation: the decode GEMV (M = 1, and M = 2 .. 8 with each
 * weight read once for all rows, as BF16(cell) x absmax; the f32-out entry above takes the
 * same route at M = 2 .. 4 with exact f32 cells) and the prefill GEMM (larger M:
 * BF16 MFMA on LDS-dequantized weight tiles). Contract: within
 * 1e-2 relative Frobenius error of an f32 GEMM on the expanded weights; results are
 * deterministic (split K adds its partial tiles in a fixed order).
 * Split-K workspace (M > 1 on the MFMA routes, both outputs): at most two per (device,
 * stream), each allocated once at full size (CUs x 512 KiB of partials plus counters,
 * 128 MiB on MI355X), its counters zeroed by a kernel on the stream, never grown; freed by
 * glint_htile_workspace_release. The eager one is allocated by the first call that
 * splits. The first launch captured into a graph takes it over as the stream's graph
 * workspace, which every later capture on that stream binds too; the next eager call gets
 * a fresh eager one. So replays and eager calls never share counters, replays of graphs
 * captured on one stream share theirs and must not overlap one another, and capture ->
 * eager cycles allocate nothing after the first. hipStreamPerThread gets its own per host
 * thread. A capture on a stream with no workspace yet runs unsplit. Same return codes. */
int launch_glint_htile_bf16_stream(const uint8_t *d_hole, const uint8_t *d_plug, const float *d_absmax,
                                   const void *d_x_bf16, uint16_t *d_y_bf16,
                                   int M, int N, int K, int blocksize, struct ihipStream_t *stream);
/* Allocate `stream`'s split-K workspace now (no-op if it has one), so that a later graph
 * capture on the stream can split K and no later call allocates. Not during capture.
 * Returns 0, or -1 if it cannot (allocation failed, or the stream is capturing). */
int glint_htile_workspace_reserve(struct ihipStream_t *stream);
/* No reference counterpart. Free `stream`'s split-K workspaces (eager and graph), after
 * waiting for the stream. Graphs captured on the stream before the call must not be
 * replayed after it; a later call allocates afresh. Not during capture. Returns 0, or -1
 * if the stream is capturing or the runtime fails. */
int glint_htile_workspace_release(struct ihipStream_t *stream);

/* No reference counterpart. For callers that cannot allocate (code under graph capture,
 * tight serving loops, harnesses that forbid hipMalloc): launch_glint_htile_bf16_stream
 * with the split-K partials and counters in a static per-GPU scratch array of the library
 * (64 MiB plus 4 KiB, held until the process ends) instead of a per-stream workspace. Same
 * kernels, split plan and results, except where launch_glint_htile_bf16_stream would run
 * Stream-K (it needs twice the partials): there whole tiles run, within the same contract,
 * the last bits possibly different. Allocates nothing. Calls that overlap on one GPU share
 * the array and race. Returns the codes above, or -5 when the split plan would need more
 * than the array holds (possible only on a part with more than 256 CUs). */
int launch_glint_htile_bf16_stream_noalloc(const uint8_t *d_hole, const uint8_t *d_plug, const float *d_absmax,
                                           const void *d_x_bf16, uint16_t *d_y_bf16,
                                           int M, int N, int K, int blocksize, struct ihipStream_t *stream);
#ifdef __cplusplus
}
#endif
#endif
