/* K-major decode path: parent-only (fold) GEMV plus the activation-selected plug
 * correction, MI355X (gfx950) build, in libglint_encode.so.
 *
 * The reference implements this path in Mojo (mojo/p7_glint_gemv_km.mojo,
 * mojo/p7_select_device.mojo, mojo/p7_glint_select_decode.mojo) with no C header; these
 * entry points are additive and carry its layouts, selection rule and summation orders:
 *   hole_k / plug_k [K][N/2] bytes: element (r, c) at byte c * N/2 + r/2, even r in the low nibble;
 *   scales_k [K/64][N] f32: scales_k[(c / 64) * N + r] = absmax[r * K/64 + c / 64];
 *   fold:       y[r] = sum_c (PARENT[h] * scale) * x[c], in slices (see below);
 *   selection:  key = bf16 bits & 0x7FFF, keep every channel with key >= T, T the largest
 *               value such that at least nsel channels have key >= T (ties kept), raised
 *               by a fixed or relational price and lowered to a floor (glint_select_topk_ex);
 *   correction: y[r] += sum_i (CELLS[h][p] - PARENT[h]) * scale * x[c_i] over the kept
 *               channels in ascending order.
 * Fold plus the correction over every channel equals the full-cell GEMV up to the order
 * of the f32 sums.
 *
 * Return codes: 0 success, -1 null pointer, -2 shape or alignment not supported, -3 launch
 * failure.
 * All calls are asynchronous on `stream` and allocate nothing. */
#ifndef GLINT_SELECT_H
#define GLINT_SELECT_H
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif
struct ihipStream_t;

/* Row-major pin planes (bs = 64, element n*K + k) -> K-major hole_k, plug_k (each
 * K*N/2 bytes) and scales_k (N*K/64 floats). N % 8 == 0, K % 64 == 0.
 * Reference: mojo/p7_glint_select_decode.mojo:126-142 (transpose_plug),
 * mojo/p7_select_device.mojo:196-206 (transpose_scales). */
int glint_kmajor_pack(const uint8_t *hole, const uint8_t *plug, const float *absmax, int N, int K, uint8_t *hole_k,
                      uint8_t *plug_k, float *scales_k, struct ihipStream_t *stream);

/* Fold GEMV, f32 out: y[r] = sum_c PARENT[h] * scale * x[c]. Summation order (the
 * reference leaves it to the implementation and validates on its gate): K is cut into ksg
 * equal slices and each slice into 8 equal parts; a part is walked as runs of channels
 * inside one 64-block, acc = fmaf(PARENT[h], x[c], acc) over a run from 0, then
 * t = fmaf(acc, scale, t); the 8 part sums are added in order, then the slices in order.
 * ksg > 1 needs part: ksg * N floats of device scratch (the slices' rows); ksg == 1 writes
 * y directly (part may be NULL). N % 32 == 0, K % (64 * ksg) == 0; x is BF16 bits [K],
 * y f32 [N]; hole_k, scales_k and x 16-B aligned.
 * Reference: mojo/p7_glint_gemv_km.mojo:17-94 (glint_gemv_km, gemv_km_combine). */
int glint_gemv_km_fold(const uint8_t *hole_k, const float *scales_k, const uint16_t *x, float *y, int N, int K,
                       int ksg, float *part, struct ihipStream_t *stream);

/* Channel selection on the device: writes the kept channels of x (BF16 bits [K]) to
 * idx in ascending order (at most K entries) and their number to cnt[0] (and to
 * cnt_log[slot] when cnt_log is not NULL). With key = bits & 0x7FFF and
 * rank(n) = the largest 15-bit T with #{key >= T} >= n (32767 for n <= 0, 0 for n > K):
 *   T = rank(nsel);
 *   tkey > 0 (price): T = max(T, tkey);
 *   tkey < 0 (relational price, tau = -tkey / 1024): T = max(T, key(tau * mean |x|)), the
 *     mean summed in f32 over 1024 ranges of ceil(K / 1024) channels and a pairwise tree,
 *     |x| = (128 + mantissa) 2^(exponent - 134) with the power clamped to [-60, 40] (0 for
 *     zero and subnormal keys), t = (sum / K) * (-tkey) / 1024 in f32, key(t) = biased
 *     exponent << 7 | 7 truncated mantissa bits, clamped to [1, 32767], 1 when t <= 0;
 *   nfloor > 0 and tkey != 0: T = max(rank(nsel), min(T, rank(nfloor)));
 *   nsel == 0: nothing is kept.
 * Every channel with key >= T is kept (ties at T included). 1 <= K <= 32768; slot >= 0
 * when cnt_log is given.
 * Reference: mojo/p7_select_device.mojo:8-151 (select_topk with tkey, nfloor, cnt_log). */
int glint_select_topk_ex(const uint16_t *x, int K, int nsel, int tkey, int nfloor, int32_t *idx, int32_t *cnt,
                         int32_t *cnt_log, int slot, struct ihipStream_t *stream);

/* The rank rule alone: glint_select_topk_ex with tkey = 0, nfloor = 0, no count log.
 * nsel == 0 keeps nothing; nsel >= K keeps everything; nsel < 0 keeps the channels with
 * key 0x7FFF (T = 32767, as the reference's bisection leaves it).
 * Reference: mojo/p7_select_device.mojo:1-151 (select_topk, the rank rule). */
int glint_select_topk(const uint16_t *x, int K, int nsel, int32_t *idx, int32_t *cnt, struct ihipStream_t *stream);

/* Plug correction: y[r] = y[r] + sum over the cnt[0] channels of idx (read on the device;
 * ascending, as glint_select_topk writes them) of (CELLS[h][p] - PARENT[h]) * scale * x[c].
 * Summation order: the list is cut into ks chunks of ceil(cnt / ks), each chunk into 8
 * parts, summed as the fold's parts (runs inside one 64-block, fmaf by the block scale);
 * part sums in order, then chunks in order, then added to y. ks > 1 needs part (ks * N
 * floats of device scratch). N % 32 == 0, K % 64 == 0; hole_k, plug_k, scales_k 16-B
 * aligned; cnt[0] <= K and every idx entry < K.
 * Reference: mojo/p7_select_device.mojo:208-236 (apply_corr_k), 253-302
 * (apply_corr_ks, combine_corr). */
int glint_apply_corr_km(const uint8_t *hole_k, const uint8_t *plug_k, const float *scales_k, const uint16_t *x,
                        const int32_t *idx, const int32_t *cnt, float *y, int N, int K, int ks, float *part,
                        struct ihipStream_t *stream);

#ifdef __cplusplus
}
#endif
#endif
