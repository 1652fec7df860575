/* launch_glint_htile_bf16_stream_noalloc: launch_glint_htile_bf16_stream for callers that
 * cannot allocate device memory (code under graph capture, serving loops, harnesses that
 * forbid hipMalloc). The split-K partial tiles and arrival counters live in `scratch`, a
 * static array the code object carries, one per GPU and held until the process ends;
 * nothing is allocated per call. Same kernels and the same split plan as the allocating
 * entry point, so the results are identical. Calls that overlap on one GPU share the
 * array and race; the counters are zero after every completed launch. */
#include "glint_common.h"
#include "glint_htile.h"
#include "tile_mfma.h"

int glint_htile_bf16_launch_ws(const uint8_t *d_hole, const uint8_t *d_plug, const float *d_absmax, const void *d_x,
                               uint16_t *d_y, int M, int N, int K, int bs, hipStream_t st, const GlintSplitWs *ws);

/* Counters first, then the f32 partial tiles. The size is what a K-split plan can need on a
 * 256-CU part: 2 x 256 counters and 256 partial tiles of 256 x 256 (64 MiB). A plan that
 * needs more (a part with more CUs) is refused with -5. Stream-K, which needs twice the
 * partials, does not fit and those shapes run whole tiles here. */
#define GLINT_NOALLOC_CTRS 512
#define GLINT_NOALLOC_CTR_BYTES 4096
#define GLINT_NOALLOC_PART_FLOATS (256u * GLINT_SPLIT_TILE_FLOATS_MAX)
#define GLINT_NOALLOC_BYTES (GLINT_NOALLOC_CTR_BYTES + (size_t)GLINT_NOALLOC_PART_FLOATS * sizeof(float))
static_assert(GLINT_NOALLOC_CTRS * sizeof(unsigned) <= GLINT_NOALLOC_CTR_BYTES, "counter area");
static __device__ __align__(256) unsigned char scratch[GLINT_NOALLOC_BYTES];

/* The device address of `scratch` on the current device. The host-side name is only a
 * stand-in, so the address comes from hipGetSymbolAddress, once per device (with that
 * device current), and its counters are zeroed then by a kernel on `st` (a kernel node,
 * not a memset, if the first call is being captured). Returns null on failure. */
static unsigned char *noalloc_scratch(hipStream_t st) {
    static std::mutex mu;
    static unsigned char *ptr[64] = {nullptr};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
        return nullptr;
    std::lock_guard<std::mutex> lock(mu);
    if (ptr[dev] == nullptr) {
        unsigned char *p = nullptr;
        if (hipGetSymbolAddress((void **)&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr)
            return nullptr;
        k_glint_zero_u32<<<1, 256, 0, st>>>((unsigned *)p, GLINT_NOALLOC_CTR_BYTES / sizeof(unsigned));
        if (hipGetLastError() != hipSuccess)
            return nullptr;
        ptr[dev] = p;
    }
    return ptr[dev];
}

GLINT_API int launch_glint_htile_bf16_stream_noalloc(const uint8_t *d_hole, const uint8_t *d_plug,
                                                     const float *d_absmax, const void *d_x, uint16_t *d_y, int M,
                                                     int N, int K, int bs, struct ihipStream_t *stream) {
    if (!d_hole || !d_plug || !d_absmax || !d_x || !d_y)
        return -1;
    unsigned char *sp = noalloc_scratch((hipStream_t)stream);
    if (sp == nullptr)
        return -3;
    const GlintSplitWs ws{(float *)(sp + GLINT_NOALLOC_CTR_BYTES), (unsigned *)sp, GLINT_NOALLOC_PART_FLOATS,
                          GLINT_NOALLOC_CTRS};
    return glint_htile_bf16_launch_ws(d_hole, d_plug, d_absmax, d_x, d_y, M, N, K, bs, (hipStream_t)stream, &ws);
}
