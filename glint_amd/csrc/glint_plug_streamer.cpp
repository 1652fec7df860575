/* GLINT plug streamer on HIP: per-layer plug bytes staged in pinned host buffers and
 * streamed into a 2-slot device ring on a copy stream, ordered against the compute stream
 * with events only (no host waits on the hot path).
 *
 * Protocol (reference cuda/glint_plug_streamer.cu:9-215, same return codes):
 *   start()      copy stream: wait slot_free[0]; copy layer 0 -> slot 0; mark copied[0]
 *   acquire(l)   copy stream: wait slot_free[(l+1)&1]; copy layer l+1 -> that slot; mark
 *                copied[l+1]; compute stream: wait copied[l] (timed as layer l's stall)
 *   release(l)   compute stream: mark slot_free[l&1]
 * so a slot is only refilled after every compute-stream read queued before its release. */
#include <hip/hip_runtime.h>
#include <string.h>

#include "glint_plug_streamer.h"

#define PS_API extern "C" __attribute__((visibility("default")))

namespace {
constexpr int kMaxLayers = 64;
}

struct GlintPlugStreamer {
    int n_layers = 0;
    uint64_t bytes[kMaxLayers] = {};
    uint64_t slot_bytes = 0;
    uint8_t *host[kMaxLayers] = {};
    uint8_t *slot[2] = {};
    hipStream_t copy = nullptr, compute = nullptr;
    hipEvent_t slot_free[2] = {};
    hipEvent_t copy_begin[kMaxLayers] = {}, copied[kMaxLayers] = {};
    hipEvent_t wait_begin[kMaxLayers] = {}, wait_end[kMaxLayers] = {};
    bool waited[kMaxLayers] = {};
    /* last layer acquired / released in the current pass; both n_layers - 1 between passes */
    int acquired = -1, released = -1;
    GlintStreamerStats stats = {};
};

/* Queue layer l's host -> slot copy on the copy stream behind the slot's last release.
 * The four codes are the caller's for: the wait, the start mark, the copy, the end mark. */
static int ps_queue_copy(GlintPlugStreamer *s, int l, int e_wait, int e_mark0, int e_copy, int e_mark1) {
    const int slot = l & 1;
    if (hipStreamWaitEvent(s->copy, s->slot_free[slot], 0) != hipSuccess)
        return e_wait;
    if (hipEventRecord(s->copy_begin[l], s->copy) != hipSuccess)
        return e_mark0;
    if (s->bytes[l] &&
        hipMemcpyAsync(s->slot[slot], s->host[l], (size_t)s->bytes[l], hipMemcpyHostToDevice, s->copy) != hipSuccess)
        return e_copy;
    if (hipEventRecord(s->copied[l], s->copy) != hipSuccess)
        return e_mark1;
    s->stats.total_h2d_bytes += s->bytes[l];
    return 0;
}

PS_API void glint_plug_streamer_destroy(GlintPlugStreamer *s) {
    if (!s)
        return;
    for (int b = 0; b < 2; ++b) {
        if (s->slot[b])
            (void)hipFree(s->slot[b]);
        if (s->slot_free[b])
            (void)hipEventDestroy(s->slot_free[b]);
    }
    for (int l = 0; l < s->n_layers; ++l) {
        if (s->host[l])
            (void)hipHostFree(s->host[l]);
        hipEvent_t *ev[4] = {&s->copy_begin[l], &s->copied[l], &s->wait_begin[l], &s->wait_end[l]};
        for (hipEvent_t *e : ev)
            if (*e)
                (void)hipEventDestroy(*e);
    }
    delete s;
}

PS_API int glint_plug_streamer_create(GlintPlugStreamer **out, int n_layers, const uint64_t *layer_bytes,
                                      struct ihipStream_t *copy_stream, struct ihipStream_t *compute_stream) {
    if (!out || !layer_bytes || n_layers < 1 || n_layers > kMaxLayers)
        return -1;
    GlintPlugStreamer *s = new (std::nothrow) GlintPlugStreamer;
    if (!s)
        return -2;
    s->n_layers = n_layers;
    s->copy = (hipStream_t)copy_stream;
    s->compute = (hipStream_t)compute_stream;
    for (int l = 0; l < n_layers; ++l) {
        s->bytes[l] = layer_bytes[l];
        if (layer_bytes[l] > s->slot_bytes)
            s->slot_bytes = layer_bytes[l];
    }
    for (int b = 0; b < 2; ++b)
        if (hipMalloc((void **)&s->slot[b], s->slot_bytes ? (size_t)s->slot_bytes : 1) != hipSuccess ||
            hipEventCreateWithFlags(&s->slot_free[b], hipEventDisableTiming) != hipSuccess) {
            glint_plug_streamer_destroy(s);
            return -3;
        }
    for (int l = 0; l < n_layers; ++l) {
        if (hipHostMalloc((void **)&s->host[l], s->bytes[l] ? (size_t)s->bytes[l] : 1, hipHostMallocDefault) !=
            hipSuccess) {
            glint_plug_streamer_destroy(s);
            return -4;
        }
        if (hipEventCreate(&s->copy_begin[l]) != hipSuccess || hipEventCreate(&s->copied[l]) != hipSuccess ||
            hipEventCreate(&s->wait_begin[l]) != hipSuccess || hipEventCreate(&s->wait_end[l]) != hipSuccess) {
            glint_plug_streamer_destroy(s);
            return -5;
        }
    }
    s->acquired = s->released = n_layers - 1;
    s->stats.n_layers = n_layers;
    *out = s;
    return 0;
}

PS_API int glint_plug_streamer_set_host_data(GlintPlugStreamer *s, int layer, const void *host_src, uint64_t bytes) {
    if (!s || !host_src || layer < 0 || layer >= s->n_layers)
        return -1;
    if (bytes != s->bytes[layer])
        return -2;
    memcpy(s->host[layer], host_src, (size_t)bytes);
    return 0;
}

PS_API int glint_plug_streamer_start(GlintPlugStreamer *s) {
    if (!s || s->n_layers < 1)
        return -1;
    if (s->released != s->n_layers - 1)
        return -6;
    const int rc = ps_queue_copy(s, 0, -5, -2, -3, -4);
    if (rc)
        return rc;
    s->acquired = s->released = -1;
    return 0;
}

PS_API int glint_plug_streamer_acquire(GlintPlugStreamer *s, int layer, const uint8_t **out_dev_plug) {
    if (!s || !out_dev_plug || layer < 0 || layer >= s->n_layers)
        return -1;
    if (s->released != layer - 1)
        return -10;
    if (layer + 1 < s->n_layers) {
        const int rc = ps_queue_copy(s, layer + 1, -2, -3, -4, -5);
        if (rc)
            return rc;
    }
    if (hipEventRecord(s->wait_begin[layer], s->compute) != hipSuccess)
        return -6;
    if (hipStreamWaitEvent(s->compute, s->copied[layer], 0) != hipSuccess)
        return -7;
    if (hipEventRecord(s->wait_end[layer], s->compute) != hipSuccess)
        return -8;
    s->waited[layer] = true;
    s->acquired = layer;
    *out_dev_plug = s->slot[layer & 1];
    return 0;
}

PS_API int glint_plug_streamer_release(GlintPlugStreamer *s, int layer) {
    if (!s || layer < 0 || layer >= s->n_layers)
        return -1;
    if (layer != s->released + 1 || layer != s->acquired)
        return -11;
    if (hipEventRecord(s->slot_free[layer & 1], s->compute) != hipSuccess)
        return -2;
    s->released = layer;
    return 0;
}

PS_API int glint_plug_streamer_get_stats(GlintPlugStreamer *s, GlintStreamerStats *stats) {
    if (!s || !stats)
        return -1;
    (void)hipDeviceSynchronize();
    double total = 0.0;
    for (int l = 0; l < s->n_layers; ++l) {
        float ms = 0.0f;
        if (!s->waited[l] || hipEventElapsedTime(&ms, s->wait_begin[l], s->wait_end[l]) != hipSuccess)
            ms = 0.0f;
        s->stats.per_layer_stall_ms[l] = (double)ms;
        total += (double)ms;
    }
    s->stats.total_stall_ms = total;
    *stats = s->stats;
    return 0;
}

PS_API void glint_plug_streamer_reset_stats(GlintPlugStreamer *s) {
    if (!s)
        return;
    (void)hipStreamSynchronize(s->copy);
    (void)hipStreamSynchronize(s->compute);
    s->stats.total_h2d_bytes = 0;
    s->stats.total_stall_ms = 0.0;
    memset(s->stats.per_layer_stall_ms, 0, sizeof(s->stats.per_layer_stall_ms));
}
