/* GLINT plug streamer: a 2-slot device ring that streams per-layer plug bytes from pinned
 * host memory while the previous layer computes. MI355X (gfx950) build, in
 * libp7_kernels.so. Reference: include/glint_plug_streamer.h:11-61
 * (cuda/glint_plug_streamer.cu:9-215); same functions, arguments, return codes and
 * ordering rules. Streams are hipStream_t (`struct ihipStream_t *`), the same opaque
 * pointer the reference types as cudaStream_t.
 *
 * Ordering: start() queues layer 0's copy. acquire(l) queues layer l+1's copy into slot
 * (l+1) & 1 on the copy stream, behind the last release of that slot, and makes the
 * compute stream wait for layer l's copy. release(l) marks, on the compute stream, the
 * point after which slot l & 1 may be overwritten. Layers go strictly in order. */
#ifndef GLINT_PLUG_STREAMER_H
#define GLINT_PLUG_STREAMER_H
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif
struct ihipStream_t;

typedef struct GlintPlugStreamer GlintPlugStreamer;

/* Same layout as the reference's stats record. */
typedef struct {
    uint64_t total_h2d_bytes;
    double total_stall_ms;
    double per_layer_stall_ms[64];
    int n_layers;
} GlintStreamerStats;

/* 1 <= n_layers <= 64. Allocates two device slots of max(layer_bytes) and one pinned host
 * buffer per layer. Returns 0; -1 bad argument; -2 out of host memory; -3 device slot or
 * slot event; -4 pinned host buffer; -5 layer event. */
int glint_plug_streamer_create(GlintPlugStreamer **out, int n_layers, const uint64_t *layer_bytes,
                               struct ihipStream_t *copy_stream, struct ihipStream_t *compute_stream);

/* Frees every device and host resource (NULL is ignored). */
void glint_plug_streamer_destroy(GlintPlugStreamer *s);

/* Copies layer `layer`'s plug bytes into its pinned buffer; bytes must equal the size given
 * at create (-2 otherwise; -1 bad argument). */
int glint_plug_streamer_set_host_data(GlintPlugStreamer *s, int layer, const void *host_src, uint64_t bytes);

/* Queues layer 0's copy. -6 while the previous pass has not released its last layer (state
 * is unchanged, so a failed start can be retried); -1 bad argument; -2..-5 runtime errors. */
int glint_plug_streamer_start(GlintPlugStreamer *s);

/* Device pointer of layer `layer`'s plug, valid for work queued on the compute stream.
 * -10 unless layer - 1 was released (or layer == 0 after start); -1 bad argument;
 * -2..-8 runtime errors. */
int glint_plug_streamer_acquire(GlintPlugStreamer *s, int layer, const uint8_t **out_dev_plug);

/* Ends layer `layer`'s reads (call after its last read is queued on the compute stream and
 * before acquire(layer + 1)). -11 unless layer was acquired and layer - 1 released;
 * -1 bad argument; -2 runtime error. */
int glint_plug_streamer_release(GlintPlugStreamer *s, int layer);

/* Synchronises the device, then fills *stats: copied bytes, total and per-layer time the
 * compute stream waited for copies. */
int glint_plug_streamer_get_stats(GlintPlugStreamer *s, GlintStreamerStats *stats);

/* Waits for both streams and clears the recorded statistics. */
void glint_plug_streamer_reset_stats(GlintPlugStreamer *s);

typedef GlintPlugStreamer P7PlugStreamer;
typedef GlintStreamerStats P7StreamerStats;
#define p7_plug_streamer_create glint_plug_streamer_create
#define p7_plug_streamer_destroy glint_plug_streamer_destroy
#define p7_plug_streamer_set_host_data glint_plug_streamer_set_host_data
#define p7_plug_streamer_start glint_plug_streamer_start
#define p7_plug_streamer_acquire glint_plug_streamer_acquire
#define p7_plug_streamer_release glint_plug_streamer_release
#define p7_plug_streamer_get_stats glint_plug_streamer_get_stats
#define p7_plug_streamer_reset_stats glint_plug_streamer_reset_stats

#ifdef __cplusplus
}
#endif
#endif
