/* HBM read ceiling for bench.py (measurement only; not part of the GLINT ABI).
 *
 * k_read_stream reads `bytes` (a multiple of 16, 16-B aligned) once, grid-stride over 16-B
 * words with 1024-thread workgroups, and folds what it reads into one word per thread that
 * it stores only if the fold hits a value the caller's data never produces (so nothing is
 * written, and nothing the compiler can drop is skipped). The same grid shape read a GEMV
 * pin's 62.4 MB in 10.5 us on one MI355X, the fastest of the grid-stride and per-row shapes
 * tried, so it stands for what a read-only pass over those bytes can reach. */
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef uint32_t probe_u32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(1024) void k_read_stream(const probe_u32x4 *__restrict__ p, int64_t n16,
                                                      uint32_t *__restrict__ sink) {
    uint32_t acc = 0;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) {
        const probe_u32x4 v = __builtin_nontemporal_load(&p[i]);
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (acc == 0x9E3779B9u)
        sink[(int64_t)blockIdx.x * blockDim.x + threadIdx.x] = acc;
}

/* Reads p[0 .. bytes) with `grid` workgroups of 1024 threads on `stream`. `sink` must hold
 * grid * 1024 words. Returns 0, -1 for a bad argument, -3 for a launch error. */
extern "C" __attribute__((visibility("default"))) int glint_probe_read(const void *p, int64_t bytes, uint32_t *sink,
                                                                     int grid, hipStream_t stream) {
    if (!p || !sink || bytes <= 0 || bytes % 16 != 0 || ((uintptr_t)p & 15) != 0 || grid < 1)
        return -1;
    k_read_stream<<<grid, 1024, 0, stream>>>((const probe_u32x4 *)p, bytes / 16, sink);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}
