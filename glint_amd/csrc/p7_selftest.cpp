/* p7_abi_selftest: the attach gate's check of this library, run through its own exported
 * entry points. A 4-layer INT8 stack (weights quantized with the pin rule) runs once with
 * every layer resident and once streamed through the plug streamer's 2-slot ring, both on
 * int8_mma_gemm. Passes (returns 0) only if the two outputs are bitwise equal, finite,
 * mostly non-zero, within 1e-4 relative of a CPU float model of the kernel arithmetic, and
 * the streamer copied exactly the layer bytes. Reference: cuda/p7_abi_selftest.cu:46-142
 * (same checks and return codes: -1 runtime, -2 GEMM, -3 streamer setup, -4 streamer
 * ordering, -5 mismatch or non-finite, -6 mostly zero, -7 CPU model, -8 byte count). */
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdio.h>
#include <string.h>

#include <vector>

#include "glint_plug_streamer.h"
#include "int8_mma_gemm.h"
#include "p7_attach.h"

#define P7_API extern "C" __attribute__((visibility("default")))

namespace {
constexpr int kLayers = 4, kM = 70, kK = 256, kN = 192, kKB = kK / 64;

/* xorshift32 -> uniform in [-1, 1) */
struct Rng {
    uint32_t s;
    float next() {
        s ^= s << 13;
        s ^= s >> 17;
        s ^= s << 5;
        return (float)(s >> 8) * (1.0f / 8388608.0f) - 1.0f;
    }
};

uint16_t bf16_rne(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}
float bf16_val(uint16_t b) {
    const uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* The pin rule per (row, 64-block): s = amax > 0 ? amax / 127 : 1, q = clamp(rint(v / s)). */
void quantize_rows(const float *v, int rows, int8_t *q, float *s) {
    for (int r = 0; r < rows; ++r)
        for (int kb = 0; kb < kKB; ++kb) {
            const float *b = v + (size_t)r * kK + kb * 64;
            float am = 0.0f;
            for (int j = 0; j < 64; ++j)
                am = fmaxf(am, fabsf(b[j]));
            const float sc = am > 0.0f ? am / 127.0f : 1.0f;
            s[(size_t)r * kKB + kb] = sc;
            for (int j = 0; j < 64; ++j) {
                int t = (int)rintf(b[j] / sc);
                t = t > 127 ? 127 : (t < -127 ? -127 : t);
                q[(size_t)r * kK + kb * 64 + j] = (int8_t)t;
            }
        }
}

/* device allocations released when the test returns */
struct DeviceBuffers {
    void *p[8] = {};
    int n = 0;
    template <typename T>
    bool alloc(T **ptr, size_t bytes) {
        if (n == 8 || hipMalloc((void **)ptr, bytes) != hipSuccess)
            return false;
        p[n++] = *ptr;
        return true;
    }
    ~DeviceBuffers() {
        for (int i = 0; i < n; ++i)
            (void)hipFree(p[i]);
    }
};
}  // namespace

P7_API int p7_abi_selftest(char *msg, size_t msg_n) {
    const size_t qbytes = (size_t)kN * kK, qpad = (qbytes + 255) / 256 * 256;
    const size_t blob = qpad + (size_t)kN * kKB * sizeof(float);
    std::vector<uint8_t> host(kLayers * blob, 0);
    Rng rng{0x2545F491u};
    std::vector<float> w((size_t)kN * kK);
    for (int l = 0; l < kLayers; ++l) {
        for (float &v : w)
            v = 0.04f * rng.next() * (1.0f + 0.5f * l);
        uint8_t *b = host.data() + l * blob;
        quantize_rows(w.data(), kN, (int8_t *)b, (float *)(b + qpad));
    }
    std::vector<uint16_t> xb((size_t)kM * kK);
    for (uint16_t &v : xb)
        v = bf16_rne(rng.next());

    DeviceBuffers d;
    uint16_t *dx;
    float *dy_res, *dy_str, *dsx;
    int8_t *dxq;
    uint8_t *dblob;
    if (!d.alloc(&dx, xb.size() * 2) || !d.alloc(&dy_res, (size_t)kM * kN * 4) ||
        !d.alloc(&dy_str, (size_t)kM * kN * 4) || !d.alloc(&dxq, int8_mma_xq_bytes(kM, kK)) ||
        !d.alloc(&dsx, int8_mma_sx_bytes(kM, kK)) || !d.alloc(&dblob, host.size()))
        return -1;
    if (hipMemcpy(dx, xb.data(), xb.size() * 2, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(dblob, host.data(), host.size(), hipMemcpyHostToDevice) != hipSuccess)
        return -1;

    /* pass 1: every layer resident */
    std::vector<float> res((size_t)kLayers * kM * kN), str(res.size());
    for (int l = 0; l < kLayers; ++l) {
        const uint8_t *b = dblob + l * blob;
        const Int8MmaLinear lin = {(const int8_t *)b, (const float *)(b + qpad), kN, kK};
        if (int8_mma_gemm(dx, lin, dy_res, kM, dxq, dsx, nullptr) != 0)
            return -2;
        if (hipMemcpy(res.data() + (size_t)l * kM * kN, dy_res, (size_t)kM * kN * 4, hipMemcpyDeviceToHost) !=
            hipSuccess)
            return -1;
    }

    /* pass 2: layers streamed through the ring */
    hipStream_t cs = nullptr, ks = nullptr;
    if (hipStreamCreateWithFlags(&cs, hipStreamNonBlocking) != hipSuccess)
        return -1;
    if (hipStreamCreateWithFlags(&ks, hipStreamNonBlocking) != hipSuccess) {
        (void)hipStreamDestroy(cs);
        return -1;
    }
    int rc = 0;
    GlintStreamerStats st = {};
    {
        uint64_t lb[kLayers];
        for (int l = 0; l < kLayers; ++l)
            lb[l] = blob;
        GlintPlugStreamer *s = nullptr;
        if (glint_plug_streamer_create(&s, kLayers, lb, (struct ihipStream_t *)cs, (struct ihipStream_t *)ks) != 0)
            rc = -3;
        for (int l = 0; !rc && l < kLayers; ++l)
            if (glint_plug_streamer_set_host_data(s, l, host.data() + l * blob, blob) != 0)
                rc = -3;
        if (!rc && glint_plug_streamer_start(s) != 0)
            rc = -4;
        for (int l = 0; !rc && l < kLayers; ++l) {
            const uint8_t *b = nullptr;
            if (glint_plug_streamer_acquire(s, l, &b) != 0) {
                rc = -4;
                break;
            }
            const Int8MmaLinear lin = {(const int8_t *)b, (const float *)(b + qpad), kN, kK};
            if (int8_mma_gemm(dx, lin, dy_str, kM, dxq, dsx, (struct ihipStream_t *)ks) != 0) {
                rc = -2;
                break;
            }
            if (hipMemcpyAsync(str.data() + (size_t)l * kM * kN, dy_str, (size_t)kM * kN * 4, hipMemcpyDeviceToHost,
                               ks) != hipSuccess ||
                hipStreamSynchronize(ks) != hipSuccess) {
                rc = -1;
                break;
            }
            if (glint_plug_streamer_release(s, l) != 0)
                rc = -4;
        }
        if (s) {
            (void)glint_plug_streamer_get_stats(s, &st);
            glint_plug_streamer_destroy(s);
        }
    }
    (void)hipStreamDestroy(cs);
    (void)hipStreamDestroy(ks);
    if (rc)
        return rc;

    long mism = 0, nonfin = 0, nonzero = 0;
    for (size_t i = 0; i < res.size(); ++i) {
        mism += memcmp(&res[i], &str[i], 4) != 0;
        nonfin += !isfinite(res[i]);
        nonzero += res[i] != 0.0f;
    }
    /* CPU model of the kernel arithmetic on layer 0 */
    double maxrel = 0.0;
    {
        const int8_t *wq = (const int8_t *)host.data();
        const float *sw = (const float *)(host.data() + qpad);
        std::vector<float> x((size_t)kM * kK), sx((size_t)kM * kKB);
        std::vector<int8_t> xq((size_t)kM * kK);
        for (size_t i = 0; i < x.size(); ++i)
            x[i] = bf16_val(xb[i]);
        quantize_rows(x.data(), kM, xq.data(), sx.data());
        for (int mi = 0; mi < kM; ++mi)
            for (int ni = 0; ni < kN; ++ni) {
                float acc = 0.0f;
                for (int kb = 0; kb < kKB; ++kb) {
                    int ic = 0;
                    for (int j = 0; j < 64; ++j)
                        ic += (int)xq[(size_t)mi * kK + kb * 64 + j] * (int)wq[(size_t)ni * kK + kb * 64 + j];
                    acc = fmaf((float)ic * sx[(size_t)mi * kKB + kb], sw[(size_t)ni * kKB + kb], acc);
                }
                const double got = res[(size_t)mi * kN + ni], err = fabs(got - (double)acc);
                const double rel = err / (fabs((double)acc) + 1e-6);
                if (err > 1e-6 && rel > maxrel)
                    maxrel = rel;
            }
    }
    if (msg && msg_n)
        snprintf(msg, msg_n,
                 "abi=%s layers=%d streamed_bytes=%llu mismatches=%ld nonfinite=%ld nonzero=%ld/%zu cpu_max_rel=%.3e",
                 p7_abi_version(), kLayers, (unsigned long long)st.total_h2d_bytes, mism, nonfin, nonzero, res.size(),
                 maxrel);
    if (mism || nonfin)
        return -5;
    if (nonzero < (long)(res.size() / 2))
        return -6;
    if (maxrel > 1e-4)
        return -7;
    if (st.total_h2d_bytes != (uint64_t)kLayers * blob)
        return -8;
    return 0;
}
