/* A C++ caller of the GLINT C ABI, compiled against include/glint_encode.h and
 * include/glint_htile.h and linked with -lglint_encode: the way the reference's own C/C++
 * tests reach the library (no ctypes, no torch). It restates, with the HIP runtime for
 * device memory:
 *
 *   gpu_ok    the glint_cuda.gpu_ok probe through glint_encode_bf16_host: BF16 [1.0, 0.0],
 *             bs 64 -> hole 0x7F, plug 0x8F, absmax 1.0 (reference glint_cuda.py:52-58).
 *   expand    glint_expand_packed_to_f32_device on a stream against
 *             glint_expand_packed_to_f32_host and against CELLS[h][p] * absmax on the host.
 *   kbounds   reference tests/test_htile_k_bounds_device.cu:40-118: shift 0/1 (pointers one
 *             element into larger buffers), K in {1 .. 256}, 5 shapes, bs 23, canaries
 *             around y, 3 launches per case, |y - ref| <= 1e-5 (1 + |ref|) against float64.
 *   ten       reference tests/test_glint_htile.cu:63-153: ten shapes, max |y - f32 CPU| < 1e-3.
 *   prefill   launch_glint_htile_s3_f32_stream at M > 1 on the aligned bs = 64 path
 *             (the MFMA route) on a stream, within the f32 summation bound
 *             (K + 2) 2^-23 sum |terms| of float64 (test_streamer_real_weights.cu:130-133).
 *
 * Usage: abi_caller [suite ...]   (no argument: every suite). Exit 0 when all pass; each
 * case prints its name before its first launch. */
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "glint_cells.h"
#include "glint_encode.h"
#include "glint_htile.h"

static void hip_ok(hipError_t e, const char *what) {
    if (e != hipSuccess) {
        std::fprintf(stderr, "HIP FAIL %s: %s\n", what, hipGetErrorString(e));
        std::exit(3);
    }
}

static uint16_t to_bf16(float f) { /* round to nearest even (no NaN inputs here) */
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}
static float from_bf16(uint16_t b) {
    const uint32_t u = (uint32_t)b << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

/* A device copy of `v` placed `shift` elements into a larger allocation. */
template <typename T>
struct DevBuf {
    T *base = nullptr, *ptr = nullptr;
    DevBuf(const std::vector<T> &v, int shift = 0) {
        hip_ok(hipMalloc((void **)&base, (v.size() + shift + 1) * sizeof(T)), "hipMalloc");
        hip_ok(hipMemset(base, 0, (v.size() + shift + 1) * sizeof(T)), "hipMemset");
        ptr = base + shift;
        if (!v.empty())
            hip_ok(hipMemcpy(ptr, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice), "H2D");
    }
    ~DevBuf() { (void)hipFree(base); }
    std::vector<T> get(size_t n) const {
        std::vector<T> out(n);
        hip_ok(hipDeviceSynchronize(), "sync");
        hip_ok(hipMemcpy(out.data(), ptr, n * sizeof(T), hipMemcpyDeviceToHost), "D2H");
        return out;
    }
};

static int suite_gpu_ok() {
    std::printf("case gpu_ok\n");
    std::fflush(stdout);
    const uint16_t w[2] = {0x3F80, 0x0000};
    uint8_t hole = 0, plug = 0;
    float am = 0.f;
    const int rc = glint_encode_bf16_host(w, 2, 64, &hole, &plug, &am);
    if (rc != 0 || hole != 0x7F || plug != 0x8F || am != 1.0f) {
        std::fprintf(stderr, "GPU_OK FAIL rc=%d hole=%02x plug=%02x absmax=%g\n", rc, hole, plug, am);
        return 1;
    }
    if (glint_encode_n_packed(2) != 1 || glint_encode_n_absmax(2, 64) != 1 || glint_encode_n_absmax(5, 0) != 0) {
        std::fprintf(stderr, "SIZE HELPERS FAIL\n");
        return 1;
    }
    std::printf("PASS gpu_ok hole=0x7f plug=0x8f absmax=1\n");
    return 0;
}

static int suite_expand() {
    const int64_t n = 64 * 1000 + 37;
    const int bs = 64;
    std::printf("case expand n=%lld bs=%d\n", (long long)n, bs);
    std::fflush(stdout);
    std::vector<uint8_t> hole((n + 1) / 2), plug((n + 1) / 2);
    std::vector<float> am((n + bs - 1) / bs);
    for (size_t i = 0; i < hole.size(); ++i) {
        hole[i] = (uint8_t)((i * 7 + 1) % 256);
        plug[i] = (uint8_t)((i * 13 + 5) % 256);
    }
    if (n & 1) { /* the pad nibble is zero */
        hole.back() &= 0x0F;
        plug.back() &= 0x0F;
    }
    for (size_t b = 0; b < am.size(); ++b)
        am[b] = 0.5f + (float)(b % 10) * 0.1f;
    std::vector<float> want(n), host_out(n);
    for (int64_t i = 0; i < n; ++i)
        want[i] = GLINT_CELLS[(hole[i >> 1] >> (4 * (i & 1))) & 15][(plug[i >> 1] >> (4 * (i & 1))) & 15] * am[i / bs];
    if (glint_expand_packed_to_f32_host(hole.data(), plug.data(), am.data(), n, bs, host_out.data()) != 0) {
        std::fprintf(stderr, "EXPAND HOST FAIL\n");
        return 1;
    }
    DevBuf<uint8_t> dh(hole), dp(plug);
    DevBuf<float> da(am), dy(std::vector<float>(n, 0.f));
    hipStream_t st;
    hip_ok(hipStreamCreate(&st), "stream");
    const int rc = glint_expand_packed_to_f32_device(dh.ptr, dp.ptr, da.ptr, n, bs, dy.ptr, st);
    hip_ok(hipStreamSynchronize(st), "stream sync");
    hip_ok(hipStreamDestroy(st), "stream destroy");
    const std::vector<float> dev_out = dy.get(n);
    if (rc != 0 || std::memcmp(dev_out.data(), want.data(), n * 4) || std::memcmp(host_out.data(), want.data(), n * 4)) {
        std::fprintf(stderr, "EXPAND FAIL rc=%d\n", rc);
        return 1;
    }
    std::printf("PASS expand host == device == CELLS[h][p] * absmax (%lld elements)\n", (long long)n);
    return 0;
}

/* The reference k-bounds inputs: deterministic nibbles and scales, x on a 1/16 grid. */
static void kbounds_inputs(int M, int N, int K, int bs, std::vector<uint8_t> &hole, std::vector<uint8_t> &plug,
                           std::vector<float> &scales, std::vector<float> &weights, std::vector<uint16_t> &x) {
    hole.assign(((int64_t)N * K + 1) / 2, 0);
    plug.assign(hole.size(), 0);
    scales.resize(((int64_t)N * K + bs - 1) / bs);
    weights.resize((size_t)N * K);
    x.resize((size_t)M * K);
    for (size_t b = 0; b < scales.size(); ++b)
        scales[b] = 0.25f + (float)(b % 7) * 0.125f;
    for (int64_t i = 0; i < (int64_t)N * K; ++i) {
        const uint8_t h = (uint8_t)((i * 7 + i / 17 + 3) % 16), p = (uint8_t)((i * 11 + i / 13 + 5) % 16);
        hole[i / 2] |= (uint8_t)(h << (4 * (i % 2)));
        plug[i / 2] |= (uint8_t)(p << (4 * (i % 2)));
        weights[i] = GLINT_CELLS[h][p] * scales[i / bs];
    }
    for (int64_t i = 0; i < (int64_t)M * K; ++i)
        x[i] = to_bf16((float)((i * 3 + i / 19) % 17 - 8) * 0.0625f);
}

/* y against the float64 sum of weight * x; returns the worst |error|, or -1 on a miss.
 * Bound: 1e-5 (1 + |ref|) (test_htile_k_bounds_device.cu:98), or with sum_bound the f32
 * summation bound (K + 2) 2^-23 sum |terms| (test_streamer_real_weights.cu:130-133). */
static double check_f64(const std::vector<float> &y, size_t y0, const std::vector<float> &weights,
                        const std::vector<uint16_t> &x, int M, int N, int K, const char *tag, bool sum_bound = false) {
    double worst = 0;
    for (int m = 0; m < M; ++m)
        for (int n = 0; n < N; ++n) {
            double ref = 0, asum = 0;
            for (int k = 0; k < K; ++k) {
                const double t = (double)weights[(size_t)n * K + k] * (double)from_bf16(x[(size_t)m * K + k]);
                ref += t;
                asum += std::fabs(t);
            }
            const double got = y[y0 + (size_t)m * N + n], err = std::fabs(got - ref);
            const double bound = sum_bound ? (K + 2) * std::ldexp(1.0, -23) * asum : 1e-5 * (1 + std::fabs(ref));
            worst = std::max(worst, err);
            if (!std::isfinite(got) || err > bound) {
                std::fprintf(stderr, "MATH FAIL %s M=%d N=%d K=%d m=%d n=%d got=%.12g ref=%.12g\n", tag, M, N, K, m,
                             n, got, ref);
                return -1;
            }
        }
    return worst;
}

static int suite_kbounds() {
    const int bs = 23, guard = 16;
    const float canary = 123456.0f;
    const int shapes[5][2] = {{1, 1}, {15, 15}, {16, 16}, {17, 19}, {33, 31}};
    int cases = 0;
    for (int shift : {0, 1})
        for (int K : {1, 32, 40, 48, 63, 64, 65, 192, 199, 256}) {
            std::printf("case kbounds shift=%d K=%d\n", shift, K);
            std::fflush(stdout);
            double worst = 0;
            for (const auto &s : shapes) {
                const int M = s[0], N = s[1];
                std::vector<uint8_t> hole, plug;
                std::vector<float> scales, weights;
                std::vector<uint16_t> x;
                kbounds_inputs(M, N, K, bs, hole, plug, scales, weights, x);
                DevBuf<uint8_t> dh(hole, shift), dp(plug, shift);
                DevBuf<float> ds(scales);
                DevBuf<uint16_t> dx(x, shift);
                DevBuf<float> dy(std::vector<float>((size_t)M * N + 2 * guard, canary));
                for (int rep = 0; rep < 3; ++rep) {
                    const int rc = launch_glint_htile_s3_f32(dh.ptr, dp.ptr, ds.ptr, dx.ptr, dy.ptr + guard, M, N, K, bs);
                    if (rc != 0) {
                        std::fprintf(stderr, "LAUNCH FAIL rc=%d M=%d N=%d K=%d\n", rc, M, N, K);
                        return 1;
                    }
                    const std::vector<float> y = dy.get((size_t)M * N + 2 * guard);
                    for (int g = 0; g < guard; ++g)
                        if (y[g] != canary || y[guard + (size_t)M * N + g] != canary) {
                            std::fprintf(stderr, "CANARY FAIL M=%d N=%d K=%d\n", M, N, K);
                            return 1;
                        }
                    const double w = check_f64(y, guard, weights, x, M, N, K, "kbounds");
                    if (w < 0)
                        return 1;
                    worst = std::max(worst, w);
                }
                ++cases;
            }
            std::printf("PASS kbounds shift=%d K=%d shapes=5 repetitions=3 max_abs_error=%.9g canaries=PASS\n", shift,
                        K, worst);
        }
    std::printf("PASS kbounds cases=%d launches=%d\n", cases, 3 * cases);
    return 0;
}

/* reference tests/test_glint_htile.cu cpu_reference: f32 sums in k order */
static int ten_case(int M, int N, int K, int bs) {
    std::printf("case ten M=%d N=%d K=%d bs=%d\n", M, N, K, bs);
    std::fflush(stdout);
    const int64_t nx = (int64_t)M * K, nw = (int64_t)N * K, npk = (nw + 1) / 2, nam = (nw + bs - 1) / bs;
    std::vector<uint16_t> x(nx);
    std::vector<float> xf(nx), am(nam);
    std::vector<uint8_t> hole(npk), plug(npk);
    for (int64_t i = 0; i < nx; ++i) {
        xf[i] = ((float)((i * 17 + 3) % 100) - 50.0f) * 0.01f;
        x[i] = to_bf16(xf[i]);
    }
    for (int64_t i = 0; i < npk; ++i) {
        hole[i] = (uint8_t)((i * 7 + 1) % 256);
        plug[i] = (uint8_t)((i * 13 + 5) % 256);
    }
    for (int64_t i = 0; i < nam; ++i)
        am[i] = 0.5f + (float)(i % 10) * 0.1f;
    std::vector<float> ref((size_t)M * N);
    for (int m = 0; m < M; ++m)
        for (int n = 0; n < N; ++n) {
            float acc = 0.f;
            for (int k = 0; k < K; ++k) {
                const int64_t i = (int64_t)n * K + k;
                const float w = GLINT_CELLS[(hole[i >> 1] >> (4 * (i & 1))) & 15][(plug[i >> 1] >> (4 * (i & 1))) & 15] *
                                am[i / bs];
                acc += w * from_bf16(x[(size_t)m * K + k]);
            }
            ref[(size_t)m * N + n] = acc;
        }
    DevBuf<uint8_t> dh(hole), dp(plug);
    DevBuf<float> da(am), dy(std::vector<float>((size_t)M * N, 0.f));
    DevBuf<uint16_t> dx(x);
    const int rc = launch_glint_htile_s3_f32(dh.ptr, dp.ptr, da.ptr, dx.ptr, dy.ptr, M, N, K, bs);
    if (rc != 0) {
        std::fprintf(stderr, "LAUNCH FAIL rc=%d\n", rc);
        return 1;
    }
    const std::vector<float> y = dy.get((size_t)M * N);
    float md = 0.f;
    for (size_t i = 0; i < y.size(); ++i)
        md = std::max(md, std::fabs(y[i] - ref[i]));
    std::printf("%s ten M=%d N=%d K=%d max_diff=%.6e\n", md < 1e-3f ? "PASS" : "FAIL", M, N, K, md);
    return md < 1e-3f ? 0 : 1;
}

static int suite_ten() {
    const int cases[10][4] = {{16, 16, 64, 64}, {16, 16, 128, 64}, {32, 32, 192, 64}, {16, 16, 32, 64},
                              {16, 16, 48, 64}, {16, 16, 40, 64},  {16, 16, 70, 64},  {16, 16, 100, 64},
                              {7, 23, 64, 64},  {4, 3072, 3072, 64}};
    int failed = 0;
    for (const auto &c : cases)
        failed += ten_case(c[0], c[1], c[2], c[3]);
    return failed ? 1 : 0;
}

static int suite_prefill() {
    const int shapes[][3] = {{2, 64, 64}, {70, 300, 4096}, {257, 129, 1088}, {64, 4096, 2048}};
    hipStream_t st;
    hip_ok(hipStreamCreate(&st), "stream");
    for (const auto &s : shapes) {
        const int M = s[0], N = s[1], K = s[2];
        std::printf("case prefill f32 M=%d N=%d K=%d bs=64\n", M, N, K);
        std::fflush(stdout);
        std::vector<uint8_t> hole, plug;
        std::vector<float> scales, weights;
        std::vector<uint16_t> x;
        kbounds_inputs(M, N, K, 64, hole, plug, scales, weights, x);
        DevBuf<uint8_t> dh(hole), dp(plug);
        DevBuf<float> ds(scales), dy(std::vector<float>((size_t)M * N, 0.f));
        DevBuf<uint16_t> dx(x);
        const int rc = launch_glint_htile_s3_f32_stream(dh.ptr, dp.ptr, ds.ptr, dx.ptr, dy.ptr, M, N, K, 64, st);
        hip_ok(hipStreamSynchronize(st), "stream sync");
        if (rc != 0) {
            std::fprintf(stderr, "LAUNCH FAIL rc=%d\n", rc);
            return 1;
        }
        const double w = check_f64(dy.get((size_t)M * N), 0, weights, x, M, N, K, "prefill", true);
        if (w < 0)
            return 1;
        std::printf("PASS prefill f32 M=%d N=%d K=%d max_abs_error=%.9g\n", M, N, K, w);
    }
    hip_ok(hipStreamDestroy(st), "stream destroy");
    return 0;
}

int main(int argc, char **argv) {
    struct Suite {
        const char *name;
        int (*run)();
    } suites[] = {{"gpu_ok", suite_gpu_ok}, {"expand", suite_expand}, {"kbounds", suite_kbounds},
                  {"ten", suite_ten}, {"prefill", suite_prefill}};
    int failed = 0, ran = 0;
    for (const Suite &s : suites) {
        bool want = argc < 2;
        for (int i = 1; i < argc; ++i)
            want = want || std::string(argv[i]) == s.name;
        if (!want)
            continue;
        ++ran;
        if (s.run() != 0) {
            std::printf("FAIL suite %s\n", s.name);
            ++failed;
        }
    }
    std::printf("%s abi_caller suites=%d failed=%d\n", failed || !ran ? "FAIL" : "PASS", ran, failed);
    return failed || !ran ? 1 : 0;
}
