"""GPU INT8 parity.

int8_mma_gemm (attach ABI): quantized activation bytes identical to the oracle
(test_int8_mma_gemm.cu:127-132) and y bit-identical to the oracle's emulation of the
per-64-slice arithmetic (the reference gates at rel <= 1e-5, :207); k_in % 64 != 0 refused.
glint_int8_gemm_i32 / _scaled_bf16: int32 results bit-exact vs an exact integer GEMM.
"""
import numpy as np
import pytest

from glint_amd import glint_hip as H
from oracle import glint_oracle as G
from tests.gpu_util import dev, host, bf16_bits, first_diff, torch_cuda

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("m,n,k", [(70, 192, 256), (37, 100, 1536), (1, 64, 64), (130, 257, 512), (70, 4096, 3072),
                                   (33, 200, 3136)])
def test_int8_mma_gemm_matches_emulation(oracle, m, n, k):
    rng = np.random.default_rng(m * 1000 + n)
    x = bf16_bits(rng.normal(0, 1, m * k).astype(np.float32))
    wq = rng.integers(-127, 128, n * k, dtype=np.int8)
    sw = rng.uniform(1e-3, 2e-2, n * (k // 64)).astype(np.float32)
    y, xq, sx = H.int8_mma_gemm(dev(x), dev(wq), dev(sw), n, k)
    oxq, osx = oracle.quant_act(x, m, k)
    gxq, gsx = host(xq), host(sx)
    assert gxq.tobytes() == oxq.tobytes(), first_diff(gxq, oxq)
    assert gsx.tobytes() == osx.tobytes()
    ref = oracle.int8_mma_emu(oxq, osx, wq, sw, m, n, k)
    got = host(y).reshape(m, n)
    assert got.tobytes() == ref.tobytes(), first_diff(got.view(np.uint32), ref.view(np.uint32))


def test_quant_act_special_values(oracle):
    vals = np.zeros(64 * 4, np.float32)
    vals[1], vals[2], vals[3] = 127.0, 2.5, -3.5                   # s = 1: ties to even
    vals[64:128] = np.linspace(-3, 3, 64)
    vals[130] = np.nan                                              # NaN skipped by the max
    vals[128:130] = [0.5, -0.25]
    vals[192:] = 1e-38
    x = bf16_bits(vals)
    n, k = 64, 256
    wq = np.ones(n * k, np.int8)
    sw = np.ones(n * (k // 64), np.float32)
    y, xq, sx = H.int8_mma_gemm(dev(x), dev(wq), dev(sw), n, k)
    oxq, osx = oracle.quant_act(x, 1, k)
    assert host(xq).tobytes() == oxq.tobytes() and host(sx).tobytes() == osx.tobytes()


def test_flat_entry_and_refusal():
    torch = torch_cuda()
    p7 = H.p7_lib()
    rng = np.random.default_rng(1)
    m, n, k = 8, 64, 128
    x = dev(bf16_bits(rng.normal(0, 1, m * k)))
    q = dev(rng.integers(-127, 128, n * k, dtype=np.int8))
    s = dev(rng.uniform(1e-3, 1e-2, n * 2).astype(np.float32))
    y1 = torch.empty(m * n, dtype=torch.float32, device="cuda")
    xq = torch.empty(m * k, dtype=torch.int8, device="cuda")
    sx = torch.empty(m * 2, dtype=torch.float32, device="cuda")
    rc = p7.p7_int8_gemm_flat(H._p(x), H._p(q), H._p(s), n, k, H._p(y1), m, H._p(xq), H._p(sx), H._stream())
    assert rc == 0
    y2, _, _ = H.int8_mma_gemm(x, q, s, n, k)
    assert torch.equal(y1.reshape(m, n), y2)
    rc = p7.p7_int8_gemm_flat(H._p(x), H._p(q), H._p(s), n, 96, H._p(y1), m, H._p(xq), H._p(sx), H._stream())
    assert rc == 1


@pytest.mark.parametrize("M,N,K", [(128, 128, 64), (200, 130, 192), (256, 512, 1024), (2048, 256, 8192),
                                   (257, 300, 640), (512, 1024, 2048), (300, 257, 64), (1000, 520, 128)])
def test_int8_gemm_exact(oracle, M, N, K):
    """The 128 x 128 tile kernel (every shape here has fewer 256 x 256 tiles than 3/4 of the
    CUs): ragged edges, one and odd numbers of K steps."""
    print(f"int8_gemm M={M} N={N} K={K}", flush=True)
    rng = np.random.default_rng(M + N + K)
    A = rng.integers(-127, 128, (M, K), dtype=np.int8)
    B = rng.integers(-127, 128, (N, K), dtype=np.int8)
    sa = rng.uniform(1e-3, 2e-2, M).astype(np.float32)
    sb = rng.uniform(1e-3, 2e-2, N).astype(np.float32)
    dA, dB = dev(A).reshape(M, K), dev(B).reshape(N, K)
    C = host(H.int8_gemm_i32(dA, dB))
    ref = oracle.int8_gemm_i32(A, B, M, N, K)
    assert np.array_equal(C, ref), first_diff(C, ref)
    out = host(H.int8_gemm_scaled_bf16(dA, dB, dev(sa), dev(sb)), np.uint16)
    assert np.array_equal(out, oracle.int8_scale_bf16(ref, sa, sb, M, N))


@pytest.mark.parametrize("M,N,K", [(4096, 3100, 640), (3000, 4100, 64), (4096, 3100, 128), (3100, 4096, 192),
                                   (4096, 3100, 448), (3100, 4096, 1216)])
def test_int8_gemm_dma_tiles_exact(oracle, M, N, K):
    """The 256 x 256 kernel whose operands go HBM -> LDS directly (a 5-slot ring of K steps,
    a barrier every two steps, the loop unrolled over 10) runs once there are at least 3/4
    as many 256 x 256 tiles as CUs: these shapes on a 256-CU part, with ragged M and N and
    10, 1, 2, 3, 7 and 19 K steps. Exact int32 against the oracle on the first and last
    256-row bands; every row and column through exact int64 row and column sums
    (sum_n C[m, n] = A[m] . sum_n B[n])."""
    print(f"int8_gemm dma M={M} N={N} K={K}", flush=True)
    rng = np.random.default_rng(M + 3 * N + K)
    A = rng.integers(-127, 128, (M, K), dtype=np.int8)
    B = rng.integers(-127, 128, (N, K), dtype=np.int8)
    sa = rng.uniform(1e-3, 2e-2, M).astype(np.float32)
    sb = rng.uniform(1e-3, 2e-2, N).astype(np.float32)
    dA, dB = dev(A).reshape(M, K), dev(B).reshape(N, K)
    C = host(H.int8_gemm_i32(dA, dB))
    out = host(H.int8_gemm_scaled_bf16(dA, dB, dev(sa), dev(sb)), np.uint16)
    for r0, r1 in ((0, 256), (M - 256, M)):
        ref = oracle.int8_gemm_i32(A[r0:r1], B, r1 - r0, N, K)
        assert np.array_equal(C[r0:r1], ref), (r0, first_diff(C[r0:r1], ref))
        assert np.array_equal(out[r0:r1], oracle.int8_scale_bf16(ref, sa[r0:r1], sb, r1 - r0, N)), r0
    A64, B64 = A.astype(np.int64), B.astype(np.int64)
    assert np.array_equal(C.astype(np.int64).sum(axis=1), A64 @ B64.sum(axis=0))
    assert np.array_equal(C.astype(np.int64).sum(axis=0), B64 @ A64.sum(axis=0))


@pytest.mark.parametrize("M,N", [(256, 256), (4096, 3328)])
def test_int8_gemm_extremes(oracle, M, N):
    """All -127 / all 127 at the largest K of the benchmark: |C| = K * 127^2 = 132 million,
    on the 128 x 128 kernel and on the 256 x 256 one (208 tiles)."""
    K = 8192
    A = np.full((M, K), -127, np.int8)
    B = np.full((N, K), 127, np.int8)
    B[1::2] = -127
    C = host(H.int8_gemm_i32(dev(A).reshape(M, K), dev(B).reshape(N, K)))
    assert (C[:, 0::2] == -K * 127 * 127).all() and (C[:, 1::2] == K * 127 * 127).all()


def _bands(m, h):
    return sorted({(0, min(h, m)), (max(m // 2 - h // 2, 0), min(m // 2 + h // 2, m)), (max(m - h, 0), m)})


@pytest.mark.parametrize("m,n,k", [(512, 24576, 640), (4096, 3100, 1088), (3000, 4100, 64), (2048, 6144, 960),
                                   (4096, 3100, 192)])
def test_int8_mma_gemm_dma_tiles_match_emulation(oracle, m, n, k):
    """int8_mma_gemm where it takes the 256 x 256 DMA-ring kernel (at least 3/4 as many
    256 x 256 tiles as CUs on a 256-CU part): ragged N; slice counts 10, 17, 1, 15 and 3
    (its loop runs four slices per pass, so every remainder mod 4 occurs). Activation
    bytes exact on the whole input; y bit-exact against the oracle's emulation on three
    64-row bands (first, middle, last)."""
    print(f"int8_mma_gemm dma m={m} n={n} k={k}", flush=True)
    rng = np.random.default_rng(m + n + k)
    x = bf16_bits(rng.normal(0, 1, m * k).astype(np.float32))
    wq = rng.integers(-127, 128, n * k, dtype=np.int8)
    sw = rng.uniform(1e-3, 2e-2, n * (k // 64)).astype(np.float32)
    y, xq, sx = H.int8_mma_gemm(dev(x), dev(wq), dev(sw), n, k)
    oxq, osx = oracle.quant_act(x, m, k)
    assert host(xq).tobytes() == oxq.tobytes() and host(sx).tobytes() == osx.tobytes()
    got = host(y).reshape(m, n)
    nkb = k // 64
    for r0, r1 in _bands(m, 64):
        ref = oracle.int8_mma_emu(oxq[r0 * k:r1 * k], osx[r0 * nkb:r1 * nkb], wq, sw, r1 - r0, n, k)
        assert got[r0:r1].tobytes() == ref.tobytes(), (r0, first_diff(got[r0:r1].view(np.uint32), ref.view(np.uint32)))


def test_int8_mma_gemm_plug_two_pass_on_dma_tiles(oracle):
    """The two-pass late plug where both passes take the DMA-ring kernel (the second one
    accumulating into y): bit-exact against base + plug on 64-row bands."""
    m, n, k = 512, 24576, 128
    print(f"int8_mma_gemm_plug dma m={m} n={n} k={k}", flush=True)
    rng = np.random.default_rng(99)
    x = bf16_bits(rng.normal(0, 1, m * k).astype(np.float32))
    wq = rng.integers(-127, 128, n * k, dtype=np.int8)
    sw = rng.uniform(1e-3, 2e-2, n * (k // 64)).astype(np.float32)
    q4 = rng.integers(0, 256, n * k // 2, dtype=np.uint8)
    sp = rng.uniform(1e-4, 2e-3, n * (k // 64)).astype(np.float32)
    got = host(H.int8_mma_gemm_plug(dev(x), dev(wq), dev(sw), dev(q4), dev(sp), n, k, fused=False)).reshape(m, n)
    xq, sx = oracle.quant_act(x, m, k)
    pq = oracle.unpack_res4(q4, n * k)
    nkb = k // 64
    for r0, r1 in _bands(m, 64):
        xs, ss = xq[r0 * k:r1 * k], sx[r0 * nkb:r1 * nkb]
        want = oracle.int8_mma_emu(xs, ss, wq, sw, r1 - r0, n, k) + oracle.int8_mma_emu(xs, ss, pq, sp, r1 - r0, n, k)
        assert got[r0:r1].tobytes() == want.tobytes(), (r0, first_diff(got[r0:r1].view(np.uint32), want.view(np.uint32)))


def test_int8_mma_gemm_config4_full_size(oracle):
    """BASELINE configs[4]'s shape on the attach ABI (bf16 x quantized per 64-block, per-64
    weight scales): 2048 x 8192 x 8192, bit-exact on two 32-row bands."""
    m, n, k = 2048, 8192, 8192
    print(f"int8_mma_gemm configs[4] m={m} n={n} k={k}", flush=True)
    torch = torch_cuda()
    g = torch.Generator(device="cuda").manual_seed(5004)
    xd = torch.randn(m, k, device="cuda", generator=g).to(torch.bfloat16)
    qd = torch.randint(-127, 128, (n * k,), device="cuda", generator=g, dtype=torch.int8)
    sd = torch.rand(n * k // 64, device="cuda", generator=g) * 0.02 + 1e-3
    y, xq, sx = H.int8_mma_gemm(xd, qd, sd, n, k)
    x = host(xd, np.uint16).reshape(-1)
    oxq, osx = oracle.quant_act(x, m, k)
    assert host(xq).tobytes() == oxq.tobytes() and host(sx).tobytes() == osx.tobytes()
    got, wq, sw = host(y).reshape(m, n), host(qd), host(sd)
    nkb = k // 64
    for r0, r1 in ((0, 32), (m - 32, m)):
        ref = oracle.int8_mma_emu(oxq[r0 * k:r1 * k], osx[r0 * nkb:r1 * nkb], wq, sw, r1 - r0, n, k)
        assert got[r0:r1].tobytes() == ref.tobytes(), (r0, first_diff(got[r0:r1].view(np.uint32), ref.view(np.uint32)))
