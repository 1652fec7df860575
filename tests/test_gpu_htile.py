"""GPU H-TILE parity.

f32 ABI (launch_glint_htile_s3_f32[_stream]): the reference's device tests restated —
  K-bounds test (test_htile_k_bounds_device.cu:44-118: shift 0/1 misaligned pointers,
  K in {1..256}, 5 shapes, bs=23, canaries, 3 repetitions, |err| <= 1e-5 (1 + |ref|) vs
  float64) and the 10-shape test (test_glint_htile.cu:63-153: max_diff < 1e-3 vs f32);
  plus the M=1 fast GEMV at the BASELINE shapes vs float64 within the f32 summation
  bound (K + 2) 2^-23 sum|terms| (test_streamer_real_weights.cu:130-133).
bf16 path (launch_glint_htile_bf16_stream): rel Frobenius <= 1e-2 vs an f32 GEMM on
  the expanded weights, and far tighter in practice.
"""
import ctypes

import numpy as np
import pytest

from glint_amd import glint_hip as H
from oracle import glint_oracle as G
from tests.gpu_util import dev, host, bf16_bits, torch_cuda

pytestmark = pytest.mark.gpu


def _kbounds_inputs(M, N, K, bs):
    i = np.arange(N * K, dtype=np.int64)
    h = ((i * 7 + i // 17 + 3) % 16).astype(np.uint8)
    p = ((i * 11 + i // 13 + 5) % 16).astype(np.uint8)
    hole = G.pack_nibbles(h)
    plug = G.pack_nibbles(p)
    nb = (N * K + bs - 1) // bs
    scales = (0.25 + (np.arange(nb) % 7) * 0.125).astype(np.float32)
    j = np.arange(M * K, dtype=np.int64)
    x = bf16_bits((((j * 3 + j // 19) % 17) - 8).astype(np.float32) * 0.0625)
    return hole, plug, scales, x


@pytest.mark.parametrize("K", [0, -5])
def test_k_nonpositive_writes_zeros(K):
    """K <= 0: no k term, so every output is the empty sum. As the reference's launcher
    (its k loop runs no iteration and stores the zero accumulators,
    cuda/glint_htile.cu:141-163), y is overwritten with zeros and the call returns 0, for
    f32 out, BF16 out and the no-allocation entry; M = 0 or N = 0 writes nothing."""
    torch = torch_cuda()
    lib = H.encode_lib()
    M, N = 3, 1000
    b = torch.zeros(64, dtype=torch.uint8, device="cuda")
    a = torch.ones(16, dtype=torch.float32, device="cuda")
    x = torch.zeros(64, dtype=torch.bfloat16, device="cuda")
    yf = torch.full((M, N), 7.0, dtype=torch.float32, device="cuda")
    yb = torch.full((M, N), 7.0, dtype=torch.bfloat16, device="cuda")
    yn = torch.full((M, N), 7.0, dtype=torch.bfloat16, device="cuda")
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    assert lib.launch_glint_htile_s3_f32_stream(P(b), P(b), P(a), P(x), P(yf), M, N, K, 64, None) == 0
    assert lib.launch_glint_htile_bf16_stream(P(b), P(b), P(a), P(x), P(yb), M, N, K, 64, None) == 0
    assert lib.launch_glint_htile_bf16_stream_noalloc(P(b), P(b), P(a), P(x), P(yn), M, N, K, 64, None) == 0
    torch.cuda.synchronize()
    assert (yf == 0).all() and (yb.view(torch.int16) == 0).all() and (yn.view(torch.int16) == 0).all()
    keep = torch.full((M, N), 7.0, dtype=torch.float32, device="cuda")
    assert lib.launch_glint_htile_s3_f32_stream(P(b), P(b), P(a), P(x), P(keep), 0, N, K, 64, None) == 0
    assert lib.launch_glint_htile_s3_f32_stream(P(b), P(b), P(a), P(x), P(keep), M, 0, K, 64, None) == 0
    assert lib.launch_glint_htile_s3_f32_stream(P(b), P(b), P(a), P(x), P(keep), M, N, K, 0, None) == -2
    torch.cuda.synchronize()
    assert (keep == 7.0).all()


@pytest.mark.parametrize("shift", [0, 1])
def test_reference_k_bounds_device_cases(oracle, shift):
    torch = torch_cuda()
    bs, guard, canary = 23, 16, 123456.0
    worst = 0.0
    for K in (1, 32, 40, 48, 63, 64, 65, 192, 199, 256):
        for M, N in ((1, 1), (15, 15), (16, 16), (17, 19), (33, 31)):
            hole, plug, scales, x = _kbounds_inputs(M, N, K, bs)
            dh, dp, dx = dev(hole, shift), dev(plug, shift), dev(x, shift)
            da = dev(scales)
            y = torch.full((M * N + 2 * guard,), canary, dtype=torch.float32, device="cuda")
            ref, _ = oracle.htile_f64(hole, plug, scales, x, M, N, K, bs)
            for _rep in range(3):
                rc = H.encode_lib().launch_glint_htile_s3_f32(
                    H._p(dh), H._p(dp), H._p(da), H._p(dx), H.VP(y.data_ptr() + 4 * guard), M, N, K, bs)
                assert rc == 0
                got = host(y)
                assert (got[:guard] == canary).all() and (got[guard + M * N:] == canary).all(), (M, N, K)
                out = got[guard:guard + M * N].reshape(M, N).astype(np.float64)
                err = np.abs(out - ref)
                assert np.isfinite(out).all()
                assert (err <= 1e-5 * (1 + np.abs(ref))).all(), (shift, M, N, K, float(err.max()))
                worst = max(worst, float(err.max()))
    assert worst < 1e-4


def test_reference_ten_shapes(oracle):
    cases = [(16, 16, 64, 64), (16, 16, 128, 64), (32, 32, 192, 64), (16, 16, 32, 64), (16, 16, 48, 64),
             (16, 16, 40, 64), (16, 16, 70, 64), (16, 16, 100, 64), (7, 23, 64, 64), (4, 3072, 3072, 64)]
    for M, N, K, bs in cases:
        nw, nx = N * K, M * K
        npk, nam = (nw + 1) // 2, (nw + bs - 1) // bs
        i = np.arange(npk, dtype=np.int64)
        hole = ((i * 7 + 1) % 256).astype(np.uint8)
        plug = ((i * 13 + 5) % 256).astype(np.uint8)
        am = (0.5 + (np.arange(nam) % 10) * 0.1).astype(np.float32)
        j = np.arange(nx, dtype=np.int64)
        x = bf16_bits((((j * 17 + 3) % 100) - 50).astype(np.float32) * 0.01)
        y = host(H.htile_f32(dev(hole), dev(plug), dev(am), dev(x), N, K, bs)).reshape(M, N)
        ref = oracle.htile_f32(hole, plug, am, x, M, N, K, bs)
        assert float(np.abs(y - ref).max()) < 1e-3, (M, N, K)


def _encoded_weight(oracle, N, K, seed, bs=64):
    torch = torch_cuda()
    g = torch.Generator(device="cuda").manual_seed(seed)
    w = (torch.randn(N * K, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    return H.encode_bf16(w, bs)


@pytest.mark.parametrize("N,K", [(14336, 4096), (4096, 14336), (100, 64), (3, 1088), (129, 2048), (1, 2048),
                                 (7, 6144), (1000, 12288), (17, 16384), (4097, 8192), (2000, 10240),
                                 (8, 18432), (100, 28672), (33, 32768),
                                 (13824, 5120), (5120, 13824), (5, 1024), (300, 3072), (77, 7168),
                                 (300, 20544), (64, 30784)])
def test_gemv_fast_path_vs_float64(oracle, N, K):
    torch = torch_cuda()
    hole, plug, am = _encoded_weight(oracle, N, K, 2002)
    g = torch.Generator(device="cuda").manual_seed(2001)
    x = torch.randn(K, device="cuda", generator=g).to(torch.bfloat16)
    y = host(H.htile_f32(hole, plug, am, x, N, K, 64)).reshape(-1).astype(np.float64)
    yb = host(H.htile_bf16(hole, plug, am, x, N, K, 64), np.uint16).reshape(-1)
    ref, asum = oracle.htile_f64(host(hole), host(plug), host(am), host(x, np.uint16), 1, N, K, 64)
    ref, asum = ref.reshape(-1), asum.reshape(-1)
    bound = (K + 2) * 2.0 ** -23 * asum
    assert (np.abs(y - ref) <= bound).all(), float((np.abs(y - ref) / bound).max())
    assert (np.abs(y - ref) <= 1e-5 * (1 + np.abs(ref))).all()
    yb64 = G.bf16_bits_to_f32(yb).astype(np.float64)
    assert (np.abs(yb64 - ref) <= np.abs(ref) * 2.0 ** -8 + bound * 1.01).all()


@pytest.mark.parametrize("N,K", [(300, 32832), (64, 34816)])
def test_m1_beyond_gemv_range(oracle, N, K):
    """M = 1 past the GEMV's K range (K above 32768) runs on the MFMA tiles: f32 out within
    the f32 sum bound and the reference's 1e-5 gate, BF16 out within 1e-2 relative
    Frobenius error of the float64 product."""
    torch = torch_cuda()
    hole, plug, am = _encoded_weight(oracle, N, K, 2302)
    g = torch.Generator(device="cuda").manual_seed(2301)
    x = torch.randn(K, device="cuda", generator=g).to(torch.bfloat16)
    y = host(H.htile_f32(hole, plug, am, x, N, K, 64)).reshape(-1).astype(np.float64)
    yb = G.bf16_bits_to_f32(host(H.htile_bf16(hole, plug, am, x, N, K, 64), np.uint16).reshape(-1)).astype(np.float64)
    ref, asum = oracle.htile_f64(host(hole), host(plug), host(am), host(x, np.uint16), 1, N, K, 64)
    ref, asum = ref.reshape(-1), asum.reshape(-1)
    assert (np.abs(y - ref) <= (K + 2) * 2.0 ** -23 * asum).all()
    assert (np.abs(y - ref) <= 1e-5 * (1 + np.abs(ref))).all()
    assert np.linalg.norm(yb - ref) <= 1e-2 * np.linalg.norm(ref)


@pytest.mark.parametrize("M", [1, 4, 64, 200])
def test_bf16_path_rel_frobenius(oracle, M):
    torch = torch_cuda()
    N, K = 1024, 4096
    hole, plug, am = _encoded_weight(oracle, N, K, 3002)
    g = torch.Generator(device="cuda").manual_seed(3001)
    x = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
    y = H.htile_bf16(hole, plug, am, x, N, K, 64).float()
    w = H.expand_f32(hole, plug, am, N * K, 64).reshape(N, K)
    ref = x.float() @ w.T
    rel = float(torch.linalg.norm(y - ref) / torch.linalg.norm(ref))
    assert rel <= 1e-2
    assert rel <= 4e-3  # BF16 rounding of the output alone is ~2^-9


@pytest.mark.parametrize("M,N,K", [(2, 14336, 4096), (3, 4096, 14336), (4, 129, 2048), (5, 1000, 12288),
                                   (8, 17, 16384), (6, 4097, 8192), (7, 7, 6144), (8, 3000, 6144),
                                   (2, 3000, 6144), (4, 300, 12288), (3, 1000, 5120), (4, 200, 13824),
                                   (2, 100, 18432), (4, 300, 28672), (3, 33, 30784), (2, 50, 1088)])
def test_small_m_gemv_vs_float64(oracle, M, N, K):
    """2 <= M <= 8 (batched decode) on the small-M GEMV: every weight looked up once for all
    M rows, its cell rounded to BF16 and multiplied into each row by v_dot2_f32_bf16, the
    block absmax applied once per row. Bound per output against float64 on the expanded
    weights: the BF16 output rounding (2^-8 |ref|), the BF16 rounding of each cell
    (2^-9 sum |w x|) and the f32 accumulation ((K + 2) 2^-23 sum |w x|). Also rel-Frobenius
    <= 4e-3 and no write past row M - 1."""
    torch = torch_cuda()
    print(f"small-M gemv M={M} N={N} K={K}", flush=True)
    hole, plug, am = _encoded_weight(oracle, N, K, 4002 + K)
    g = torch.Generator(device="cuda").manual_seed(4001 + M)
    x = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
    y = torch.full((M + 1, N), 1234.0, dtype=torch.bfloat16, device="cuda")
    rc = H.encode_lib().launch_glint_htile_bf16_stream(H._p(hole), H._p(plug), H._p(am), H._p(x), H._p(y), M, N, K,
                                                       64, H._stream())
    assert rc == 0
    yh = host(y, np.uint16)
    assert (yh[M] == np.uint16(0x449A)).all()  # 1234.0 in BF16: row M untouched
    got = G.bf16_bits_to_f32(yh[:M].reshape(-1)).astype(np.float64).reshape(M, N)
    ref, asum = oracle.htile_f64(host(hole), host(plug), host(am), host(x, np.uint16), M, N, K, 64)
    ref, asum = ref.reshape(M, N), asum.reshape(M, N)
    bound = np.abs(ref) * 2.0 ** -8 + asum * (2.0 ** -9 + (K + 2) * 2.0 ** -23) * 1.01
    assert (np.abs(got - ref) <= bound).all(), float((np.abs(got - ref) / bound).max())
    rel = float(np.linalg.norm(got - ref) / np.linalg.norm(ref))
    assert rel <= 4e-3, rel


# 9 <= M <= 64 with K % 128 == 0: the register-dequantized tiles (one, two or four MFMA row
# blocks; a workgroup of about N / CUs rows, the last strip partly filled; K split 4 ways
# where N is small). Odd W-chunk counts leave the last x chunk half used (K = 640, 896,
# 14464); N = 13 and 56 give workgroups of fewer rows than one strip; N = 14336 at M = 9 is
# the gate shape with 56-row workgroups, 4096 x 14336 the down shape split 4 ways.
RD_SHAPES = [(9, 14336, 4096), (16, 777, 896), (17, 56, 2048), (32, 4097, 1152), (33, 300, 14464),
             (48, 2000, 640), (64, 13, 512), (64, 1000, 2304), (64, 4096, 14336), (40, 130, 128)]


@pytest.mark.parametrize("M,N,K", RD_SHAPES)
def test_bf16_small_m_tiles_vs_float64(oracle, M, N, K):
    """9 <= M <= 64 on the register-dequantized MFMA tiles, each output bounded against
    float64 on the expanded weights: the BF16 output rounding (2^-8 |ref|), the BF16 rounding
    of each weight (2^-9 sum |w x|) and f32 accumulation in any order ((K + 2) 2^-23
    sum |w x|). Also rel-Frobenius <= 4e-3, no write past row M - 1, and a repeat equal bit
    for bit (the K split adds its partials in a fixed order)."""
    torch = torch_cuda()
    print(f"small-M tiles M={M} N={N} K={K}", flush=True)
    hole, plug, am = _encoded_weight(oracle, N, K, 5002 + K)
    g = torch.Generator(device="cuda").manual_seed(5001 + M)
    x = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
    y = torch.full((M + 1, N), 1234.0, dtype=torch.bfloat16, device="cuda")
    lib = H.encode_lib()
    assert lib.launch_glint_htile_bf16_stream(H._p(hole), H._p(plug), H._p(am), H._p(x), H._p(y), M, N, K, 64,
                                              H._stream()) == 0
    yh = host(y, np.uint16)
    assert (yh[M] == np.uint16(0x449A)).all()  # 1234.0 in BF16: row M untouched
    got = G.bf16_bits_to_f32(yh[:M].reshape(-1)).astype(np.float64).reshape(M, N)
    ref, asum = oracle.htile_f64(host(hole), host(plug), host(am), host(x, np.uint16), M, N, K, 64)
    ref, asum = ref.reshape(M, N), asum.reshape(M, N)
    bound = np.abs(ref) * 2.0 ** -8 + asum * (2.0 ** -9 + (K + 2) * 2.0 ** -23) * 1.01
    assert (np.abs(got - ref) <= bound).all(), float((np.abs(got - ref) / bound).max())
    rel = float(np.linalg.norm(got - ref) / np.linalg.norm(ref))
    assert rel <= 4e-3, rel
    again = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    assert lib.launch_glint_htile_bf16_stream(H._p(hole), H._p(plug), H._p(am), H._p(x), H._p(again), M, N, K, 64,
                                              H._stream()) == 0
    assert torch.equal(again.view(torch.int16), y[:M].view(torch.int16))


@pytest.mark.parametrize("f32", [False, True])
@pytest.mark.parametrize("M,N,K", [(16, 300, 1152), (64, 64, 14464)])
def test_small_m_tiles_nonfinite_x_stays_in_its_row(oracle, M, N, K, f32):
    """An infinite x value reaches its own output row only. K % 256 == 128 leaves the last
    W line of a row half used, so the second half of the last x chunk lies past the row's end
    (the next row's first 128 values), or past the split's chunks where K is split (N = 64 at
    K = 14464: 4 splits); those halves are not loaded, so no zero weight meets them. x row 1
    holds +inf at k = 5, row 2 -inf at k = K - 3: rows 1 and 2 come out non-finite, every
    other row finite and within the bound against float64 (BF16 out and the f32 ABI)."""
    torch = torch_cuda()
    print(f"small-M non-finite x M={M} N={N} K={K} f32={f32}", flush=True)
    hole, plug, am = _encoded_weight(oracle, N, K, 5100 + K)
    rng = np.random.default_rng(5101 + M)
    xb = bf16_bits(rng.normal(0, 1, M * K).astype(np.float32)).reshape(M, K)
    xb[1, 5] = 0x7F80   # +inf
    xb[2, K - 3] = 0xFF80  # -inf
    x = dev(xb.reshape(-1))
    if f32:
        got = host(H.htile_f32(hole, plug, am, x.reshape(M, K), N, K, 64)).reshape(M, N).astype(np.float64)
    else:
        got = G.bf16_bits_to_f32(host(H.htile_bf16(hole, plug, am, x.reshape(M, K), N, K, 64), np.uint16).reshape(-1))
        got = got.astype(np.float64).reshape(M, N)
    assert not np.isfinite(got[1:3]).any()
    rows = np.array([r for r in range(M) if r not in (1, 2)])
    ref, asum = oracle.htile_f64(host(hole), host(plug), host(am), xb[rows].reshape(-1), rows.size, N, K, 64)
    ref, asum = ref.reshape(rows.size, N), asum.reshape(rows.size, N)
    g = got[rows]
    assert np.isfinite(g).all()
    if f32:
        bound = (K + 2) * 2.0 ** -23 * asum
    else:
        bound = np.abs(ref) * 2.0 ** -8 + asum * (2.0 ** -9 + (K + 2) * 2.0 ** -23) * 1.01
    assert (np.abs(g - ref) <= bound).all(), float((np.abs(g - ref) / bound).max())


@pytest.mark.parametrize("M,N,K", [(256, 1024, 4096), (300, 1000, 576), (513, 1100, 1024), (2048, 384, 640),
                                   (2000, 6100, 1088), (4096, 4096, 576)])
def test_bf16_prefill_tiles_rel_frobenius(oracle, M, N, K):
    """The large-M prefill tiles (256 x 128, and 256 x 256 with x loaded straight into LDS
    once there are at least 3/4 as many 256 x 256 tiles as CUs: the last two shapes on a
    256-CU part): ragged M and N, an odd number of K steps; bf16 out within 4e-3 relative
    Frobenius of fp32 on the expanded weights (the contract asks 1e-2)."""
    torch = torch_cuda()
    print(f"prefill M={M} N={N} K={K}", flush=True)
    hole, plug, am = _encoded_weight(oracle, N, K, 3003)
    g = torch.Generator(device="cuda").manual_seed(3004)
    x = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
    y = H.htile_bf16(hole, plug, am, x, N, K, 64).float()
    w = H.expand_f32(hole, plug, am, N * K, 64).reshape(N, K)
    ref = x.float() @ w.T
    rel = float(torch.linalg.norm(y - ref) / torch.linalg.norm(ref))
    assert rel <= 4e-3, rel
    # every row and column was written (no stale tile): max error per row bounded too
    row_rel = torch.linalg.norm(y - ref, dim=1) / torch.linalg.norm(ref, dim=1)
    assert float(row_rel.max()) <= 1e-2


SPLIT_SHAPES = [(64, 64, 2368), (40, 200, 1088), (64, 14336, 4096), (64, 4096, 14336), (200, 512, 8192),
                (512, 4096, 14336), (17, 1000, 2304), (33, 136, 768), (2, 14336, 4096),
                (1024, 4096, 14336), (1000, 4000, 14336)]


@pytest.mark.parametrize("M,N,K", SPLIT_SHAPES)
def test_bf16_split_k(oracle, M, N, K):
    """Shapes whose output tiles alone would leave most of the device idle split K over
    several workgroups per tile (K = 64 * 37 gives a ragged last split; K = 2304 and 768
    give odd counts of 4-step super-steps with ragged M and N; M = 1024 and 1000 the
    256 x 256 tiles split 4 ways, the latter with ragged tiles; M = 2 on the gate shape runs
    the small-M GEMV);
    the last workgroup of a tile adds the partial tiles in split order. Checked: relative Frobenius error
    against fp32 on the expanded weights (a lost or doubled partial fails it), every row
    bounded, bitwise-equal repeats, and bitwise-equal results from two streams running at
    once (each stream has its own partials and counters)."""
    torch = torch_cuda()
    print(f"split-K M={M} N={N} K={K}", flush=True)
    hole, plug, am = _encoded_weight(oracle, N, K, 3005 + K)
    g = torch.Generator(device="cuda").manual_seed(3006 + M)
    x = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
    y = H.htile_bf16(hole, plug, am, x, N, K, 64)
    w = H.expand_f32(hole, plug, am, N * K, 64).reshape(N, K)
    ref = x.float() @ w.T
    yf = y.float()
    rel = float(torch.linalg.norm(yf - ref) / torch.linalg.norm(ref))
    assert rel <= 4e-3, rel
    row_rel = torch.linalg.norm(yf - ref, dim=1) / torch.linalg.norm(ref, dim=1)
    assert float(row_rel.max()) <= 1e-2
    del w, ref
    again = H.htile_bf16(hole, plug, am, x, N, K, 64)
    assert torch.equal(again.view(torch.int16), y.view(torch.int16))
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    s1.wait_stream(torch.cuda.current_stream())
    s2.wait_stream(torch.cuda.current_stream())
    outs = []
    for s in (s1, s2, s1, s2):
        with torch.cuda.stream(s):
            outs.append(H.htile_bf16(hole, plug, am, x, N, K, 64, stream=s))
    torch.cuda.synchronize()
    for o in outs:
        assert torch.equal(o.view(torch.int16), y.view(torch.int16))


def test_bf16_split_k_workspace_growth(oracle):
    """A small split launch, then a larger one (the stream's workspace grows), then the small
    one again: the repeat equals the first result bit for bit (counters were left at zero)."""
    torch = torch_cuda()
    res = []
    for (M, N, K) in [(64, 64, 2368), (64, 4096, 14336), (64, 64, 2368)]:
        print(f"split-K growth M={M} N={N} K={K}", flush=True)
        hole, plug, am = _encoded_weight(oracle, N, K, 3100 + N)
        g = torch.Generator(device="cuda").manual_seed(3101)
        x = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
        res.append(H.htile_bf16(hole, plug, am, x, N, K, 64))
    torch.cuda.synchronize()
    assert torch.equal(res[0].view(torch.int16), res[2].view(torch.int16))


# Shapes whose whole-tile plans fill 256 CUs poorly, so they run Stream-K on a 256-CU part:
# 336 and 330 256 x 256 tiles (two rounds, the second about 1/3 full; 21 and 12.9 K steps per
# workgroup, so ranges hold up to 3 segments), and two shapes whose 256 x 128 tiles fill 75%
# and 66% (84 and 42 K steps per workgroup over 96 and 168 256 x 256 tiles: up to 4 and 3
# workgroups share a tile); ragged M and N in the second and third.
SK_SHAPES = [(1536, 14336, 1024), (1300, 14000, 640), (1500, 4000, 14336), (768, 14336, 4096)]


@pytest.mark.parametrize("M,N,K", SK_SHAPES)
def test_bf16_stream_k(oracle, M, N, K):
    """Where whole 256 x 256 tiles would leave CUs idle, the tiles run Stream-K: one
    workgroup per CU over equal ranges of (tile, K step) units, each range cut into
    segments at tile edges; a tile shared by several workgroups is added up by the last to
    arrive, in workgroup order. Checked: relative Frobenius error against fp32 on the
    expanded weights (a lost or doubled segment fails it), every row bounded, bitwise-equal
    repeats and two streams at once (each with its own workspace), and agreement with the
    whole-tile kernel (the no-allocation entry: its fixed workspace is too small for the
    Stream-K plan, so it runs one tile per workgroup) within the same tolerance."""
    torch = torch_cuda()
    print(f"stream-K M={M} N={N} K={K}", flush=True)
    hole, plug, am = _encoded_weight(oracle, N, K, 3205 + K)
    g = torch.Generator(device="cuda").manual_seed(3206 + M)
    x = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
    y = H.htile_bf16(hole, plug, am, x, N, K, 64)
    w = H.expand_f32(hole, plug, am, N * K, 64).reshape(N, K)
    ref = x.float() @ w.T
    del w
    yf = y.float()
    rel = float(torch.linalg.norm(yf - ref) / torch.linalg.norm(ref))
    assert rel <= 4e-3, rel
    row_rel = torch.linalg.norm(yf - ref, dim=1) / torch.linalg.norm(ref, dim=1)
    assert float(row_rel.max()) <= 1e-2
    whole = torch.empty_like(y)
    rc = H.encode_lib().launch_glint_htile_bf16_stream_noalloc(H._p(hole), H._p(plug), H._p(am), H._p(x),
                                                               H._p(whole), M, N, K, 64, H._stream())
    assert rc == 0
    wrel = float(torch.linalg.norm(whole.float() - ref) / torch.linalg.norm(ref))
    assert wrel <= 4e-3, wrel
    assert float(torch.linalg.norm(yf - whole.float()) / torch.linalg.norm(ref)) <= 4e-3
    del ref
    again = H.htile_bf16(hole, plug, am, x, N, K, 64)
    assert torch.equal(again.view(torch.int16), y.view(torch.int16))
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    s1.wait_stream(torch.cuda.current_stream())
    s2.wait_stream(torch.cuda.current_stream())
    outs = []
    for s in (s1, s2, s1, s2):
        with torch.cuda.stream(s):
            outs.append(H.htile_bf16(hole, plug, am, x, N, K, 64, stream=s))
    torch.cuda.synchronize()
    for o in outs:
        assert torch.equal(o.view(torch.int16), y.view(torch.int16))


F32_SHAPES = [(2, 64, 64), (3, 300, 1088), (64, 1024, 4096), (127, 520, 2368), (128, 4096, 576), (300, 1100, 1024),
              (513, 2048, 4096), (64, 4096, 14336), (100, 14336, 4096), (24, 1000, 2304), (32, 300, 1152),
              (48, 777, 640)]


@pytest.mark.parametrize("M,N,K", F32_SHAPES)
def test_f32_prefill_mfma_vs_float64(oracle, M, N, K):
    """The f32-out ABI at M > 1, bs 64 (launch_glint_htile_s3_f32_stream on BF16 MFMA with the
    weights in three exact BF16 planes): against float64, every output within the f32
    summation bound (K + 2) 2^-23 sum|t| and within the reference's 1e-5 (1 + |ref|);
    ragged M and N: M <= 64 with K % 128 == 0 on the register-dequantized kernel (one, two or
    four MFMA row blocks; K split 4 ways on the 4096 x 14336 down shape; half-used last W
    lines at K = 1152 and 640), 64 x 128 tiles below M = 128 otherwise, 128 x 128 above;
    split K, odd K steps."""
    torch = torch_cuda()
    print(f"f32 prefill M={M} N={N} K={K}", flush=True)
    hole, plug, am = _encoded_weight(oracle, N, K, 3200 + M)
    g = torch.Generator(device="cuda").manual_seed(3201 + N)
    x = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
    y = host(H.htile_f32(hole, plug, am, x, N, K, 64)).reshape(M, N).astype(np.float64)
    rows = np.unique(np.linspace(0, M - 1, min(M, 24)).astype(np.int64))
    xs = host(x, np.uint16).reshape(M, K)[rows]
    ref, asum = oracle.htile_f64(host(hole), host(plug), host(am), xs, rows.size, N, K, 64)
    err = np.abs(y[rows] - ref)
    assert (err <= (K + 2) * 2.0 ** -23 * asum).all(), float((err / ((K + 2) * 2.0 ** -23 * asum)).max())
    assert (err <= 1e-5 * (1 + np.abs(ref))).all(), float(err.max())
    again = H.htile_f32(hole, plug, am, x, N, K, 64)
    assert np.array_equal(host(again).reshape(M, N), y.astype(np.float32))


def test_f32_prefill_mfma_full_size_gate(oracle):
    """BASELINE configs[2] shape on the f32 ABI: M = 2048 x 14336 x 4096; 16 rows against
    float64 within both bounds, all rows finite."""
    torch = torch_cuda()
    M, N, K = 2048, 14336, 4096
    print(f"f32 prefill full M={M} N={N} K={K}", flush=True)
    hole, plug, am = _encoded_weight(oracle, N, K, 3002)
    g = torch.Generator(device="cuda").manual_seed(3001)
    x = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
    yd = H.htile_f32(hole, plug, am, x, N, K, 64)
    assert bool(torch.isfinite(yd).all())
    rows = np.linspace(0, M - 1, 16).astype(np.int64)
    y = host(yd).reshape(M, N)[rows].astype(np.float64)
    ref, asum = oracle.htile_f64(host(hole), host(plug), host(am), host(x, np.uint16).reshape(M, K)[rows], 16, N, K, 64)
    err = np.abs(y - ref)
    assert (err <= (K + 2) * 2.0 ** -23 * asum).all()
    assert (err <= 1e-5 * (1 + np.abs(ref))).all()


def test_f32_prefill_mfma_special_absmax(oracle):
    """Blocks with an infinite or NaN absmax, and one whose CELLS * absmax overflows f32:
    the MFMA path gives NaN and +-inf exactly where the f32 restatement does, and the
    finite outputs agree within the bounds."""
    torch = torch_cuda()
    M, N, K = 8, 64, 256
    rng = np.random.default_rng(77)
    i = np.arange(N * K // 2)
    hole = ((i * 7 + 1) % 256).astype(np.uint8)
    plug = ((i * 13 + 5) % 256).astype(np.uint8)
    am = rng.uniform(0.5, 1.5, N * K // 64).astype(np.float32)
    am[4 * 3 + 1] = np.inf          # row 3, block 1
    am[4 * 10 + 0] = np.nan         # row 10, block 0
    am[4 * 20 + 2] = np.finfo(np.float32).max  # row 20: CELLS * absmax overflows where |cells| > 1
    am[4 * 30 + 3] = np.float32(2.0 ** 126)
    # small x keeps every product of a finite weight finite, so overflow cannot depend on order
    x = bf16_bits(rng.normal(0, 1e-3, M * K).astype(np.float32))
    x[5] = 0  # a zero x against the infinite block
    y = host(H.htile_f32(dev(hole), dev(plug), dev(am), dev(x), N, K, 64)).reshape(M, N)
    ref32 = oracle.htile_f32(hole, plug, am, x, M, N, K, 64)
    assert np.array_equal(np.isnan(y), np.isnan(ref32))
    assert np.array_equal(np.isinf(y), np.isinf(ref32)) and np.array_equal(y[np.isinf(y)], ref32[np.isinf(ref32)])
    fin = np.isfinite(ref32)
    ref, asum = oracle.htile_f64(hole, plug, am, x, M, N, K, 64)
    err = np.abs(y[fin].astype(np.float64) - ref[fin])
    assert (err <= (K + 2) * 2.0 ** -23 * asum[fin] + 1e-30).all()


@pytest.mark.parametrize("M,N,K", [(2, 14336, 4096), (3, 4096, 14336), (4, 1000, 2048), (4, 17, 16384),
                                   (2, 4097, 8192), (2, 300, 5120), (4, 100, 13824), (3, 64, 3072),
                                   (5, 1000, 4096), (6, 129, 5120), (7, 64, 2048), (8, 300, 14336)])
def test_small_m_f32_gemv_vs_float64(oracle, M, N, K):
    """The f32-out ABI on the small-M GEMV: 2 <= M <= 4 in one launch, 5 <= M <= 8 as the
    4-row launch and a second one for the rest (the M = 1 GEMV for one row; M = 5 here),
    any K % 64 == 0 (a partial last slice at K = 5120, 13824, 3072). Exact f32 cells, one
    FMA per weight and row. Every output within the f32 summation bound (K + 2) 2^-23
    sum|t| and the reference's 1e-5 (1 + |ref|); repeats bit-equal."""
    torch = torch_cuda()
    print(f"small-M f32 gemv M={M} N={N} K={K}", flush=True)
    hole, plug, am = _encoded_weight(oracle, N, K, 4100 + K)
    g = torch.Generator(device="cuda").manual_seed(4101 + M)
    x = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
    y = host(H.htile_f32(hole, plug, am, x, N, K, 64)).reshape(M, N).astype(np.float64)
    ref, asum = oracle.htile_f64(host(hole), host(plug), host(am), host(x, np.uint16), M, N, K, 64)
    err = np.abs(y - ref)
    assert (err <= (K + 2) * 2.0 ** -23 * asum).all(), float((err / ((K + 2) * 2.0 ** -23 * asum)).max())
    assert (err <= 1e-5 * (1 + np.abs(ref))).all(), float(err.max())
    again = H.htile_f32(hole, plug, am, x, N, K, 64)
    assert np.array_equal(host(again).reshape(M, N), y.astype(np.float32))


@pytest.mark.parametrize("M,K", [(1, 2048), (1, 4096), (1, 1088), (1, 3072), (1, 14336), (1, 28672), (2, 2048), (4, 4096),
                                 (5, 2048), (8, 4096)])
def test_f32_gemv_special_absmax(oracle, M, K):
    """The f32-out GEMVs (M = 1: in 512-thread workgroups up to K = 4096 and wider ones
    above, with a partial last K slice at K = 1088 and 3072; and the small-M form) on
    blocks with an infinite or NaN absmax,
    one whose CELLS * absmax overflows f32 and one at 2^126: such a block takes the
    reference's per-weight products (cell * absmax, then the FMA with x), so NaN and +-inf
    land exactly where the f32 restatement puts them; the finite outputs agree within the
    bound."""
    torch = torch_cuda()
    N = 64
    nb = K // 64
    rng = np.random.default_rng(78 + K + M)
    i = np.arange(N * K // 2)
    hole = ((i * 7 + 1) % 256).astype(np.uint8)
    plug = ((i * 13 + 5) % 256).astype(np.uint8)
    am = rng.uniform(0.5, 1.5, N * nb).astype(np.float32)
    am[nb * 3 + 1] = np.inf          # row 3, block 1
    am[nb * 10 + 0] = np.nan         # row 10, block 0
    am[nb * 20 + 2] = np.finfo(np.float32).max  # row 20: CELLS * absmax overflows where |cells| > 1
    am[nb * 30 + 3] = np.float32(2.0 ** 126)
    am[nb * 40 + 5] = -np.inf        # row 40: a negative infinite absmax
    x = bf16_bits(rng.normal(0, 1e-3, M * K).astype(np.float32))
    x[64 + 5] = 0  # a zero x against row 3's infinite block (element 69 of x row 0)
    y = host(H.htile_f32(dev(hole), dev(plug), dev(am), dev(x).reshape(M, K), N, K, 64)).reshape(M, N)
    ref32 = oracle.htile_f32(hole, plug, am, x, M, N, K, 64).reshape(M, N)
    assert np.isnan(ref32).any()  # mixed-sign infinite products; the factored form would give +-inf
    assert np.array_equal(np.isnan(y), np.isnan(ref32))
    assert np.array_equal(np.isinf(y), np.isinf(ref32)) and np.array_equal(y[np.isinf(y)], ref32[np.isinf(ref32)])
    fin = np.isfinite(ref32)
    ref, asum = oracle.htile_f64(hole, plug, am, x, M, N, K, 64)
    err = np.abs(y[fin].astype(np.float64) - ref.reshape(M, N)[fin])
    assert (err <= (K + 2) * 2.0 ** -23 * asum.reshape(M, N)[fin] + 1e-30).all()


def test_split_workspace_under_graph_capture(oracle):
    """A split-K launch captured into a graph keeps the workspace it bound: after the
    capture, eager calls on the capture stream get a fresh workspace (they never share
    counters with the graph), and every replay, with eager split launches and
    synchronisations between them, equals the eager result bit for bit."""
    torch = torch_cuda()
    M, N, K = 64, 4096, 14336
    print(f"graph capture split-K M={M} N={N} K={K}", flush=True)
    hole, plug, am = _encoded_weight(oracle, N, K, 3301)
    g = torch.Generator(device="cuda").manual_seed(3302)
    x = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
    x2 = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        want = H.htile_bf16(hole, plug, am, x, N, K, 64, stream=s)  # reserves the stream's workspace
        want2 = H.htile_bf16(hole, plug, am, x2, N, K, 64, stream=s)
    s.synchronize()
    out = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        H.htile_bf16(hole, plug, am, x, N, K, 64, out=out, stream=s)
    torch.cuda.synchronize()
    for rep in range(4):
        out.zero_()
        graph.replay()
        with torch.cuda.stream(s):
            e = H.htile_bf16(hole, plug, am, x2, N, K, 64, stream=s)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), want.view(torch.int16)), rep
        assert torch.equal(e.view(torch.int16), want2.view(torch.int16)), rep


def test_workspace_reserve_entry():
    torch = torch_cuda()
    s = torch.cuda.Stream()
    assert H.encode_lib().glint_htile_workspace_reserve(H._stream(s)) == 0
    assert H.encode_lib().glint_htile_workspace_reserve(H._stream(s)) == 0


def test_split_workspace_capture_cycles_bounded(oracle):
    """Capture -> eager cycles on one stream allocate nothing after the first: every capture
    binds the stream's one graph workspace and every eager call its one eager workspace, so
    device memory stays flat over five more cycles; each graph's replays, interleaved with
    eager split launches on the same stream, equal the eager result bit for bit. Then
    glint_htile_workspace_release frees both workspaces and a later call allocates afresh
    with the same result."""
    torch = torch_cuda()
    M, N, K = 64, 4096, 14336
    hole, plug, am = _encoded_weight(oracle, N, K, 3401)
    g = torch.Generator(device="cuda").manual_seed(3402)
    x = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    sh = H._stream(s)
    lib = H.encode_lib()
    with torch.cuda.stream(s):
        want = H.htile_bf16(hole, plug, am, x, N, K, 64, stream=s)
    outs = [torch.empty(M, N, dtype=torch.bfloat16, device="cuda") for _ in range(6)]
    eager = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    graphs = []
    torch.cuda.synchronize()
    free0 = None
    for c in range(6):
        print(f"capture/eager cycle {c}", flush=True)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            H.htile_bf16(hole, plug, am, x, N, K, 64, out=outs[c], stream=s)
        graphs.append(graph)
        with torch.cuda.stream(s):
            H.htile_bf16(hole, plug, am, x, N, K, 64, out=eager, stream=s)
        torch.cuda.synchronize()
        assert torch.equal(eager.view(torch.int16), want.view(torch.int16)), c
        if c == 0:
            free0 = torch.cuda.mem_get_info()[0]
    free5 = torch.cuda.mem_get_info()[0]
    assert free0 - free5 < 16 << 20, (free0 - free5) / 2 ** 20  # without the bound: 5 x 64 MiB
    for rep in range(2):
        for c, graph in enumerate(graphs):
            with torch.cuda.stream(s):
                outs[c].zero_()
                graph.replay()
                H.htile_bf16(hole, plug, am, x, N, K, 64, out=eager, stream=s)
            torch.cuda.synchronize()
            assert torch.equal(outs[c].view(torch.int16), want.view(torch.int16)), (rep, c)
            assert torch.equal(eager.view(torch.int16), want.view(torch.int16)), (rep, c)
    del graphs
    torch.cuda.synchronize()
    before = torch.cuda.mem_get_info()[0]
    assert lib.glint_htile_workspace_release(sh) == 0
    after = torch.cuda.mem_get_info()[0]
    assert after - before >= 100 << 20, (after - before) / 2 ** 20  # the eager and the graph workspace
    assert lib.glint_htile_workspace_release(sh) == 0  # nothing left: a no-op
    with torch.cuda.stream(s):
        again = H.htile_bf16(hole, plug, am, x, N, K, 64, stream=s)
    torch.cuda.synchronize()
    assert torch.equal(again.view(torch.int16), want.view(torch.int16))
    assert lib.glint_htile_workspace_release(sh) == 0
