"""GPU parity for the W8A16 tile GEMM over an INT8 pin linear (int8_tile_gemm_bf16).

The checks restate the reference's own test (tests/test_int8_tile_gemm.cu):
- its synthetic shape grid, m x n x k over {1..130} x {1..129} x {1..1040}, including
  k_in that are not multiples of 64, so a weight row's scale blocks start mid-row;
- x and q at odd offsets;
- the pending-error rule;
- the bound |y - dot| <= 1e-4 * sum |terms| against a double sum of BF16(x) * BF16(q s)
  (:13, :89-113).

Two bit-exact checks of the dequantization are added: one-hot activations make
y = W^T exactly, on both the MFMA path and the generic path. Large-M shapes cover the
256 x 128 and 256 x 256 tiles.
"""
import ctypes

import numpy as np
import pytest

from glint_amd import glint_hip as H
from tests.gpu_util import dev, host, bf16_bits, first_diff, torch_cuda

pytestmark = pytest.mark.gpu
TOL = 1e-4  # test_int8_tile_gemm.cu:13


def _case(rng, m, n, k):
    """q uniform in [-127, 127], scales in [1e-3, 2.1e-2), x uniform in [-2, 2) as BF16
    (test_int8_tile_gemm.cu:57-61, 122-133), drawn from numpy for speed."""
    q = rng.integers(-127, 128, n * k, dtype=np.int8)
    s = (1e-3 + 2e-2 * rng.random((n * k + 63) // 64)).astype(np.float32)
    x = bf16_bits((4.0 * rng.random(m * k) - 2.0).astype(np.float32))
    return x, q, s


def _check(oracle, got, x, q, s, m, n, k, label):
    want, absdot = oracle.int8_tile_f64(x, q, s, m, n, k)
    got = np.asarray(got, np.float64).reshape(m, n)
    ratio = np.abs(got - want) / np.where(absdot > 0, absdot, 1e-30)
    assert np.all(ratio <= TOL), f"{label} m={m} n={n} k={k}: max err/absdot {ratio.max():.3e}"


MS = [1, 2, 3, 7, 16, 17, 63, 64, 65, 130]
NS = [1, 8, 63, 64, 65, 100, 129]
KS = [1, 16, 37, 63, 64, 80, 129, 200, 208, 1000, 1024, 1040]


@pytest.mark.parametrize("m", MS)
def test_synthetic_grid(oracle, m):
    """test_int8_tile_gemm.cu:292-299, every (n, k) for this m."""
    torch_cuda()
    rng = np.random.default_rng(9000 + m)
    for n in NS:
        for k in KS:
            print(f"int8_tile m={m} n={n} k={k}", flush=True)
            x, q, s = _case(rng, m, n, k)
            y = H.int8_tile_gemm(dev(x), dev(q), dev(s), n, k, m=m)
            _check(oracle, host(y), x, q, s, m, n, k, "synthetic")


@pytest.mark.parametrize("x_off,q_off", [(1, 0), (0, 1), (1, 1)])
@pytest.mark.parametrize("m,n,k", [(17, 65, 208), (130, 129, 1040)])
def test_unaligned_pointers(oracle, x_off, q_off, m, n, k):
    """test_int8_tile_gemm.cu:301-307: x and q views at odd element offsets."""
    print(f"int8_tile unaligned x+{x_off} q+{q_off} m={m} n={n} k={k}", flush=True)
    rng = np.random.default_rng(x_off * 10 + q_off + m)
    x, q, s = _case(rng, m, n, k)
    y = H.int8_tile_gemm(dev(x, pad_front=x_off), dev(q, pad_front=q_off), dev(s), n, k, m=m)
    _check(oracle, host(y), x, q, s, m, n, k, "unaligned")


@pytest.mark.parametrize("m,n,k", [(256, 129, 1024), (300, 1000, 576), (513, 64, 64), (2048, 384, 640),
                                   (1024, 4096, 4096), (64, 14336, 4096), (64, 4096, 14336), (100, 200, 8192),
                                   (2000, 6400, 576), (4096, 4096, 640)])
def test_large_m_tiles(oracle, m, n, k):
    """The last two shapes have at least 3/4 as many 256 x 256 tiles as a 256-CU part has
    CUs, so they run the 256 x 256 tile with x loaded straight into LDS."""
    print(f"int8_tile large m={m} n={n} k={k}", flush=True)
    rng = np.random.default_rng(m + n + k)
    x, q, s = _case(rng, m, n, k)
    y = host(H.int8_tile_gemm(dev(x), dev(q), dev(s), n, k, m=m))
    if m * n * k <= 1 << 30:
        _check(oracle, y, x, q, s, m, n, k, "large")
    else:  # a row sample of the output against the double sum
        rows = np.unique(np.concatenate([[0, m - 1], rng.integers(0, m, 24)]))
        xs = x.reshape(m, k)[rows].reshape(-1)
        _check(oracle, y[rows], xs, q, s, rows.size, n, k, "large (row sample)")


@pytest.mark.parametrize("m,n,k", [(1, 14336, 4096), (1, 4096, 14336), (2, 1000, 2048), (3, 129, 16384),
                                   (4, 520, 6144), (1, 1, 2048)])
def test_small_m_gemv_path(oracle, m, n, k):
    """m <= 4 with k_in % 2048 == 0 takes the GEMV-shaped kernel: same bound as the tiles."""
    print(f"int8_tile gemv m={m} n={n} k={k}", flush=True)
    rng = np.random.default_rng(m * 31 + n + k)
    x, q, s = _case(rng, m, n, k)
    y = host(H.int8_tile_gemm(dev(x), dev(q), dev(s), n, k, m=m))
    if n * k <= 1 << 26:
        _check(oracle, y, x, q, s, m, n, k, "gemv")
    else:  # a column sample: rows of W
        cols = np.unique(np.concatenate([[0, n - 1], rng.integers(0, n, 40)]))
        qs = q.reshape(n, k)[cols].reshape(-1)
        ss = s.reshape(n, k // 64)[cols].reshape(-1)
        _check(oracle, y.reshape(m, n)[:, cols], x, qs, ss, m, cols.size, k, "gemv (row sample)")


def test_small_m_gemv_one_hot_is_exact(oracle):
    """x = e_c on the GEMV path: y[n] = BF16(q[n, c] * scale) for every row."""
    n, k = 300, 2048
    rng = np.random.default_rng(8)
    q = rng.integers(-127, 128, n * k, dtype=np.int8)
    s = np.ldexp(1.0 + rng.random(n * k // 64), rng.integers(-12, -4, n * k // 64)).astype(np.float32)
    w = oracle.int8_pin_dequant_bf16(q, s).reshape(n, k)
    dq, ds = dev(q), dev(s)
    for c in (0, 1, 63, 64, 1000, 2047):
        x = np.zeros(k, np.uint16)
        x[c] = 0x3F80
        y = host(H.int8_tile_gemm(dev(x), dq, ds, n, k, m=1))
        want = (w[:, c].astype(np.uint32) << 16).view(np.float32)
        assert y.view(np.uint32).tobytes() == want.view(np.uint32).tobytes(), c


def test_small_m_gemv_extreme_scales_are_exact(oracle):
    """The GEMV path forms q s as fma(q + 128, s, -128 s), which is the f32 product
    exactly while -128 s is finite. Blocks with s = 2^121 (-128 s overflows: the lane must
    take the plain multiply; q is kept in {-1, 0, 1} so q s stays finite), the smallest
    subnormal, subnormal products and zero: one-hot x gives y[n] = BF16(q[n, c] * s) bit
    for bit."""
    n, k = 64, 2048
    rng = np.random.default_rng(9)
    q = rng.integers(-127, 128, n * k, dtype=np.int8)
    s = np.ldexp(1.0 + rng.random(n * k // 64), rng.integers(-12, -4, n * k // 64)).astype(np.float32)
    special = [np.float32(2.0 ** 121), np.float32(-(2.0 ** 121)), np.float32(2.0 ** -149), np.float32(2.0 ** -140),
               np.float32(3.0 * 2.0 ** -135), np.float32(0.0)]
    for i, v in enumerate(special):
        for blk in range(i, n * k // 64, 7 * len(special)):
            s[blk] = v
            if abs(v) > 1.0:
                q[blk * 64:(blk + 1) * 64] = rng.integers(-1, 2, 64, dtype=np.int8)
    w = oracle.int8_pin_dequant_bf16(q, s).reshape(n, k)
    dq, ds = dev(q), dev(s)
    for c in (0, 5, 64, 1000, 2047):
        x = np.zeros(k, np.uint16)
        x[c] = 0x3F80
        y = host(H.int8_tile_gemm(dev(x), dq, ds, n, k, m=1))
        want = (w[:, c].astype(np.uint32) << 16).view(np.float32) + np.float32(0.0)  # the sum starts at +0
        assert y.view(np.uint32).tobytes() == want.view(np.uint32).tobytes(), \
            (c, first_diff(y.view(np.uint32), want.view(np.uint32)))


@pytest.mark.parametrize("k,aligned", [(64, True), (128, True), (640, True), (100, False), (37, False),
                                       (4096, True)])
def test_one_hot_rows_give_the_dequantized_weights_exactly(oracle, k, aligned):
    """x = I (m = k one-hot rows): y[m, n] = BF16(q[n, m] * scale) exactly, since every sum
    has one nonzero term. Pins the in-register dequantization bit for bit; k = 4096 with
    n = 3100 (208 tiles of 256 x 256) runs the 256 x 256 tile whose x goes straight into
    LDS, so it pins that tile's x placement too."""
    n = 3100 if k == 4096 else 100
    print(f"int8_tile one-hot k={k}", flush=True)
    rng = np.random.default_rng(k)
    q = rng.integers(-127, 128, n * k, dtype=np.int8)
    s = np.ldexp(1.0 + rng.random((n * k + 63) // 64), rng.integers(-12, -4, (n * k + 63) // 64)).astype(np.float32)
    x = bf16_bits(np.eye(k, dtype=np.float32))
    y = host(H.int8_tile_gemm(dev(x, pad_front=0 if aligned else 1), dev(q), dev(s), n, k, m=k))
    w = oracle.int8_pin_dequant_bf16(q, s).reshape(n, k)
    want = (w.astype(np.uint32) << 16).view(np.float32).T
    assert y.view(np.uint32).tobytes() == np.ascontiguousarray(want).view(np.uint32).tobytes(), \
        first_diff(y.view(np.uint32), np.ascontiguousarray(want).view(np.uint32))


def test_pending_error_is_returned_without_launching():
    """test_int8_tile_gemm.cu:242-278: a failed allocation leaves an error pending; the first
    call returns it and leaves y alone, the second runs."""
    torch = torch_cuda()
    lib = H.p7_lib()
    x = torch.zeros(16, dtype=torch.int16, device="cuda")
    q = torch.zeros(16, dtype=torch.int8, device="cuda")
    s = torch.ones(1, dtype=torch.float32, device="cuda")
    y = torch.full((1,), 7.0, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    lin = H.Int8PinLinear(q.data_ptr(), s.data_ptr(), 1, 16)
    # hipMalloc of the runtime this library is bound to (dlsym through its dependencies)
    hip_malloc = lib.hipMalloc
    hip_malloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
    hip_malloc.restype = ctypes.c_int
    p = ctypes.c_void_p()
    provoked = hip_malloc(ctypes.byref(p), 1 << 50)
    first = lib.int8_tile_gemm_bf16(x.data_ptr(), lin, y.data_ptr(), 1, None)
    torch.cuda.synchronize()
    y_first = float(y.cpu()[0])
    second = lib.int8_tile_gemm_bf16(x.data_ptr(), lin, y.data_ptr(), 1, None)
    torch.cuda.synchronize()
    y_after = float(y.cpu()[0])
    print(f"provoked={provoked} first={first} second={second} y={y_first} -> {y_after}", flush=True)
    assert provoked != 0 and first == provoked and y_first == 7.0
    assert second == 0 and y_after == 0.0


def test_argument_rules():
    torch = torch_cuda()
    lib = H.p7_lib()
    x = torch.zeros(64, dtype=torch.int16, device="cuda")
    q = torch.zeros(64, dtype=torch.int8, device="cuda")
    s = torch.ones(1, dtype=torch.float32, device="cuda")
    y = torch.full((1,), 7.0, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    lin = H.Int8PinLinear(q.data_ptr(), s.data_ptr(), 1, 64)
    assert lib.int8_tile_gemm_bf16(x.data_ptr(), lin, y.data_ptr(), 0, None) == 0  # m == 0: nothing to do
    assert lib.int8_tile_gemm_bf16(x.data_ptr(), lin, y.data_ptr(), -1, None) == 1
    assert lib.int8_tile_gemm_bf16(None, lin, y.data_ptr(), 1, None) == 1
    assert lib.int8_tile_gemm_bf16(x.data_ptr(), H.Int8PinLinear(q.data_ptr(), s.data_ptr(), 0, 64), y.data_ptr(), 1,
                                   None) == 1
    assert lib.int8_tile_gemm_bf16(x.data_ptr(), H.Int8PinLinear(q.data_ptr(), s.data_ptr(), 1, 0), y.data_ptr(), 1,
                                   None) == 1
    assert lib.int8_tile_gemm_bf16(x.data_ptr(), H.Int8PinLinear(q.data_ptr(), None, 1, 64), y.data_ptr(), 1,
                                   None) == 1
    torch.cuda.synchronize()
    assert float(y.cpu()[0]) == 7.0
