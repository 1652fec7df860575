"""GPU parity for the K-major decode path (include/glint_select.h): layout conversion,
fold GEMV, channel selection and plug correction, each bit for bit against the oracle
(the kernels keep the oracle's summation orders), plus the chained decode step and the
argument codes."""
import ctypes
import os

import numpy as np
import pytest

from glint_amd import glint_hip as H
from oracle import glint_oracle as G
from tests.gpu_util import dev, host, first_diff, torch_cuda

pytestmark = pytest.mark.gpu


def _pin(oracle, N, K, seed):
    rng = np.random.default_rng(seed)
    w = rng.normal(0, 0.02, N * K).astype(np.float32)
    w[:64] = 0.0
    w[rng.integers(0, N * K, 50)] *= 10
    return oracle.encode_f32(w, 64)


def _x(K, seed):
    return G.f32_to_bf16_bits(np.random.default_rng(seed).normal(0, 1, K).astype(np.float32))


PACK_SHAPES = [(8, 64), (24, 192), (104, 640), (1000, 320), (14336, 4096), (4096, 14336)]
FOLD_SHAPES = [(32, 64), (96, 512), (1024, 320), (2080, 1024), (14336, 4096), (4096, 14336)]


@pytest.mark.parametrize("N,K", PACK_SHAPES)
def test_kmajor_pack_matches_oracle(oracle, N, K):
    torch_cuda()
    print(f"kmajor pack N={N} K={K}", flush=True)
    h, p, am = _pin(oracle, N, K, N + K)
    hk, pk, sk = oracle.kmajor_pack(h, p, am, N, K)
    dhk, dpk, dsk = H.kmajor_pack(dev(h), dev(p), dev(am), N, K)
    assert host(dhk).tobytes() == hk.tobytes(), first_diff(host(dhk), hk)
    assert host(dpk).tobytes() == pk.tobytes(), first_diff(host(dpk), pk)
    assert host(dsk).tobytes() == sk.tobytes()


@pytest.mark.parametrize("N,K", FOLD_SHAPES)
def test_fold_matches_oracle(oracle, N, K):
    torch_cuda()
    print(f"fold N={N} K={K}", flush=True)
    h, p, am = _pin(oracle, N, K, N + K)
    hk, pk, sk = oracle.kmajor_pack(h, p, am, N, K)
    dhk, dsk = dev(hk), dev(sk)
    x = _x(K, K)
    dx = dev(x)
    for ksg in (1, 2, 8):
        if K % (64 * ksg):
            continue
        want = oracle.gemv_km_fold(hk, sk, x, N, K, ksg)
        got = host(H.gemv_km_fold(dhk, dsk, dx, N, K, ksg))
        assert got.tobytes() == want.tobytes(), (ksg, first_diff(got.view(np.uint32), want.view(np.uint32)))


@pytest.mark.parametrize("K", [1, 64, 1000, 4096, 14336, 32768])
def test_select_matches_oracle(oracle, K):
    torch_cuda()
    print(f"select K={K}", flush=True)
    x = _x(K, 7 + K)
    if K > 200:
        x[100:160] = x[3]  # ties at many thresholds
    dx = dev(x)
    for nsel in sorted({-1, 0, 1, 2, K // 10, K // 2, K - 1, K, K + 3}):
        want = oracle.select_topk(x, K, nsel)
        idx, cnt = H.select_topk(dx, nsel)
        n = int(host(cnt)[0])
        assert n == want.size, (nsel, n, want.size)
        assert np.array_equal(host(idx)[:n], want), nsel


@pytest.mark.parametrize("K", [1, 100, 4096, 14336, 32768])
def test_select_price_floor_and_log_match_oracle(oracle, K):
    """glint_select_topk_ex: fixed price (tkey > 0), relational price (tkey < 0, the f32
    mean in the rule's order), the floor, and the count log slot, against the oracle."""
    torch = torch_cuda()
    print(f"select_ex K={K}", flush=True)
    rng = np.random.default_rng(K + 5)
    x = G.f32_to_bf16_bits((rng.normal(0, 1, K) * 2.0 ** rng.integers(-6, 6, K)).astype(np.float32))
    if K > 64:
        x[10:40] = x[3]
        x[50] = 0x7F80  # inf key, clamped in the mean
        x[51] = 0x0003  # subnormal key, 0 in the mean
    dx = dev(x)
    keys = (x & 0x7FFF).astype(np.int64)
    log = torch.full((8,), -7, dtype=torch.int32, device="cuda")
    cases = [(max(K // 10, 1), int(np.median(keys)), 0), (max(K // 10, 1), -1024, 0), (max(K // 10, 1), -300, 0),
             (max(K // 2, 1), -4000, max(K // 20, 1)), (max(K // 50, 1), 32000, max(K // 5, 1)),
             (max(K // 50, 1), -1, 3), (0, -1024, 5), (-1, 100, 2), (K, -2048, 1), (3, 0, 2)]
    for slot, (nsel, tkey, nfloor) in enumerate(cases):
        want = oracle.select_ex(x, K, nsel, tkey, nfloor)
        idx, cnt = H.select_topk(dx, nsel, tkey=tkey, nfloor=nfloor, cnt_log=log, slot=slot % 8)
        n = int(host(cnt)[0])
        assert n == want.size, (nsel, tkey, nfloor, n, want.size)
        assert np.array_equal(host(idx)[:n], want), (nsel, tkey, nfloor)
        assert int(host(log)[slot % 8]) == n


@pytest.mark.parametrize("N,K,frac,ks", [(96, 640, 0.1, 1), (1024, 320, 0.5, 3), (2080, 1024, 0.3, 2),
                                         (14336, 4096, 0.1, 8), (4096, 14336, 0.05, 1), (4096, 14336, 1.0, 8)])
def test_decode_step_matches_oracle(oracle, N, K, frac, ks):
    """fold -> select (on the device) -> correction, every stage bit-exact; with every
    channel selected the result is the H-TILE GEMV within the f32 bound."""
    torch = torch_cuda()
    print(f"decode step N={N} K={K} frac={frac} ks={ks}", flush=True)
    h, p, am = _pin(oracle, N, K, 3 * N + K)
    hk, pk, sk = oracle.kmajor_pack(h, p, am, N, K)
    x = _x(K, 11 + K)
    nsel = int(np.ceil(frac * K))
    ksg = 4 if K % 256 == 0 else 1
    y0 = oracle.gemv_km_fold(hk, sk, x, N, K, ksg)
    sel = oracle.select_topk(x, K, nsel)
    want = oracle.apply_corr_km(hk, pk, sk, x, sel, N, K, y0, ks)
    dhk, dpk, dsk, dx = dev(hk), dev(pk), dev(sk), dev(x)
    y = H.gemv_km_fold(dhk, dsk, dx, N, K, ksg)
    idx, cnt = H.select_topk(dx, nsel)
    H.apply_corr_km(dhk, dpk, dsk, dx, idx, cnt, y, N, K, ks)
    got = host(y)
    assert got.tobytes() == want.tobytes(), first_diff(got.view(np.uint32), want.view(np.uint32))
    if frac == 1.0:
        ref, absum = oracle.htile_f64(h, p, am, x, 1, N, K, 64)
        assert np.all(np.abs(got.astype(np.float64) - ref[0]) <= (K + 4) * 2.0 ** -23 * absum[0] * 2)
    del torch


def test_correction_reads_plug_rows_from_pinned_host_memory(oracle):
    """The reference keeps the K-major plug plane in pinned host memory and reads only the
    selected channels' rows (mojo/p7_glint_select_decode.mojo:1-4). The same call with
    plug_k in pinned host memory (read over the bus, zero copy) gives the bytes of the
    device-resident plug, and the oracle's, at the decode shape."""
    torch = torch_cuda()
    N, K, ks = 14336, 4096, 8
    print(f"host plug correction N={N} K={K} ks={ks}", flush=True)
    h, p, am = _pin(oracle, N, K, 99)
    hk, pk, sk = oracle.kmajor_pack(h, p, am, N, K)
    x = _x(K, 1234)
    dhk, dsk, dx = dev(hk), dev(sk), dev(x)
    # mapped pinned host memory and its device address (hipHostMalloc + hipHostGetDevicePointer)
    hip = ctypes.CDLL(os.path.join(os.path.dirname(torch.__file__), "lib", "libamdhip64.so"))
    hbuf, dptr = ctypes.c_void_p(), ctypes.c_void_p()
    assert hip.hipHostMalloc(ctypes.byref(hbuf), ctypes.c_size_t(pk.nbytes), ctypes.c_uint(0x2)) == 0  # Mapped
    try:
        assert hip.hipHostGetDevicePointer(ctypes.byref(dptr), hbuf, ctypes.c_uint(0)) == 0 and dptr.value
        ctypes.memmove(hbuf, pk.ctypes.data, pk.nbytes)
        y0 = H.gemv_km_fold(dhk, dsk, dx, N, K, 16)
        idx, cnt = H.select_topk(dx, K // 10)
        y_dev = H.apply_corr_km(dhk, dev(pk), dsk, dx, idx, cnt, y0.clone(), N, K, ks)
        y_host = y0.clone()
        lib = H.encode_lib()
        P = lambda t: ctypes.c_void_p(t.data_ptr())
        assert lib.glint_apply_corr_km(P(dhk), dptr, P(dsk), P(dx), P(idx), P(cnt), P(y_host), N, K, ks,
                                       P(torch.empty(ks * N, dtype=torch.float32, device="cuda")), None) == 0
    finally:
        torch.cuda.synchronize()  # nothing may still read the buffer when it is freed
        hip.hipHostFree(hbuf)
    assert host(y_host).tobytes() == host(y_dev).tobytes()
    want = oracle.apply_corr_km(hk, pk, sk, x, oracle.select_topk(x, K, K // 10), N, K, host(y0), ks)
    assert host(y_host).tobytes() == want.tobytes()


def test_decode_step_under_graph_capture(oracle):
    """Fold, select and correction captured into one graph, on a stream that has a split
    workspace (the slices meet in-kernel through its counters) and on one that has none
    (the capture cannot allocate: the slices meet in the combine kernel). Every replay,
    with eager decode steps and synchronisations between them, equals the eager result
    bit for bit."""
    torch = torch_cuda()
    N, K, ksg, ks = 4096, 4096, 16, 8
    print(f"graph capture decode step N={N} K={K}", flush=True)
    h, p, am = _pin(oracle, N, K, 4501)
    hk, pk, sk = oracle.kmajor_pack(h, p, am, N, K)
    x, x2 = _x(K, 4502), _x(K, 4503)
    dhk, dpk, dsk, dx, dx2 = dev(hk), dev(pk), dev(sk), dev(x), dev(x2)
    part = torch.empty(32 * N, dtype=torch.float32, device="cuda")

    def step(xx, y, idx, cnt, stream):
        H.gemv_km_fold(dhk, dsk, xx, N, K, ksg, y=y, part=part, stream=stream)
        H.select_topk(xx, K // 10, idx=idx, cnt=cnt, stream=stream)
        H.apply_corr_km(dhk, dpk, dsk, xx, idx, cnt, y, N, K, ks, part=part, stream=stream)

    for warm in (True, False):
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        y = torch.empty(N, dtype=torch.float32, device="cuda")
        idx = torch.empty(K, dtype=torch.int32, device="cuda")
        cnt = torch.empty(1, dtype=torch.int32, device="cuda")
        ye = torch.empty_like(y)
        if warm:
            assert H.encode_lib().glint_htile_workspace_reserve(ctypes.c_void_p(s.cuda_stream)) == 0
        s.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            step(dx, y, idx, cnt, s)
        torch.cuda.synchronize()
        want = oracle.apply_corr_km(hk, pk, sk, x, oracle.select_topk(x, K, K // 10), N, K,
                                    oracle.gemv_km_fold(hk, sk, x, N, K, ksg), ks)
        want2 = oracle.apply_corr_km(hk, pk, sk, x2, oracle.select_topk(x2, K, K // 10), N, K,
                                     oracle.gemv_km_fold(hk, sk, x2, N, K, ksg), ks)
        for rep in range(3):
            # the replay and the eager step share `part`: both go on `s`, one after the other
            with torch.cuda.stream(s):
                y.zero_()
                graph.replay()
                e_idx, e_cnt = torch.empty_like(idx), torch.empty_like(cnt)
                step(dx2, ye, e_idx, e_cnt, s)
            torch.cuda.synchronize()
            assert host(y).tobytes() == want.tobytes(), (warm, rep)
            assert host(ye).tobytes() == want2.tobytes(), (warm, rep)
        del graph


def test_fold_and_correction_allocate_nothing(oracle):
    """The fold and the correction with K slices (ksg, ks > 1) never allocate: on a stream
    with no split-K workspace they meet their slices in the combine kernel (device memory
    unchanged), on a stream with one (reserved ahead) through its arrival counters; both
    equal the oracle bit for bit."""
    torch = torch_cuda()
    N, K, ksg, ks = 4096, 14336, 8, 4
    h, p, am = _pin(oracle, N, K, 41)
    hk, pk, sk = oracle.kmajor_pack(h, p, am, N, K)
    dhk, dpk, dsk = dev(hk), dev(pk), dev(sk)
    x = _x(K, 42)
    dx = dev(x)
    idx = oracle.select_topk(x, K, K // 10)
    fold = oracle.gemv_km_fold(hk, sk, x, N, K, ksg)
    want = oracle.apply_corr_km(hk, pk, sk, x, idx, N, K, fold, ks)
    part = torch.empty(32 * N, dtype=torch.float32, device="cuda")
    y = torch.empty(N, dtype=torch.float32, device="cuda")
    di, dc = torch.empty(K, dtype=torch.int32, device="cuda"), torch.empty(1, dtype=torch.int32, device="cuda")
    got_fold = torch.empty_like(y)
    for reserve in (False, True):
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        if reserve:
            assert H.encode_lib().glint_htile_workspace_reserve(H._stream(s)) == 0
        torch.cuda.synchronize()
        free0 = torch.cuda.mem_get_info()[0]
        with torch.cuda.stream(s):
            H.gemv_km_fold(dhk, dsk, dx, N, K, ksg, y=y, part=part, stream=s)
            got_fold.copy_(y)
            H.select_topk(dx, K // 10, idx=di, cnt=dc, stream=s)
            H.apply_corr_km(dhk, dpk, dsk, dx, di, dc, y, N, K, ks, part=part, stream=s)
        torch.cuda.synchronize()
        assert torch.cuda.mem_get_info()[0] == free0, reserve
        assert host(got_fold).tobytes() == fold.tobytes(), reserve
        assert host(y).tobytes() == want.tobytes(), reserve
        assert H.encode_lib().glint_htile_workspace_release(H._stream(s)) == 0


def test_argument_codes():
    torch = torch_cuda()
    lib = H.encode_lib()
    b = torch.zeros(4096, dtype=torch.uint8, device="cuda")
    f = torch.zeros(4096, dtype=torch.float32, device="cuda")
    i = torch.zeros(64, dtype=torch.int32, device="cuda")
    P = lambda t: t.data_ptr()
    assert lib.glint_kmajor_pack(None, P(b), P(f), 8, 64, P(b), P(b), P(f), None) == -1
    assert lib.glint_kmajor_pack(P(b), P(b), P(f), 12, 64, P(b), P(b), P(f), None) == -2  # N % 8
    assert lib.glint_kmajor_pack(P(b), P(b), P(f), 8, 96, P(b), P(b), P(f), None) == -2  # K % 64
    assert lib.glint_gemv_km_fold(P(b), P(f), P(b), P(f), 32, 128, 2, None, None) == -1  # part needed
    assert lib.glint_gemv_km_fold(P(b), P(f), P(b), P(f), 32, 192, 2, P(f), None) == -2  # K % (64 ksg)
    assert lib.glint_gemv_km_fold(P(b), P(f), P(b), P(f), 40, 128, 1, None, None) == -2  # N % 32
    assert lib.glint_select_topk(P(b), 0, 1, P(i), P(i), None) == -2
    assert lib.glint_select_topk(P(b), 40000, 1, P(i), P(i), None) == -2
    assert lib.glint_select_topk_ex(P(b), 64, 1, 0, 0, P(i), P(i), P(i), -1, None) == -2  # slot < 0 with a log
    assert lib.glint_select_topk_ex(None, 64, 1, 0, 0, P(i), P(i), None, 0, None) == -1
    assert lib.glint_apply_corr_km(P(b), P(b), P(f), P(b), P(i), P(i), P(f), 32, 64, 2, None, None) == -1
    assert lib.glint_apply_corr_km(P(b), P(b), P(f), P(b), P(i), P(i), P(f), 48, 64, 1, None, None) == -2
    torch.cuda.synchronize()
