"""GPU parity for the rest of the attach ABI.

The INT8 late-plug family is checked bit for bit against the oracle:
- int8_mma_gemm_plug is two passes;
- int8_mma_gemm_plug_fused is one kernel;
- p7_int8_gemm_plug_flat is the fused kernel with flat arguments;
- int8_mma_gemm_resolve adds a re-quantized activation residual.

The plug streamer's 2-slot ring is checked in five ways:
- delayed readers over several passes, with 1, 2, 3 and 8 layers: only 3+ layers can
  observe a refill that skipped its slot_free wait (test_glint_plug_streamer.cu:1-4);
- poison after release (test_plug_evict_real.cu:1-12): each acquired slot is compared with
  a resident copy and then overwritten with poison before release, over two passes; the
  control pass poisons before the compare and must see mismatches;
- GLINT plug planes streamed into launch_glint_htile_s3_f32_stream over plain, poisoned
  and delayed passes, bitwise equal to the resident plug (test_streamer_real_weights.cu:
  1-9, 216-233);
- the ordering return codes;
- the attach self-test.

When oracle/_ref holds it, the reference's own checker, cuda/p7_attach_check.c built
from source, is also run against the library.
"""
import subprocess
from pathlib import Path

import numpy as np
import pytest

from glint_amd import glint_hip as H
from tests.gpu_util import dev, host, bf16_bits, first_diff, torch_cuda

pytestmark = pytest.mark.gpu
ROOT = Path(__file__).resolve().parent.parent


def _case(rng, m, n, k):
    x = bf16_bits(rng.normal(0, 1, m * k).astype(np.float32))
    wq = rng.integers(-127, 128, n * k, dtype=np.int8)
    sw = rng.uniform(1e-3, 2e-2, n * (k // 64)).astype(np.float32)
    q4 = rng.integers(0, 256, (n * k + 1) // 2, dtype=np.uint8)
    sp = rng.uniform(1e-4, 2e-3, n * (k // 64)).astype(np.float32)
    return x, wq, sw, q4, sp


SHAPES = [(70, 192, 256), (1, 64, 64), (33, 100, 640), (130, 257, 512)]


@pytest.mark.parametrize("m,n,k", SHAPES)
def test_plug_two_pass_and_fused_match_oracle(oracle, m, n, k):
    print(f"plug m={m} n={n} k={k}", flush=True)
    rng = np.random.default_rng(m * 7 + n)
    x, wq, sw, q4, sp = _case(rng, m, n, k)
    xq, sx = oracle.quant_act(x, m, k)
    pq = oracle.unpack_res4(q4, n * k)
    base = oracle.int8_mma_emu(xq, sx, wq, sw, m, n, k)
    want2 = base + oracle.int8_mma_emu(xq, sx, pq, sp, m, n, k)
    wantf = oracle.int8_mma_plug_fused(xq, sx, wq, sw, pq, sp, m, n, k)
    dx, dq, ds, dq4, dsp = dev(x), dev(wq), dev(sw), dev(q4), dev(sp)
    got2 = host(H.int8_mma_gemm_plug(dx, dq, ds, dq4, dsp, n, k, fused=False))
    assert got2.tobytes() == want2.tobytes(), first_diff(got2.view(np.uint32), want2.view(np.uint32))
    gotf = host(H.int8_mma_gemm_plug(dx, dq, ds, dq4, dsp, n, k, fused=True))
    assert gotf.tobytes() == wantf.tobytes(), first_diff(gotf.view(np.uint32), wantf.view(np.uint32))
    # the flat FFI entry is the fused kernel
    torch = torch_cuda()
    y = torch.empty(m * n, dtype=torch.float32, device="cuda")
    xqb = torch.empty(m * k, dtype=torch.int8, device="cuda")
    sxb = torch.empty(m * (k // 64), dtype=torch.float32, device="cuda")
    p = lambda t: t.data_ptr()
    st = torch.cuda.current_stream().cuda_stream
    assert H.p7_lib().p7_int8_gemm_plug_flat(p(dx), p(dq), p(ds), p(dq4), p(dsp), n, k, p(y), m, p(xqb), p(sxb),
                                             st) == 0
    assert host(y).tobytes() == wantf.tobytes()


@pytest.mark.parametrize("with_plug", [False, True])
def test_resolve_matches_oracle(oracle, with_plug):
    m, n, k = 45, 130, 384
    print(f"resolve plug={with_plug}", flush=True)
    rng = np.random.default_rng(31 + with_plug)
    x, wq, sw, q4, sp = _case(rng, m, n, k)
    xq, sx = oracle.quant_act(x, m, k)
    rq, sr = oracle.quant_act_resid(x, xq, sx, m, k)
    want = oracle.int8_mma_emu(xq, sx, wq, sw, m, n, k)
    want = want + oracle.int8_mma_emu(rq, sr, wq, sw, m, n, k)
    if with_plug:
        pq = oracle.unpack_res4(q4, n * k)
        want = want + oracle.int8_mma_emu(xq, sx, pq, sp, m, n, k)
        want = want + oracle.int8_mma_emu(rq, sr, pq, sp, m, n, k)
    args = dict(plug_q4=dev(q4), plug_scale=dev(sp)) if with_plug else {}
    y, gxq, gsx, grq, gsr = H.int8_mma_gemm_resolve(dev(x), dev(wq), dev(sw), n, k, **args)
    assert host(gxq).tobytes() == xq.tobytes() and host(gsx).tobytes() == sx.tobytes()
    assert host(grq).tobytes() == rq.tobytes(), first_diff(host(grq), rq)
    assert host(gsr).tobytes() == sr.tobytes()
    got = host(y)
    assert got.tobytes() == want.tobytes(), first_diff(got.view(np.uint32), want.view(np.uint32))


# ------------------------------------------------------------------ plug streamer
N_OUT, K_IN = 256, 512
QPAD = (N_OUT * K_IN + 255) // 256 * 256
BLOB = QPAD + N_OUT * (K_IN // 64) * 4


def _layer_blob(l):
    rng = np.random.default_rng(100 + l)
    q = rng.integers(-127, 128, N_OUT * K_IN, dtype=np.int8)
    s = rng.uniform(1e-3, 2e-2, N_OUT * (K_IN // 64)).astype(np.float32)
    b = np.zeros(BLOB, np.uint8)
    b[:q.size] = q.view(np.uint8)
    b[QPAD:] = s.view(np.uint8)
    return b


def _gemm_on(torch, p7, x, qptr, y, xq, sx, stream):
    lin = H.Int8MmaLinear(qptr, qptr + QPAD, N_OUT, K_IN)
    m = x.numel() // K_IN
    assert p7.int8_mma_gemm(x.data_ptr(), lin, y.data_ptr(), m, xq.data_ptr(), sx.data_ptr(), stream.cuda_stream) == 0


@pytest.mark.parametrize("n_layers", [1, 2, 3, 8])
def test_streamer_delayed_readers_see_their_own_layer(n_layers):
    """Every read is preceded on the compute stream by a ~1 ms spin. Each pass must compute
    exactly what the resident layer computes; the stats count every layer once per pass."""
    torch = torch_cuda()
    p7 = H.p7_lib()
    print(f"streamer n_layers={n_layers}", flush=True)
    blobs = [_layer_blob(l) for l in range(n_layers)]
    m = 40
    x = dev(bf16_bits(np.random.default_rng(5).normal(0, 1, m * K_IN).astype(np.float32)))
    xq = torch.empty(m * K_IN, dtype=torch.int8, device="cuda")
    sx = torch.empty(m * (K_IN // 64), dtype=torch.float32, device="cuda")
    main = torch.cuda.current_stream()
    ref = []
    for b in blobs:
        db = dev(b)
        y = torch.empty(m * N_OUT, dtype=torch.float32, device="cuda")
        _gemm_on(torch, p7, x, db.data_ptr(), y, xq, sx, main)
        ref.append(host(y))
    copy_s, comp_s = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    ps = H.PlugStreamer([BLOB] * n_layers, copy_s, comp_s)
    try:
        for l, b in enumerate(blobs):
            assert ps.set_host_data(l, b.tobytes()) == 0
        passes = 3
        outs = [[torch.empty(m * N_OUT, dtype=torch.float32, device="cuda") for _ in range(n_layers)]
                for _ in range(passes)]
        xqs = torch.empty(m * K_IN, dtype=torch.int8, device="cuda")
        sxs = torch.empty(m * (K_IN // 64), dtype=torch.float32, device="cuda")
        spin = int(2.4e6)  # ~1 ms of GPU clock: a bounded busy wait
        for p in range(passes):
            assert ps.start() == 0
            for l in range(n_layers):
                rc, ptr = ps.acquire(l)
                assert rc == 0 and ptr
                with torch.cuda.stream(comp_s):
                    torch.cuda._sleep(spin)
                _gemm_on(torch, p7, x, ptr, outs[p][l], xqs, sxs, comp_s)
                assert ps.release(l) == 0
        torch.cuda.synchronize()
        for p in range(passes):
            for l in range(n_layers):
                got = host(outs[p][l])
                assert got.tobytes() == ref[l].tobytes(), f"pass {p} layer {l}"
        st = ps.stats()
        assert st.total_h2d_bytes == passes * n_layers * BLOB
        assert st.n_layers == n_layers
        assert st.total_stall_ms >= 0.0
    finally:
        ps.close()


class _DevBytes:
    """A raw device byte range as a torch tensor view (through __cuda_array_interface__)."""

    def __init__(self, ptr, nbytes):
        self.__cuda_array_interface__ = {"shape": (nbytes,), "typestr": "|u1", "data": (ptr, False), "version": 3,
                                         "strides": None}


def _slot_view(torch, ptr, nbytes):
    return torch.as_tensor(_DevBytes(ptr, nbytes), device="cuda")


def test_streamer_poison_after_release_and_control():
    """test_plug_evict_real.cu restated on synthetic layers of mixed sizes (>= 64 KiB, one
    odd): for every layer, acquire, compare the slot byte for byte with a resident copy,
    overwrite the slot with poison, release, all on the compute stream. If a read ever saw
    a slot before its copy landed, or a refill overwrote a slot still being read, bytes
    would differ. Two passes, so a stale slot from pass 1 cannot satisfy pass 2. Control:
    with the poison moved before the compare, mismatches must appear, or the harness could
    not see poison at all."""
    torch = torch_cuda()
    sizes = [65536, 200_000, 1_048_583, 98_304, 300_000]
    rng = np.random.default_rng(77)
    data = [rng.integers(0, 256, n, dtype=np.uint8) for n in sizes]
    for d in data:
        d[d == 0xA5] = 0x5A  # no byte equals the poison, so the control counts every byte
    ref = [dev(d) for d in data]
    copy_s, comp_s = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    ps = H.PlugStreamer(sizes, copy_s, comp_s)
    bad = torch.zeros(1, dtype=torch.int64, device="cuda")

    def run_pass(poison_before_read):
        bad.zero_()
        torch.cuda.synchronize()
        assert ps.start() == 0
        for l, n in enumerate(sizes):
            rc, ptr = ps.acquire(l)
            assert rc == 0 and ptr
            with torch.cuda.stream(comp_s):
                slot = _slot_view(torch, ptr, n)
                if poison_before_read:
                    slot.fill_(0xA5)
                bad.add_((slot != ref[l]).sum())
                if not poison_before_read:
                    slot.fill_(0xA5)
            assert ps.release(l) == 0
        torch.cuda.synchronize()
        return int(bad.item())

    try:
        for l, d in enumerate(data):
            assert ps.set_host_data(l, d.tobytes()) == 0
        for p in range(2):
            print(f"poison-after-release pass {p}", flush=True)
            assert run_pass(False) == 0, p
        print("control pass: poison before the compare", flush=True)
        assert run_pass(True) == sum(sizes)
        assert ps.stats().total_h2d_bytes == 3 * sum(sizes)
    finally:
        torch.cuda.synchronize()
        ps.close()


def test_streamer_glint_plug_into_htile(oracle):
    """test_streamer_real_weights.cu restated on synthetic GLINT units: the plug planes of
    four encoded weights (mixed N, K, bs 64) go through the 2-slot streamer into
    launch_glint_htile_s3_f32_stream on the compute stream (M = 4), hole and absmax resident.
    Over six back-to-back passes (plain, plain, poisoned, poisoned, delayed, delayed) every
    streamed output equals the output of the resident plug bit for bit. A poisoned pass
    copies random bytes into each released slot on the copy stream behind the release; a
    delayed pass spins about 1 ms on the compute stream before each launch, so a refill
    that skipped its slot wait would land under the reader."""
    torch = torch_cuda()
    M = 4
    shapes = [(256, 1024), (512, 2048), (384, 4096), (128, 2048)]
    rng = np.random.default_rng(91)
    units = []
    for i, (N, K) in enumerate(shapes):
        w = rng.normal(0, 0.02, N * K).astype(np.float32)
        hole, plug, am = oracle.encode_f32(w, 64)
        x = bf16_bits(rng.normal(0, 1, M * K).astype(np.float32))
        units.append(dict(N=N, K=K, hole=dev(hole), plug=plug, dplug=dev(plug), am=dev(am), x=dev(x)))
    copy_s, comp_s = torch.cuda.Stream(), torch.cuda.Stream()
    lib = H.encode_lib()
    cs = H._stream(comp_s)

    def htile(u, plug_ptr, y):
        assert lib.launch_glint_htile_s3_f32_stream(u["hole"].data_ptr(), plug_ptr, u["am"].data_ptr(),
                                                    u["x"].data_ptr(), y.data_ptr(), M, u["N"], u["K"], 64, cs) == 0

    torch.cuda.synchronize()
    resident = []
    for u in units:
        y = torch.empty(M * u["N"], dtype=torch.float32, device="cuda")
        htile(u, u["dplug"].data_ptr(), y)
        resident.append(y)
    torch.cuda.synchronize()
    sizes = [u["plug"].size for u in units]
    poison = torch.from_numpy(rng.integers(0, 256, max(sizes), dtype=np.uint8)).pin_memory()
    kinds = ["plain", "plain", "poisoned", "poisoned", "delayed", "delayed"]
    outs = [[torch.empty(M * u["N"], dtype=torch.float32, device="cuda") for u in units] for _ in kinds]
    ps = H.PlugStreamer(sizes, copy_s, comp_s)
    try:
        for i, u in enumerate(units):
            assert ps.set_host_data(i, u["plug"].tobytes()) == 0
        for p, kind in enumerate(kinds):
            print(f"streamed H-TILE pass {p} ({kind})", flush=True)
            assert ps.start() == 0
            assert ps.acquire(1)[0] == -10  # layer 1 before layer 0 is released
            for i, u in enumerate(units):
                rc, ptr = ps.acquire(i)
                assert rc == 0 and ptr
                if kind == "delayed":
                    with torch.cuda.stream(comp_s):
                        torch.cuda._sleep(int(2.4e6))  # a bounded ~1 ms spin
                htile(u, ptr, outs[p][i])
                assert ps.release(i) == 0
                if kind == "poisoned":
                    ev = torch.cuda.Event()
                    ev.record(comp_s)
                    copy_s.wait_event(ev)
                    with torch.cuda.stream(copy_s):
                        _slot_view(torch, ptr, sizes[i]).copy_(poison[:sizes[i]], non_blocking=True)
        torch.cuda.synchronize()
        for p, kind in enumerate(kinds):
            for i, u in enumerate(units):
                got, want = host(outs[p][i]), host(resident[i])
                assert got.tobytes() == want.tobytes(), (p, kind, i, first_diff(got.view(np.uint32), want.view(np.uint32)))
    finally:
        torch.cuda.synchronize()
        ps.close()


def test_streamer_ordering_codes():
    """test_glint_plug_streamer.cu:79-98: out-of-order release/acquire/start are refused."""
    torch = torch_cuda()
    copy_s, comp_s = torch.cuda.Stream(), torch.cuda.Stream()
    ps = H.PlugStreamer([4096] * 3, copy_s, comp_s)
    try:
        for l in range(3):
            assert ps.set_host_data(l, bytes([l]) * 4096) == 0
        assert ps.set_host_data(0, b"x" * 10) == -2
        assert ps.release(0) == -11            # before start
        assert ps.acquire(0)[0] == -10         # before start
        assert ps.start() == 0
        assert ps.release(0) == -11            # before acquire(0)
        assert ps.acquire(1)[0] == -10         # out of order
        assert ps.acquire(0)[0] == 0
        assert ps.release(1) == -11            # before release(0)
        assert ps.release(0) == 0
        assert ps.release(0) == -11            # twice
        assert ps.release(1) == -11            # before acquire(1)
        assert ps.start() == -6                # pass not finished
        assert ps.acquire(1)[0] == 0 and ps.release(1) == 0
        assert ps.acquire(2)[0] == 0 and ps.release(2) == 0
        assert ps.start() == 0                 # next pass after the last release
        for l in range(3):
            assert ps.acquire(l)[0] == 0 and ps.release(l) == 0
        torch.cuda.synchronize()
        assert ps.stats().total_h2d_bytes == 2 * 3 * 4096
    finally:
        ps.close()


def test_attach_selftest_passes():
    rc, msg = H.p7_selftest()
    print(msg, flush=True)
    assert rc == 0, msg
    assert "abi=p7_attach_abi_v1" in msg and "mismatches=0" in msg


def test_reference_attach_checker():
    """cuda/p7_attach_check.c, compiled from the reference source into oracle/_ref, loads the
    library, requires its 12 symbols and the ABI string, and runs the self-test."""
    chk = ROOT / "oracle" / "_ref" / "p7_attach_check"
    if not chk.is_file():
        pytest.skip("oracle/_ref/p7_attach_check not built (needs the reference sources)")
    lib = H.p7_lib_path()
    out = subprocess.run([str(chk), str(lib), "p7_attach_abi_v1"], capture_output=True, text=True, timeout=120)
    print(out.stdout, out.stderr, flush=True)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "P7_SELFTEST rc=0" in out.stdout
