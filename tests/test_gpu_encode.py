"""GPU encode parity: pin bytes (hole, plug, absmax) identical to the CPU oracle.

Covers the reference's known answers and seeded data, every bf16 bit pattern, the
BASELINE 4096x4096 config at full size, ragged n, odd block sizes, misaligned pointers,
special blocks (zero, NaN, inf, absmax outside the fast divide's range), the f32 input
path and the host-pointer ABI."""
import random

import numpy as np
import pytest

from glint_amd import glint_hip as H
from oracle import glint_oracle as G
from tests.gpu_util import dev, host, first_diff, bf16_bits, torch_cuda

pytestmark = pytest.mark.gpu


def _gauss(n, seed, scale=0.02):
    rng = random.Random(seed)
    return [rng.gauss(0.0, scale) for _ in range(n)]


def gpu_encode(u16, bs, pad=0):
    w = dev(np.asarray(u16, np.uint16), pad)
    hole, plug, am = H.encode_bf16(w, bs)
    return host(hole), host(plug), host(am)


def assert_same(got, want, what=""):
    for name, g, w in zip(("hole", "plug", "absmax"), got, want):
        g = np.asarray(g)
        w = np.asarray(w)
        assert g.tobytes() == w.tobytes(), f"{what} {name}: {first_diff(g.view(np.uint8), w.view(np.uint8))}"


def test_gpu_ok_known_answer():
    from glint_amd import glint_cuda
    assert glint_cuda.gpu_ok()
    hole, plug, am = glint_cuda.encode_bf16_cuda(b"\x80\x3f\x00\x00", 2, 64)
    assert hole == b"\x7f" and plug == b"\x8f" and np.frombuffer(am, "<f4").tolist() == [1.0]
    h, p, a = gpu_encode(np.frombuffer(b"\x80\x3f\x00\x00", "<u2"), 64)
    assert bytes(h) == b"\x7f" and bytes(p) == b"\x8f" and a.tolist() == [1.0]


def test_reference_seeded_data(oracle):
    w = _gauss(64 * 41 + 7, 5)
    w[128:192] = [0.0] * 64
    u16 = bf16_bits(w)
    assert_same(gpu_encode(u16, 64), oracle.encode_bf16(u16, 64), "gauss(2631,5)")
    a = _gauss(16 * 64, 1)
    b = _gauss(8 * 63, 2)
    c = _gauss(4 * 128, 3)
    c[:64] = [0.0] * 64
    for i, vals in enumerate((a, b, c)):
        u16 = bf16_bits(vals)
        assert_same(gpu_encode(u16, 64), oracle.encode_bf16(u16, 64), f"toy shard {i}")


@pytest.mark.parametrize("order", ["natural", "shuffled"])
def test_every_bf16_pattern(oracle, order):
    u16 = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    if order == "shuffled":
        u16 = np.random.default_rng(42).permutation(u16)
    for bs in (64, 23):
        assert_same(gpu_encode(u16, bs), oracle.encode_bf16(u16, bs), f"all bf16 {order} bs={bs}")


def test_baseline_config_full_size(oracle):
    """W[4096x4096] ~ N(0, 0.02^2), seed 1001, 0.1% outliers x10,
    bs=64; against the oracle and the committed fixture digests (tests/golden/)."""
    import hashlib
    import json
    import sys
    from pathlib import Path
    gdir = Path(__file__).resolve().parent / "golden"
    sys.path.insert(0, str(gdir))
    import make_golden
    fixture = json.loads((gdir / "encode_4096x4096_outliers.json").read_text())
    u16 = make_golden.config0_input()
    n = u16.size
    sha = lambda a: hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()
    assert sha(u16) == fixture["input_bf16_sha256"]
    got = gpu_encode(u16, 64)
    want = oracle.encode_bf16(u16, 64)
    assert_same(got, want, "4096x4096")
    for name, a in zip(("hole", "plug", "absmax"), got):
        assert sha(a) == fixture[f"{name}_sha256"], name
    rec16 = host(H.expand_bf16(*(dev(a) for a in got), n, 64), np.uint16)
    assert sha(rec16) == fixture["expand_bf16_sha256"]
    rec = host(H.expand_f32(*(dev(a) for a in got), n, 64))
    assert rec.tobytes() == oracle.expand_f32(*want, n, 64).tobytes()
    rmse = float(np.sqrt(np.mean((G.bf16_bits_to_f32(rec16).astype(np.float64) - G.bf16_bits_to_f32(u16)) ** 2)))
    assert abs(rmse - fixture["expand_rmse"]) <= 1e-12
    # round trip through the GPU expand reproduces the oracle's reconstruction exactly
    torch = torch_cuda()
    hole, plug, am = (dev(a) for a in got)
    rec = host(H.expand_f32(hole, plug, am, n, 64))
    assert rec.tobytes() == oracle.expand_f32(*want, n, 64).tobytes()
    rmse = float(np.sqrt(np.mean((rec.astype(np.float64) - G.bf16_bits_to_f32(u16)) ** 2)))
    assert rmse < 5e-4


@pytest.mark.parametrize("bs", [1, 23, 64, 100, 128, 4096])
@pytest.mark.parametrize("pad", [0, 1])
def test_ragged_sizes_blocksizes_alignment(oracle, bs, pad):
    rng = np.random.default_rng(bs * 7 + pad)
    for n in (1, 2, 63, 64, 65, 511, 512, 513, 1000, 4097, 100003):
        u16 = bf16_bits(rng.normal(0, 0.02, n))
        assert_same(gpu_encode(u16, bs, pad), oracle.encode_bf16(u16, bs), f"n={n} bs={bs} pad={pad}")


def test_encode_in_pieces(oracle):
    """A tensor above 2^17 wave chunks (67 M elements) is encoded as equal consecutive
    launches: n = 2 * 2^17 * 512 + 5 * 512 + 100 gives three pieces of 87383 chunks and a
    100-element tail for the generic kernels. The bytes around every piece boundary and the
    tail match the oracle, and every absmax equals the block's largest magnitude."""
    torch = torch_cuda()
    n = 2 * (1 << 17) * 512 + 5 * 512 + 100
    print(f"encode in pieces n={n}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(515)
    w = (torch.randn(n, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    hole, plug, am = H.encode_bf16(w, 64)
    nch = (n // 512)
    per = (nch + 2) // 3
    edges = [0, per * 512, 2 * per * 512, (n // 512) * 512, n]
    for e in edges:
        lo, hi = max(0, (e - 4096) // 64 * 64), min(n, e + 4096)
        u16 = host(w[lo:hi].view(torch.int16), np.uint16)
        want = oracle.encode_bf16(u16, 64)
        got = (host(hole[lo // 2:(hi + 1) // 2]), host(plug[lo // 2:(hi + 1) // 2]), host(am[lo // 64:(hi + 63) // 64]))
        assert_same(got, want, f"edge {e}")
    full = n // 64 * 64
    amx = w[:full].float().abs().reshape(-1, 64).amax(dim=1)
    assert bool(torch.equal(amx, am[:full // 64])), "absmax"


def test_special_blocks(oracle):
    blocks = []
    z = np.zeros(64, np.float32)
    blocks.append(z.copy())                                  # all zero -> 0x77 / 0x88, absmax 0
    b = z.copy(); b[5] = np.nan; blocks.append(b)            # NaN in a zero block -> (7, 8)
    b = np.full(64, 0.25, np.float32); b[9] = np.nan; blocks.append(b)   # NaN skipped by absmax -> (0, 0)
    b = np.linspace(-1, 1, 64).astype(np.float32); b[3] = np.inf; blocks.append(b)  # absmax inf
    b = np.linspace(-1, 1, 64).astype(np.float32); b[3] = -np.inf; b[4] = np.inf; b[7] = np.nan; blocks.append(b)
    blocks.append((np.linspace(-1, 1, 64) * 1e30).astype(np.float32))   # absmax > 2^90: IEEE divide path
    blocks.append((np.linspace(-1, 1, 64) * 1e-30).astype(np.float32))  # absmax < 2^-90
    blocks.append((np.linspace(-1, 1, 64) * 1e-39).astype(np.float32))  # subnormal values
    b = np.full(64, -0.0, np.float32); b[0] = 1e-3; blocks.append(b)    # -0 against a tiny absmax
    blocks.append(np.float32([(-1) ** i * 2.0 ** (-(i % 40)) for i in range(64)]))
    u16 = bf16_bits(np.concatenate(blocks))
    u16 = np.concatenate([u16, bf16_bits(np.random.default_rng(0).normal(0, 1, 512 * 3))])
    want = oracle.encode_bf16(u16, 64)
    assert_same(gpu_encode(u16, 64), want, "special blocks")
    h = G.unpack_nibbles(want[0], u16.size)
    p = G.unpack_nibbles(want[1], u16.size)
    assert (h[64 + 5], p[64 + 5]) == (7, 8) and (h[128 + 9], p[128 + 9]) == (0, 0)


def test_f32_input_path(oracle):
    rng = np.random.default_rng(9)
    f, par = G.CELLS_FLAT, G.PARENT_F32
    mids = ((f[1:] + f[:-1]) / 2).astype(np.float32)
    edge = np.concatenate([f, mids, np.nextafter(mids, 2), np.nextafter(mids, -2), par,
                           ((par[1:] + par[:-1]) / 2).astype(np.float32)])
    for w in (rng.normal(0, 0.02, 100001).astype(np.float32),
              np.concatenate([np.float32([1.0]), edge]).astype(np.float32),
              np.float32([np.nan, 0.5, -np.inf, 3.0, 0.0, -0.0, 1e-40])):
        for bs in (64, 23):
            got = H.encode_f32(dev(w), bs)
            assert_same([host(t) for t in got], oracle.encode_f32(w, bs), f"f32 n={w.size} bs={bs}")


def test_host_pointer_abi(oracle):
    """glint_encode_bf16_host / glint_encode_f32_host (allocate, copy, encode, copy back)."""
    rng = np.random.default_rng(3)
    for n in (2, 513, 70001):
        u16 = bf16_bits(rng.normal(0, 0.02, n))
        hole, plug, am = H.encode_bf16_host(u16.tobytes(), n, 64)
        want = oracle.encode_bf16(u16, 64)
        assert hole == want[0].tobytes() and plug == want[1].tobytes() and am == want[2].tobytes()
    w = rng.normal(0, 0.02, 999).astype(np.float32)
    import ctypes
    lib = H.encode_lib()
    hole = np.zeros(500, np.uint8)
    plug = np.zeros(500, np.uint8)
    am = np.zeros(16, np.float32)
    rc = lib.glint_encode_f32_host(w.ctypes.data, 999, 64, hole.ctypes.data, plug.ctypes.data, am.ctypes.data)
    assert rc == 0
    assert_same((hole, plug, am), oracle.encode_f32(w, 64), "f32 host")
