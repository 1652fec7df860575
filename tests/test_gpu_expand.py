"""GPU expand parity: f32 and BF16 unpin outputs identical to the CPU oracle (the f32
values are one multiply, so exactness is the bar; the reference's own --cuda gate is
max_abs < 1e-5)."""
import numpy as np
import pytest

from glint_amd import glint_hip as H
from oracle import glint_oracle as G
from tests.gpu_util import dev, host, first_diff, bf16_bits

pytestmark = pytest.mark.gpu


def planes(rng, n, bs, lo=0.01, hi=2.0):
    hole = rng.integers(0, 256, (n + 1) // 2, dtype=np.uint8)
    plug = rng.integers(0, 256, (n + 1) // 2, dtype=np.uint8)
    am = rng.uniform(lo, hi, (n + bs - 1) // bs).astype(np.float32)
    return hole, plug, am


@pytest.mark.parametrize("bs", [1, 23, 32, 64, 96, 4096])
@pytest.mark.parametrize("pad", [0, 1])
def test_expand_matches_oracle(oracle, bs, pad):
    rng = np.random.default_rng(bs + 100 * pad)
    for n in (1, 31, 32, 33, 2047, 2048, 65536 + 17, 300000):
        hole, plug, am = planes(rng, n, bs)
        dh, dp, da = dev(hole, pad), dev(plug, pad), dev(am)
        f = host(H.expand_f32(dh, dp, da, n, bs))
        b = host(H.expand_bf16(dh, dp, da, n, bs), np.uint16)
        wf = oracle.expand_f32(hole, plug, am, n, bs)
        wb = oracle.expand_bf16(hole, plug, am, n, bs)
        assert f.tobytes() == wf.tobytes(), f"f32 n={n} bs={bs} pad={pad}: {first_diff(f.view(np.uint32), wf.view(np.uint32))}"
        assert b.tobytes() == wb.tobytes(), f"bf16 n={n} bs={bs} pad={pad}: {first_diff(b, wb)}"


def test_expand_special_absmax(oracle):
    rng = np.random.default_rng(5)
    n, bs = 64 * 16, 64
    hole, plug, _ = planes(rng, n, bs)
    am = np.float32([0.0, -0.0, np.inf, 1e-40, 3.4e38, 1.0, 2.0 ** -126, 1e-45,
                     65504.0, 1e30, 7.0, 0.5, 1.0, 1.0, 1.0, 1.0])
    dh, dp, da = dev(hole), dev(plug), dev(am)
    f = host(H.expand_f32(dh, dp, da, n, bs))
    b = host(H.expand_bf16(dh, dp, da, n, bs), np.uint16)
    assert f.tobytes() == oracle.expand_f32(hole, plug, am, n, bs).tobytes()
    assert b.tobytes() == oracle.expand_bf16(hole, plug, am, n, bs).tobytes()
    # zero block -> -0.0 for the (7, 8) code; BF16 0x8000
    z = np.full(32, 0x87, np.uint8)  # hole 7 / 8 nibbles
    hz, pz = np.full(32, 0x77, np.uint8), np.full(32, 0x88, np.uint8)
    bz = host(H.expand_bf16(dev(hz), dev(pz), dev(np.float32([0.0])), 64, 64), np.uint16)
    assert set(bz.tolist()) == {0x8000}
    del z


def test_expand_nan_absmax_produces_nan():
    """NaN absmax cannot come out of encode (NaN is skipped); the expand still yields NaN
    (f32) and a BF16 NaN pattern for every element of such a block."""
    hole = np.full(32, 0x5A, np.uint8)
    plug = np.full(32, 0xA5, np.uint8)
    am = np.float32([np.nan])
    f = host(H.expand_f32(dev(hole), dev(plug), dev(am), 64, 64))
    b = host(H.expand_bf16(dev(hole), dev(plug), dev(am), 64, 64), np.uint16)
    assert np.isnan(f).all()
    assert ((b & 0x7F80) == 0x7F80).all() and ((b & 0x7F) != 0).all()


def test_host_pointer_expand(oracle):
    from glint_amd import glint_cuda
    rng = np.random.default_rng(8)
    for n, bs in ((7, 64), (4096 + 5, 64), (1000, 23)):
        hole, plug, am = planes(rng, n, bs)
        got = glint_cuda.expand_cuda(hole.tobytes(), plug.tobytes(), am.tobytes(), n, bs)
        assert got == oracle.expand_f32(hole, plug, am, n, bs).tobytes()
        gotb = H.expand_bf16_host(hole.tobytes(), plug.tobytes(), am.tobytes(), n, bs)
        assert gotb == oracle.expand_bf16(hole, plug, am, n, bs).tobytes()


def test_encode_expand_round_trip_large(oracle):
    """Size-independent properties at a full model-tensor size (14336 x 4096): every
    reconstructed weight is within the codec's worst-case error (0.0174 * absmax, the
    largest |v - CELLS[code(v)]| over v in [-1, 1]) plus BF16 rounding of its own block,
    and a seeded sample of blocks is byte-identical to the oracle's encode and expand."""
    torch = pytest.importorskip("torch")
    n = 14336 * 4096
    g = torch.Generator(device="cuda").manual_seed(2002)
    w = (torch.randn(n, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    hole, plug, am = H.encode_bf16(w, 64)
    rec = H.expand_bf16(hole, plug, am, n, 64)
    amx = am.repeat_interleave(64)
    err = (rec.float() - w.float()).abs()
    bound = 0.0175 * amx + rec.float().abs() * 2.0 ** -8
    assert bool((err <= bound).all())
    rng = np.random.default_rng(0)
    blocks = np.sort(rng.choice(n // 64, 512, replace=False))
    hh, pp, aa, rr = host(hole), host(plug), host(am), host(rec, np.uint16)
    ww = host(w, np.uint16)
    for b in blocks:
        sl = slice(b * 64, b * 64 + 64)
        wh, wp, wa = oracle.encode_bf16(ww[sl], 64)
        assert wh.tobytes() == hh[b * 32:b * 32 + 32].tobytes() and wp.tobytes() == pp[b * 32:b * 32 + 32].tobytes()
        assert wa[0] == aa[b]
        assert oracle.expand_bf16(wh, wp, wa, 64, 64).tobytes() == rr[sl].tobytes()
