"""Pins the CPU oracle before anything is checked against it.

Each test checks the oracle against something other than its own formula: published
hashes, known answers derived by hand from the table, the reference's own seeded
test data and edge corpus, brute force, or an independent restatement.
"""
import hashlib
import math
import random
import struct
import subprocess
from pathlib import Path

import numpy as np
import pytest

from oracle import glint_oracle as G
from glint_amd import codebook

ROOT = Path(__file__).resolve().parent.parent
REF_BUILT = ROOT / "oracle" / "_ref"


def _gauss(n, seed, scale=0.02):
    """random.Random(seed).gauss(0, scale): the reference tests' generator
    (test_glint_tools.py:28-30), reproducible from the standard library."""
    rng = random.Random(seed)
    return [rng.gauss(0.0, scale) for _ in range(n)]


# ------------------------------------------------------------------- tables
def test_cells_hash_matches_published_codebook():
    assert codebook.cells_sha256() == codebook.CELLS_SHA256
    assert hashlib.sha256(G.CELLS_F32.astype("<f4").tobytes()).hexdigest() == codebook.CELLS_SHA256


def test_committed_header_is_generated_from_definition():
    assert (ROOT / "include" / "glint_cells.h").read_text() == codebook.header_text()


def test_parent_table_is_nf4_in_f32():
    assert [float(x) for x in G.PARENT_F32] == [codebook.f32(x) for x in codebook.PARENT]


def test_table_structure():
    flat = G.CELLS_FLAT
    assert np.all(np.diff(flat) > 0), "flattened table must be strictly ascending"
    edges = codebook.voronoi_edges()
    for k in range(16):  # each row lies inside its parent's Voronoi cell
        assert edges[k] <= G.CELLS_F32[k, 0] and G.CELLS_F32[k, 15] <= edges[k + 1]


@pytest.mark.skipif(not (REF_BUILT / "ref_cells.bin").is_file(), reason="oracle/_ref not built (no /root/reference)")
def test_cells_equal_reference_header_bytes():
    assert (REF_BUILT / "ref_cells.bin").read_bytes() == G.CELLS_F32.astype("<f4").tobytes()


@pytest.mark.skipif(not (REF_BUILT / "test_cells").is_file(), reason="oracle/_ref not built")
def test_reference_host_tests_pass():
    for exe, marker in (("test_cells", "TEST_CELLS_OK"), ("test_htile_k_bounds", "PASS 5 K-tail")):
        out = subprocess.run([str(REF_BUILT / exe)], capture_output=True, text=True, timeout=120)
        assert out.returncode == 0 and marker in out.stdout, out.stdout + out.stderr


# ------------------------------------------------------------------- encode KATs
def test_kat_gpu_ok_vector(oracle):
    """glint_cuda.py:79-85 encodes b"\\x80\\x3f\\x00\\x00" = [1.0, 0.0]: 1.0 is parent 15 /
    child 15 (CELLS[15][15]=0.992 is the largest); 0.0 is parent 7 / child 8
    (|0 - (-1.85e-4)| < |0 - 5.13e-3|)."""
    u16 = np.frombuffer(b"\x80\x3f\x00\x00", dtype="<u2")
    for hole, plug, am in (oracle.encode_bf16(u16, 64), G.encode_bf16(u16, 64)):
        assert bytes(hole) == b"\x7f" and bytes(plug) == b"\x8f"
        assert am.tolist() == [1.0]


def test_kat_zero_block_and_negative_zero(oracle):
    u16 = np.zeros(64, np.uint16)
    hole, plug, am = oracle.encode_bf16(u16, 64)
    assert set(hole.tolist()) == {0x77} and set(plug.tolist()) == {0x88} and am.tolist() == [0.0]
    out = oracle.expand_bf16(hole, plug, am, 64, 64)
    assert set(out.tolist()) == {0x8000}, "CELLS[7][8] < 0 times 0 is -0.0"


def test_kat_nan_inf_handling(oracle):
    w = np.full(128, 0.5, np.float32)
    w[3] = np.nan          # block 0: NaN skipped by absmax, encodes as (0, 0)
    w[64:128] = 0.0
    w[70] = np.nan         # block 1: absmax 0 -> v = 0 for every element, NaN too
    hole, plug, am = oracle.encode_f32(w, 64)
    assert am.tolist() == [0.5, 0.0]
    h = G.unpack_nibbles(hole, 128)
    p = G.unpack_nibbles(plug, 128)
    assert (h[3], p[3]) == (0, 0)
    assert (h[70], p[70]) == (7, 8)
    assert (h[0], p[0]) == (15, 15)
    w2 = np.array([np.inf, 1.0, -2.0, 0.0], np.float32)   # absmax inf: inf/inf = NaN -> (0,0), finite/inf = 0
    hole2, plug2, am2 = oracle.encode_f32(w2, 64)
    assert math.isinf(am2[0])
    assert G.unpack_nibbles(hole2, 4).tolist() == [0, 7, 7, 7] and G.unpack_nibbles(plug2, 4).tolist() == [0, 8, 8, 8]
    for impl in (oracle.encode_f32, G.encode_f32):
        a = impl(w, 64)
        assert bytes(a[0]) == bytes(hole) and bytes(a[1]) == bytes(plug)


def test_kat_odd_n_pad_nibble(oracle):
    u16 = G.f32_to_bf16_bits(np.float32([0.1, -0.3, 0.7]))
    hole, plug, _ = oracle.encode_bf16(u16, 64)
    assert hole.size == 2 and (hole[-1] >> 4) == 0 and (plug[-1] >> 4) == 0


# --------------------------------------------------------- encode vs reference data
def test_numpy_nearest_equals_linear_scan_on_reference_edge_corpus(oracle):
    """The reference's own corpus (test_glint_tools.py:186-213): table points,
    midpoints, their f32 neighbours, +-0, +-1 and 50k uniform values (default_rng(0)).
    The C oracle is a literal linear scan; the numpy path is searchsorted."""
    f, par = G.CELLS_FLAT, G.PARENT_F32
    mids = ((f[1:] + f[:-1]) / 2).astype(np.float32)
    pmid = ((par[1:] + par[:-1]) / 2).astype(np.float32)
    up = lambda a: np.nextafter(a, np.float32(2))
    dn = lambda a: np.nextafter(a, np.float32(-2))
    rng = np.random.default_rng(0)
    v = np.concatenate([f, mids, pmid, par, up(mids), dn(mids), up(pmid), dn(pmid), up(f), dn(f),
                        np.float32([1, -1, 0, -0.0]), rng.uniform(-1, 1, 50000).astype(np.float32)]).astype(np.float32)
    # absmax 1.0 in every block makes v = w exactly; put a 1.0 at each block start.
    bs = 64
    n = v.size
    blocks = (n + bs - 2) // (bs - 1)
    w = np.zeros(blocks * bs, np.float32)
    idx = np.arange(blocks * bs)
    data_pos = idx[(idx % bs) != 0][:n]
    w[idx % bs == 0] = 1.0
    w[data_pos] = v
    h1, p1, _ = oracle.encode_f32(w, bs)
    h2, p2, _ = G.encode_f32(w, bs)
    assert bytes(h1) == bytes(h2) and bytes(p1) == bytes(p2)
    hv = G.unpack_nibbles(h1, w.size)[data_pos]
    pv = G.unpack_nibbles(p1, w.size)[data_pos]
    # direct scan in numpy (reference test's scan(), restated) on the same values
    def scan(vals, tab):
        best = np.zeros(vals.shape, np.uint8)
        bd = np.abs(vals - tab[:, 0])
        for k in range(1, 16):
            d = np.abs(vals - tab[:, k])
            t = d < bd
            best[t] = k
            bd = np.where(t, d, bd)
        return best
    h_ref = scan(v, np.broadcast_to(par, (v.size, 16)))
    p_ref = scan(v, G.CELLS_F32[h_ref])
    assert (hv == h_ref).all() and (pv == p_ref).all()


def test_f32_encode_equals_f64_codec_on_reference_seeded_data(oracle):
    """test_glint_tools.py:108-119: numpy f32 encode == pure-Python encode on
    _gauss(64*41+7, 5) with a zero block at [128:192]."""
    w = _gauss(64 * 41 + 7, 5)
    w[128:192] = [0.0] * 64
    wf = np.array(w, dtype=np.float32)
    hole, plug, am = oracle.encode_f32(wf, 64)
    hi, pi, ai = G.codec_encode_f64([G.f32(x) for x in w], 64)
    assert bytes(hole) == G.pack_indices(hi)
    assert bytes(plug) == G.pack_indices(pi)
    assert am.tolist() == [G.f32(x) for x in ai]
    h2, p2, a2 = G.encode_f32(wf, 64)
    assert bytes(h2) == bytes(hole) and bytes(p2) == bytes(plug) and a2.tobytes() == am.tobytes()


def test_toy_shards_encode_agree(oracle):
    """The reference's toy shards (test_glint_tools.py:61-76): 16x64, odd 8x63
    (blocks straddle rows), 4x128 with an all-zero block."""
    a = _gauss(16 * 64, 1)
    b = _gauss(8 * 63, 2)
    c = _gauss(4 * 128, 3)
    c[:64] = [0.0] * 64
    for vals in (a, b, c):
        u16 = G.f32_to_bf16_bits(np.array(vals, np.float32))
        r1 = oracle.encode_bf16(u16, 64)
        r2 = G.encode_bf16(u16, 64)
        for x, y in zip(r1, r2):
            assert x.tobytes() == y.tobytes()
        hi, pi, _ = G.codec_encode_f64([float(x) for x in G.bf16_bits_to_f32(u16)], 64)
        assert bytes(r1[0]) == G.pack_indices(hi) and bytes(r1[1]) == G.pack_indices(pi)


def test_generic_blocksizes_agree(oracle):
    rng = np.random.default_rng(7)
    for bs in (1, 2, 23, 63, 64, 100, 256, 1000):
        w = (rng.standard_normal(3001) * 0.02).astype(np.float32)
        r1 = oracle.encode_f32(w, bs)
        r2 = G.encode_f32(w, bs)
        for x, y in zip(r1, r2):
            assert x.tobytes() == y.tobytes(), bs


# ------------------------------------------------------------------- expand / RNE
def test_rne_known_answers(oracle):
    """test_glint_tools.py:31-37: 1+ulp/2 -> 1, 1+1.5ulp -> 1+2ulp, 1+0.75ulp -> 1+ulp,
    -(1+ulp/2) -> -1; NaN stays NaN."""
    ulp = 2.0 ** -7
    vals = np.float32([1 + ulp / 2, 1 + 1.5 * ulp, 1 + 0.75 * ulp, -(1 + ulp / 2), np.nan])
    got = G.bf16_bits_to_f32(G.f32_to_bf16_bits(vals))
    assert got[:4].tolist() == [1.0, 1 + 2 * ulp, 1 + ulp, -1.0]
    assert math.isnan(got[4])
    out = np.empty(5, np.uint16)
    oracle.lib.oracle_f32_to_bf16(G._ptr(vals), 5, G._ptr(out))
    assert out.tolist() == G.f32_to_bf16_bits(vals).tolist()
    # overflow rounds to inf; inf stays inf
    big = np.float32([np.finfo(np.float32).max, np.inf, -np.inf])
    assert G.f32_to_bf16_bits(big).tolist() == [0x7F80, 0x7F80, 0xFF80]


def test_expand_is_table_times_absmax(oracle):
    rng = np.random.default_rng(3)
    n, bs = 1001, 23
    hole = rng.integers(0, 256, (n + 1) // 2, dtype=np.uint8)
    plug = rng.integers(0, 256, (n + 1) // 2, dtype=np.uint8)
    am = rng.uniform(0.5, 2.0, (n + bs - 1) // bs).astype(np.float32)
    got = oracle.expand_f32(hole, plug, am, n, bs)
    for i in (0, 1, 2, 22, 23, 500, 1000):
        hb, pb = hole[i // 2], plug[i // 2]
        h = (hb >> 4) if i & 1 else (hb & 15)
        p = (pb >> 4) if i & 1 else (pb & 15)
        assert got[i] == np.float32(G.CELLS_F32[h, p] * am[i // bs])
    assert got.tobytes() == G.expand(hole, plug, am, n, bs).tobytes()
    assert oracle.expand_bf16(hole, plug, am, n, bs).tobytes() == G.expand_bf16(hole, plug, am, n, bs).tobytes()


# ------------------------------------------------------------------- H-TILE
def test_htile_oracle_against_f64_brute_force(oracle):
    rng = np.random.default_rng(11)
    for (M, N, K, bs) in ((1, 1, 1, 1), (3, 5, 65, 23), (4, 17, 199, 64), (2, 8, 256, 64)):
        hole = rng.integers(0, 256, (N * K + 1) // 2, dtype=np.uint8)
        plug = rng.integers(0, 256, (N * K + 1) // 2, dtype=np.uint8)
        am = rng.uniform(0.25, 1.0, (N * K + bs - 1) // bs).astype(np.float32)
        x = G.f32_to_bf16_bits(rng.standard_normal(M * K).astype(np.float32))
        y32 = oracle.htile_f32(hole, plug, am, x, M, N, K, bs)
        y64, asum = oracle.htile_f64(hole, plug, am, x, M, N, K, bs)
        ynp = G.htile_ref_f64(hole, plug, am, x, M, N, K, bs)
        assert np.allclose(y64, ynp, rtol=1e-12, atol=1e-12)
        bound = (K + 2) * 2.0 ** -23 * asum
        assert np.all(np.abs(y32 - y64) <= bound)


def test_htile_single_term_known_answer(oracle):
    # K=1: y = CELLS[h][p] * absmax * x exactly; hole nibble 15, plug 15 -> 0.992...
    hole = np.array([0x0F], np.uint8)
    plug = np.array([0x0F], np.uint8)
    am = np.float32([2.0])
    x = G.f32_to_bf16_bits(np.float32([0.5]))
    y = oracle.htile_f32(hole, plug, am, x, 1, 1, 1, 64)
    assert y[0, 0] == np.float32(G.CELLS_F32[15, 15])


# ------------------------------------------------------------------- INT8
def test_quant_act_known_answers(oracle):
    # a block with amax 127 -> s = 1 exactly; rint ties to even on 2.5 and 3.5
    vals = np.zeros(64, np.float32)
    vals[0], vals[1], vals[2], vals[3] = 127.0, 2.5, 3.5, -2.5
    x = G.f32_to_bf16_bits(vals)
    xq, sx = oracle.quant_act(x, 1, 64)
    assert sx.tolist() == [1.0]
    assert xq[:4].tolist() == [127, 2, 4, -2]
    xq0, sx0 = oracle.quant_act(np.zeros(64, np.uint16), 1, 64)
    assert sx0.tolist() == [1.0] and not xq0.any()


def test_quant_act_nan_converts_like_the_cuda_cast(oracle):
    """A NaN activation is skipped by the block max and quantizes to 0: the reference's
    (int)rintf(NaN / s) is a saturating cvt.rzi.s32.f32, which maps NaN to 0."""
    vals = np.linspace(-2, 2, 64).astype(np.float32)
    vals[7] = np.nan
    xq, sx = oracle.quant_act(G.f32_to_bf16_bits(vals), 1, 64)
    assert sx.tolist() == [np.float32(2.0) / np.float32(127.0)]
    assert xq[7] == 0 and xq[0] == -127 and xq[63] == 127


def test_int8_integer_parts_are_exact(oracle):
    rng = np.random.default_rng(5)
    M, N, K = 7, 9, 192
    A = rng.integers(-127, 128, (M, K), dtype=np.int8)
    B = rng.integers(-127, 128, (N, K), dtype=np.int8)
    C = oracle.int8_gemm_i32(A, B, M, N, K)
    assert np.array_equal(C, A.astype(np.int64) @ B.astype(np.int64).T)
    # emulation with unit scales is the exact integer sum converted per slice
    sx = np.ones(M * (K // 64), np.float32)
    sw = np.ones(N * (K // 64), np.float32)
    y = oracle.int8_mma_emu(A.reshape(-1), sx, B.reshape(-1), sw, M, N, K)
    assert np.array_equal(y.astype(np.int64), C.astype(np.int64))
    sa = rng.uniform(1e-3, 2e-2, M).astype(np.float32)
    sb = rng.uniform(1e-3, 2e-2, N).astype(np.float32)
    out = oracle.int8_scale_bf16(C, sa, sb, M, N)
    ref = G.f32_to_bf16_bits((C.astype(np.float32) * sa[:, None]) * sb[None, :])
    assert np.array_equal(out, ref)


def _round_f32(q):
    """The f32 nearest to the rational q, ties to even (exact, no double rounding)."""
    from fractions import Fraction
    f = np.float32(float(q))
    best = None
    for cand in (np.nextafter(f, np.float32(-np.inf)), f, np.nextafter(f, np.float32(np.inf))):
        if not np.isfinite(cand):
            continue
        d = abs(Fraction(float(cand)) - q)
        if best is None or d < best[0] or (d == best[0] and int(cand.view(np.uint32)) % 2 == 0):
            best = (d, cand)
    return best[1]


def test_fmaf_is_one_rounding(oracle):
    """The oracle's fused multiply-add is RN(a * b + c) computed once: checked against exact
    rational arithmetic on random triples, on cancelling triples (c = -RN(a * b), where a
    separate multiply and add gives exactly 0 and the fused form keeps the product's
    rounding error) and on the INT8 epilogue's own operand ranges."""
    from fractions import Fraction
    rng = np.random.default_rng(11)
    a = rng.standard_normal(400).astype(np.float32) * np.float32(3.0)
    b = rng.standard_normal(400).astype(np.float32)
    c = rng.standard_normal(400).astype(np.float32)
    c[:100] = -(a[:100] * b[:100])  # cancellation
    a[300:] = (rng.integers(-260000, 260000, 100) * rng.uniform(1e-5, 1e-3, 100)).astype(np.float32)
    b[300:] = rng.uniform(1e-4, 2e-2, 100).astype(np.float32)
    c[300:] = rng.standard_normal(100).astype(np.float32) * np.float32(100.0)
    got = oracle.fmaf(a, b, c)
    for i in range(a.size):
        want = _round_f32(Fraction(float(a[i])) * Fraction(float(b[i])) + Fraction(float(c[i])))
        assert got[i] == want, (i, a[i], b[i], c[i], got[i], want)
    assert (got[:100] != 0).sum() > 50  # the separate form would give 0 for all of them


def test_int8_emulation_within_the_reference_gate(oracle):
    """The kernel-arithmetic emulation (fused last step, as nvcc's default contraction
    compiles the reference kernel) against the reference test's host emulation (separate
    multiply and add): within that test's pre-registered 1e-5 relative gate
    (tests/test_int8_mma_gemm.cu:207) on its own kind of data (bf16 activations quantized by
    the rule, N(0, 0.02) weights quantized per 64-block), and different in some bits, so the
    two emulations are not the same function."""
    rng = np.random.default_rng(12)
    m, n, k = 9, 70, 1024
    x = rng.standard_normal(m * k).astype(np.float32)
    xq, sx = oracle.quant_act(G.f32_to_bf16_bits(x), m, k)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    wb = w.reshape(n, k // 64, 64)
    sw = (np.abs(wb).max(axis=2) / np.float32(127.0)).astype(np.float32)
    wq = np.clip(np.rint(wb / sw[:, :, None]), -127, 127).astype(np.int8).reshape(-1)
    fused = oracle.int8_mma_emu(xq, sx, wq, sw.reshape(-1), m, n, k)
    sep = oracle.int8_mma_emu_sep(xq, sx, wq, sw.reshape(-1), m, n, k)
    rel = float(np.linalg.norm((fused - sep).astype(np.float64)) / np.linalg.norm(sep.astype(np.float64)))
    assert rel <= 1e-5, rel
    assert (fused.view(np.uint32) != sep.view(np.uint32)).any()


def test_int8_scale_bf16_special_cases(oracle):
    """The bf16 epilogue RNE(f32(acc) * sa * sb) on inputs whose answer is fixed without
    the formula: unit scales on |acc| <= 256 give the integer itself (exact in bf16);
    power-of-two scales shift the exponent only; 257 rounds to even (256), 259 to 260;
    a row scale of 0 gives +0 / -0 by the sign of acc."""
    M, N = 4, 6
    C = np.array([[0, 1, -1, 255, -256, 256], [257, 259, -257, 3, 100, -7],
                  [1, 2, 3, 4, 5, 6], [-1, -2, 9, 0, 11, 13]], np.int32)
    ones_m, ones_n = np.ones(M, np.float32), np.ones(N, np.float32)
    got = G.bf16_bits_to_f32(oracle.int8_scale_bf16(C, ones_m, ones_n, M, N))
    want = C.astype(np.float64)
    want[1, 0], want[1, 1], want[1, 2] = 256.0, 260.0, -256.0
    assert np.array_equal(got.astype(np.float64), want)
    sa = np.array([0.5, 0.25, 2.0 ** -10, 4.0], np.float32)
    sb = np.array([1.0, 2.0, 0.125, 1.0, 2.0 ** -7, 8.0], np.float32)
    got = G.bf16_bits_to_f32(oracle.int8_scale_bf16(C, sa, sb, M, N)).astype(np.float64)
    scaled = np.where(np.abs(want) <= 256, C.astype(np.float64), want) * sa[:, None].astype(np.float64) * sb[None, :]
    small = np.abs(C) <= 256
    assert np.array_equal(got[small], scaled[small])
    zero = oracle.int8_scale_bf16(C, np.zeros(M, np.float32), ones_n, M, N)
    assert np.array_equal(zero, np.where(C < 0, 0x8000, 0).astype(np.uint16))


def test_unpack_res4_known_answers(oracle):
    """p7_plug_res4_v1 (tools/plug_encode.c:3-6): element 2i in the low nibble, biased +8."""
    got = oracle.unpack_res4(np.array([0x80, 0x0F, 0x88, 0x79, 0xF1], np.uint8), 10)
    assert got.tolist() == [-8, 0, 7, -8, 0, 0, 1, -1, -7, 7]
    assert oracle.unpack_res4(np.array([0x3C], np.uint8), 1).tolist() == [4]  # odd n: high nibble unused


def _small_int8_case(rng, m, n, k, lo=-3, hi=4):
    nkb = k // 64
    xq = rng.integers(lo, hi, m * k).astype(np.int8)
    wq = rng.integers(lo, hi, n * k).astype(np.int8)
    pq = rng.integers(-7, 8, n * k).astype(np.int8)
    sx = (2.0 ** rng.integers(-2, 3, m * nkb)).astype(np.float32)
    sw = (2.0 ** rng.integers(-2, 3, n * nkb)).astype(np.float32)
    sp = (2.0 ** rng.integers(-2, 3, n * nkb)).astype(np.float32)
    return xq, sx, wq, sw, pq, sp


def _exact_formula(xq, sx, wq, sw, m, n, k):
    """sum_kb ic_kb * sx * sw in float64 (exact for the small-integer, power-of-two cases)."""
    nkb = k // 64
    X = xq.astype(np.int64).reshape(m, nkb, 64)
    W = wq.astype(np.int64).reshape(n, nkb, 64)
    ic = np.einsum("mbt,nbt->mnb", X, W).astype(np.float64)
    return (ic * sx.reshape(m, 1, nkb) * sw.reshape(1, n, nkb)).sum(axis=2)


def test_plug_forms_exact_on_power_of_two_scales(oracle):
    """With small integers and power-of-two scales every f32 step is exact, so the fused
    late plug, the two-pass plug (base pass + plug pass added) and the integer formula
    agree bit for bit; a transposed scale or a plug on the wrong operand would not."""
    rng = np.random.default_rng(11)
    m, n, k = 5, 7, 256
    xq, sx, wq, sw, pq, sp = _small_int8_case(rng, m, n, k)
    want = _exact_formula(xq, sx, wq, sw, m, n, k) + _exact_formula(xq, sx, pq, sp, m, n, k)
    fused = oracle.int8_mma_plug_fused(xq, sx, wq, sw, pq, sp, m, n, k)
    two = oracle.int8_mma_emu(xq, sx, wq, sw, m, n, k) + oracle.int8_mma_emu(xq, sx, pq, sp, m, n, k)
    assert np.array_equal(fused.astype(np.float64), want)
    assert np.array_equal(two.astype(np.float64), want)


def test_zero_plug_equals_base(oracle):
    """Nibbles 0x88 decode to 0: both plug forms reproduce the base bit for bit."""
    rng = np.random.default_rng(12)
    m, n, k = 6, 9, 192
    xq = rng.integers(-127, 128, m * k).astype(np.int8)
    wq = rng.integers(-127, 128, n * k).astype(np.int8)
    sx = rng.uniform(1e-3, 2e-2, m * k // 64).astype(np.float32)
    sw = rng.uniform(1e-3, 2e-2, n * k // 64).astype(np.float32)
    sp = rng.uniform(1e-3, 2e-2, n * k // 64).astype(np.float32)
    pq = oracle.unpack_res4(np.full(n * k // 2, 0x88, np.uint8), n * k)
    base = oracle.int8_mma_emu(xq, sx, wq, sw, m, n, k)
    assert np.array_equal(oracle.int8_mma_plug_fused(xq, sx, wq, sw, pq, sp, m, n, k), base)
    assert np.array_equal(base + oracle.int8_mma_emu(xq, sx, pq, sp, m, n, k), base)


def test_quant_act_resid_pins(oracle):
    """The residual r = x - xq sx re-quantized: (1) a block on the quantization grid has
    r = 0 exactly (rq = 0, sr = 1); (2) elsewhere |r - rq sr| <= sr / 2 (rounding), so the
    two-level reconstruction xq sx + rq sr is ~127x closer to x than xq sx alone; a sign
    flip of r or a scale from the wrong block breaks both."""
    grid = (np.arange(-127, 128, 4)[:64] * 2.0 ** -7).astype(np.float32)  # 64 values, amax 125 * 2^-7
    grid[0] = 127 * 2.0 ** -7
    rng = np.random.default_rng(13)
    m, k = 9, 320
    x = rng.normal(0, 1, m * k).astype(np.float32)
    x[:64] = grid
    u16 = G.f32_to_bf16_bits(x)
    xq, sx = oracle.quant_act(u16, m, k)
    rq, sr = oracle.quant_act_resid(u16, xq, sx, m, k)
    assert np.all(rq[:64] == 0) and sr[0] == 1.0
    xf = G.bf16_bits_to_f32(u16).astype(np.float64)
    blk = np.repeat(np.arange(m * k // 64), 64)
    r = xf - xq.astype(np.float64) * sx[blk]
    err2 = np.abs(r - rq.astype(np.float64) * sr[blk])
    # rounding of rint, plus the f32 evaluation of r (a rounded product, a rounded difference)
    f32_r = 2.0 ** -23 * np.maximum(np.abs(xf), np.abs(xq.astype(np.float64) * sx[blk]))
    assert np.all(err2 <= sr[blk] * (0.5 + 1e-6) + f32_r)
    e1, e2 = np.abs(r).max(), err2.max()
    assert e2 * 60 < e1, (e1, e2)


# ------------------------------------------------------------ W8A16 over an INT8 pin
def test_int8_pin_dequant_known_answers(oracle):
    """BF16 RNE of (float)q * s (test_int8_tile_gemm.cu:53-55), worked by hand:
    1 * (1 + 2^-8) is halfway between 1.0 and 1 + 2^-7 and ties to even (0x3F80);
    1 * (1 + 3 * 2^-8) is halfway between 0x3F81 and 0x3F82 and ties to even (0x3F82);
    3 * (1 + 2^-8) = 3.01171875 is 0.75 of a 2^-6 step above 3 (0x4041);
    127 * (1 + 2^-8) = 127.49609375 rounds to 127.5 (0x42FF); q = 0 gives +0."""
    s = np.array([1 + 2.0 ** -8] * 1, np.float32)
    q = np.array([1, 3, -1, 0, 127, -127], np.int8)
    got = oracle.int8_pin_dequant_bf16(q, s)
    assert got.tolist() == [0x3F80, 0x4041, 0xBF80, 0x0000, 0x42FF, 0xC2FF]
    got = oracle.int8_pin_dequant_bf16(np.array([1], np.int8), np.array([1 + 3 * 2.0 ** -8], np.float32))
    assert got.tolist() == [0x3F82]


def test_int8_pin_scale_index_is_flat(oracle):
    """k_in = 37: a row's 64-blocks start mid-row, w[i] uses scale[i // 64] over the flat
    index (int8_tile_gemm.h:10-12). A numpy restatement agrees; a row-local index does not."""
    n, k = 7, 37
    rng = np.random.default_rng(3)
    q = rng.integers(-127, 128, n * k, dtype=np.int8)
    s = (1e-3 + 2e-2 * rng.random((n * k + 63) // 64)).astype(np.float32)
    got = oracle.int8_pin_dequant_bf16(q, s)
    flat = G.f32_to_bf16_bits(q.astype(np.float32) * s[np.arange(n * k) // 64])
    assert np.array_equal(got, flat)
    rowlocal = G.f32_to_bf16_bits(q.astype(np.float32) * s[(np.arange(n * k) % k) // 64])
    assert not np.array_equal(got, rowlocal)


def test_int8_tile_f64_is_exact_on_dyadic_data(oracle):
    """Small integer x, q and power-of-two scales: every BF16 rounding is exact and the
    double sums are exact, so y must equal the integer GEMM scaled by the flat blocks'
    2^-e (numpy int64), and the |term| sums likewise. k_in = 100 crosses blocks mid-row;
    m != n catches a transposed operand."""
    m, n, k = 5, 9, 100
    rng = np.random.default_rng(11)
    xi = rng.integers(-4, 5, (m, k))
    q = rng.integers(-127, 128, n * k, dtype=np.int8)
    e = rng.integers(3, 12, (n * k + 63) // 64)
    s = np.ldexp(np.ones(e.size), -e).astype(np.float32)
    emax = int(e.max())
    wi = q.astype(np.int64) * (np.int64(1) << (emax - e[np.arange(n * k) // 64]))  # w * 2^emax, exact
    wi = wi.reshape(n, k)
    want = (xi @ wi.T).astype(np.float64) / 2.0 ** emax
    want_abs = (np.abs(xi) @ np.abs(wi).T).astype(np.float64) / 2.0 ** emax
    y, a = oracle.int8_tile_f64(G.f32_to_bf16_bits(xi.astype(np.float32)), q, s, m, n, k)
    assert np.array_equal(y, want) and np.array_equal(a, want_abs)


# ------------------------------------------------------------- K-major decode path
def _pin_planes(oracle, N, K, seed):
    rng = np.random.default_rng(seed)
    w = (rng.normal(0, 0.02, N * K)).astype(np.float32)
    w[: 64] = 0.0
    return oracle.encode_f32(w, 64)


def test_kmajor_pack_is_the_transpose(oracle):
    """hole_k[c N/2 + r/2] is element (r, c), even r low (p7_glint_select_decode.mojo:126-142);
    scales_k[(c/64) N + r] = absmax[r K/64 + c/64] (p7_select_device.mojo:196-206), checked
    against a numpy transpose of the unpacked planes."""
    N, K = 24, 192
    h, p, am = _pin_planes(oracle, N, K, 1)
    hk, pk, sk = oracle.kmajor_pack(h, p, am, N, K)
    for src, dst in ((h, hk), (p, pk)):
        nib = G.unpack_nibbles(src, N * K).reshape(N, K).T.reshape(-1)
        assert np.array_equal(G.pack_nibbles(nib), dst)
    assert np.array_equal(sk, am.reshape(N, K // 64).T.reshape(-1))


def test_fold_and_correction_on_one_hot_x(oracle):
    """x = e_c: the fold is PARENT[h(r, c)] * scale(r, c) exactly and the correction over
    [c] adds (CELLS[h][p] - PARENT[h]) * scale exactly (one nonzero term), for every slice
    and chunk count."""
    N, K = 16, 256
    h, p, am = _pin_planes(oracle, N, K, 2)
    hk, pk, sk = oracle.kmajor_pack(h, p, am, N, K)
    H = G.unpack_nibbles(h, N * K).reshape(N, K)
    Pn = G.unpack_nibbles(p, N * K).reshape(N, K)
    A = am.reshape(N, K // 64)
    for c in (0, 63, 64, 200, 255):
        x = np.zeros(K, np.uint16)
        x[c] = 0x3F80  # 1.0
        want_fold = (G.PARENT_F32[H[:, c]] * A[:, c // 64]).astype(np.float32)
        for ksg in (1, 2, 4):
            assert oracle.gemv_km_fold(hk, sk, x, N, K, ksg).tobytes() == want_fold.tobytes()
        d = (G.CELLS_F32[H[:, c], Pn[:, c]] - G.PARENT_F32[H[:, c]]).astype(np.float32)
        want_corr = (np.zeros(N, np.float32) + (d * A[:, c // 64]).astype(np.float32))  # y starts at +0
        for ks in (1, 3):
            got = oracle.apply_corr_km(hk, pk, sk, x, np.array([c], np.int32), N, K, np.zeros(N, np.float32), ks)
            assert got.tobytes() == want_corr.tobytes()


def test_fold_order_runs_and_parts(oracle):
    """Two channels of one 64-block in one part form a run: round(round(P1 + P2) * s). In
    different parts (K/ksg/8 channels each) they are two terms: round(round(P1 s) + round(P2 s)).
    Both are computed exactly in float64 (a sum or product of two f32 is exact there) and
    rounded once, so a different order shows."""
    N, K = 8, 1024
    h, p, am = _pin_planes(oracle, N, K, 6)
    hk, pk, sk = oracle.kmajor_pack(h, p, am, N, K)
    Hn = G.unpack_nibbles(h, N * K).reshape(N, K)
    A = am.reshape(N, K // 64).astype(np.float64)
    P = G.PARENT_F32.astype(np.float64)
    f32 = lambda v: np.asarray(v, np.float64).astype(np.float32)
    ksg = 2  # parts of 1024 / 2 / 8 = 64 channels: block b is part b within its slice
    for c1, c2, same_part in ((130, 140, True), (190, 200, False)):
        x = np.zeros(K, np.uint16)
        x[c1] = x[c2] = 0x3F80
        got = oracle.gemv_km_fold(hk, sk, x, N, K, ksg)
        b1, b2 = c1 // 64, c2 // 64
        if same_part:
            assert b1 == b2
            want = f32(f32(P[Hn[:, c1]] + P[Hn[:, c2]]).astype(np.float64) * A[:, b1])
        else:
            assert b1 != b2
            t1, t2 = f32(P[Hn[:, c1]] * A[:, b1]), f32(P[Hn[:, c2]] * A[:, b2])
            want = f32(t1.astype(np.float64) + t2.astype(np.float64))
        assert got.tobytes() == want.tobytes(), (c1, c2)


def test_select_matches_a_sort(oracle):
    """The kept set is every channel whose key (bf16 bits & 0x7FFF) is at least the nsel-th
    largest key, ties all kept, in ascending order; nsel = 0 keeps nothing and nsel >= K
    keeps everything (p7_select_device.mojo:1-151)."""
    rng = np.random.default_rng(3)
    K = 1000
    x = G.f32_to_bf16_bits(rng.normal(0, 1, K).astype(np.float32))
    x[100:140] = x[7]  # a block of ties
    x[500] |= 0x8000   # sign does not matter
    keys = x & 0x7FFF
    desc = np.sort(keys)[::-1]
    for nsel in (0, 1, 2, 30, 33, 500, K - 1, K, K + 5):
        got = oracle.select_topk(x, K, nsel)
        if nsel == 0:
            want = np.zeros(0, np.int32)
        elif nsel >= K:
            want = np.arange(K, dtype=np.int32)
        else:
            want = np.flatnonzero(keys >= desc[nsel - 1]).astype(np.int32)
        assert np.array_equal(got, want), nsel
        assert nsel == 0 or got.size >= min(nsel, K)


def _rank_brute(keys, n):
    """The largest 15-bit T with #{key >= T} >= n, by trying every T (0 when none)."""
    counts = np.cumsum(np.bincount(keys, minlength=32768)[::-1])[::-1]  # counts[T] = #{key >= T}
    ok = np.flatnonzero(counts >= n)
    return int(ok.max()) if ok.size else 0


def _key_of(t):
    """The rule's key of a positive float: biased exponent << 7 | 7 truncated mantissa bits."""
    m, e = np.frexp(np.float64(t))  # t = m 2^e, m in [0.5, 1)
    return int(((e - 1 + 127) << 7) | int((m * 2 - 1) * 128))


def test_select_rules_against_brute_force(oracle):
    """Threshold of the rank, price, relational and floor rules (p7_select_device.mojo:8-151)
    against a brute-force rank and a float64 mean: rank(n) for every n (n <= 0 -> 32767);
    tkey > 0 raises T to tkey; tkey < 0 raises it to key(tau mean|x|) (skipping draws whose
    tau mean|x| sits within 1e-4 of a 7-bit key boundary, where f32 order decides);
    nfloor lowers a price to the floor's rank but never below the cap; nsel == 0 keeps nothing."""
    rng = np.random.default_rng(11)
    for trial in range(40):
        K = int(rng.integers(1, 3000))
        x = G.f32_to_bf16_bits((rng.normal(0, 1, K) * 2.0 ** rng.integers(-8, 8, K)).astype(np.float32))
        if trial % 5 == 0:
            x[: K // 3] = x[0]  # ties
        keys = (x & 0x7FFF).astype(np.int64)
        for nsel in sorted({-1, 1, 2, K // 7, K // 2, K, K + 1}):
            cap = 32767 if nsel <= 0 else _rank_brute(keys, nsel)
            assert oracle.select_threshold(x, K, nsel) == cap, (trial, nsel)
            tk = int(rng.integers(1, 32768))
            assert oracle.select_threshold(x, K, nsel, tkey=tk) == max(cap, tk)
            tau = int(rng.integers(1, 4096))
            ex = keys >> 7
            mag = np.where(ex > 0, (128 + (keys & 127)) * 2.0 ** np.clip(ex - 134, -60, 40), 0.0)
            t = mag.sum() / K * tau / 1024
            rel = oracle.select_price_key(x, K, -tau)
            if t > 0:
                lo, hi = _key_of(t * (1 - 1e-4)), _key_of(t * (1 + 1e-4))
                if lo == hi:
                    assert rel == min(max(lo, 1), 32767), (trial, tau, t)
            assert oracle.select_threshold(x, K, nsel, tkey=-tau) == max(cap, rel)
            nf = int(rng.integers(1, K + 1))
            for tkey in (tk, -tau):
                price = max(cap, tkey if tkey > 0 else rel)
                want = max(cap, min(price, _rank_brute(keys, nf)))
                assert oracle.select_threshold(x, K, nsel, tkey=tkey, nfloor=nf) == want
            assert oracle.select_threshold(x, K, nsel, tkey=0, nfloor=nf) == cap  # no price: no floor
        assert oracle.select_ex(x, K, 0, tkey=-tau, nfloor=3).size == 0
        thr = oracle.select_threshold(x, K, K // 3 + 1, tkey=-tau, nfloor=5)
        assert np.array_equal(oracle.select_ex(x, K, K // 3 + 1, tkey=-tau, nfloor=5), np.flatnonzero(keys >= thr))


def test_select_relational_known_answers(oracle):
    """Equal magnitudes make mean|x| exact: |x| = 1 for all channels gives key(tau) for tau =
    -tkey / 1024; zero and subnormal keys count 0 but still divide by K; an inf key is read as
    (128) 2^40 by the clamp; nsel < 0 leaves T = 32767, so only 0x7FFF keys are kept."""
    one = np.full(1000, 0x3F80, np.uint16)
    one[::2] |= 0x8000
    assert oracle.select_price_key(one, 1000, -1024) == 0x3F80  # tau 1
    assert oracle.select_price_key(one, 1000, -512) == 0x3F00   # tau 1/2
    assert oracle.select_price_key(one, 1000, -1536) == 0x3FC0  # tau 3/2
    assert oracle.select_ex(one, 1000, 1, tkey=-1536).size == 0
    assert oracle.select_ex(one, 1000, 1, tkey=-1024).size == 1000
    half = one.copy()
    half[500:] = 0x0001  # subnormal: contributes 0
    assert oracle.select_price_key(half, 1000, -1024) == 0x3F00  # mean 1/2
    z = np.zeros(64, np.uint16)
    assert oracle.select_price_key(z, 64, -1024) == 1  # t = 0
    inf = np.zeros(1024, np.uint16)
    inf[0] = 0x7F80  # 2^47 / 1024 = 2^37
    assert oracle.select_price_key(inf, 1024, -1024) == (37 + 127) << 7
    nan = np.array([0x7FFF, 0x3F80, 0xFFFF, 0x0000], np.uint16)
    assert np.array_equal(oracle.select_ex(nan, 4, -1), [0, 2])
    assert oracle.select_ex(nan, 4, 0).size == 0


def test_fold_plus_full_correction_is_the_htile_sum(oracle):
    """PARENT + (CELLS - PARENT) = CELLS: fold plus the correction over every channel is the
    H-TILE GEMV up to f32 rounding, bounded by (K + 4) 2^-23 sum |terms| against float64."""
    N, K = 32, 512
    h, p, am = _pin_planes(oracle, N, K, 4)
    hk, pk, sk = oracle.kmajor_pack(h, p, am, N, K)
    x = G.f32_to_bf16_bits(np.random.default_rng(5).normal(0, 1, K).astype(np.float32))
    ref, absum = oracle.htile_f64(h, p, am, x, 1, N, K, 64)
    for ksg, ks in ((1, 1), (4, 8)):
        y = oracle.gemv_km_fold(hk, sk, x, N, K, ksg)
        y = oracle.apply_corr_km(hk, pk, sk, x, np.arange(K, dtype=np.int32), N, K, y, ks)
        assert np.all(np.abs(y.astype(np.float64) - ref[0]) <= (K + 4) * 2.0 ** -23 * absum[0] * 2)


# ------------------------------------------------------- the pins catch planted mistakes
def test_planted_mistakes_are_caught():
    """Mutations of the numpy oracle that a plausible bug would introduce must fail
    the known answers above: hi-then-lo nibbles, '<=' instead of '<', parent-only."""
    u16 = np.frombuffer(b"\x80\x3f\x00\x00", dtype="<u2")
    w = G.bf16_bits_to_f32(u16)
    h = G.nearest(w, G.PARENT_F32, 0)
    p = G.nearest(w, G.CELLS_FLAT, h.astype(np.int64) * 16)
    swapped = ((h[1] & 15) | (h[0] << 4), (p[1] & 15) | (p[0] << 4))
    assert swapped != (0x7F, 0x8F)
    # '<=' (last minimum) differs on the reference edge corpus's exact midpoints
    par = G.PARENT_F32
    mids = ((par[1:] + par[:-1]) / 2).astype(np.float32)
    first = G.nearest(mids, par, 0)
    last = np.array([max(range(16), key=lambda k: (-abs(float(np.float32(m - par[k]))), k)) for m in mids])
    assert (first != last).any()
