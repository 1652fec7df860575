"""bench.py on the CPU: the one-GPU refusal, and the counter summary's arithmetic on a
synthetic rocprofv3 database (phase assignment by kernel name and dispatch order, byte
scaling by the copy calibration, duration weighting)."""
import json
import sqlite3
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))
import bench  # noqa: E402


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr


def _db(path, rows, counters=True):
    """rows: (dispatch_id, kernel name, start ns, end ns, {counter: value})"""
    con = sqlite3.connect(path)
    con.execute("create table counters_collection (dispatch_id, kernel_name, counter_name, value, start, end)")
    con.execute("create table kernels (dispatch_id, name, start, end)")
    for did, name, t0, t1, ctrs in rows:
        con.execute("insert into kernels values (?,?,?,?)", (did, name, t0, t1))
        if counters:
            for c, v in ctrs.items():
                con.execute("insert into counters_collection values (?,?,?,?,?,?)", (did, name, c, v, t0, t1))
    con.commit()
    con.close()


def test_counter_summary_arithmetic(tmp_path):
    copy = 256 << 20
    # two copies, then three encodes: the first belongs to an earlier phase (skip 1)
    man = {"cu_num": 4, "simd_num": 16, "phases": [
        {"name": "hbm_copy_256mib", "kernel": "copyBuffer", "skip": 0, "count": 2, "algorithmic_bytes": 4 * copy,
         "ops": None, "elements": None, "note": ""},
        {"name": "enc", "kernel": "k_encode_bf16_b64", "skip": 1, "count": 2, "algorithmic_bytes": 3000.0,
         "ops": None, "elements": 1024, "note": ""},
        {"name": "mm", "kernel": "k_tile_big<2,GlintTileProducer", "skip": 0, "count": 1, "algorithmic_bytes": None,
         "ops": 5e12, "elements": None, "note": ""}]}
    mp = tmp_path / "manifest.json"
    mp.write_text(json.dumps(man))
    names = ["__amd_rocclr_copyBuffer"] * 2 + ["k_encode_bf16_b64(x)"] * 3 + ["void k_tile_big<2, GlintTileProducer, X>"]
    durs = [1000, 1000, 500, 1000, 3000, 2_000_000]  # ns
    per = {  # counter values per dispatch, in dispatch order
        "FETCH_SIZE": [copy / 2048, copy / 2048, 9e9, 1.0, 2.0, 7.0],  # KiB, half of the copy's true bytes
        "WRITE_SIZE": [copy / 1024, copy / 1024, 9e9, 0.5, 0.25, 1.0],
        "VALUBusy": [0, 0, 99, 30.0, 60.0, 10.0], "MfmaUtil": [0, 0, 0, 0, 0, 25.0],
        "LDSBankConflict": [0, 0, 0, 1.0, 4.0, 2.0],
        "SQ_INSTS_VALU": [0, 0, 5, 100, 300, 7], "SQ_INSTS_LDS": [0] * 6, "SQ_INSTS_MFMA": [0, 0, 0, 0, 0, 9],
        "SQ_LDS_IDX_ACTIVE": [0, 0, 0, 40, 80, 4], "SQ_WAVES": [1] * 6, "GRBM_GUI_ACTIVE": [10] * 6,
    }
    dbs = {}
    for tag, ctrs in (("fetch", ["FETCH_SIZE"]), ("write", ["WRITE_SIZE"]),
                      ("util", ["VALUBusy", "MfmaUtil", "LDSBankConflict"]),
                      ("inst", ["SQ_INSTS_VALU", "SQ_INSTS_LDS", "SQ_INSTS_MFMA", "SQ_LDS_IDX_ACTIVE", "SQ_WAVES",
                                "GRBM_GUI_ACTIVE"]), ("trace", [])):
        rows, t = [], 0
        for i, (n, d) in enumerate(zip(names, durs)):
            rows.append((100 + i, n, t, t + d, {c: per[c][i] for c in ctrs}))
            t += d + 10
        dbs[tag] = tmp_path / f"{tag}.db"
        _db(dbs[tag], rows, counters=bool(ctrs))
    out = bench.summarize_counters(mp, {k: str(v) for k, v in dbs.items()}, out_path=tmp_path / "c.json")
    assert out["byte_scale"]["FETCH_SIZE"] == pytest.approx(2.0) and out["byte_scale"]["WRITE_SIZE"] == 1.0
    enc = out["phases"]["enc"]
    assert enc["kernel_us_total"] == pytest.approx(4.0)
    assert enc["hbm_fetch_bytes"] == pytest.approx((1.0 + 2.0) * 1024 * 2)
    assert enc["hbm_write_bytes"] == pytest.approx(0.75 * 1024)
    assert enc["traffic_over_algorithmic"] == pytest.approx((6144 + 768) / 3000)
    assert enc["hbm_frac"] == pytest.approx(3000 / 4e-6 / 1e9 / bench.HBM_PEAK_GBS)
    assert enc["VALUBusy"] == pytest.approx((30 * 1 + 60 * 3) / 4)  # duration weighted
    assert enc["lds_active_pct"] == pytest.approx((100 * 40 / 10 / 4 * 1 + 100 * 80 / 10 / 4 * 3) / 4)
    assert enc["valu_insts_per_512_elements"] == pytest.approx(400 / 2)
    mm = out["phases"]["mm"]
    assert mm["tera_ops_per_s"] == pytest.approx(5e12 / 2e-3 / 1e12)
    assert mm["mfma_frac"] == pytest.approx(mm["tera_ops_per_s"] / bench.BF16_PEAK_TFLOPS)
    assert mm["MfmaUtil"] == 25.0
    assert json.loads((tmp_path / "c.json").read_text())["phases"]["enc"]["dispatches"] == 2


def test_committed_counter_summary_is_quoted_by_the_bench_line():
    c = bench.load_counters()
    assert c is not None
    assert 0.0 < c["encode_model_set"]["hbm_frac"] < 1.0
    assert 0.0 < c["prefill_m2048_14336x4096"]["MfmaUtil"] < 100.0
    assert 0.0 < c["int8_gemm_2048x8192x8192"]["mfma_frac"] < 1.0
