"""bench.py's host-side pieces that need no GPU: the per-config profiler table built from
rocprofv3 counter CSVs (the byte counters scaled by the calibration copy, one table entry per
measured config), its attachment to measured configs, and the decode step's per-instance traffic
table."""
from __future__ import annotations

import csv
import importlib.util
import json
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


@pytest.fixture(scope="module")
def bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", ROOT / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    sys.modules["bench_under_test"] = mod
    spec.loader.exec_module(mod)
    return mod


def write_pass(path: Path, counters: dict, per_kernel: dict, copy_value: dict) -> None:
    """A counter CSV as rocprofv3 writes it: one row per dispatch, counter and hardware instance
    (here each dispatch's value split over two instances, which the summary must add back)."""
    cols = ["Dispatch_Id", "Kernel_Name", "Grid_Size", "Counter_Name", "Counter_Value"]
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, cols)
        w.writeheader()
        did = 0
        rows = [("__amd_rocclr_copyBuffer", 131072, copy_value)] + [
            (f"void tars::(anonymous namespace)::{name}(Args)", grid, per_kernel[(name, grid)])
            for name, grid in per_kernel]
        for name, grid, vals in rows:
            for _ in range(3):
                did += 1
                for c in counters:
                    for half in (0.25, 0.75):
                        w.writerow({"Dispatch_Id": did, "Kernel_Name": name, "Grid_Size": grid,
                                    "Counter_Name": c, "Counter_Value": vals.get(c, 0.0) * half})


def test_pmc_summary_scales_and_attaches(bench, tmp_path, monkeypatch):
    kernels = sorted(set(bench.CONFIG_KERNELS.values()))
    fetch = {k: {"FETCH_SIZE": 1000.0 + i} for i, k in enumerate(kernels)}
    write = {k: {"WRITE_SIZE": 10.0 + i} for i, k in enumerate(kernels)}
    mfma = {k: {"SQ_VALU_MFMA_BUSY_CYCLES": 1024.0 * 768, "SQ_INSTS_VALU_MFMA_MOPS_I8": 2.0} for k in kernels}
    valu = {k: {"SQ_INSTS_VALU": 1024.0 * 100} for k in kernels}
    # the copy of 256 MiB reads FETCH_SIZE = 131072 KiB (64 B units counted as 32) and writes 262144 KiB
    paths = []
    for i, (cnt, table, copy) in enumerate((
            (["FETCH_SIZE"], fetch, {"FETCH_SIZE": 131072.0}),
            (["WRITE_SIZE"], write, {"WRITE_SIZE": 262144.0}),
            (["SQ_VALU_MFMA_BUSY_CYCLES", "SQ_INSTS_VALU_MFMA_MOPS_I8"], mfma, {}),
            (["SQ_INSTS_VALU"], valu, {}))):
        p = tmp_path / f"p{i}.csv"
        write_pass(p, cnt, table, copy)
        paths.append(str(p))
    detail = tmp_path / "detail.json"
    detail.write_text(json.dumps({"configs": {k: {"bytes_per_call": 2_000_000} for k in bench.CONFIG_KERNELS}}))
    out = tmp_path / "table.json"
    assert bench.pmc_summary(paths, str(detail), str(out)) == 0
    t = json.loads(out.read_text())
    assert t["fetch_scale"] == 2.0 and t["write_scale"] == 1.0
    for key, (name, grid) in bench.CONFIG_KERNELS.items():
        e = t["configs"][key]
        i = kernels.index((name, grid))
        assert e["dispatches"] == 3
        assert e["read_bytes"] == round((1000.0 + i) * 1024 * 2) and e["write_bytes"] == round((10.0 + i) * 1024)
        assert e["traffic_bytes"] == e["read_bytes"] + e["write_bytes"]
        assert e["mfma_busy_cycles_per_simd"] == 768 and e["mfma_i8_ops"] == 1024
        assert e["valu_instructions_per_simd"] == 100
    monkeypatch.setattr(bench, "COUNTER_FILE", out)
    key = "c4_prefill_M256_K1024_N3072"
    res = {key: {"bytes_per_call": 2_000_000, "us_per_call": 1.0},
           "c1_gemv_qwen3_gate_M1_K1024_N3072": {"bytes_per_call": 123, "us_per_call": 1.0}}
    bench.attach_counters(res)
    c = res[key]["counters"]
    assert c["mfma_busy_frac"] == round(768 / 2400, 4) and c["valu_issue_frac"] == round(400 / 2400, 4)
    assert "counters" not in res["c1_gemv_qwen3_gate_M1_K1024_N3072"]     # other bytes: a stale entry


def test_pmc_summary_refuses_a_missing_kernel(bench, tmp_path):
    paths = []
    for i, c in enumerate(("FETCH_SIZE", "WRITE_SIZE", "SQ_VALU_MFMA_BUSY_CYCLES", "SQ_INSTS_VALU")):
        p = tmp_path / f"only_copy{i}.csv"
        write_pass(p, [c], {}, {c: 131072.0})
        paths.append(str(p))
    detail = tmp_path / "detail.json"
    detail.write_text(json.dumps({"configs": {}}))
    with pytest.raises(SystemExit, match="0 kernels match"):
        bench.pmc_summary(paths, str(detail), str(tmp_path / "o.json"))


def test_pmc_step_summary_separates_grids_and_scales(bench, tmp_path):
    """The decode step's traffic per row: one kernel instance's dispatches of two grids (28 q/k/v-like
    and one head-like per step) kept apart by grid size, the byte counters scaled by the 1 GiB
    copy's readings, the algorithmic bytes taken from the detail's rows."""
    name = "quant_gemv_w8a8_kernel<64, 1, 4, true, false>"
    cols = ["Dispatch_Id", "Kernel_Name", "Grid_Size", "Counter_Name", "Counter_Value"]
    paths = []
    for c, copy_kib, small, big in (("FETCH_SIZE", 524288.0, 100.0, 1000.0), ("WRITE_SIZE", 1048576.0, 4.0, 40.0)):
        p = tmp_path / f"{c}.csv"
        with open(p, "w", newline="") as f:
            w = csv.DictWriter(f, cols)
            w.writeheader()
            rows = [("__amd_rocclr_copyBuffer", 1 << 20, copy_kib)] + \
                [(f"void tars::(anonymous namespace)::{name}(float const*, long)", 65536, small)] * 28 + \
                [(f"void tars::(anonymous namespace)::{name}(float const*, long)", 2430976, big)]
            for did, (kn, grid, v) in enumerate(rows):
                w.writerow({"Dispatch_Id": did, "Kernel_Name": kn, "Grid_Size": grid, "Counter_Name": c,
                            "Counter_Value": v})
        paths.append(str(p))
    detail = tmp_path / "detail.json"
    rows = {f"{name} @ qkv": {"kernel": name, "role": "qkv", "grid_items": 65536, "avg_bytes_per_launch": 4_229_120},
            f"{name} @ head": {"kernel": name, "role": "head", "grid_items": 2430976, "avg_bytes_per_launch": 156_806_144}}
    detail.write_text(json.dumps({"roofline_rows": rows}))
    out = tmp_path / "step.json"
    assert bench.pmc_step_summary(paths[0], paths[1], str(detail), str(out)) == 0
    t = json.loads(out.read_text())
    assert t["fetch_scale"] == 2.0 and t["write_scale"] == 1.0
    q, h = t["rows"][f"{name} @ qkv"], t["rows"][f"{name} @ head"]
    assert q["dispatches"] == 28 and h["dispatches"] == 1
    assert q["read_bytes"] == round(100.0 * 1024 * 2) and h["read_bytes"] == round(1000.0 * 1024 * 2)
    assert q["write_bytes"] == round(4.0 * 1024) and h["write_bytes"] == round(40.0 * 1024)
    assert q["traffic_bytes"] == q["read_bytes"] + q["write_bytes"] and q["algorithmic_bytes"] == 4_229_120
    rows[f"{name} @ qkv"]["grid_items"] = 12345
    detail.write_text(json.dumps({"roofline_rows": rows}))
    with pytest.raises(SystemExit, match="0 dispatch groups"):
        bench.pmc_step_summary(paths[0], paths[1], str(detail), str(out))


def test_trace_summary_per_row(bench, tmp_path):
    """Kernel-trace durations per row (instance and grid) against the line's figures: the mean
    over a row's dispatches, the HBM fraction it gives for the row's algorithmic bytes, and the
    roofline row's ratio of trace to bench duration."""
    name = "quant_gemv_w8a8_kernel<64, 1, 6, true, false>"
    other = "quant_gemv_w8a8_kernel<64, 3, 1, true, false>"
    p = tmp_path / "kernel_trace.csv"
    with open(p, "w", newline="") as f:
        w = csv.DictWriter(f, ["Kernel_Name", "Grid_Size_X", "Grid_Size_Y", "Grid_Size_Z", "Start_Timestamp",
                               "End_Timestamp"])
        w.writeheader()
        for i, d in enumerate((2000, 2200, 2400)):
            w.writerow({"Kernel_Name": f"void tars::(anonymous namespace)::{name}(float const*)", "Grid_Size_X": 65536,
                        "Grid_Size_Y": 1, "Grid_Size_Z": 1, "Start_Timestamp": 10_000 * i, "End_Timestamp": 10_000 * i + d})
        w.writerow({"Kernel_Name": f"void tars::(anonymous namespace)::{other}(float const*)", "Grid_Size_X": 65536,
                    "Grid_Size_Y": 1, "Grid_Size_Z": 1, "Start_Timestamp": 0, "End_Timestamp": 1500})
    rows = {f"{name} @ gate_up": {"kernel": name, "role": "gate_up", "grid_items": 65536, "launches_per_step": 28,
                                  "avg_bytes_per_launch": 6_344_704, "us_per_launch": 2.25, "hbm_frac": 0.35},
            f"{other} @ down": {"kernel": other, "role": "down", "grid_items": 65536, "launches_per_step": 28,
                                "avg_bytes_per_launch": 3_166_208, "us_per_launch": 1.5, "hbm_frac": 0.26}}
    roof = {"kernel": name, "shape": "gate_up", "frac": 0.35, "avg_us_per_launch": 2.25, "avg_bytes_per_launch": 6_344_704}
    detail = tmp_path / "detail.json"
    detail.write_text(json.dumps({"roofline_rows": rows, "roofline": roof}))
    out = tmp_path / "kernels.json"
    assert bench.trace_summary(str(p), str(detail), str(out)) == 0
    t = json.loads(out.read_text())
    r = t["rows"][f"{name} @ gate_up"]
    assert r["trace_dispatches"] == 3 and r["trace_avg_us"] == 2.2 and r["trace_min_us"] == 2.0
    assert r["hbm_frac_from_trace"] == round(6_344_704 / 2.2 / 1e3 / 8000, 4)
    assert t["roofline_row"] == f"{name} @ gate_up" and t["trace_over_bench_duration"] == round(2.2 / 2.25, 4)
    assert t["rows"][f"{other} @ down"]["trace_dispatches"] == 1
    assert (tmp_path / "kernels.table.md").read_text().count("\n") == 4



def test_quantiles_match_numpy(bench):
    """The per-config p10 / median / p90 use numpy's default (linear) quantiles."""
    import numpy as np
    rng = np.random.default_rng(7)
    for n in (1, 2, 3, 10, 11, 500):
        xs = list(rng.normal(3.0, 0.2, n))
        assert np.allclose(bench.quantiles(xs), np.quantile(xs, [0.1, 0.5, 0.9]), rtol=0, atol=1e-12)
