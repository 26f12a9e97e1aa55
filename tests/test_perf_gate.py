"""perf_gate.py's host logic (merge and compare of synthetic run files): the
median of medians, the spread, the clock-normalised comparison of MFMA-bound
configs and the refusal of runs from different software."""

import json

import pytest

import perf_gate as G


def run_file(tmp_path, name, configs, arch="gfx950", host="box-a", torch_v="2.10"):
    env = {"hostname": host, "device_arch": arch, "torch": torch_v, "hip": "7.0",
           "device_name": "MI355X", "git_head": None, "source_digest": "x"}
    entries = {}
    for cfg, (bound, ms, mhz) in configs.items():
        entries[cfg] = {"bound": bound, "rounds_ms": [ms], "median_ms": ms,
                        "rounds_sclk_mhz": [mhz], "sclk_mhz": mhz, "config": {"w": cfg}}
    p = tmp_path / name
    p.write_text(json.dumps({"schema": 1, "kind": "run", "note": "", "env": env, "steps": 20,
                             "configs": entries}))
    return p


def test_merge_takes_median_of_medians_and_spread(tmp_path, capsys):
    runs = [run_file(tmp_path, f"r{i}.json", {"c2": ("mfma", ms, 1850.0), "c3": ("hbm", 0.66, 2390.0)})
            for i, ms in enumerate((0.120, 0.126, 0.122))]
    out = tmp_path / "m.json"
    assert G.main(["merge", "--runs", *map(str, runs), "--out", str(out)]) == 0
    m = json.loads(out.read_text())["configs"]
    assert m["c2"]["median_ms"] == pytest.approx(0.122)
    assert m["c2"]["spread_pct"] == pytest.approx(100 * 0.006 / 0.120, abs=1e-3)
    assert m["c2"]["median_kcycles"] == pytest.approx(0.122 * 1850.0)
    assert m["c3"]["spread_pct"] == 0


def test_compare_normalises_mfma_configs_by_clock(tmp_path):
    # 5% slower in ms but at a 5% lower clock: the same cycles, so it passes;
    # the HBM-bound config is judged by ms.
    base = run_file(tmp_path, "b.json", {"c2": ("mfma", 0.120, 1900.0), "c3": ("hbm", 0.660, 2390.0)})
    slow_clock = run_file(tmp_path, "c.json", {"c2": ("mfma", 0.120 * 1.05, 1900.0 / 1.05),
                                               "c3": ("hbm", 0.665, 2300.0)}, host="box-b")
    assert G.main(["compare", "--baseline", str(base), "--candidate", str(slow_clock)]) == 0
    assert G.main(["compare", "--baseline", str(base), "--candidate", str(slow_clock), "--raw"]) == 1
    regress = run_file(tmp_path, "d.json", {"c2": ("mfma", 0.130, 1900.0), "c3": ("hbm", 0.660, 2390.0)})
    assert G.main(["compare", "--baseline", str(base), "--candidate", str(regress)]) == 1
    hbm_regress = run_file(tmp_path, "e.json", {"c2": ("mfma", 0.120, 1900.0), "c3": ("hbm", 0.70, 2390.0)})
    assert G.main(["compare", "--baseline", str(base), "--candidate", str(hbm_regress)]) == 1
    assert G.main(["compare", "--baseline", str(base), "--candidate", str(hbm_regress),
                   "--threshold", "10"]) == 0


def test_compare_refuses_other_software(tmp_path):
    base = run_file(tmp_path, "b.json", {"c2": ("mfma", 0.12, 1900.0)})
    other = run_file(tmp_path, "c.json", {"c2": ("mfma", 0.12, 1900.0)}, torch_v="2.9")
    with pytest.raises(SystemExit, match="torch differs"):
        G.main(["compare", "--baseline", str(base), "--candidate", str(other)])
    arch = run_file(tmp_path, "d.json", {"c2": ("mfma", 0.12, 1900.0)}, arch="gfx942")
    with pytest.raises(SystemExit, match="device_arch differs"):
        G.main(["merge", "--runs", str(base), str(arch), "--out", str(tmp_path / "m.json")])


def test_compare_without_clock_falls_back_to_ms(tmp_path):
    base = run_file(tmp_path, "b.json", {"c2": ("mfma", 0.120, None)})
    cand = run_file(tmp_path, "c.json", {"c2": ("mfma", 0.125, 1800.0)})
    assert G.main(["compare", "--baseline", str(base), "--candidate", str(cand)]) == 1
