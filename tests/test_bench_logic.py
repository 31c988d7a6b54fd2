"""Host logic of bench.py (no GPU): the rotating-call helper, the per-config
summary and roofline the JSON line carries, and the compute-bound figures of
the f64 activations.  The numbers fed in are made up; what is checked is the
arithmetic the line reports and which op it names."""

import importlib
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


@pytest.fixture(scope="module")
def bench():
    sys.path.insert(0, str(ROOT))
    return importlib.import_module("bench")


def test_rot_cycles_in_order(bench):
    seen = []
    r = bench.Rot([lambda k=k: seen.append(k) or k for k in range(3)])
    assert [r() for _ in range(7)] == [0, 1, 2, 0, 1, 2, 0]
    assert seen == [0, 1, 2, 0, 1, 2, 0]


def test_config_summary(bench, monkeypatch):
    monkeypatch.setitem(bench.COPY, "GBps", 6400.0)
    monkeypatch.setitem(bench.TRAFFIC, "cfgX.big", 1234.0)
    cf = bench.Config("cfgX", "test workload")
    cf.add("small", "k_a", 8_000_000, 1_000_000, 1.0)                        # 8000 GB/s, one launch
    cf.add("big", "k_b + k_c", 64_000_000, 16_000_000, 9.0, 10.0, 2)         # op 10 us over 2 launches
    cf.add("host", "k_d", 4_000_000, 1_000_000, 0.8, 1.0, 2, host_call_us=2.0)
    s = cf.summary({"value": 10.0, "kind": "port", "cores": 1})
    # ops: [op us, % of 8 TB/s]
    assert s["ops"]["small"] == [1.0, 100.0]
    assert s["ops"]["big"] == [10.0, 80.0]
    assert s["ops"]["host"] == [1.0, 50.0]
    # the roofline names the longest op and prices its bytes over its op time
    rf = s["roofline"]
    assert rf["kernel"] == "big" and rf["us"] == 10.0 and rf["bytes"] == 64_000_000
    assert rf["achieved"] == 6400.0 and rf["frac"] == 0.8 and rf["traffic"] == 1234.0
    # aggregate = all bytes over all op time; % of the same-run copy
    agg = (8 + 64 + 4) * 1e6 / (1.0 + 10.0 + 1.0) / 1e3
    assert s["GBps"] == round(agg, 1)
    assert s["pct_of_copy"] == round(100.0 * agg / 6400.0, 1)
    assert s["multi_launch"] == {"big": {"launches": 2, "first_kernel_us": 9.0},
                                 "host": {"launches": 2, "first_kernel_us": 0.8}}
    assert s["host_call"] == {"host": [2.0, 25.0]}
    assert s["cpu"]["speedup"] == round(s["GBps"] / 10.0, 1)
    assert cf.ops["big"]["pct_copy"] == 100.0


def test_compute_bound(bench, monkeypatch):
    # 1e9 VALU wave instructions in 1 ms: 4e9 SIMD cycles against 1024 SIMDs
    # x 2.4 GHz x 1 ms = 2.4576e9 -> issue fraction 1.6276 (VALU-bound); 1e6
    # instructions -> 0.0016 (HBM-bound).  FP64: 7.86e10 FLOP in 1 ms = 78.6
    # TFLOP/s = the whole peak.
    monkeypatch.setattr(bench, "VALU", {"heavy": {"valu": 1e9, "fp64_flops": 7.86e10},
                                        "light": {"valu": 1e6, "fp64_flops": 0.0}})
    cf = bench.Config("cfg3_f64", "t")
    cf.add("heavy", "k", 4_000_000_000, 1, 1000.0)   # 4 GB in 1 ms: 50% of HBM
    cf.add("light", "k", 1_000_000_000, 1, 200.0)    # 5 TB/s: 62.5%
    summ = cf.summary()
    bench.compute_bound(cf, summ)
    h, l_ = summ["compute"]["heavy"], summ["compute"]["light"]
    assert h["fp64_tflops"] == 78.6 and h["fp64_frac"] == 1.0
    assert h["valu_issue_frac"] == round(4e9 / (1024 * 2.4e9 * 1e-3), 4)
    assert l_["valu_issue_frac"] == round(4e6 / (1024 * 2.4e9 * 2e-4), 4)
    assert summ["bound_by_op"] == {"heavy": "valu", "light": "hbm"}
    # the roofline's op is the longest one (heavy), so its bound is VALU
    assert summ["roofline"]["kernel"] == "heavy" and summ["roofline"]["bound"] == "valu"


def test_gpus_above_one_exits(bench, monkeypatch, capsys):
    monkeypatch.setattr(sys, "argv", ["bench.py", "--gpus", "2"])
    with pytest.raises(SystemExit) as e:
        bench.main()
    assert e.value.code == 2
    assert "one GPU" in capsys.readouterr().err
