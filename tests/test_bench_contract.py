"""bench.py's host logic (no GPU): the one-GPU guard, the rocprofv3 CSV
reductions behind profiles/traffic.json and the counter tables, and the
untimed clock warm-up."""
import csv
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def _write_csv(d, rows):
    os.makedirs(d, exist_ok=True)
    with open(os.path.join(d, "p_counter_collection.csv"), "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Dispatch_Id", "Kernel_Name", "Counter_Name",
                                          "Counter_Value"])
        w.writeheader()
        for r in rows:
            w.writerow(dict(zip(w.fieldnames, r)))


def test_more_than_one_gpu_exits_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_pmc_summary_scales_by_the_copy_and_sums_dimensions(tmp_path):
    # the copy's FETCH_SIZE reads half its bytes (KiB, split over two
    # dimension rows), WRITE_SIZE all of them; a kernel with two dispatches
    # averages them; prefill = the forward prep + chain instantiations only
    mib = 1024  # KiB per MiB
    copy = "__amd_rocclr_copyBuffer"
    prep_f = "void gdn::chunk_prep_kernel<128, false, true, false>(int)"
    chain_f = "void gdn::chunk_chain_sw_kernel<128, false, true, 1, true, true>(int)"
    prep_b = "void gdn::chunk_prep_kernel<128, true, false, false>(int)"
    fetch = [(1, copy, "FETCH_SIZE", 64 * mib), (1, copy, "FETCH_SIZE", 64 * mib),
             (2, prep_f, "FETCH_SIZE", 10 * mib), (3, prep_f, "FETCH_SIZE", 30 * mib),
             (4, chain_f, "FETCH_SIZE", 50 * mib), (5, prep_b, "FETCH_SIZE", 7 * mib)]
    write = [(1, copy, "WRITE_SIZE", 256 * mib), (2, prep_f, "WRITE_SIZE", 4 * mib),
             (3, prep_f, "WRITE_SIZE", 4 * mib), (4, chain_f, "WRITE_SIZE", 8 * mib),
             (5, prep_b, "WRITE_SIZE", 1 * mib)]
    _write_csv(str(tmp_path / "f"), fetch)
    _write_csv(str(tmp_path / "w"), write)
    out = str(tmp_path / "traffic.json")
    bench.pmc_summary(str(tmp_path / "f"), str(tmp_path / "w"), out)
    res = json.load(open(out))
    assert res["fetch_size_factor"] == 2.0 and res["write_size_factor"] == 1.0
    k = res["per_kernel"]
    assert k["gdn::chunk_prep_kernel<128, false, true, false>"] == {
        "fetch_bytes": 2 * 20 << 20, "write_bytes": 4 << 20}
    assert k["gdn::chunk_chain_sw_kernel<128, false, true, 1, true, true>"] == {
        "fetch_bytes": 100 << 20, "write_bytes": 8 << 20}
    assert res["prefill"] == (40 + 4 + 100 + 8) << 20
    assert res["backward"] == (14 + 1) << 20
    assert copy not in k


def test_pmc_summary_needs_the_calibration_copy(tmp_path):
    _write_csv(str(tmp_path / "f"), [(1, "gdn::k(int)", "FETCH_SIZE", 1)])
    _write_csv(str(tmp_path / "w"), [(1, "gdn::k(int)", "WRITE_SIZE", 1)])
    with pytest.raises(SystemExit):
        bench.pmc_summary(str(tmp_path / "f"), str(tmp_path / "w"), str(tmp_path / "t.json"))


def test_pmc_table_averages_dispatches(tmp_path, capsys):
    rows = [(1, "void gdn::a<1>(int)", "SQ_WAVES", 4), (1, "void gdn::a<1>(int)", "SQ_WAVES", 4),
            (2, "void gdn::a<1>(int)", "SQ_WAVES", 2)]
    _write_csv(str(tmp_path / "p"), rows)
    bench.pmc_table([str(tmp_path / "p")])
    line = json.loads(capsys.readouterr().out.strip())
    assert line == {"kernel": "gdn::a<1>", "SQ_WAVES": 5.0}


def test_clock_warmup_runs_for_the_time_asked(monkeypatch):
    calls = []
    syncs = []
    monkeypatch.setattr(bench.torch.cuda, "synchronize", lambda dev=None: syncs.append(dev))
    t = [0.0]

    def fake_clock():
        return t[0]

    def fn():
        calls.append(1)
        t[0] += 0.001   # 1 ms of work per call

    monkeypatch.setattr(bench.time, "perf_counter", fake_clock)
    bench._clock_warmup("cpu", fn, ms=20)
    # runs whole groups of 8 calls until 20 ms have passed: 24 calls
    assert len(calls) == 24
    assert len(syncs) >= 2
