"""CPU tests of the evaluation runner (cupilot-kernels_amd/evaluate.py): its
table schema is the reference's (latency_summary.csv:1), its problem set covers
every operator of the package, and it refuses to run without a device."""
import csv
import importlib

import pytest

# latency_summary.csv:1 of the reference, the schema the runner writes
REFERENCE_HEADER = ("Problem_ID,Kernels,Target_PyTorch_Latency(ms),Generated_Kernel_Latency(ms),"
                    "Ratio_to_Target")


@pytest.fixture(scope="module")
def ev(ck):
    return importlib.import_module(ck.__name__ + ".evaluate")


def test_header_is_reference_schema(ev):
    assert ",".join(ev.HEADER) == REFERENCE_HEADER
    assert ev.EXT_HEADER[:5] == ev.HEADER


@pytest.mark.parametrize("preset", ["baseline", "small"])
def test_problem_set_covers_every_operator(ck, ev, preset):
    probs = ev._problems(ck, preset)
    assert sorted(p.pid for p in probs) == sorted(ck.PIDS)
    for p in probs:
        assert (p.flops > 0) or (p.nbytes > 0), p.pid


def test_write_csv_round_trip(ev, tmp_path):
    rows = [{"Problem_ID": 1, "Kernels": ev.KERNELS_LABEL, "Target_PyTorch_Latency(ms)": 10.0,
             "Generated_Kernel_Latency(ms)": 8.0, "Ratio_to_Target": 1.25, "Shape": "8x8x8",
             "Work": "", "Generated_Throughput": 1.0, "Unit": "TFLOP/s",
             "Max_Norm_Diff_vs_Torch": 1.5e-7, "CPU_Torch_Latency(ms)": None, "CPU_Threads": None}]
    p = tmp_path / "t.csv"
    ev.write_csv(rows, str(p))
    got = list(csv.reader(open(p)))
    assert ",".join(got[0]) == REFERENCE_HEADER
    assert got[1][:5] == ["1", ev.KERNELS_LABEL, "10.0", "8.0", "1.25"]
    pe = tmp_path / "t_ext.csv"
    ev.write_csv(rows, str(pe), extended=True)
    got = list(csv.DictReader(open(pe)))
    assert got[0]["Shape"] == "8x8x8" and got[0]["CPU_Torch_Latency(ms)"] == ""


def test_refuses_without_device(ev):
    import torch
    if torch.cuda.is_available():
        pytest.skip("a device is present")
    with pytest.raises(RuntimeError, match="HIP device"):
        ev.run([1])


def test_timing_rounds_alternate_and_report_medians(ev, monkeypatch):
    """Both operators are warmed up, then timed in rounds whose order flips
    every round (neither always runs first); each latency is the median of its
    rounds, so one disturbed round does not move it."""
    import torch
    calls, order = [], []
    ref = lambda: calls.append("ref")
    ours = lambda: calls.append("ours")
    samples = {"ref": iter([5.0, 1.0, 2.0, 3.0, 2.5]), "ours": iter([1.0, 1.5, 9.0, 1.2, 1.1])}

    def fake_time(fn, args, reps):
        name = "ref" if fn is ref else "ours"
        order.append(name)
        return next(samples[name])

    monkeypatch.setattr(ev, "_time_reps", fake_time)
    monkeypatch.setattr(torch.cuda, "synchronize", lambda *a, **k: None)
    t_ref, t_ours = ev._time_pair(ref, ours, (), warmup=2, reps=10, rounds=5)
    assert calls == ["ref", "ref", "ours", "ours"]
    assert order == ["ref", "ours", "ours", "ref", "ref", "ours", "ours", "ref", "ref", "ours"]
    assert (t_ref, t_ours) == (2.5, 1.2)
