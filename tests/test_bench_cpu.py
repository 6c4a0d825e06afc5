"""bench.py's host-side parts: the one-GPU guard, the labelling of decode
dispatches by walk group, and the counter summary's calibration against a
copy of known size (on synthetic rocprofv3-style listings)."""
import csv
import importlib.util
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def bench():
    spec = importlib.util.spec_from_file_location("bench", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=60)
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def decode_listing(steps, layers, prefill=3):
    """Dispatch listing of `prefill` + `steps` decode steps: per layer the
    q/k/v walk, attention, o, w1/w3 and w2 walks, then the LM head and a
    small kernel; values encode the kind."""
    code = {"qkv": 1, "o": 2, "ffn13": 3, "ffn2": 4, "lm": 5, "attention": 6}
    rows, d = [], 0
    for s in range(prefill + steps):
        for L in range(layers):
            for kind in ("qkv", "attention", "o", "ffn13", "ffn2"):
                name = "iam::k_attn<double>(...)" if kind == "attention" else "void iam::k_walk<double, 8, 4>(...)"
                rows.append((d, name, code[kind] * 1000 + s))
                d += 1
        rows.append((d, "void iam::k_walk<double, 8, 4>(...)", code["lm"] * 1000 + s))
        rows.append((d + 1, "iam::k_set_int(int*, int)", 0))
        d += 2
    return rows, code


def test_label_dispatches_takes_the_last_steps_by_kind(bench):
    steps, layers, prefill = 4, 3, 3
    rows, code = decode_listing(steps, layers, prefill)
    lab = bench.label_dispatches(rows, steps, layers)
    for kind, c in code.items():
        n = steps if kind == "lm" else steps * layers
        assert len(lab[kind]) == n, kind
        assert all(v // 1000 == c and v % 1000 >= prefill for _, _, v in lab[kind]), kind


def test_counter_summary_calibrates_on_the_copy(bench, tmp_path, capsys):
    steps, layers = 2, 2
    rows, code = decode_listing(steps, layers, prefill=1)
    copy_bytes = 1 << 20
    probe = {"steps": steps, "layers": layers, "copy_bytes": copy_bytes, "kv_bytes": 4096.0,
             "groups": {g: {"weight_bytes": 0.0, "bytes": 1024.0 * code[g]} for g in bench.GROUPS}}
    pj = tmp_path / "probe.json"
    pj.write_text("log line\n" + json.dumps(probe) + "\n")
    paths = []
    for ctr, per_kib in (("FETCH_SIZE", 0.5), ("WRITE_SIZE", 1.0)):
        path = tmp_path / f"{ctr}.csv"
        with open(path, "w", newline="") as f:
            w = csv.writer(f)
            w.writerow(["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"])
            for d, name, v in rows:
                kib = (v // 1000) * per_kib       # kind k moves k KiB (FETCH_SIZE reads half)
                # two agent-level rows per dispatch, summed by the reader
                w.writerow([d, name, ctr, kib / 2])
                w.writerow([d, name, ctr, kib / 2])
            w.writerow([len(rows), "__amd_rocclr_copyBuffer", ctr, copy_bytes / 1024 * per_kib])
        paths.append(str(path))

    class A:
        counter_summary = paths
        probe = str(pj)
        trace = None
    bench.run_counter_summary(A)
    out = capsys.readouterr().out
    # both counters calibrate to k KiB read and k KiB written for kind k:
    # traffic / algorithmic = 2 for every walk group (algorithmic k KiB),
    # 3 for attention (12 KiB moved, 4 KiB algorithmic)
    for g in bench.GROUPS + ("attention",):
        line = next(ln for ln in out.splitlines() if ln.startswith(f"| {g} |") and ln.count("|") == 6)
        assert line.split("|")[-2].strip() == ("3.000" if g == "attention" else "2.000"), line
    assert "| traffic / algorithmic (every walk launch) | 2.000 |" in out
