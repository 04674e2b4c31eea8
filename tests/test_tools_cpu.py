"""The measurement tools' host-side logic, on the CPU: the reference-host
input writer (vocalarc_hip.host_inputs) and the per-request split of a
profiled host run (vocalarc_hip.kernel_stats host) on a synthetic trace."""

import csv
import json
import subprocess
import sys
from pathlib import Path

from vocalarc_hip import audio, kernel_stats, pack
from vocalarc_hip.dims import REFERENCE_DIMS

PKG = Path(__file__).resolve().parents[1] / "karaoke-platform-sidecar-native_amd"


def test_host_inputs(tmp_path):
    out = tmp_path / "in"
    subprocess.run([sys.executable, "-m", "vocalarc_hip.host_inputs", str(out), "--seconds", "0.5",
                    "--requests", "3"], check=True, cwd=PKG, capture_output=True)
    lines = [json.loads(x) for x in (out / "requests.jsonl").read_text().splitlines()]
    assert [x["type"] for x in lines] == ["ping", "load", "separate", "separate", "separate", "shutdown"]
    assert lines[1]["modelPath"] == str(out / "model.f32")
    assert all(x["inputPath"] == str(out / "in.wav") for x in lines[2:5])
    assert (out / "model.f32").stat().st_size == pack.pack_bytes(REFERENCE_DIMS)
    x = audio.read_wav_float(out / "in.wav")[0]
    assert x.shape == (2, int(0.5 * audio.RATE))


def _write_csv(path: Path, fields, rows):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=fields)
        w.writeheader()
        w.writerows(rows)


def test_host_trace_split(tmp_path):
    """Two requests 50 ms apart: kernels and copies are summed per request,
    the device span runs from the first start to the last end of each."""
    run = tmp_path / "run"
    run.mkdir()
    ms = 1_000_000
    kern = [("k_a", 0, 2 * ms), ("k_b", 3 * ms, 4 * ms), ("k_a", 60 * ms, 61 * ms)]
    copies = [(1 * ms, int(1.5 * ms)), (62 * ms, int(62.25 * ms))]
    _write_csv(run / "hp_kernel_trace.csv", ["Kernel_Name", "Start_Timestamp", "End_Timestamp"],
               [{"Kernel_Name": n, "Start_Timestamp": a, "End_Timestamp": b} for n, a, b in kern])
    _write_csv(run / "hp_memory_copy_trace.csv", ["Direction", "Start_Timestamp", "End_Timestamp"],
               [{"Direction": "MEMORY_COPY_HOST_TO_DEVICE", "Start_Timestamp": a, "End_Timestamp": b}
                for a, b in copies])
    resp = tmp_path / "resp.jsonl"
    resp.write_text("\n".join(json.dumps(x) for x in (
        {"type": "pong"}, {"type": "separated", "inferenceMs": 9.5}, {"type": "separated", "inferenceMs": 3.25})))
    out = tmp_path / "host.md"
    assert kernel_stats.host(str(run), str(resp), str(out), "cmd") == 0
    rows = [r for r in out.read_text().splitlines() if r.startswith("| 1 ") or r.startswith("| 2 ")]
    assert len(rows) == 2
    c1 = [c.strip() for c in rows[0].split("|")[1:-1]]
    c2 = [c.strip() for c in rows[1].split("|")[1:-1]]
    assert c1[:5] == ["1", "9.5", "4.0", "3.0", "0.5 (1)"]
    assert c2[:5] == ["2", "3.2", "2.2", "1.0", "0.2 (1)"]
    assert c1[5].startswith("k_a 2.0; k_b 1.0")
