"""Inputs for running the reference host (native/vocalarc_separation.c) by
hand, e.g. under a profiler: a seeded pack at the reference shape, a
config-0-recipe mix (6 sines per channel plus N(0, 0.01^2) noise), and the
JSONL requests of the host's protocol (ping, load, `requests` separations,
shutdown; native/vocalarc_separation.c:1537-1605) to pipe into it:

    python -m vocalarc_hip.host_inputs OUT_DIR [--seconds 10] [--requests 4]
    HOST --model OUT_DIR/model.f32 --threads N < OUT_DIR/requests.jsonl
"""

from __future__ import annotations

import argparse
import json
from pathlib import Path

from . import audio, pack
from .dims import REFERENCE_DIMS


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("out")
    ap.add_argument("--seconds", type=float, default=10.0)
    ap.add_argument("--requests", type=int, default=4)
    args = ap.parse_args()
    out = Path(args.out).resolve()
    out.mkdir(parents=True, exist_ok=True)
    pack.write_pack(out / "model.f32", pack.synthetic_pack(REFERENCE_DIMS, 1234))
    audio.write_wav_float(out / "in.wav", audio.sine_mix(args.seconds, 2026))
    lines = [{"id": 1, "type": "ping"}, {"id": 2, "type": "load", "modelPath": str(out / "model.f32")}]
    for r in range(args.requests):
        lines.append({"id": 10 + r, "type": "separate", "inputPath": str(out / "in.wav"),
                      "vocalsPath": str(out / "vocals.wav"), "instrumentalPath": str(out / "instrumental.wav")})
    lines.append({"id": 99, "type": "shutdown"})
    (out / "requests.jsonl").write_text("".join(json.dumps(x) + "\n" for x in lines))
    print(out / "requests.jsonl")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
