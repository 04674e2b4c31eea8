"""Write tests/golden/reference_tiny.npz from the reference CPU executable.

Runs oracle/_ref/vocalarc-separation (built from the reference sources by
oracle/Makefile) on a 0.05 s seeded stereo mix with the seed-1234 synthetic
VSCNAT01 pack, with VOCALARC_DEBUG_DUMP set, and stores the input, the output
waveforms and the dumped intermediate tensors (the 90x256 feature tensors
subsampled every 7th value to keep the fixture small).

    python tests/golden/make_golden.py
"""

import sys
import tempfile
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT / "karaoke-platform-sidecar-native_amd"))
sys.path.insert(0, str(ROOT / "oracle"))

import oracle as O  # noqa: E402
from vocalarc_hip import audio, pack  # noqa: E402
from vocalarc_hip.dims import REFERENCE_DIMS  # noqa: E402

PACK_SEED = 1234
AUDIO_SEED = 4242
SECONDS = 0.05
FEATURE_STRIDE = 7


def main() -> None:
    if not O.REF_EXE.exists():
        raise SystemExit("build the reference executable first: make -C oracle ref")
    blob = pack.synthetic_pack(REFERENCE_DIMS, PACK_SEED)
    x = audio.sine_mix(SECONDS, AUDIO_SEED)
    with tempfile.TemporaryDirectory() as tmp:
        t = Path(tmp)
        pack.write_pack(t / "m.f32", blob)
        audio.write_wav_float(t / "in.wav", x)
        resp = O.run_reference(O.REF_EXE, t / "m.f32", t / "in.wav", t / "v.wav", t / "i.wav", threads=4,
                               dump_prefix=str(t / "d"))
        assert any(r.get("type") == "separated" for r in resp), resp
        v, _ = audio.read_wav_float(t / "v.wav")
        inst, _ = audio.read_wav_float(t / "i.wav")
        dumps = {n: np.fromfile(t / f"d-{n}.f32", np.float32)
                 for n in ("source", "band", "features0", "features1", "features16", "mask")}
    T = REFERENCE_DIMS.frames(x.shape[1])
    out = {
        "pack_seed": np.int64(PACK_SEED), "audio_seed": np.int64(AUDIO_SEED), "frames": np.int64(T),
        "feature_stride": np.int64(FEATURE_STRIDE),
        "audio": x, "vocals": v, "instrumental": inst,
        "source": dumps["source"], "mask": dumps["mask"],
    }
    for n in ("band", "features1", "features16"):
        out[n] = dumps[n][::FEATURE_STRIDE].copy()
    np.savez_compressed(Path(__file__).with_name("reference_tiny.npz"), **out)
    print("wrote reference_tiny.npz", {k: getattr(v, "shape", v) for k, v in out.items()})


if __name__ == "__main__":
    main()
