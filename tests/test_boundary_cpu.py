"""The drop-in boundary without a GPU (CPU only): the library loads, exports
every entry point its headers declare, links no vendor BLAS, and the
reference host linked against it falls back to the CPU path."""

import re
import subprocess
from pathlib import Path

import pytest

from vocalarc_hip import native

ROOT = Path(__file__).resolve().parent.parent
HEADERS = [ROOT / "include" / "native_gpu.h", ROOT / "include" / "vocalarc_hip.h"]


def declared_functions(path: Path) -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", path.read_text(), flags=re.S)
    names = re.findall(r"^[A-Za-z_][\w \*]*?\b(\w+)\s*\(", text, flags=re.M)
    return sorted({n for n in names if n not in ("if", "defined")})


def test_headers_match_binding_lists():
    assert declared_functions(HEADERS[0]) == sorted(native.ABI_SYMBOLS)
    assert declared_functions(HEADERS[1]) == sorted(native.HARNESS_SYMBOLS)


def test_library_exports_every_declared_symbol():
    if not native.LIB_PATH.exists():
        pytest.skip("library not built")
    lib = native.lib()
    for h in HEADERS:
        for name in declared_functions(h):
            assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", str(native.LIB_PATH)], capture_output=True, text=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    for h in HEADERS:
        assert set(declared_functions(h)) <= exported


def test_no_vendor_blas_or_cuda():
    if not native.LIB_PATH.exists():
        pytest.skip("library not built")
    deps = subprocess.run(["ldd", str(native.LIB_PATH)], capture_output=True, text=True).stdout
    for banned in ("blas", "cublas", "cudart", "hipblas", "rocblas", "miopen"):
        assert banned not in deps.lower(), banned


def test_reference_host_protocol_without_gpu(tmp_path):
    """native/scripts/test_native.sh: ping/load/shutdown; with no device the
    provider returns NULL and the host reports the CPU backend."""
    import oracle as O
    from vocalarc_hip import pack
    from vocalarc_hip.dims import REFERENCE_DIMS
    from helpers import gpu_available
    if not O.REF_GPU_EXE.exists():
        pytest.skip("reference host not linked (make -C oracle gpu-host)")
    if gpu_available():
        pytest.skip("a GPU is present")
    p = tmp_path / "m.f32"
    pack.write_pack(p, pack.synthetic_pack(REFERENCE_DIMS, 1))
    proc = subprocess.run([str(O.REF_GPU_EXE), "--threads", "1"], capture_output=True, text=True, timeout=120,
                          input='{"id":1,"type":"ping"}\n{"id":2,"type":"load","modelPath":"%s"}\n'
                                '{"id":3,"type":"shutdown"}\n' % p)
    assert proc.returncode == 0, proc.stderr
    assert '"type":"pong"' in proc.stdout and '"backend":"native-cpu"' in proc.stdout
    assert '"type":"loaded"' in proc.stdout and '"type":"shutdown"' in proc.stdout


def test_pack_sizes():
    from vocalarc_hip import pack
    from vocalarc_hip.dims import CONFIG_DIMS, REFERENCE_DIMS
    # native/assets/manifest.json:6
    assert pack.pack_bytes(REFERENCE_DIMS) == 267_386_408
    assert pack.pack_bytes(CONFIG_DIMS) > pack.pack_bytes(CONFIG_DIMS.with_depth(1))
