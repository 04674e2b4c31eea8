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


LLVM_BIN = Path("/opt/rocm/llvm/bin")


def _gfx950_disassembly(tmp_path: Path) -> dict[str, list[str]]:
    """Instructions per kernel of the library's own gfx950 code object."""
    for tool in ("llvm-objcopy", "clang-offload-bundler", "llvm-objdump"):
        if not (LLVM_BIN / tool).exists():
            pytest.skip(f"{tool} not available")
    fatbin, code = tmp_path / "fatbin", tmp_path / "gfx950.o"
    subprocess.run([str(LLVM_BIN / "llvm-objcopy"), f"--dump-section=.hip_fatbin={fatbin}", str(native.LIB_PATH),
                    str(tmp_path / "host.so")], check=True)
    subprocess.run([str(LLVM_BIN / "clang-offload-bundler"), "--unbundle", "--type=o",
                    "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", f"--input={fatbin}", f"--output={code}"], check=True)
    text = subprocess.run([str(LLVM_BIN / "llvm-objdump"), "-d", "--mcpu=gfx950", str(code)], capture_output=True,
                          text=True, check=True).stdout
    funcs: dict[str, list[str]] = {}
    cur = None
    for line in text.splitlines():
        m = re.match(r"^[0-9a-f]+ <(.+)>:", line)
        if m:
            cur = funcs.setdefault(m.group(1), [])
        elif cur is not None and line.strip() and not line.startswith("Disassembly"):
            cur.append(line.split("//")[0].strip())
    return funcs


def test_lds_dma_owns_m0(tmp_path):
    """The pipelined GEMMs (bf16 and split) set m0 (the LDS base of a
    global->LDS load) from inline assembly, unseen by the compiler: in every
    kernel that loads straight into LDS, each m0 write must directly feed its
    load, and nothing else may use m0."""
    if not native.LIB_PATH.exists():
        pytest.skip("library not built")
    funcs = _gfx950_disassembly(tmp_path)
    dma = [f for f in funcs if any(x.startswith("global_load_lds") for x in funcs[f])]
    assert any("gemm_bf16_dma" in f for f in dma), "pipelined bf16 GEMM kernels missing from the library"
    assert any("gemm_split" in f for f in dma), "split GEMM kernels missing from the library"
    for f in dma:
        ins = funcs[f]
        loads = [i for i, x in enumerate(ins) if x.startswith("global_load_lds")]
        assert loads, f
        for i, x in enumerate(ins):
            if re.search(r"\bm0\b", x):
                assert re.fullmatch(r"s_mov_b32 m0, s\d+", x), (f, x)
                assert ins[i + 1].startswith("global_load_lds_dwordx4"), (f, x, ins[i + 1])
        assert all(re.fullmatch(r"s_mov_b32 m0, s\d+", ins[i - 1]) for i in loads), f
