"""ctypes binding of lib/libvocalarc_hip.so (include/vocalarc_hip.h and
include/native_gpu.h).

Device buffers are passed as raw pointers; the tests and the benchmark use
torch tensors on cuda:0 for device memory and streams.  There is no fallback:
if the library is missing the import of `lib()` raises.
"""

from __future__ import annotations

import ctypes
import os
import weakref
from pathlib import Path

from .dims import CDims, ModelDims, to_c

PKG = Path(__file__).resolve().parent.parent
# VOCALARC_HIP_LIB names another build of the library (e.g. to compare two)
LIB_PATH = Path(os.environ.get("VOCALARC_HIP_LIB", PKG / "lib" / "libvocalarc_hip.so"))

EPI_STORE, EPI_GELU, EPI_TANH, EPI_RESIDUAL, EPI_GEGLU = range(5)
PRECISION_FP32, PRECISION_BF16, PRECISION_FP32_MFMA = 0, 1, 2
BF16_A, BF16_C, BF16_STAGED = 1, 2, 4  # vh_gemm_bf16 operand flags; STAGED forces the register-staged kernel
ATT_OUT_BF16, ATT_BF16, ATT_SPLIT, ATT_H2, ATT_OUT_H2 = 1, 2, 4, 8, 16  # vh_attention flags
NOALLOC_MAX_LENGTH = 4096  # VH_NOALLOC_MAX_LENGTH
SPEC_REFERENCE, SPEC_FRAME_MAJOR = 0, 1  # spectrum layouts: [F][C][T][2] / [C][T][F][2]

_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_lib = None

# Signatures (result, arguments) of every entry point declared in
# include/vocalarc_hip.h (vh_*) and include/native_gpu.h (native_gpu_*).
SIGNATURES = {
    "vh_create": (_P, []), "vh_destroy": (None, [_P]), "vh_set_stream": (_I, [_P, _P]),
    "vh_synchronize": (_I, [_P]), "vh_last_error": (ctypes.c_char_p, []), "vh_device_name": (ctypes.c_char_p, [_P]),
    "vh_rmsnorm": (_I, [_P, _I64, _I, _P, _P, _P]), "vh_rmsnorm_bf16": (_I, [_P, _I64, _I, _P, _P, _P]),
    "vh_rmsnorm_h2": (_I, [_P, _I64, _I, _P, _P, _P, _P]),
    "vh_softmax_rows": (_I, [_P, _I64, _I, _P, _P]),
    "vh_rope_bhld": (_I, [_P, _I64, _I, _I, _P]),
    "vh_geglu": (_I, [_P, _I64, _I, _P, _P]),
    "vh_residual_add": (_I, [_P, _I64, _P, _P]),
    "vh_gemm": (_I, [_P, _I64, _I, _I, _P, _I, _P, _I, _P, _P, _I, _I]),
    "vh_gemm_bf16": (_I, [_P, _I64, _I, _I, _P, _I, _P, _I, _P, _P, _I, _I, _I]),
    "vh_gemm_split": (_I, [_P, _I64, _I, _I, _P, _I, _P, _P, _P, _I, _I]),
    "vh_split_bytes": (ctypes.c_size_t, [_I, _I]),
    "vh_split_weights": (_I, [_P, _I, _I, _P, _I, _P]),
    "vh_gemm_h2": (_I, [_P, _I64, _I, _I, _P, _I, ctypes.c_float, _P, _P, _P, _I, _I, _I]),
    "vh_gemm_h2_ex": (_I, [_P, _I64, _I, _I, _P, _I, _P, _P, _P, _P, _I, _I, _I, _P, _P]),
    "vh_h2_bytes": (ctypes.c_size_t, [_I, _I]),
    "vh_split_weights_h2": (_I, [_P, _I, _I, _P, _I, _P]),
    "vh_operand_bounds": (_I, [_P, _P, _I, _P, _I, _P, _I, _P]),
    "vh_to_bf16": (_I, [_P, _I64, _I, _P, _P, _I]),
    "vh_attention": (_I, [_P, _I, _I, _I, _P, _P, _I, _I]),
    "vh_attention_noalloc": (_I, [_P, _I, _I, _I, _P, _P, _I, _I]),
    "vh_model_load": (_P, [_P, ctypes.POINTER(CDims), _P, ctypes.c_size_t]),
    "vh_model_free": (None, [_P]), "vh_model_set_precision": (_I, [_P, _I]),
    "vh_transformer": (_I, [_P, _P, _I, _I, _P, _I, _I]),
    "vh_stft": (_I, [_P, _P, _P, _I, _P, _I]),
    "vh_istft": (_I, [_P, _P, _P, _P, _I, _P, _I]),
    "vh_band_split": (_I, [_P, _P, _P, _I, _P, _I]),
    "vh_mask_estimate": (_I, [_P, _P, _P, _I, _P, _I]),
    "vh_forward": (_I, [_P, _P, _P, _I, _P, _P]),
    "vh_separate": (_I, [_P, _P, _P, _I, _I, _I, _I, _P, _P]),
    "vh_timing_enable": (_I, [_P, ctypes.c_char_p]), "vh_timing_reset": (_I, [_P]),
    "vh_timing_get": (_I, [_P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(_I64)]),
    "native_gpu_create": (_P, []), "native_gpu_destroy": (None, [_P]),
    "native_gpu_matmul": (_I, [_P, _I64, _I, _I, _P, _P, _P, _P]),
    "native_gpu_backend": (ctypes.c_char_p, [_P]), "native_gpu_device": (ctypes.c_char_p, [_P]),
    "native_gpu_uses_full_batches": (_I, [_P]), "native_gpu_can_use_full_batches": (_I, [_P, _I]),
    "native_gpu_transformer": (_I, [_P, _I, _I, _P, _P, _P, _P, _P, _P]),
    "native_gpu_resident_begin": (_I, [_P, _I, _I, _P]),
    "native_gpu_resident_transformer": (_I, [_P, _I, _I, _P]),
    "native_gpu_resident_transpose": (_I, [_P, _I, _I]),
    "native_gpu_resident_end": (_I, [_P, _P]),
    "native_gpu_resident_mask": (_I, [_P, _I, _P, _P, _P, _I]),
}
HARNESS_SYMBOLS = [n for n in SIGNATURES if n.startswith("vh_")]
ABI_SYMBOLS = [n for n in SIGNATURES if n.startswith("native_gpu_")]


class NativeError(RuntimeError):
    pass


def lib():
    """Load the HIP library (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise NativeError(f"{LIB_PATH} is missing: build it with `make -C {PKG}`")
    L = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def last_error() -> str:
    e = lib().vh_last_error()
    return e.decode() if e else ""


def _ok(rc: int, what: str) -> None:
    if not rc:
        raise NativeError(f"{what} failed: {last_error()}")


def ptr(t) -> int:
    """Device (or host) address of a torch tensor / numpy array."""
    if hasattr(t, "data_ptr"):
        return t.data_ptr()
    return t.ctypes.data


def _opt(t):
    """ptr(t), or a null pointer for None."""
    return ptr(t) if t is not None else None


def _out_cols(N: int, epilogue: int) -> int:
    """Output columns of a linear with N weight rows (GELU-GLU halves them)."""
    return N // 2 if epilogue == EPI_GEGLU else N


def _att_flags(out_bf16: bool, bf16: bool, split: bool, h2: bool) -> int:
    return ((ATT_OUT_BF16 if out_bf16 else 0) | (ATT_BF16 if bf16 else 0) | (ATT_SPLIT if split else 0) |
            (ATT_H2 if h2 else 0))


class Context:
    """vh_context bound to a HIP stream (default: torch's current stream)."""

    def __init__(self, stream: int | None = None):
        self.models = weakref.WeakSet()  # vh_destroy frees them with the context
        self.h = lib().vh_create()
        if not self.h:
            raise NativeError(f"vh_create failed: {last_error()}")
        if stream is None:
            try:
                import torch
                stream = torch.cuda.current_stream().cuda_stream
            except Exception:  # noqa: BLE001 - no torch: the null stream
                stream = 0
        _ok(lib().vh_set_stream(self.h, stream), "vh_set_stream")

    def close(self):
        if self.h:
            for m in list(self.models):  # freed by vh_destroy below
                m.h = None
            lib().vh_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # noqa: BLE001
            pass

    @property
    def device_name(self) -> str:
        return lib().vh_device_name(self.h).decode()

    def sync(self):
        _ok(lib().vh_synchronize(self.h), "vh_synchronize")

    def set_stream(self, stream: int):
        """Issue the context's work on the HIP stream handle `stream` (0: the null stream)."""
        _ok(lib().vh_set_stream(self.h, stream), "vh_set_stream")

    # -- isolated kernels (device pointers) --
    def rmsnorm(self, x, gamma, y, rows: int, dim: int):
        _ok(lib().vh_rmsnorm(self.h, rows, dim, ptr(x), ptr(gamma), ptr(y)), "vh_rmsnorm")

    def rmsnorm_bf16(self, x, gamma, y, rows: int, dim: int):
        _ok(lib().vh_rmsnorm_bf16(self.h, rows, dim, ptr(x), ptr(gamma), ptr(y)), "vh_rmsnorm_bf16")

    def rmsnorm_h2(self, x, gamma, bound, y, rows: int, dim: int):
        """y as h2 rows (fp16 pieces of y * 2^e, e from the device float bound[0]) for gemm_h2(a_rows=True)."""
        _ok(lib().vh_rmsnorm_h2(self.h, rows, dim, ptr(x), ptr(gamma), ptr(bound), ptr(y)), "vh_rmsnorm_h2")

    def softmax_rows(self, x, y, rows: int, length: int):
        _ok(lib().vh_softmax_rows(self.h, rows, length, ptr(x), ptr(y)), "vh_softmax_rows")

    def rope_bhld(self, x, bh: int, length: int, dim_head: int = 64):
        _ok(lib().vh_rope_bhld(self.h, bh, length, dim_head, ptr(x)), "vh_rope_bhld")

    def geglu(self, x, y, rows: int, width: int):
        _ok(lib().vh_geglu(self.h, rows, width, ptr(x), ptr(y)), "vh_geglu")

    def residual_add(self, x, r, n: int):
        _ok(lib().vh_residual_add(self.h, n, ptr(x), ptr(r)), "vh_residual_add")

    def gemm(self, A, W, C, M: int, N: int, K: int, bias=None, epilogue: int = EPI_STORE,
             lda: int | None = None, ldw: int | None = None, ldc: int | None = None):
        _ok(lib().vh_gemm(self.h, M, N, K, ptr(A), lda or K, ptr(W), ldw or K,
                          _opt(bias), ptr(C),
                          ldc or _out_cols(N, epilogue), epilogue), "vh_gemm")

    def gemm_bf16(self, A, Wh, C, M: int, N: int, K: int, ldw: int, bias=None, epilogue: int = EPI_STORE,
                  lda: int | None = None, ldc: int | None = None, flags: int = 0):
        """Wh: bf16 weight copy [N][ldw] (see to_bf16); flags: BF16_A / BF16_C operand types, BF16_STAGED."""
        _ok(lib().vh_gemm_bf16(self.h, M, N, K, ptr(A), lda or K, ptr(Wh), ldw,
                               _opt(bias), ptr(C),
                               ldc or _out_cols(N, epilogue), epilogue, flags), "vh_gemm_bf16")

    @staticmethod
    def split_bytes(N: int, K: int) -> int:
        """Bytes of the bf16 pieces of an N x K weight (see split_weights)."""
        return int(lib().vh_split_bytes(N, K))

    def split_weights(self, W, Ws, N: int, K: int, ldw_in: int | None = None):
        """fp32 W [N][ldw_in] -> its tile-major bf16 pieces Ws (split_bytes(N, K) bytes)."""
        _ok(lib().vh_split_weights(self.h, N, K, ptr(W), ldw_in or K, ptr(Ws)), "vh_split_weights")

    def gemm_split(self, A, Ws, C, M: int, N: int, K: int, bias=None, epilogue: int = EPI_STORE,
                   lda: int | None = None, ldc: int | None = None):
        """fp32-accurate linear on bf16 matrix cores; Ws from split_weights."""
        _ok(lib().vh_gemm_split(self.h, M, N, K, ptr(A), lda or K, ptr(Ws),
                                _opt(bias), ptr(C),
                                ldc or _out_cols(N, epilogue), epilogue), "vh_gemm_split")

    @staticmethod
    def h2_bytes(N: int, K: int) -> int:
        """Bytes of the fp16 pieces of an N x K weight (see split_weights_h2)."""
        return int(lib().vh_h2_bytes(N, K))

    def split_weights_h2(self, W, Wp, N: int, K: int, ldw_in: int | None = None):
        """fp32 W [N][ldw_in] -> max|W| and the tile-major fp16 pieces Wp (h2_bytes(N, K) bytes)."""
        _ok(lib().vh_split_weights_h2(self.h, N, K, ptr(W), ldw_in or K, ptr(Wp)), "vh_split_weights_h2")

    def gemm_h2(self, A, Wp, C, M: int, N: int, K: int, bias=None, epilogue: int = EPI_STORE,
                lda: int | None = None, ldc: int | None = None, a_bound: float = 0.0, a_rows: bool = False):
        """fp32-accurate linear on fp16 matrix cores; Wp from split_weights_h2; a_bound bounds |A| (0: max|A|);
        a_rows: A is given as h2 rows split with a_bound (rmsnorm_h2)."""
        _ok(lib().vh_gemm_h2(self.h, M, N, K, ptr(A), lda or K, float(a_bound), ptr(Wp),
                             _opt(bias), ptr(C),
                             ldc or _out_cols(N, epilogue), epilogue, 1 if a_rows else 0),
            "vh_gemm_h2")

    def gemm_h2_ex(self, A, Wp, C, M: int, N: int, K: int, a_bound, bias=None, epilogue: int = EPI_STORE,
                   lda: int | None = None, ldc: int | None = None, row_norm: bool = False, zero_slot=None,
                   amax=None):
        """gemm_h2 with a device bound a_bound; row_norm: C = op(rms(A) (A Wp^T) + bias) with the RMSNorm gain folded
        into Wp; zero_slot set to 0; amax (residual epilogue) raised to max|C| (see vh_gemm_h2_ex)."""
        _ok(lib().vh_gemm_h2_ex(self.h, M, N, K, ptr(A), lda or K, ptr(a_bound), ptr(Wp), _opt(bias), ptr(C),
                                ldc or _out_cols(N, epilogue), epilogue, 2 if row_norm else 0, _opt(zero_slot),
                                _opt(amax)),
            "vh_gemm_h2_ex")

    def operand_bounds(self, gamma, D: int, out, W=None, N: int = 0, bias=None, square: bool = False):
        """Device bounds out[0..1] of the A operands after an RMSNorm with gain gamma (see vh_operand_bounds)."""
        _ok(lib().vh_operand_bounds(self.h, ptr(gamma), D, _opt(W), N,
                                    _opt(bias), 1 if square else 0, ptr(out)),
            "vh_operand_bounds")

    def to_bf16(self, src, dst, rows: int, cols: int, ld: int):
        _ok(lib().vh_to_bf16(self.h, rows, cols, ptr(src), ptr(dst), ld), "vh_to_bf16")

    def attention(self, qkv, out, sequences: int, length: int, heads: int, rotary: bool = True, out_bf16: bool = False,
                  bf16: bool = False, split: bool = False, h2: bool = False, out_h2: bool = False):
        """bf16: qkv is bf16 and the bf16-MFMA kernel runs; out_bf16: out is bf16; split: fp32 accuracy on the
        bf16 matrix cores (three-piece splits, length > 64); h2: fp32 accuracy on the fp16 matrix cores (two-piece
        splits, scales from max|qkv|, any length); out_h2 (with h2): out as h2 rows scaled from max|qkv|."""
        _ok(lib().vh_attention(self.h, sequences, length, heads, ptr(qkv), ptr(out), int(rotary),
                               _att_flags(out_bf16, bf16, split, h2) | (ATT_OUT_H2 if out_h2 else 0)), "vh_attention")

    def attention_noalloc(self, qkv, out, sequences: int, length: int, heads: int, rotary: bool = True,
                          out_bf16: bool = False, bf16: bool = False, split: bool = False, h2: bool = False) -> int:
        """vh_attention_noalloc (no device allocation; length <= NOALLOC_MAX_LENGTH); returns its status."""
        return lib().vh_attention_noalloc(self.h, sequences, length, heads, ptr(qkv), ptr(out), int(rotary),
                                          _att_flags(out_bf16, bf16, split, h2))

    # -- timing --
    def timing(self, classes: str | None = "*"):
        """Time the named kernel classes (comma list, "*" = all, None = off)."""
        _ok(lib().vh_timing_enable(self.h, classes.encode() if classes else None), "vh_timing_enable")

    def timing_reset(self):
        _ok(lib().vh_timing_reset(self.h), "vh_timing_reset")

    def timing_get(self, name: str) -> tuple[float, int]:
        ms = ctypes.c_double(0.0)
        n = _I64(0)
        if not lib().vh_timing_get(self.h, name.encode(), ctypes.byref(ms), ctypes.byref(n)):
            return 0.0, 0
        return ms.value, n.value


class Model:
    """A VSCNAT01 pack uploaded to the device."""

    def __init__(self, ctx: Context, dims: ModelDims, pack) -> None:
        self.ctx = ctx
        self.dims = dims
        self._cd = to_c(dims)
        self.h = lib().vh_model_load(ctx.h, ctypes.byref(self._cd), ptr(pack), pack.nbytes)
        if not self.h:
            raise NativeError(f"vh_model_load failed: {last_error()}")
        ctx.models.add(self)

    def close(self):
        if self.h:
            lib().vh_model_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # noqa: BLE001
            pass

    def set_precision(self, precision: int):
        _ok(lib().vh_model_set_precision(self.h, precision), "vh_model_set_precision")

    def transformer(self, layer: int, axis: int, x, sequences: int, length: int):
        _ok(lib().vh_transformer(self.ctx.h, self.h, layer, axis, ptr(x), sequences, length), "vh_transformer")

    def stft(self, audio, length: int, source, layout: int = SPEC_REFERENCE):
        _ok(lib().vh_stft(self.ctx.h, self.h, ptr(audio), length, ptr(source), layout), "vh_stft")

    def istft(self, source, mask, length: int, audio, layout: int = SPEC_REFERENCE):
        _ok(lib().vh_istft(self.ctx.h, self.h, ptr(source), ptr(mask), length, ptr(audio), layout), "vh_istft")

    def band_split(self, source, frames: int, out, layout: int = SPEC_REFERENCE):
        _ok(lib().vh_band_split(self.ctx.h, self.h, ptr(source), frames, ptr(out), layout), "vh_band_split")

    def mask_estimate(self, features, frames: int, mask, layout: int = SPEC_REFERENCE):
        _ok(lib().vh_mask_estimate(self.ctx.h, self.h, ptr(features), frames, ptr(mask), layout), "vh_mask_estimate")

    def forward(self, audio, length: int, vocals, instrumental=None):
        _ok(lib().vh_forward(self.ctx.h, self.h, ptr(audio), length, ptr(vocals),
                             _opt(instrumental)), "vh_forward")

    def separate(self, audio, length: int, chunk: int, step: int, batch: int, vocals, instrumental=None):
        _ok(lib().vh_separate(self.ctx.h, self.h, ptr(audio), length, chunk, step, batch, ptr(vocals),
                              _opt(instrumental)), "vh_separate")
