"""Model shapes of the BS-RoFormer separation path.

The reference host fixes its shape at compile time
(native/vocalarc_separation.c:33-57); the HIP provider and this package carry
the same numbers as data so the benchmark configurations (dim 384, 62 bands,
hop 441, GELU-GLU) run through the same kernels.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass, field, replace

MAX_BANDS = 256

# native/vocalarc_separation.c:50-57: 90 contiguous bands, sum 1025 bins.
REFERENCE_BAND_WIDTHS = [2] * 24 + [4] * 36 + [12] * 16 + [24] * 8 + [48] * 4 + [128, 129]

# 62-band split used by the dim-384 configurations (no reference table exists
# for 62 bands): 2x24, 4x12, 12x8, 24x8, 48x8, 128, 129 -> 1025 bins.
BAND_WIDTHS_62 = [2] * 24 + [4] * 12 + [12] * 8 + [24] * 8 + [48] * 8 + [128, 129]


@dataclass(frozen=True)
class ModelDims:
    dim: int = 256
    depth: int = 16
    heads: int = 8
    dim_head: int = 64
    ff_dim: int = 1024
    ffn_glu: bool = False
    gated: bool = True
    mask_hidden: int = 1024
    n_fft: int = 2048
    hop: int = 512
    channels: int = 2
    band_widths: tuple = field(default_factory=lambda: tuple(REFERENCE_BAND_WIDTHS))
    # header field 11 of the VSCNAT01 pack (MODEL_FRAMES, checked by the
    # reference host only; native/vocalarc_separation.c:541)
    model_frames: int = 1722

    @property
    def bands(self) -> int:
        return len(self.band_widths)

    @property
    def freq_bins(self) -> int:
        return self.n_fft // 2 + 1

    @property
    def inner(self) -> int:
        return self.heads * self.dim_head

    @property
    def qkv_dim(self) -> int:
        return 3 * self.inner

    @property
    def ff1_out(self) -> int:
        return 2 * self.ff_dim if self.ffn_glu else self.ff_dim

    def input_dims(self) -> list[int]:
        return [w * self.channels * 2 for w in self.band_widths]

    def frames(self, length: int) -> int:
        return length // self.hop + 1

    def first_frequencies(self) -> list[int]:
        out, f = [], 0
        for w in self.band_widths:
            out.append(f)
            f += w
        return out

    def validate(self) -> None:
        if sum(self.band_widths) != self.freq_bins:
            raise ValueError(f"band widths sum to {sum(self.band_widths)}, expected {self.freq_bins}")
        if self.bands > MAX_BANDS:
            raise ValueError("too many bands")
        if self.dim_head % 4 or self.dim % 4:
            raise ValueError("dim and dim_head must be multiples of 4")

    def with_depth(self, depth: int) -> "ModelDims":
        return replace(self, depth=depth)


# The bundled bs_leap_xe_voc shape (native/assets/manifest.json:9-15,
# native/vocalarc_separation.c:33-46).
REFERENCE_DIMS = ModelDims()

# Benchmark shape: dim 384, 62 bands, hop 441, 8x64 heads, FFN mult 4 with
# GELU-GLU, mask hidden 4*dim, depth 12 for the full model.
CONFIG_DIMS = ModelDims(dim=384, depth=12, heads=8, dim_head=64, ff_dim=1536, ffn_glu=True,
                        gated=True, mask_hidden=1536, n_fft=2048, hop=441, channels=2,
                        band_widths=tuple(BAND_WIDTHS_62), model_frames=0)


class CDims(ctypes.Structure):
    """C mirror of the dims struct shared by the oracle (or_dims) and the HIP
    library (vh_dims); both have this exact field order."""

    _fields_ = [
        ("dim", ctypes.c_int), ("depth", ctypes.c_int), ("bands", ctypes.c_int),
        ("heads", ctypes.c_int), ("dim_head", ctypes.c_int), ("ff_dim", ctypes.c_int),
        ("ffn_glu", ctypes.c_int), ("gated", ctypes.c_int), ("mask_hidden", ctypes.c_int),
        ("n_fft", ctypes.c_int), ("hop", ctypes.c_int), ("channels", ctypes.c_int),
        ("band_widths", ctypes.c_int * MAX_BANDS),
    ]


def to_c(d: ModelDims) -> CDims:
    d.validate()
    c = CDims()
    c.dim, c.depth, c.bands = d.dim, d.depth, d.bands
    c.heads, c.dim_head, c.ff_dim = d.heads, d.dim_head, d.ff_dim
    c.ffn_glu, c.gated, c.mask_hidden = int(d.ffn_glu), int(d.gated), d.mask_hidden
    c.n_fft, c.hop, c.channels = d.n_fft, d.hop, d.channels
    for i, w in enumerate(d.band_widths):
        c.band_widths[i] = w
    return c
