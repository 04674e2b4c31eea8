"""VSCNAT01 model packs.

Layout (native/vocalarc_separation.c:528-589): 8-byte magic "VSCNAT01", 14
little-endian u32 header fields, then every tensor as a u64 element count
followed by its float32 data.  Matrices are stored in the reference's packed
layout: full 32-wide output tiles [in][32], then the out%32 tail [in][tail]
(native/vocalarc_separation.c:428-457).

Tensor order: per layer, per axis (time, band): gamma, qkv, gate weight, gate
bias, out, ff gamma, ff1 weight, ff1 bias, ff2 weight, ff2 bias; per band:
gamma, weight, bias; final gamma; per band: mask first weight, first bias,
second weight, second bias.  With the reference dimensions this is exactly the
bundled model's format (267,386,408 bytes).
"""

from __future__ import annotations

import struct
from dataclasses import dataclass

import numpy as np

from .dims import ModelDims

MAGIC = b"VSCNAT01"
HEADER_BYTES = 64


@dataclass(frozen=True)
class TensorSpec:
    name: str
    kind: str          # "matrix" | "bias" | "gamma"
    out: int           # rows of the logical [out][in] matrix (or vector length)
    inp: int = 0       # columns (0 for vectors)

    @property
    def count(self) -> int:
        return self.out * self.inp if self.kind == "matrix" else self.out


def tensor_specs(d: ModelDims) -> list[TensorSpec]:
    specs: list[TensorSpec] = []
    for layer in range(d.depth):
        for axis in range(2):
            p = f"layers.{layer}.{axis}."
            specs += [
                TensorSpec(p + "gamma", "gamma", d.dim),
                TensorSpec(p + "qkv", "matrix", d.qkv_dim, d.dim),
                TensorSpec(p + "gate_weight", "matrix", d.heads, d.dim),
                TensorSpec(p + "gate_bias", "bias", d.heads),
                TensorSpec(p + "out_weight", "matrix", d.dim, d.inner),
                TensorSpec(p + "ff_gamma", "gamma", d.dim),
                TensorSpec(p + "ff1_weight", "matrix", d.ff1_out, d.dim),
                TensorSpec(p + "ff1_bias", "bias", d.ff1_out),
                TensorSpec(p + "ff2_weight", "matrix", d.dim, d.ff_dim),
                TensorSpec(p + "ff2_bias", "bias", d.dim),
            ]
    for b, in_dim in enumerate(d.input_dims()):
        specs += [
            TensorSpec(f"bands.{b}.gamma", "gamma", in_dim),
            TensorSpec(f"bands.{b}.weight", "matrix", d.dim, in_dim),
            TensorSpec(f"bands.{b}.bias", "bias", d.dim),
        ]
    specs.append(TensorSpec("final_gamma", "gamma", d.dim))
    for b, in_dim in enumerate(d.input_dims()):
        specs += [
            TensorSpec(f"masks.{b}.first_weight", "matrix", d.mask_hidden, d.dim),
            TensorSpec(f"masks.{b}.first_bias", "bias", d.mask_hidden),
            TensorSpec(f"masks.{b}.second_weight", "matrix", 2 * in_dim, d.mask_hidden),
            TensorSpec(f"masks.{b}.second_bias", "bias", 2 * in_dim),
        ]
    return specs


def pack_bytes(d: ModelDims) -> int:
    return HEADER_BYTES + sum(8 + 4 * s.count for s in tensor_specs(d))


def header(d: ModelDims) -> bytes:
    fields = [1, d.dim, d.depth, d.bands, d.heads, d.dim_head, d.freq_bins, d.channels,
              d.n_fft, d.hop, d.n_fft, d.model_frames, 0, 0]
    return MAGIC + struct.pack("<14I", *fields)


def pack_matrix(w: np.ndarray) -> np.ndarray:
    """[out][in] -> packed layout (32-wide output tiles, then the tail)."""
    out, inp = w.shape
    full = (out // 32) * 32
    parts = []
    if full:
        parts.append(w[:full].reshape(full // 32, 32, inp).transpose(0, 2, 1).reshape(-1))
    if out > full:
        parts.append(w[full:].T.reshape(-1))
    return np.ascontiguousarray(np.concatenate(parts).astype(np.float32))


def unpack_matrix(p: np.ndarray, out: int, inp: int) -> np.ndarray:
    full = (out // 32) * 32
    w = np.empty((out, inp), np.float32)
    if full:
        w[:full] = p[: full * inp].reshape(full // 32, inp, 32).transpose(0, 2, 1).reshape(full, inp)
    if out > full:
        w[full:] = p[full * inp:].reshape(inp, out - full).T
    return w


def synthetic_pack(d: ModelDims, seed: int, std: float = 0.02) -> np.ndarray:
    """Seeded random-init pack as a uint8 array.

    Matrices and biases are N(0, std), gammas N(1, std), drawn tensor by tensor
    in pack order from numpy's PCG64 (default_rng(seed)).  Matrices are drawn
    directly in packed order: the entries are i.i.d., so the distribution is
    the same as drawing [out][in] and packing.
    """
    d.validate()
    rng = np.random.default_rng(seed)
    specs = tensor_specs(d)
    total = pack_bytes(d)
    blob = np.zeros(total, np.uint8)
    blob[:HEADER_BYTES] = np.frombuffer(header(d), np.uint8)
    off = HEADER_BYTES
    for s in specs:
        blob[off:off + 8] = np.frombuffer(struct.pack("<Q", s.count), np.uint8)
        off += 8
        vals = rng.standard_normal(s.count, dtype=np.float32) * np.float32(std)
        if s.kind == "gamma":
            vals += np.float32(1.0)
        blob[off:off + 4 * s.count] = vals.view(np.uint8)
        off += 4 * s.count
    assert off == total
    return blob


def tensor_views(d: ModelDims, blob: np.ndarray) -> dict[str, np.ndarray]:
    """Name -> float32 view (packed order) into a pack blob."""
    out: dict[str, np.ndarray] = {}
    off = HEADER_BYTES
    for s in tensor_specs(d):
        (count,) = struct.unpack_from("<Q", blob, off)
        if count != s.count:
            raise ValueError(f"{s.name}: count {count} != {s.count}")
        off += 8
        out[s.name] = blob[off:off + 4 * s.count].view(np.float32)
        off += 4 * s.count
    return out


def write_pack(path, blob: np.ndarray) -> None:
    with open(path, "wb") as f:
        f.write(blob.tobytes())
