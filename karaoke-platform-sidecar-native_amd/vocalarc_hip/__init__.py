"""Host-side helpers of the MI355X VocalArc provider: model shapes, VSCNAT01
packs, seeded audio, and the ctypes binding of lib/libvocalarc_hip.so."""

from .dims import BAND_WIDTHS_62, CONFIG_DIMS, REFERENCE_BAND_WIDTHS, REFERENCE_DIMS, ModelDims  # noqa: F401
