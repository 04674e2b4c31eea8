"""vh_attention_noalloc (no device allocation: its scratch is one fixed
device array per GPU) against vh_attention, through the C-ABI.

Both entry points run the same kernels on the same host-built rotary table
and the same device-computed bound, so the outputs must agree bit for bit.
Two calls in a row on the shared scratch, the second with a smaller input,
for each kernel family (fp32 MFMA, fp16 two-piece, three-piece bf16, bf16);
the no-allocation calls come first in a fresh context, so nothing they use
was left behind by the allocating entry point.
"""

import numpy as np
import pytest

from helpers import gpu_available

pytestmark = pytest.mark.gpu

if gpu_available():
    import torch
    from vocalarc_hip import native

MODES = {
    "fp32": {},
    "h2": {"h2": True},
    "split": {"split": True},
    "bf16": {"bf16": True, "out_bf16": True},
}


@pytest.mark.parametrize("mode", list(MODES))
def test_noalloc_matches_attention(mode):
    if not gpu_available():
        pytest.skip("no GPU")
    kw = MODES[mode]
    H = 8
    # (S, L) of two calls in a row; the second is smaller.  The three-piece
    # split kernel serves lengths above 64 only.
    shapes = [(4, 801), (3, 130)] if mode == "split" else [(4, 801), (20, 62)]
    g = torch.Generator(device="cuda:0")
    g.manual_seed(11)
    inputs = []
    for S, L in shapes:
        qkv = torch.randn(S * L, 3 * H * 64, device="cuda:0", generator=g)
        inputs.append(qkv.to(torch.bfloat16) if kw.get("bf16") else qkv)
    odt = torch.bfloat16 if kw.get("out_bf16") else torch.float32

    ctx = native.Context()
    try:
        got = []
        for (S, L), qkv in zip(shapes, inputs):
            out = torch.empty(S * L, H * 64, device="cuda:0", dtype=odt)
            assert ctx.attention_noalloc(qkv, out, S, L, H, rotary=True, **kw) == 1, native.last_error()
            ctx.sync()
            got.append(out.clone())
        for (S, L), qkv, o in zip(shapes, inputs, got):
            ref = torch.empty(S * L, H * 64, device="cuda:0", dtype=odt)
            ctx.attention(qkv, ref, S, L, H, rotary=True, **kw)
            ctx.sync()
            assert torch.equal(o, ref), f"{mode} S={S} L={L}"
        print(f"no-allocation attention ({mode}): {shapes} bit-identical to vh_attention")
    finally:
        ctx.close()


def test_noalloc_rejects_beyond_scratch():
    """A length past the scratch's maximum fails with an error before any
    launch (a host-side check)."""
    if not gpu_available():
        pytest.skip("no GPU")
    ctx = native.Context()
    try:
        L = native.NOALLOC_MAX_LENGTH + 1
        qkv = torch.zeros(L, 3 * 64, device="cuda:0")
        out = torch.empty(L, 64, device="cuda:0")
        assert ctx.attention_noalloc(qkv, out, 1, L, 1) == 0
        assert "exceeds" in native.last_error()
    finally:
        ctx.close()


@pytest.mark.parametrize("mode", ["fp32", "h2"])
def test_noalloc_graph_capture(mode):
    """vh_attention_noalloc with the rotary table, captured in a HIP graph on
    a capturing stream (no copy, synchronisation or allocation may happen in
    the call), replayed four times with new inputs in the same buffer and
    eager work between the replays: every replay bit-identical to
    vh_attention on that input.  In the h2 mode the third input is scaled
    far outside the two-piece kernels' range (max|qkv| ~ 1e25), so the
    replays exercise the choice the kernels make on the device between the
    two-piece products and those without piece scales (v scaled, as in
    test_attention_h2_outside_scale_range)."""
    if not gpu_available():
        pytest.skip("no GPU")
    kw = MODES[mode]
    S, L, H = 3, 801, 8
    g = torch.Generator(device="cuda:0")
    g.manual_seed(12)
    # the v columns scaled (q and k of ~1e25 would overflow the scores of
    # every kernel): the output, a convex combination of v rows, stays finite
    scales = [1.0, 0.25, 1e25, 1.0] if mode == "h2" else [1.0, 0.25, 3.0, 1.0]
    datas = []
    for sc in scales:
        d = torch.randn(S * L, 3 * H * 64, device="cuda:0", generator=g)
        d[:, 2 * H * 64:] *= sc
        datas.append(d)
    qkv = torch.empty_like(datas[0])
    out = torch.empty(S * L, H * 64, device="cuda:0")

    ctx = native.Context()
    try:
        qkv.copy_(datas[0])
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        cap = torch.cuda.Stream()
        with torch.cuda.graph(graph, stream=cap):
            ctx.set_stream(torch.cuda.current_stream().cuda_stream)
            status = ctx.attention_noalloc(qkv, out, S, L, H, rotary=True, **kw)
        ctx.set_stream(torch.cuda.current_stream().cuda_stream)
        assert status == 1, native.last_error()
        for i, d in enumerate(datas):
            qkv.copy_(d)
            junk = torch.randn(1 << 20, device="cuda:0", generator=g).sum()  # eager work between replays
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            got = out.clone()
            ref = torch.empty_like(out)
            ctx.attention(qkv, ref, S, L, H, rotary=True, **kw)
            ctx.sync()
            assert torch.isfinite(got).all(), f"{mode} replay {i}"
            assert torch.equal(got, ref), f"{mode} replay {i} (input scale {scales[i]:g})"
            del junk
        print(f"no-allocation attention ({mode}) in a graph: {len(datas)} replays bit-identical to vh_attention")
    finally:
        ctx.close()
