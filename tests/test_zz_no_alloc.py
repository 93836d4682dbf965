"""The zero-allocation routed decode (exl3_moe_decode_noalloc) through the C
ABI: two calls in a row on the library's fixed scratch, the second with a
smaller layer and fewer rows, each bitwise equal to exl3_moe_decode_routed on
a caller-provided scratch and within the bar of the oracle."""

from __future__ import annotations

import numpy as np
import pytest

from dsv4_carve_amd import synth
from tests.helpers import assert_close, to_dev
from tests.test_gpu_moe import Layer

pytestmark = pytest.mark.gpu


def _call(lib_fn, layer, x, ids, w, out, extra):
    from dsv4_carve_amd import _lib, ops
    import torch

    t = layer.tables
    args = [x.data_ptr(), 0, out.data_ptr(), 2, x.shape[0], layer.H, layer.I, layer.E, ids.shape[1],
            *[int(t[k].data_ptr()) for k in ops.MOE_TABLE_KEYS],
            ids.data_ptr(), 0, w.data_ptr(), 2, None, 0,
            layer.ebits.data_ptr(), 0, layer.mask, ops.CB_MCG, 10.0, *extra,
            int(torch.cuda.current_stream().cuda_stream)]
    _lib.check(lib_fn(*args))


def test_noalloc_matches_scratch_entry_point(dev):
    import torch
    from dsv4_carve_amd import _lib, ops

    L = _lib.load()
    assert L.exl3_moe_noalloc_scratch_bytes() == 128 << 20
    big = Layer(dev, 24, 1024, 768, [3, 2] * 12, seed=71)
    small = Layer(dev, 12, 512, 256, [2, 3, 4] * 4, seed=72)
    for layer, m, topk in ((big, 11, 8), (small, 3, 6)):
        print(f"noalloc H={layer.H} I={layer.I} m={m} top{topk}", flush=True)
        ids, w = synth.routing(m, layer.E, topk, seed=700 + m)
        x16 = synth.activations(m, layer.H, seed=701 + m)
        x, idd, wd = to_dev(x16, dev), to_dev(ids, dev), to_dev(w, dev)
        scratch = torch.zeros(ops.moe_scratch_bytes(layer.H, layer.I, topk), dtype=torch.uint8, device=dev)
        want = torch.empty((m, layer.H), dtype=torch.float32, device=dev)
        got = torch.full((m, layer.H), float("nan"), dtype=torch.float32, device=dev)
        _call(L.exl3_moe_decode_routed, layer, x, idd, wd, want, [scratch.data_ptr(), scratch.numel()])
        _call(L.exl3_moe_decode_noalloc, layer, x, idd, wd, got, [])
        torch.cuda.synchronize()
        assert torch.equal(got, want), "the fixed-scratch call differs from the caller-scratch call"
        assert_close(got.cpu().numpy(), layer.ref(x16, ids, w), what=f"noalloc H={layer.H} m={m}")


def test_noalloc_rejects_oversized_layer(dev):
    import torch
    from dsv4_carve_amd import _lib, ops

    L = _lib.load()
    assert ops.moe_scratch_bytes(8192, 4096, 9) > L.exl3_moe_noalloc_scratch_bytes()
    x = torch.zeros((1, 8192), dtype=torch.float16, device=dev)
    out = torch.empty((1, 8192), dtype=torch.float32, device=dev)
    ids = torch.zeros((1, 9), dtype=torch.int32, device=dev)
    w = torch.zeros((1, 9), dtype=torch.float32, device=dev)
    tab = torch.zeros(1, dtype=torch.int64, device=dev)
    rc = L.exl3_moe_decode_noalloc(x.data_ptr(), 0, out.data_ptr(), 2, 1, 8192, 4096, 1, 9,
                                   *([tab.data_ptr()] * 9), ids.data_ptr(), 0, w.data_ptr(), 2, None, 0,
                                   None, 2, 0, ops.CB_MCG, 10.0, int(torch.cuda.current_stream().cuda_stream))
    assert rc < 0 and b"128 MiB" in L.exl3_last_error()


def test_noalloc_error_word(dev):
    """The fixed scratch's error word through exl3_moe_noalloc_error: a call
    whose bits_mask lacks a routed expert's width reports ERR_WIDTH (those
    experts contribute zero, every launch completes); clearing resets it; a
    full reset of the control words leaves the next call correct."""
    import torch
    from dsv4_carve_amd import _lib, ops

    L = _lib.load()
    stream = int(torch.cuda.current_stream().cuda_stream)
    bits = [3, 2, 5, 3, 2, 5, 3, 2]                  # experts 2 and 5 are 5-bit
    layer = Layer(dev, 8, 512, 256, bits, seed=41)
    m, topk = 6, 4
    ids, w = synth.routing(m, 8, topk, seed=42)
    x16 = synth.activations(m, 512, seed=43)
    keep = np.where(np.isin(ids, [2, 5]), 0.0, w).astype(np.float32)
    assert (keep != w).any(), "the route must reach a 5-bit expert"
    x, idd, wd = to_dev(x16, dev), to_dev(ids, dev), to_dev(w, dev)
    out = torch.empty((m, 512), dtype=torch.float32, device=dev)
    _lib.check(L.exl3_moe_noalloc_error(2, stream))             # start from zeroed control words
    lacking = (1 << 2) | (1 << 3)                                # the launch covers 2 and 3 bits only
    layer_mask, layer.mask = layer.mask, lacking
    print("noalloc error word: unlisted 5-bit experts", flush=True)
    _call(L.exl3_moe_decode_noalloc, layer, x, idd, wd, out, [])
    layer.mask = layer_mask
    assert _lib.check(L.exl3_moe_noalloc_error(0, stream)) == ops.ERR_WIDTH
    assert_close(out.cpu().numpy(), layer.ref(x16, ids, keep), what="noalloc: unlisted width dropped")
    assert _lib.check(L.exl3_moe_noalloc_error(1, stream)) == ops.ERR_WIDTH   # read, then clear
    assert _lib.check(L.exl3_moe_noalloc_error(0, stream)) == 0
    print("noalloc error word: full mask after a reset", flush=True)
    _lib.check(L.exl3_moe_noalloc_error(2, stream))
    _call(L.exl3_moe_decode_noalloc, layer, x, idd, wd, out, [])
    assert _lib.check(L.exl3_moe_noalloc_error(0, stream)) == 0
    assert_close(out.cpu().numpy(), layer.ref(x16, ids, w), what="noalloc: full mask after the reset")
    assert L.exl3_moe_noalloc_error(3, stream) < 0
