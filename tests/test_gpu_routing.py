"""Routing glue on the device: the routed-expert kernels fed the router's own
tensors (int64 or int32 global ids, bf16/fp16/fp32 weights, an int64
global -> local expert map) give bitwise the result of feeding them
map_topk_to_local's int32 local ids and fp32 weights, on both decode
schedules and on the prefill path, and the plugin's apply returns the same
through either hand-off.  The host mapping is the reference's rule
(recipe-lna/vllm_exl3_exl3.py.lna:963-985; its own behaviour is pinned in
tests/test_host.py), so bitwise equality pins the on-device mapping; one case
per path also checks against the oracle."""

from __future__ import annotations

import numpy as np
import pytest

from dsv4_carve_amd import synth
from tests.helpers import assert_close, to_dev
from tests.test_gpu_moe import LIMIT, Layer, moe_path

pytestmark = pytest.mark.gpu

TOPK = 6


@pytest.fixture(scope="module")
def layer(dev):
    bits = [3, 2, 4, 3, 2, 2, 3, 4, 2, 3, 3, 2]
    return Layer(dev, 12, 512, 256, bits, seed=23)


def routed_case(rows, E, n_global, seed):
    """A global -> local map placing E local experts among n_global (others
    -1, one entry pointing past the local range), and ids mixing local,
    remote, negative and past-the-map values."""
    rng = np.random.default_rng(seed)
    emap = np.full(n_global, -1, np.int64)
    local_at = rng.choice(n_global, E, replace=False)
    emap[local_at] = rng.permutation(E)
    spare = [g for g in range(n_global) if emap[g] < 0]
    emap[spare[0]] = E + 3                      # maps outside [0, E): skipped
    ids = rng.integers(-2, n_global + 3, size=(rows, TOPK)).astype(np.int64)
    pick = rng.random((rows, TOPK)) < 0.6
    ids[pick] = rng.choice(local_at, int(pick.sum()))
    ids[0, 0] = spare[0]
    logits = rng.standard_normal((rows, TOPK))
    w = (np.exp(logits) / np.exp(logits).sum(axis=1, keepdims=True)).astype(np.float32)   # router softmax
    return emap, ids, w


def _mapped(ids_t, E, emap_t):
    import torch
    from dsv4_carve_amd import vllm_exl3 as V

    return V.map_topk_to_local(ids_t, E, emap_t).reshape(ids_t.shape).to(torch.int32).contiguous()


def _run(layer, fn, x, ids, w, emap=None):
    import torch

    out = torch.empty(x.shape, dtype=torch.float32, device=x.device)
    fn(x, out, layer.tables, ids, w, intermediate=layer.I, expert_bits=layer.ebits, bits_mask=layer.mask,
       swiglu_limit=LIMIT, expert_map=emap)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("path", ["ticket", "phased"])
@pytest.mark.parametrize("rows", [1, 5, 16])
@pytest.mark.parametrize("wdt", ["bfloat16", "float16", "float32"])
def test_decode_routed_equals_host_mapping(dev, layer, path, rows, wdt):
    import torch
    from dsv4_carve_amd import ops

    print(f"routed decode path={path} rows={rows} w={wdt}", flush=True)
    emap, ids, w = routed_case(rows, layer.E, 40, seed=rows)
    x = to_dev(synth.activations(rows, layer.H, seed=500 + rows), dev)
    ids_t, emap_t = to_dev(ids, dev), to_dev(emap, dev)
    w_t = to_dev(w, dev).to(getattr(torch, wdt))
    with moe_path(path):
        want = _run(layer, ops.moe_decode, x, _mapped(ids_t, layer.E, emap_t), w_t.float())
        got = _run(layer, ops.moe_decode, x, ids_t, w_t, emap_t)
        got32 = _run(layer, ops.moe_decode, x, ids_t.to(torch.int32), w_t, emap_t)
    assert torch.equal(got, want) and torch.equal(got32, want), "on-device mapping differs from the host mapping"
    if rows == 5 and wdt == "float32":
        local = _mapped(ids_t, layer.E, emap_t).cpu().numpy()
        assert_close(got.cpu().numpy(), layer.ref(x.cpu().numpy(), local, w), what=f"routed {path}")


def test_decode_routed_without_map_takes_local_ids(dev, layer):
    import torch
    from dsv4_carve_amd import ops

    rows = 7
    ids = np.tile(np.array([-1, 3, layer.E, 5, 10 ** 6, 11], np.int64), (rows, 1))
    w = synth.routing(rows, layer.E, TOPK, seed=3)[1]
    x = to_dev(synth.activations(rows, layer.H, seed=510), dev)
    ids_t, w_h = to_dev(ids, dev), to_dev(w, dev).half()
    want = _run(layer, ops.moe_decode, x, _mapped(ids_t, layer.E, None), w_h.float())
    got = _run(layer, ops.moe_decode, x, ids_t, w_h)
    assert torch.equal(got, want), "local int64 ids / fp16 weights differ from the host-mapped call"


@pytest.mark.parametrize("rows", [40, 97])
def test_prefill_routed_equals_host_mapping(dev, layer, rows):
    import torch
    from dsv4_carve_amd import ops

    print(f"routed prefill rows={rows}", flush=True)
    emap, ids, w = routed_case(rows, layer.E, 33, seed=100 + rows)
    x = to_dev(synth.activations(rows, layer.H, seed=520 + rows), dev)
    ids_t, emap_t = to_dev(ids, dev), to_dev(emap, dev)
    w_t = to_dev(w, dev).to(torch.bfloat16)
    want = _run(layer, ops.moe_prefill, x, _mapped(ids_t, layer.E, emap_t), w_t.float())
    got = _run(layer, ops.moe_prefill, x, ids_t, w_t, emap_t)
    assert torch.equal(got, want), "on-device mapping differs from the host mapping (prefill)"
    if rows == 40:
        local = _mapped(ids_t, layer.E, emap_t).cpu().numpy()
        assert_close(got.cpu().numpy(), layer.ref(x.cpu().numpy(), local, w_t.float().cpu().numpy()),
                     what="routed prefill")


def test_routed_argument_errors(dev, layer):
    import torch
    from dsv4_carve_amd import ops

    x = to_dev(synth.activations(2, layer.H, seed=530), dev)
    ids = torch.zeros((2, TOPK), dtype=torch.int64, device=dev)
    w = torch.ones((2, TOPK), dtype=torch.float32, device=dev)
    with pytest.raises(RuntimeError, match="int32/int64"):
        _run(layer, ops.moe_decode, x, ids.to(torch.int16), w)
    with pytest.raises(RuntimeError, match="fp16/bf16/fp32"):
        _run(layer, ops.moe_decode, x, ids, w.double())
    with pytest.raises(RuntimeError, match="expert_map"):
        _run(layer, ops.moe_decode, x, ids, w, torch.zeros(4, dtype=torch.int32, device=dev))
    with pytest.raises(RuntimeError, match="expert_map"):
        _run(layer, ops.moe_decode, x, ids, w, torch.zeros(4, dtype=torch.int64))


@pytest.mark.parametrize("rows", [3, 30, 40])
def test_plugin_apply_with_router_tensors(dev, monkeypatch, rows):
    """apply_exl3_experts with int32 global ids, bf16 weights and an expert
    map equals the unique-expert loop (which maps on the host)."""
    import torch
    from dsv4_carve_amd import vllm_exl3 as V
    from tests.test_gpu_plugin import Experts

    monkeypatch.setenv("VLLM_EXL3_MOE_STRICT", "2")
    monkeypatch.setenv("VLLM_EXL3_MOE_KERNEL", "lna2")
    E = 8
    ex = Experts(dev, E, 256, 512, [3] * E, seed=61)
    V.build_exl3_fused_state(ex.layer, ex.layer._exl3_inners)
    assert ex.layer._exl3_lna_ready, ex.layer._exl3_lna_error
    emap, ids, w = routed_case(rows, E, 20, seed=200 + rows)
    ex.layer.expert_map = to_dev(emap, dev)
    x = to_dev(synth.activations(rows, 256, seed=540 + rows), dev).to(torch.bfloat16)
    ids_t = to_dev(ids, dev).to(torch.int32)
    w_t = to_dev(w, dev).to(torch.bfloat16)
    fused = V.apply_exl3_experts(x, ids_t, w_t, ex.layer)
    assert ex.layer._exl3_last_apply == ("lna2" if rows <= V.lna2_max_rows() else "prefill")
    monkeypatch.setenv("VLLM_EXL3_MOE_KERNEL", "loop")
    loop = V.apply_exl3_experts(x, ids_t.long(), w_t, ex.layer)
    assert ex.layer._exl3_last_apply == "loop"
    assert_close(fused.float().cpu().numpy(), loop.float().cpu().numpy(), max_abs=3e-2, rel=4e-3,
                 what=f"plugin routed rows={rows}")
