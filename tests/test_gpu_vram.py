"""VRAM gate: the shared scratch is per device, not per layer.

The reference's gate (recipe-lna/lna2/gate_vram.py:18-57) prepares every layer
and then measures the scratch bytes held per device.  Here 43 routed-MoE
layers (the DSV4 decode block count; hidden 4096, intermediate 2048, eight
3-bit experts each, the weights of one seeded set loaded into every layer) and
43 dense shared-expert modules (gate_up 4096 -> 2 x 2048 and down 2048 -> 4096,
6-bit) are built the way vLLM builds them: create_weights, the per-tensor
weight loaders, process_weights_after_loading.  After all of them, and after
a decode call, a prefill call and a dense forward at every row count the
decode kernels take, the library holds exactly one decode scratch, one
prefill scratch and one dense GEMV scratch on the device, of the sizes the
sizing functions give for the largest shape, whatever the layer count.  The
bytes are printed; the fixed array of the zero-allocation entry point comes
on top of them only in a process that calls it."""

from __future__ import annotations

import numpy as np
import pytest

from dsv4_carve_amd import synth
from tests.helpers import assert_close, to_dev

pytestmark = pytest.mark.gpu

LAYERS = 43
H, I, E, BITS, TOPK = 4096, 2048, 8, 3, 8
SHARED_BITS = 6
LIMIT = 10.0


def _moe_layer(dev, experts, index):
    import torch
    from dsv4_carve_amd import vllm_exl3 as V

    class Moe:
        swiglu_limit = LIMIT

    layer = torch.nn.Module()
    layer.prefix = f"model.layers.{index}.ffn.experts"
    layer._exl3_topk = TOPK
    meth = V.Exl3MoEMethod(Moe(), bits=BITS)
    meth.create_weights(layer, E, H, I)
    mcg = torch.tensor([V.MCG_MARKER_SIGNED_INT32], dtype=torch.int32)
    for e, ex in enumerate(experts):
        for shard, proj in (("w1", "gate"), ("w3", "up"), ("w2", "down")):
            for suffix in ("trellis", "suh", "svh"):
                p = getattr(layer, ("w13_" if shard != "w2" else "w2_") + suffix)
                p.weight_loader(p, ex[proj][suffix], f"experts.{e}.{shard}.{suffix}", shard, e)
            p = layer.w13_mcg if shard != "w2" else layer.w2_mcg
            p.weight_loader(p, mcg, f"experts.{e}.{shard}.mcg", shard, e)
    layer.to(dev)
    meth.process_weights_after_loading(layer)
    assert layer._exl3_lna_ready, layer._exl3_lna_error
    return layer, meth


def _dense_module(dev, prefix, k, shards, host):
    import torch
    from dsv4_carve_amd import vllm_exl3 as V

    layer = torch.nn.Module()
    layer.prefix = prefix
    meth = V.Exl3LinearMethod(None, bits=SHARED_BITS)
    with torch.device(dev):
        meth.create_weights(layer, k, list(shards), k, sum(shards), params_dtype=torch.bfloat16)
    for j, h in enumerate(host):
        for suffix in ("trellis", "suh", "svh"):
            p = getattr(layer, suffix)
            p.weight_loader(p, h[suffix], j)
        layer.mcg.weight_loader(layer.mcg, torch.tensor(V.MCG_MARKER_SIGNED_INT32, dtype=torch.int32), j)
    meth.process_weights_after_loading(layer)
    return layer, meth


def test_scratch_is_per_device_not_per_layer(dev, monkeypatch):
    import torch
    from dsv4_carve_amd import _lib, ops
    from dsv4_carve_amd import vllm_exl3 as V

    monkeypatch.setenv("VLLM_EXL3_MOE_KERNEL", "lna2")
    monkeypatch.setenv("VLLM_EXL3_MOE_STRICT", "2")
    monkeypatch.setenv("LNA_EXL3_DENSE_GROUP", "0")
    monkeypatch.setattr(ops, "SCRATCH", ops._ScratchPool())       # this process's earlier tests aside
    host_experts = []
    for e in range(E):
        ex = synth.expert(e, H, I, BITS, seed=500)
        host_experts.append({p: {k: torch.from_numpy(ex[p][k]) for k in ("trellis", "suh", "svh")}
                             for p in ("gate", "up", "down")})
    gu_host = [synth.dense(H, I, SHARED_BITS, seed=510 + j) for j in range(2)]
    dn_host = [synth.dense(I, H, SHARED_BITS, seed=520)]
    gu_dev = [{k: to_dev(h[k], dev) for k in ("trellis", "suh", "svh")} for h in gu_host]
    dn_dev = [{k: to_dev(h[k], dev) for k in ("trellis", "suh", "svh")} for h in dn_host]

    moe, dense, after_first = [], [], None
    for i in range(LAYERS):
        moe.append(_moe_layer(dev, host_experts, i))
        dense.append((_dense_module(dev, f"model.layers.{i}.ffn.shared_experts.gate_up_proj", H, [I, I], gu_dev),
                      _dense_module(dev, f"model.layers.{i}.ffn.shared_experts.down_proj", I, [H], dn_dev)))
        if i == 0:
            after_first = ops.SCRATCH.resident_bytes()
    print(f"{LAYERS} routed layers + {2 * LAYERS} dense modules prepared", flush=True)
    assert ops.SCRATCH.resident_bytes() == after_first, "scratch grew with the layer count"

    # one call of every kind on the last layer, at every row count the decode
    # kernels take, and the 512-token prefill
    layer, meth = moe[-1]
    for m in (1, 16, V.lna2_max_rows(), 512):
        ids, w = synth.routing(m, E, TOPK, seed=530 + m)
        x = to_dev(synth.activations(m, H, seed=531 + m), dev)
        y = meth.apply(layer, x, to_dev(w, dev), to_dev(ids.astype(np.int64), dev))
        assert layer._exl3_last_apply == ("prefill" if m > V.lna2_max_rows() else "lna2")
        assert torch.isfinite(y.float()).all()
    (gu, gu_meth), (dn, dn_meth) = dense[-1]
    for m in range(1, V.AUTO_RECONSTRUCT_THRESHOLD + 1):
        xg = to_dev(synth.activations(m, H, seed=540 + m), dev)
        hidden = gu_meth.apply(gu, xg)
        dn_meth.apply(dn, hidden[:, :I].contiguous())
    torch.cuda.synchronize()
    assert ops.moe_scratch_errors(dev) == {"moe": 0, "moe_prefill": 0}

    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    held = {purpose: int(buf.numel()) for (d, purpose), buf in ops.SCRATCH._bufs.items() if d == idx}
    want_decode = ops.moe_scratch_bytes(H, I, V.LNA2_MAX_TOPK, rows=V.lna2_max_rows())
    want_prefill = ops.moe_prefill_scratch_bytes(512, H, I, TOPK, E)
    want_gemm = max(ops._lib.check(_lib.load().exl3_gemm_scratch_bytes(m, k, n))
                    for m in range(1, V.AUTO_RECONSTRUCT_THRESHOLD + 1) for k, n in ((H, I), (I, H)))
    noalloc = int(_lib.load().exl3_moe_noalloc_scratch_bytes())
    mib = lambda b: f"{b / 2 ** 20:.1f} MiB"
    print(f"scratch per device: decode {mib(held.get('moe', 0))}, prefill {mib(held.get('moe_prefill', 0))}, "
          f"dense GEMV {mib(held.get('gemm', 0))}; zero-allocation entry's fixed array {mib(noalloc)} "
          f"(only where exl3_moe_decode_noalloc is called)", flush=True)
    assert set(held) == {"moe", "moe_prefill", "gemm"}, held
    assert held["moe"] == want_decode
    assert held["moe_prefill"] == max(want_prefill, 256)
    assert held["gemm"] == max(want_gemm, 256)
    assert sum(held.values()) < 1 << 30


def test_decode_scratch_serves_a_layer_like_the_checked_ones(dev, monkeypatch):
    """One more routed layer of the same shape, built after the others, reuses
    the device's scratch and matches the loop on it."""
    import torch
    from dsv4_carve_amd import ops
    from dsv4_carve_amd import vllm_exl3 as V

    monkeypatch.setenv("VLLM_EXL3_MOE_KERNEL", "lna2")
    monkeypatch.setenv("VLLM_EXL3_MOE_STRICT", "2")
    host_experts = []
    for e in range(E):
        ex = synth.expert(e, H, I, BITS, seed=550)
        host_experts.append({p: {k: torch.from_numpy(ex[p][k]) for k in ("trellis", "suh", "svh")}
                             for p in ("gate", "up", "down")})
    layer, meth = _moe_layer(dev, host_experts, 0)
    before = ops.SCRATCH.resident_bytes()
    ids, w = synth.routing(5, E, TOPK, seed=560)
    x = to_dev(synth.activations(5, H, seed=561), dev)
    y = meth.apply(layer, x, to_dev(w, dev), to_dev(ids.astype(np.int64), dev))
    torch.cuda.synchronize()
    # measured before the loop below: its dense GEMMs size the dense scratch for
    # their own row counts, which earlier tests in the process may not have
    assert ops.SCRATCH.resident_bytes() == before
    ref = V.apply_exl3_python_loop(x, to_dev(ids.astype(np.int64), dev), to_dev(w, dev), layer._exl3_inners, None,
                                   LIMIT)
    torch.cuda.synchronize()
    assert_close(y.float().cpu().numpy(), ref.cpu().numpy(), max_abs=2e-2 + 8e-3)


def test_vram_trace_phases_match_the_scratch_sizes(dev, monkeypatch, caplog):
    """LNA_EXL3_VRAM_TRACE=1 (recipe-lna/vllm_exl3_exl3.py.lna:92-118) on a fresh
    scratch pool: one routed layer and one two-shard dense module log each
    allocating phase, and every delta is what that phase keeps: the MoE
    pointer and width tables, the decode scratch, the dense GEMV scratch, no
    device tables for a T0 group, and the first call's two fp32 outputs."""
    import logging
    import re

    import torch
    from dsv4_carve_amd import ops
    from dsv4_carve_amd import vllm_exl3 as V

    monkeypatch.setenv("LNA_EXL3_VRAM_TRACE", "1")
    monkeypatch.setenv("VLLM_EXL3_MOE_KERNEL", "lna2")
    monkeypatch.setenv("VLLM_EXL3_MOE_STRICT", "2")
    monkeypatch.setenv("LNA_EXL3_DENSE_GROUP", "1")
    monkeypatch.setattr(ops, "SCRATCH", ops._ScratchPool())
    V.reset_dense_group_state()
    host_experts = []
    for e in range(E):
        ex = synth.expert(e, H, I, BITS, seed=570)
        host_experts.append({p: {k: torch.from_numpy(ex[p][k]) for k in ("trellis", "suh", "svh")}
                             for p in ("gate", "up", "down")})
    gu_host = [synth.dense(H, I, SHARED_BITS, seed=575 + j) for j in range(2)]
    gu_dev = [{k: to_dev(h[k], dev) for k in ("trellis", "suh", "svh")} for h in gu_host]
    m = 4
    with caplog.at_level(logging.INFO, logger=V.logger.name):
        _moe_layer(dev, host_experts, 0)
        gu, gu_meth = _dense_module(dev, "model.layers.0.ffn.shared_experts.gate_up_proj", H, [I, I], gu_dev)
        gu_meth.apply(gu, to_dev(synth.activations(m, H, seed=576), dev))
        torch.cuda.synchronize()
    pat = re.compile(r"F2 VRAM phase=(\S+) layer=(\S+) before_mib=([\d.]+) after_mib=([\d.]+) delta_mib=([+-][\d.]+)")
    delta = {}                                        # MiB, as logged (three decimals)
    for r in caplog.records:
        hit = pat.fullmatch(r.getMessage())
        if hit:
            assert hit.group(1) not in delta, f"phase {hit.group(1)} logged twice"
            delta[hit.group(1)] = float(hit.group(5))
    print("traced deltas (MiB):", delta, flush=True)
    blocks = lambda b: -(-b // 512) * 512             # the caching allocator's 512-byte rounding
    near = lambda phase, nbytes: abs(delta[phase] - nbytes / 2 ** 20) <= 5e-4 + 1e-9   # the log's rounding
    assert set(delta) == {"moe.tables", "moe.scratch", "registration.gemv_scratch", "registration.local_tables",
                          "registration.local_scratch", "first_call"}, delta
    # one int64 entry per expert in each pointer table, one int8 width per expert
    assert near("moe.tables", len(V.MOE_TABLE_KEYS) * blocks(E * 8) + blocks(E))
    assert near("moe.scratch", blocks(ops.moe_scratch_bytes(H, I, V.LNA2_MAX_TOPK, rows=V.lna2_max_rows())))
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    held = {purpose: int(buf.numel()) for (d, purpose), buf in ops.SCRATCH._bufs.items() if d == idx}
    assert near("registration.gemv_scratch", blocks(held["gemm"]))
    assert delta["registration.local_tables"] == 0.0
    assert near("registration.local_scratch", blocks(held["gemm_group"]))
    assert near("first_call", 2 * blocks(m * I * 4))
