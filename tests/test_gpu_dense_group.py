"""GPU parity of the same-input fan (exl3_gemm_group: several EXL3 matrices
that read one input, one fused call) through the C ABI, and of the plugin's
run_exl3_group surface.

Every member is checked against the oracle (float64 matmul on the
oracle-dequantized weights, max-abs 2e-2 / rel-L2 1e-3) and against its own
solo exl3_gemm call.  The solo call may chunk K differently (the fan sizes its
chunks over all members' column blocks), so the two agree to fp32
reassociation, not bitwise.  Shapes include the reference's h-fan (wq_a, wkv,
compressor wkv/wgate, indexer compressor x2: 4096 -> 1024/512/1024/1024/256/256)
and q_a-fan (1024 -> 32768 and 8192; recipe-lna orders REVIEW-F2-glm-bandwidth.md:39-47)."""

from __future__ import annotations

import contextlib
import os

import numpy as np
import pytest

from dsv4_carve_amd import synth
from oracle import oracle as O
from tests.helpers import assert_close, rel_l2, to_dev

pytestmark = pytest.mark.gpu


class Fan:
    def __init__(self, dev, k, ns, bits, seed):
        self.k, self.ns, self.bits = k, list(ns), list(bits)
        self.host = [synth.dense(k, n, b, seed=seed + 17 * j) for j, (n, b) in enumerate(zip(ns, bits))]
        self.dev = [(to_dev(L["trellis"], dev), to_dev(L["suh"], dev), to_dev(L["svh"], dev)) for L in self.host]

    def ref(self, x, j):
        L = self.host[j]
        return O.linear(x, L["trellis"], L["suh"], L["svh"], L["bits"], O.CB_MCG)


def _run(fan, dev, rows, seed, out_dtype=None):
    import torch
    from dsv4_carve_amd import ops

    x = synth.activations(rows, fan.k, seed=seed)
    xd = to_dev(x, dev)
    outs = ops.gemm_group(xd, fan.dev, ops.CB_MCG, out_dtype or torch.float32)
    torch.cuda.synchronize()
    return x, xd, outs


@pytest.mark.parametrize("rows", [1, 2, 5, 16, 21])
def test_mixed_fan_against_oracle_and_solo(dev, rows):
    import torch
    from dsv4_carve_amd import ops

    print(f"fan k=512 rows={rows}", flush=True)
    fan = Fan(dev, 512, [256, 128, 512, 384], [4, 2, 3, 6], seed=31)
    x, xd, outs = _run(fan, dev, rows, seed=900 + rows)
    for j, out in enumerate(outs):
        got = out.cpu().numpy()
        assert_close(got, fan.ref(x, j), what=f"member {j} rows={rows}")
        solo = ops.gemm(xd, *fan.dev[j], ops.CB_MCG, torch.float32).cpu().numpy()
        assert rel_l2(got, solo) < 1e-5, f"member {j}: fan and solo call differ beyond fp32 reassociation"


def test_fan_bitwise_repeat_and_dtypes(dev):
    import torch

    fan = Fan(dev, 1024, [512, 256], [3, 3], seed=41)
    _, xd, a = _run(fan, dev, 7, seed=950)
    _, _, b = _run(fan, dev, 7, seed=950)
    for u, v in zip(a, b):
        assert torch.equal(u, v), "fan call is not bitwise repeatable"
    _, _, h = _run(fan, dev, 7, seed=950, out_dtype=torch.float16)
    for u, v in zip(a, h):
        assert v.dtype == torch.float16
        assert rel_l2(v.float().cpu().numpy(), u.cpu().numpy()) < 1e-3


def test_reference_h_fan(dev):
    """The h-fan of one dense layer: six 6-bit members reading the 4096-wide input."""
    print("h-fan 4096 -> 1024/512/1024/1024/256/256", flush=True)
    fan = Fan(dev, 4096, [1024, 512, 1024, 1024, 256, 256], [6] * 6, seed=51)
    x, _, outs = _run(fan, dev, 4, seed=960)
    for j, out in enumerate(outs):
        assert_close(out.cpu().numpy(), fan.ref(x, j), what=f"h-fan member {j}")


def test_reference_q_a_fan(dev):
    """wq_b (1024 -> 32768) with indexer.wq_b (1024 -> 8192), 6-bit, one row."""
    print("q_a-fan 1024 -> 32768/8192", flush=True)
    fan = Fan(dev, 1024, [32768, 8192], [6, 6], seed=61)
    x, _, outs = _run(fan, dev, 1, seed=970)
    for j, out in enumerate(outs):
        assert_close(out.cpu().numpy(), fan.ref(x, j), what=f"q_a-fan member {j}")


def test_fan_in_graph_replays(dev):
    """Captured in a HIP graph, every replay (with eager work between) matches
    the eager call."""
    import torch
    from dsv4_carve_amd import ops

    fan = Fan(dev, 512, [256, 384], [2, 4], seed=71)
    x = to_dev(synth.activations(3, 512, seed=980), dev)
    eager = [t.clone() for t in ops.gemm_group(x, fan.dev)]
    outs = [torch.empty_like(t) for t in eager]
    ops.gemm_group(x, fan.dev, outs=outs)          # scratch reserved before capture
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        ops.gemm_group(x, fan.dev, outs=outs)
    for _ in range(3):
        for t in outs:
            t.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        for u, v in zip(outs, eager):
            assert torch.equal(u, v), "graph replay differs from the eager call"


def test_fan_argument_errors(dev):
    import torch
    from dsv4_carve_amd import ops

    fan = Fan(dev, 512, [256, 256], [2, 2], seed=81)
    x = to_dev(synth.activations(2, 512, seed=990), dev)
    with pytest.raises(RuntimeError, match="1..8"):
        ops.gemm_group(x, fan.dev * 5)
    with pytest.raises(RuntimeError, match="feature dimension"):
        ops.gemm_group(to_dev(synth.activations(2, 1024, seed=991), dev), fan.dev)
    with pytest.raises(RuntimeError, match="fp16"):
        ops.gemm_group(x.float(), fan.dev)
    outs = [torch.empty((2, 256), dtype=torch.float32, device=dev), torch.empty((2, 256), dtype=torch.float16,
                                                                                device=dev)]
    with pytest.raises(RuntimeError, match="one dtype"):
        ops.gemm_group(x, fan.dev, outs=outs)


# ---------------------------------------------------------------- plugin surface


@contextlib.contextmanager
def dense_group(mode):
    old = os.environ.get("LNA_EXL3_DENSE_GROUP")
    os.environ["LNA_EXL3_DENSE_GROUP"] = str(mode)
    try:
        yield
    finally:
        if old is None:
            os.environ.pop("LNA_EXL3_DENSE_GROUP", None)
        else:
            os.environ["LNA_EXL3_DENSE_GROUP"] = old


class _Module:
    def __init__(self, linears, prefix):
        self._exl3_linears = linears
        self.prefix = prefix


def _module(dev, prefix="model.layers.3.attn.fused_wqa_wkv", ns=(1024, 512), bits=(6, 6)):
    from dsv4_carve_amd import vllm_exl3 as V

    fan = Fan(dev, 1024, list(ns), list(bits), seed=91)
    lins = [V.make_linear_exl3(t, su, sv, mcg=V.torch.tensor([V.MCG_MARKER_SIGNED_INT32]))
            for (t, su, sv) in fan.dev]
    return fan, _Module(lins, prefix)


def test_run_exl3_group_t0(dev):
    import torch
    from dsv4_carve_amd import vllm_exl3 as V

    fan, mod = _module(dev)
    x = to_dev(synth.activations(4, 1024, seed=995), dev)
    V.reset_dense_group_state()
    with dense_group(0):
        solo = V.run_exl3_group(mod, x)
    assert V.dense_group_call_counts() == {1: 0, 2: 0}
    with dense_group(1):
        fused = V.run_exl3_group(mod, x)
    torch.cuda.synchronize()
    assert V.dense_group_call_counts()[1] == 1 and V.dense_group_stats()["t0_active"] == 1
    for j, (a, b) in enumerate(zip(fused, solo)):
        assert a.dtype == torch.float32 and a.shape == b.shape
        assert rel_l2(a.cpu().numpy(), b.float().cpu().numpy()) < 1e-5, f"member {j}"


def test_run_exl3_group_declines(dev):
    import torch
    from dsv4_carve_amd import vllm_exl3 as V

    fan, mod = _module(dev)
    x = to_dev(synth.activations(17, 1024, seed=996), dev)
    V.reset_dense_group_state()
    with dense_group(1):
        out = V.run_exl3_group(mod, x)                         # 17 rows: outside the fused range
        assert len(out) == 2 and V.dense_group_call_counts()[1] == 0
        V.run_exl3_group(mod, x[:2].to(torch.bfloat16))        # not fp16
        V.run_exl3_group(mod, x[:2], out_dtype=torch.float16)  # C must be fp32
    fb = V.dense_group_stats()["fallbacks"]
    assert any(k.startswith("rows:") for k in fb) and any(k.startswith("input:") for k in fb)
    assert any(k.startswith("dtype:") for k in fb)
    with dense_group(7):
        V.run_exl3_group(mod, x[:2])                           # unsupported mode fails closed (solo)
    assert any(k.startswith("config:") for k in V.dense_group_stats()["fallbacks"])
    assert V.dense_group_call_counts()[1] == 0


def test_run_exl3_group_t1_falls_back_to_t0(dev):
    from dsv4_carve_amd import vllm_exl3 as V

    fan, mod = _module(dev)
    x = to_dev(synth.activations(2, 1024, seed=997), dev)
    V.reset_dense_group_state()
    with dense_group(2):
        outs = V.run_exl3_group(mod, x)
    stats = V.dense_group_stats()
    assert stats["t0_active"] == 1 and any(k.startswith("registration:") for k in stats["fallbacks"])
    for j, out in enumerate(outs):
        assert_close(out.cpu().numpy(), fan.ref(x.cpu().numpy(), j), what=f"T0 member {j}")
