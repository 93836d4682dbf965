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


@pytest.mark.parametrize("rows", [1, 2, 5, 16, 21, 32, 45])
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


@pytest.mark.parametrize("cb", [O.CB_3INST, O.CB_MUL1])
def test_fan_other_codebooks(dev, cb):
    """The fan with the 3INST and MUL1 codebooks (mixed widths, 1 and 16 rows),
    against the oracle with the same codebook and against each member's solo
    call."""
    import torch
    from dsv4_carve_amd import ops

    fan = Fan(dev, 512, [256, 128, 512], [4, 2, 6], seed=33)
    for rows in (1, 16):
        print(f"fan codebook {cb} rows={rows}", flush=True)
        x = synth.activations(rows, 512, seed=960 + rows)
        xd = to_dev(x, dev)
        outs = ops.gemm_group(xd, fan.dev, cb, torch.float32)
        for j, out in enumerate(outs):
            L = fan.host[j]
            got = out.cpu().numpy()
            assert_close(got, O.linear(x, L["trellis"], L["suh"], L["svh"], L["bits"], cb),
                         what=f"codebook {cb} member {j} rows={rows}")
            solo = ops.gemm(xd, *fan.dev[j], cb, torch.float32).cpu().numpy()
            assert rel_l2(got, solo) < 1e-5


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


# ---------------------------------------------------------------- the quant method's lifecycle and T1 fans


def _quant_module(dev, prefix, k, shards, bits, seed, bf16=(), cfg=None, tp_rank=0, tp_size=1):
    """A dense module built the way vLLM builds it: create_weights, one
    weight_loader call per (tensor kind, shard), process_weights_after_loading.
    Returns (layer, host shards); bf16 shards get a random bf16 weight."""
    import torch
    from dsv4_carve_amd import vllm_exl3 as V

    host = [synth.dense(k, n, bits, seed=seed + 13 * j) for j, n in enumerate(shards)]
    layer = torch.nn.Module()
    layer.prefix = prefix
    meth = V.Exl3LinearMethod(cfg, bits=bits, tp_rank=tp_rank, tp_size=tp_size)
    with torch.device(dev):
        meth.create_weights(layer, k, list(shards), k, sum(shards), params_dtype=torch.bfloat16)
    g = torch.Generator().manual_seed(seed)
    for j, h in enumerate(host):
        if j in bf16:
            h["bf16"] = (torch.randn((shards[j], k), generator=g) / k ** 0.5).to(torch.bfloat16)
            layer.weight.weight_loader(layer.weight, h["bf16"].to(dev), j)
            continue
        for suffix in ("trellis", "suh", "svh"):
            p = getattr(layer, suffix)
            p.weight_loader(p, torch.from_numpy(h[suffix]).to(dev), j)
        layer.mcg.weight_loader(layer.mcg, torch.tensor(V.MCG_MARKER_SIGNED_INT32, dtype=torch.int32), j)
    meth.process_weights_after_loading(layer)
    return layer, meth, host


def _module_ref(host, x16, bf16=()):
    outs = []
    for j, h in enumerate(host):
        if j in bf16:
            outs.append(x16.astype(np.float32) @ h["bf16"].float().numpy().T)
        else:
            outs.append(O.linear(x16, h["trellis"], h["suh"], h["svh"], h["bits"]))
    return np.concatenate(outs, axis=1)


def test_linear_method_prewarms_groups_and_captures(dev):
    """LNA_EXL3_DENSE_GROUP=1: after process_weights_after_loading the
    module's shards run as one fused call, the scratch is reserved for every
    decode row count (no prepare_gemm by hand), and a graph captured at each
    row count 1..16 replays to the oracle's result; so do graphs at 24 and 32
    rows, where the group declines and each shard takes the GEMV (which runs
    up to AUTO_RECONSTRUCT_THRESHOLD rows), with no scratch grown by the
    capture."""
    import torch
    from dsv4_carve_amd import ops, vllm_exl3 as V

    V.reset_dense_group_state()
    with dense_group(1):
        layer, meth, host = _quant_module(dev, "model.layers.2.ffn.shared_experts.gate_up_proj", 1024,
                                          [512, 512], 4, seed=1200)
        assert V.dense_group_stats()["prewarm_groups"] == 1
        before = ops.SCRATCH.resident_bytes()
        for rows in [*range(1, 17), 24, V.AUTO_RECONSTRUCT_THRESHOLD]:
            x16 = synth.activations(rows, 1024, seed=1300 + rows)
            x = to_dev(x16.astype(np.float32), dev)          # fp32 in and out: no output cast on the bar
            static_out = None
            stream = torch.cuda.Stream()
            stream.wait_stream(torch.cuda.current_stream())
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                static_out = meth.apply(layer, x)
            for rep in range(2):
                graph.replay()
                torch.cuda.synchronize()
                assert_close(static_out.cpu().numpy(), _module_ref(host, x16),
                             what=f"captured apply rows={rows} replay {rep}")
        assert ops.SCRATCH.resident_bytes() == before, "capture needed scratch the prewarm did not reserve"
    assert V.dense_group_call_counts()[1] > 0


def _attention_fans(dev, k=1024, seed=1400):
    """One attention layer's T1 members: the h-fan (fused_wqa_wkv with two
    shards, compressor and indexer compressor with two each) and the q-fan
    (wq_b and indexer.wq_b, one shard each, reading a 512-wide latent)."""
    base = "model.layers.7.attn"
    spec = {"qkv": (f"{base}.fused_wqa_wkv", k, [512, 256]),
            "compressor": (f"{base}.compressor.fused_wkv_wgate", k, [256, 256]),
            "indexer_compressor": (f"{base}.indexer.compressor.fused_wkv_wgate", k, [128, 128]),
            "qb": (f"{base}.wq_b", 512, [1024]),
            "indexer_qb": (f"{base}.indexer.wq_b", 512, [512])}
    return {role: _quant_module(dev, prefix, kk, shards, 6, seed=seed + 97 * i)
            for i, (role, (prefix, kk, shards)) in enumerate(spec.items())}


def test_t1_fans_one_fused_call_per_input(dev):
    """LNA_EXL3_DENSE_GROUP=2: the first h-fan member called on the hidden
    state runs all six matrices in one call, the other two modules take their
    outputs from it; likewise the q-fan.  Outputs match the oracle, eagerly
    and replayed from a captured graph."""
    import torch
    from dsv4_carve_amd import vllm_exl3 as V

    V.reset_dense_group_state()
    with dense_group(2):
        mods = _attention_fans(dev)
        for role, (layer, _, _) in mods.items():
            assert getattr(layer, "_exl3_dense_fan", None) is not None, f"{role} did not join its fan"

        def step(h, q):
            return {r: mods[r][1].apply(mods[r][0], h if r in ("qkv", "compressor", "indexer_compressor") else q)
                    for r in ("qkv", "qb", "compressor", "indexer_qb", "indexer_compressor")}

        for rows in (1, 5, 16):
            h16 = synth.activations(rows, 1024, seed=1500 + rows)
            q16 = synth.activations(rows, 512, seed=1600 + rows)
            h, q = to_dev(h16.astype(np.float32), dev), to_dev(q16.astype(np.float32), dev)
            calls = V.dense_group_call_counts()[2]
            out = step(h, q)
            torch.cuda.synchronize()
            assert V.dense_group_call_counts()[2] == calls + 2, "one fused call per fan and input"
            for r, y in out.items():
                x16 = h16 if r in ("qkv", "compressor", "indexer_compressor") else q16
                assert_close(y.cpu().numpy(), _module_ref(mods[r][2], x16), what=f"T1 {r} rows={rows}")
        assert V.dense_group_stats()["t1_cached"] >= 6
        # the same step captured once and replayed
        h = to_dev(synth.activations(4, 1024, seed=1700).astype(np.float32), dev)
        q = to_dev(synth.activations(4, 512, seed=1701).astype(np.float32), dev)
        eager = {r: y.clone() for r, y in step(h, q).items()}
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            static = step(h, q)
        for rep in range(3):
            graph.replay()
            torch.cuda.synchronize()
            for r in eager:
                assert torch.equal(static[r], eager[r]), f"T1 {r}: replay {rep} differs from the eager step"
    V.reset_dense_group_state()


def test_bf16_shards_apply(dev):
    """A module with a bf16 shard between two EXL3 shards: EXL3 shards
    through the GEMV, the bf16 one as a plain linear, concatenated in order."""
    import torch
    from dsv4_carve_amd import vllm_exl3 as V

    prefix = "model.layers.1.attn.fused_qkv"
    cfg = V.Exl3Config(bits=3, non_routed_exl3={"layers": {prefix: {"bf16_shards": [1]}}})
    layer, meth, host = _quant_module(dev, prefix, 512, [256, 128, 256], 3, seed=1800, bf16=(1,), cfg=cfg)
    for rows in (1, 6, 40):
        x16 = synth.activations(rows, 512, seed=1900 + rows)
        y = meth.apply(layer, to_dev(x16.astype(np.float32), dev))
        ref = _module_ref(host, x16, bf16=(1,))
        assert_close(y[:, :256].cpu().numpy(), ref[:, :256], what="EXL3 shard 0")
        assert_close(y[:, 384:].cpu().numpy(), ref[:, 384:], what="EXL3 shard 2")
        # the bf16 shard is a bf16 product (the reference's F.linear on the bf16 weight): bf16's bar
        assert rel_l2(y[:, 256:384].cpu().numpy(), ref[:, 256:384]) < 1e-2


def test_wo_a_rank_slice_apply(dev):
    """wo_a at TP8, rank 5: of the eight pre-sliced groups only rank 5's is
    loaded, and the module computes that group's product."""
    import torch
    from dsv4_carve_amd import vllm_exl3 as V

    layer = torch.nn.Module()
    layer.prefix = "model.layers.9.attn.wo_a"
    meth = V.Exl3LinearMethod(bits=4, tp_rank=5, tp_size=8)
    with torch.device(dev):
        meth.create_weights(layer, 512, [256], 4096, 2048)
    groups = [synth.dense(512, 256, 4, seed=2000 + r) for r in range(8)]
    for r, h in enumerate(groups):
        for suffix in ("trellis", "suh", "svh"):
            p = getattr(layer, suffix)
            p.weight_loader(p, torch.from_numpy(h[suffix]).to(dev), f"wo_a.slice.{r}")
        layer.mcg.weight_loader(layer.mcg, torch.tensor(V.MCG_MARKER_SIGNED_INT32, dtype=torch.int32),
                                f"wo_a.slice.{r}")
    meth.process_weights_after_loading(layer)
    x = synth.activations(3, 512, seed=2100)
    y = meth.apply(layer, to_dev(x, dev))
    h = groups[5]
    assert_close(y.float().cpu().numpy(), O.linear(x, h["trellis"], h["suh"], h["svh"], 4), what="wo_a rank 5")
