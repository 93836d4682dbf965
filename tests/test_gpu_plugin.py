"""GPU parity of the plugin call surface (dsv4_carve_amd.vllm_exl3) against the
oracle: LinearEXL3.forward on its three paths (the GEMV up to
AUTO_RECONSTRUCT_THRESHOLD rows, row Hadamards around an hgemm on Wq up to
1024 rows, the folded weight beyond), Exl3LinearMethod with several output shards,
apply_exl3_experts through the routed kernel and through the LinearEXL3 loop,
expert_map remapping, decline / strict behaviour and the full Exl3MoEMethod
create -> load -> finalize -> apply flow.  Tolerance: max-abs 2e-2, rel-L2 1e-3
(for fp16 outputs, the output rounding on top)."""

from __future__ import annotations

import numpy as np
import pytest

from dsv4_carve_amd import synth
from oracle import oracle as O
from tests.helpers import assert_close, to_dev

pytestmark = pytest.mark.gpu

LIMIT = 10.0


def _linear(dev, lin, **kw):
    import torch
    from dsv4_carve_amd import vllm_exl3 as V

    mcg = torch.tensor([V.MCG_MARKER_SIGNED_INT32], dtype=torch.int32, device=dev)
    return V.make_linear_exl3(to_dev(lin["trellis"], dev), to_dev(lin["suh"], dev), to_dev(lin["svh"], dev),
                              mcg, **kw)


@pytest.mark.parametrize("rows", [1, 5, 16, 32, 33, 40, 64, 144, 200, 520, 1100])
def test_linear_forward_paths(dev, rows):
    import torch

    lin = synth.dense(512, 768, 3, seed=41)
    x = synth.activations(rows, 512, seed=42 + rows)
    m = _linear(dev, lin)
    y = m.forward(to_dev(x, dev), {}, out_dtype=torch.float32)
    assert y.dtype == torch.float32 and tuple(y.shape) == (rows, 768)
    assert_close(y.cpu().numpy(), O.linear(x, lin["trellis"], lin["suh"], lin["svh"], 3))


def test_linear_forward_3d_fp16_out_and_bias(dev):
    import torch

    lin = synth.dense(256, 512, 4, seed=43)
    x = synth.activations(6, 256, seed=44)
    bias = np.linspace(-1, 1, 512).astype(np.float16)
    m = _linear(dev, lin)
    m.bias = to_dev(bias, dev)
    y = m.forward(to_dev(x, dev).view(2, 3, 256), {})
    assert y.dtype == torch.float16 and tuple(y.shape) == (2, 3, 512)
    want = O.linear(x, lin["trellis"], lin["suh"], lin["svh"], 4) + bias.astype(np.float32)
    assert_close(y.float().cpu().numpy().reshape(6, 512), want, max_abs=2e-2 + 4e-3)
    y2 = m.forward(to_dev(x, dev).view(2, 3, 256), {"reconstruct": True}, out_dtype=torch.float32)
    assert_close(y2.cpu().numpy().reshape(6, 512), want, max_abs=2e-2 + 4e-3)


@pytest.mark.parametrize("rows", [300, 1030])
@pytest.mark.parametrize("x_dtype", ["float16", "bfloat16"])
def test_linear_reconstruct_dtypes(dev, rows, x_dtype):
    """Both reconstruct paths (row-Hadamard launches around a GEMM on Wq below
    1024 rows, the folded weight from there) with fp16/bf16 inputs and
    fp16/bf16/fp32 outputs."""
    import torch

    lin = synth.dense(256, 384, 3, seed=47)
    x = synth.activations(rows, 256, seed=48 + rows)
    xt = to_dev(x, dev).to(getattr(torch, x_dtype))
    want = O.linear(xt.float().cpu().numpy().astype(np.float16), lin["trellis"], lin["suh"], lin["svh"], 3)
    m = _linear(dev, lin)
    for out_dtype, extra in ((torch.float32, 0.0), (torch.float16, 4e-3), (torch.bfloat16, 3e-2)):
        y = m.forward(xt, {}, out_dtype=out_dtype)
        assert y.dtype == out_dtype and tuple(y.shape) == (rows, 384)
        assert_close(y.float().cpu().numpy(), want, max_abs=2e-2 + extra, rel=1e-3 if extra < 1e-2 else 5e-3,
                     what=f"reconstruct rows={rows} x={x_dtype} out={out_dtype}")


def test_execute_exl3_linear(dev):
    from dsv4_carve_amd import vllm_exl3 as V
    import torch

    lin = synth.dense(256, 256, 2, seed=45)
    x = synth.activations(3, 256, seed=46)
    mcg = torch.tensor([V.MCG_MARKER_SIGNED_INT32], dtype=torch.int32, device=dev)
    y = V.execute_exl3_linear(to_dev(x, dev), to_dev(lin["trellis"], dev), to_dev(lin["suh"], dev),
                              to_dev(lin["svh"], dev), mcg)
    assert_close(y.cpu().numpy(), O.linear(x, lin["trellis"], lin["suh"], lin["svh"], 2))


def test_linear_method_shards(dev):
    import torch
    from dsv4_carve_amd import vllm_exl3 as V

    sizes = [512, 256, 128]
    shards = [synth.dense(256, n, 3, seed=50 + i) for i, n in enumerate(sizes)]
    layer = torch.nn.Module()
    meth = V.Exl3LinearMethod(bits=3)
    meth.create_weights(layer, 256, sizes, 256, sum(sizes))
    t0 = o0 = 0
    for i, (n, s) in enumerate(zip(sizes, shards)):
        layer.trellis.data[:, t0:t0 + n // 16] = torch.from_numpy(s["trellis"])
        layer.suh.data[i] = torch.from_numpy(s["suh"])
        layer.svh.data[o0:o0 + n] = torch.from_numpy(s["svh"])
        layer.mcg.data[i] = V.MCG_MARKER_SIGNED_INT32
        t0 += n // 16
        o0 += n
    layer.to(dev)
    meth.process_weights_after_loading(layer)
    x = synth.activations(4, 256, seed=55)
    y = meth.apply(layer, to_dev(x, dev).to(torch.bfloat16).float())
    xq = to_dev(x, dev).to(torch.bfloat16).float().to(torch.float16).cpu().numpy()
    want = np.concatenate([O.linear(xq, s["trellis"], s["suh"], s["svh"], 3) for s in shards], axis=1)
    assert y.dtype == torch.float32
    assert_close(y.cpu().numpy(), want)


class Experts:
    """A routed-expert layer as the plugin holds it: LinearEXL3 triples."""

    def __init__(self, dev, E, H, I, bits, seed):
        import torch

        self.experts = [synth.expert(e, H, I, bits[e], seed) for e in range(E)]
        self.layer = torch.nn.Module()
        self.layer._exl3_inners = [{p: _linear(dev, ex[p]) for p in ("gate", "up", "down")} for ex in self.experts]
        self.layer._exl3_hidden_size = H
        self.layer._exl3_intermediate_local = I
        self.layer._exl3_topk = 8
        self.cache = {}

    def ref(self, x16, ids, w):
        return O.moe(x16, ids, w, self.experts, LIMIT, cache=self.cache)


@pytest.fixture(scope="module")
def experts(dev):
    from dsv4_carve_amd import vllm_exl3 as V

    bits = [3, 2, 4, 3, 2, 2, 3, 4, 2, 3, 3, 2]
    ex = Experts(dev, len(bits), 512, 256, bits, seed=61)
    V.build_exl3_fused_state(ex.layer, ex.layer._exl3_inners)
    assert ex.layer._exl3_lna_ready, ex.layer._exl3_lna_error
    return ex


@pytest.mark.parametrize("m", [1, 4, 16])
@pytest.mark.parametrize("backend", ["lna2", "loop"])
def test_apply_experts_backends(dev, experts, monkeypatch, m, backend):
    import torch
    from dsv4_carve_amd import vllm_exl3 as V

    monkeypatch.setenv("VLLM_EXL3_MOE_KERNEL", backend)
    monkeypatch.setenv("VLLM_EXL3_MOE_STRICT", "2" if backend == "lna2" else "0")
    ids, w = synth.routing(m, 12, 6, seed=70 + m)
    x = synth.activations(m, 512, seed=71 + m)
    V.reset_moe_kernel_call_counts()
    y = V.apply_exl3_experts(to_dev(x, dev), to_dev(ids.astype(np.int64), dev), to_dev(w, dev), experts.layer)
    assert y.dtype == torch.float16 and tuple(y.shape) == (m, 512)
    assert experts.layer._exl3_last_apply == backend
    assert V.moe_kernel_call_counts()[backend] == 1
    assert_close(y.float().cpu().numpy(), experts.ref(x, ids, w), max_abs=2e-2 + 8e-3)


def test_apply_experts_expert_map(dev, experts, monkeypatch):
    import torch
    from dsv4_carve_amd import vllm_exl3 as V

    monkeypatch.setenv("VLLM_EXL3_MOE_KERNEL", "lna2")
    monkeypatch.setenv("VLLM_EXL3_MOE_STRICT", "2")
    # 24 global experts, this rank holds 12 of them in a shuffled order
    rng = np.random.default_rng(5)
    glob = rng.permutation(24)[:12]
    emap = np.full(24, -1, np.int64)
    emap[glob] = np.arange(12)
    experts.layer.expert_map = torch.from_numpy(emap)
    try:
        ids = rng.integers(-1, 25, size=(5, 6))
        w = rng.random((5, 6)).astype(np.float32)
        x = synth.activations(5, 512, seed=80)
        y = V.apply_exl3_experts(to_dev(x, dev), to_dev(ids, dev), to_dev(w, dev), experts.layer)
        local = np.array([[emap[i] if 0 <= i < 24 and emap[i] >= 0 else 12 for i in row] for row in ids])
        assert_close(y.float().cpu().numpy(), experts.ref(x, local, w), max_abs=2e-2 + 8e-3)
        y2 = V.apply_exl3_experts(to_dev(x, dev), to_dev(ids, dev), to_dev(w, dev), experts.layer, fused=False)
        assert experts.layer._exl3_last_apply == "loop"
        assert_close(y2.float().cpu().numpy(), experts.ref(x, local, w), max_abs=2e-2 + 8e-3)
    finally:
        del experts.layer.expert_map


def test_apply_experts_large_batches_use_prefill(dev, experts, monkeypatch):
    """Above 32 rows the routed path switches to the prefill kernel (no decline,
    so strict level 2 does not raise); the loop backend still serves them."""
    from dsv4_carve_amd import vllm_exl3 as V

    monkeypatch.setenv("VLLM_EXL3_MOE_KERNEL", "lna2")
    monkeypatch.setenv("VLLM_EXL3_MOE_STRICT", "2")
    ids, w = synth.routing(40, 12, 6, seed=90)
    x = synth.activations(40, 512, seed=91)
    V.reset_moe_kernel_call_counts()
    y = V.apply_exl3_experts(to_dev(x, dev), to_dev(ids.astype(np.int64), dev), to_dev(w, dev), experts.layer)
    assert experts.layer._exl3_last_apply == "prefill" and V.moe_kernel_call_counts()["prefill"] == 1
    assert_close(y.float().cpu().numpy(), experts.ref(x, ids, w), max_abs=2e-2 + 8e-3)
    monkeypatch.setenv("VLLM_EXL3_MOE_KERNEL", "loop")
    y2 = V.apply_exl3_experts(to_dev(x, dev), to_dev(ids.astype(np.int64), dev), to_dev(w, dev), experts.layer)
    assert experts.layer._exl3_last_apply == "loop"
    assert_close(y2.float().cpu().numpy(), experts.ref(x, ids, w), max_abs=2e-2 + 8e-3)


def test_apply_experts_long_batches_run_in_token_slices(dev, experts, monkeypatch):
    """Batches past the prefill kernel's pair limit run in token slices (the
    reference's fat-chunk slicing); a row's result does not depend on which
    slice it is in as long as the slices split K alike (here every call is
    below 4096 (token, slot) pairs), so the output is bitwise the one-call
    output."""
    import torch
    from dsv4_carve_amd import vllm_exl3 as V

    monkeypatch.setenv("VLLM_EXL3_MOE_KERNEL", "lna2")
    monkeypatch.setenv("VLLM_EXL3_MOE_STRICT", "2")
    ids, w = synth.routing(40, 12, 6, seed=94)
    x = to_dev(synth.activations(40, 512, seed=95), dev)
    args = (x, to_dev(ids.astype(np.int64), dev), to_dev(w, dev), experts.layer)
    whole = V.apply_exl3_experts(*args)
    monkeypatch.setattr(V, "PREFILL_MAX_PAIRS", 60)            # 10-token slices
    sliced = V.apply_exl3_experts(*args)
    torch.cuda.synchronize()
    assert experts.layer._exl3_last_apply == "prefill"
    assert torch.equal(whole, sliced), "token slices changed the result"
    assert_close(sliced.float().cpu().numpy(), experts.ref(x.cpu().numpy(), ids, w), max_abs=2e-2 + 8e-3)


def test_apply_experts_declines_bad_geometry(dev, experts, monkeypatch):
    from dsv4_carve_amd import vllm_exl3 as V

    monkeypatch.setenv("VLLM_EXL3_MOE_KERNEL", "lna2")
    monkeypatch.setenv("VLLM_EXL3_MOE_STRICT", "0")
    ids, w = synth.routing(3, 12, 6, seed=92)
    x = synth.activations(3, 512, seed=93)
    xf = to_dev(x, dev).float()                     # fp32 input: the kernels take fp16/bf16
    y = V.apply_exl3_experts(xf, to_dev(ids.astype(np.int64), dev), to_dev(w, dev), experts.layer)
    assert experts.layer._exl3_last_apply == "loop" and y.dtype == xf.dtype
    assert any("geometry" in r for r in V.moe_kernel_declined_reasons())
    monkeypatch.setenv("VLLM_EXL3_MOE_STRICT", "2")
    with pytest.raises(RuntimeError, match="STRICT=2"):
        V.apply_exl3_experts(xf, to_dev(ids.astype(np.int64), dev), to_dev(w, dev), experts.layer)


def test_native_selfcheck(dev, experts, monkeypatch):
    """LNA_EXL3_NATIVE_SELFCHECK=2: the first two eager calls (decode, then
    prefill) are checked on the live weights against the loop, for a bitwise
    repeat and finite values; the third is not.  A loop that disagrees fails
    the check: raised under LNA_EXL3_NATIVE_STRICT=1 (not swallowed into a
    fallback), logged otherwise with the kernel's output returned."""
    from dsv4_carve_amd import vllm_exl3 as V

    monkeypatch.setenv("VLLM_EXL3_MOE_KERNEL", "lna2")
    monkeypatch.setenv("VLLM_EXL3_MOE_STRICT", "0")
    monkeypatch.setenv("LNA_EXL3_NATIVE_SELFCHECK", "2")
    monkeypatch.setenv("LNA_EXL3_NATIVE_STRICT", "1")
    layer = experts.layer
    layer._exl3_lna_selfcheck_done, layer._exl3_lna_selfcheck = 0, []
    try:
        for m in (5, 40, 7):
            print(f"selfcheck m={m}", flush=True)
            ids, w = synth.routing(m, 12, 6, seed=300 + m)
            x = synth.activations(m, 512, seed=301 + m)
            y = V.apply_exl3_experts(to_dev(x, dev), to_dev(ids.astype(np.int64), dev), to_dev(w, dev), layer)
            assert_close(y.float().cpu().numpy(), experts.ref(x, ids, w), max_abs=2e-2 + 8e-3)
        recs = layer._exl3_lna_selfcheck
        assert [r["kernel"] for r in recs] == ["lna2", "prefill"] and [r["rows"] for r in recs] == [5, 40]
        assert all(r["ok"] and r["bitwise"] and r["finite"] and r["rel_l2"] < 1e-3 for r in recs), recs

        loop = V.apply_exl3_python_loop
        monkeypatch.setattr(V, "apply_exl3_python_loop", lambda *a, **k: loop(*a, **k) * 1.01)
        ids, w = synth.routing(4, 12, 6, seed=310)
        args = (to_dev(synth.activations(4, 512, seed=311), dev), to_dev(ids.astype(np.int64), dev),
                to_dev(w, dev), layer)
        layer._exl3_lna_selfcheck_done = 0
        with pytest.raises(V.Exl3SelfCheckError, match="rel="):
            V.apply_exl3_experts(*args)
        monkeypatch.setenv("LNA_EXL3_NATIVE_STRICT", "0")
        layer._exl3_lna_selfcheck_done = 0
        V.apply_exl3_experts(*args)
        assert layer._exl3_last_apply == "lna2" and not layer._exl3_lna_selfcheck[-1]["ok"]
    finally:
        del layer._exl3_lna_selfcheck_done, layer._exl3_lna_selfcheck


def test_stale_pointer_tables_decline(dev, monkeypatch):
    from dsv4_carve_amd import vllm_exl3 as V

    monkeypatch.setenv("VLLM_EXL3_MOE_KERNEL", "lna2")
    monkeypatch.setenv("VLLM_EXL3_MOE_STRICT", "1")
    ex = Experts(dev, 4, 256, 256, [2, 2, 3, 3], seed=93)
    V.build_exl3_fused_state(ex.layer, ex.layer._exl3_inners)
    ex.layer._exl3_inners[2]["gate"] = _linear(dev, ex.experts[2]["gate"])     # re-bound weight
    ids, w = synth.routing(2, 4, 2, seed=94)
    x = synth.activations(2, 256, seed=95)
    with pytest.raises(RuntimeError, match="stale"):
        V.apply_exl3_experts(to_dev(x, dev), to_dev(ids.astype(np.int64), dev), to_dev(w, dev), ex.layer)


def test_moe_method_flow(dev, monkeypatch):
    import torch
    from dsv4_carve_amd import vllm_exl3 as V

    monkeypatch.setenv("VLLM_EXL3_MOE_KERNEL", "lna2")
    monkeypatch.setenv("VLLM_EXL3_MOE_STRICT", "2")
    E, H, I, bits = 6, 256, 512, 3
    experts = [synth.expert(e, H, I, bits, seed=97) for e in range(E)]
    layer = torch.nn.Module()
    layer._exl3_topk = 4

    class Moe:
        swiglu_limit = LIMIT

    meth = V.Exl3MoEMethod(Moe(), bits=bits)
    meth.create_weights(layer, E, H, I)
    mcg = torch.tensor([V.MCG_MARKER_SIGNED_INT32], dtype=torch.int32)
    for e, ex in enumerate(experts):
        for shard, proj in (("w1", "gate"), ("w3", "up"), ("w2", "down")):
            for suffix in ("trellis", "suh", "svh"):
                name = "w13_" + suffix if shard != "w2" else "w2_" + suffix
                p = getattr(layer, name)
                p.weight_loader(p, torch.from_numpy(ex[proj][suffix]), f"experts.{e}.{shard}.{suffix}", shard, e)
            p = layer.w13_mcg if shard != "w2" else layer.w2_mcg
            p.weight_loader(p, mcg, f"experts.{e}.{shard}.mcg", shard, e)
    layer.to(dev)
    meth.process_weights_after_loading(layer)
    assert layer._exl3_lna_ready, layer._exl3_lna_error
    ids, w = synth.routing(7, E, 4, seed=98)
    x = synth.activations(7, H, seed=99)
    y = meth.apply(layer, to_dev(x, dev).to(torch.bfloat16), to_dev(w, dev), to_dev(ids.astype(np.int64), dev))
    assert y.dtype == torch.bfloat16 and layer._exl3_last_apply == "lna2"
    xq = to_dev(x, dev).to(torch.bfloat16).to(torch.float16).cpu().numpy()
    want = O.moe(xq, ids, w, experts, LIMIT)
    # bf16 output: its rounding alone (half an ulp = 2^-9 relative) is above
    # the fp32 bar, so the bound adds that quantisation
    assert_close(y.float().cpu().numpy(), want, max_abs=2e-2 + 3e-2, rel=4e-3)
