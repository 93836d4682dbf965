"""GPU parity of layers built from a synthetic EXL3 pack by the checkpoint
loader: routed-expert layers (K2 source names, K3 HF names) through
Exl3MoEMethod.apply on the routed kernel (5 rows) and the grouped prefill
(40 rows), TP2 and EP2 shards whose outputs sum to the whole layer, and EXL3
dense modules (a fused column-parallel pair, a row-parallel TP2 split) through
Exl3LinearMethod.apply -- all against the oracle on the pack's own tensors.
Tolerance: max-abs 2e-2 / rel-L2 1e-3, plus the fp16 output rounding where
the plugin returns fp16 (half an ulp, 2^-11 relative, per rounded output)."""

from __future__ import annotations

import numpy as np
import pytest

from dsv4_carve_amd import synth
from oracle import oracle as O
from tests import packs
from tests.helpers import assert_close, to_dev

pytestmark = pytest.mark.gpu

LIMIT = 10.0
FP16_OUT = dict(max_abs=2e-2 + 1e-2, rel=2e-3)


class _Moe:
    swiglu_limit = LIMIT


@pytest.fixture(scope="module")
def pack(tmp_path_factory):
    from dsv4_carve_amd import checkpoint as C

    sp = packs.SmallPack(str(tmp_path_factory.mktemp("gpack")), E=8, H=512, I=512, seed=21)
    p = C.Exl3Pack(sp.root)
    p.sp = sp
    return p


@pytest.fixture(autouse=True)
def _lna2(monkeypatch):
    monkeypatch.setenv("VLLM_EXL3_MOE_KERNEL", "lna2")
    monkeypatch.setenv("VLLM_EXL3_MOE_STRICT", "2")


def _routed(layer, meth, dev, x, ids, w):
    import torch

    return meth.apply(layer, to_dev(x, dev), to_dev(w, dev), to_dev(ids.astype(np.int64), dev)).float()


@pytest.mark.parametrize("prefix,which", [("layers.0.ffn", "experts0"), ("model.layers.1.mlp", "experts1")])
@pytest.mark.parametrize("rows", [5, 40])
def test_loaded_experts_against_oracle(dev, pack, prefix, which, rows):
    from dsv4_carve_amd import checkpoint as C

    print(f"pack layer {prefix} rows={rows}", flush=True)
    layer, meth = C.load_experts(pack, prefix, device=dev, moe=_Moe())
    assert layer._exl3_lna_ready, layer._exl3_lna_error
    ids, w = synth.routing(rows, 8, 4, seed=300 + rows)
    x = synth.activations(rows, 512, seed=301 + rows)
    y = _routed(layer, meth, dev, x, ids, w)
    assert layer._exl3_last_apply == ("lna2" if rows <= 16 else "prefill")
    want = O.moe(x, ids, w, getattr(pack.sp, which), LIMIT)
    assert_close(y.cpu().numpy(), want, what=f"{prefix} rows={rows}", **FP16_OUT)


@pytest.mark.parametrize("mode", ["tp", "ep"])
def test_sharded_experts_sum_to_whole(dev, pack, mode):
    from dsv4_carve_amd import checkpoint as C

    print(f"pack layer 0 {mode}2 shards", flush=True)
    ids, w = synth.routing(7, 8, 4, seed=310)
    x = synth.activations(7, 512, seed=311)
    total = 0
    for r in range(2):
        kw = dict(tp_rank=r, tp_size=2) if mode == "tp" else dict(ep_rank=r, ep_size=2)
        layer, meth = C.load_experts(pack, "layers.0.ffn", device=dev, moe=_Moe(), **kw)
        assert layer._exl3_lna_ready, layer._exl3_lna_error
        total = total + _routed(layer, meth, dev, x, ids, w).cpu().numpy()
        assert layer._exl3_last_apply == "lna2"
    want = O.moe(x, ids, w, pack.sp.experts0, LIMIT)
    assert_close(total, want, what=f"{mode}2 sum", **FP16_OUT)


def test_loaded_linears_against_oracle(dev, pack):
    import torch
    from dsv4_carve_amd import checkpoint as C

    sp = pack.sp
    x = synth.activations(3, 512, seed=320)
    xd = to_dev(x, dev).float()
    names = ["layers.0.attn.wq_a", "layers.0.attn.wkv"]
    layer, meth = C.load_linear(pack, names, module_prefix="layers.0.attn.fused_wqa_wkv", device=dev)
    y = meth.apply(layer, xd)
    assert y.dtype == torch.float32 and tuple(y.shape) == (3, 384)
    want = np.concatenate([O.linear(x, **{k: sp.dense[n][k] for k in ("trellis", "suh", "svh")},
                                    bits=6) for n in names], axis=1)
    assert_close(y.cpu().numpy(), want, what="fused wq_a+wkv")

    # shared expert down projection split by input rows over two ranks: the
    # rank outputs sum to the whole product (the all-reduce's input)
    h = synth.activations(3, 512, seed=321)
    parts = []
    for r in range(2):
        lay, m = C.load_linear(pack, "layers.0.ffn.shared_experts.w2", device=dev, tp_rank=r, tp_size=2,
                               row_parallel=True)
        parts.append(m.apply(lay, to_dev(h[:, 256 * r:256 * r + 256], dev).float()).cpu().numpy())
    lin = sp.dense["layers.0.ffn.shared_experts.w2"]
    assert_close(parts[0] + parts[1], O.linear(h, lin["trellis"], lin["suh"], lin["svh"], 4), what="row TP2 sum")
