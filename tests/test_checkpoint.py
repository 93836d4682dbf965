"""Checkpoint loader on the CPU: synthetic EXL3 packs written here are read
back through Exl3Pack / load_experts / load_linear and every parameter is
compared bitwise with the pack's bytes, whole and TP/EP-sharded; malformed
packs raise with the offending tensor named."""

from __future__ import annotations

import json
import os

import numpy as np
import pytest
import torch

from dsv4_carve_amd import checkpoint as C
from dsv4_carve_amd import vllm_exl3 as V
from tests import packs


@pytest.fixture(scope="module")
def pack(tmp_path_factory):
    sp = packs.SmallPack(str(tmp_path_factory.mktemp("pack")))
    p = C.Exl3Pack(sp.root)
    p.sp = sp
    return p


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a))


def test_pack_discovery(pack):
    assert sorted(pack.expert_layers) == ["layers.0.ffn", "model.layers.1.mlp"]
    a, b = pack.expert_layers["layers.0.ffn"], pack.expert_layers["model.layers.1.mlp"]
    assert (a.num_experts, a.hidden, a.intermediate, a.bits) == (4, 512, 512, 2)
    assert (b.num_experts, b.hidden, b.intermediate, b.bits) == (4, 512, 512, 3)
    d = pack.dense_modules["layers.0.attn.wkv"]
    assert (d.in_features, d.out_features, d.bits, d.codebook) == (512, 128, 6, "mcg")
    assert pack.config.bits_for_prefix("model.layers.1.mlp") == 3 and pack.config.bits_for_prefix("layers.0.ffn") == 2
    fused = C.dsv4_fused_linears(pack, 0)
    assert fused["layers.0.attn.fused_wqa_wkv"] == ["layers.0.attn.wq_a", "layers.0.attn.wkv"]
    assert fused["layers.0.ffn.shared_experts.gate_up_proj"] == ["layers.0.ffn.shared_experts.w1",
                                                                 "layers.0.ffn.shared_experts.w3"]
    assert fused["layers.0.ffn.shared_experts.w2"] == ["layers.0.ffn.shared_experts.w2"]


@pytest.mark.parametrize("prefix,which", [("layers.0.ffn", "experts0"), ("model.layers.1.mlp", "experts1")])
def test_load_experts_whole(pack, prefix, which):
    layer, meth = C.load_experts(pack, prefix)
    experts = getattr(pack.sp, which)
    assert meth.bits == experts[0]["bits"] and len(layer._exl3_inners) == 4
    for e, ex in enumerate(experts):
        for j, proj in enumerate(("gate", "up")):
            assert torch.equal(layer.w13_trellis[e, j], _t(ex[proj]["trellis"]))
            assert torch.equal(layer.w13_suh[e, j], _t(ex[proj]["suh"]))
            assert torch.equal(layer.w13_svh[e, j], _t(ex[proj]["svh"]))
        assert torch.equal(layer.w2_trellis[e], _t(ex["down"]["trellis"]))
        assert torch.equal(layer.w2_suh[e], _t(ex["down"]["suh"]))
        assert torch.equal(layer.w2_svh[e], _t(ex["down"]["svh"]))
    assert torch.all(layer.w13_mcg == V.MCG_MARKER_SIGNED_INT32) and torch.all(layer.w2_mcg == V.MCG_MARKER_SIGNED_INT32)
    assert getattr(layer, "expert_map", None) is None


def test_load_experts_tp_shards_concatenate_to_whole(pack):
    whole, _ = C.load_experts(pack, "layers.0.ffn")
    parts = [C.load_experts(pack, "layers.0.ffn", tp_rank=r, tp_size=2)[0] for r in range(2)]
    assert tuple(parts[0].w13_trellis.shape) == (4, 2, 32, 16, 32) and parts[0]._exl3_intermediate_local == 256
    assert torch.equal(torch.cat([p.w13_trellis for p in parts], dim=3), whole.w13_trellis)
    assert torch.equal(torch.cat([p.w13_svh for p in parts], dim=2), whole.w13_svh)
    assert torch.equal(parts[1].w13_suh, whole.w13_suh)                 # gate/up input side is not split
    assert torch.equal(torch.cat([p.w2_trellis for p in parts], dim=1), whole.w2_trellis)
    assert torch.equal(torch.cat([p.w2_suh for p in parts], dim=1), whole.w2_suh)
    assert torch.equal(parts[0].w2_svh, whole.w2_svh)


def test_load_experts_ep_partition(pack):
    whole, _ = C.load_experts(pack, "layers.0.ffn")
    layer, _ = C.load_experts(pack, "layers.0.ffn", ep_rank=1, ep_size=2)
    assert layer.w13_trellis.shape[0] == 2
    assert layer.expert_map.tolist() == [-1, -1, 0, 1]
    assert torch.equal(layer.w13_trellis, whole.w13_trellis[2:]) and torch.equal(layer.w2_svh, whole.w2_svh[2:])
    ids = torch.tensor([[0, 2], [3, 1]])
    assert V.map_topk_to_local(ids, 2, layer.expert_map).tolist() == [2, 0, 1, 2]
    with pytest.raises(ValueError, match="split evenly"):
        C.load_experts(pack, "layers.0.ffn", ep_rank=0, ep_size=3)


def test_load_linear_fused_column_and_row(pack):
    sp = pack.sp
    names = ["layers.0.attn.wq_a", "layers.0.attn.wkv"]
    layer, meth = C.load_linear(pack, names, module_prefix="layers.0.attn.fused_wqa_wkv")
    assert meth.bits == 6 and layer._exl3_linear_output_partition_sizes == [256, 128]
    a, b = layer._exl3_linears
    assert torch.equal(a.trellis, _t(sp.dense[names[0]]["trellis"])) and torch.equal(b.svh, _t(sp.dense[names[1]]["svh"]))
    assert a.mcg and b.mcg
    # column TP: each rank holds half of every shard's output tiles
    w1, w3 = sp.dense["layers.0.ffn.shared_experts.w1"], sp.dense["layers.0.ffn.shared_experts.w3"]
    for r in range(2):
        lay, _ = C.load_linear(pack, ["layers.0.ffn.shared_experts.w1", "layers.0.ffn.shared_experts.w3"],
                               module_prefix="layers.0.ffn.shared_experts.gate_up_proj", tp_rank=r, tp_size=2)
        g, u = lay._exl3_linears
        assert torch.equal(g.trellis, _t(w1["trellis"][:, 16 * r:16 * r + 16])) and torch.equal(u.svh, _t(w3["svh"][256 * r:256 * r + 256]))
        assert torch.equal(g.suh, _t(w1["suh"]))
    # row TP: each rank holds half of the input rows and every output
    w2 = sp.dense["layers.0.ffn.shared_experts.w2"]
    lay, _ = C.load_linear(pack, "layers.0.ffn.shared_experts.w2", tp_rank=1, tp_size=2, row_parallel=True)
    (d,) = lay._exl3_linears
    assert d.in_features == 256 and torch.equal(d.trellis, _t(w2["trellis"][16:])) and torch.equal(d.suh, _t(w2["suh"][256:]))
    assert torch.equal(d.svh, _t(w2["svh"]))


def test_linear_weight_loader_surface():
    layer = torch.nn.Module()
    meth = V.Exl3LinearMethod(bits=2)
    meth.create_weights(layer, 128, [128, 64, 64], 128, 256)
    t = torch.ones((8, 4, 32), dtype=torch.int16)
    layer.trellis.weight_loader(layer.trellis, t * 5, "v")            # qkv names map to shards 0..2
    assert int(layer.trellis[:, 12:].float().mean()) == 5
    layer.mcg.weight_loader(layer.mcg, torch.tensor(V.MCG_MARKER_SIGNED_INT32, dtype=torch.int32), 1)
    assert int(layer.mcg[1, 0]) == V.MCG_MARKER_SIGNED_INT32
    with pytest.raises(ValueError, match="unknown shard_id"):
        layer.suh.weight_loader(layer.suh, torch.ones(128, dtype=torch.float16), "x")
    with pytest.raises(ValueError, match="out of range"):
        layer.suh.weight_loader(layer.suh, torch.ones(128, dtype=torch.float16), 3)
    with pytest.raises(RuntimeError, match="shape mismatch"):
        layer.svh.weight_loader(layer.svh, torch.ones(96, dtype=torch.float16), 0)


def test_config_parsing_and_validation():
    cfg = V.Exl3Config.from_config({"bits": 2, "layer_bits": {"42": 3}, "tensor_storage": {"big": 1},
                                    "non_routed_exl3": {"modules": ["attn.wq_b"], "bits": 6,
                                                        "layer_bits": {"attn.wq_b": 5}}})
    assert cfg.bits_for_prefix("model.layers.42.mlp.experts") == 3 and cfg.bits_for_prefix("layers.7.ffn") == 2
    assert cfg._matches_non_routed_exl3("model.layers.3.attn.wq_b") and cfg._bits_for_non_routed("x.attn.wq_b") == 5
    assert not cfg._matches_non_routed_exl3("model.layers.3.attn.wq_bx")
    for bad in ({"bits": 7}, {"bits": 2, "layer_bits": {"1": 9}}, {"codebook": "3inst"},
                {"non_routed_exl3": {"codebook": "x"}}, {"non_routed_exl3": {"layers": {"a": 3}}}):
        with pytest.raises(ValueError):
            V.Exl3Config.from_config(bad)


def test_single_file_and_unindexed_dir(tmp_path):
    ex = [packs.synth.expert(e, 256, 256, 2, 3) for e in range(2)]
    t = packs.expert_tensors("layers.5.ffn", ex)
    packs.write_pack(str(tmp_path / "a"), t, n_files=1, index=False)
    single = C.Exl3Pack(str(tmp_path / "a" / "model-00001-of-00001.safetensors"))
    assert single.config is None and single.expert_layers["layers.5.ffn"].bits == 2
    packs.write_pack(str(tmp_path / "b"), t, n_files=2, index=False)
    layer, meth = C.load_experts(C.Exl3Pack(str(tmp_path / "b")), "layers.5.ffn")
    assert meth.bits == 2 and torch.equal(layer.w2_trellis[1], _t(ex[1]["down"]["trellis"]))


def _broken(tmp_path, name, mutate, **kw):
    ex = [packs.synth.expert(e, 256, 256, 2, 3) for e in range(2)]
    t = packs.expert_tensors("layers.0.ffn", ex)
    t.update(packs.dense_tensors("layers.0.attn.wq_b", packs.synth.dense(256, 128, 3, seed=4)))
    mutate(t)
    return packs.write_pack(str(tmp_path / name), t, **kw)


@pytest.mark.parametrize("name,mutate,msg", [
    ("missing", lambda t: t.pop("layers.0.ffn.experts.1.w3.svh"), "expert 1 w3 has no svh"),
    ("dtype", lambda t: t.update({"layers.0.ffn.experts.0.w1.suh": t["layers.0.ffn.experts.0.w1.suh"].float()}),
     "stores suh as F16"),
    ("shape", lambda t: t.update({"layers.0.ffn.experts.1.w2.trellis": t["layers.0.ffn.experts.1.w2.trellis"][:8]}),
     "w2.trellis: shape"),
    ("ids", lambda t: [t.update({k.replace("experts.1.", "experts.2."): t.pop(k)}) for k in
                       [k for k in list(t) if "experts.1." in k]], "not 0..1"),
    ("mul1", lambda t: t.update({"layers.0.ffn.experts.0.w1.mul1": torch.tensor([1], dtype=torch.int32)}), "MCG-only"),
    ("dense", lambda t: t.pop("layers.0.attn.wq_b.suh"), "wq_b: EXL3 linear has no suh"),
])
def test_malformed_packs_raise(tmp_path, name, mutate, msg):
    root = _broken(tmp_path, name, mutate)
    with pytest.raises(C.Exl3PackError, match=msg):
        C.Exl3Pack(root)


def test_index_naming_a_missing_tensor(tmp_path):
    root = _broken(tmp_path, "idx", lambda t: None)
    path = os.path.join(root, C.INDEX_NAME)
    with open(path) as f:
        idx = json.load(f)
    idx["weight_map"]["layers.0.ffn.experts.9.w1.trellis"] = "model-00001-of-00002.safetensors"
    with open(path, "w") as f:
        json.dump(idx, f)
    with pytest.raises(C.Exl3PackError, match="lack"):
        C.Exl3Pack(root)


def test_config_bits_disagreeing_with_trellis_fails_the_load(tmp_path):
    root = _broken(tmp_path, "k", lambda t: None, quant_config={"bits": 3})
    pack = C.Exl3Pack(root)
    with pytest.raises(RuntimeError, match="shape mismatch"):
        C.load_experts(pack, "layers.0.ffn")


def test_wrong_marker_value_fails_processing(tmp_path):
    def mutate(t):
        t["layers.0.ffn.experts.1.w2.mcg"] = torch.tensor([7], dtype=torch.int32)
    pack = C.Exl3Pack(_broken(tmp_path, "mk", mutate))
    with pytest.raises(RuntimeError, match="marker"):
        C.load_experts(pack, "layers.0.ffn")
