"""Writes small synthetic EXL3 packs (safetensors shards + index + quantization
config) in the layout the recipe's pack tools produce, from the seeded tensors
of dsv4_carve_amd.synth, for the checkpoint-loader tests."""

from __future__ import annotations

import json
import os

import numpy as np
import torch

from dsv4_carve_amd import synth

MCG = synth.MCG_MARKER
NAMES_SOURCE = {"gate": "w1", "up": "w3", "down": "w2"}
NAMES_HF = {"gate": "gate_proj", "up": "up_proj", "down": "down_proj"}


def expert_tensors(prefix: str, experts: list[dict], names=NAMES_SOURCE, scalar_marker=False) -> dict:
    out = {}
    for e, ex in enumerate(experts):
        for proj, tag in names.items():
            base = f"{prefix}.experts.{e}.{tag}"
            for s in ("trellis", "suh", "svh"):
                out[f"{base}.{s}"] = torch.from_numpy(np.ascontiguousarray(ex[proj][s]))
            out[f"{base}.mcg"] = torch.tensor(MCG if scalar_marker else [MCG], dtype=torch.int32)
    return out


def dense_tensors(prefix: str, lin: dict, marker="mcg") -> dict:
    out = {f"{prefix}.{s}": torch.from_numpy(np.ascontiguousarray(lin[s])) for s in ("trellis", "suh", "svh")}
    if marker == "mcg":
        out[f"{prefix}.mcg"] = torch.tensor(MCG, dtype=torch.int32)       # dense markers are scalar
    return out


def write_pack(root: str, tensors: dict, quant_config: dict | None = None, n_files: int = 2,
               index: bool = True) -> str:
    """Spread `tensors` round-robin (by sorted key) over n_files shards."""
    from safetensors.torch import save_file

    os.makedirs(root, exist_ok=True)
    keys = sorted(tensors)
    names = [f"model-{i + 1:05d}-of-{n_files:05d}.safetensors" for i in range(n_files)]
    weight_map = {}
    for i, name in enumerate(names):
        part = {k: tensors[k].contiguous() for j, k in enumerate(keys) if j % n_files == i}
        save_file(part, os.path.join(root, name), metadata={"format": "pt"})
        weight_map.update({k: name for k in part})
    if index:
        with open(os.path.join(root, "model.safetensors.index.json"), "w", encoding="utf-8") as f:
            json.dump({"metadata": {}, "weight_map": weight_map}, f)
    if quant_config is not None:
        with open(os.path.join(root, "quantization_config.json"), "w", encoding="utf-8") as f:
            json.dump(quant_config, f)
    return root


class SmallPack:
    """Two routed-expert layers (K2 with source names, K3 with HF names), the
    shared expert's w1/w3/w2 and an attention fan (wq_a + wkv), all synthetic."""

    def __init__(self, root: str, E=4, H=512, I=512, seed=7, n_files=3):
        self.E, self.H, self.I = E, H, I
        self.experts0 = [synth.expert(e, H, I, 2, seed) for e in range(E)]
        self.experts1 = [synth.expert(e, H, I, 3, seed + 1) for e in range(E)]
        self.dense = {
            "layers.0.attn.wq_a": synth.dense(H, 256, 6, seed=seed + 10),
            "layers.0.attn.wkv": synth.dense(H, 128, 6, seed=seed + 11),
            "layers.0.ffn.shared_experts.w1": synth.dense(H, I, 4, seed=seed + 12),
            "layers.0.ffn.shared_experts.w3": synth.dense(H, I, 4, seed=seed + 13),
            "layers.0.ffn.shared_experts.w2": synth.dense(I, H, 4, seed=seed + 14),
        }
        t = {}
        t.update(expert_tensors("layers.0.ffn", self.experts0))
        t.update(expert_tensors("model.layers.1.mlp", self.experts1, NAMES_HF, scalar_marker=True))
        for p, lin in self.dense.items():
            t.update(dense_tensors(p, lin))
        self.tensors = t
        self.config = {"quant_method": "exl3", "bits": 2, "codebook": "mcg", "layer_bits": {"1": 3},
                       "non_routed_exl3": {"codebook": "mcg", "layers": {
                           "layers.0.attn.fused_wqa_wkv": {"bits": 6},
                           "layers.0.ffn.shared_experts.gate_up_proj": {"bits": 4},
                           "layers.0.ffn.shared_experts.w2": {"bits": 4}}}}
        self.root = write_pack(root, t, self.config, n_files=n_files)
