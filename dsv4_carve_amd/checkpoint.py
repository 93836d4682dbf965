"""EXL3 safetensors packs -> the plugin's quant methods (routed experts and
EXL3 dense linears), TP- and EP-sharded per rank.

This plays the part vLLM's weight iteration plays for the plugin: it reads the
pack's index and shard headers, groups the EXL3 tensors per module, creates the
module's parameters through ``Exl3MoEMethod.create_weights`` /
``Exl3LinearMethod.create_weights`` and feeds every tensor through the
parameter's ``weight_loader`` with the shard id and (local) expert id vLLM's
FusedMoE expert mapping would pass, then calls ``process_weights_after_loading``.
The sharding itself lives in those loaders, as in the plugin
(recipe-lna/vllm_exl3_exl3.py.lna:2060-2195, 2323-2633).

Pack layout (the one recipe tools write, tools/layer_overlay.py:46-60,
tools/dense_bake.py:30-57, 643-658):

  * ``model.safetensors.index.json`` with a ``weight_map`` (key -> shard file),
    or a directory of ``*.safetensors`` files, or one ``.safetensors`` file;
  * routed experts ``<prefix>.experts.<e>.<w1|w3|w2>.<suffix>`` (DeepSeek
    source names) or ``<prefix>.experts.<e>.<gate_proj|up_proj|down_proj>.<suffix>``
    (HF names), suffix trellis (I16 [in/16, out/16, 16K]), suh (F16 [in]),
    svh (F16 [out]), mcg (I32 [1] or scalar);
  * dense EXL3 linears ``<module>.<trellis|suh|svh|mcg|mul1>``;
  * ``quantization_config.json``, or ``config.json``'s ``quantization_config``,
    giving K per layer (``bits`` / ``layer_bits``) and the ``non_routed_exl3``
    block.

Tensors are read with ``safetensors.safe_open`` only, which parses a JSON
header and maps raw little-endian bytes: nothing in a pack is executed.
"""

from __future__ import annotations

import json
import os
import re
from dataclasses import dataclass, field
from typing import Iterable

import torch

from . import vllm_exl3 as V

INDEX_NAME = "model.safetensors.index.json"
QUANT_CONFIG_NAME = "quantization_config.json"
CONFIG_NAME = "config.json"

SUFFIX_DTYPE = {"trellis": "I16", "suh": "F16", "svh": "F16", "mcg": "I32", "mul1": "I32"}
EXPERT_SUFFIXES = ("trellis", "suh", "svh", "mcg")
PROJ_SHARD = {"w1": "w1", "gate_proj": "w1", "w3": "w3", "up_proj": "w3", "w2": "w2", "down_proj": "w2"}

_EXPERT_RE = re.compile(r"^(?P<prefix>.+)\.experts\.(?P<expert>[0-9]+)\."
                        r"(?P<proj>w[123]|gate_proj|up_proj|down_proj)\."
                        r"(?P<suffix>trellis|suh|svh|mcg|mul1)$")
_DENSE_RE = re.compile(r"^(?P<module>.+)\.(?P<suffix>trellis|suh|svh|mcg|mul1)$")

# Same-input EXL3 linears the serving model fuses into one module, in shard
# order, keyed by the source name's tail after ``layers.<n>.``
# (tools/dense_bake.py:643-658); shard 0 of a pair is the first name.
DSV4_FUSED_MODULES = {
    "attn.fused_wqa_wkv": ("attn.wq_a", "attn.wkv"),
    "attn.compressor.fused_wkv_wgate": ("attn.compressor.wkv", "attn.compressor.wgate"),
    "attn.indexer.compressor.fused_wkv_wgate": ("attn.indexer.compressor.wkv", "attn.indexer.compressor.wgate"),
    "ffn.shared_experts.gate_up_proj": ("ffn.shared_experts.w1", "ffn.shared_experts.w3"),
}


class Exl3PackError(ValueError):
    """A pack whose names, dtypes or shapes do not form the EXL3 checkpoint ABI."""


@dataclass
class ExpertLayer:
    """One routed-expert layer of a pack, from its tensor headers."""

    prefix: str
    num_experts: int
    hidden: int
    intermediate: int
    bits: int
    keys: dict = field(repr=False)          # (expert, "w1"|"w3"|"w2", suffix) -> key


@dataclass
class DenseModule:
    """One EXL3 dense linear of a pack: y[out] = x[in] W."""

    prefix: str
    in_features: int
    out_features: int
    bits: int
    codebook: str                           # "mcg", "mul1" or "3inst" (no marker)
    keys: dict = field(repr=False)          # suffix -> key


class Exl3Pack:
    """Read-only view of an EXL3 pack: headers parsed up front, tensors read on demand."""

    def __init__(self, path: str | os.PathLike):
        from safetensors import safe_open

        self._safe_open = safe_open
        self.path = os.fspath(path)
        self.weight_map = self._discover_files()
        self._handles: dict[str, object] = {}
        self.meta: dict[str, tuple[str, tuple[int, ...]]] = {}
        for fname in sorted(set(self.weight_map.values())):
            h = self._handle(fname)
            for key in h.keys():
                if self.weight_map.get(key) == fname:
                    s = h.get_slice(key)
                    self.meta[key] = (s.get_dtype(), tuple(int(d) for d in s.get_shape()))
        missing = [k for k in self.weight_map if k not in self.meta]
        if missing:
            raise Exl3PackError(f"index names {len(missing)} tensors its shard files lack, e.g. {missing[0]}")
        self.config = self._read_quant_config()
        self.expert_layers = self._group_experts()
        self.dense_modules = self._group_dense()

    # ---------------------------------------------------------------- files

    def _discover_files(self) -> dict[str, str]:
        if os.path.isfile(self.path):
            self.root = os.path.dirname(os.path.abspath(self.path))
            return {k: os.path.basename(self.path) for k in self._keys_of(self.path)}
        self.root = self.path
        index = os.path.join(self.path, INDEX_NAME)
        if os.path.isfile(index):
            with open(index, encoding="utf-8") as f:
                weight_map = json.load(f).get("weight_map")
            if not isinstance(weight_map, dict) or not weight_map:
                raise Exl3PackError(f"{index}: no weight_map")
            return {str(k): str(v) for k, v in weight_map.items()}
        files = sorted(n for n in os.listdir(self.path) if n.endswith(".safetensors"))
        if not files:
            raise Exl3PackError(f"{self.path}: no {INDEX_NAME} and no .safetensors files")
        out: dict[str, str] = {}
        for n in files:
            for k in self._keys_of(os.path.join(self.path, n)):
                if k in out:
                    raise Exl3PackError(f"tensor {k} is in both {out[k]} and {n}")
                out[k] = n
        return out

    def _keys_of(self, fpath: str) -> list[str]:
        with self._safe_open(fpath, framework="pt", device="cpu") as f:
            return list(f.keys())

    def _handle(self, fname: str):
        h = self._handles.get(fname)
        if h is None:
            fpath = os.path.join(self.root, fname)
            if not os.path.isfile(fpath):
                raise Exl3PackError(f"shard file {fname} named by the index is missing")
            h = self._safe_open(fpath, framework="pt", device="cpu")
            self._handles[fname] = h
        return h

    def close(self) -> None:
        self._handles.clear()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def _read_quant_config(self):
        qpath = os.path.join(self.root, QUANT_CONFIG_NAME)
        cpath = os.path.join(self.root, CONFIG_NAME)
        raw = None
        if os.path.isfile(qpath):
            with open(qpath, encoding="utf-8") as f:
                raw = json.load(f)
        elif os.path.isfile(cpath):
            with open(cpath, encoding="utf-8") as f:
                raw = json.load(f).get("quantization_config")
        return V.Exl3Config.from_config(raw) if raw else None

    def tensor(self, key: str) -> torch.Tensor:
        """The tensor `key` as stored, on the CPU (dtypes were checked when the headers were grouped)."""
        if key not in self.meta:
            raise Exl3PackError(f"tensor {key} is not in the pack")
        return self._handle(self.weight_map[key]).get_tensor(key)

    # ---------------------------------------------------------------- grouping

    def _check_dtype(self, key: str, suffix: str) -> tuple[int, ...]:
        dtype, shape = self.meta[key]
        if dtype != SUFFIX_DTYPE[suffix]:
            raise Exl3PackError(f"{key}: dtype {dtype}, the EXL3 ABI stores {suffix} as {SUFFIX_DTYPE[suffix]}")
        return shape

    def _group_experts(self) -> dict[str, ExpertLayer]:
        groups: dict[str, dict] = {}
        for key in self.meta:
            m = _EXPERT_RE.match(key)
            if m:
                groups.setdefault(m["prefix"], {})[(int(m["expert"]), PROJ_SHARD[m["proj"]], m["suffix"])] = key
        return {p: self._expert_layer(p, keys) for p, keys in sorted(groups.items())}

    def _expert_layer(self, prefix: str, keys: dict) -> ExpertLayer:
        experts = sorted({e for e, _, _ in keys})
        if experts != list(range(len(experts))):
            raise Exl3PackError(f"{prefix}: expert ids are not 0..{len(experts) - 1}")
        if any(s == "mul1" for _, _, s in keys):
            raise Exl3PackError(f"{prefix}: routed experts are MCG-only in the EXL3 MoE ABI (found a mul1 marker)")
        want = [(e, sh, s) for e in experts for sh in ("w1", "w3", "w2") for s in EXPERT_SUFFIXES]
        absent = [t for t in want if t not in keys]
        if absent:
            e, sh, s = absent[0]
            raise Exl3PackError(f"{prefix}: expert {e} {sh} has no {s} tensor ({len(absent)} missing)")
        g = self._check_dtype(keys[(0, "w1", "trellis")], "trellis")
        if len(g) != 3 or g[2] % 16 or not 1 <= g[2] // 16 <= 8:
            raise Exl3PackError(f"{prefix}: w1 trellis shape {g} is not [in/16, out/16, 16K]")
        hidden, inter, bits = g[0] * 16, g[1] * 16, g[2] // 16
        up = (hidden // 16, inter // 16, 16 * bits)
        shapes = {
            ("w1", "trellis"): up, ("w3", "trellis"): up, ("w2", "trellis"): (inter // 16, hidden // 16, 16 * bits),
            ("w1", "suh"): (hidden,), ("w3", "suh"): (hidden,), ("w2", "suh"): (inter,),
            ("w1", "svh"): (inter,), ("w3", "svh"): (inter,), ("w2", "svh"): (hidden,),
        }
        for (e, sh, s), key in keys.items():
            shape = self._check_dtype(key, s)
            if s == "mcg":
                if shape not in ((), (1,)):
                    raise Exl3PackError(f"{key}: marker shape {shape}, expected [1] or scalar")
            elif shape != shapes[(sh, s)]:
                raise Exl3PackError(f"{key}: shape {shape} != {shapes[(sh, s)]} "
                                    f"(layer geometry hidden={hidden} intermediate={inter} K={bits})")
        return ExpertLayer(prefix, len(experts), hidden, inter, bits, keys)

    def _group_dense(self) -> dict[str, DenseModule]:
        groups: dict[str, dict] = {}
        for key in self.meta:
            if _EXPERT_RE.match(key):
                continue
            m = _DENSE_RE.match(key)
            if m:
                groups.setdefault(m["module"], {})[m["suffix"]] = key
        out = {}
        for prefix, keys in sorted(groups.items()):
            for s in ("trellis", "suh", "svh"):
                if s not in keys:
                    raise Exl3PackError(f"{prefix}: EXL3 linear has no {s} tensor")
            g = self._check_dtype(keys["trellis"], "trellis")
            if len(g) != 3 or g[2] % 16 or not 1 <= g[2] // 16 <= 8:
                raise Exl3PackError(f"{prefix}: trellis shape {g} is not [in/16, out/16, 16K]")
            k, n = g[0] * 16, g[1] * 16
            if self._check_dtype(keys["suh"], "suh") != (k,) or self._check_dtype(keys["svh"], "svh") != (n,):
                raise Exl3PackError(f"{prefix}: suh/svh shapes do not match trellis {g}")
            cb = "3inst"
            for s in ("mcg", "mul1"):
                if s in keys:
                    if self._check_dtype(keys[s], s) not in ((), (1,)):
                        raise Exl3PackError(f"{keys[s]}: marker is not one int32")
                    cb = s if cb == "3inst" else "both"
            if cb == "both":
                raise Exl3PackError(f"{prefix}: both mcg and mul1 markers present")
            out[prefix] = DenseModule(prefix, k, n, g[2] // 16, cb, keys)
        return out


# ---------------------------------------------------------------- loading


def _expert_partition(num_experts: int, ep_rank: int, ep_size: int) -> tuple[int, int]:
    if ep_size < 1 or not 0 <= ep_rank < ep_size:
        raise ValueError(f"ep_rank={ep_rank} is not in 0..{ep_size - 1}")
    if num_experts % ep_size:
        raise ValueError(f"{num_experts} experts do not split evenly over {ep_size} EP ranks")
    n_local = num_experts // ep_size
    return ep_rank * n_local, n_local


def load_experts(pack: Exl3Pack, prefix: str, *, device="cpu", tp_rank: int = 0, tp_size: int = 1,
                 ep_rank: int = 0, ep_size: int = 1, moe=None, layer: torch.nn.Module | None = None):
    """Build one routed-expert layer of `pack` for one (TP, EP) rank.

    TP splits the intermediate dimension (gate/up by output columns, down by
    input rows) in ``Exl3MoEMethod._load_exl3``; EP gives this rank the
    contiguous block of num_experts/ep_size experts and sets ``expert_map``
    (global id -> local id, -1 elsewhere), as vLLM's default expert placement
    does.  K is the pack config's ``bits_for_prefix(prefix)`` (the trellis
    width when the pack has no config); a trellis of another width fails the
    loader's shape check, as it does in the plugin.  Returns (layer, method)."""
    if prefix not in pack.expert_layers:
        raise Exl3PackError(f"no routed-expert layer {prefix!r} in the pack")
    info = pack.expert_layers[prefix]
    bits = pack.config.bits_for_prefix(prefix) if pack.config is not None else info.bits
    first, n_local = _expert_partition(info.num_experts, ep_rank, ep_size)
    if info.intermediate % (16 * tp_size):
        raise ValueError(f"{prefix}: intermediate {info.intermediate} does not split into 16-wide tiles over "
                         f"{tp_size} TP ranks")
    layer = layer if layer is not None else torch.nn.Module()
    layer.prefix = prefix
    method = V.Exl3MoEMethod(moe, pack.config, bits=bits, tp_rank=tp_rank, tp_size=tp_size)
    with torch.device(device):
        method.create_weights(layer, n_local, info.hidden, info.intermediate // tp_size)
    if ep_size > 1:
        emap = torch.full((info.num_experts,), -1, dtype=torch.long)
        emap[first:first + n_local] = torch.arange(n_local)
        layer.expert_map = emap
    for local in range(n_local):
        e = first + local
        for shard in ("w1", "w3", "w2"):
            group = "w13_" if shard != "w2" else "w2_"
            for suffix in EXPERT_SUFFIXES:
                t = pack.tensor(info.keys[(e, shard, suffix)])
                if suffix == "mcg" and t.dim() == 0:
                    t = t.reshape(1)         # scalar markers load into the [1] parameter
                param = getattr(layer, group + suffix)
                param.weight_loader(param, t, f"{prefix}.experts.{group}{suffix}", shard, local)
    method.process_weights_after_loading(layer)
    return layer, method


def load_linear(pack: Exl3Pack, prefixes: str | Iterable[str], *, device="cpu", tp_rank: int = 0,
                tp_size: int = 1, row_parallel: bool = False, module_prefix: str | None = None,
                layer: torch.nn.Module | None = None):
    """Build one EXL3 dense module from one or more same-input pack linears
    (the fused module's output shards, in order).

    Column-parallel modules keep the full input and split each shard's output
    columns over TP (trellis dim 1, svh); row-parallel ones split the input
    rows (trellis dim 0, suh) and keep every output.  K comes from the pack
    config's non_routed_exl3 entry for `module_prefix` when it has one, else
    from the trellis width; every shard must have that width.  Returns
    (layer, method)."""
    prefixes = [prefixes] if isinstance(prefixes, str) else list(prefixes)
    if not prefixes:
        raise ValueError("no EXL3 linears named")
    missing = [p for p in prefixes if p not in pack.dense_modules]
    if missing:
        raise Exl3PackError(f"no EXL3 linear {missing[0]!r} in the pack")
    infos = [pack.dense_modules[p] for p in prefixes]
    name = module_prefix or prefixes[0]
    cfg = pack.config
    bits = cfg._bits_for_non_routed(name) if cfg is not None and cfg._matches_non_routed_exl3(name) \
        else infos[0].bits
    k = infos[0].in_features
    if any(i.in_features != k for i in infos):
        raise Exl3PackError(f"{name}: fused shards read different input widths {[i.in_features for i in infos]}")
    div = tp_size * 16
    if (row_parallel and k % div) or (not row_parallel and any(i.out_features % div for i in infos)):
        raise ValueError(f"{name}: {'input' if row_parallel else 'output'} width does not split into 16-wide "
                         f"tiles over {tp_size} TP ranks")
    sizes = [i.out_features if row_parallel else i.out_features // tp_size for i in infos]
    k_local = k // tp_size if row_parallel else k
    layer = layer if layer is not None else torch.nn.Module()
    layer.prefix = name
    method = V.Exl3LinearMethod(cfg, bits=bits, tp_rank=tp_rank, tp_size=tp_size)
    with torch.device(device):
        method.create_weights(layer, k_local, sizes, k, sum(i.out_features for i in infos),
                              is_row_parallel=row_parallel)
    for shard, info in enumerate(infos):
        for suffix, key in info.keys.items():
            param = getattr(layer, suffix)
            param.weight_loader(param, pack.tensor(key), shard)
    method.process_weights_after_loading(layer)
    return layer, method


def dsv4_fused_linears(pack: Exl3Pack, layer_index: int, root: str = "layers") -> dict[str, list[str]]:
    """The serving model's EXL3 dense modules of one layer: fused-module name
    -> the pack linears that are its output shards, in shard order; a linear
    that is not part of a fused module maps to itself."""
    base = f"{root}.{layer_index}."
    present = {p for p in pack.dense_modules if p.startswith(base)}
    out: dict[str, list[str]] = {}
    for fused, tails in DSV4_FUSED_MODULES.items():
        members = [base + t for t in tails]
        have = [m for m in members if m in present]
        if have and len(have) != len(members):
            raise Exl3PackError(f"{base}{fused}: pack has {have} but not every shard of {members}")
        if have:
            out[base + fused] = members
            present -= set(members)
    for p in sorted(present):
        out[p] = [p]
    return out
