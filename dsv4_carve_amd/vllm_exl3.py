"""The vllm-exl3 plugin's EXL3 linear / routed-MoE call surface, over libexl3_amd.

Mirrors what vLLM calls on this path, with the same names, argument meaning and
error behaviour, so the plugin's dispatch code can switch to this package:

  * ``LinearEXL3`` / ``make_linear_exl3`` / ``execute_exl3_linear`` -- the
    exllamav3 linear (recipe-lna/exllamav3/exl3.py.lna:16-218,
    recipe-lna/vllm_exl3_exl3.py.lna:889-926).  Up to AUTO_RECONSTRUCT_THRESHOLD
    rows run the trellis-decode GEMV kernel; more rows reconstruct the fp16
    weight on the GPU and run one hgemm, between row-Hadamard launches below
    FUSED_RECONSTRUCT_MIN_ROWS rows and on the Hadamard-folded weight from
    there on.
  * ``apply_exl3_experts`` and its helpers -- routed experts
    (recipe-lna/vllm_exl3_exl3.py.lna:951-1296, 1543-1569, 1707-1779): backend
    selection by VLLM_EXL3_MOE_KERNEL, strict levels by VLLM_EXL3_MOE_STRICT,
    one-shot decline logging, per-backend call counters, the shared zeroed
    scratch, and the unique-expert LinearEXL3 loop.
  * ``run_exl3_group`` and its helpers -- one fused call for the EXL3 shards
    of a module that read the same input, by LNA_EXL3_DENSE_GROUP
    (recipe-lna/vllm_exl3_exl3.py.lna:62-802), and the cross-module T1 fans
    whose later members read the fused call's cached outputs.
  * LNA_EXL3_VRAM_TRACE=1 logs the torch allocator's bytes before and after
    each allocating phase (group and fan registration, their scratch, each
    group's first call, the MoE tables and scratch), as the reference's trace
    does (recipe-lna/vllm_exl3_exl3.py.lna:92-118).
  * ``Exl3MoEMethod`` / ``Exl3LinearMethod`` -- create_weights /
    process_weights_after_loading / apply (recipe-lna/vllm_exl3_exl3.py.lna:2045-2307,
    2310-2853), importable without vLLM.

Backends here: ``lna2`` is the gfx950 routed-MoE decode kernel (default under
``auto``); ``loop`` is the unique-expert loop over LinearEXL3, whose every
matrix product is the same library's GEMV/GEMM.  Both run on the GPU only: a
CPU tensor fails in the op dispatcher, and there is no CPU fallback.

Beyond the reference's kernel ABI the routed kernel accepts one bit width per
expert (the experts of a layer may mix widths), top-k up to 8 and any hidden /
intermediate size that is a multiple of 256.
"""

from __future__ import annotations

import logging
import os
import re
from typing import Any

import torch
import torch.nn.functional as F
from torch.nn import Parameter

from . import ops

logger = logging.getLogger("vllm." + __name__)

MCG_MULTIPLIER = 0xCBAC1FED
MCG_MARKER_SIGNED_INT32 = -877912083
MUL1_MULTIPLIER = 0x83DCD12D
MUL1_MARKER_SIGNED_INT32 = -2082680531
EXL3_SUFFIXES = ("trellis", "suh", "svh", "mcg", "mul1")
SWIGLU_LIMIT_DEFAULT = 10.0
# Rows up to AUTO_RECONSTRUCT_THRESHOLD take the decode GEMV; more take the
# reconstruct path.  The reference switches at 144 rows
# (recipe-lna/exllamav3/exl3.py.lna:10); on MI355X the GEMV is faster up to 32
# rows (one 32-row block) and the reconstruct path from 48 rows on the
# 4096x4096, 4096x1536, 1536x4096 and 4096x12288 matrices (at 144 rows the
# GEMV takes 2.8x its time on 4096x4096).  From FUSED_RECONSTRUCT_MIN_ROWS
# rows the rotations are folded into the reconstructed weight (the
# reference's rule, exl3.py.lna:184).
AUTO_RECONSTRUCT_THRESHOLD = 32
FUSED_RECONSTRUCT_MIN_ROWS = 1024
MAX_RECONSTRUCT_SLICE_N = 32768
MOE_TABLE_KEYS = ops.MOE_TABLE_KEYS
PREFILL_MAX_PAIRS = 65536
_FAT_CHUNK_LOGGED = False


# ---------------------------------------------------------------- linear


class NullConfig:
    """Stand-in for exllamav3's config when a linear is built without a model."""

    class infer_params:
        no_reconstruct = False


class LinearEXL3:
    """One EXL3 linear: y = had_out(had_in(x * suh) @ Wq) * svh (+ bias).

    Constructor checks and forward semantics follow
    recipe-lna/exllamav3/exl3.py.lna:18-99, 114-139."""

    quant_type: str = "exl3"

    def __init__(self, config, in_features: int, out_features: int, scale=None, su=None, sv=None,
                 suh=None, svh=None, trellis=None, mcg=None, mul1=None, bias=None, out_dtype=None,
                 transformers_fix: bool = False, key: str | None = None):
        assert scale is None, "scale is no longer used"
        assert su is not None or suh is not None, "either su (packed) or suh (unpacked) is required"
        assert sv is not None or svh is not None, "either sv (packed) or svh (unpacked) is required"
        assert trellis is not None, "trellis is required"
        if su is not None:
            assert su.dtype == torch.int16, "su is wrong datatype"
        if sv is not None:
            assert sv.dtype == torch.int16, "sv is wrong datatype"
        if suh is not None:
            assert suh.dtype == torch.half, "suh is wrong datatype"
        if svh is not None:
            assert svh.dtype == torch.half, "svh is wrong datatype"
        assert trellis.dtype == torch.int16, "trellis is wrong datatype"
        assert len(trellis.shape) == 3, "trellis must have dim = 3"
        if bias is not None and bias.dtype == torch.float:
            bias = bias.to(torch.half)
        self.config = config if config is not None else NullConfig()
        self.transformers_fix = transformers_fix
        self.key = key
        self.suh = (suh if suh is not None else self.unpack_bf(su)).contiguous()
        self.svh = (svh if svh is not None else self.unpack_bf(sv)).contiguous()
        self.trellis = trellis.contiguous()
        self.K = trellis.shape[-1] // 16
        self.in_features = in_features
        self.out_features = out_features
        assert self.trellis.shape[0] * 16 == in_features and self.trellis.shape[1] * 16 == out_features, \
            "trellis shape does not match in/out features"
        self.bias = bias
        self.out_dtype = out_dtype
        self.default_out_dtype = out_dtype or torch.half
        self.mcg_tensor = mcg
        self.mul1_tensor = mul1
        self.mcg = mcg is not None
        self.mul1 = mul1 is not None
        self.codebook = ops.codebook_id(self.mcg, self.mul1)

    @staticmethod
    def unpack_bf(bitfield: torch.Tensor) -> torch.Tensor:
        """Packed sign bits -> fp16 +-1: bit i of int16 word j is element 16*j+i,
        set means -1 (recipe-lna/exllamav3/exl3.py.lna:142-158)."""
        bits = bitfield.reshape(-1).view(torch.uint16).to(torch.int32)
        shifts = torch.arange(16, device=bits.device, dtype=torch.int32)
        b = (bits.unsqueeze(-1) >> shifts) & 1
        return (1.0 - 2.0 * b.to(torch.float16)).reshape(-1).contiguous()

    def forward(self, x: torch.Tensor, params: dict, out_dtype: torch.dtype | None = None) -> torch.Tensor:
        if "ovr" in params:
            ovr = params["ovr"]
            if self.key in ovr and getattr(ovr[self.key], "inner", None) is not self:
                return ovr[self.key].forward(x, params, out_dtype)
        assert x.is_contiguous(), f"LinearEXL3 {self.key}: non-contiguous input {tuple(x.shape)}"
        dtype = out_dtype or self.default_out_dtype
        rows = x.numel() // x.shape[-1]
        if not params.get("reconstruct") and (rows <= AUTO_RECONSTRUCT_THRESHOLD
                                              or self.config.infer_params.no_reconstruct):
            x2 = x.view(rows, self.in_features)
            if x2.dtype != torch.float16:
                x2 = x2.to(torch.float16)
            y = torch.empty((rows, self.out_features), dtype=dtype if dtype in ops.OUT_KIND else torch.float32,
                            device=x.device)
            ops.gemm_into(x2, self.trellis, self.suh, self.svh, y, self.codebook)
            if y.dtype != dtype:
                y = y.to(dtype)
            if self.bias is not None:
                y += self.bias
            return y.view(*x.shape[:-1], self.out_features)
        return self.reconstruct_hgemm(x, out_dtype)

    def reconstruct_hgemm(self, x: torch.Tensor, out_dtype) -> torch.Tensor:
        """Many rows (recipe-lna/exllamav3/exl3.py.lna:161-218).  Below
        FUSED_RECONSTRUCT_MIN_ROWS rows the input and output rotations run as
        row-Hadamard launches around a GEMM on the raw codebook matrix Wq; from
        there on both rotations and sign vectors are folded into the
        reconstructed weight and the GEMM reads x itself.  fp16 GEMM with fp32
        accumulation (hipBLASLt), on the weight stored [out][in], the operand
        layout it reads fastest."""
        rows = x.numel() // x.shape[-1]
        x2 = x.view(rows, self.in_features)
        dtype = out_dtype or self.default_out_dtype
        if rows >= FUSED_RECONSTRUCT_MIN_ROWS:
            x16 = x2 if x2.dtype == torch.float16 else x2.to(torch.float16)
            wt = ops.dequant_trellis_nk(self.trellis, self.suh, self.svh, self.K, self.mcg, self.mul1).t()
            y = torch.mm(x16, wt) if dtype == torch.float16 else torch.mm(x16, wt, out_dtype=torch.float32).to(dtype)
        else:
            xh = torch.empty((rows, self.in_features), dtype=torch.float16, device=x.device)
            ops.had_r_128(x2, xh, self.suh, None, 1.0)
            wt = ops.reconstruct_weight_nk(self.trellis, self.codebook).t()
            y32 = torch.mm(xh, wt, out_dtype=torch.float32)
            y = torch.empty((rows, self.out_features), dtype=dtype if dtype in ops.OUT_KIND else torch.float32,
                            device=x.device)
            ops.had_r_128(y32, y, None, self.svh, 1.0)
            if y.dtype != dtype:
                y = y.to(dtype)
        if self.bias is not None:
            y += self.bias
        return y.view(*x.shape[:-1], self.out_features)

    def get_weight_tensor(self) -> torch.Tensor:
        return ops.dequant_trellis(self.trellis, self.suh, self.svh, self.K, self.mcg, self.mul1)

    def get_inner_weight_tensor(self) -> torch.Tensor:
        return ops.reconstruct_weight(self.trellis, self.codebook)

    def get_bias_tensor(self) -> torch.Tensor | None:
        return self.bias


def make_linear_exl3(trellis, suh, svh, mcg=None, mul1=None, *, out_dtype=torch.float16) -> LinearEXL3:
    """A LinearEXL3 over already-sharded packed tensors
    (recipe-lna/vllm_exl3_exl3.py.lna:889-911)."""
    return LinearEXL3(None, int(suh.numel()), int(svh.numel()), trellis=trellis.contiguous(),
                      suh=suh.contiguous(), svh=svh.contiguous(),
                      mcg=mcg.contiguous() if mcg is not None else None,
                      mul1=mul1.contiguous() if mul1 is not None else None,
                      out_dtype=out_dtype, transformers_fix=True)


def execute_exl3_linear(x, trellis, suh, svh, mcg=None, mul1=None, *, out_dtype=torch.float32):
    """recipe-lna/vllm_exl3_exl3.py.lna:914-926."""
    inner = make_linear_exl3(trellis, suh, svh, mcg, mul1, out_dtype=torch.float16)
    return inner.forward(x.contiguous().half(), {}, out_dtype=out_dtype)


# ---------------------------------------------------------------- dense groups (same-input fans)
#
# LNA_EXL3_DENSE_GROUP (recipe-lna/vllm_exl3_exl3.py.lna:121-135): 0 = off
# (every shard its own call), 1 = T0 (the EXL3 shards of one module, which read
# the same input, in one fused call), 2 = T1 (cross-module fans: the modules of
# one attention layer that read the same tensor run as one fused call, issued
# by the first of them to be called; the later ones take their outputs from
# that call, recipe-lna/vllm_exl3_exl3.py.lna:183-545, 616-802).
#
# The two T1 fans of a DSV4 attention layer:
#   h-fan: fused_wqa_wkv (role qkv), compressor.fused_wkv_wgate (compressor),
#          indexer.compressor.fused_wkv_wgate (indexer_compressor) -- all read
#          the layer's hidden state; complete once qkv and one more are loaded;
#   q-fan: wq_b (qb) and indexer.wq_b (indexer_qb) -- both read the q latent.

DENSE_GROUP_MAX_MATRICES = 8
DENSE_GROUP_MAX_ROWS = 16
_DENSE_GROUP_STATS: dict[str, int] = {"t0_active": 0, "t1_active": 0, "t1_cached": 0, "fallback_total": 0,
                                      "prewarm_groups": 0}
_DENSE_GROUP_FALLBACK_COUNTS: dict[str, int] = {}
_DENSE_GROUP_CALL_COUNTS: dict[int, int] = {1: 0, 2: 0}
_DENSE_GROUP_ACTIVE_LOGGED: set[str] = set()
_DENSE_FAN_ROLES = ((".indexer.compressor.fused_wkv_wgate", "h", "indexer_compressor"),
                    (".compressor.fused_wkv_wgate", "h", "compressor"),
                    (".fused_wqa_wkv", "h", "qkv"),
                    (".indexer.wq_b", "q", "indexer_qb"),
                    (".wq_b", "q", "qb"))
_DENSE_FAN_ORDER = {"h": ("qkv", "compressor", "indexer_compressor"), "q": ("qb", "indexer_qb")}
_DENSE_FAN_REGISTRY: dict[str, dict[str, Any]] = {}     # group id -> role -> weakref(module)


def dense_group_mode() -> int:
    """0 (off), 1 (T0) or 2 (T1); malformed values fail closed
    (recipe-lna/vllm_exl3_exl3.py.lna:121-132)."""
    raw = os.environ.get("LNA_EXL3_DENSE_GROUP", "0")
    try:
        mode = int(raw)
    except (TypeError, ValueError):
        _dense_group_fallback("config", f"invalid LNA_EXL3_DENSE_GROUP={raw!r}")
        return 0
    if mode not in (0, 1, 2):
        _dense_group_fallback("config", f"unsupported LNA_EXL3_DENSE_GROUP={raw!r}")
        return 0
    return mode


def dense_group_enabled() -> bool:
    return dense_group_mode() != 0


def _dense_group_fallback(reason: str, detail: str, group_id: str | None = None) -> None:
    key = f"{reason}:{group_id or '*'}"
    count = _DENSE_GROUP_FALLBACK_COUNTS.get(key, 0) + 1
    _DENSE_GROUP_FALLBACK_COUNTS[key] = count
    _DENSE_GROUP_STATS["fallback_total"] += 1
    if count == 1:
        logger.warning("DENSE_GROUP declined: %s: %s (group=%s)", reason, detail, group_id or "*")


def _dense_group_active(mode: int, group_id: str) -> None:
    _DENSE_GROUP_STATS["t0_active" if mode == 1 else "t1_active"] += 1
    _DENSE_GROUP_CALL_COUNTS[mode] = _DENSE_GROUP_CALL_COUNTS.get(mode, 0) + 1
    if group_id not in _DENSE_GROUP_ACTIVE_LOGGED:
        _DENSE_GROUP_ACTIVE_LOGGED.add(group_id)
        logger.info("DENSE_GROUP=%d ACTIVE for %s", mode, group_id)


def dense_group_stats() -> dict[str, Any]:
    return {**_DENSE_GROUP_STATS, "fallbacks": dict(_DENSE_GROUP_FALLBACK_COUNTS),
            "active_groups": sorted(_DENSE_GROUP_ACTIVE_LOGGED), "call_counts": dense_group_call_counts()}


def dense_group_call_counts() -> dict[int, int]:
    """Fused calls issued: T0 groups (1) and T1 fans (2)."""
    return dict(_DENSE_GROUP_CALL_COUNTS)


def reset_dense_group_state() -> None:
    """Clears the counters, the T1 registry and every fan's cached generation
    (tests; modules keep their T0 groups)."""
    for entries in _DENSE_FAN_REGISTRY.values():
        for ref in entries.values():
            module = ref()
            if module is not None and hasattr(module, "_exl3_dense_fan"):
                module._exl3_dense_fan = None
    _DENSE_FAN_REGISTRY.clear()
    for key in _DENSE_GROUP_STATS:
        _DENSE_GROUP_STATS[key] = 0
    _DENSE_GROUP_FALLBACK_COUNTS.clear()
    _DENSE_GROUP_ACTIVE_LOGGED.clear()
    _VRAM_FIRST_CALL_TRACED.clear()
    _DENSE_GROUP_CALL_COUNTS.update({1: 0, 2: 0})


# ---------------------------------------------------------------- VRAM trace

_VRAM_FIRST_CALL_TRACED: set = set()


def _vram_mark(device) -> int | None:
    """Bytes the torch allocator holds on `device` after a synchronize, or None
    unless LNA_EXL3_VRAM_TRACE=1 (the reference's opt-in trace of allocation
    deltas per phase, recipe-lna/vllm_exl3_exl3.py.lna:92-118).  The library's
    own static arrays (the no-alloc entry's fixed scratch) are not torch
    allocations and never show here."""
    if os.environ.get("LNA_EXL3_VRAM_TRACE") != "1" or device is None:
        return None
    device = torch.device(device)
    if device.type != "cuda":
        return None
    torch.cuda.synchronize(device)
    return int(torch.cuda.memory_allocated(device))


def _vram_report(phase: str, group_id: str, before: int | None, after: int | None) -> None:
    """One log line per traced phase, in the reference's format (log scrapers
    read it): phase, layer, allocated MiB before and after, and the delta."""
    if before is None or after is None:
        return
    mib = 1024.0 * 1024.0
    logger.info("F2 VRAM phase=%s layer=%s before_mib=%.3f after_mib=%.3f delta_mib=%+.3f",
                phase, group_id, before / mib, after / mib, (after - before) / mib)


def _vram_first_call(group_id: str, device):
    """Mark before a group's first call (None when traced already or off)."""
    if group_id in _VRAM_FIRST_CALL_TRACED:
        return None
    return _vram_mark(device)


def _vram_first_call_done(group_id: str, device, before) -> None:
    if before is None:
        return
    _vram_report("first_call", group_id, before, _vram_mark(device))
    _VRAM_FIRST_CALL_TRACED.add(group_id)


def _dense_group_members(linears: list, group_id: str) -> dict:
    """Validated group descriptor (recipe-lna/vllm_exl3_exl3.py.lna:208-250): EXL3
    members without bias, one codebook and in_features, out features multiples
    of 128, at most eight.  Widths and output order are free here."""
    if not linears:
        raise ValueError("empty EXL3 group")
    if not all(isinstance(lin, LinearEXL3) for lin in linears):
        raise ValueError("non-EXL3 member")
    if not all(lin.bias is None for lin in linears):
        raise ValueError("a fused group never applies bias")
    if len({lin.codebook for lin in linears}) != 1:
        raise ValueError("mcg/mul1 must be uniform")
    k = int(linears[0].in_features)
    if not all(int(lin.in_features) == k for lin in linears):
        raise ValueError("k must be uniform")
    ns = [int(lin.out_features) for lin in linears]
    if not all(n % 128 == 0 for n in ns) or k % 128:
        raise ValueError(f"a fused group needs k and every n to be multiples of 128, k={k}, ns={ns}")
    if len(ns) > DENSE_GROUP_MAX_MATRICES:
        raise ValueError("dense group exceeds the matrix capacity")
    if len({lin.trellis.device for lin in linears}) != 1:
        raise ValueError("members live on different devices")
    return {"group_id": group_id, "members": [(lin.trellis, lin.suh, lin.svh) for lin in linears],
            "codebook": linears[0].codebook, "k": k, "ns": ns, "device": linears[0].trellis.device}


def _dense_prewarm_rows() -> tuple[int, ...]:
    """LNA_EXL3_PREWARM_ROWS (default 1,2,4,8,16): row counts whose scratch is
    reserved before graph capture (recipe-lna/vllm_exl3_exl3.py.lna:352-369)."""
    rows = []
    for value in os.environ.get("LNA_EXL3_PREWARM_ROWS", "1,2,4,8,16").split(","):
        if not value.strip():
            continue
        try:
            row = int(value)
        except ValueError:
            _dense_group_fallback("prewarm", f"invalid row bucket {value!r}")
            continue
        if 1 <= row <= DENSE_GROUP_MAX_ROWS:
            rows.append(row)
        else:
            _dense_group_fallback("prewarm", f"row bucket {row} outside 1..{DENSE_GROUP_MAX_ROWS}")
    return tuple(dict.fromkeys(rows))


def _prewarm_group(group: dict, outs_for=None) -> bool:
    """Runs the fused call once per prewarm row count (and at the largest row
    count the group runs, so every later row count fits) so the shared scratch
    exists before any capture.  False (logged) on failure."""
    device = group["device"]
    if device.type != "cuda":
        return False
    try:
        for rows in sorted(set(_dense_prewarm_rows()) | {DENSE_GROUP_MAX_ROWS}):
            x = torch.zeros((rows, group["k"]), dtype=torch.float16, device=device)
            ops.gemm_group(x, group["members"], group["codebook"], torch.float32,
                           outs=None if outs_for is None else outs_for(rows))
        _DENSE_GROUP_STATS["prewarm_groups"] += 1
        return True
    except Exception as exc:
        _dense_group_fallback("prewarm", repr(exc), group["group_id"])
        return False


def build_exl3_dense_group(module) -> None:
    """Build the module's group descriptor once after load (and before graph
    capture).  Sentinels on ``_exl3_dense_group`` as in the reference
    (recipe-lna/vllm_exl3_exl3.py.lna:508-545): missing = not yet checked,
    None = checked and declined, dict = ready.  In T1 mode the module also
    joins its layer's fan, if its name makes it a fan member."""
    if not dense_group_enabled() or hasattr(module, "_exl3_dense_group"):
        return
    linears = [lin for lin in getattr(module, "_exl3_linears", None) or [] if lin is not None]
    if getattr(module, "_exl3_linear_bf16_shards", []):
        module._exl3_dense_group = None            # never fused: mixed bf16 shards
        return
    if len(linears) < 2:
        module._exl3_dense_group = None            # a one-shard module may still join a fan
    else:
        group_id = f"local:{getattr(module, 'prefix', '?')}:{id(module)}"
        before = _vram_mark(linears[0].trellis.device)
        try:
            module._exl3_dense_group = _dense_group_members(linears, group_id)
        except ValueError as exc:
            module._exl3_dense_group = None
            _dense_group_fallback("registration", str(exc), group_id)
        _vram_report("registration.local_tables", group_id, before, _vram_mark(linears[0].trellis.device))
    if dense_group_mode() == 2:
        _register_dense_fan(module)


def prewarm_exl3_dense_group(module) -> None:
    """Reserve the fused call's scratch for the prewarm row counts."""
    group = getattr(module, "_exl3_dense_group", None)
    if group:
        before = _vram_mark(group["device"])
        _prewarm_group(group)
        _vram_report("registration.local_scratch", group["group_id"], before, _vram_mark(group["device"]))


# ---------------------------------------------------------------- T1 fans


def _fan_spec(prefix: str | None):
    """(kind, base prefix, role) of a fan member's module name, or None."""
    for suffix, kind, role in _DENSE_FAN_ROLES:
        if prefix and prefix.endswith(suffix):
            return kind, prefix[: -len(suffix)], role
    return None


def _in_dense_fan(module) -> bool:
    return _fan_spec(getattr(module, "prefix", None)) is not None


def _fan_outputs(fan: dict, rows: int) -> list[torch.Tensor]:
    """Row-count views of the fan's outputs in its own fp32 buffer (16 rows x
    the members' total columns, reserved when the fan is built: under 3 MB for
    the largest DSV4 fan, so every fan keeps its own and no fan waits for
    another's generation to be read), one per member."""
    buf = fan["outbuf"]
    outs, off = [], 0
    for n in fan["ns"]:
        outs.append(buf[off:off + rows * n].view(rows, n))
        off += rows * n
    return outs


def _register_dense_fan(module) -> None:
    spec = _fan_spec(getattr(module, "prefix", None))
    if spec is None:
        return
    kind, base, role = spec
    group_id = f"{base}:{kind}fan"
    import weakref

    _DENSE_FAN_REGISTRY.setdefault(group_id, {})[role] = weakref.ref(module)
    _publish_dense_fan(group_id, kind)


def _publish_dense_fan(group_id: str, kind: str) -> None:
    """Builds the fan once enough members are loaded: the h-fan needs qkv and
    at least one compressor, the q-fan both of its modules
    (recipe-lna/vllm_exl3_exl3.py.lna:423-505).  Members are the modules'
    EXL3 linears in role order; the output buffer and the scratch are reserved
    and every prewarm row count is run once."""
    live = {role: ref() for role, ref in _DENSE_FAN_REGISTRY.get(group_id, {}).items() if ref() is not None}
    roles = [r for r in _DENSE_FAN_ORDER[kind] if r in live]
    complete = ("qkv" in live and len(roles) >= 2) if kind == "h" else len(roles) == len(_DENSE_FAN_ORDER["q"])
    if not complete:
        return
    modules = [live[r] for r in roles]
    flat, positions = [], {}
    for module in modules:
        members = [lin for lin in getattr(module, "_exl3_linears", None) or [] if lin is not None]
        if not members or getattr(module, "_exl3_linear_bf16_shards", []):
            for m in modules:
                m._exl3_dense_fan = None
            _dense_group_fallback("registration", "a fan member has bf16 or no EXL3 shards", group_id)
            return
        positions[id(module)] = tuple(range(len(flat), len(flat) + len(members)))
        flat.extend(members)
    tables_before = _vram_mark(flat[0].trellis.device)
    try:
        fan = _dense_group_members(flat, group_id)
    except ValueError as exc:
        for m in modules:
            m._exl3_dense_fan = None
        _dense_group_fallback("registration", str(exc), group_id)
        return
    import weakref

    device = fan["device"]
    fan.update({"kind": kind, "positions": positions, "member_ids": frozenset(id(m) for m in modules),
                "member_refs": tuple(weakref.ref(m) for m in modules), "cache": None, "last_completed": None,
                "generation": 0, "prewarm_failed": True,
                "outbuf": torch.empty(DENSE_GROUP_MAX_ROWS * sum(fan["ns"]), dtype=torch.float32, device=device)})
    _vram_report("registration.fan_tables", group_id, tables_before, _vram_mark(device))
    if device.type == "cuda":
        scratch_before = _vram_mark(device)
        fan["prewarm_failed"] = not _prewarm_group(fan, lambda rows: _fan_outputs(fan, rows))
        _vram_report("registration.fan_scratch", group_id, scratch_before, _vram_mark(device))
    for m in modules:
        m._exl3_dense_fan = fan


def _source_key(source: torch.Tensor):
    base = source
    while getattr(base, "_base", None) is not None:
        base = base._base
    return (id(base), int(source.data_ptr()), tuple(source.shape), source.dtype, str(source.device))


def _run_fan(module, fan: dict, x_fp16: torch.Tensor, source: torch.Tensor, m: int):
    """T1: the first member called on a source tensor runs the whole fan and
    caches every member's output; the other members called on the same source
    (same tensor object and storage, rows and stream) read their outputs from
    that call.  A generation ends once every member has read it.  A call that
    cannot read the open generation (another source, or a member reading it a
    second time) starts a new one, so a member never gets outputs computed
    from another input.  Like the reference, a source tensor rewritten in
    place between the members' calls is not detected.  Returns this module's
    outputs, or None after a logged decline (the caller runs its shards solo)."""
    group_id = fan["group_id"]
    if fan.get("prewarm_failed"):
        _dense_group_fallback("prewarm", "fan was not prewarmed", group_id)
        return None
    if int(x_fp16.shape[1]) != fan["k"]:
        _dense_group_fallback("input", f"fan k={fan['k']} got {x_fp16.shape[1]}", group_id)
        return None
    if source.dim() != 2 or not source.is_contiguous():
        _dense_group_fallback("input", "source must be contiguous 2D", group_id)
        return None
    positions = fan["positions"].get(id(module))
    if positions is None:
        _dense_group_fallback("registration", "caller is not a registered member", group_id)
        return None
    key = _source_key(source)
    stream = int(torch.cuda.current_stream(x_fp16.device).cuda_stream)
    cache = fan["cache"]
    if cache is not None and cache["key"] == key and cache["m"] == m and id(module) not in cache["used"]:
        if cache["stream"] != stream:
            _dense_group_fallback("stream", f"trigger stream changed {cache['stream']}->{stream}", group_id)
            return None
        cache["used"].add(id(module))
        result = [cache["outs"][i] for i in positions]
        _DENSE_GROUP_STATS["t1_cached"] += 1
        if cache["used"] == fan["member_ids"]:
            fan["last_completed"] = {"key": key, "m": m, "stream": stream}
            fan["cache"] = None
        return result
    if cache is not None:
        # the open generation's readers that did not come lose it (logged once)
        _dense_group_fallback("generation", "a new input started a generation before every member read the "
                              "previous one", group_id)
        fan["cache"] = None
    outs = _fan_outputs(fan, m)
    first = None if torch.cuda.is_current_stream_capturing() else _vram_first_call(group_id, x_fp16.device)
    try:
        ops.gemm_group(x_fp16, fan["members"], fan["codebook"], torch.float32, outs=outs)
    except Exception as exc:
        _dense_group_fallback("error", repr(exc), group_id)
        return None
    _vram_first_call_done(group_id, x_fp16.device, first)
    fan["generation"] += 1
    fan["cache"] = {"key": key, "m": m, "stream": stream, "used": {id(module)}, "outs": outs,
                    "source_ref": source}
    _dense_group_active(2, group_id)
    return [outs[i] for i in positions]


def run_exl3_group(module, x_fp16: torch.Tensor, out_dtype: torch.dtype = torch.float32, *,
                   source_tensor: torch.Tensor | None = None) -> list:
    """Forward every EXL3 shard of one module call on the same contiguous fp16
    input (recipe-lna/vllm_exl3_exl3.py.lna:616-802).  LNA_EXL3_DENSE_GROUP=1:
    the module's shards in one fused call (T0); =2: the module's layer fan
    (T1) when it is a member, else its T0 group.  Any decline falls back to
    the per-linear forwards used when the flag is off.  Returns one output per
    entry of module._exl3_linears, of dtype `out_dtype`.  T1 outputs are views
    of the fan's buffer, which its next generation reuses: callers copy them
    (apply concatenates or casts) before the fan runs again."""
    linears = getattr(module, "_exl3_linears", None) or []
    solo = lambda: [lin.forward(x_fp16, {}, out_dtype=out_dtype) for lin in linears]
    mode = dense_group_mode()
    fan = getattr(module, "_exl3_dense_fan", None) if mode == 2 else None
    if mode == 0:
        return solo()
    if len(linears) < 2 and fan is None:
        _dense_group_fallback("registration", "no fused group is available for this single-shard module")
        return solo()
    if x_fp16.dtype is not torch.float16 or not x_fp16.is_contiguous() or x_fp16.dim() != 2:
        _dense_group_fallback("input", "input must be contiguous 2D fp16", fan["group_id"] if fan else None)
        return solo()
    if out_dtype is not torch.float32:
        _dense_group_fallback("dtype", f"unsupported C dtype {out_dtype}", fan["group_id"] if fan else None)
        return solo()
    m = x_fp16.shape[0]
    if m > DENSE_GROUP_MAX_ROWS or m < 1:
        _dense_group_fallback("rows", f"rows={m} outside fused range 1..{DENSE_GROUP_MAX_ROWS}",
                              fan["group_id"] if fan else None)
        return solo()
    if mode == 2 and fan is None and _in_dense_fan(module):
        _, base, _ = _fan_spec(getattr(module, "prefix", None))
        _dense_group_fallback("registration", "T1 fan is not complete; using the registered local T0 group",
                              f"{base}:fan")
    if fan is not None:
        res = _run_fan(module, fan, x_fp16, source_tensor if source_tensor is not None else x_fp16, m)
        if res is not None:
            return res
        if len(linears) < 2:
            return solo()
    group = getattr(module, "_exl3_dense_group", None)
    if group is None and not hasattr(module, "_exl3_dense_group"):
        if torch.cuda.is_current_stream_capturing():
            _dense_group_fallback("capture", "group tables missing during capture")
            return solo()
        build_exl3_dense_group(module)
        group = getattr(module, "_exl3_dense_group", None)
    if not group:
        _dense_group_fallback("registration", "dense group tables are unavailable")
        return solo()
    if int(x_fp16.shape[1]) != group["k"]:
        _dense_group_fallback("input", f"group k={group['k']} got {x_fp16.shape[1]}", group["group_id"])
        return solo()
    first = None if torch.cuda.is_current_stream_capturing() else _vram_first_call(group["group_id"], x_fp16.device)
    try:
        outs = ops.gemm_group(x_fp16, group["members"], group["codebook"], out_dtype)
    except Exception as exc:
        _dense_group_fallback("error", repr(exc), group["group_id"])
        return solo()
    _vram_first_call_done(group["group_id"], x_fp16.device, first)
    _dense_group_active(1, group["group_id"])
    return outs


# ---------------------------------------------------------------- backend selection


def get_moe_kernel_backend() -> str:
    """VLLM_EXL3_MOE_KERNEL: "lna2" (the routed-MoE decode kernel), "loop" (the
    unique-expert LinearEXL3 loop) or "auto" (= lna2).  Unknown values warn and
    mean auto (recipe-lna/vllm_exl3_exl3.py.lna:1052-1067)."""
    requested = os.environ.get("VLLM_EXL3_MOE_KERNEL", "auto").strip().lower()
    if requested not in {"lna2", "loop", "auto"}:
        logger.warning("Unknown VLLM_EXL3_MOE_KERNEL=%r; using auto selection", requested)
        requested = "auto"
    return "lna2" if requested == "auto" else requested


def moe_kernel_strict() -> int:
    """VLLM_EXL3_MOE_STRICT: 1 raises when the kernel is not ready, 2 also on
    shape declines (recipe-lna/vllm_exl3_exl3.py.lna:1070-1089)."""
    try:
        return int(os.environ.get("VLLM_EXL3_MOE_STRICT", "0") or 0)
    except ValueError:
        return 0


_MOE_CALLS = {"lna2": 0, "prefill": 0, "loop": 0}
_LNA2_REJECT_LOGGED: set[str] = set()
_LNA2_ACTIVE_LOGGED = False


def moe_kernel_call_counts() -> dict[str, int]:
    return dict(_MOE_CALLS)


def reset_moe_kernel_call_counts() -> None:
    for k in _MOE_CALLS:
        _MOE_CALLS[k] = 0


def moe_kernel_declined_reasons() -> list[str]:
    return sorted(_LNA2_REJECT_LOGGED)


def _lna2_log_active() -> None:
    global _LNA2_ACTIVE_LOGGED
    if not _LNA2_ACTIVE_LOGGED:
        _LNA2_ACTIVE_LOGGED = True
        logger.warning("LNA2 MoE kernel ACTIVE (gfx950 routed-MoE decode)")


def _lna2_log_reject(why: str, *, not_ready: bool = False) -> None:
    """One log line per distinct decline reason; raises under the strict level
    that covers this class of decline (recipe-lna/vllm_exl3_exl3.py.lna:1143-1156)."""
    if why not in _LNA2_REJECT_LOGGED and len(_LNA2_REJECT_LOGGED) < 12:
        _LNA2_REJECT_LOGGED.add(why)
        logger.warning("LNA2 declined (falling back to the LinearEXL3 loop): %s", why)
    level = moe_kernel_strict()
    if level >= (1 if not_ready else 2):
        raise RuntimeError("VLLM_EXL3_MOE_KERNEL=lna2 with VLLM_EXL3_MOE_STRICT=%d, but the lna2 kernel "
                           "declined this call: %s" % (level, why))


def lna2_moe_kernel_available() -> bool:
    try:
        ops._lib.load()
        return True
    except Exception:
        return False


def lna2_max_rows() -> int:
    return ops.moe_max_rows()


# ---------------------------------------------------------------- routing glue


def pin_exl3_expert_map(layer, device: torch.device) -> torch.Tensor | None:
    """Move expert_map to `device` (int64) once, before any graph capture
    (recipe-lna/vllm_exl3_exl3.py.lna:951-960)."""
    emap = getattr(layer, "expert_map", None)
    if emap is None:
        return None
    if emap.device != device or emap.dtype != torch.long:
        layer.expert_map = emap.to(device=device, dtype=torch.long)
    return layer.expert_map


def map_topk_to_local(ids: torch.Tensor, n_local: int, expert_map: torch.Tensor | None) -> torch.Tensor:
    """Flattened global ids -> local ids; negative, out-of-range or unmapped ids
    become the sentinel n_local (recipe-lna/vllm_exl3_exl3.py.lna:963-985)."""
    flat = ids.reshape(-1)
    sentinel = flat.new_full(flat.shape, n_local)
    if expert_map is None:
        return torch.where((flat < 0) | (flat >= n_local), sentinel, flat)
    if expert_map.device != flat.device or expert_map.dtype != torch.long:
        raise RuntimeError("EXL3 expert_map is not pinned to the hidden-state device; "
                           "call pin_exl3_expert_map before fused apply (CUDA graphs forbid the copy)")
    n_global = int(expert_map.numel())
    if n_global == 0:
        return sentinel
    mapped = expert_map[flat.clamp(0, n_global - 1)]
    bad = (flat < 0) | (flat >= n_global) | (mapped < 0) | (mapped >= n_local)
    return torch.where(bad, sentinel, mapped)


# ---------------------------------------------------------------- routed experts


def apply_exl3_python_loop(x2d, ids, weights, inners, expert_map, limit, *, only_experts=None, out=None):
    """Unique-expert LinearEXL3 loop (recipe-lna/vllm_exl3_exl3.py.lna:988-1027):
    for each distinct routed expert, gate and up in fp32, clamped SiLU*mul,
    fp16 activation, down in fp32, scaled and index-added into an fp32 output."""
    tokens, hidden = x2d.shape
    if out is None:
        out = torch.zeros(tokens, hidden, dtype=torch.float32, device=x2d.device)
    for raw in torch.unique(ids).tolist():
        e = int(raw)
        if e < 0:
            continue
        if expert_map is not None:
            e = int(expert_map[e].item()) if expert_map.numel() > e else e
            if e < 0:
                continue
        if e >= len(inners) or (only_experts is not None and e not in only_experts):
            continue
        token_idx, k_pos = (ids == int(raw)).nonzero(as_tuple=True)
        h = x2d.index_select(0, token_idx).contiguous().half()
        pack = inners[e]
        gate = pack["gate"].forward(h, {}, out_dtype=torch.float32)
        up = pack["up"].forward(h, {}, out_dtype=torch.float32)
        act = F.silu(gate.clamp(max=limit)) * up.clamp(min=-limit, max=limit)
        down = pack["down"].forward(act.contiguous().half(), {}, out_dtype=torch.float32)
        out.index_add_(0, token_idx, down * weights[token_idx, k_pos].unsqueeze(-1).to(torch.float32))
    return out


def _validate_lna_pointer_contract(inners, hidden: int, intermediate: int) -> None:
    """Every expert's packed tensors must be contiguous, on one device, and of
    the layer's geometry before their addresses go into the pointer tables
    (recipe-lna/vllm_exl3_exl3.py.lna:1318-1374)."""
    dev = inners[0]["gate"].trellis.device
    for e, pack in enumerate(inners):
        for name, k, n in (("gate", hidden, intermediate), ("up", hidden, intermediate),
                           ("down", intermediate, hidden)):
            lin = pack[name]
            kb = lin.K
            if kb != pack["gate"].K:
                raise RuntimeError(f"expert {e}: {name} has {kb} bits, gate has {pack['gate'].K}")
            want = (k // 16, n // 16, 16 * kb)
            for what, t, shape, dt in (("trellis", lin.trellis, want, torch.int16),
                                       ("suh", lin.suh, (k,), torch.float16),
                                       ("svh", lin.svh, (n,), torch.float16)):
                if tuple(t.shape) != shape or t.dtype != dt or not t.is_contiguous() or t.device != dev:
                    raise RuntimeError(f"expert {e} {name}.{what}: {tuple(t.shape)} {t.dtype} "
                                       f"contiguous={t.is_contiguous()} {t.device}; want {shape} {dt} on {dev}")
            if lin.codebook != inners[0]["gate"].codebook:
                raise RuntimeError(f"expert {e} {name}: codebook differs from the layer's")


LNA2_MAX_TOPK = 9            # routed top-k plus a shared expert appended as one more slot


def _lna2_scratch_for(layer, device: torch.device) -> torch.Tensor:
    """The shared routed-MoE decode scratch of this device (ops.SCRATCH's "moe"
    buffer, the one ops.moe_decode uses), zeroed once on creation and
    self-resetting after (recipe-lna/vllm_exl3_exl3.py.lna:1276-1296).  Sized
    for the largest top-k and row count the decode kernels take, so a route
    with a shared-expert slot or a batch of up to lna2_max_rows() rows never
    needs a bigger buffer at apply time (which capture forbids), and every
    layer of the model shares it: layers of other shapes need no more.
    One launch at a time per device: launches on concurrent streams would share
    it."""
    hidden = int(layer._exl3_hidden_size)
    inter = int(layer._exl3_intermediate_local)
    nbytes = ops.moe_scratch_bytes(hidden, inter, LNA2_MAX_TOPK, rows=lna2_max_rows())
    if torch.cuda.is_current_stream_capturing():
        buf = ops.SCRATCH.current(device, "moe")
        if buf is None or buf.numel() < nbytes:
            raise RuntimeError("LNA2 scratch was not prewarmed for this device")
    return ops.SCRATCH.get(device, "moe", nbytes)


def lna2_scratch_bytes_resident() -> int:
    """Bytes of every shared scratch buffer the library holds (decode, prefill
    and dense, on every device, with the ones a captured graph keeps alive)."""
    return ops.SCRATCH.resident_bytes()


def lna2_scratch_error(device: torch.device, clear: bool = True) -> int:
    """Error word of this device's routed-MoE scratch (ops.ERR_* bits, 0 = none)."""
    buf = ops.SCRATCH.current(device, "moe")
    return 0 if buf is None else ops.moe_error(buf, clear)


def _prepare_lna_state(layer, inners) -> None:
    """Preflight: validate the pointer contract and reserve the scratch; sets
    layer._exl3_lna_ready / _exl3_lna_error (recipe-lna/vllm_exl3_exl3.py.lna:1395-1449)."""
    layer._exl3_lna_ready = False
    try:
        _validate_lna_pointer_contract(inners, int(layer._exl3_hidden_size), int(layer._exl3_intermediate_local))
        ops._lib.load()
        _lna2_scratch_for(layer, inners[0]["gate"].trellis.device)
        layer._exl3_lna_ready = True
        layer._exl3_lna_error = None
    except Exception as exc:
        layer._exl3_lna_error = repr(exc)
        logger.warning("LNA2 preflight FAILED for %s: %r -- the MoE will fall back to the LinearEXL3 loop",
                       getattr(layer, "prefix", "?"), exc)
        if moe_kernel_strict():
            raise


def build_exl3_fused_state(layer, inners: list[dict[str, Any]]) -> None:
    """Pointer tables (int64 data_ptr per expert and tensor), the per-expert
    bit-width table and its mask, once after load; then the preflight
    (recipe-lna/vllm_exl3_exl3.py.lna:1543-1594).  The weights must stay alive
    and must not move while the tables are in use."""
    device = inners[0]["gate"].trellis.device
    layer_id = getattr(layer, "prefix", "?")
    before = _vram_mark(device)
    tables = {}
    for key in MOE_TABLE_KEYS:
        which, attr = key.split("_", 1)
        tables[key] = torch.tensor([int(getattr(p[which], attr).data_ptr()) for p in inners],
                                   dtype=torch.int64, device=device)
    layer._exl3_ptrs = tables
    bits = [int(p["gate"].K) for p in inners]
    layer._exl3_bits_table = torch.tensor(bits, dtype=torch.int8, device=device)
    layer._exl3_bits_mask = ops.bits_mask_of(bits)
    layer._exl3_codebook = int(inners[0]["gate"].codebook)
    layer._exl3_ptr_sources = [(p["gate"].trellis, p["down"].trellis) for p in inners]
    if len(set(bits)) == 1:
        layer._exl3_k = bits[0]
    _vram_report("moe.tables", layer_id, before, _vram_mark(device))
    if get_moe_kernel_backend() == "lna2":
        before = _vram_mark(device)
        _prepare_lna_state(layer, inners)
        _vram_report("moe.scratch", layer_id, before, _vram_mark(device))


def _ptrs_stale(layer, inners) -> bool:
    """The tables hold raw addresses: a re-bound weight invalidates them."""
    src = getattr(layer, "_exl3_ptr_sources", None)
    return src is None or len(src) != len(inners) or any(
        a is not p["gate"].trellis or b is not p["down"].trellis for (a, b), p in zip(src, inners))


def _apply_lna2_moe(x2d, ids, weights, layer, inners, expert_map, limit):
    """The routed-MoE decode kernel, or None (logged) when it declines
    (recipe-lna/vllm_exl3_exl3.py.lna:1190-1248)."""
    if not lna2_moe_kernel_available() or not getattr(layer, "_exl3_lna_ready", False):
        _lna2_log_reject("module=%s lna_ready=%s lna_error=%s" % (
            lna2_moe_kernel_available(), getattr(layer, "_exl3_lna_ready", None),
            getattr(layer, "_exl3_lna_error", None)), not_ready=True)
        return None
    hidden = int(getattr(layer, "_exl3_hidden_size", -1))
    inter = int(getattr(layer, "_exl3_intermediate_local", -1))
    topk = int(ids.shape[-1])
    rows = int(x2d.shape[0]) if x2d.dim() == 2 else -1
    if (not x2d.is_cuda or x2d.dim() != 2 or rows < 1
            or int(x2d.shape[1]) != hidden or hidden % 256 or inter % 256 or hidden > 16384 or inter > 16384
            or not 1 <= topk <= 9 or x2d.dtype not in (torch.float16, torch.bfloat16) or not float(limit) > 0.0):
        _lna2_log_reject("geometry x=%s dtype=%s hidden=%s inter=%s topk=%s limit=%s" % (
            tuple(x2d.shape), x2d.dtype, hidden, inter, topk, limit))
        return None
    ptrs = getattr(layer, "_exl3_ptrs", None)
    if not isinstance(ptrs, dict) or any(k not in ptrs for k in MOE_TABLE_KEYS):
        _lna2_log_reject("ptr table incomplete", not_ready=True)
        return None
    if _ptrs_stale(layer, inners):
        _lna2_log_reject("ptr tables are stale (weights re-bound after build_exl3_fused_state)", not_ready=True)
        return None
    # The router's ids (int32/int64), weights (fp16/bf16/fp32) and the pinned
    # expert_map go to the kernels as they are: the global -> local mapping
    # (map_topk_to_local's rule), the widening and the weight cast happen in
    # the kernels' route planning, so no launches run before the layer.
    route_ids = ids if ids.dtype in ops.IDS_KIND and ids.is_contiguous() else ids.to(torch.long).contiguous()
    route_w = weights if weights.dtype in ops.OUT_KIND and weights.is_contiguous() else \
        weights.to(torch.float32).contiguous()
    x_in = x2d if x2d.is_contiguous() else x2d.contiguous()
    out = torch.empty_like(x_in)
    if expert_map is not None and expert_map.numel() == 0:
        return out.zero_()                  # an empty map routes nothing here
    kw = dict(intermediate=inter, expert_bits=layer._exl3_bits_table, bits_mask=layer._exl3_bits_mask,
              codebook=layer._exl3_codebook, swiglu_limit=float(limit), expert_map=expert_map)
    if rows <= lna2_max_rows():
        def run(dst):
            ops.moe_decode(x_in, dst, ptrs, route_ids, route_w, scratch=_lna2_scratch_for(layer, x2d.device), **kw)
        kind = "lna2"
    else:
        # many rows: the grouped-GEMM prefill path (the reference falls back to
        # exllamav3's fused exl3_moe here, vllm_exl3_exl3.py.lna:1597-1704).
        # One call takes up to PREFILL_MAX_PAIRS (token, slot) pairs and any
        # number of rows per expert; longer batches run in token slices, as the
        # reference's fat-chunk slicing does (:1627-1643).
        chunk = max(1, PREFILL_MAX_PAIRS // topk)
        if rows > chunk:
            global _FAT_CHUNK_LOGGED
            if not _FAT_CHUNK_LOGGED:
                logger.info("EXL3 prefill token slicing ACTIVE (tokens=%d, slice=%d)", rows, chunk)
                _FAT_CHUNK_LOGGED = True

        def run(dst):
            for s0 in range(0, rows, chunk):
                s1 = min(rows, s0 + chunk)
                ops.moe_prefill(x_in[s0:s1], dst[s0:s1], ptrs, route_ids[s0:s1], route_w[s0:s1], **kw)
        kind = "prefill"
    run(out)
    _MOE_CALLS[kind] += 1
    _native_selfcheck(layer, kind, run, out, x_in, ids, weights, inners, expert_map, limit)
    return out


# ---------------------------------------------------------------- live self-check
#
# LNA_EXL3_NATIVE_SELFCHECK=N (the reference's switch,
# recipe-lna/vllm_exl3_exl3.py.lna:1508-1539): the first N eager calls of the
# routed kernels on each layer are checked on the live weights against the
# LinearEXL3 loop, for a bitwise repeat (the same call again into a second
# buffer) and for finite values.  Eager only: the loop allocates and the
# check synchronises, neither of which a graph capture allows.  A failure is
# logged; with LNA_EXL3_NATIVE_STRICT=1 it raises Exl3SelfCheckError, which
# apply_exl3_experts passes to the caller instead of falling back.

SELFCHECK_REL_L2 = 2e-3          # the reference's bar against the loop (:1532)


class Exl3SelfCheckError(RuntimeError):
    """The routed kernel disagreed with the loop, was not bitwise repeatable
    or produced non-finite values, under LNA_EXL3_NATIVE_STRICT=1."""


def native_selfcheck_calls() -> int:
    try:
        return max(0, int(os.environ.get("LNA_EXL3_NATIVE_SELFCHECK", "0") or 0))
    except ValueError:
        return 0


def _native_selfcheck(layer, kind, run, out, x_in, ids, weights, inners, expert_map, limit) -> None:
    n_chk = native_selfcheck_calls()
    if n_chk <= 0 or torch.cuda.is_current_stream_capturing():
        return
    done = int(getattr(layer, "_exl3_lna_selfcheck_done", 0))
    if done >= n_chk:
        return
    layer._exl3_lna_selfcheck_done = done + 1
    ref = apply_exl3_python_loop(x_in, ids, weights, inners, expert_map, limit)
    repeat = torch.empty_like(out)
    run(repeat)
    torch.cuda.synchronize(out.device)
    got = out.float()
    rel = float(((got - ref).norm() / (ref.norm() + 1e-6)).item())
    bitwise = bool(torch.equal(out, repeat))
    finite = bool(torch.isfinite(got).all().item())
    record = {"call": done + 1, "kernel": kind, "rows": int(x_in.shape[0]), "rel_l2": rel, "bitwise": bitwise,
              "finite": finite, "ok": rel <= SELFCHECK_REL_L2 and bitwise and finite}
    layer._exl3_lna_selfcheck = [*getattr(layer, "_exl3_lna_selfcheck", []), record]
    logger.info("EXL3 native selfcheck %s call=%d kernel=%s m=%d rel=%.3g bitwise=%s finite=%s",
                getattr(layer, "prefix", "?"), done + 1, kind, record["rows"], rel, bitwise, finite)
    if not record["ok"]:
        msg = (f"EXL3 native selfcheck failed on {getattr(layer, 'prefix', '?')} call {done + 1} ({kind}, "
               f"m={record['rows']}): rel={rel:.3g} (bar {SELFCHECK_REL_L2}) bitwise={bitwise} finite={finite}")
        if os.environ.get("LNA_EXL3_NATIVE_STRICT", "0") == "1":
            raise Exl3SelfCheckError(msg)
        logger.warning(msg)


def apply_exl3_experts(x, topk_ids, topk_weights, layer, *, limit: float = SWIGLU_LIMIT_DEFAULT,
                       fused: bool | None = None) -> torch.Tensor:
    """Routed-expert apply (recipe-lna/vllm_exl3_exl3.py.lna:1707-1779): the
    routed kernel when selected and able, else the LinearEXL3 loop.  `fused`
    False forces the loop; True requires the pointer tables.  Output has x's
    shape and dtype."""
    inners = getattr(layer, "_exl3_inners", None)
    if not inners:
        raise RuntimeError("EXL3 experts were not built after weight load")
    tokens, hidden = x.shape[-2], x.shape[-1]
    x2d = x.reshape(tokens, hidden)
    ids = topk_ids.reshape(tokens, -1)
    if ids.dtype not in (torch.int32, torch.int64):
        ids = ids.to(torch.long)
    weights = topk_weights.reshape(tokens, -1)
    expert_map = pin_exl3_expert_map(layer, x2d.device)
    have_ptrs = bool(getattr(layer, "_exl3_ptrs", None))
    if fused is True and not have_ptrs:
        raise RuntimeError("EXL3 fused apply requested but pointer tables are missing")
    if get_moe_kernel_backend() == "lna2" and fused is not False:
        try:
            res = _apply_lna2_moe(x2d, ids, weights, layer, inners, expert_map, limit)
        except Exception as exc:
            if moe_kernel_strict() or isinstance(exc, Exl3SelfCheckError):
                raise
            res = None
            layer._exl3_lna2_error = repr(exc)
            logger.warning("LNA2 dispatch failed; falling back: %s", exc)
        if res is not None:
            layer._exl3_last_apply = "lna2" if int(x2d.shape[0]) <= lna2_max_rows() else "prefill"
            _lna2_log_active()
            return res.to(dtype=x.dtype).reshape(x.shape)
    out = apply_exl3_python_loop(x2d, ids, weights, inners, expert_map, limit)
    _MOE_CALLS["loop"] += 1
    layer._exl3_last_apply = "loop"
    return out.to(dtype=x.dtype).reshape(x.shape)


# ---------------------------------------------------------------- TP sharding of packed tensors


def _narrow_tp(t: torch.Tensor, dim: int, rank: int, size: int) -> torch.Tensor:
    if size == 1:
        return t
    n = t.shape[dim]
    if n % size:
        raise ValueError(f"dimension {dim} of size {n} does not split over {size} ranks")
    step = n // size
    return t.narrow(dim, rank * step, step).contiguous()


def shard_exl3_col(loaded: torch.Tensor, suffix: str, tp_rank: int, tp_size: int) -> torch.Tensor:
    """Column split (output features): trellis dim 1, svh (recipe-lna/vllm_exl3_exl3.py.lna:855-861)."""
    if suffix == "trellis":
        return _narrow_tp(loaded, 1, tp_rank, tp_size)
    if suffix == "svh":
        return _narrow_tp(loaded, 0, tp_rank, tp_size)
    return loaded


def shard_exl3_row(loaded: torch.Tensor, suffix: str, tp_rank: int, tp_size: int) -> torch.Tensor:
    """Row split (input features): trellis dim 0, suh (recipe-lna/vllm_exl3_exl3.py.lna:864-870)."""
    if suffix == "trellis":
        return _narrow_tp(loaded, 0, tp_rank, tp_size)
    if suffix == "suh":
        return _narrow_tp(loaded, 0, tp_rank, tp_size)
    return loaded


def _suffix_from_mapped_name(weight_name: str) -> str:
    tail = weight_name.rsplit(".", 1)[-1]
    for suffix in EXL3_SUFFIXES:
        if tail == suffix or tail.endswith("_" + suffix):
            return suffix
    raise ValueError(f"not an EXL3 packed name: {weight_name}")


# ---------------------------------------------------------------- quantization config

SUPPORTED_BITS = (2, 3, 4, 5, 6)
_LAYER_RE = re.compile(r"(?:^|\.)layers\.(\d+)(?:\.|$)")


def _prefix_has_suffix(prefix: str, suffix: str) -> bool:
    return prefix == suffix or prefix.endswith("." + suffix)


class Exl3Config:
    """The pack's ``quantization_config`` for this path
    (recipe-lna/vllm_exl3_exl3.py.lna:1795-1960): routed experts at ``bits``
    with an optional per-layer ``layer_bits`` override (a mixed-K pack), and
    the optional ``non_routed_exl3`` block that names which dense linears are
    EXL3 and at which K.  Same validation and error text classes."""

    def __init__(self, bits: int = 4, codebook: str = "mcg", scope: str = "glm53_routed_experts_only",
                 **kwargs: Any) -> None:
        self.bits = int(bits)
        self.codebook = str(codebook)
        self.scope = str(scope)
        raw = kwargs.pop("layer_bits", None) or {}
        self.layer_bits: dict[int, int] = {int(k): int(v) for k, v in dict(raw).items()}
        for idx, k in self.layer_bits.items():
            if k not in SUPPORTED_BITS:
                raise ValueError(f"unsupported EXL3 bits={k} for layer {idx}")
        self.non_routed_exl3: dict[str, Any] = dict(kwargs.pop("non_routed_exl3", None) or {})
        nr = self.non_routed_exl3
        if nr.get("bits") is not None and nr["bits"] not in SUPPORTED_BITS:
            raise ValueError(f"unsupported non_routed_exl3 bits={nr['bits']}")
        for suffix, k in (nr.get("layer_bits") or {}).items():
            if k not in SUPPORTED_BITS:
                raise ValueError(f"unsupported non_routed_exl3 bits={k} for suffix {suffix}")
        for prefix, cfg in (nr.get("layers") or {}).items():
            if not isinstance(cfg, dict):
                raise ValueError(f"non_routed_exl3 layers[{prefix}] must be a dict, got {type(cfg)}")
            if cfg.get("bits") is not None and cfg["bits"] not in SUPPORTED_BITS:
                raise ValueError(f"unsupported non_routed_exl3 layers[{prefix}] bits={cfg['bits']}")
        if nr.get("codebook", "mcg") not in ("mcg", "mul1"):
            raise ValueError(f"unsupported non_routed_exl3 codebook={nr.get('codebook')!r}; must be 'mcg' or 'mul1'")
        self.extra = kwargs
        if self.codebook not in ("mcg", "mul1"):
            raise ValueError(f"unsupported codebook={self.codebook!r}; must be 'mcg' or 'mul1'")
        if self.bits not in SUPPORTED_BITS:
            raise ValueError(f"unsupported EXL3 bits={self.bits}")

    @classmethod
    def from_config(cls, config: dict[str, Any]) -> "Exl3Config":
        skip = {"bits", "codebook", "scope", "quant_method", "tensor_storage", "non_routed_exl3",
                "non_routed_quantization", "mtp_experts", "mtp_experts_start_layer"}
        return cls(bits=int(config.get("bits", 4)), codebook=str(config.get("codebook", "mcg")),
                   scope=str(config.get("scope", "glm53_routed_experts_only")),
                   non_routed_exl3=config.get("non_routed_exl3"),
                   **{k: v for k, v in config.items() if k not in skip})

    def get_name(self) -> str:
        return "exl3"

    def bits_for_prefix(self, prefix: str) -> int:
        """Routed-expert K of the layer named in `prefix`: its layer_bits entry, else bits."""
        if not self.layer_bits:
            return self.bits
        m = _LAYER_RE.search(prefix or "")
        return self.bits if m is None else self.layer_bits.get(int(m.group(1)), self.bits)

    def _matches_non_routed_exl3(self, prefix: str) -> bool:
        nr = self.non_routed_exl3
        if not nr:
            return False
        if prefix in (nr.get("layers") or {}):
            return True
        return any(_prefix_has_suffix(prefix, m) for m in (nr.get("modules") or []))

    def _bits_for_non_routed(self, prefix: str) -> int:
        nr = self.non_routed_exl3
        if not nr:
            return self.bits
        layers = nr.get("layers") or {}
        if prefix in layers:
            return int(layers[prefix].get("bits", nr.get("bits", self.bits)))
        matched = next((s for s in (nr.get("modules") or []) if _prefix_has_suffix(prefix, s)), None)
        if matched is None:
            return self.bits
        return int((nr.get("layer_bits") or {}).get(matched, nr.get("bits", self.bits)))

    def _bf16_shards_for(self, prefix: str) -> list[int]:
        layers = (self.non_routed_exl3 or {}).get("layers") or {}
        return list(layers[prefix].get("bf16_shards", [])) if prefix in layers else []


# ---------------------------------------------------------------- vLLM quant methods


class Exl3MoEMethod:
    """Packed MCG trellis routed experts: create / load / finalize / apply
    (recipe-lna/vllm_exl3_exl3.py.lna:2045-2307).  One bit width per layer, as
    in the checkpoint ABI (w13_* [E, 2, ...], w2_* [E, ...])."""

    def __init__(self, moe=None, quant_config=None, bits: int | None = None, tp_rank: int = 0, tp_size: int = 1):
        self.moe = moe
        self.quant_config = quant_config
        self.bits = int(bits) if bits is not None else int(getattr(quant_config, "bits", 0))
        self.tp_rank, self.tp_size = tp_rank, tp_size

    def get_fused_moe_quant_config(self, layer):
        return None

    def create_weights(self, layer, num_experts: int, hidden_size: int, intermediate_size_per_partition: int,
                       params_dtype=None, **extra_weight_attrs) -> None:
        del params_dtype, extra_weight_attrs
        inter = intermediate_size_per_partition
        if hidden_size % 16 or inter % 16:
            raise ValueError(f"EXL3 trellis tiles are 16-wide; hidden={hidden_size} intermediate_local={inter}")
        kw, it, ot = self.bits * 16, hidden_size // 16, inter // 16
        shapes = {
            "w13_trellis": ((num_experts, 2, it, ot, kw), torch.int16),
            "w13_suh": ((num_experts, 2, hidden_size), torch.float16),
            "w13_svh": ((num_experts, 2, inter), torch.float16),
            "w13_mcg": ((num_experts, 2, 1), torch.int32),
            "w2_trellis": ((num_experts, ot, it, kw), torch.int16),
            "w2_suh": ((num_experts, inter), torch.float16),
            "w2_svh": ((num_experts, hidden_size), torch.float16),
            "w2_mcg": ((num_experts, 1), torch.int32),
        }
        for name, (shape, dt) in shapes.items():
            p = Parameter(torch.empty(shape, dtype=dt), requires_grad=False)
            p.weight_loader = self._load_exl3
            layer.register_parameter(name, p)
        layer._exl3_hidden_size = hidden_size
        layer._exl3_intermediate_local = inter
        layer._exl3_k_words = kw
        layer._exl3_bits = self.bits

    def _load_exl3(self, param: Parameter, loaded_weight: torch.Tensor, weight_name: str,
                   shard_id: str = "w1", expert_id: int = 0, return_success: bool = False):
        """Copy one checkpoint tensor of one expert (w1 = gate, w3 = up, w2 =
        down) into its slot, TP-sharded (recipe-lna/vllm_exl3_exl3.py.lna:2147-2195)."""
        suffix = _suffix_from_mapped_name(weight_name)
        loaded = loaded_weight.detach().contiguous()
        if shard_id in ("w1", "w3"):
            sharded = shard_exl3_col(loaded, suffix, self.tp_rank, self.tp_size)
            dest = param.data[expert_id, 0 if shard_id == "w1" else 1]
        elif shard_id == "w2":
            sharded = shard_exl3_row(loaded, suffix, self.tp_rank, self.tp_size)
            dest = param.data[expert_id]
        else:
            raise ValueError(f"unknown EXL3 shard_id={shard_id}")
        if tuple(dest.shape) != tuple(sharded.shape):
            raise RuntimeError(f"EXL3 load shape mismatch {weight_name} shard={shard_id} expert={expert_id}: "
                               f"dest {tuple(dest.shape)} != loaded {tuple(sharded.shape)}")
        dest.copy_(sharded)
        return True if return_success else None

    def process_weights_after_loading(self, layer) -> None:
        if not hasattr(layer, "w13_trellis"):
            return
        for m in (layer.w13_mcg.reshape(-1), layer.w2_mcg.reshape(-1)):
            if not torch.all(m == MCG_MARKER_SIGNED_INT32):
                raise RuntimeError("EXL3 mcg marker is not the MCG int32 0xCBAC1FED / "
                                   f"{MCG_MARKER_SIGNED_INT32}; packed ABI mismatch")
        inners = []
        for e in range(int(layer.w13_trellis.shape[0])):
            inners.append({
                "gate": make_linear_exl3(layer.w13_trellis[e, 0], layer.w13_suh[e, 0], layer.w13_svh[e, 0],
                                         layer.w13_mcg[e, 0]),
                "up": make_linear_exl3(layer.w13_trellis[e, 1], layer.w13_suh[e, 1], layer.w13_svh[e, 1],
                                       layer.w13_mcg[e, 1]),
                "down": make_linear_exl3(layer.w2_trellis[e], layer.w2_suh[e], layer.w2_svh[e], layer.w2_mcg[e]),
            })
        layer._exl3_inners = inners
        if layer.w13_trellis.is_cuda:
            build_exl3_fused_state(layer, inners)

    def apply(self, layer, x, topk_weights, topk_ids, shared_experts=None, shared_experts_input=None):
        del shared_experts, shared_experts_input
        limit = getattr(self.moe, "swiglu_limit", None) or SWIGLU_LIMIT_DEFAULT
        return apply_exl3_experts(x, topk_ids, topk_weights, layer, limit=float(limit))


_WO_A_SLICE_RE = re.compile(r"wo_a\.slice\.(?P<rank>\d+)")
WO_A_TP_SIZE = 8


def _wo_a_slice_rank(loaded_shard_id) -> int | None:
    """Group rank named by a wo_a shard id: an int, a digit string or a
    ``wo_a.slice.N`` name (recipe-lna/vllm_exl3_exl3.py.lna:833-843)."""
    if isinstance(loaded_shard_id, int):
        return loaded_shard_id
    if loaded_shard_id is None:
        return None
    text = str(loaded_shard_id)
    if text.isdigit():
        return int(text)
    match = _WO_A_SLICE_RE.search(text)
    return int(match.group("rank")) if match else None


def _is_wo_a_layer(layer) -> bool:
    """The attention output's low-rank input projection, stored as one
    pre-sliced group per TP rank (recipe-lna/vllm_exl3_exl3.py.lna:846-852)."""
    prefix = str(getattr(layer, "prefix", ""))
    return _prefix_has_suffix(prefix, "attn.wo_a") or (bool(getattr(layer, "is_bmm", False))
                                                        and prefix.endswith(".wo_a"))


class Exl3LinearMethod:
    """EXL3 dense linear with one or more same-input output shards, some of
    which may be plain bf16 (recipe-lna/vllm_exl3_exl3.py.lna:2310-2853)."""

    def __init__(self, quant_config=None, bits: int | None = None, tp_rank: int = 0, tp_size: int = 1):
        self.quant_config = quant_config
        self.bits = int(bits) if bits is not None else int(getattr(quant_config, "bits", 0))
        self.tp_rank, self.tp_size = tp_rank, tp_size

    def create_weights(self, layer, input_size_per_partition: int, output_partition_sizes: list[int],
                       input_size: int = 0, output_size: int = 0, params_dtype=None, *,
                       is_row_parallel: bool = False, **extra_weight_attrs):
        """Fused parameters over the module's same-input output shards
        (recipe-lna/vllm_exl3_exl3.py.lna:2323-2493).  vLLM tells row from
        column parallelism by the layer class; here the caller says which.
        Shards the config lists as bf16 (``non_routed_exl3.layers[prefix]
        .bf16_shards``) load into a bf16 ``weight`` staging parameter instead;
        a wo_a module holds one pre-sliced group per TP rank (TP 8 only).
        Every parameter gets a weight_loader bound to its tensor kind."""
        del input_size, output_size, extra_weight_attrs
        k = input_size_per_partition
        for i, n in enumerate(output_partition_sizes):
            if k % 16 or n % 16:
                raise ValueError(f"EXL3 trellis tiles are 16-wide; shard {i}: in={k} out={n}")
        is_wo_a = _is_wo_a_layer(layer)
        if is_wo_a and self.tp_size != WO_A_TP_SIZE:
            raise NotImplementedError("EXL3 wo_a requires TP=8 (one local group per rank); "
                                      f"got tp_size={self.tp_size}")
        bf16 = self.quant_config._bf16_shards_for(getattr(layer, "prefix", "")) \
            if hasattr(self.quant_config, "_bf16_shards_for") else []
        if bf16 and self.tp_size > 1:
            raise RuntimeError(f"EXL3 bf16 shards are not supported with TP size > 1; tp_size={self.tp_size}")
        if any(not 0 <= i < len(output_partition_sizes) for i in bf16):
            raise ValueError(f"bf16 shard indices {bf16} outside the module's {len(output_partition_sizes)} shards")
        n_shards = len(output_partition_sizes)
        total_tiles = sum(n // 16 for n in output_partition_sizes)
        params = {
            "trellis": torch.empty(k // 16, total_tiles, self.bits * 16, dtype=torch.int16),
            "suh": torch.empty(n_shards, k, dtype=torch.float16),
            "svh": torch.empty(sum(output_partition_sizes), dtype=torch.float16),
            "mcg": torch.zeros(n_shards, 1, dtype=torch.int32),
            "mul1": torch.zeros(n_shards, 1, dtype=torch.int32),
        }
        if not is_wo_a:
            bf16_rows = sum(output_partition_sizes[i] for i in bf16)
            params["weight"] = torch.empty(bf16_rows, k, dtype=params_dtype or torch.bfloat16)
        for name, t in params.items():
            p = Parameter(t, requires_grad=False)
            p.weight_loader = self._make_weight_loader(name, n_shards, list(output_partition_sizes),
                                                       is_row_parallel, list(bf16), is_wo_a)
            layer.register_parameter(name, p)
        layer._exl3_linear_n_shards = n_shards
        layer._exl3_linear_output_partition_sizes = list(output_partition_sizes)
        layer._exl3_linear_input_size_per_partition = k
        layer._exl3_linear_is_row_parallel = bool(is_row_parallel)
        layer._exl3_linear_bf16_shards = list(bf16)
        layer._exl3_linear_is_wo_a = is_wo_a
        layer._exl3_linear_tp_size = self.tp_size
        layer._exl3_linear_tp_rank = self.tp_rank

    def _make_weight_loader(self, suffix: str, n_shards: int, sizes: list[int], is_row_parallel: bool,
                            bf16: list[int], is_wo_a: bool):
        """weight_loader(param, loaded_weight[, shard_id]) for one tensor kind
        (recipe-lna/vllm_exl3_exl3.py.lna:2495-2633): shard ids "q"/"k"/"v" or
        an int name the fused output shard; trellis/suh/svh are TP-narrowed
        (row: trellis dim 0 + suh, column: trellis dim 1 + svh) and copied into
        the shard's slice; mcg/mul1 store the marker value; ``weight`` keeps
        only the bf16 shards' rows (an EXL3 shard's stale bf16 copy is
        dropped).  For wo_a the shard id is the group rank (``wo_a.slice.N``)
        and only this rank's group, already sliced, is kept."""
        tp_rank, tp_size = self.tp_rank, self.tp_size

        def load_wo_a(param: Parameter, loaded_weight: torch.Tensor, loaded_shard_id) -> None:
            rank = _wo_a_slice_rank(loaded_shard_id)
            if rank is None:
                raise ValueError("EXL3 wo_a loader requires a wo_a.slice.N shard id")
            if rank != tp_rank:
                return
            loaded = loaded_weight.detach().contiguous()
            if suffix in ("mcg", "mul1"):
                param.data[0, 0] = int(loaded.item()) if loaded.numel() else 0
                return
            dest = {"trellis": param.data, "suh": param.data[0], "svh": param.data}.get(suffix)
            if dest is None:
                raise ValueError(f"unknown EXL3 wo_a suffix={suffix}")
            if tuple(dest.shape) != tuple(loaded.shape):
                raise RuntimeError(f"EXL3 wo_a load shape mismatch slice={rank} suffix={suffix}: "
                                   f"dest {tuple(dest.shape)} != loaded {tuple(loaded.shape)}")
            dest.copy_(loaded)

        def weight_loader(param: Parameter, loaded_weight: torch.Tensor, loaded_shard_id=None) -> None:
            if is_wo_a:
                return load_wo_a(param, loaded_weight, loaded_shard_id)
            shard_idx = 0
            if isinstance(loaded_shard_id, str):
                shard_map = {"q": 0, "k": 1, "v": 2}
                if loaded_shard_id not in shard_map:
                    raise ValueError(f"unknown shard_id={loaded_shard_id} for EXL3 linear")
                shard_idx = shard_map[loaded_shard_id]
            elif isinstance(loaded_shard_id, int):
                shard_idx = loaded_shard_id
            if shard_idx >= n_shards:
                raise ValueError(f"shard_idx={shard_idx} out of range for n_shards={n_shards}")
            if suffix in ("mcg", "mul1"):
                dest = param.data[shard_idx]
                if tuple(dest.shape) != (1,):
                    raise RuntimeError(f"EXL3 {suffix} marker shape mismatch: expected (1,) got {tuple(dest.shape)}")
                dest[0] = int(loaded_weight.detach().item()) if loaded_weight.numel() > 0 else 0
                return
            if suffix == "weight":
                want = (sizes[shard_idx], param.shape[1])
                loaded = loaded_weight.detach()
                if tuple(loaded.shape) != want:
                    raise RuntimeError(f"EXL3 weight load shape mismatch shard={shard_idx}: expected {want} "
                                       f"got {tuple(loaded.shape)}")
                if shard_idx in bf16:
                    r0 = sum(sizes[i] for i in bf16[: bf16.index(shard_idx)])
                    param.data[r0:r0 + sizes[shard_idx]].copy_(loaded)
                return
            loaded = loaded_weight.detach().contiguous()
            sharded = (shard_exl3_row if is_row_parallel else shard_exl3_col)(loaded, suffix, tp_rank, tp_size)
            if suffix == "trellis":
                t0 = sum(s // 16 for s in sizes[:shard_idx])
                dest = param.data[:, t0:t0 + sizes[shard_idx] // 16, :]
            elif suffix == "suh":
                dest = param.data[shard_idx]
            elif suffix == "svh":
                o0 = sum(sizes[:shard_idx])
                dest = param.data[o0:o0 + sizes[shard_idx]]
            else:
                raise ValueError(f"unknown EXL3 suffix={suffix}")
            if tuple(dest.shape) != tuple(sharded.shape):
                raise RuntimeError(f"EXL3 linear load shape mismatch shard={shard_idx} suffix={suffix}: "
                                   f"dest {tuple(dest.shape)} != loaded {tuple(sharded.shape)}")
            dest.copy_(sharded)

        return weight_loader

    def process_weights_after_loading(self, layer) -> None:
        """The reference's post-load lifecycle (recipe-lna/vllm_exl3_exl3.py.lna:2649-2768):
        check each EXL3 shard's codebook marker; build one LinearEXL3 per EXL3
        shard (None for bf16 shards, whose rows are kept as
        ``_exl3_bf16_weight``); free the fused staging parameters, so only the
        per-shard tensors stay resident; register the module's T0 group (and
        its T1 fan); then run every linear and the group once per
        LNA_EXL3_PREWARM_ROWS row count, so the shared scratch exists before
        any graph capture."""
        if not hasattr(layer, "trellis"):
            return
        sizes = layer._exl3_linear_output_partition_sizes
        bf16 = list(getattr(layer, "_exl3_linear_bf16_shards", []))
        mcg_vals = [int(v) for v in layer.mcg.reshape(-1).tolist()]
        mul1_vals = [int(v) for v in layer.mul1.reshape(-1).tolist()]
        linears, t0, o0 = [], 0, 0
        for i, n in enumerate(sizes):
            if i in bf16:
                linears.append(None)
            else:
                mcg_set, mul1_set = mcg_vals[i] != 0, mul1_vals[i] != 0
                if mcg_set == mul1_set:
                    raise RuntimeError(f"EXL3 linear shard {i}: {'both' if mcg_set else 'neither'} mcg and mul1 "
                                       "markers are set; exactly one codebook marker must be present")
                if mcg_set and mcg_vals[i] != MCG_MARKER_SIGNED_INT32:
                    raise RuntimeError(f"EXL3 linear shard {i}: mcg marker is {mcg_vals[i]}, expected "
                                       f"{MCG_MARKER_SIGNED_INT32}")
                if mul1_set and mul1_vals[i] != MUL1_MARKER_SIGNED_INT32:
                    raise RuntimeError(f"EXL3 linear shard {i}: mul1 marker is {mul1_vals[i]}, expected "
                                       f"{MUL1_MARKER_SIGNED_INT32}")
                trellis = layer.trellis[:, t0:t0 + n // 16].contiguous()
                if trellis.data_ptr() == layer.trellis.data_ptr() and len(sizes) > 1:
                    trellis = trellis.clone()
                linears.append(make_linear_exl3(trellis, layer.suh[i].clone(), layer.svh[o0:o0 + n].clone(),
                                                layer.mcg[i].clone() if mcg_set else None,
                                                layer.mul1[i].clone() if mul1_set else None))
            t0 += n // 16
            o0 += n
        layer._exl3_linears = linears
        weight = getattr(layer, "weight", None)
        layer._exl3_bf16_weight = weight.data.clone() if bf16 and weight is not None else None
        for name in ("weight", "trellis", "suh", "svh", "mcg", "mul1"):
            if hasattr(layer, name):
                delattr(layer, name)
        build_exl3_dense_group(layer)
        self._prewarm(layer)

    @staticmethod
    def _prewarm(layer) -> None:
        """Reserve the shared scratch of every call this module can make before
        any graph capture: each shard's GEMV for every row count it takes (up
        to AUTO_RECONSTRUCT_THRESHOLD rows, whatever LNA_EXL3_PREWARM_ROWS
        says: a capture at a row count without an earlier eager call would
        otherwise need a larger buffer), and the fused group at its row counts
        (up to DENSE_GROUP_MAX_ROWS)."""
        lins = [lin for lin in layer._exl3_linears if lin is not None]
        if not lins or lins[0].trellis.device.type != "cuda":
            return
        dev = lins[0].trellis.device
        try:
            before = _vram_mark(dev)
            for lin in lins:
                ops.prepare_gemm(dev, AUTO_RECONSTRUCT_THRESHOLD, int(lin.in_features), int(lin.out_features))
            _vram_report("registration.gemv_scratch", getattr(layer, "prefix", "?"), before, _vram_mark(dev))
            prewarm_exl3_dense_group(layer)
        except Exception as exc:
            logger.warning("EXL3 prewarm skipped for %s: %s", getattr(layer, "prefix", "?"), exc)

    def apply(self, layer, x: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
        """recipe-lna/vllm_exl3_exl3.py.lna:2770-2853: EXL3 shards on a
        contiguous fp16 copy of x (through the module's T0 group or T1 fan when
        LNA_EXL3_DENSE_GROUP asks for one), bf16 shards as plain linears,
        outputs concatenated in shard order, cast to x's dtype, + bias."""
        linears = getattr(layer, "_exl3_linears", None)
        if not linears:
            raise RuntimeError("EXL3 linear layers were not built after weight load")
        orig = x.shape
        x2 = x.reshape(-1, orig[-1])
        xh = x2.to(torch.float16).contiguous()
        bf16 = getattr(layer, "_exl3_linear_bf16_shards", [])
        sizes = layer._exl3_linear_output_partition_sizes
        if not bf16 and (len(linears) > 1 or (dense_group_mode() == 2
                                              and getattr(layer, "_exl3_dense_fan", None) is not None)):
            outs = run_exl3_group(layer, xh, torch.float32, source_tensor=x2)
        else:
            outs = []
            weight = getattr(layer, "_exl3_bf16_weight", None)
            for i, lin in enumerate(linears):
                if i in bf16:
                    if weight is None:
                        raise RuntimeError(f"EXL3 bf16 shard {i} but _exl3_bf16_weight is missing")
                    r0 = sum(sizes[j] for j in bf16[: bf16.index(i)])
                    outs.append(F.linear(x2.to(weight.dtype), weight[r0:r0 + sizes[i]]).to(torch.float32))
                elif lin is None:
                    raise RuntimeError(f"EXL3 linear shard {i} is None")
                else:
                    outs.append(lin.forward(xh, {}, out_dtype=torch.float32))
        # a fresh tensor always: fused-fan outputs are views its next call reuses
        y = torch.cat(outs, dim=1) if len(outs) > 1 else outs[0].to(x.dtype, copy=True)
        if y.dtype != x.dtype:
            y = y.to(x.dtype)
        if bias is not None:
            y = y + bias
        return y.reshape(*orig[:-1], y.shape[-1])
