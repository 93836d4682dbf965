"""CPU tests of the host side: the C-ABI library loads and exports every symbol
include/exl3_amd.h declares, its argument checks answer without a device, and
the plugin surface's dispatch / routing / loader logic (no kernel launches)."""

from __future__ import annotations

import ctypes
import os
import re
import subprocess

import numpy as np
import pytest
import torch

from dsv4_carve_amd import _lib, ops
from dsv4_carve_amd import vllm_exl3 as V

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "exl3_amd.h")


def header_symbols() -> set[str]:
    text = open(HEADER).read()
    return set(re.findall(r"^[a-z][\w\s\*]*?\b(exl3_\w+)\s*\(", text, flags=re.M))


def test_header_matches_binding_table():
    assert header_symbols() == set(_lib.EXPORTS)
    assert set(_lib._SIGS) == set(_lib.EXPORTS)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in header_symbols():
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l}
    assert header_symbols() <= exported


def test_library_targets_gfx950_only():
    # the code object bundle names its targets; there is exactly one
    blob = open(_lib.LIB_PATH, "rb").read()
    targets = set(re.findall(rb"amdgcn-amd-amdhsa--(gfx\w+)", blob))
    assert targets == {b"gfx950"}, targets


def _err():
    return _lib.load().exl3_last_error().decode()


def test_moe_host_arithmetic_without_device():
    lib = _lib.load()
    assert lib.exl3_moe_max_rows() == 32
    a = lib.exl3_moe_scratch_bytes(4096, 2048, 8)
    b = lib.exl3_moe_scratch_bytes(4096, 256, 6)
    assert a > b > 0 and a % 256 == 0
    assert lib.exl3_moe_scratch_bytes(4000, 2048, 8) == -1 and "multiples of 256" in _err()
    assert lib.exl3_moe_scratch_bytes(4096, 2048, 10) == -1 and "topk" in _err()
    assert lib.exl3_moe_scratch_bytes(4096, 2048, 9) > 0
    assert lib.exl3_moe_scratch_bytes(16640, 256, 8) == -1 and "16384" in _err()
    # up to 16 rows one size; past 16 rows the data regions grow with the row count
    assert lib.exl3_moe_scratch_bytes_rows(4096, 2048, 8, 1) == lib.exl3_moe_scratch_bytes_rows(4096, 2048, 8, 16) == a
    a24, a32 = lib.exl3_moe_scratch_bytes_rows(4096, 2048, 8, 24), lib.exl3_moe_scratch_bytes_rows(4096, 2048, 8, 32)
    assert a < a24 < a32 and a32 % 256 == 0
    assert lib.exl3_moe_scratch_bytes_rows(4096, 2048, 8, 33) == -1 and "row count" in _err()
    assert lib.exl3_moe_scratch_bytes_rows(4096, 2048, 8, 0) == -1 and "row count" in _err()


def _moe_call(**kw):
    lib = _lib.load()
    one = ctypes.c_void_p(16)
    args = dict(x=one, x_kind=0, out=one, out_kind=2, m=1, hidden=512, intermediate=256, n_experts=4, topk=2,
                tabs=[one] * 9, ids=one, w=one, ebits=None, bits=3, mask=0, cb=1, limit=10.0, scratch=one,
                scratch_bytes=1 << 30, stream=None)
    args.update(kw)
    return lib.exl3_moe_decode(args["x"], args["x_kind"], args["out"], args["out_kind"], args["m"], args["hidden"],
                               args["intermediate"], args["n_experts"], args["topk"], *args["tabs"], args["ids"],
                               args["w"], args["ebits"], args["bits"], args["mask"], args["cb"], args["limit"],
                               args["scratch"], args["scratch_bytes"], args["stream"])


@pytest.mark.parametrize("kw,msg", [
    ({"x": None}, "null pointer"),
    ({"tabs": [ctypes.c_void_p(16)] * 8 + [None]}, "null pointer table"),
    ({"x_kind": 2}, "fp16 or bf16"),
    ({"out_kind": 3}, "fp16, bf16 or fp32"),
    ({"m": 0}, "row count"),
    ({"m": 33}, "row count"),
    ({"hidden": 500}, "multiples of 256"),
    ({"intermediate": 128}, "multiples of 256"),
    ({"n_experts": 0}, "expert count"),
    ({"topk": 10}, "topk"),
    ({"hidden": 16640}, "16384"),
    ({"limit": 0.0}, "SwiGLU limit"),
    ({"limit": float("inf")}, "SwiGLU limit"),
    ({"limit": float("nan")}, "SwiGLU limit"),
    ({"cb": 3}, "codebook"),
    ({"bits": 0}, "bits must be in 1..8"),
    ({"bits": 9}, "bits must be in 1..8"),
    ({"ebits": ctypes.c_void_p(16), "mask": 1}, "bits_mask"),
    ({"ebits": ctypes.c_void_p(16), "mask": 0}, "bits_mask"),
    ({"scratch_bytes": 16}, "scratch too small"),
])
def test_moe_argument_errors_without_device(kw, msg):
    assert _moe_call(**kw) == -1
    assert msg in _err()


def _routed_call(entry, **kw):
    lib = _lib.load()
    one = ctypes.c_void_p(16)
    a = dict(x=one, x_kind=0, out=one, out_kind=2, m=1, hidden=512, intermediate=256, n_experts=4, topk=2,
             tabs=[one] * 9, ids=one, ids_kind=1, w=one, w_kind=1, emap=None, n_global=0, ebits=None, bits=3,
             mask=0, cb=1, limit=10.0, scratch=one, scratch_bytes=1 << 30, stream=None)
    a.update(kw)
    return getattr(lib, entry)(a["x"], a["x_kind"], a["out"], a["out_kind"], a["m"], a["hidden"], a["intermediate"],
                               a["n_experts"], a["topk"], *a["tabs"], a["ids"], a["ids_kind"], a["w"], a["w_kind"],
                               a["emap"], a["n_global"], a["ebits"], a["bits"], a["mask"], a["cb"], a["limit"],
                               a["scratch"], a["scratch_bytes"], a["stream"])


@pytest.mark.parametrize("entry", ["exl3_moe_decode_routed", "exl3_moe_prefill_routed"])
@pytest.mark.parametrize("kw,msg", [
    ({"ids_kind": 2}, "int32 or int64"),
    ({"w_kind": 3}, "fp16, bf16 or fp32"),
    ({"emap": ctypes.c_void_p(16), "n_global": 0}, "expert map length"),
    ({"emap": ctypes.c_void_p(16), "n_global": (1 << 20) + 1}, "expert map length"),
    ({"ids": None}, "null pointer"),
    ({"w": None}, "null pointer"),
    ({"hidden": 500}, "multiples of 256"),
    ({"limit": 0.0}, "SwiGLU limit"),
])
def test_moe_routed_argument_errors_without_device(entry, kw, msg):
    assert _routed_call(entry, **kw) == -1
    assert msg in _err()


def test_prefill_input_alignment_without_device():
    """The prefill path reads 16-byte pieces of the input rows."""
    assert _routed_call("exl3_moe_prefill_routed", x=ctypes.c_void_p(18)) == -1
    assert "16-byte aligned" in _err()


def test_prefill_pair_limit_without_device():
    """One prefill call takes up to 65536 (token, slot) pairs: 8192 tokens at
    top-8 are accepted, one more token is refused by the sizing function and
    by the entry itself."""
    lib = _lib.load()
    assert lib.exl3_moe_prefill_scratch_bytes(8192, 4096, 2048, 8, 256) > 0
    assert lib.exl3_moe_prefill_scratch_bytes(8193, 4096, 2048, 8, 256) == -1 and "65536" in _err()
    assert _routed_call("exl3_moe_prefill_routed", m=32769, topk=2) == -1 and "65536" in _err()


def test_prefill_scratch_drops_where_k_stops_splitting():
    """The prefill GEMMs split K in two below 4096 (down) and 8192 (gate/up)
    (token, slot) pairs and keep it whole from there, so the scratch, which
    holds one fp32 partial per part, shrinks as a call crosses each count
    although the call grows (hidden 4096, intermediate 2048, top-8, 256
    experts: 511 -> 512 tokens crosses 4096 pairs, 1023 -> 1024 crosses 8192).
    Away from the two counts it grows with the tokens."""
    lib = _lib.load()
    size = lambda t: _lib.check(lib.exl3_moe_prefill_scratch_bytes(t, 4096, 2048, 8, 256))
    # the second down part ([pairs][hidden] fp32) goes away at 4096 pairs
    assert size(511) - size(512) > 0.9 * (511 * 8) * 4096 * 4
    # the second gate/up part ([2][pairs][intermediate] fp32) at 8192
    assert size(1023) - size(1024) > 0.9 * 2 * (1023 * 8) * 2048 * 4
    for t in (100, 600, 2000):
        assert size(t + 1) > size(t)


@pytest.mark.parametrize("k,n,cb,kind,msg", [
    (100, 256, 1, 2, "k must be a positive multiple of 128"),
    (256, 100, 1, 2, "n must be a positive multiple of 128"),
    (256, 256, 5, 2, "codebook"),
    (256, 256, 1, 7, "c_kind"),
])
def test_gemm_argument_errors_without_device(k, n, cb, kind, msg):
    lib = _lib.load()
    p = ctypes.c_void_p(16)
    assert lib.exl3_gemm(p, 1, k, p, n, 3, cb, p, p, p, kind, p, 1 << 30, None) == -1
    assert msg in _err()


@pytest.mark.parametrize("m,k,ns,msg", [
    (0, 512, [256], "m must be positive"),
    (1, 500, [256], "k must be a positive multiple of 128"),
    (1, 512, [], "1..8"),
    (1, 512, [256] * 9, "1..8"),
    (1, 512, [256, 100], "every n must be a positive multiple of 128"),
])
def test_gemm_group_argument_errors_without_device(m, k, ns, msg):
    lib = _lib.load()
    arr = (ctypes.c_int64 * max(len(ns), 1))(*ns)
    assert lib.exl3_gemm_group_scratch_bytes(m, k, len(ns), arr) == -1 and msg in _err()
    p = ctypes.c_void_p(16)
    ptrs = (ctypes.c_void_p * 9)(*([16] * 9))
    bits = (ctypes.c_int32 * 9)(*([3] * 9))
    assert lib.exl3_gemm_group(p, m, k, len(ns), ptrs, ptrs, ptrs, arr, bits, 1, ptrs, 2, p, 1 << 30, None) == -1
    assert msg in _err()


def test_gemm_group_width_and_kind_errors_without_device():
    lib = _lib.load()
    arr = (ctypes.c_int64 * 2)(256, 512)
    p = ctypes.c_void_p(16)
    ptrs = (ctypes.c_void_p * 2)(16, 16)
    assert lib.exl3_gemm_group(p, 1, 512, 2, ptrs, ptrs, ptrs, arr, (ctypes.c_int32 * 2)(3, 9), 1, ptrs, 2, p,
                               1 << 30, None) == -1 and "bits" in _err()
    assert lib.exl3_gemm_group(p, 1, 512, 2, ptrs, ptrs, ptrs, arr, (ctypes.c_int32 * 2)(3, 4), 1, ptrs, 5, p,
                               1 << 30, None) == -1 and "c_kind" in _err()


@pytest.mark.parametrize("env,want,fallback", [(None, 0, False), ("0", 0, False), ("1", 1, False), ("2", 2, False),
                                               ("x", 0, True), ("3", 0, True)])
def test_dense_group_mode(monkeypatch, env, want, fallback):
    V.reset_dense_group_state()
    if env is None:
        monkeypatch.delenv("LNA_EXL3_DENSE_GROUP", raising=False)
    else:
        monkeypatch.setenv("LNA_EXL3_DENSE_GROUP", env)
    assert V.dense_group_mode() == want
    assert any(k.startswith("config:") for k in V.dense_group_stats()["fallbacks"]) == fallback


def test_dense_group_registration_checks(monkeypatch):
    """Group descriptors: members must share in_features and codebook, carry
    no bias, and at most eight; a declined module is marked None."""
    monkeypatch.setenv("LNA_EXL3_DENSE_GROUP", "1")
    V.reset_dense_group_state()

    def lin(k, n, bits=3, mul1=False):
        t = torch.zeros((k // 16, n // 16, 16 * bits), dtype=torch.int16)
        mk = torch.tensor([V.MUL1_MARKER_SIGNED_INT32 if mul1 else V.MCG_MARKER_SIGNED_INT32])
        return V.make_linear_exl3(t, torch.ones(k, dtype=torch.float16), torch.ones(n, dtype=torch.float16),
                                  mcg=None if mul1 else mk, mul1=mk if mul1 else None)

    class M:
        def __init__(self, linears):
            self._exl3_linears = linears
            self.prefix = "model.layers.0.attn.fused_wqa_wkv"

    ok = M([lin(512, 256), lin(512, 384, bits=6)])
    V.build_exl3_dense_group(ok)
    assert ok._exl3_dense_group["ns"] == [256, 384] and ok._exl3_dense_group["k"] == 512
    for bad in (M([lin(512, 256), lin(256, 256)]), M([lin(512, 256), lin(512, 256, mul1=True)]),
                M([lin(512, 256)] * 9)):
        V.build_exl3_dense_group(bad)
        assert bad._exl3_dense_group is None
    single = M([lin(512, 256)])
    V.build_exl3_dense_group(single)
    assert single._exl3_dense_group is None
    assert V.dense_group_stats()["fallbacks"]


def test_dequant_argument_errors_without_device():
    lib = _lib.load()
    p = ctypes.c_void_p(16)
    assert lib.exl3_dequant(p, 24, 32, 3, 1, None, None, p, None) == -1 and "multiples of 16" in _err()
    assert lib.exl3_dequant(p, 32, 32, 9, 1, None, None, p, None) == -1 and "bits" in _err()
    assert lib.exl3_dequant(p, 32, 32, 3, 1, p, None, p, None) == -1 and "both" in _err()
    assert lib.exl3_dequant(p, 32, 32, 3, 1, p, p, p, None) == -1 and "128" in _err()


def test_check_raises_library_message():
    lib = _lib.load()
    assert lib.exl3_moe_scratch_bytes(1, 1, 1) == -1
    with pytest.raises(_lib.Exl3Error, match="multiples of 256"):
        _lib.check(-1)


# ---------------------------------------------------------------- no CPU fallback


def test_ops_refuse_cpu_tensors():
    t = torch.zeros((8, 8, 48), dtype=torch.int16)
    with pytest.raises((NotImplementedError, RuntimeError)):
        ops.reconstruct_weight(t)
    x = torch.zeros((1, 128), dtype=torch.float16)
    with pytest.raises((NotImplementedError, RuntimeError)):
        ops.gemm(x, t, torch.ones(128, dtype=torch.float16), torch.ones(128, dtype=torch.float16))


# ---------------------------------------------------------------- plugin host logic


def test_map_topk_to_local_without_map():
    ids = torch.tensor([[0, 3, -1], [7, 2, 8]])
    got = V.map_topk_to_local(ids, 8, None).reshape(ids.shape)
    assert got.tolist() == [[0, 3, 8], [7, 2, 8]]


def test_map_topk_to_local_with_expert_map():
    emap = torch.tensor([-1, 0, 1, -1, 2, 3], dtype=torch.long)     # 6 global -> 4 local
    ids = torch.tensor([[1, 4, 0, 5], [6, -2, 2, 3]])
    got = V.map_topk_to_local(ids, 4, emap).reshape(ids.shape)
    assert got.tolist() == [[0, 2, 4, 3], [4, 4, 1, 4]]
    with pytest.raises(RuntimeError, match="not pinned"):
        V.map_topk_to_local(ids, 4, emap.to(torch.int32))
    assert V.map_topk_to_local(ids, 4, torch.empty(0, dtype=torch.long)).tolist() == [4] * 8


def test_pin_expert_map():
    class L:
        expert_map = torch.tensor([1, 0], dtype=torch.int32)

    layer = L()
    m = V.pin_exl3_expert_map(layer, torch.device("cpu"))
    assert m.dtype == torch.long and layer.expert_map is m
    assert V.pin_exl3_expert_map(object(), torch.device("cpu")) is None


@pytest.mark.parametrize("env,want", [(None, "lna2"), ("auto", "lna2"), ("LNA2", "lna2"), ("loop", "loop"),
                                      ("exllamav3", "lna2"), ("bogus", "lna2")])
def test_backend_selection(monkeypatch, env, want):
    if env is None:
        monkeypatch.delenv("VLLM_EXL3_MOE_KERNEL", raising=False)
    else:
        monkeypatch.setenv("VLLM_EXL3_MOE_KERNEL", env)
    assert V.get_moe_kernel_backend() == want


def test_strict_levels(monkeypatch):
    V._LNA2_REJECT_LOGGED.clear()
    monkeypatch.setenv("VLLM_EXL3_MOE_STRICT", "0")
    V._lna2_log_reject("shape a")
    V._lna2_log_reject("ready b", not_ready=True)
    assert V.moe_kernel_declined_reasons() == ["ready b", "shape a"]
    monkeypatch.setenv("VLLM_EXL3_MOE_STRICT", "1")
    V._lna2_log_reject("shape a")
    with pytest.raises(RuntimeError, match="STRICT=1"):
        V._lna2_log_reject("ready b", not_ready=True)
    monkeypatch.setenv("VLLM_EXL3_MOE_STRICT", "2")
    with pytest.raises(RuntimeError, match="STRICT=2"):
        V._lna2_log_reject("shape a")
    monkeypatch.setenv("VLLM_EXL3_MOE_STRICT", "x")
    assert V.moe_kernel_strict() == 0
    V._LNA2_REJECT_LOGGED.clear()


def test_unpack_bf():
    rng = np.random.default_rng(1)
    words = rng.integers(0, 1 << 16, 8, dtype=np.uint16)
    got = V.LinearEXL3.unpack_bf(torch.from_numpy(words.view(np.int16))).numpy()
    want = np.array([-1.0 if (int(w) >> i) & 1 else 1.0 for w in words for i in range(16)], np.float16)
    assert np.array_equal(got, want)


def test_linear_constructor_checks():
    t = torch.zeros((8, 8, 48), dtype=torch.int16)
    h = torch.ones(128, dtype=torch.float16)
    with pytest.raises(AssertionError, match="scale"):
        V.LinearEXL3(None, 128, 128, scale=torch.ones(1), suh=h, svh=h, trellis=t)
    with pytest.raises(AssertionError, match="trellis is wrong datatype"):
        V.LinearEXL3(None, 128, 128, suh=h, svh=h, trellis=t.float())
    with pytest.raises(AssertionError, match="suh"):
        V.LinearEXL3(None, 128, 128, suh=h.float(), svh=h, trellis=t)
    lin = V.LinearEXL3(None, 128, 128, suh=h, svh=h, trellis=t, mcg=torch.tensor([V.MCG_MARKER_SIGNED_INT32]))
    assert lin.K == 3 and lin.mcg and not lin.mul1 and lin.codebook == ops.CB_MCG
    with pytest.raises(AssertionError, match="non-contiguous"):
        lin.forward(torch.zeros((128, 2), dtype=torch.float16).t(), {})
    with pytest.raises(RuntimeError, match="Specified both"):
        V.LinearEXL3(None, 128, 128, suh=h, svh=h, trellis=t, mcg=torch.ones(1), mul1=torch.ones(1))


def test_tp_sharding_of_packed_tensors():
    t = torch.arange(4 * 8 * 32, dtype=torch.int16).reshape(4, 8, 32)
    col = V.shard_exl3_col(t, "trellis", 1, 2)
    assert torch.equal(col, t[:, 4:])
    row = V.shard_exl3_row(t, "trellis", 1, 4)
    assert torch.equal(row, t[1:2])
    v = torch.arange(8, dtype=torch.float16)
    assert torch.equal(V.shard_exl3_col(v, "svh", 0, 2), v[:4])
    assert torch.equal(V.shard_exl3_col(v, "suh", 0, 2), v)
    assert torch.equal(V.shard_exl3_row(v, "suh", 1, 2), v[4:])
    with pytest.raises(ValueError):
        V.shard_exl3_col(v, "svh", 0, 3)
    assert V._suffix_from_mapped_name("layers.3.ffn.experts.7.w1.trellis") == "trellis"
    assert V._suffix_from_mapped_name("experts.w13_svh") == "svh"
    with pytest.raises(ValueError):
        V._suffix_from_mapped_name("experts.w13_weight")


def _moe_layer_cpu(E=2, H=256, I=256, bits=2):
    layer = torch.nn.Module()
    meth = V.Exl3MoEMethod(bits=bits)
    meth.create_weights(layer, E, H, I)
    return layer, meth


def test_moe_method_create_and_load():
    layer, meth = _moe_layer_cpu()
    assert tuple(layer.w13_trellis.shape) == (2, 2, 16, 16, 32)
    assert tuple(layer.w2_trellis.shape) == (2, 16, 16, 32)
    tr = torch.ones((16, 16, 32), dtype=torch.int16)
    layer.w13_trellis.weight_loader(layer.w13_trellis, tr * 3, "experts.1.w3.trellis", "w3", 1)
    assert int(layer.w13_trellis[1, 1].sum()) == 3 * tr.numel() and int(layer.w13_trellis[1, 0].abs().sum()) >= 0
    with pytest.raises(RuntimeError, match="shape mismatch"):
        meth._load_exl3(layer.w2_trellis, tr[:8], "experts.0.w2.trellis", "w2", 0)
    with pytest.raises(ValueError, match="shard_id"):
        meth._load_exl3(layer.w2_trellis, tr, "experts.0.w2.trellis", "w4", 0)
    with pytest.raises(ValueError):
        V.Exl3MoEMethod(bits=2).create_weights(torch.nn.Module(), 2, 250, 256)


def test_moe_method_rejects_wrong_marker():
    layer, meth = _moe_layer_cpu()
    layer.w13_mcg.data.fill_(V.MCG_MARKER_SIGNED_INT32)
    layer.w2_mcg.data.fill_(V.MUL1_MARKER_SIGNED_INT32)
    with pytest.raises(RuntimeError, match="marker"):
        meth.process_weights_after_loading(layer)


def test_moe_apply_has_no_cpu_fallback():
    layer, meth = _moe_layer_cpu()
    for p in (layer.w13_trellis, layer.w2_trellis):
        p.data.zero_()
    for p in (layer.w13_suh, layer.w13_svh, layer.w2_suh, layer.w2_svh):
        p.data.fill_(1.0)
    layer.w13_mcg.data.fill_(V.MCG_MARKER_SIGNED_INT32)
    layer.w2_mcg.data.fill_(V.MCG_MARKER_SIGNED_INT32)
    meth.process_weights_after_loading(layer)
    assert len(layer._exl3_inners) == 2 and layer._exl3_inners[0]["down"].in_features == 256
    x = torch.zeros((1, 256), dtype=torch.float16)
    with pytest.raises((NotImplementedError, RuntimeError)):
        meth.apply(layer, x, torch.ones((1, 1)), torch.zeros((1, 1), dtype=torch.long))
    with pytest.raises(RuntimeError, match="not built"):
        V.apply_exl3_experts(x, torch.zeros((1, 1), dtype=torch.long), torch.ones((1, 1)), torch.nn.Module())


def test_linear_method_shards():
    layer = torch.nn.Module()
    meth = V.Exl3LinearMethod(bits=2)
    meth.create_weights(layer, 128, [256, 128], 128, 384)
    assert tuple(layer.trellis.shape) == (8, 24, 32) and tuple(layer.suh.shape) == (2, 128)
    layer.mcg.data.fill_(V.MCG_MARKER_SIGNED_INT32)
    layer.trellis.data.copy_(torch.arange(layer.trellis.numel(), dtype=torch.int32).reshape(8, 24, 32).to(torch.int16))
    fused = layer.trellis.detach().clone()
    meth.process_weights_after_loading(layer)
    a, b = layer._exl3_linears
    assert (a.out_features, b.out_features) == (256, 128)
    assert torch.equal(a.trellis, fused[:, :16]) and torch.equal(b.trellis, fused[:, 16:])
    assert a.trellis.is_contiguous() and b.trellis.is_contiguous()
    # the fused staging parameters are freed once the shards are built
    names = {n for n, _ in layer.named_parameters()}
    assert not names & {"trellis", "suh", "svh", "mcg", "mul1", "weight"}, names
    with pytest.raises(RuntimeError, match="not built"):
        meth.apply(torch.nn.Module(), torch.zeros(1, 128))


def test_linear_method_markers_checked():
    """Exactly one codebook marker per EXL3 shard, with the marker's value
    (recipe-lna/vllm_exl3_exl3.py.lna:2655-2690)."""
    for fill, msg in (((0, 0), "neither"), ((V.MCG_MARKER_SIGNED_INT32, V.MUL1_MARKER_SIGNED_INT32), "both"),
                      ((123, 0), "mcg marker is 123")):
        layer = torch.nn.Module()
        meth = V.Exl3LinearMethod(bits=2)
        meth.create_weights(layer, 128, [128], 128, 128)
        layer.mcg.data.fill_(fill[0])
        layer.mul1.data.fill_(fill[1])
        with pytest.raises(RuntimeError, match=msg):
            meth.process_weights_after_loading(layer)


def test_linear_method_bf16_shards_and_loader():
    """Shards the config lists as bf16 load into the bf16 staging weight (the
    EXL3 shards' stale bf16 copies are dropped) and are kept after processing
    as _exl3_bf16_weight, with no LinearEXL3 (recipe-lna/vllm_exl3_exl3.py.lna:2467-2600)."""
    cfg = V.Exl3Config(bits=2, non_routed_exl3={"layers": {"model.layers.0.attn.fused_qkv": {"bf16_shards": [1]}}})
    layer = torch.nn.Module()
    layer.prefix = "model.layers.0.attn.fused_qkv"
    meth = V.Exl3LinearMethod(cfg, bits=2)
    meth.create_weights(layer, 128, [128, 64, 128], 128, 320, params_dtype=torch.bfloat16)
    assert tuple(layer.weight.shape) == (64, 128) and layer.weight.dtype == torch.bfloat16
    w1 = torch.randn(64, 128).to(torch.bfloat16)
    layer.weight.weight_loader(layer.weight, torch.randn(128, 128).to(torch.bfloat16), 0)   # EXL3 shard: dropped
    layer.weight.weight_loader(layer.weight, w1, 1)
    with pytest.raises(RuntimeError, match="shape mismatch"):
        layer.weight.weight_loader(layer.weight, torch.zeros(32, 128, dtype=torch.bfloat16), 1)
    layer.mcg.data.fill_(V.MCG_MARKER_SIGNED_INT32)
    layer.mcg.data[1] = 0                      # a bf16 shard carries no marker
    meth.process_weights_after_loading(layer)
    lins = layer._exl3_linears
    assert lins[1] is None and lins[0] is not None and lins[2] is not None
    assert torch.equal(layer._exl3_bf16_weight, w1)
    tp2 = torch.nn.Module()
    tp2.prefix = "model.layers.0.attn.fused_qkv"
    with pytest.raises(RuntimeError, match="TP size"):
        V.Exl3LinearMethod(cfg, bits=2, tp_rank=0, tp_size=2).create_weights(tp2, 128, [128, 64, 128])
    bad = torch.nn.Module()
    bad.prefix = "model.layers.0.attn.fused_qkv"
    with pytest.raises(ValueError, match="outside"):
        V.Exl3LinearMethod(cfg, bits=2).create_weights(bad, 128, [128], 128, 128)


def test_wo_a_loader_keeps_this_ranks_slice():
    """wo_a: one pre-sliced group per TP8 rank; the loader keeps the slice
    whose rank matches and never narrows it again
    (recipe-lna/vllm_exl3_exl3.py.lna:2355-2362, 2533-2568)."""
    layer = torch.nn.Module()
    layer.prefix = "model.layers.5.attn.wo_a"
    with pytest.raises(NotImplementedError, match="TP=8"):
        V.Exl3LinearMethod(bits=2, tp_rank=0, tp_size=2).create_weights(layer, 256, [128])
    layer = torch.nn.Module()
    layer.prefix = "model.layers.5.attn.wo_a"
    meth = V.Exl3LinearMethod(bits=2, tp_rank=3, tp_size=8)
    meth.create_weights(layer, 256, [128], 2048, 1024)
    assert not hasattr(layer, "weight")
    for rank in range(8):
        t = torch.full((16, 8, 32), rank, dtype=torch.int16)
        layer.trellis.weight_loader(layer.trellis, t, f"wo_a.slice.{rank}")
        layer.svh.weight_loader(layer.svh, torch.full((128,), float(rank), dtype=torch.float16), rank)
        layer.suh.weight_loader(layer.suh, torch.full((256,), float(rank), dtype=torch.float16), str(rank))
        layer.mcg.weight_loader(layer.mcg, torch.tensor(V.MCG_MARKER_SIGNED_INT32, dtype=torch.int32),
                                f"wo_a.slice.{rank}")
    assert int(layer.trellis.float().mean()) == 3 and float(layer.svh[0]) == 3.0 and float(layer.suh[0, 0]) == 3.0
    with pytest.raises(ValueError, match="wo_a.slice.N"):
        layer.trellis.weight_loader(layer.trellis, torch.zeros((16, 8, 32), dtype=torch.int16), "q")
    with pytest.raises(RuntimeError, match="shape mismatch"):
        layer.trellis.weight_loader(layer.trellis, torch.zeros((8, 8, 32), dtype=torch.int16), "wo_a.slice.3")
    meth.process_weights_after_loading(layer)
    (lin,) = layer._exl3_linears
    assert lin.in_features == 256 and lin.out_features == 128 and int(lin.trellis.float().mean()) == 3


def test_scratch_pool_frees_replaced_buffers_unless_captured(monkeypatch):
    """A buffer that a larger one replaces is freed, except one that was
    current during a graph capture (a captured graph keeps its address)."""
    import torch
    from dsv4_carve_amd import ops

    pool = ops._ScratchPool()
    cpu = torch.device("cpu", 0)
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: False)
    a = pool.get(cpu, "moe", 1000)
    assert pool.get(cpu, "moe", 500) is a                  # large enough: reused
    b = pool.get(cpu, "moe", 4000)
    assert b is not a and pool.resident_bytes() == 4000     # `a` is no longer held by the pool
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: True)
    assert pool.get(cpu, "moe", 100) is b                  # a capture used `b`
    with pytest.raises(RuntimeError, match="not prewarmed"):
        pool.get(cpu, "moe", 8000)
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: False)
    c = pool.get(cpu, "moe", 8000)
    assert pool.resident_bytes() == 8000 + 4000             # `b` retired, kept alive
    assert pool.get(cpu, "moe", 16000) is not c and pool.resident_bytes() == 16000 + 4000


def test_vram_trace_is_opt_in_and_logs_the_reference_format(monkeypatch, caplog):
    """LNA_EXL3_VRAM_TRACE=1 (recipe-lna/vllm_exl3_exl3.py.lna:92-118): no mark
    unless it is set, none for a CPU device, and one line per phase with the
    before / after MiB and the signed delta."""
    import logging

    monkeypatch.delenv("LNA_EXL3_VRAM_TRACE", raising=False)
    assert V._vram_mark(torch.device("cpu")) is None
    monkeypatch.setenv("LNA_EXL3_VRAM_TRACE", "1")
    assert V._vram_mark(torch.device("cpu")) is None
    assert V._vram_mark(None) is None
    with caplog.at_level(logging.INFO, logger=V.logger.name):
        V._vram_report("registration.fan_scratch", "layers.3:hfan", 3 << 20, (3 << 20) + (1 << 19))
        V._vram_report("first_call", "g", None, 5)           # no mark, no line
        V._vram_report("moe.scratch", "x", 2 << 20, 1 << 20)
    lines = [r.getMessage() for r in caplog.records]
    assert lines == [
        "F2 VRAM phase=registration.fan_scratch layer=layers.3:hfan before_mib=3.000 after_mib=3.500 "
        "delta_mib=+0.500",
        "F2 VRAM phase=moe.scratch layer=x before_mib=2.000 after_mib=1.000 delta_mib=-1.000",
    ]
