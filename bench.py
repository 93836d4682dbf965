#!/usr/bin/env python3
"""Routed-MoE decode layer benchmark (one MI355X).

Workload: 256 experts, top-8 routing, hidden 4096, expert intermediate 2048
(gate+up 4096 -> 2x2048, clamped SiLU*mul, down 2048 -> 4096); experts 0-127 at
3 bits, 128-255 at 2 bits (EXL3 MCG trellis); seeded synthetic weights, N(0,1)
router logits, fp16 activations.  One step = one layer decode over a batch of
`--rows` rows (default 16).  Every step of a run uses a different routing from a
seeded pool, so consecutive steps read different experts (no reuse through the
256 MB MALL), and the steps are replayed from a HIP graph.

Prints ONE JSON line; `value` is microseconds per layer at --rows (lower is
better), `roofline` the achieved HBM bandwidth on the algorithmic bytes of the
experts actually read (over the whole layer: its gate/up, activation, down and
finishing launches), `cpu_baseline` the CPU restatement of the reference's
CPU path timed on a bounded sample on this host.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

HIDDEN, INTER, EXPERTS, TOPK = 4096, 2048, 256, 8
LATENCY_ITERS = 40
HBM_PEAK_GBS = 8000.0
POOL = 64


def expert_bytes(hidden: int, inter: int, bits: int) -> int:
    """Algorithmic bytes of one expert: packed trellis + suh + svh of gate, up, down."""
    per = 3 * hidden * inter * bits // 8
    return per + 2 * 2 * (hidden + inter) + 2 * (inter + hidden)


def step_bytes(ids: np.ndarray, bits: list[int], hidden: int, inter: int, x_bytes=2, out_bytes=4) -> int:
    m = ids.shape[0]
    active = sorted({int(e) for e in ids.reshape(-1) if 0 <= e < len(bits)})
    return sum(expert_bytes(hidden, inter, bits[e]) for e in active) + m * hidden * (x_bytes + out_bytes)


class DeviceLayer:
    def __init__(self, dev, n_experts, hidden, inter, bits, seed):
        import torch
        from dsv4_carve_amd import synth
        from dsv4_carve_amd.ops import MOE_TABLE_KEYS

        self.hidden, self.inter, self.bits = hidden, inter, list(bits)
        self.keep = []
        cols = {k: [] for k in MOE_TABLE_KEYS}
        for e in range(n_experts):
            ex = synth.expert(e, hidden, inter, self.bits[e], seed)
            for p in ("gate", "up", "down"):
                for part in ("trellis", "suh", "svh"):
                    t = torch.from_numpy(ex[p][part]).to(dev)
                    self.keep.append(t)
                    cols[f"{p}_{part}"].append(int(t.data_ptr()))
        self.tables = {k: torch.tensor(v, dtype=torch.int64, device=dev) for k, v in cols.items()}
        self.ebits = torch.tensor(self.bits, dtype=torch.int8, device=dev)
        self.mask = sum(1 << b for b in set(self.bits))


REPLAYS = 5             # timed graph replays per measurement (the median is reported)
STABLE_TOL = 0.01       # warm-up replays continue until two in a row agree this closely
MAX_WARM_REPLAYS = 10


def _replay_timed(graph) -> float:
    """ms of one replay, timed with events on the current stream (where the
    replay runs)."""
    import torch

    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    graph.replay()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b)


def replay_median(graph, steps: int) -> tuple[float, list[float]]:
    """us per step: untimed replays until two consecutive ones agree within
    STABLE_TOL (clocks settled, graph uploaded), then the median of REPLAYS
    timed replays; also returns every timed replay's us per step."""
    prev = None
    for _ in range(MAX_WARM_REPLAYS):
        t = _replay_timed(graph)
        if prev is not None and abs(t - prev) <= STABLE_TOL * prev:
            break
        prev = t
    per = sorted(_replay_timed(graph) * 1000.0 / steps for _ in range(REPLAYS))
    return per[len(per) // 2], per


def moe_c_call(lib, entry, x, out, layer, ids, w, scratch):
    """One routed-MoE call straight through the C ABI of `lib` (the product
    library or its timing-only twin), with the arguments ops.moe_decode /
    ops.moe_prefill would pass."""
    import torch
    from dsv4_carve_amd import _lib, ops

    t = layer.tables
    rc = getattr(lib, entry)(
        x.data_ptr(), 0, out.data_ptr(), 2, x.shape[0], layer.hidden, layer.inter, len(layer.bits), ids.shape[1],
        *[int(t[k].data_ptr()) for k in ops.MOE_TABLE_KEYS], ids.data_ptr(), 0, w.data_ptr(), 2, None, 0,
        layer.ebits.data_ptr(), 0, layer.mask, ops.CB_MCG, 10.0, scratch.data_ptr(), scratch.numel(),
        int(torch.cuda.current_stream().cuda_stream))
    if rc < 0:
        raise _lib.Exl3Error(lib.exl3_last_error().decode())


def time_layer(layer, dev, rows, topk, steps, warmup, seed, same_routing=False, eager=False, lib=None):
    """Returns (us per step, mean algorithmic bytes per step).  The K steps are
    replayed from one HIP graph, the median over REPLAYS timed replays after
    the clock has settled; `eager` launches them one by one instead (for
    counter collection, which sees every dispatch).  `lib`: call that
    library's C ABI instead of the ops (the null-decode twin)."""
    import torch
    from dsv4_carve_amd import ops, synth

    n_exp = len(layer.bits)
    pool = [synth.routing(rows, n_exp, topk, seed=seed * 1000 + (0 if same_routing else i)) for i in range(POOL)]
    ids = torch.tensor(np.stack([p[0] for p in pool]), dtype=torch.int32, device=dev)
    wts = torch.tensor(np.stack([p[1] for p in pool]), dtype=torch.float32, device=dev)
    x = torch.from_numpy(synth.activations(rows, layer.hidden, seed=seed)).to(dev)
    out = torch.empty((rows, layer.hidden), dtype=torch.float32, device=dev)
    scratch = ops.moe_scratch(dev, layer.hidden, layer.inter, topk, rows=rows)

    def launch(i):
        if lib is not None:
            moe_c_call(lib, "exl3_moe_decode_routed", x, out, layer, ids[i % POOL], wts[i % POOL], scratch)
            return
        ops.moe_decode(x, out, layer.tables, ids[i % POOL], wts[i % POOL], intermediate=layer.inter,
                       expert_bits=layer.ebits, bits_mask=layer.mask, scratch=scratch)

    for i in range(warmup):
        launch(i)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    nbytes = float(np.mean([step_bytes(pool[i % POOL][0], layer.bits, layer.hidden, layer.inter)
                            for i in range(steps)]))
    if eager:
        start.record()
        for i in range(steps):
            launch(i)
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) * 1000.0 / steps, nbytes
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for i in range(steps):
            launch(i)
    torch.cuda.synchronize()
    us, _ = replay_median(graph, steps)
    return us, nbytes


def layer_latency(layer, dev, rows, topk, iters, seed, cold: bool) -> dict:
    """Per-call latency distribution: `iters` layer calls launched one by one,
    each bracketed by events.  Cold: fresh routing per call and a 1 GiB read
    of another buffer before it (untimed), so neither the experts nor the
    256 MB MALL hold anything the call reads; warm: the same routing and no
    flush.  Returns p50/p95/mean in us."""
    import ctypes

    import torch
    from dsv4_carve_amd import build as B
    from dsv4_carve_amd import ops, synth

    n_exp = len(layer.bits)
    pool = [synth.routing(rows, n_exp, topk, seed=seed * 1000 + (i if cold else 0)) for i in range(POOL)]
    ids = torch.tensor(np.stack([p[0] for p in pool]), dtype=torch.int32, device=dev)
    wts = torch.tensor(np.stack([p[1] for p in pool]), dtype=torch.float32, device=dev)
    x = torch.from_numpy(synth.activations(rows, layer.hidden, seed=seed)).to(dev)
    out = torch.empty((rows, layer.hidden), dtype=torch.float32, device=dev)
    scratch = ops.moe_scratch(dev, layer.hidden, layer.inter, topk, rows=rows)
    probe = ctypes.CDLL(B.PROBE_LIB)
    probe.exl3_probe_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    flush = torch.ones((1 << 30) // 4, dtype=torch.int32, device=dev) if cold else None
    blocks = torch.cuda.get_device_properties(dev).multi_processor_count * 8
    sink = torch.empty(blocks * 256, dtype=torch.int32, device=dev)
    stream = int(torch.cuda.current_stream(dev).cuda_stream)
    times = []
    for i in range(iters + 3):
        if cold:
            probe.exl3_probe_read(flush.data_ptr(), flush.numel() * 4, sink.data_ptr(), blocks, stream)
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        ops.moe_decode(x, out, layer.tables, ids[i % POOL], wts[i % POOL], intermediate=layer.inter,
                       expert_bits=layer.ebits, bits_mask=layer.mask, scratch=scratch)
        b.record()
        torch.cuda.synchronize()
        if i >= 3:
            times.append(a.elapsed_time(b) * 1000.0)
    del flush
    t = np.array(times)
    return {"p50_us": round(float(np.percentile(t, 50)), 2), "p95_us": round(float(np.percentile(t, 95)), 2),
            "mean_us": round(float(t.mean()), 2), "iters": iters}


def time_glue(layer, dev, rows, topk, steps=40, seed=77):
    """us per layer from the router's tensors (int64 global ids, bf16 weights)
    under graph replay, three ways: the kernel alone on ready int32 local ids
    and fp32 weights; the plugin's host-side glue (map_topk_to_local and the
    casts, each its own launch) before it; and the glue folded into the
    kernels (the routed entry point).  With and without an expert map (here
    the identity map over every expert, so the routed work is the same)."""
    import torch
    from dsv4_carve_amd import ops, synth
    from dsv4_carve_amd import vllm_exl3 as V

    n_exp = len(layer.bits)
    pool = [synth.routing(rows, n_exp, topk, seed=seed * 1000 + i) for i in range(POOL)]
    ids64 = torch.tensor(np.stack([p[0] for p in pool]), dtype=torch.int64, device=dev)
    w16 = torch.tensor(np.stack([p[1] for p in pool]), dtype=torch.float32, device=dev).to(torch.bfloat16)
    ids32 = ids64.to(torch.int32)
    w32 = w16.float()
    emap = torch.arange(n_exp, dtype=torch.int64, device=dev)
    x = torch.from_numpy(synth.activations(rows, layer.hidden, seed=seed)).to(dev)
    out = torch.empty((rows, layer.hidden), dtype=torch.float32, device=dev)
    kw = dict(intermediate=layer.inter, expert_bits=layer.ebits, bits_mask=layer.mask,
              scratch=ops.moe_scratch(dev, layer.hidden, layer.inter, topk))

    def kernel(i, m):
        ops.moe_decode(x, out, layer.tables, ids32[i % POOL], w32[i % POOL], **kw)

    def host(i, m):
        local = V.map_topk_to_local(ids64[i % POOL], n_exp, m).reshape(rows, topk)
        ops.moe_decode(x, out, layer.tables, local.to(torch.int32).contiguous(),
                       w16[i % POOL].reshape(local.shape).to(torch.float32).contiguous(), **kw)

    def device(i, m):
        ops.moe_decode(x, out, layer.tables, ids64[i % POOL], w16[i % POOL], expert_map=m, **kw)

    def timed(fn, m):
        for i in range(3):
            fn(i, m)
        torch.cuda.synchronize()
        stream = torch.cuda.Stream()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for i in range(steps):
                fn(i, m)
        return round(replay_median(graph, steps)[0], 2)

    res = {"kernel_only_us": timed(kernel, None)}
    for name, m in (("no_map", None), ("expert_map", emap)):
        res[name] = {"host_glue_us": timed(host, m), "device_glue_us": timed(device, m)}
    return res


DENSE_SHAPES = ((4096, 4096), (4096, 1536), (1536, 4096), (4096, 12288))
DENSE_BITS = (2, 3, 4, 6)
DENSE_ROWS = (1, 2, 4, 8, 16, 32, 64, 144)     # above 16: 32-row blocks, the LinearEXL3 GEMV range
FAN_ROWS = (1, 2, 4, 8, 16)                     # the row range the plugin fuses


def dense_bytes(k: int, n: int, bits: int, rows: int) -> int:
    """Algorithmic bytes of one dense call: trellis + suh + svh, x in, fp16 y out."""
    return k * n * bits // 8 + 2 * (k + n) + rows * k * 2 + rows * n * 2


# Same-input fans of one dense layer (6-bit): the h-fan (wq_a, wkv, compressor
# wkv/wgate, indexer compressor x2 read the 4096-wide hidden state) and the
# q_a-fan (wq_b and indexer.wq_b read the 1024-wide q latent).
FANS = {"h_fan_4096_to_1024_512_1024_1024_256_256": (4096, [1024, 512, 1024, 1024, 256, 256], 6),
        "q_a_fan_1024_to_32768_8192": (1024, [32768, 8192], 6)}


def time_fan(dev, k, ns, bits, rows_list, steps=40):
    """us per fan call, cold (distinct weight copies cycled so none is still in
    the MALL): one fused exl3_gemm_group call, and the members' solo exl3_gemm
    calls one after another."""
    import torch
    from dsv4_carve_amd import ops

    g = torch.Generator(device=dev)
    g.manual_seed(k * 131 + sum(ns) + bits)
    wbytes = sum(k * n * bits // 8 for n in ns)
    copies = max(2, -(-(600 << 20) // wbytes))

    def member(n):
        t = torch.randint(-32768, 32767, (k // 16, n // 16, 16 * bits), dtype=torch.int16, device=dev, generator=g)
        suh = (torch.randint(0, 2, (k,), device=dev, generator=g) * 2 - 1).to(torch.float16)
        svh = ((torch.randint(0, 2, (n,), device=dev, generator=g) * 2 - 1) *
               (torch.rand(n, device=dev, generator=g) * 1.5 + 0.5) / k ** 0.5).to(torch.float16)
        return t, suh, svh

    pool = [[member(n) for n in ns] for _ in range(copies)]
    res = {}
    for rows in rows_list:
        x = torch.randn((rows, k), device=dev, generator=g).to(torch.float16)
        outs = [torch.empty((rows, n), dtype=torch.float32, device=dev) for n in ns]
        for n in ns:
            ops.prepare_gemm(dev, rows, k, n)
        out = {}
        calls = {"fused": lambda mem: ops.gemm_group(x, mem, outs=outs),
                 "solo": lambda mem: [ops.gemm_into(x, t, su, sv, o) for (t, su, sv), o in zip(mem, outs)]}
        for mode, call in calls.items():
            order = [i % copies for i in range(steps)]
            for i in order[:3]:
                call(pool[i])
            torch.cuda.synchronize()
            stream = torch.cuda.Stream()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                for i in order:
                    call(pool[i])
            out[mode] = replay_median(graph, steps)[0]
        nb = sum(dense_bytes(k, n, bits, rows) for n in ns)
        res[str(rows)] = {"fused_us": round(out["fused"], 2), "solo_us": round(out["solo"], 2),
                          "fused_GBps": round(nb / (out["fused"] * 1e-6) / 1e9, 1)}
    del pool
    torch.cuda.empty_cache()
    return res


def time_dense(dev, k, n, bits, rows_list, steps=40, lib=None):
    """us per call of the trellis-decode GEMV for each row count, cold (cycling
    through > 512 MB of distinct weight copies, so no copy is still in the
    256 MB MALL when reused) and warm (one copy).  Weights are seeded on the
    device: this measures speed only (parity is the tests' job).  `lib`: call
    that library's exl3_gemm instead of the op (the null-decode twin)."""
    import torch
    from dsv4_carve_amd import _lib, ops

    def gemm_into(x, t, su, sv, y):
        if lib is None:
            return ops.gemm_into(x, t, su, sv, y)
        scratch = ops.gemm_scratch(dev, x.shape[0], k, n)
        if lib.exl3_gemm(x.data_ptr(), x.shape[0], k, t.data_ptr(), n, bits, ops.CB_MCG, su.data_ptr(),
                         sv.data_ptr(), y.data_ptr(), 0, scratch.data_ptr(), scratch.numel(),
                         int(torch.cuda.current_stream().cuda_stream)) < 0:
            raise _lib.Exl3Error(lib.exl3_last_error().decode())

    g = torch.Generator(device=dev)
    g.manual_seed(k * 131 + n * 7 + bits)
    wbytes = k * n * bits // 8
    copies = max(2, -(-(600 << 20) // wbytes))
    pool = [torch.randint(-32768, 32767, (k // 16, n // 16, 16 * bits), dtype=torch.int16, device=dev,
                          generator=g) for _ in range(copies)]
    suh = (torch.randint(0, 2, (k,), device=dev, generator=g) * 2 - 1).to(torch.float16)
    svh = ((torch.randint(0, 2, (n,), device=dev, generator=g) * 2 - 1) *
           (torch.rand(n, device=dev, generator=g) * 1.5 + 0.5) / k ** 0.5).to(torch.float16)
    res = {}
    for rows in rows_list:
        x = torch.randn((rows, k), device=dev, generator=g).to(torch.float16)
        y = torch.empty((rows, n), dtype=torch.float16, device=dev)
        ops.prepare_gemm(dev, rows, k, n)
        out = {}
        for mode, order in (("cold", [i % copies for i in range(steps)]), ("warm", [0] * steps)):
            for i in order[:3]:
                gemm_into(x, pool[i], suh, svh, y)
            torch.cuda.synchronize()
            stream = torch.cuda.Stream()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                for i in order:
                    gemm_into(x, pool[i], suh, svh, y)
            out[mode] = replay_median(graph, steps)[0]
        nb = dense_bytes(k, n, bits, rows)
        res[str(rows)] = {"us": round(out["cold"], 2), "GBps": round(nb / (out["cold"] * 1e-6) / 1e9, 1),
                          "warm_us": round(out["warm"], 2)}
    del pool
    torch.cuda.empty_cache()
    return res


LINEAR_SHAPES = ((4096, 4096), (4096, 12288))
LINEAR_ROWS = (32, 64, 144, 512, 2048)


def time_linear(dev, k, n, bits, rows_list, steps=20):
    """us per LinearEXL3.forward call (the plugin's dense entry: the decode
    GEMV up to its row threshold, the reconstruct path beyond), cold over
    > 512 MB of distinct weight copies, fp16 output."""
    import torch
    from dsv4_carve_amd import ops
    from dsv4_carve_amd import vllm_exl3 as V

    g = torch.Generator(device=dev)
    g.manual_seed(k * 17 + n + bits)
    copies = max(2, -(-(600 << 20) // (k * n * bits // 8)))
    mcg = torch.tensor([V.MCG_MARKER_SIGNED_INT32], dtype=torch.int32, device=dev)
    mods = []
    for _ in range(copies):
        tr = torch.randint(-32768, 32767, (k // 16, n // 16, 16 * bits), dtype=torch.int16, device=dev, generator=g)
        suh = (torch.randint(0, 2, (k,), device=dev, generator=g) * 2 - 1).to(torch.float16)
        svh = ((torch.randint(0, 2, (n,), device=dev, generator=g) * 2 - 1) / k ** 0.5).to(torch.float16)
        mods.append(V.make_linear_exl3(tr, suh, svh, mcg))
    res = {}
    for rows in rows_list:
        x = torch.randn((rows, k), device=dev, generator=g).to(torch.float16)
        ops.prepare_gemm(dev, rows, k, n)
        order = [i % copies for i in range(steps)]
        for i in order[:3]:
            mods[i].forward(x, {}, out_dtype=torch.float16)
        torch.cuda.synchronize()
        stream = torch.cuda.Stream()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for i in order:
                mods[i].forward(x, {}, out_dtype=torch.float16)
        us = replay_median(graph, steps)[0]
        path = ("gemv" if rows <= V.AUTO_RECONSTRUCT_THRESHOLD else
                "reconstruct_folded" if rows >= V.FUSED_RECONSTRUCT_MIN_ROWS else "reconstruct")
        res[str(rows)] = {"us": round(us, 2), "path": path,
                          "tflops": round(2.0 * rows * k * n / (us * 1e-6) / 1e12, 1)}
        del graph
    del mods
    torch.cuda.empty_cache()
    return res


MFMA_PEAK_F16 = 2.5e15


def time_prefill(layer, dev, tokens, topk, steps, warmup, seed, zipf=True, lib=None, hot8=False):
    """Prefill-shaped layer (grouped GEMMs): us per layer over `tokens` tokens
    with Zipf(1.1) top-k routing (`zipf`; otherwise the decode benchmark's
    N(0,1)-logit routing), fresh routing each step from a pool of 4.  `hot8`:
    every token on the same 8 experts (8i .. 8i + 7 for pool entry i, all
    3-bit here), so every expert runs wide tiles only.
    Returns (us, algorithmic flops, algorithmic bytes, mean distinct experts).
    `lib`: call that library's C ABI instead of the ops (the null-decode twin)."""
    import torch
    from dsv4_carve_amd import ops, synth

    n_exp = len(layer.bits)
    route = synth.zipf_routing if zipf else synth.routing
    pool = [route(tokens, n_exp, topk, seed=seed + i) for i in range(4)]
    if hot8:
        pool = [(np.tile(np.arange(topk, dtype=p[0].dtype) + 8 * i, (tokens, 1)), p[1]) for i, p in enumerate(pool)]
    ids = [torch.from_numpy(p[0]).to(dev) for p in pool]
    wts = [torch.from_numpy(p[1]).to(dev) for p in pool]
    x = torch.from_numpy(synth.activations(tokens, layer.hidden, seed=seed)).to(dev)
    out = torch.empty((tokens, layer.hidden), dtype=torch.float32, device=dev)
    scratch = ops.moe_prefill_scratch(dev, tokens, layer.hidden, layer.inter, topk, n_exp)

    def launch(i):
        if lib is not None:
            moe_c_call(lib, "exl3_moe_prefill_routed", x, out, layer, ids[i % 4], wts[i % 4], scratch)
            return
        ops.moe_prefill(x, out, layer.tables, ids[i % 4], wts[i % 4], intermediate=layer.inter,
                        expert_bits=layer.ebits, bits_mask=layer.mask, scratch=scratch)

    for i in range(warmup):
        launch(i)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for i in range(steps):
            launch(i)
    us = replay_median(graph, steps)[0]
    flops = float(np.mean([2.0 * 3 * layer.hidden * layer.inter * int(((p[0] >= 0) & (p[0] < n_exp)).sum())
                           for p in pool]))
    nbytes = float(np.mean([step_bytes(p[0], layer.bits, layer.hidden, layer.inter) for p in pool]))
    distinct = float(np.mean([len(set(p[0].reshape(-1).tolist())) for p in pool]))
    return us, flops, nbytes, distinct


def prefill_tiles(c: int) -> int:
    """Tiles the prefill GEMMs run for an expert with c routed rows
    (csrc/exl3_prefill_capi.hip pf_plan_kernel): one narrow tile of up to 32
    rows, or above 32 rows wide tiles of up to 64 rows with a last part of at
    most 32 rows in a narrow tile.  Each tile decodes the expert once."""
    if c <= 32:
        return 1 if c > 0 else 0
    full, rem = divmod(c, 64)
    return full + (1 if rem > 0 else 0)


def prefill_decoded_weights(layer, tokens: int, topk: int, seed: int) -> tuple[float, float]:
    """Weights the prefill GEMMs decode per layer on time_prefill's routing
    pool (each expert's gate, up and down once per tile, prefill_tiles), and
    the minimum (each active expert once), means over the pool."""
    from dsv4_carve_amd import synth

    n_exp = len(layer.bits)
    per = 3.0 * layer.hidden * layer.inter
    dec, low = [], []
    for i in range(4):
        ids = synth.zipf_routing(tokens, n_exp, topk, seed=seed + i)[0].reshape(-1)
        cnt = np.bincount(ids[(ids >= 0) & (ids < n_exp)], minlength=n_exp)
        dec.append(float(sum(prefill_tiles(int(c)) for c in cnt)) * per)
        low.append(float((cnt > 0).sum()) * per)
    return float(np.mean(dec)), float(np.mean(low))


C3_LAYERS = 43


class StackLayer:
    """One decode MoE block of the 43-layer stack: the 256 routed experts (3-bit
    then 2-bit halves) plus a 6-bit shared expert (4096 -> 2x2048 -> 4096) as
    expert 256, whose slot every row gets with weight 1.  Weights are seeded on
    the device (speed only; parity is the tests' job)."""

    def __init__(self, dev, seed):
        import torch
        from dsv4_carve_amd.ops import MOE_TABLE_KEYS

        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        H, I = HIDDEN, INTER
        self.bits = synth_bits = [3] * (EXPERTS // 2) + [2] * (EXPERTS // 2) + [6]
        words = {b: H * I * b // 16 for b in set(synth_bits)}
        self.keep = []
        tr = {}
        for b in sorted(set(synth_bits)):
            n_e = synth_bits.count(b)
            t = torch.randint(-32768, 32767, (n_e, 3, words[b]), dtype=torch.int16, device=dev, generator=g)
            self.keep.append(t)
            tr[b] = t
        n = len(synth_bits)
        vh = ((torch.randint(0, 2, (n, 3, H), device=dev, generator=g) * 2 - 1).to(torch.float16) / 64)
        vi = ((torch.randint(0, 2, (n, 3, I), device=dev, generator=g) * 2 - 1).to(torch.float16) / 45)
        self.keep += [vh, vi]
        idx = {b: 0 for b in tr}
        cols = {k: [] for k in MOE_TABLE_KEYS}
        for e, b in enumerate(synth_bits):
            j = idx[b]
            idx[b] += 1
            base = tr[b][j]
            for p, proj in enumerate(("gate", "up", "down")):
                cols[f"{proj}_trellis"].append(int(base[p].data_ptr()))
            cols["gate_suh"].append(int(vh[e, 0].data_ptr()))
            cols["up_suh"].append(int(vh[e, 1].data_ptr()))
            cols["down_svh"].append(int(vh[e, 2].data_ptr()))
            cols["gate_svh"].append(int(vi[e, 0].data_ptr()))
            cols["up_svh"].append(int(vi[e, 1].data_ptr()))
            cols["down_suh"].append(int(vi[e, 2].data_ptr()))
        self.tables = {k: torch.tensor(v, dtype=torch.int64, device=dev) for k, v in cols.items()}
        self.ebits = torch.tensor(synth_bits, dtype=torch.int8, device=dev)
        self.mask = sum(1 << b for b in set(synth_bits))


def time_stack(dev, rows, steps, warmup):
    """us per decode step of C3_LAYERS routed+shared MoE blocks (one launch per
    block, each block's output is the next block's input), with independent
    routing per layer and step; returns (us per step, algorithmic bytes per step)."""
    import torch
    from dsv4_carve_amd import ops, synth

    layers = []
    for l in range(C3_LAYERS):
        layers.append(StackLayer(dev, 9000 + l))
        if l % 10 == 9:
            torch.cuda.synchronize()
            print(f"[bench] stack: {l + 1} layers built", file=sys.stderr, flush=True)
    torch.cuda.synchronize()
    shared = EXPERTS
    pools, nbytes = [], 0.0
    for l in range(C3_LAYERS):
        pl = []
        for i in range(4):
            ids, w = synth.routing(rows, EXPERTS, TOPK, seed=70000 + 97 * l + i)
            ids = np.concatenate([ids, np.full((rows, 1), shared, np.int32)], axis=1)
            w = np.concatenate([w, np.ones((rows, 1), np.float32)], axis=1)
            pl.append((torch.from_numpy(ids).to(dev), torch.from_numpy(w).to(dev)))
            nbytes += step_bytes(ids, layers[l].bits, HIDDEN, INTER) / 4
        pools.append(pl)
    acts = [torch.from_numpy(synth.activations(rows, HIDDEN, seed=5)).to(dev)]
    acts += [torch.empty((rows, HIDDEN), dtype=torch.float16, device=dev) for _ in range(C3_LAYERS)]
    scratch = ops.moe_scratch(dev, HIDDEN, INTER, TOPK + 1)

    def step(i):
        for l in range(C3_LAYERS):
            ids, w = pools[l][i % 4]
            ops.moe_decode(acts[l], acts[l + 1], layers[l].tables, ids, w, intermediate=INTER,
                           expert_bits=layers[l].ebits, bits_mask=layers[l].mask, scratch=scratch)

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for i in range(steps):
            step(i)
    us = replay_median(graph, steps)[0]
    del layers, graph
    torch.cuda.empty_cache()
    return us, nbytes


def time_read_ceiling(dev, gib: int = 2, reps: int = 10) -> dict:
    """Achievable cold HBM read rate: the probe kernel (csrc/exl3_probe.hip)
    streams a `gib` GiB buffer once per run, after a 1 GiB read of another
    buffer has flushed the 256 MB MALL; p50/max over `reps` runs for a few
    grid sizes.  This is the ceiling the decode kernels' weight streams are
    compared with, beside the nominal 8 TB/s."""
    import ctypes

    import torch
    from dsv4_carve_amd import build as B

    lib = ctypes.CDLL(B.PROBE_LIB)
    lib.exl3_probe_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    lib.exl3_probe_read.restype = ctypes.c_int
    threads = int(lib.exl3_probe_threads())
    nbytes = gib << 30
    buf = torch.ones(nbytes // 4, dtype=torch.int32, device=dev)
    flush = torch.ones((1 << 30) // 4, dtype=torch.int32, device=dev)
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    stream = int(torch.cuda.current_stream(dev).cuda_stream)
    res = {}
    for per_cu in (4, 8, 16):
        blocks = cus * per_cu
        sink = torch.empty(blocks * threads, dtype=torch.int32, device=dev)
        times = []
        for _ in range(reps + 1):
            assert lib.exl3_probe_read(flush.data_ptr(), flush.numel() * 4, sink.data_ptr(), blocks, stream) == 0
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            assert lib.exl3_probe_read(buf.data_ptr(), nbytes, sink.data_ptr(), blocks, stream) == 0
            b.record()
            torch.cuda.synchronize()
            times.append(a.elapsed_time(b) * 1e-3)
        rates = sorted(nbytes / t / 1e9 for t in times[1:])
        res[f"{per_cu}_blocks_per_cu"] = {"p50_GBps": round(rates[len(rates) // 2], 1), "max_GBps": round(rates[-1], 1)}
    best = max(v["p50_GBps"] for v in res.values())
    del buf, flush
    torch.cuda.empty_cache()
    return {"buffer_GiB": gib, "runs": reps, "best_p50_GBps": best, "frac_of_8TBps": round(best / HBM_PEAK_GBS, 4),
            **res}


def time_handoff(dev, blocks: int = 2048, pairs: int = 100, reps: int = 3) -> dict:
    """Cross-launch hand-off through the XCDs' L2s (csrc/exl3_probe.hip
    probe_handoff_*): a launch writes 4 KB per workgroup (8 MB over 2048
    workgroups), the next reads it back; us per (write, read) pair, in a
    captured graph of `pairs` pairs, when each reading workgroup reads a
    region written on its own XCD (shift a multiple of 8) or on another one.
    This is what the dense GEMV's XCD-keyed item order relies on."""
    import ctypes

    import torch
    from dsv4_carve_amd import build as B

    lib = ctypes.CDLL(B.PROBE_LIB)
    lib.exl3_probe_handoff.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                       ctypes.c_void_p]
    lib.exl3_probe_handoff.restype = ctypes.c_int
    buf = torch.empty(blocks * 256 * 4, dtype=torch.int32, device=dev)
    sink = torch.empty(blocks * 256, dtype=torch.int32, device=dev)
    res = {}
    for shift in (0, 8, 1, 3):
        s = torch.cuda.Stream(dev)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(s):
            assert lib.exl3_probe_handoff(buf.data_ptr(), sink.data_ptr(), blocks, shift, 1, s.cuda_stream) == 0
            torch.cuda.synchronize()
            with torch.cuda.graph(g, stream=s):
                assert lib.exl3_probe_handoff(buf.data_ptr(), sink.data_ptr(), blocks, shift, pairs,
                                              s.cuda_stream) == 0
        times = []
        for _ in range(reps + 1):
            times.append(_replay_timed(g) * 1e3 / pairs)
        res[f"shift_{shift}"] = round(sorted(times[1:])[len(times[1:]) // 2], 3)
        del g
    return {"unit": "us per (write, read) pair", "bytes": blocks * 256 * 16, "own_xcd": [res["shift_0"], res["shift_8"]],
            "other_xcd": [res["shift_1"], res["shift_3"]], **res}


def time_decode_ceiling(dev, iters: int = 512, reps: int = 5) -> dict:
    """Decode-rate ceiling: the decode kernels' inner loop (decode + MFMA on
    tiles held in registers, csrc/exl3_probe.hip) at their residency of two
    single-wave workgroups per SIMD, per bit width.  Returns the decoded
    weights per second (median of `reps` timed launches after one warm-up),
    the shader clock the loop ran at, and the SIMD cycles it spends per 64
    weights (one weight per lane).  `split` takes the loop apart at the same
    residency, shorter runs: the decode alone, the MFMAs alone, and the whole
    loop at four waves per SIMD, with its accumulators in AGPRs, and with each
    weight's addends summed on the VALU so half the MFMAs run."""
    import ctypes

    import torch
    from dsv4_carve_amd import build as B

    lib = ctypes.CDLL(B.PROBE_LIB)
    lib.exl3_probe_decode_mode.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                           ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    lib.exl3_probe_decode_mode.restype = ctypes.c_int
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    simds = 4 * cus
    g = torch.Generator().manual_seed(11)
    words = torch.randint(0, 2 ** 31 - 1, (64 * 8 * 6,), generator=g, dtype=torch.int64).to(torch.int32).to(dev)
    sink = torch.empty(4 * simds * 64, dtype=torch.float32, device=dev)
    clk = torch.zeros(2 * 4 * simds, dtype=torch.int64, device=dev)
    stream = int(torch.cuda.current_stream(dev).cuda_stream)

    def run(bits, mode, waves, n_iter, n_reps):
        blocks = waves * simds
        times = []
        for _ in range(n_reps + 1):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            assert lib.exl3_probe_decode_mode(bits, mode, blocks, n_iter, words.data_ptr(), sink.data_ptr(),
                                              clk.data_ptr(), stream) == 0
            b.record()
            torch.cuda.synchronize()
            times.append(a.elapsed_time(b) * 1e-3)
        t = sorted(times[1:])[n_reps // 2]
        c = clk[:2 * blocks].view(blocks, 2).double().sum(0).tolist()
        ghz = c[0] / c[1] * 0.1                      # reference ticks at 100 MHz
        weights = blocks * n_iter * 16384.0
        return {"Gweights_per_s": round(weights / t / 1e9, 1), "clock_GHz": round(ghz, 3),
                "simd_cycles_per_64_weights": round(t * ghz * 1e9 * simds / (weights / 64.0), 2)}

    res = {f"K{bits}": run(bits, 0, 2, iters, reps) for bits in (2, 3, 4, 6)}
    split = {}
    for bits in (2, 3, 4, 6):
        split[f"K{bits}"] = {
            "decode_only": run(bits, 1, 2, iters // 4, 3)["simd_cycles_per_64_weights"],
            "mfma_only": run(bits, 2, 2, iters // 4, 3)["simd_cycles_per_64_weights"],
            "full_4_waves_per_simd": run(bits, 0, 4, iters // 4, 3)["simd_cycles_per_64_weights"],
            "full_agpr_acc": run(bits, 3, 2, iters // 4, 3)["simd_cycles_per_64_weights"],
            "full_agpr_acc_4_waves_per_simd": run(bits, 3, 4, iters // 4, 3)["simd_cycles_per_64_weights"],
            "addends_summed_half_mfmas": run(bits, 4, 2, iters // 4, 3)["simd_cycles_per_64_weights"]}
    # Wave roles (exl3_probe_roles): one workgroup per CU with two or three
    # waves per SIMD, each running the whole loop, or some decoding only and
    # others running only the MFMAs of the same work.  Cycles are per 64
    # weights of complete work (decoded and multiplied); `mixed` is the share of
    # SIMDs whose waves had both roles (read back from HW_ID).
    lib.exl3_probe_roles.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                     ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    lib.exl3_probe_roles.restype = ctypes.c_int
    rsink = torch.empty(cus * 768, dtype=torch.float32, device=dev)
    rclk = torch.zeros(3 * 12 * cus, dtype=torch.int64, device=dev)
    role_of = {1: [0, 0, 0, 0, 1, 1, 1, 1], 2: [0, 1, 0, 1, 0, 1, 0, 1], 3: [0] * 8 + [1] * 4}

    def run_roles(bits, mode, n_iter, n_reps):
        times = []
        for _ in range(n_reps + 1):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            assert lib.exl3_probe_roles(bits, mode, cus, n_iter, words.data_ptr(), rsink.data_ptr(), rclk.data_ptr(),
                                        stream) == 0
            b.record()
            torch.cuda.synchronize()
            times.append(a.elapsed_time(b) * 1e-3)
        t = sorted(times[1:])[n_reps // 2]
        nw = 12 if mode >= 3 else 8
        c = rclk.view(cus, 12, 3)[:, :nw].double().cpu()
        ghz = float(c[:, :, 0].sum() / c[:, :, 1].sum()) * 0.1
        units = cus * {0: 8, 1: 4, 2: 4, 3: 8, 4: 12}[mode] * n_iter * 16384.0
        out = {"simd_cycles_per_64_weights": round(t * ghz * 1e9 * simds / (units / 64.0), 2)}
        if mode in role_of:
            simd_of = c[:, :, 2].long().tolist()
            mixed = total = 0
            for wg in simd_of:
                for sm in range(4):
                    r = {role_of[mode][w] for w in range(nw) if wg[w] == sm}
                    total += 1
                    mixed += len(r) == 2
            out["mixed"] = round(mixed / total, 3)
        return out

    roles = {}
    for bits in (2, 3):
        roles[f"K{bits}"] = {
            "both_waves_whole_loop": run_roles(bits, 0, iters // 4, 3)["simd_cycles_per_64_weights"],
            "waves_0_3_decode_4_7_mfma": run_roles(bits, 1, iters // 4, 3),
            "even_waves_decode_odd_mfma": run_roles(bits, 2, iters // 4, 3),
            "three_waves_whole_loop": run_roles(bits, 4, iters // 4, 3)["simd_cycles_per_64_weights"],
            "two_decode_waves_one_mfma_wave": run_roles(bits, 3, iters // 4, 3)}
    del words, sink, clk, rsink, rclk
    return {"workgroups": 2 * simds, "iters": iters, "codebook": "MCG", **res,
            "split_simd_cycles_per_64_weights": split, "wave_roles_simd_cycles_per_64_weights": roles}


ROWS_CFG = ((1, 1), (2, 1), (2, 2), (3, 2), (4, 2), (4, 4), (6, 4), (8, 4))


def time_row_blocks(dev, iters: int = 256, reps: int = 3) -> dict:
    """The grouped GEMM's inner loop with each decoded B operand applied to
    RB 16-row blocks, each lane decoding 16/D of its tile's columns
    (csrc/exl3_probe.hip probe_rows_kernel; single-wave workgroups, two per
    SIMD).  Returns SIMD cycles per decoded weight (per 64 weights, one per
    lane) and per weight-row (divided by 16 RB) for each (RB, D) at 2 and 3
    bits."""
    import ctypes

    import torch
    from dsv4_carve_amd import build as B

    lib = ctypes.CDLL(B.PROBE_LIB)
    lib.exl3_probe_rows.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                    ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    lib.exl3_probe_rows.restype = ctypes.c_int
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    simds = 4 * cus
    blocks = 2 * simds
    g = torch.Generator().manual_seed(11)
    words = torch.randint(0, 2 ** 31 - 1, (64 * 8 * 3,), generator=g, dtype=torch.int64).to(torch.int32).to(dev)
    sink = torch.empty(blocks * 64, dtype=torch.float32, device=dev)
    clk = torch.zeros(2 * blocks, dtype=torch.int64, device=dev)
    stream = int(torch.cuda.current_stream(dev).cuda_stream)
    out = {}
    for bits in (2, 3):
        for cfg, (rb, d) in enumerate(ROWS_CFG):
            times = []
            for _ in range(reps + 1):
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record()
                assert lib.exl3_probe_rows(bits, cfg, blocks, iters, words.data_ptr(), sink.data_ptr(),
                                           clk.data_ptr(), stream) == 0
                b.record()
                torch.cuda.synchronize()
                times.append(a.elapsed_time(b) * 1e-3)
            t = sorted(times[1:])[reps // 2]
            c = clk[:2 * blocks].view(blocks, 2).double().sum(0).tolist()
            ghz = c[0] / c[1] * 0.1
            weights = blocks * iters * 16384.0 / d
            cyc = t * ghz * 1e9 * simds / (weights / 64.0)
            out[f"K{bits}_rb{rb}_d{d}"] = {"per_64_weights": round(cyc, 2), "per_64_weight_rows": round(cyc / (16 * rb), 3)}
    del words, sink, clk
    return {"unit": "SIMD cycles", "iters": iters, **out}


GEMM_STEPS = ("narrow_1_row_block", "narrow_2_row_blocks", "wide_4_row_blocks", "wide_4_row_blocks_addends_summed")


def time_gemm_steps(dev, iters: int = 256, reps: int = 3) -> dict:
    """The prefill GEMM's own step functions (csrc/exl3_probe.hip
    probe_gemm_step_kernel: mma_tile2 with one or two row blocks, mma_tile_wide
    with four, and a wide step with each weight's addends summed on the VALU
    so half the MFMAs run) on register-resident tile and A words, single-wave
    workgroups, two per SIMD.  Returns SIMD cycles per 64 decoded weights (one per lane)
    and per 64 weight-rows, at 2 and 3 bits."""
    import ctypes

    import torch
    from dsv4_carve_amd import build as B

    lib = ctypes.CDLL(B.PROBE_LIB)
    lib.exl3_probe_gemm_step.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                         ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    lib.exl3_probe_gemm_step.restype = ctypes.c_int
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    simds = 4 * cus
    blocks = 2 * simds
    g = torch.Generator().manual_seed(11)
    words = torch.randint(0, 2 ** 31 - 1, (64 * 8 * 3,), generator=g, dtype=torch.int64).to(torch.int32).to(dev)
    sink = torch.empty(blocks * 64, dtype=torch.float32, device=dev)
    clk = torch.zeros(2 * blocks, dtype=torch.int64, device=dev)
    stream = int(torch.cuda.current_stream(dev).cuda_stream)
    out = {}
    for bits in (2, 3):
        for kind, (name, rows) in enumerate(zip(GEMM_STEPS, (16, 32, 64, 64))):
            times = []
            for _ in range(reps + 1):
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record()
                assert lib.exl3_probe_gemm_step(bits, kind, blocks, iters, words.data_ptr(), sink.data_ptr(),
                                                clk.data_ptr(), stream) == 0
                b.record()
                torch.cuda.synchronize()
                times.append(a.elapsed_time(b) * 1e-3)
            t = sorted(times[1:])[reps // 2]
            c = clk[:2 * blocks].view(blocks, 2).double().sum(0).tolist()
            ghz = c[0] / c[1] * 0.1
            weights = blocks * iters * (8192.0 if rows == 64 else 16384.0)
            cyc = t * ghz * 1e9 * simds / (weights / 64.0)
            out[f"K{bits}_{name}"] = {"per_64_weights": round(cyc, 2), "per_64_weight_rows": round(cyc / rows, 3)}
    del words, sink, clk
    return {"unit": "SIMD cycles", "iters": iters, **out}


ISA_OPS = ("v_and_b32", "v_xor_b32", "v_lshrrev_b32", "v_bitop3_b32", "v_mul_lo_u16", "v_add_u32",
           "v_bfe_u32", "v_alignbit_b32", "v_perm_b32", "v_mul_lo_u32", "v_lshlrev_b32", "v_add3_u32",
           "v_mad_u32_u16", "v_mad_u32_u16 op_sel hi", "v_pk_mad_u16", "v_pk_mul_lo_u16",
           "v_mad_u16 op_sel hi", "v_mul_u32_u24", "v_mul_hi_u32_u24", "v_mad_u32_u24", "v_mul_hi_u32",
           "v_lshl_or_b32", "v_and_or_b32", "v_bfi_b32", "v_alignbyte_b32", "v_xad_u32", "v_or3_b32",
           "v_lshl_add_u32", "v_lshrrev_b32 vgpr shift", "v_lshlrev_b32 vgpr shift", "v_dot2_u32_u16",
           "v_pk_lshrrev_b16", "v_mul_lo_u16_sdwa dst hi", "v_mul_u32_u24_sdwa src hi",
           "v_lshrrev_b32_sdwa shift hi", "v_and_b32_sdwa src lo", "v_pk_add_f16", "v_add_f16", "v_fma_f32",
           "v_cvt_f32_u32",
           "seq mul_lo_u32+and", "seq mul_lo_u32+and+xor", "seq mul_lo_u32+bitop3", "seq bfe+mul_lo_u32+bitop3",
           "seq lshrrev+and+mul_lo_u32+bitop3", "seq lshrrev+mul_lo_u32+bitop3", "seq and+mul_lo_u32+bitop3",
           "seq perm+and", "seq bfe+mul_lo_u32+bitop3 interleaved")


def time_isa_rates(dev, iters: int = 2048) -> dict:
    """Issue rates of the decode's VALU instruction kinds (csrc/exl3_probe.hip
    probe_isa_kernel): each kind alone in a loop of eight independent chains,
    four-wave workgroups (a wave per SIMD of a CU) at 1, 2 and 4 waves per
    SIMD.  Returns SIMD cycles per wave64 instruction two ways: from the
    launch's event time at the loop's shader clock (median of three after one
    warm-up), and from each wave's own loop cycles divided by the waves
    sharing its SIMD."""
    import ctypes

    import torch
    from dsv4_carve_amd import build as B

    lib = ctypes.CDLL(B.PROBE_LIB)
    lib.exl3_probe_isa.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                                   ctypes.c_void_p]
    lib.exl3_probe_isa.restype = ctypes.c_int
    assert int(lib.exl3_probe_isa_ops()) == len(ISA_OPS)
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    simds = 4 * cus
    sink = torch.empty(4 * simds * 64, dtype=torch.int32, device=dev)
    clk = torch.zeros(2 * 4 * simds, dtype=torch.int64, device=dev)
    stream = int(torch.cuda.current_stream(dev).cuda_stream)
    out = {}
    for op, name in enumerate(ISA_OPS):
        per = {}
        for waves in (1, 2, 4):
            blocks = waves * cus
            nw = 4 * blocks
            ev, own = [], []
            for _ in range(4):
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record()
                assert lib.exl3_probe_isa(op, blocks, iters, sink.data_ptr(), clk.data_ptr(), stream) == 0
                b.record()
                torch.cuda.synchronize()
                t = a.elapsed_time(b) * 1e-3
                c = clk[:2 * nw].view(nw, 2).double()
                ghz = c[:, 0].sum().item() / c[:, 1].sum().item() * 0.1      # reference ticks at 100 MHz
                ev.append(t * ghz * 1e9 * simds / (nw * iters * 64.0))
                own.append(c[:, 0].mean().item() / (waves * iters * 64.0))
            per[f"{waves}_waves_per_simd"] = {"event": round(sorted(ev[1:])[1], 2),
                                              "per_wave_loop": round(sorted(own[1:])[1], 2)}
        out[name] = per
    del sink, clk
    return {"unit": "SIMD cycles per wave64 instruction", "chains_per_lane": 8, "iters": iters, **out}


def decode_floor_us(rate: dict, rows: int, bits: list[int], hidden: int, inter: int, topk: int, seed: int) -> float:
    """Lower bound on one routed layer's time from the decode rate alone: the
    mean, over the headline's routing pool, of each distinct expert's
    3*hidden*inter weights divided by its width's decode rate."""
    from dsv4_carve_amd import synth

    per = []
    for i in range(POOL):
        ids = synth.routing(rows, len(bits), topk, seed=seed * 1000 + i)[0]
        active = {int(e) for e in ids.reshape(-1) if 0 <= e < len(bits)}
        per.append(sum(3.0 * hidden * inter / (rate[f"K{bits[e]}"]["Gweights_per_s"] * 1e9) for e in active))
    return float(np.mean(per)) * 1e6


CPU_SAMPLE = 10          # experts per bit width timed on the CPU


def cpu_baseline(rows: int, bits: list[int], seed: int, us_ids: np.ndarray) -> dict:
    """CPU restatement timed on ten 3-bit and ten 2-bit experts of the layer
    (about 10 s of CPU work), scaled to the mean set of distinct experts per
    step at this row count."""
    import torch
    from dsv4_carve_amd import synth
    from oracle import cpu_baseline as CB

    def timed(e, b):
        t = CB.time_expert(synth.expert(e, HIDDEN, INTER, b, seed), rows)
        print(f"[bench] cpu baseline: expert {e} ({b}-bit) {t * 1e3:.0f} ms", file=sys.stderr, flush=True)
        return t

    t3 = float(np.mean([timed(e, 3) for e in range(CPU_SAMPLE)]))
    t2 = float(np.mean([timed(e, 2) for e in range(128, 128 + CPU_SAMPLE)]))
    n3 = n2 = 0.0
    for ids in us_ids:
        act = {int(e) for e in ids.reshape(-1)}
        n3 += sum(1 for e in act if bits[e] == 3)
        n2 += sum(1 for e in act if bits[e] == 2)
    n3 /= len(us_ids)
    n2 /= len(us_ids)
    return {
        "value": round((n3 * t3 + n2 * t2) * 1e6, 1),
        "unit": "us/layer",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"experts 0-{CPU_SAMPLE - 1} (3-bit) and 128-{127 + CPU_SAMPLE} (2-bit) of the layer, {rows} rows each: gate+up+down with "
                   f"per-call dequant + fp32 matmul (the reference CPU path), median of 3 after 1 warm-up per "
                   f"expert; mean {t3 * 1e3:.0f} ms (3-bit) and {t2 * 1e3:.0f} ms (2-bit) per expert, scaled by "
                   f"the mean distinct experts per step ({n3:.1f} 3-bit + {n2:.1f} 2-bit)"),
    }


EXTRA_LEGS = ("ceiling", "null", "sweep", "rows17", "tp8", "prefill", "stack", "dense", "fan", "glue")


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--rows", type=int, default=16)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-extra", action="store_true", help="only the headline measurement")
    ap.add_argument("--extra", default=",".join(EXTRA_LEGS),
                    help="comma-separated extra measurements to run: " + ", ".join(EXTRA_LEGS))
    ap.add_argument("--eager", action="store_true", help="launch the timed steps one by one (no graph)")
    ap.add_argument("--dense-shapes", default=",".join(f"{k}x{n}" for k, n in DENSE_SHAPES),
                    help="dense leg: comma-separated KxN shapes")
    ap.add_argument("--dense-bits", default=",".join(str(b) for b in DENSE_BITS), help="dense leg: bit widths")
    ap.add_argument("--dense-rows", default=",".join(str(r) for r in DENSE_ROWS), help="dense leg: row counts")
    ap.add_argument("--prefill-routing", default="zipf,hot8",
                    help="prefill leg: zipf (Zipf(1.1) over 256 experts), hot8 (every token on 8 experts), or both")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="end with one device-to-device copy of this many MiB (HBM counter calibration)")
    a = ap.parse_args()
    legs = set() if a.no_extra else {x for x in a.extra.split(",") if x}
    if legs - set(EXTRA_LEGS):
        print(f"unknown --extra legs: {sorted(legs - set(EXTRA_LEGS))}", file=sys.stderr)
        return 2
    if a.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {a.gpus}); "
              "the layer fits one MI355X and value is that GPU's throughput.", file=sys.stderr)
        return 2
    import torch
    from dsv4_carve_amd import ops, synth

    if not torch.cuda.is_available():
        print("no HIP device", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    t0 = time.time()
    bits = synth.mixed_bits(EXPERTS)
    layer = DeviceLayer(dev, EXPERTS, HIDDEN, INTER, bits, seed=1)
    print(f"[bench] layer built in {time.time() - t0:.1f}s", file=sys.stderr, flush=True)

    us, nbytes = time_layer(layer, dev, a.rows, TOPK, a.steps, a.warmup, seed=a.rows, eager=a.eager)
    gbs = nbytes / (us * 1e-6) / 1e9
    print(f"[bench] rows={a.rows}: {us:.1f} us/layer, {gbs:.0f} GB/s", file=sys.stderr, flush=True)
    latency = {"cold": layer_latency(layer, dev, a.rows, TOPK, LATENCY_ITERS, seed=a.rows, cold=True),
               "warm": layer_latency(layer, dev, a.rows, TOPK, LATENCY_ITERS, seed=a.rows, cold=False)}
    print(f"[bench] per-call latency rows={a.rows}: {latency}", file=sys.stderr, flush=True)

    extra = {}
    if "ceiling" in legs:
        extra["hbm_read_ceiling"] = time_read_ceiling(dev)
        print(f"[bench] read ceiling: {extra['hbm_read_ceiling']}", file=sys.stderr, flush=True)
        extra["xcd_handoff"] = time_handoff(dev)
        print(f"[bench] cross-launch hand-off: {extra['xcd_handoff']}", file=sys.stderr, flush=True)
        dc = time_decode_ceiling(dev)
        floor = decode_floor_us(dc, a.rows, layer.bits, HIDDEN, INTER, TOPK, seed=a.rows)
        mem = nbytes / (extra["hbm_read_ceiling"]["best_p50_GBps"] * 1e9) * 1e6
        dc[f"layer_floor_us_rows{a.rows}"] = {"decode": round(floor, 1), "memory_at_read_ceiling": round(mem, 1),
                                              "measured": round(us, 1)}
        extra["decode_ceiling"] = dc
        print(f"[bench] decode ceiling: {dc}", file=sys.stderr, flush=True)
        extra["isa_issue_rates"] = time_isa_rates(dev)
        print(f"[bench] instruction issue rates: {extra['isa_issue_rates']}", file=sys.stderr, flush=True)
        extra["row_block_rates"] = time_row_blocks(dev)
        print(f"[bench] row-block rates: {extra['row_block_rates']}", file=sys.stderr, flush=True)
        extra["gemm_step_rates"] = time_gemm_steps(dev)
        print(f"[bench] prefill step rates: {extra['gemm_step_rates']}", file=sys.stderr, flush=True)
    if "null" in legs:
        # The same workloads on the timing-only twin library (each decoded
        # weight replaced by a loaded tile word): the skeleton of loads, MFMAs,
        # stores and launches the decode runs on, measured, not argued.
        from dsv4_carve_amd import _lib, build as B

        twin = _lib.load_twin(B.NULL_LIB)
        nl = {}
        for m in (1, a.rows):
            u_null, _ = time_layer(layer, dev, m, TOPK, a.steps, 3, seed=m, lib=twin)
            u_real = us if m == a.rows else time_layer(layer, dev, m, TOPK, a.steps, 3, seed=m)[0]
            nl[f"layer_rows{m}"] = {"null_decode_us": round(u_null, 2), "with_decode_us": round(u_real, 2)}
        up_null = time_prefill(layer, dev, 512, TOPK, 10, 2, seed=4242, lib=twin)[0]
        up_real = time_prefill(layer, dev, 512, TOPK, 10, 2, seed=4242)[0]
        nl["prefill_512_tokens"] = {"null_decode_us": round(up_null, 1), "with_decode_us": round(up_real, 1)}
        dn = time_dense(dev, 4096, 4096, 6, [1], lib=twin)["1"]["us"]
        dr = time_dense(dev, 4096, 4096, 6, [1])["1"]["us"]
        nl["dense_4096x4096_K6_rows1"] = {"null_decode_us": dn, "with_decode_us": dr}
        extra["null_decode"] = {"library": "libexl3_null.so (EXL3_NULL_DECODE=1)", **nl}
        print(f"[bench] null decode: {extra['null_decode']}", file=sys.stderr, flush=True)
    if "sweep" in legs:
        sweep = {}
        for m in (1, 2, 4, 8, 16):
            u, b = time_layer(layer, dev, m, TOPK, a.steps, 3, seed=m)
            uw, bw = time_layer(layer, dev, m, TOPK, a.steps, 3, seed=m, same_routing=True)
            sweep[str(m)] = {"us": round(u, 2), "GBps": round(b / (u * 1e-6) / 1e9, 1),
                             "frac": round(b / (u * 1e-6) / 1e9 / HBM_PEAK_GBS, 4), "bytes": int(b),
                             "warm_us": round(uw, 2), "warm_GBps": round(bw / (uw * 1e-6) / 1e9, 1),
                             "latency_per_call": {
                                 "cold": layer_latency(layer, dev, m, TOPK, LATENCY_ITERS, seed=m, cold=True),
                                 "warm": layer_latency(layer, dev, m, TOPK, LATENCY_ITERS, seed=m, cold=False)}}
            print(f"[bench] sweep m={m}: {sweep[str(m)]}", file=sys.stderr, flush=True)
        extra["rows_sweep"] = sweep
    if "rows17" in legs:
        # 17-32 rows (the reference's lna2 takes up to 24): the decode
        # launches, and the grouped-GEMM (prefill) path on the same routing.
        big = {}
        for m in (17, 20, 24, 32):
            u, b = time_layer(layer, dev, m, TOPK, a.steps, 3, seed=m)
            up, _, _, _ = time_prefill(layer, dev, m, TOPK, 20, 2, seed=m * 1000, zipf=False)
            big[str(m)] = {"us": round(u, 2), "GBps": round(b / (u * 1e-6) / 1e9, 1),
                           "frac": round(b / (u * 1e-6) / 1e9 / HBM_PEAK_GBS, 4), "grouped_gemm_us": round(up, 2)}
            print(f"[bench] rows m={m}: {big[str(m)]}", file=sys.stderr, flush=True)
        extra["rows_17_32"] = big
    if "tp8" in legs:
        # The reference's own geometry: one GPU's share of the layer under TP8
        # (hidden 4096, intermediate 256, top-6, all experts at one width).
        tp = {}
        for kb in (2, 3):
            tl = DeviceLayer(dev, EXPERTS, HIDDEN, 256, [kb] * EXPERTS, seed=7 + kb)
            tp[f"K{kb}"] = {}
            for m in (1, 2, 4, 8, 16):
                u, b = time_layer(tl, dev, m, 6, 40, 3, seed=100 + m)
                # per call, the reference's method (recipe-lna/lna2/bench_lna.py:26-60):
                # a > 512 MB flush before every call, 40 calls, p50 / p95
                cold = layer_latency(tl, dev, m, 6, LATENCY_ITERS, seed=100 + m, cold=True)
                tp[f"K{kb}"][str(m)] = {"us": round(u, 2), "GBps": round(b / (u * 1e-6) / 1e9, 1),
                                        "per_call_cold": cold}
                print(f"[bench] tp8 slice K{kb} m={m}: {tp[f'K{kb}'][str(m)]}", file=sys.stderr, flush=True)
            del tl
            torch.cuda.empty_cache()
        extra["tp8_slice_h4096_i256_top6"] = tp

    if "prefill" in legs and "hot8" in a.prefill_routing:
        ush, flh, _, _ = time_prefill(layer, dev, 512, TOPK, 10, 2, seed=4242, hot8=True)
        extra["prefill_512_tokens_hot8"] = {"us_per_layer": round(ush, 1), "tokens_per_s": round(512 / (ush * 1e-6), 0),
                                            "tflops": round(flh / (ush * 1e-6) / 1e12, 2),
                                            "mfma_frac_fp16": round(flh / (ush * 1e-6) / MFMA_PEAK_F16, 4),
                                            "decoded_gweights": round(8 * 8 * 3.0 * HIDDEN * INTER / 1e9, 2)}
        print(f"[bench] prefill 512 tokens, 8 hot experts: {extra['prefill_512_tokens_hot8']}", file=sys.stderr,
              flush=True)
    if "prefill" in legs and "zipf" in a.prefill_routing:
        usp, fl, bp, dist = time_prefill(layer, dev, 512, TOPK, 10, 2, seed=4242)
        extra["prefill_512_tokens_zipf1.1"] = {
            "us_per_layer": round(usp, 1), "tokens_per_s": round(512 / (usp * 1e-6), 0),
            "tflops": round(fl / (usp * 1e-6) / 1e12, 2), "mfma_frac_fp16": round(fl / (usp * 1e-6) / MFMA_PEAK_F16, 4),
            "GBps": round(bp / (usp * 1e-6) / 1e9, 1), "hbm_frac": round(bp / (usp * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "distinct_experts": dist, "algorithmic_gflop": round(fl / 1e9, 1), "bytes": int(bp)}
        dw, dmin = prefill_decoded_weights(layer, 512, TOPK, seed=4242)
        extra["prefill_512_tokens_zipf1.1"]["decoded_gweights"] = round(dw / 1e9, 2)
        extra["prefill_512_tokens_zipf1.1"]["decoded_gweights_min"] = round(dmin / 1e9, 2)
        print(f"[bench] prefill 512 tokens: {extra['prefill_512_tokens_zipf1.1']}", file=sys.stderr, flush=True)
    if "stack" in legs:
        us3, b3 = time_stack(dev, 16, 4, 1)
        extra["stack_43_layers_routed_plus_shared_rows16"] = {
            "us_per_step": round(us3, 1), "GBps": round(b3 / (us3 * 1e-6) / 1e9, 1),
            "frac": round(b3 / (us3 * 1e-6) / 1e9 / HBM_PEAK_GBS, 4), "bytes_per_step": int(b3)}
        print(f"[bench] 43-layer stack: {extra['stack_43_layers_routed_plus_shared_rows16']}", file=sys.stderr,
              flush=True)
    if "dense" in legs:
        dense = {}
        shapes = [tuple(int(v) for v in sh.split("x")) for sh in a.dense_shapes.split(",") if sh]
        dense_rows = [int(r) for r in a.dense_rows.split(",") if r]
        for (k, n) in shapes:
            for b in (int(v) for v in a.dense_bits.split(",") if v):
                key = f"{k}x{n}_K{b}"
                dense[key] = time_dense(dev, k, n, b, dense_rows)
                print(f"[bench] dense {key}: {dense[key]}", file=sys.stderr, flush=True)
        extra["dense_gemv_cold"] = dense
        lin = {}
        for (k, n) in LINEAR_SHAPES:
            lin[f"{k}x{n}_K3"] = time_linear(dev, k, n, 3, LINEAR_ROWS)
            print(f"[bench] linear {k}x{n}_K3: {lin[f'{k}x{n}_K3']}", file=sys.stderr, flush=True)
        extra["dense_linear_forward"] = lin
        if not a.no_cpu:
            # the single-linear CPU reference path (4096 x 4096, 6-bit, one row),
            # and every dense shape and width of the sweep at one row
            from oracle import cpu_baseline as CB
            lin = synth.dense(4096, 4096, 6, seed=3)
            t = CB.time_linear(lin, 1)
            extra["dense_4096x4096_K6_cpu"] = {"us": round(t * 1e6, 1), "cores": CB.threads(),
                                               "sample": "dequant + fp32 matmul per call, median of 5 after 1 warm-up"}
            print(f"[bench] dense cpu: {extra['dense_4096x4096_K6_cpu']}", file=sys.stderr, flush=True)
            sweep_cpu = {}
            for (k, n) in shapes:
                for b in DENSE_BITS:
                    sweep_cpu[f"{k}x{n}_K{b}"] = round(CB.time_linear(synth.dense(k, n, b, seed=3), 1, reps=3) * 1e6, 1)
            extra["dense_cpu_1row_us"] = {"us": sweep_cpu, "cores": CB.threads(),
                                          "sample": "one row, dequant + fp32 matmul per call, median of 3 after 1 warm-up"}
            print(f"[bench] dense cpu sweep: {extra['dense_cpu_1row_us']}", file=sys.stderr, flush=True)

    if "fan" in legs:
        fans = {}
        for name, (k, ns, b) in FANS.items():
            fans[name] = time_fan(dev, k, ns, b, FAN_ROWS)
            print(f"[bench] fan {name}: {fans[name]}", file=sys.stderr, flush=True)
        extra["dense_fan_cold"] = fans

    if "glue" in legs:
        glue = {}
        for m in (1, 4, 16):
            glue[str(m)] = time_glue(layer, dev, m, TOPK)
            print(f"[bench] routing glue m={m}: {glue[str(m)]}", file=sys.stderr, flush=True)
        extra["routing_glue_graph_replay"] = glue

    cpu = None
    if not a.no_cpu:
        pool_ids = [synth.routing(a.rows, EXPERTS, TOPK, seed=a.rows * 1000 + i)[0] for i in range(POOL)]
        cpu = cpu_baseline(a.rows, bits, seed=1, us_ids=pool_ids)
        print(f"[bench] cpu baseline: {cpu}", file=sys.stderr, flush=True)
        key = "stack_43_layers_routed_plus_shared_rows16"
        if key in extra and a.rows == 16:
            # the stack on CPU: one block (this routed layer + the 6-bit shared
            # expert, both timed) times 43
            from oracle import cpu_baseline as CB
            t6 = CB.time_expert(synth.expert(EXPERTS, HIDDEN, INTER, 6, seed=1), a.rows)
            block_us = cpu["value"] + t6 * 1e6
            extra[key]["cpu_estimate"] = {
                "us_per_step": round(C3_LAYERS * block_us, 0), "cores": CB.threads(),
                "sample": (f"one block timed and multiplied by {C3_LAYERS}: the routed layer's CPU baseline "
                           f"({cpu['value']:.0f} us) plus one 6-bit shared expert at 16 rows ({t6 * 1e6:.0f} us)")}
            print(f"[bench] stack cpu estimate: {extra[key]['cpu_estimate']}", file=sys.stderr, flush=True)

    if a.calib_copy_mib:
        src = torch.ones(a.calib_copy_mib << 18, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        print(f"[bench] calibration copy: {a.calib_copy_mib} MiB read + {a.calib_copy_mib} MiB written",
              file=sys.stderr, flush=True)

    # HBM bytes per layer from the committed counter profile of this workload
    # at 16 rows (not measured in this run; reported only at that row count)
    traffic, traffic_source = None, None
    prof = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "moe_c2_m16_traffic.json")
    if a.rows == 16 and os.path.isfile(prof):
        with open(prof) as f:
            meta = json.load(f)
        traffic = meta.get("hbm_bytes_per_layer")
        traffic_source = meta.get("source") or "profiles/moe_c2_m16_traffic.json (rocprofv3 --pmc, 16 rows)"

    line = {
        "metric": "routed-MoE decode us/layer + achieved HBM GB/s (% of 8 TB/s), rows 1-16",
        "value": round(us, 2),
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(us / 1000.0, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic (seeded EXL3 trellis weights, N(0,1) router logits and activations)",
        "config": {"workload": "routed-MoE decode layer: 256 experts, top-8, hidden 4096, intermediate 2048, "
                               "experts 0-127 3-bit / 128-255 2-bit EXL3 MCG, fresh routing each step",
                   "rows": a.rows, "experts": EXPERTS, "topk": TOPK, "hidden": HIDDEN, "intermediate": INTER},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic, "traffic_source": traffic_source,
                     "bytes_per_layer": int(nbytes)},
        "latency_per_call": latency,
        "cpu_baseline": cpu,
    }
    line.update(extra)
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
