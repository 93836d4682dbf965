"""CPU baseline for bench.py -- part of the oracle (test infrastructure).

A multithreaded torch-CPU restatement of the reference's CPU path for this
layer: vllm_exl3_c.exl3_gemv's CPU fallback re-dequantizes the trellis on every
call (dequant_trellis -> dequant_cpu: window extraction, codebook, tile
permutation, both 128-block Hadamards with suh/svh) and multiplies in fp32
(recipe-lna/lna2/bindings.cpp:16-101, 135-148); the routed layer is the python
loop over distinct experts (recipe-lna/vllm_exl3_exl3.py.lna:988-1027).  The
decode here is vectorised with torch integer ops and the Hadamards run as fp32
block matmuls, so every host core is used; it is timed, never checked against.
"""

from __future__ import annotations

import os
import time

import numpy as np
import torch

from oracle import oracle as O


def _tables(bits: int):
    i0, i1, s = O._window_tables(bits)
    return (torch.from_numpy(i0.astype(np.int64)), torch.from_numpy(i1.astype(np.int64)),
            torch.from_numpy(s.astype(np.int64)), torch.from_numpy(O._perm().astype(np.int64)))


_H128 = None


def _h128() -> torch.Tensor:
    global _H128
    if _H128 is None:
        import scipy.linalg

        _H128 = torch.from_numpy(scipy.linalg.hadamard(128).astype(np.float32))
    return _H128


def dequant_full(trellis: torch.Tensor, suh: torch.Tensor, svh: torch.Tensor, bits: int,
                 lut: torch.Tensor) -> torch.Tensor:
    """W = diag(suh) H Wq H diag(svh) / 128 as fp32 [K, N] (CPU, all threads)."""
    kt, nt, _ = trellis.shape
    i0, i1, s, perm = _tables(bits)
    words = trellis.view(torch.int32).reshape(-1, 8 * bits).to(torch.int64) & 0xFFFFFFFF
    merged = (words[:, i0] << 32) | words[:, i1]
    win = (merged >> s) & 0xFFFF
    w = lut[win].reshape(kt, nt, 256)[:, :, perm].reshape(kt, nt, 16, 16)
    W = w.permute(0, 2, 1, 3).reshape(kt * 16, nt * 16).to(torch.float32)
    K, N = W.shape
    H = _h128()
    W = (W.reshape(K, N // 128, 128) @ H).reshape(K, N)                  # row transforms
    W = (H @ W.reshape(K // 128, 128, N)).reshape(K, N)                  # column transforms
    return W * (suh.to(torch.float32)[:, None] / 128.0) * svh.to(torch.float32)[None, :]


def linear(x32: torch.Tensor, p: dict, bits: int, lut: torch.Tensor) -> torch.Tensor:
    W = dequant_full(torch.from_numpy(p["trellis"]), torch.from_numpy(p["suh"]),
                     torch.from_numpy(p["svh"]), bits, lut)
    return x32 @ W


def expert_rows(x16: np.ndarray, ex: dict, limit: float, lut: torch.Tensor) -> torch.Tensor:
    x = torch.from_numpy(x16.astype(np.float32))
    g = linear(x, ex["gate"], ex["bits"], lut)
    u = linear(x, ex["up"], ex["bits"], lut)
    act = torch.nn.functional.silu(g.clamp(max=limit)) * u.clamp(min=-limit, max=limit)
    return linear(act.half().float(), ex["down"], ex["bits"], lut)


def threads() -> int:
    """Host threads for the baseline: every core, capped by OMP_NUM_THREADS when set."""
    n = os.cpu_count() or 1
    env = os.environ.get("OMP_NUM_THREADS")
    return min(n, int(env)) if env and env.isdigit() and int(env) > 0 else n


def time_expert(ex: dict, rows: int, reps: int = 3, limit: float = 10.0) -> float:
    """Median seconds for one expert's gate+up+down on `rows` rows (dequant each call)."""
    torch.set_num_threads(threads())
    lut = torch.from_numpy(O.codebook_lut(O.CB_MCG).view(np.float16).copy())
    x = np.random.default_rng(0).standard_normal((rows, ex["gate"]["suh"].size)).astype(np.float16)
    expert_rows(x, ex, limit, lut)                 # warm-up
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        expert_rows(x, ex, limit, lut)
        ts.append(time.perf_counter() - t0)
    return float(np.median(ts))


def time_linear(p: dict, rows: int, reps: int = 5) -> float:
    """Median seconds for one dense linear (dequant each call + fp32 matmul)."""
    torch.set_num_threads(threads())
    lut = torch.from_numpy(O.codebook_lut(O.CB_MCG).view(np.float16).copy())
    x = torch.from_numpy(np.random.default_rng(1).standard_normal((rows, p["suh"].size)).astype(np.float32))
    linear(x, p, p["bits"], lut)
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        linear(x, p, p["bits"], lut)
        ts.append(time.perf_counter() - t0)
    return float(np.median(ts))
