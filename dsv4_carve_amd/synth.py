"""Seeded synthetic EXL3 tensors of the benchmark shapes (numpy, CPU).

Packed trellis bits are uniform random from the seed; suh is a random +-1 fp16
sign vector; svh is +-1 times a per-output-channel scale drawn uniformly from
[0.5, 2] / sqrt(in_features) (the checkpoint ABI has no separate scale tensor:
LinearEXL3 asserts scale is None, recipe-lna/exllamav3/exl3.py.lna:38, so the
scale lives in svh).  The same bytes are copied to the GPU, so CPU and GPU see
identical inputs."""

from __future__ import annotations

import numpy as np

MCG_MARKER = -877912083


def _rng(*seed) -> np.random.Generator:
    return np.random.default_rng([int(s) & 0xFFFFFFFF for s in seed])


def signs(rng: np.random.Generator, n: int) -> np.ndarray:
    return np.where(rng.integers(0, 2, n) == 1, 1.0, -1.0).astype(np.float16)


def dense(k: int, n: int, bits: int, seed: int) -> dict:
    """One EXL3 linear: trellis int16 [k/16, n/16, 16*bits], suh fp16 [k], svh fp16 [n]."""
    rng = _rng(seed, k, n, bits)
    trellis = rng.integers(0, 1 << 16, size=(k // 16, n // 16, 16 * bits), dtype=np.uint16).view(np.int16)
    suh = signs(rng, k)
    scale = rng.uniform(0.5, 2.0, n) / np.sqrt(k)
    svh = (signs(rng, n).astype(np.float64) * scale).astype(np.float16)
    return {"trellis": trellis, "suh": suh, "svh": svh, "bits": bits}


def activations(rows: int, k: int, seed: int, dtype=np.float16) -> np.ndarray:
    return _rng(seed, rows, k, 7).standard_normal((rows, k)).astype(dtype)


def expert(e: int, hidden: int, inter: int, bits: int, seed: int) -> dict:
    """gate/up: hidden -> inter, down: inter -> hidden, all at `bits`."""
    return {
        "bits": bits,
        "gate": dense(hidden, inter, bits, seed * 1_000_003 + 3 * e + 0),
        "up": dense(hidden, inter, bits, seed * 1_000_003 + 3 * e + 1),
        "down": dense(inter, hidden, bits, seed * 1_000_003 + 3 * e + 2),
    }


def mixed_bits(n_experts: int, hi: int = 3, lo: int = 2) -> list[int]:
    """The MoE layer's bit rule: the first half of the experts at `hi` bits, the rest at `lo`."""
    return [hi if e < n_experts // 2 else lo for e in range(n_experts)]


def routing(m: int, n_experts: int, topk: int, seed: int) -> tuple[np.ndarray, np.ndarray]:
    """Top-k of N(0,1) router logits per row (distinct ids), softmax over the k."""
    logits = _rng(seed, m, n_experts, 11).standard_normal((m, n_experts)).astype(np.float32)
    ids = np.argsort(-logits, axis=1, kind="stable")[:, :topk].astype(np.int32)
    top = np.take_along_axis(logits, ids, axis=1)
    w = np.exp(top - top.max(axis=1, keepdims=True))
    w = (w / w.sum(axis=1, keepdims=True)).astype(np.float32)
    return ids, w


def zipf_routing(tokens: int, n_experts: int, topk: int, seed: int, s: float = 1.1):
    """Top-k without replacement from a Zipf(s) popularity over a seeded expert
    permutation, softmax weights from N(0,1) logits (prefill-shaped routing)."""
    rng = _rng(seed, tokens, n_experts, 13)
    perm = rng.permutation(n_experts)
    p = 1.0 / np.arange(1, n_experts + 1) ** s
    p = p / p.sum()
    ids = np.empty((tokens, topk), np.int32)
    for t in range(tokens):
        ids[t] = perm[rng.choice(n_experts, size=topk, replace=False, p=p)]
    logits = rng.standard_normal((tokens, topk)).astype(np.float32)
    w = np.exp(logits - logits.max(axis=1, keepdims=True))
    return ids, (w / w.sum(axis=1, keepdims=True)).astype(np.float32)
