"""EXL3 decode-path ORACLE -- test infrastructure only.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker.  The product path
(``dsv4_carve_amd``) never imports it.

Two restatements of the same algorithm live here:

* the bit-serial C spec in ``exl3_oracle.c`` (loaded through ctypes), and
* a vectorised numpy restatement (``reconstruct_np`` and friends) that gathers
  every window of every tile at once through precomputed word/shift tables.

Tests pin the two against each other, against the reference's own host helpers
(``orders/F1-ref/exl3_dequant.cuh`` built into ``oracle/_ref``), against numpy's
IEEE binary16 conversion and against the published m16n8k16 fragment layout.

Reference rounding points reproduced (file:line in the reference tree):

* codebooks: ``orders/F1-ref/exl3_dequant.cuh:73-92`` with round-to-nearest-even
  half arithmetic (the GPU canon ``recipe-lna/lna2/primitive_gate.cu:25-31``);
* tile permutation: ``recipe-lna/lna2/bindings.cpp:33-77``;
* input rotation: ``recipe-lna/lna2/lna_moe_ticket.cu:119-144`` (x*suh in half,
  fp32 butterflies, *1/sqrt(128), RNE to half);
* output rotation + svh in fp32: ``lna_moe_ticket.cu:342-343, 376``;
* full dequant order: ``recipe-lna/lna2/bindings.cpp:80-99``;
* dense linear: ``recipe-lna/lna2/bindings.cpp:135-148`` (dequant then an fp32
  matmul; here the matmul runs in float64, which is at least as accurate);
* routed MoE: ``recipe-lna/vllm_exl3_exl3.py.lna:988-1027`` (python loop) with the
  lna2 precision boundaries ``lna_moe_ticket.cu:5-12, 344-354, 409-428``
  (act = silu(min(g,L)) * clamp(u,-L,L) in fp32 -> half; expert sum in fp32 in
  top-k slot order).

The weights of that path are the codebook values rounded to binary16.  The
same layer on the exact sums of each value's binary16 addends
(``codebook_addend_sum_lut``, ``reconstruct_exact``,
``moe(..., exact_addends=True)``: the two masked halves of 3INST and MCG; MUL1
has one addend, its binary16 value) is what the GPU kernels compute, since
their matrix cores add the addends themselves; the tests use it beside the
rounded-weight oracle.  Its values are pinned against the numpy restatement
of the addends and by rounding back to the binary16 codebook.
"""

from __future__ import annotations

import ctypes
import os
from functools import lru_cache

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libexl3_oracle.so")
_REF_PATH = os.path.join(_HERE, "_ref", "libexl3_ref.so")

HAD_NORM = np.float32(0.08838834764831845)
MCG_MARKER = -877912083
MUL1_MARKER = -2082680531
CB_3INST, CB_MCG, CB_MUL1 = 0, 1, 2


def build_oracle() -> None:
    """Compile the C oracle (and the reference helper library when present)."""
    import subprocess

    subprocess.run(["make", "-s", "-C", _HERE, "all"], check=True)
    if os.path.isfile("/root/reference/orders/F1-ref/exl3_dequant.cuh"):
        subprocess.run(["make", "-s", "-C", _HERE, "ref"], check=True)


@lru_cache(maxsize=1)
def lib() -> ctypes.CDLL:
    if not os.path.isfile(_LIB_PATH):
        build_oracle()
    L = ctypes.CDLL(_LIB_PATH)
    u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
    f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
    L.ora_window.argtypes = [u16p, ctypes.c_int, ctypes.c_int]
    L.ora_window.restype = ctypes.c_uint16
    L.ora_codebook.argtypes = [ctypes.c_uint16, ctypes.c_int]
    L.ora_codebook.restype = ctypes.c_uint16
    L.ora_codebook_lut.argtypes = [ctypes.c_int, u16p]
    L.ora_codebook_addend_sum_lut.argtypes = [ctypes.c_int, np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")]
    L.ora_tile_t.argtypes = [ctypes.c_int, ctypes.c_int]
    L.ora_tile_t.restype = ctypes.c_int
    L.ora_reconstruct.argtypes = [u16p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, u16p]
    L.ora_reconstruct_fast.argtypes = [u16p, ctypes.c_int, ctypes.c_int, ctypes.c_int, u16p, u16p]
    L.ora_fwht.argtypes = [f32p, ctypes.c_int]
    L.ora_had_in.argtypes = [u16p, u16p, ctypes.c_int, ctypes.c_int, u16p]
    L.ora_had_out.argtypes = [f32p, u16p, ctypes.c_int, ctypes.c_int, f32p]
    L.ora_dequant_full.argtypes = [u16p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                   u16p, u16p, f32p, u16p, u16p]
    L.ora_double_to_half.argtypes = [ctypes.c_double]
    L.ora_double_to_half.restype = ctypes.c_uint16
    L.ora_half_to_float.argtypes = [ctypes.c_uint16]
    L.ora_half_to_float.restype = ctypes.c_float
    return L


@lru_cache(maxsize=1)
def ref_lib() -> ctypes.CDLL | None:
    """The reference's own host helpers (orders/F1-ref/exl3_dequant.cuh), if built."""
    if not os.path.isfile(_REF_PATH):
        return None
    L = ctypes.CDLL(_REF_PATH)
    u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
    f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
    L.ref_read_window.argtypes = [u16p, ctypes.c_size_t, ctypes.c_size_t]
    L.ref_read_window.restype = ctypes.c_uint16
    L.ref_decode_codebook_bits.argtypes = [ctypes.c_uint16, ctypes.c_int]
    L.ref_decode_codebook_bits.restype = ctypes.c_uint16
    L.ref_decode_weight.argtypes = [u16p, ctypes.c_size_t, ctypes.c_int, ctypes.c_int, ctypes.c_int]
    L.ref_decode_weight.restype = ctypes.c_float
    L.ref_half_bits_to_float.argtypes = [ctypes.c_uint16]
    L.ref_half_bits_to_float.restype = ctypes.c_float
    L.ref_float_to_half_bits.argtypes = [ctypes.c_float]
    L.ref_float_to_half_bits.restype = ctypes.c_uint16
    L.ref_hadamard.argtypes = [f32p, ctypes.c_int]
    return L


def _u16(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a).view(np.uint16) if a.dtype in (np.int16, np.float16) else \
        np.ascontiguousarray(a, dtype=np.uint16)


# ---------------------------------------------------------------- C spec wrappers

def window(tile: np.ndarray, bits: int, t: int) -> int:
    return int(lib().ora_window(_u16(tile), bits, t))


def codebook(w: int, cb: int = CB_MCG) -> int:
    return int(lib().ora_codebook(w, cb))


@lru_cache(maxsize=3)
def codebook_lut(cb: int = CB_MCG) -> np.ndarray:
    """All 65536 codebook outputs as binary16 bit patterns (uint16)."""
    out = np.empty(65536, np.uint16)
    lib().ora_codebook_lut(cb, out)
    out.setflags(write=False)
    return out


def tile_t(k: int, n: int) -> int:
    return int(lib().ora_tile_t(k, n))


def reconstruct_c(trellis: np.ndarray, bits: int, cb: int = CB_MCG) -> np.ndarray:
    """Bit-serial C reconstruct: trellis int16 [K/16, N/16, 16*bits] -> fp16 [K, N]."""
    kt, nt, tw = trellis.shape
    assert tw == 16 * bits
    out = np.empty((kt * 16, nt * 16), np.uint16)
    lib().ora_reconstruct(_u16(trellis).reshape(-1), kt * 16, nt * 16, bits, cb, out.reshape(-1))
    return out.view(np.float16)


def reconstruct_fast(trellis: np.ndarray, bits: int, cb: int = CB_MCG) -> np.ndarray:
    """Funnel-shift C reconstruct with the codebook LUT (same result as reconstruct_c)."""
    kt, nt, tw = trellis.shape
    assert tw == 16 * bits
    out = np.empty((kt * 16, nt * 16), np.uint16)
    lib().ora_reconstruct_fast(_u16(trellis).reshape(-1), kt * 16, nt * 16, bits,
                               np.ascontiguousarray(codebook_lut(cb)), out.reshape(-1))
    return out.view(np.float16)


@lru_cache(maxsize=3)
def codebook_addend_sum_lut(cb: int = CB_MCG) -> np.ndarray:
    """All 65536 exact sums (float64) of the binary16 addends whose rounded sum
    is the codebook value: the two masked halves for 3INST and MCG; MUL1 is a
    single-rounded half FMA, one addend, so its entry is the binary16 value.
    codebook_lut(cb) is this rounded to nearest even."""
    out = np.empty(65536, np.float64)
    lib().ora_codebook_addend_sum_lut(cb, out)
    out.setflags(write=False)
    return out


def reconstruct_exact(trellis: np.ndarray, bits: int, cb: int = CB_MCG) -> np.ndarray:
    """Each element's exact addend sum (codebook_addend_sum_lut), float64
    [K, N]: the weight the GPU kernels use, which hand the addends to the
    matrix core and add them there in fp32.  The windows come from the same
    reconstruct as reconstruct_fast, run with the identity table."""
    kt, nt, tw = trellis.shape
    assert tw == 16 * bits
    win = np.empty((kt * 16, nt * 16), np.uint16)
    lib().ora_reconstruct_fast(_u16(trellis).reshape(-1), kt * 16, nt * 16, bits,
                               np.arange(65536, dtype=np.uint16), win.reshape(-1))
    return codebook_addend_sum_lut(cb)[win]


def dequant_full_c(trellis, suh, svh, bits, cb=CB_MCG) -> np.ndarray:
    kt, nt, _ = trellis.shape
    K, N = kt * 16, nt * 16
    scratch = np.empty(K * N, np.float32)
    wq = np.empty(K * N, np.uint16)
    out = np.empty((K, N), np.uint16)
    lib().ora_dequant_full(_u16(trellis).reshape(-1), K, N, bits, cb, _u16(suh), _u16(svh),
                           scratch, wq, out.reshape(-1))
    return out.view(np.float16)


def had_in_c(x16: np.ndarray, suh: np.ndarray) -> np.ndarray:
    rows, K = x16.shape
    out = np.empty((rows, K), np.uint16)
    lib().ora_had_in(_u16(x16).reshape(-1), _u16(suh), rows, K, out.reshape(-1))
    return out.view(np.float16)


def had_out_c(c: np.ndarray, svh: np.ndarray) -> np.ndarray:
    rows, N = c.shape
    out = np.empty((rows, N), np.float32)
    lib().ora_had_out(np.ascontiguousarray(c, np.float32).reshape(-1), _u16(svh), rows, N,
                      out.reshape(-1))
    return out


# ---------------------------------------------------------------- vectorised restatement

@lru_cache(maxsize=16)
def _window_tables(bits: int):
    """Per element t: (word index of the first window bit, of the last bit, right shift)."""
    nwords = 8 * bits
    t = np.arange(256)
    b0 = (t + 257) * bits - 16
    b1 = b0 + 16
    i0 = (b0 // 32) % nwords
    i1u = (b1 - 1) // 32
    s = (i1u + 1) * 32 - b1
    return i0.astype(np.intp), (i1u % nwords).astype(np.intp), s.astype(np.uint64)


@lru_cache(maxsize=1)
def _perm():
    """perm[k*16+n] = t(k, n)."""
    k = np.arange(16)[:, None]
    n = np.arange(16)[None, :]
    t = 8 * (4 * (n & 7) + ((k & 7) >> 1)) + 4 * (n >> 3) + 2 * (k >> 3) + (k & 1)
    return t.reshape(-1).astype(np.intp)


def windows_np(trellis: np.ndarray, bits: int) -> np.ndarray:
    """All 16-bit windows: trellis [..., 16*bits] int16 -> uint16 [..., 256] (index = t)."""
    lead = trellis.shape[:-1]
    words = np.ascontiguousarray(trellis).view(np.uint32).reshape(-1, 8 * bits).astype(np.uint64)
    i0, i1, s = _window_tables(bits)
    merged = (words[:, i0] << np.uint64(32)) | words[:, i1]
    w = ((merged >> s[None, :]) & np.uint64(0xFFFF)).astype(np.uint16)
    return w.reshape(lead + (256,))


def reconstruct_np(trellis: np.ndarray, bits: int, cb: int = CB_MCG) -> np.ndarray:
    """Vectorised reconstruct: int16 [K/16, N/16, 16*bits] -> fp16 [K, N]."""
    kt, nt, tw = trellis.shape
    assert tw == 16 * bits, (trellis.shape, bits)
    lut = codebook_lut(cb)
    dec = lut[windows_np(trellis, bits)]                 # [kt, nt, 256] by t
    tiles = dec[:, :, _perm()].reshape(kt, nt, 16, 16)   # [kt, nt, k, n]
    return tiles.transpose(0, 2, 1, 3).reshape(kt * 16, nt * 16).view(np.float16)


def fwht128_np(v: np.ndarray) -> np.ndarray:
    """Natural-order FWHT over the last axis in blocks of 128, same op order as the
    scalar loop (exl3_dequant.cuh:136-147), vectorised across blocks; fp32 in/out
    when given fp32 (each output is the same sequence of IEEE adds/subs)."""
    shape = v.shape
    a = v.reshape(-1, 128).copy()
    h = 1
    while h < 128:
        a = a.reshape(-1, 128 // (2 * h), 2, h)
        x = a[:, :, 0, :].copy()
        y = a[:, :, 1, :].copy()
        a[:, :, 0, :] = x + y
        a[:, :, 1, :] = x - y
        h *= 2
    return a.reshape(shape)


def had_in_np(x16: np.ndarray, suh: np.ndarray) -> np.ndarray:
    xs = (x16.astype(np.float32) * suh.astype(np.float32)).astype(np.float16)   # RNE half mul
    h = fwht128_np(xs.astype(np.float32))
    return (h * HAD_NORM).astype(np.float16)


def had_out_np(c: np.ndarray, svh: np.ndarray, dtype=np.float32) -> np.ndarray:
    h = fwht128_np(np.asarray(c, dtype))
    return h * dtype(HAD_NORM) * svh.astype(dtype)


def to_half_rne(x: np.ndarray) -> np.ndarray:
    """fp32/fp64 -> binary16 with round-to-nearest-even (numpy's IEEE conversion)."""
    return np.asarray(x, np.float32).astype(np.float16)


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


# ---------------------------------------------------------------- dense linear + MoE

def linear(x16: np.ndarray, trellis: np.ndarray, suh: np.ndarray, svh: np.ndarray,
           bits: int, cb: int = CB_MCG, w: np.ndarray | None = None) -> np.ndarray:
    """y = had_out(had_in(x) @ Wq) * svh, returned as float32 [rows, N].

    x16 fp16 [rows, K].  Matmul in float64 (>= the reference's fp32 at::mm,
    bindings.cpp:147); output rotation in float64 then rounded to fp32."""
    xh = had_in_np(x16, suh)
    if w is None:
        w = reconstruct_fast(trellis, bits, cb)
    acc = xh.astype(np.float64) @ w.astype(np.float64)
    return had_out_np(acc, svh, np.float64).astype(np.float32)


def swiglu_clamp(g: np.ndarray, u: np.ndarray, limit: float) -> np.ndarray:
    """act = silu(min(g, L)) * clamp(u, -L, L) in fp32 (lna_moe_ticket.cu:344-354)."""
    g = np.minimum(g.astype(np.float32), np.float32(limit))
    u = np.clip(u.astype(np.float32), np.float32(-limit), np.float32(limit))
    return (g / (np.float32(1.0) + np.exp(-g))) * u


def moe(x16: np.ndarray, ids: np.ndarray, weights: np.ndarray, experts: list[dict],
        limit: float, cb: int = CB_MCG, cache: dict | None = None, exact_addends: bool = False) -> np.ndarray:
    """Routed-expert decode reference, float32 [m, H].

    experts[e] = {"bits": K, "gate": {"trellis", "suh", "svh"}, "up": {...}, "down": {...}}.
    ids int [m, topk]; ids outside [0, len(experts)) contribute nothing.  Each
    distinct (expert, row) pair is computed once; the expert sum walks the
    top-k slots of each row in order, in fp32.  exact_addends: the weights are
    the exact sums of the codebook addends (reconstruct_exact), as the GPU
    kernels use them; otherwise the rounded weights of the reference's CPU
    path."""
    m, H = x16.shape
    topk = ids.shape[1]
    n_exp = len(experts)
    down_rows: dict[tuple[int, int], np.ndarray] = {}

    def expert_rows(e):
        rows = sorted({r for r in range(m) if e in [int(v) for v in ids[r]]})
        ex = experts[e]
        b = ex["bits"]

        def W(name):
            key = (e, name, cb, exact_addends)
            if cache is not None and key in cache:
                return cache[key]
            wq = (reconstruct_exact if exact_addends else reconstruct_fast)(ex[name]["trellis"], b, cb)
            if cache is not None:
                cache[key] = wq
            return wq

        def lin(h, name):
            p = ex[name]
            return linear(h, p["trellis"], p["suh"], p["svh"], b, cb, w=W(name))

        h = x16[rows]
        g = lin(h, "gate")
        u = lin(h, "up")
        act = to_half_rne(swiglu_clamp(g, u, limit))
        d = lin(act, "down")
        return [((e, r), d[i]) for i, r in enumerate(rows)]

    # Experts are independent: large layers run them on a thread pool (the C
    # reconstruct and numpy's matmul release the GIL); the slot-order sum below
    # is the same whatever the order they finish in.
    active = sorted({int(v) for v in ids.reshape(-1) if 0 <= int(v) < n_exp})
    workers = min(16, os.cpu_count() or 1, len(active))
    if workers > 1 and len(active) >= 8:
        from concurrent.futures import ThreadPoolExecutor

        with ThreadPoolExecutor(max_workers=workers) as pool:
            for pairs in pool.map(expert_rows, active):
                down_rows.update(pairs)
    else:
        for e in active:
            down_rows.update(expert_rows(e))
    out = np.zeros((m, H), np.float32)
    for r in range(m):
        acc = np.zeros(H, np.float32)
        for k in range(topk):
            e = int(ids[r, k])
            if 0 <= e < n_exp:
                acc = acc + np.float32(weights[r, k]) * down_rows[(e, r)]
        out[r] = acc
    return out
