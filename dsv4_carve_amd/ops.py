"""Torch custom ops over the C ABI (include/exl3_amd.h).

Every op is registered in the ``exl3_amd`` torch.library namespace with a CUDA
(= HIP on ROCm) implementation only, so a CPU tensor fails in the dispatcher and
a missing ``libexl3_amd.so`` fails at the first call: there is no fallback.
Launches go to torch's current stream and never allocate, so they are
capturable with ``torch.cuda.graph`` once the shared scratch exists.

Reference call surfaces mirrored here:
  * ``dequant_trellis``  -- vllm_exl3_c, recipe-lna/lna2/bindings.cpp:118-133
  * ``reconstruct``      -- exllamav3_ext, used at recipe-lna/exllamav3/exl3.py.lna:197
  * ``exl3_gemm``        -- exllamav3_ext, recipe-lna/exllamav3/exl3_gemm.cu.lna:336-364
  * ``exl3_gemv``        -- vllm_exl3_c, recipe-lna/lna2/bindings.cpp:135-148
  * ``lna2_moe_decode`` and its helpers -- vllm_exl3_c,
    recipe-lna/lna2/lna_moe_ticket.cu:481-581, bindings.cpp:212-219
"""

from __future__ import annotations

import threading

import torch

from . import _lib

CB_3INST, CB_MCG, CB_MUL1 = 0, 1, 2
OUT_KIND = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}
X_KIND = {torch.float16: 0, torch.bfloat16: 1}
IDS_KIND = {torch.int32: 0, torch.int64: 1}


def codebook_id(mcg: bool, mul1: bool) -> int:
    """Codebook selection of exl3_gemm_gr (exl3_gemm.cu.lna:186-189)."""
    if mcg and mul1:
        raise RuntimeError("Specified both mcg and mul1")
    return CB_MCG if mcg else (CB_MUL1 if mul1 else CB_3INST)


def _stream(device: torch.device) -> int:
    return int(torch.cuda.current_stream(device).cuda_stream)


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else int(t.data_ptr())


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


# ------------------------------------------------------------------ shared scratch

class _ScratchPool:
    """One zeroed scratch buffer per (device, purpose), grown outside capture.

    The kernels' counters must be zero before the first launch and are left
    zero by every launch (recipe-lna/vllm_exl3_exl3.py.lna:1276-1296 is the
    same contract), so a buffer is zeroed exactly once, when it is created.
    A buffer that a larger one replaces is freed (after the device finished
    the work queued on it), unless a graph was captured while it was current:
    such a graph keeps launching on its address, so that buffer is kept alive
    until the process ends."""

    def __init__(self):
        self._bufs: dict[tuple[int, str], torch.Tensor] = {}
        self._captured: set[tuple[int, str]] = set()
        self._retired: list[torch.Tensor] = []
        self._lock = threading.Lock()

    def get(self, device: torch.device, purpose: str, nbytes: int) -> torch.Tensor:
        idx = device.index if device.index is not None else torch.cuda.current_device()
        key = (int(idx), purpose)
        with self._lock:
            buf = self._bufs.get(key)
            capturing = torch.cuda.is_current_stream_capturing()
            if buf is None or buf.numel() < nbytes:
                if capturing:
                    raise RuntimeError(
                        f"exl3 {purpose} scratch was not prewarmed for device {idx} "
                        f"(need {nbytes} bytes during graph capture)")
                if buf is not None:
                    if key in self._captured:
                        self._retired.append(buf)
                        self._captured.discard(key)
                    elif buf.is_cuda:
                        torch.cuda.synchronize(buf.device)
                    del self._bufs[key]
                    del buf
                buf = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=device)
                self._bufs[key] = buf
            if capturing:
                self._captured.add(key)
            return buf

    def current(self, device: torch.device, purpose: str) -> torch.Tensor | None:
        idx = device.index if device.index is not None else torch.cuda.current_device()
        return self._bufs.get((int(idx), purpose))

    def resident_bytes(self) -> int:
        return sum(int(b.numel()) for b in self._bufs.values()) + sum(int(b.numel()) for b in self._retired)


SCRATCH = _ScratchPool()

# ------------------------------------------------------------------ op registration

_LIB = torch.library.Library("exl3_amd", "DEF")
_LIB.define("dequant(Tensor trellis, Tensor? suh, Tensor? svh, int bits, int codebook, Tensor(a!) out) -> ()")
_LIB.define("gemm(Tensor a, Tensor b, Tensor(a!) c, Tensor suh, Tensor svh, int codebook, "
            "Tensor(b!) scratch) -> ()")
_LIB.define("moe_decode(Tensor x, Tensor(a!) out, Tensor gate_trellis, Tensor gate_suh, Tensor gate_svh, "
            "Tensor up_trellis, Tensor up_suh, Tensor up_svh, Tensor down_trellis, Tensor down_suh, "
            "Tensor down_svh, Tensor expert_ids, Tensor routing_weights, Tensor? expert_map, "
            "Tensor? expert_bits, int bits, int bits_mask, int codebook, float swiglu_limit, int hidden, "
            "int intermediate, Tensor(b!) scratch) -> ()")


def _dequant_impl(trellis, suh, svh, bits, codebook, out):
    L = _lib.load()
    k = trellis.shape[0] * 16
    n = trellis.shape[1] * 16
    _lib.check(L.exl3_dequant(_ptr(trellis), k, n, int(bits), int(codebook), _ptr(suh), _ptr(svh),
                              _ptr(out), _stream(trellis.device)))


_LIB.define("dequant_nk(Tensor trellis, Tensor? suh, Tensor? svh, int bits, int codebook, Tensor(a!) out) -> ()")


def _dequant_nk_impl(trellis, suh, svh, bits, codebook, out):
    L = _lib.load()
    k = trellis.shape[0] * 16
    n = trellis.shape[1] * 16
    _lib.check(L.exl3_dequant_nk(_ptr(trellis), k, n, int(bits), int(codebook), _ptr(suh), _ptr(svh),
                                 _ptr(out), _stream(trellis.device)))


_LIB.define("had_rows(Tensor x, Tensor(a!) y, Tensor? pre_scale, Tensor? post_scale, float scale) -> ()")


def _had_rows_impl(x, y, pre_scale, post_scale, scale):
    L = _lib.load()
    cols = x.shape[-1]
    _lib.check(L.exl3_had_rows(_ptr(x), OUT_KIND[x.dtype], _ptr(y), OUT_KIND[y.dtype], x.numel() // cols, cols,
                               _ptr(pre_scale), _ptr(post_scale), float(scale), _stream(x.device)))


def _gemm_impl(a, b, c, suh, svh, codebook, scratch):
    L = _lib.load()
    m, k = a.shape
    n = b.shape[1] * 16
    bits = b.shape[2] // 16
    _lib.check(L.exl3_gemm(_ptr(a), m, k, _ptr(b), n, bits, int(codebook), _ptr(suh), _ptr(svh),
                           _ptr(c), OUT_KIND[c.dtype], _ptr(scratch), scratch.numel(), _stream(a.device)))


def _route_args(ids, w, emap):
    return (_ptr(ids), IDS_KIND[ids.dtype], _ptr(w), OUT_KIND[w.dtype], _ptr(emap),
            0 if emap is None else emap.numel())


def _moe_impl(x, out, gt, gsu, gsv, ut, usu, usv, dt, dsu, dsv, ids, w, emap, expert_bits, bits, bits_mask,
              codebook, limit, hidden, intermediate, scratch):
    L = _lib.load()
    m = x.shape[0]
    _lib.check(L.exl3_moe_decode_routed(
        _ptr(x), X_KIND[x.dtype], _ptr(out), OUT_KIND[out.dtype], m, int(hidden), int(intermediate),
        gt.numel(), ids.shape[1],
        _ptr(gt), _ptr(gsu), _ptr(gsv), _ptr(ut), _ptr(usu), _ptr(usv), _ptr(dt), _ptr(dsu), _ptr(dsv),
        *_route_args(ids, w, emap), _ptr(expert_bits), int(bits), int(bits_mask), int(codebook), float(limit),
        _ptr(scratch), scratch.numel(), _stream(x.device)))


_LIB.define("moe_prefill(Tensor x, Tensor(a!) out, Tensor gate_trellis, Tensor gate_suh, Tensor gate_svh, "
            "Tensor up_trellis, Tensor up_suh, Tensor up_svh, Tensor down_trellis, Tensor down_suh, "
            "Tensor down_svh, Tensor expert_ids, Tensor routing_weights, Tensor? expert_map, "
            "Tensor? expert_bits, int bits, int bits_mask, int codebook, float swiglu_limit, int hidden, "
            "int intermediate, Tensor(b!) scratch) -> ()")


def _prefill_impl(x, out, gt, gsu, gsv, ut, usu, usv, dt, dsu, dsv, ids, w, emap, expert_bits, bits, bits_mask,
                  codebook, limit, hidden, intermediate, scratch):
    L = _lib.load()
    _lib.check(L.exl3_moe_prefill_routed(
        _ptr(x), X_KIND[x.dtype], _ptr(out), OUT_KIND[out.dtype], x.shape[0], int(hidden), int(intermediate),
        gt.numel(), ids.shape[1],
        _ptr(gt), _ptr(gsu), _ptr(gsv), _ptr(ut), _ptr(usu), _ptr(usv), _ptr(dt), _ptr(dsu), _ptr(dsv),
        *_route_args(ids, w, emap), _ptr(expert_bits), int(bits), int(bits_mask), int(codebook), float(limit),
        _ptr(scratch), scratch.numel(), _stream(x.device)))


_LIB.define("gemm_group(Tensor a, Tensor[] b, Tensor(a!)[] c, Tensor[] suh, Tensor[] svh, int codebook, "
            "Tensor(b!) scratch) -> ()")


def _host_array(ctype, values):
    return (ctype * len(values))(*values)


def _gemm_group_impl(a, b, c, suh, svh, codebook, scratch):
    import ctypes

    L = _lib.load()
    m, k = a.shape
    count = len(b)
    ns = _host_array(ctypes.c_int64, [int(t.shape[1]) * 16 for t in b])
    bits = _host_array(ctypes.c_int32, [int(t.shape[2]) // 16 for t in b])
    ptrs = lambda ts: _host_array(ctypes.c_void_p, [int(t.data_ptr()) for t in ts])
    _lib.check(L.exl3_gemm_group(_ptr(a), m, k, count, ptrs(b), ptrs(suh), ptrs(svh), ns, bits, int(codebook),
                                 ptrs(c), OUT_KIND[c[0].dtype], _ptr(scratch), scratch.numel(), _stream(a.device)))


_LIB.impl("moe_prefill", _prefill_impl, "CUDA")
_LIB.impl("gemm_group", _gemm_group_impl, "CUDA")
_LIB.impl("dequant", _dequant_impl, "CUDA")
_LIB.impl("dequant_nk", _dequant_nk_impl, "CUDA")
_LIB.impl("had_rows", _had_rows_impl, "CUDA")
_LIB.impl("gemm", _gemm_impl, "CUDA")
_LIB.impl("moe_decode", _moe_impl, "CUDA")

# ------------------------------------------------------------------ dequant


def _check_trellis(trellis: torch.Tensor, bits: int | None = None) -> int:
    _check(trellis.dim() == 3 and trellis.dtype == torch.int16,
           "trellis must be int16 [rows/16, cols/16, 16*K]")
    _check(trellis.is_contiguous(), "trellis must be contiguous")
    _check(trellis.shape[2] % 16 == 0 and 1 <= trellis.shape[2] // 16 <= 8,
           "trellis last dimension must be 16*K with 1 <= K <= 8")
    k = trellis.shape[2] // 16
    if bits is not None:
        _check(k == bits, "trellis last dimension must be 16*K")
    _check(trellis.shape[0] > 0 and trellis.shape[1] > 0, "trellis dimensions must be positive")
    return k


def reconstruct_weight(trellis: torch.Tensor, codebook: int = CB_MCG) -> torch.Tensor:
    """Raw codebook matrix Wq fp16 [in, out] (no rotations)."""
    bits = _check_trellis(trellis)
    out = torch.empty((trellis.shape[0] * 16, trellis.shape[1] * 16), dtype=torch.float16,
                      device=trellis.device)
    torch.ops.exl3_amd.dequant(trellis, None, None, bits, codebook, out)
    return out


def reconstruct_weight_nk(trellis: torch.Tensor, codebook: int = CB_MCG) -> torch.Tensor:
    """Raw codebook matrix stored transposed: Wq^T fp16 [out, in] (bitwise reconstruct_weight(...).t())."""
    bits = _check_trellis(trellis)
    out = torch.empty((trellis.shape[1] * 16, trellis.shape[0] * 16), dtype=torch.float16,
                      device=trellis.device)
    torch.ops.exl3_amd.dequant_nk(trellis, None, None, bits, codebook, out)
    return out


def dequant_trellis_nk(trellis: torch.Tensor, suh: torch.Tensor, svh: torch.Tensor, K: int,
                       mcg: bool = True, mul1: bool = False) -> torch.Tensor:
    """dequant_trellis stored transposed: W^T fp16 [out, in], bitwise dequant_trellis(...).t()."""
    _check_trellis(trellis, K)
    _check(suh.dtype == torch.float16 and svh.dtype == torch.float16, "suh and svh must be float16")
    _check(suh.numel() >= trellis.shape[0] * 16 and svh.numel() >= trellis.shape[1] * 16,
           "suh/svh are too short")
    _check(trellis.shape[0] % 8 == 0 and trellis.shape[1] % 8 == 0,
           "trellis dimensions must reconstruct whole 128-element Hadamard blocks")
    out = torch.empty((trellis.shape[1] * 16, trellis.shape[0] * 16), dtype=torch.float16,
                      device=trellis.device)
    torch.ops.exl3_amd.dequant_nk(trellis, suh.contiguous(), svh.contiguous(), K, codebook_id(mcg, mul1), out)
    return out


def reconstruct(w: torch.Tensor, trellis: torch.Tensor, K: int, mcg: bool, mul1: bool) -> None:
    """exllamav3_ext.reconstruct(w, trellis, K, mcg, mul1): fills w with Wq."""
    _check_trellis(trellis, K)
    _check(w.dtype == torch.float16 and w.is_contiguous() and
           tuple(w.shape) == (trellis.shape[0] * 16, trellis.shape[1] * 16), "w must be fp16 [in, out]")
    torch.ops.exl3_amd.dequant(trellis, None, None, K, codebook_id(mcg, mul1), w)


def dequant_trellis(trellis: torch.Tensor, suh: torch.Tensor, svh: torch.Tensor, K: int,
                    mcg: bool = True, mul1: bool = False) -> torch.Tensor:
    """vllm_exl3_c.dequant_trellis: W = diag(suh) H Wq H diag(svh)/128, fp16 [in, out]
    (bindings.cpp:118-133; bit widths 1..8 instead of {2,3,4,8})."""
    _check_trellis(trellis, K)
    _check(suh.dtype == torch.float16 and svh.dtype == torch.float16, "suh and svh must be float16")
    _check(suh.numel() >= trellis.shape[0] * 16 and svh.numel() >= trellis.shape[1] * 16,
           "suh/svh are too short")
    _check(trellis.shape[0] % 8 == 0 and trellis.shape[1] % 8 == 0,
           "trellis dimensions must reconstruct whole 128-element Hadamard blocks")
    out = torch.empty((trellis.shape[0] * 16, trellis.shape[1] * 16), dtype=torch.float16,
                      device=trellis.device)
    torch.ops.exl3_amd.dequant(trellis, suh.contiguous(), svh.contiguous(), K, codebook_id(mcg, mul1), out)
    return out

# ------------------------------------------------------------------ dense GEMV / GEMM


def had_r_128(x: torch.Tensor, y: torch.Tensor, pre_scale: torch.Tensor | None, post_scale: torch.Tensor | None,
              scale: float = 1.0) -> None:
    """exllamav3_ext.had_r_128(input, output, pre_scale, post_scale, scale): y = H128 (x * pre) / sqrt(128)
    * scale * post per 128-block of each row (recipe-lna/exllamav3/exl3.py.lna:190, 214).  x, y fp16 / bf16 /
    fp32 with the same shape, contiguous, last dimension a multiple of 128; y may be x."""
    _check(x.shape == y.shape and x.is_contiguous() and y.is_contiguous(), "x and y must be contiguous, same shape")
    _check(x.dtype in OUT_KIND and y.dtype in OUT_KIND, "x and y must be fp16, bf16 or fp32")
    _check(x.dim() >= 1 and x.shape[-1] % 128 == 0 and x.numel() > 0, "last dimension must be a multiple of 128")
    for t in (pre_scale, post_scale):
        _check(t is None or (t.dtype == torch.float16 and t.is_contiguous() and t.numel() >= x.shape[-1]),
               "scales must be contiguous fp16 covering the last dimension")
    torch.ops.exl3_amd.had_rows(x, y, pre_scale, post_scale, float(scale))


def gemm_scratch(device: torch.device, m: int, k: int, n: int) -> torch.Tensor:
    nbytes = _lib.check(_lib.load().exl3_gemm_scratch_bytes(m, k, n))
    return SCRATCH.get(device, "gemm", nbytes)


def prepare_gemm(device: torch.device, max_rows: int, k: int, n: int) -> None:
    """Reserve the shared dense scratch before any graph capture (the role of
    LNA_EXL3_PREWARM_ROWS, recipe-lna/vllm_exl3_exl3.py.lna:2718-2742)."""
    for m in range(1, max_rows + 1):
        gemm_scratch(device, m, k, n)


def gemm_into(x: torch.Tensor, trellis: torch.Tensor, suh: torch.Tensor, svh: torch.Tensor,
              c: torch.Tensor, codebook: int = CB_MCG) -> torch.Tensor:
    """c = had_out(had_in(x*suh) @ Wq) * svh for x fp16 [m, k]; c fp16/bf16/fp32 [m, n]."""
    bits = _check_trellis(trellis)
    _check(x.dim() == 2 and x.dtype == torch.float16 and x.is_contiguous(), "x must be contiguous fp16 [m, k]")
    m, k = x.shape
    n = trellis.shape[1] * 16
    _check(k == trellis.shape[0] * 16, "x feature dimension does not match trellis")
    _check(k % 128 == 0 and n % 128 == 0, "in and out features must be multiples of 128")
    _check(c.dtype in OUT_KIND and c.is_contiguous() and tuple(c.shape) == (m, n), "c must be [m, n] contiguous")
    _check(suh.dtype == torch.float16 and suh.numel() == k and suh.is_contiguous(), "suh must be fp16 [k]")
    _check(svh.dtype == torch.float16 and svh.numel() == n and svh.is_contiguous(), "svh must be fp16 [n]")
    for t in (trellis, suh, svh, c):
        _check(t.device == x.device, "all tensors must be on the same device")
    scratch = gemm_scratch(x.device, m, k, n)
    torch.ops.exl3_amd.gemm(x, trellis, c, suh, svh, codebook, scratch)
    return c


def gemm(x: torch.Tensor, trellis: torch.Tensor, suh: torch.Tensor, svh: torch.Tensor,
         codebook: int = CB_MCG, out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    c = torch.empty((x.shape[0], trellis.shape[1] * 16), dtype=out_dtype, device=x.device)
    return gemm_into(x, trellis, suh, svh, c, codebook)


MAX_GROUP = 8


def gemm_group_scratch(device: torch.device, m: int, k: int, ns) -> torch.Tensor:
    import ctypes

    arr = (ctypes.c_int64 * len(ns))(*[int(n) for n in ns])
    nbytes = _lib.check(_lib.load().exl3_gemm_group_scratch_bytes(m, k, len(ns), arr))
    return SCRATCH.get(device, "gemm_group", nbytes)


def gemm_group(x: torch.Tensor, members, codebook: int = CB_MCG,
               out_dtype: torch.dtype = torch.float32, outs=None) -> list[torch.Tensor]:
    """One fused call for several EXL3 matrices that read the same input:
    members = [(trellis, suh, svh), ...] (1..8, same in_features, any out
    features and bit widths); returns [had_out(had_in(x*suh_j) @ Wq_j) * svh_j].
    The role of exllamav3_ext.exl3_mgemm with a broadcast A
    (recipe-lna/vllm_exl3_exl3.py.lna:546-613)."""
    _check(x.dim() == 2 and x.dtype == torch.float16 and x.is_contiguous(), "x must be contiguous fp16 [m, k]")
    _check(1 <= len(members) <= MAX_GROUP, "a group has 1..8 matrices")
    m, k = x.shape
    ts, us, vs, ns = [], [], [], []
    for trellis, suh, svh in members:
        _check_trellis(trellis)
        n = trellis.shape[1] * 16
        _check(trellis.shape[0] * 16 == k, "every member must read the input's feature dimension")
        _check(n % 128 == 0 and k % 128 == 0, "in and out features must be multiples of 128")
        _check(suh.dtype == torch.float16 and suh.numel() == k and suh.is_contiguous(), "suh must be fp16 [k]")
        _check(svh.dtype == torch.float16 and svh.numel() == n and svh.is_contiguous(), "svh must be fp16 [n]")
        for t in (trellis, suh, svh):
            _check(t.device == x.device, "all tensors must be on the same device")
        ts.append(trellis); us.append(suh); vs.append(svh); ns.append(n)
    if outs is None:
        outs = [torch.empty((m, n), dtype=out_dtype, device=x.device) for n in ns]
    _check(len(outs) == len(ns), "one output per member")
    for c, n in zip(outs, ns):
        _check(c.dtype == outs[0].dtype and c.dtype in OUT_KIND and c.is_contiguous() and tuple(c.shape) == (m, n),
               "outputs must be contiguous [m, n_j] of one dtype")
    scratch = gemm_group_scratch(x.device, m, k, ns)
    torch.ops.exl3_amd.gemm_group(x, ts, outs, us, vs, codebook, scratch)
    return outs


def exl3_gemm(A: torch.Tensor, B: torch.Tensor, C: torch.Tensor, suh: torch.Tensor | None,
              A_had: torch.Tensor | None, svh: torch.Tensor | None, force_shape_idx: int = -1,
              mcg: bool = False, mul1: bool = False, force_num_sms: int = 0) -> int:
    """exllamav3_ext.exl3_gemm(A, B, C, suh, A_had, svh, force_shape_idx, mcg, mul1,
    force_num_sms) -> shape tag (exl3_gemm.cu.lna:336-364).  A is [..., k] fp16,
    C [..., n] fp16 or fp32.  A_had, force_shape_idx and force_num_sms only steer
    the reference's tile autotuner and are accepted for drop-in compatibility."""
    del A_had, force_shape_idx, force_num_sms
    _check(suh is not None and svh is not None, "suh and svh are required")
    _check(A.dtype == torch.float16, "A must be float16")
    _check(C.dtype in (torch.float16, torch.float32), "C must be float16 or float32")
    a2 = A.reshape(-1, A.shape[-1])
    c2 = C.view(-1, C.shape[-1])
    gemm_into(a2, B, suh, svh, c2, codebook_id(mcg, mul1))
    return 0


def exl3_gemv(x: torch.Tensor, trellis: torch.Tensor, suh: torch.Tensor, svh: torch.Tensor,
              K: int, mcg: bool = True, mmode: int = 1) -> torch.Tensor:
    """vllm_exl3_c.exl3_gemv(x, trellis, suh, svh, K, mcg, mmode), bindings.cpp:135-148:
    output in x's dtype; m is not limited to 8 here."""
    _check(x.dim() >= 2, "x must have shape [..., in_features]")
    _check(mmode in (0, 1), "mmode must be 0 or 1")
    _check_trellis(trellis, K)
    _check(x.shape[-1] == trellis.shape[0] * 16, "x feature dimension does not match trellis")
    x2 = x.contiguous().view(-1, x.shape[-1]).to(torch.float16)
    out = gemm(x2, trellis, suh, svh, CB_MCG if mcg else CB_MUL1, torch.float32)
    return out.to(x.dtype).view(*x.shape[:-1], -1)

# ------------------------------------------------------------------ routed MoE decode

MOE_TABLE_KEYS = ("gate_trellis", "gate_suh", "gate_svh", "up_trellis", "up_suh", "up_svh",
                  "down_trellis", "down_suh", "down_svh")


def moe_max_rows() -> int:
    return int(_lib.load().exl3_moe_max_rows())


ERR_WIDTH = 1      # an expert width outside bits_mask was routed (its contribution was zero)
ERR_WAIT = 2       # a bounded wait of the ticket schedule gave up


def moe_error(scratch: torch.Tensor, clear: bool = True) -> int:
    """The error word of a decode or prefill scratch (ERR_* bits; 0 = none).
    Synchronises with the device; call it outside captured regions.  A decode
    scratch keeps bits until cleared; a prefill scratch reports its last call."""
    off = int(_lib.load().exl3_moe_error_offset())
    word = scratch[off:off + 4]
    value = int(word.view(torch.int32).item())
    if clear and value:
        word.zero_()
    return value


def moe_scratch_errors(device: torch.device, clear: bool = True) -> dict[str, int]:
    """Error words of this device's shared decode and prefill scratch buffers."""
    out = {}
    for purpose in ("moe", "moe_prefill"):
        buf = SCRATCH.current(device, purpose)
        if buf is not None:
            out[purpose] = moe_error(buf, clear)
    return out


_WIDTHS_CHECKED: dict[tuple, bool] = {}


def check_expert_bits(expert_bits: torch.Tensor, bits_mask: int) -> None:
    """Every width in the per-expert table must be in bits_mask, the set the
    kernel instance is chosen for (the role of the reference's TORCH_CHECKs on
    K, lna_moe_ticket.cu:516-553).  Read from the device once per table
    version; inside a graph capture an unchecked table is left to the
    kernels' error word."""
    key = (expert_bits.device.index, int(expert_bits.data_ptr()), int(expert_bits.numel()),
           int(expert_bits._version), int(bits_mask))
    if key in _WIDTHS_CHECKED:
        return
    if torch.cuda.is_current_stream_capturing():
        return
    widths = {int(b) for b in expert_bits.cpu().tolist()}
    bad = sorted(b for b in widths if not (1 <= b <= 8 and (int(bits_mask) >> b) & 1))
    _check(not bad, f"expert_bits holds widths {bad} outside bits_mask 0x{int(bits_mask):x}")
    if len(_WIDTHS_CHECKED) > 4096:
        _WIDTHS_CHECKED.clear()
    _WIDTHS_CHECKED[key] = True


def moe_scratch_bytes(hidden: int, intermediate: int, topk: int, rows: int = 16) -> int:
    """Scratch bytes for calls of up to `rows` rows (16 rows and fewer share one size)."""
    lib = _lib.load()
    if rows <= 16:
        return int(_lib.check(lib.exl3_moe_scratch_bytes(hidden, intermediate, topk)))
    return int(_lib.check(lib.exl3_moe_scratch_bytes_rows(hidden, intermediate, topk, rows)))


def moe_scratch(device: torch.device, hidden: int, intermediate: int, topk: int, rows: int = 16) -> torch.Tensor:
    """The shared per-device MoE scratch (zeroed once, self-resetting afterwards).
    Up to 16 rows share one size; a call of more rows sizes it once for
    moe_max_rows(), so batches growing past 16 rows allocate one more buffer,
    not one per row count."""
    if rows > 16:
        rows = moe_max_rows()
    return SCRATCH.get(device, "moe", moe_scratch_bytes(hidden, intermediate, topk, rows))


def moe_info() -> list[int]:
    """[cus, waves per launch, threads per wave, max rows, max pairs, step k,
    cols, control-region bytes, LDS bytes per workgroup]."""
    import ctypes

    buf = (ctypes.c_int64 * 9)()
    n = _lib.check(_lib.load().exl3_moe_info(buf, 9))
    return [int(buf[i]) for i in range(n)]


def bits_mask_of(bits) -> int:
    return sum(1 << int(b) for b in set(int(b) for b in bits))


def _check_route(expert_ids, routing_weights, rows: int, device, expert_map, what: str) -> None:
    _check(expert_ids.is_cuda and expert_ids.device == device and expert_ids.dtype in IDS_KIND and
           expert_ids.is_contiguous() and expert_ids.dim() == 2 and expert_ids.shape[0] == rows,
           f"expert_ids must be contiguous int32/int64 [{what}, topk] on the input device")
    _check(routing_weights.is_cuda and routing_weights.device == device and routing_weights.dtype in OUT_KIND and
           routing_weights.is_contiguous() and routing_weights.shape == expert_ids.shape,
           f"routing_weights must be contiguous fp16/bf16/fp32 [{what}, topk] on the input device")
    if expert_map is not None:
        _check(expert_map.is_cuda and expert_map.device == device and expert_map.dtype == torch.int64 and
               expert_map.dim() == 1 and expert_map.is_contiguous() and expert_map.numel() >= 1,
               "expert_map must be a contiguous int64 [global experts] tensor on the input device")


def moe_decode(x: torch.Tensor, out: torch.Tensor, tables, expert_ids: torch.Tensor,
               routing_weights: torch.Tensor, *, intermediate: int, bits: int | None = None,
               expert_bits: torch.Tensor | None = None, bits_mask: int | None = None,
               codebook: int = CB_MCG, swiglu_limit: float = 10.0,
               scratch: torch.Tensor | None = None, expert_map: torch.Tensor | None = None) -> torch.Tensor:
    """Routed-expert decode of x [m, hidden] into out [m, hidden].

    tables: the nine int64 device pointer tables (dict keyed by MOE_TABLE_KEYS,
    or a sequence in that order).  Either `bits` (every expert) or
    `expert_bits` (int8 [E] device tensor) with `bits_mask` (set of widths).
    expert_ids int32/int64 and routing_weights fp16/bf16/fp32, [m, topk], as
    the router produced them; with `expert_map` (int64 [global experts],
    negative for other ranks' experts) the ids are global and are mapped to
    local ones inside the kernels, as map_topk_to_local does on the host."""
    if isinstance(tables, dict):
        tabs = [tables[k] for k in MOE_TABLE_KEYS]
    else:
        tabs = list(tables)
    _check(len(tabs) == 9, "nine pointer tables are required")
    _check(x.is_cuda and x.dtype in X_KIND, "input must be HIP fp16 or bf16")
    _check(x.dim() == 2 and x.is_contiguous(), "input must be contiguous [m, hidden]")
    m, hidden = x.shape
    _check(1 <= m <= moe_max_rows(), "row count out of range (1 <= m <= moe_max_rows())")
    _check(out.is_cuda and out.device == x.device and tuple(out.shape) == tuple(x.shape) and out.is_contiguous(),
           "output must match x shape/device and be contiguous")
    _check(out.dtype in OUT_KIND, "output must be fp16/bf16/fp32")
    _check_route(expert_ids, routing_weights, m, x.device, expert_map, "m")
    n_experts = tabs[0].numel()
    for t in tabs:
        _check(t.is_cuda and t.device == x.device and t.dtype == torch.int64 and t.is_contiguous() and
               t.numel() == n_experts, "pointer tables must be contiguous int64 [experts] on the input device")
    if expert_bits is not None:
        _check(expert_bits.is_cuda and expert_bits.dtype == torch.int8 and expert_bits.numel() == n_experts,
               "expert_bits must be int8 [experts] on the device")
        _check(bits_mask is not None and bits_mask > 0, "bits_mask is required with expert_bits")
        check_expert_bits(expert_bits, bits_mask)
        b, mask = 0, int(bits_mask)
    else:
        _check(bits is not None and 1 <= int(bits) <= 8, "bits must be in 1..8")
        b, mask = int(bits), 0
    if scratch is None:
        scratch = moe_scratch(x.device, hidden, intermediate, expert_ids.shape[1], rows=m)
    torch.ops.exl3_amd.moe_decode(x, out, *tabs, expert_ids, routing_weights, expert_map, expert_bits, b, mask,
                                  int(codebook), float(swiglu_limit), int(hidden), int(intermediate), scratch)
    return out


# vllm_exl3_c names (recipe-lna/lna2/bindings.cpp:212-219, lna_moe_ticket.cu:481-581).
# The reference kernel is fixed at hidden=4096, intermediate=256, top-6 and one
# width per launch; here intermediate is a keyword (default: that geometry),
# top-k comes from the ids' shape and `bits` may be a per-expert int8 table.

def lna2_moe_decode(x, out, gate_trellis, gate_suh, gate_svh, up_trellis, up_suh, up_svh,
                    down_trellis, down_suh, down_svh, expert_ids, routing_weights, bits,
                    swiglu_limit, scratch, *, intermediate: int = 256, bits_mask: int | None = None,
                    codebook: int = CB_MCG):
    tabs = (gate_trellis, gate_suh, gate_svh, up_trellis, up_suh, up_svh, down_trellis, down_suh, down_svh)
    limit = float(swiglu_limit)
    _check(limit > 0.0 and limit == limit and limit != float("inf"), "requires a finite positive SwiGLU limit")
    _check(scratch.is_cuda and scratch.dtype == torch.uint8 and scratch.is_contiguous() and
           scratch.numel() >= moe_scratch_bytes(x.shape[1], intermediate, expert_ids.shape[1], rows=x.shape[0]),
           "scratch too small")
    if isinstance(bits, torch.Tensor):
        mask = bits_mask if bits_mask is not None else bits_mask_of(bits.cpu().tolist())
        return moe_decode(x, out, tabs, expert_ids, routing_weights, intermediate=intermediate,
                          expert_bits=bits, bits_mask=mask, codebook=codebook, swiglu_limit=limit,
                          scratch=scratch)
    return moe_decode(x, out, tabs, expert_ids, routing_weights, intermediate=intermediate, bits=int(bits),
                      codebook=codebook, swiglu_limit=limit, scratch=scratch)


def lna2_moe_scratch_bytes(hidden: int = 4096, intermediate: int = 256, topk: int = 6) -> int:
    """Enough for every row count lna2_moe_max_rows() allows, as the
    reference's size is for its build-time row capacity."""
    return moe_scratch_bytes(hidden, intermediate, topk, rows=moe_max_rows())


def lna2_moe_max_rows() -> int:
    return moe_max_rows()


def lna2_moe_prepare(bits: int) -> None:
    _check(1 <= int(bits) <= 8, "bits must be in 1..8")
    moe_info()


def lna2_moe_info(bits: int) -> list[int]:
    """The reference's 14 positions (lna_moe_ticket.cu:494-505): [sms, resident,
    width, teams, threads, cfg, pfd, rows_cap, smem, ctrl_bytes, scratch_bytes,
    max_m, max_pairs, streams].  Here a "team" is one wave, cfg is 0, pfd is the
    one step of tile prefetch, scratch_bytes is for the reference geometry and
    streams is 1 (one launch at a time per scratch buffer)."""
    lna2_moe_prepare(bits)
    cus, waves, width, max_m, max_pairs, _, _, ctrl, lds = moe_info()
    return [cus, waves, width, waves, width, 0, 1, max_m, lds, ctrl, lna2_moe_scratch_bytes(), max_m,
            max_pairs, 1]


# ------------------------------------------------------------------ routed MoE, many tokens (prefill)


def moe_prefill_scratch_bytes(tokens: int, hidden: int, intermediate: int, topk: int, n_experts: int) -> int:
    return int(_lib.check(_lib.load().exl3_moe_prefill_scratch_bytes(tokens, hidden, intermediate, topk,
                                                                      n_experts)))


def moe_prefill_scratch(device: torch.device, tokens: int, hidden: int, intermediate: int, topk: int,
                        n_experts: int) -> torch.Tensor:
    """Shared per-device prefill scratch (grown outside capture; never needs zeroing)."""
    return SCRATCH.get(device, "moe_prefill", moe_prefill_scratch_bytes(tokens, hidden, intermediate, topk,
                                                                        n_experts))


def moe_prefill(x: torch.Tensor, out: torch.Tensor, tables, expert_ids: torch.Tensor,
                routing_weights: torch.Tensor, *, intermediate: int, bits: int | None = None,
                expert_bits: torch.Tensor | None = None, bits_mask: int | None = None,
                codebook: int = CB_MCG, swiglu_limit: float = 10.0,
                scratch: torch.Tensor | None = None, expert_map: torch.Tensor | None = None) -> torch.Tensor:
    """Routed-expert layer over many tokens (grouped GEMMs): x [tokens, hidden]
    -> out [tokens, hidden]; arguments as moe_decode, any number of tokens with
    tokens * topk <= 65536."""
    tabs = [tables[k] for k in MOE_TABLE_KEYS] if isinstance(tables, dict) else list(tables)
    _check(len(tabs) == 9, "nine pointer tables are required")
    _check(x.is_cuda and x.dtype in X_KIND and x.dim() == 2 and x.is_contiguous(),
           "input must be contiguous HIP fp16/bf16 [tokens, hidden]")
    T, hidden = x.shape
    _check(out.is_cuda and out.device == x.device and tuple(out.shape) == (T, hidden) and out.is_contiguous()
           and out.dtype in OUT_KIND, "output must be contiguous fp16/bf16/fp32 [tokens, hidden] on x's device")
    _check_route(expert_ids, routing_weights, T, x.device, expert_map, "tokens")
    n_experts = tabs[0].numel()
    for t in tabs:
        _check(t.is_cuda and t.device == x.device and t.dtype == torch.int64 and t.is_contiguous() and
               t.numel() == n_experts, "pointer tables must be contiguous int64 [experts] on the input device")
    if expert_bits is not None:
        _check(expert_bits.is_cuda and expert_bits.dtype == torch.int8 and expert_bits.numel() == n_experts,
               "expert_bits must be int8 [experts] on the device")
        _check(bits_mask is not None and bits_mask > 0, "bits_mask is required with expert_bits")
        check_expert_bits(expert_bits, bits_mask)
        b, mask = 0, int(bits_mask)
    else:
        _check(bits is not None and 1 <= int(bits) <= 8, "bits must be in 1..8")
        b, mask = int(bits), 0
    if scratch is None:
        scratch = moe_prefill_scratch(x.device, T, hidden, intermediate, expert_ids.shape[1], n_experts)
    torch.ops.exl3_amd.moe_prefill(x, out, *tabs, expert_ids, routing_weights, expert_map, expert_bits, b, mask,
                                   int(codebook), float(swiglu_limit), int(hidden), int(intermediate), scratch)
    return out
