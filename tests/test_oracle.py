"""Pins the CPU oracle (no GPU).  Each check is chosen so that a plausible
mistake (a dropped term, a wrong sign, bit or index order, a transposed
operand) fails it, and none of them retypes the oracle's own formula:

* windows: the bit-serial C spec vs the funnel-shift restatement vs the
  reference's own host helper (orders/F1-ref/exl3_dequant.cuh:109-127, built
  from the reference tree into oracle/_ref), over the primitive-gate streams of
  recipe-lna/lna2/primitive_gate.cu:107-121 at every element and bit width;
* codebooks: against numpy's IEEE binary16 arithmetic, against the reference's
  truncating helper (which must differ by exactly one ulp toward zero where it
  differs), and against the format's invariants;
* tile permutation: against the published m16n8k16 B-fragment layout (PTX ISA,
  "mma.m16n8k16 .f16 B fragment") with the reference's lane ownership
  (lane L decodes t = 8L..8L+7 into frag0/frag1, lna_gemv_core.cuh:186-195);
* Hadamard: against scipy's Sylvester matrix and the reference's own loop;
* dense linear / MoE: against independent dense-matrix formulations.
"""

from __future__ import annotations

import numpy as np
import pytest
import scipy.linalg

from oracle import oracle as O

BITS = list(range(1, 9))


def primitive_streams(bits: int) -> np.ndarray:
    """The four streams of primitive_gate.cu:107-121 as uint16 tiles [4, 16*bits]."""
    words = 8 * bits
    out = np.zeros((4, words), np.uint32)
    for i in range(words):
        out[0, i] = 0
        out[1, i] = 0xFFFFFFFF
        out[2, i] = 1 << ((7 * i + 3) & 31)
        x = (0x9E3779B9 ^ i) & 0xFFFFFFFF
        x ^= (x << 13) & 0xFFFFFFFF
        x ^= x >> 17
        x ^= (x << 5) & 0xFFFFFFFF
        out[3, i] = x
    return out.view(np.uint16).reshape(4, 16 * bits)


@pytest.mark.parametrize("bits", BITS)
def test_windows_all_restatements_agree(bits):
    rng = np.random.default_rng(100 + bits)
    tiles = np.concatenate([primitive_streams(bits),
                            rng.integers(0, 1 << 16, (4, 16 * bits), dtype=np.uint16)])
    vec = O.windows_np(tiles.view(np.int16), bits)
    ref = O.ref_lib()
    for i, tile in enumerate(tiles):
        for t in range(256):
            w = O.window(tile, bits, t)
            assert w == vec[i, t], (bits, i, t)
            if ref is not None:
                start = (t + 257) * bits - 16
                assert w == ref.ref_read_window(tile, 16 * bits, start), (bits, i, t)


def test_windows_trellis_recurrence():
    """Tail-biting trellis: w_{t+1} = ((w_t << K) | next K bits) & 0xFFFF."""
    rng = np.random.default_rng(7)
    for bits in BITS:
        tile = rng.integers(0, 1 << 16, 16 * bits, dtype=np.uint16)
        w = O.windows_np(tile.view(np.int16)[None], bits)[0].astype(np.int64)
        stream = np.unpackbits(tile.view(np.uint32).byteswap().view(np.uint8))  # MSB first per word
        for t in range(256):
            nxt = (t + 1) % 256
            e = ((nxt + 1) * bits) % (256 * bits)
            code = 0
            for b in range(bits):
                code = (code << 1) | int(stream[(e - bits + b) % (256 * bits)])
            assert w[nxt] == (((w[t] << bits) | code) & 0xFFFF), (bits, t)


def _mcg_parts(cb):
    w = np.arange(65536, dtype=np.uint64)
    x = (w * 89226354 + 64248484) if cb == O.CB_3INST else (w * 0xCBAC1FED)
    x = ((x & 0xFFFFFFFF) & 0x8FFF8FFF) ^ 0x3B603B60
    lo = (x & 0xFFFF).astype(np.uint16).view(np.float16)
    hi = (x >> 16).astype(np.uint16).view(np.float16)
    return lo, hi


@pytest.mark.parametrize("cb", [O.CB_MCG, O.CB_3INST])
def test_codebook_mcg_3inst_vs_numpy_rne(cb):
    lo, hi = _mcg_parts(cb)
    expect = (lo.astype(np.float32) + hi.astype(np.float32)).astype(np.float16).view(np.uint16)
    assert np.array_equal(O.codebook_lut(cb), expect)
    # invariants of the masked halves: exponent field 12..15 -> |addend| in [0.125, 2)
    for part in (lo, hi):
        a = np.abs(part.astype(np.float32))
        assert a.min() >= 0.125 and a.max() < 2.0
    h = O.codebook_lut(cb).view(np.float16).astype(np.float32)
    assert np.isfinite(h).all()
    nz = h[h != 0]
    assert np.abs(nz).min() >= 2.0 ** -14      # never subnormal


def test_codebook_mul1_vs_numpy():
    w = np.arange(65536, dtype=np.uint64)
    x = (w * 0x83DCD12D) & 0xFFFFFFFF
    s = 0x6400 + (x & 0xFF) + ((x >> 8) & 0xFF) + ((x >> 16) & 0xFF) + ((x >> 24) & 0xFF)
    sh = s.astype(np.uint16).view(np.float16).astype(np.float64)
    a = np.array([0x1EEE], np.uint16).view(np.float16).astype(np.float64)[0]
    c = np.array([0xC931], np.uint16).view(np.float16).astype(np.float64)[0]
    expect = (sh * a + c).astype(np.float16).view(np.uint16)   # exact in f64, one RNE rounding
    assert np.array_equal(O.codebook_lut(O.CB_MUL1), expect)


@pytest.mark.parametrize("cb", [O.CB_MCG, O.CB_3INST])
def test_codebook_addend_sum_mcg_3inst_vs_numpy(cb):
    """The MCG / 3INST addend sum is the exact sum of the two masked binary16
    halves (the GPU kernels add them in the matrix core); rounded, it is the
    codebook, and the rounding changes a large share of the values (so weights
    with and without it differ measurably)."""
    lo, hi = _mcg_parts(cb)
    s = O.codebook_addend_sum_lut(cb)
    assert np.array_equal(s, lo.astype(np.float64) + hi.astype(np.float64))
    assert np.array_equal(s.astype(np.float16).view(np.uint16), O.codebook_lut(cb))
    assert np.mean(s != s.astype(np.float16).astype(np.float64)) > 0.3


def test_codebook_addend_sum_mul1_is_its_value():
    """MUL1 is one single-rounded half FMA: its one addend is the codebook
    value itself (the kernels hand it to the matrix core with a zero)."""
    s = O.codebook_addend_sum_lut(O.CB_MUL1)
    assert np.array_equal(s, O.codebook_lut(O.CB_MUL1).view(np.float16).astype(np.float64))


@pytest.mark.parametrize("bits,cb", [(2, O.CB_MCG), (3, O.CB_MCG), (6, O.CB_3INST), (4, O.CB_MUL1)])
def test_reconstruct_exact_rounds_to_reconstruct(bits, cb):
    """Every element of the exact-addend reconstruct rounds to the binary16
    reconstruct: the two read the same window for every element."""
    rng = np.random.default_rng(bits)
    tr = rng.integers(-32768, 32768, size=(8, 6, 16 * bits), dtype=np.int64).astype(np.int16)
    e = O.reconstruct_exact(tr, bits, cb)
    assert e.dtype == np.float64 and e.shape == (128, 96)
    assert np.array_equal(e.astype(np.float16).view(np.uint16), O.reconstruct_fast(tr, bits, cb).view(np.uint16))


@pytest.mark.parametrize("cb", [O.CB_MCG, O.CB_3INST, O.CB_MUL1])
def test_codebook_vs_reference_truncating_helper(cb):
    """The reference host helper truncates (exl3_dequant.cuh:40-53); the canon
    rounds.  They may differ only by one ulp, always with the RNE value closer."""
    ref = O.ref_lib()
    if ref is None:
        pytest.skip("reference helper library oracle/_ref not built")
    lut = O.codebook_lut(cb)
    got = np.array([ref.ref_decode_codebook_bits(w, cb) for w in range(65536)], np.uint16)
    diff = got != lut
    assert np.all(np.abs(got[diff].astype(np.int32) - lut[diff].astype(np.int32)) == 1)
    # truncation moves toward zero: |trunc| < |rne| where they differ
    assert np.all(np.abs(got[diff].view(np.float16).astype(np.float32))
                  < np.abs(lut[diff].view(np.float16).astype(np.float32)))
    if cb == O.CB_MCG:
        lo, hi = _mcg_parts(cb)
        exact = lo.astype(np.float64) + hi.astype(np.float64)
        err_rne = np.abs(lut.view(np.float16).astype(np.float64) - exact)
        err_tr = np.abs(got.view(np.float16).astype(np.float64) - exact)
        assert np.all(err_rne <= err_tr)
        assert diff.sum() == 16550   # recorded: MCG codes where truncation != RNE


def test_half_rounding_vs_numpy():
    rng = np.random.default_rng(3)
    vals = np.concatenate([
        rng.standard_normal(20000) * 10.0 ** rng.integers(-9, 6, 20000),
        np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26, 1e-8, -1e-8]),
    ]).astype(np.float32)
    L = O.lib()
    got = np.array([L.ora_double_to_half(float(v)) for v in vals], np.uint16)
    assert np.array_equal(got, vals.astype(np.float16).view(np.uint16))


def test_tile_permutation_matches_mma_fragment_layout():
    """W[k][n] must be the value a lane decodes at (t = 8L + j) under the
    m16n8k16 .f16 B-fragment layout: b_i (i = j & 3) of lane L holds row
    k = 2*(L % 4) + (i & 1) + 8*(i >> 1), col n = L // 4 (+8 for frag1, j >= 4)."""
    seen = set()
    for L in range(32):
        for j in range(8):
            i = j & 3
            k = 2 * (L % 4) + (i & 1) + 8 * (i >> 1)
            n = L // 4 + (8 if j >= 4 else 0)
            assert O.tile_t(k, n) == 8 * L + j
            seen.add((k, n))
    assert len(seen) == 256


def test_reconstruct_restatements_agree():
    rng = np.random.default_rng(11)
    for bits in BITS:
        tr = rng.integers(0, 1 << 16, (3, 5, 16 * bits), dtype=np.uint16).view(np.int16)
        for cb in (0, 1, 2):
            a = O.reconstruct_c(tr, bits, cb).view(np.uint16)
            assert np.array_equal(a, O.reconstruct_np(tr, bits, cb).view(np.uint16))
            assert np.array_equal(a, O.reconstruct_fast(tr, bits, cb).view(np.uint16))


def test_hadamard_vs_scipy_and_reference():
    rng = np.random.default_rng(5)
    H = scipy.linalg.hadamard(128).astype(np.float64)
    v = rng.standard_normal((4, 128)).astype(np.float32)
    got = O.fwht128_np(v)
    assert np.allclose(got, v.astype(np.float64) @ H, rtol=1e-5, atol=1e-4)
    ref = O.ref_lib()
    L = O.lib()
    for row in v:
        a = row.copy()
        L.ora_fwht(a, 128)
        assert np.array_equal(a, O.fwht128_np(row[None])[0])
        if ref is not None:
            b = row.copy()
            ref.ref_hadamard(b, 128)
            assert np.array_equal(a, b)
    assert np.allclose(H @ H, 128 * np.eye(128))


def test_had_in_c_vs_numpy():
    rng = np.random.default_rng(9)
    x = rng.standard_normal((3, 512)).astype(np.float16)
    suh = np.where(rng.integers(0, 2, 512) == 1, 1.0, -1.0).astype(np.float16) * np.float16(0.7)
    assert np.array_equal(O.had_in_c(x, suh).view(np.uint16), O.had_in_np(x, suh).view(np.uint16))
    c = rng.standard_normal((2, 256)).astype(np.float32)
    svh = rng.standard_normal(256).astype(np.float16)
    assert np.allclose(O.had_out_c(c, svh), O.had_out_np(c, svh), rtol=1e-6, atol=1e-6)


def test_dequant_full_vs_matrix_form():
    """W = diag(suh) H Wq H diag(svh) / 128 built from scipy matrices."""
    rng = np.random.default_rng(21)
    K, N, bits = 256, 384, 3
    tr = rng.integers(0, 1 << 16, (K // 16, N // 16, 16 * bits), dtype=np.uint16).view(np.int16)
    suh = (np.where(rng.integers(0, 2, K) == 1, 1.0, -1.0)).astype(np.float16)
    svh = (rng.uniform(0.5, 2, N) / 16).astype(np.float16)
    wq = O.reconstruct_fast(tr, bits).astype(np.float64)
    Hb = np.kron(np.eye(K // 128), scipy.linalg.hadamard(128))
    Hn = np.kron(np.eye(N // 128), scipy.linalg.hadamard(128))
    expect = np.diag(suh.astype(np.float64)) @ Hb @ wq @ Hn @ np.diag(svh.astype(np.float64)) / 128.0
    got = O.dequant_full_c(tr, suh, svh, bits).astype(np.float64)
    assert np.abs(got - expect).max() <= 2e-3 * np.abs(expect).max()


def test_linear_equals_dense_matmul():
    """had_out(had_in(x) Wq) svh == x @ W_full up to the fp16 rounding points."""
    from dsv4_carve_amd import synth

    L = synth.dense(256, 512, 4, seed=5)
    x = synth.activations(3, 256, seed=5)
    y = O.linear(x, L["trellis"], L["suh"], L["svh"], 4)
    wf = O.dequant_full_c(L["trellis"], L["suh"], L["svh"], 4).astype(np.float64)
    ref = x.astype(np.float64) @ wf
    assert np.linalg.norm(y - ref) / np.linalg.norm(ref) < 2e-3
    # a transposed operand or a dropped rotation breaks it by O(1)
    bad = x.astype(np.float64) @ O.reconstruct_fast(L["trellis"], 4).astype(np.float64)
    assert np.linalg.norm(bad - ref) / np.linalg.norm(ref) > 0.5


def test_moe_oracle_brute_force_tiny():
    """Tiny MoE against a per-slot brute force using dense matrices."""
    from dsv4_carve_amd import synth

    H, I, E, topk, m, limit = 256, 256, 6, 3, 4, 10.0
    experts = [synth.expert(e, H, I, 2 + (e % 2), seed=3) for e in range(E)]
    ids = np.array([[0, 3, 5], [1, 1, 2], [5, -1, 9], [4, 0, 3]], np.int32)   # dup, invalid ids
    w = np.array([[0.5, 0.25, 0.25], [0.6, 0.3, 0.1], [1.0, 2.0, 3.0], [0.2, 0.3, 0.5]], np.float32)
    x = synth.activations(m, H, seed=4)
    got = O.moe(x, ids, w, experts, limit)
    full = {}
    for e, ex in enumerate(experts):
        full[e] = {p: O.dequant_full_c(ex[p]["trellis"], ex[p]["suh"], ex[p]["svh"], ex["bits"]).astype(np.float64)
                   for p in ("gate", "up", "down")}
    ref = np.zeros((m, H))
    for r in range(m):
        for k in range(topk):
            e = int(ids[r, k])
            if not 0 <= e < E:
                continue
            g = x[r].astype(np.float64) @ full[e]["gate"]
            u = x[r].astype(np.float64) @ full[e]["up"]
            g = np.minimum(g, limit)
            act = (g / (1 + np.exp(-g))) * np.clip(u, -limit, limit)
            ref[r] += w[r, k] * (act.astype(np.float16).astype(np.float64) @ full[e]["down"])
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) < 5e-3
    assert np.abs(got[2] - 1.0 * ref[2]).max() < 1e-2 * np.abs(ref[2]).max()


def test_golden_fixtures():
    """Committed fixtures (tests/golden/make_golden.py) still match the oracle."""
    import os

    path = os.path.join(os.path.dirname(__file__), "golden", "exl3_golden.npz")
    g = np.load(path, allow_pickle=False)
    import hashlib

    for cb in (0, 1, 2):
        assert hashlib.sha256(O.codebook_lut(cb).tobytes()).hexdigest() == str(g[f"lut_sha256_cb{cb}"])
    for bits in (2, 3, 4, 6):
        tr = g[f"tile_trellis_k{bits}"]
        assert np.array_equal(O.reconstruct_c(tr, bits).view(np.uint16), g[f"tile_wq_k{bits}"])
        assert np.array_equal(O.windows_np(tr, bits).reshape(-1), g[f"tile_windows_k{bits}"].reshape(-1))
    d = g["dense_x"], g["dense_trellis"], g["dense_suh"], g["dense_svh"]
    y = O.linear(d[0], d[1], d[2], d[3], int(g["dense_bits"]))
    assert np.allclose(y, g["dense_y"], rtol=1e-6, atol=1e-6)
