"""GPU parity of the dense path through the C ABI: dequant bit-exact against the
oracle, GEMV/GEMM within the fp tolerance, bitwise repeatable."""

from __future__ import annotations

import numpy as np
import pytest

from dsv4_carve_amd import synth
from oracle import oracle as O
from tests.helpers import assert_close, to_dev

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops(dev):
    from dsv4_carve_amd import ops as _ops
    return _ops


@pytest.mark.parametrize("bits", list(range(1, 9)))
@pytest.mark.parametrize("cb", [O.CB_MCG, O.CB_3INST, O.CB_MUL1])
def test_reconstruct_bit_exact(ops, dev, bits, cb):
    print(f"reconstruct bits={bits} cb={cb}", flush=True)
    rng = np.random.default_rng(1000 + 10 * bits + cb)
    tr = rng.integers(0, 1 << 16, (16, 24, 16 * bits), dtype=np.uint16).view(np.int16)
    got = ops.reconstruct_weight(to_dev(tr, dev), cb).cpu().numpy().view(np.uint16)
    ref = O.reconstruct_fast(tr, bits, cb).view(np.uint16)
    bad = np.argwhere(got != ref)
    assert bad.size == 0, f"{len(bad)} mismatches, first at {bad[:4].tolist()}"


@pytest.mark.parametrize("bits", [2, 3, 4, 6, 8])
def test_reconstruct_primitive_streams(ops, dev, bits):
    """The four primitive-gate streams (primitive_gate.cu:107-121) as tiles."""
    from tests.test_oracle import primitive_streams

    tiles = primitive_streams(bits).view(np.int16).reshape(1, 4, 16 * bits)
    got = ops.reconstruct_weight(to_dev(tiles, dev)).cpu().numpy().view(np.uint16)
    assert np.array_equal(got, O.reconstruct_c(tiles, bits).view(np.uint16))


@pytest.mark.parametrize("bits,cb", [(2, O.CB_MCG), (3, O.CB_MCG), (4, O.CB_MCG), (6, O.CB_MCG), (8, O.CB_MCG),
                                     (1, O.CB_MCG), (5, O.CB_MCG), (7, O.CB_MCG),
                                     (3, O.CB_3INST), (4, O.CB_3INST), (2, O.CB_MUL1), (6, O.CB_MUL1)])
def test_dequant_trellis_bit_exact(ops, dev, bits, cb):
    print(f"dequant_trellis bits={bits} cb={cb}", flush=True)
    L = synth.dense(256, 384, bits, seed=bits + 10 * cb)
    got = ops.dequant_trellis(to_dev(L["trellis"], dev), to_dev(L["suh"], dev), to_dev(L["svh"], dev), bits,
                              mcg=cb == O.CB_MCG, mul1=cb == O.CB_MUL1)
    ref = O.dequant_full_c(L["trellis"], L["suh"], L["svh"], bits, cb)
    g = got.cpu().numpy()
    bad = np.argwhere(g.view(np.uint16) != ref.view(np.uint16))
    if bad.size:
        d = np.abs(g.view(np.int16).astype(np.int32) - ref.view(np.int16).astype(np.int32))
        k, n = bad[0]
        raise AssertionError(f"{len(bad)} of {g.size} differ, max {d.max()} ulp; first ({k},{n}) "
                             f"got {g[k, n]!r} ref {ref[k, n]!r}; rows {sorted(set(bad[:, 0] % 128))[:8]} "
                             f"cols {sorted(set(bad[:, 1] % 128))[:8]}")


def _gemm_case(ops, dev, k, n, bits, rows, out_dtype, seed=0, cb=O.CB_MCG):
    import torch

    print(f"gemm k={k} n={n} bits={bits} rows={rows} out={out_dtype} cb={cb}", flush=True)
    L = synth.dense(k, n, bits, seed=seed + bits)
    x = synth.activations(rows, k, seed=seed + rows)
    tr, su, sv = to_dev(L["trellis"], dev), to_dev(L["suh"], dev), to_dev(L["svh"], dev)
    xd = to_dev(x, dev)
    y = ops.gemm(xd, tr, su, sv, cb, out_dtype)
    y2 = ops.gemm(xd, tr, su, sv, cb, out_dtype)
    torch.cuda.synchronize()
    assert torch.equal(y, y2), "not bitwise repeatable"
    ref = O.linear(x, L["trellis"], L["suh"], L["svh"], bits, cb)
    return y.float().cpu().numpy(), ref


@pytest.mark.parametrize("bits", [2, 3, 4, 6])
@pytest.mark.parametrize("rows", [1, 2, 4, 8, 16])
def test_gemm_small(ops, dev, bits, rows):
    import torch

    got, ref = _gemm_case(ops, dev, 512, 768, bits, rows, torch.float32)
    assert_close(got, ref, what=f"K{bits} rows={rows}")


@pytest.mark.parametrize("bits", [2, 3, 4, 6])
@pytest.mark.parametrize("k,n", [(4096, 4096), (4096, 1536), (1536, 4096), (4096, 12288)])
def test_gemm_baseline_shapes(ops, dev, k, n, bits):
    """The dense sweep at its full sizes, every combination: each shape and
    width at 1, 2, 4, 8 and 16 rows against the oracle (the weight is
    reconstructed once per shape and width)."""
    import torch

    L = synth.dense(k, n, bits, seed=k + n + bits)
    tr, su, sv = to_dev(L["trellis"], dev), to_dev(L["suh"], dev), to_dev(L["svh"], dev)
    w = O.reconstruct_fast(L["trellis"], bits, O.CB_MCG)
    for rows in (1, 2, 4, 8, 16):
        print(f"gemm {k}x{n} K{bits} rows={rows}", flush=True)
        x = synth.activations(rows, k, seed=k + n + rows)
        y = ops.gemm(to_dev(x, dev), tr, su, sv, O.CB_MCG, torch.float32)
        ref = O.linear(x, L["trellis"], L["suh"], L["svh"], bits, O.CB_MCG, w=w)
        assert_close(y.cpu().numpy(), ref, what=f"{k}x{n} K{bits} rows={rows}")


@pytest.mark.parametrize("bits,cb", [(6, O.CB_MCG), (2, O.CB_MCG), (3, O.CB_3INST), (4, O.CB_MUL1)])
def test_gemm_c0_config(ops, dev, bits, cb):
    """K=N=4096, 1 row (6 bits: the CPU-reference configuration).  Against the
    oracle of the reference's CPU path (weights rounded to binary16) at the
    standard bar, and against the oracle on the weights the kernel uses (the
    exact sum of each weight's binary16 codebook addends, which the matrix
    core adds itself; for MUL1, one addend, the two oracles coincide) at fp32
    rounding: rel-L2 2e-6 (measured 1.7e-7)."""
    import torch

    got, ref = _gemm_case(ops, dev, 4096, 4096, bits, 1, torch.float32, seed=2026, cb=cb)
    assert_close(got, ref, what="C0")
    L = synth.dense(4096, 4096, bits, seed=2026 + bits)
    x = synth.activations(1, 4096, seed=2026 + 1)
    exact = O.linear(x, L["trellis"], L["suh"], L["svh"], bits, cb, w=O.reconstruct_exact(L["trellis"], bits, cb))
    mae, rel = assert_close(got, exact, max_abs=2e-5, rel=2e-6, what="C0 (exact addends)")
    print(f"C0 K{bits} cb={cb}: against exact addends max-abs {mae:.3e} rel-L2 {rel:.3e}", flush=True)


@pytest.mark.parametrize("rows", [17, 31, 32, 33, 40, 64, 100, 144])
def test_gemm_many_rows(ops, dev, rows):
    """More than 16 rows run in 32-row blocks (two MFMA row blocks per
    decoded step), the last block ragged."""
    import torch

    got, ref = _gemm_case(ops, dev, 256, 512, 3, rows, torch.float32)
    assert_close(got, ref, what=f"rows={rows}")


@pytest.mark.parametrize("bits,rows", [(2, 1), (6, 20), (4, 37), (3, 16)])
def test_gemm_half_column_block(ops, dev, bits, rows):
    """n = 640: the last 256-column block holds 128 columns; k = 384: six
    64-row steps, so items of 2 steps."""
    import torch

    got, ref = _gemm_case(ops, dev, 384, 640, bits, rows, torch.float32, seed=77)
    assert_close(got, ref, what=f"384x640 K{bits} rows={rows}")


@pytest.mark.parametrize("k,n,bits,rows", [(4096, 4096, 6, 32), (4096, 1536, 2, 144), (1536, 4096, 3, 48)])
def test_gemm_baseline_shapes_many_rows(ops, dev, k, n, bits, rows):
    import torch

    got, ref = _gemm_case(ops, dev, k, n, bits, rows, torch.float32, seed=k + n + rows)
    assert_close(got, ref, what=f"{k}x{n} K{bits} rows={rows}")


@pytest.mark.parametrize("out_dtype", ["float16", "bfloat16"])
def test_gemm_out_dtypes(ops, dev, out_dtype):
    import torch

    dt = getattr(torch, out_dtype)
    got, ref = _gemm_case(ops, dev, 512, 256, 4, 3, dt)
    tol = 4e-3 if out_dtype == "bfloat16" else 1e-3
    assert_close(got, ref, rel=tol, what=out_dtype)


@pytest.mark.parametrize("cb", [O.CB_3INST, O.CB_MUL1])
def test_gemm_other_codebooks(ops, dev, cb):
    import torch

    got, ref = _gemm_case(ops, dev, 512, 512, 3, 2, torch.float32, cb=cb)
    assert_close(got, ref, what=f"cb={cb}")


@pytest.mark.parametrize("bits,cb", [(1, O.CB_MCG), (5, O.CB_MCG), (7, O.CB_MCG), (8, O.CB_MCG),
                                     (5, O.CB_3INST), (6, O.CB_3INST), (2, O.CB_3INST)])
def test_gemm_other_widths(ops, dev, bits, cb):
    """Widths and codebooks outside the sweep (1, 5, 7, 8 bits; 3INST at 2, 5
    and 6 bits): windows inside a word, on a word's half and across a word
    boundary occur at each of them, for MCG and 3INST."""
    import torch

    got, ref = _gemm_case(ops, dev, 512, 512, bits, 3, torch.float32, cb=cb)
    assert_close(got, ref, what=f"K{bits} cb={cb}")


def test_reference_call_surfaces(ops, dev):
    """exllamav3-style exl3_gemm and vllm_exl3_c-style exl3_gemv entry points."""
    import torch

    L = synth.dense(256, 256, 3, seed=77)
    x = synth.activations(5, 256, seed=77)
    tr, su, sv = to_dev(L["trellis"], dev), to_dev(L["suh"], dev), to_dev(L["svh"], dev)
    ref = O.linear(x, L["trellis"], L["suh"], L["svh"], 3)
    C = torch.empty((5, 256), dtype=torch.float32, device=dev)
    assert ops.exl3_gemm(to_dev(x, dev), tr, C, su, None, sv, -1, True, False, 0) == 0
    assert_close(C.cpu().numpy(), ref)
    y = ops.exl3_gemv(to_dev(x, dev), tr, su, sv, 3, True)
    assert y.dtype == torch.float16
    assert_close(y.float().cpu().numpy(), ref, rel=2e-3)


def test_argument_errors(ops, dev):
    import torch

    L = synth.dense(256, 256, 3, seed=1)
    tr, su, sv = to_dev(L["trellis"], dev), to_dev(L["suh"], dev), to_dev(L["svh"], dev)
    with pytest.raises(RuntimeError):
        ops.gemm(torch.zeros((1, 128), dtype=torch.float16, device=dev), tr, su, sv)
    with pytest.raises(RuntimeError):
        ops.gemm(torch.zeros((1, 256), dtype=torch.float32, device=dev), tr, su, sv)
    with pytest.raises(RuntimeError):
        ops.exl3_gemm(torch.zeros((1, 256), dtype=torch.float16, device=dev), tr,
                      torch.empty((1, 256), device=dev), su, None, sv, -1, True, True, 0)


@pytest.mark.parametrize("rows,cols", [(1, 128), (5, 384), (33, 1024)])
def test_had_r_128_against_oracle_rotations(ops, dev, rows, cols):
    """The row Hadamard with a pre scale (fp16 in and out) is the GEMV input
    rotation bit for bit; with a post scale (fp32 in and out) it is the output
    rotation bit for bit.  Odd block counts cover the dropped half-wave."""
    import torch

    print(f"had_r_128 rows={rows} cols={cols}", flush=True)
    rng = np.random.default_rng(rows * 7 + cols)
    x16 = rng.standard_normal((rows, cols)).astype(np.float16)
    suh = (rng.integers(0, 2, cols) * 2 - 1).astype(np.float16)
    svh = ((rng.integers(0, 2, cols) * 2 - 1) * rng.uniform(0.5, 2.0, cols) / 64).astype(np.float16)
    xh = torch.empty((rows, cols), dtype=torch.float16, device=dev)
    ops.had_r_128(to_dev(x16, dev), xh, to_dev(suh, dev), None, 1.0)
    assert np.array_equal(xh.cpu().numpy().view(np.uint16), O.had_in_c(x16, suh).view(np.uint16))
    c = rng.standard_normal((rows, cols)).astype(np.float32)
    y = to_dev(c, dev)
    ops.had_r_128(y, y, None, to_dev(svh, dev), 1.0)                  # in place
    assert np.array_equal(y.cpu().numpy().view(np.uint32), O.had_out_c(c, svh).view(np.uint32))


def test_had_r_128_kinds_scale_and_errors(ops, dev):
    """bf16 input rounds through fp16 before the pre scale; the scale argument
    multiplies after the 1/sqrt(128); outputs in every kind agree with an fp64
    Sylvester-Hadamard product within their rounding."""
    import torch
    from scipy.linalg import hadamard

    rng = np.random.default_rng(3)
    rows, cols = 4, 256
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    suh = (rng.integers(0, 2, cols) * 2 - 1).astype(np.float16)
    H = hadamard(128).astype(np.float64) / np.sqrt(128.0)
    xb = torch.from_numpy(x).to(torch.bfloat16)
    x_in = xb.float().numpy().astype(np.float16).astype(np.float64) * suh.astype(np.float64)
    want = np.concatenate([x_in[:, b:b + 128] @ H for b in range(0, cols, 128)], axis=1) * 0.5
    for out_dtype, tol in ((torch.float32, 1e-5), (torch.float16, 2e-3), (torch.bfloat16, 1e-2)):
        y = torch.empty((rows, cols), dtype=out_dtype, device=dev)
        ops.had_r_128(xb.to(dev), y, to_dev(suh, dev), None, 0.5)
        got = y.float().cpu().numpy()
        assert np.max(np.abs(got - want)) <= tol * max(1.0, np.max(np.abs(want))), out_dtype
    with pytest.raises(RuntimeError):
        ops.had_r_128(torch.zeros((2, 100), device=dev), torch.zeros((2, 100), device=dev), None, None)
    with pytest.raises(RuntimeError):
        ops.had_r_128(torch.zeros((2, 128), device=dev), torch.zeros((2, 256), device=dev), None, None)
    with pytest.raises(RuntimeError):
        ops.had_r_128(torch.zeros((2, 128), device=dev), torch.zeros((2, 128), device=dev),
                      torch.zeros(64, dtype=torch.float16, device=dev), None)


@pytest.mark.parametrize("bits,cb", [(2, O.CB_MCG), (3, O.CB_MCG), (6, O.CB_MCG), (4, O.CB_3INST),
                                     (3, O.CB_MUL1), (8, O.CB_MCG)])
def test_dequant_nk_is_the_transpose(ops, dev, bits, cb):
    """The [n][k] layouts hold bitwise the transposes of the raw and the
    Hadamard-folded matrices, which are themselves the oracle's."""
    print(f"dequant_nk bits={bits} cb={cb}", flush=True)
    L = synth.dense(384, 256, bits, seed=60 + bits + cb)
    tr, su, sv = to_dev(L["trellis"], dev), to_dev(L["suh"], dev), to_dev(L["svh"], dev)
    raw_t = ops.reconstruct_weight_nk(tr, cb).cpu().numpy()
    assert raw_t.shape == (256, 384)
    assert np.array_equal(raw_t.view(np.uint16).T, O.reconstruct_c(L["trellis"], bits, cb).view(np.uint16))
    w_t = ops.dequant_trellis_nk(tr, su, sv, bits, mcg=cb == O.CB_MCG, mul1=cb == O.CB_MUL1).cpu().numpy()
    ref = O.dequant_full_c(L["trellis"], L["suh"], L["svh"], bits, cb)
    assert np.array_equal(w_t.view(np.uint16).T, ref.view(np.uint16))


@pytest.mark.parametrize("rows", [1, 16, 32])
def test_xcd_keyed_order_is_bitwise_the_plain_order(ops, dev, monkeypatch, rows):
    """The XCD-keyed item order (a column block's split-K items and its finish
    on one XCD) only moves items between workgroups: a 4096x4096 call and a fan
    whose column blocks are a multiple of 8 give bitwise the outputs of the
    plain order (EXL3_XCD_ORDER=0), and match the oracle."""
    import torch

    k, n, bits = 4096, 4096, 3
    L = synth.dense(k, n, bits, seed=910)
    t, u, v = (to_dev(L[key], dev) for key in ("trellis", "suh", "svh"))
    x_np = synth.activations(rows, k, seed=911)
    x = to_dev(x_np, dev)
    fan_ns = (1024, 512, 1024, 1024, 256, 256)          # 16 column blocks
    fan = [synth.dense(k, fn, 6, seed=920 + i) for i, fn in enumerate(fan_ns)]
    members = [tuple(to_dev(f[key], dev) for key in ("trellis", "suh", "svh")) for f in fan]

    def run():
        y = ops.gemm(x, t, u, v, ops.CB_MCG, torch.float32)
        ys = ops.gemm_group(x, members, ops.CB_MCG, torch.float32) if rows <= 16 else []
        torch.cuda.synchronize()
        return [y.cpu().numpy()] + [z.cpu().numpy() for z in ys]

    monkeypatch.setenv("EXL3_XCD_ORDER", "0")
    plain = run()
    monkeypatch.delenv("EXL3_XCD_ORDER")
    keyed = run()
    for a, b in zip(plain, keyed):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    ref = O.linear(x_np, L["trellis"], L["suh"], L["svh"], bits, O.CB_MCG)
    assert_close(keyed[0], ref, what=f"keyed order rows={rows}")
