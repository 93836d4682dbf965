"""GPU parity of the routed-MoE prefill path (grouped GEMMs, exl3_moe_prefill)
through the C ABI: against the oracle on small layers, with uniform and
Zipf-skewed routing (experts with several tiles, narrow and wide), wide tiles
bitwise against narrow ones, invalid and duplicate
ids, dtypes, a shared expert as an extra slot; against the decode kernel
(itself checked against the oracle) at the full 256-expert shape, row by row.
Tolerance: max-abs 2e-2, rel-L2 1e-3 against the oracle; decode vs prefill
differ only by fp32 summation order (split-K partials vs one pass)."""

from __future__ import annotations

import numpy as np
import pytest

from dsv4_carve_amd import synth
from oracle import oracle as O
from tests.helpers import assert_close, rel_l2, to_dev
from tests.test_gpu_moe import Layer

pytestmark = pytest.mark.gpu

LIMIT = 10.0


def run_prefill(layer, x, ids, w, out_dtype=None, limit=LIMIT, uniform=False):
    import torch
    from dsv4_carve_amd import ops

    dev = layer.ebits.device
    xd = x if isinstance(x, torch.Tensor) else to_dev(x, dev)
    out = torch.empty(xd.shape, dtype=out_dtype or torch.float32, device=dev)
    widths = dict(bits=layer.bits[0]) if uniform else dict(expert_bits=layer.ebits, bits_mask=layer.mask)
    ops.moe_prefill(xd, out, layer.tables, to_dev(ids.astype(np.int32), dev), to_dev(w.astype(np.float32), dev),
                    intermediate=layer.I, swiglu_limit=limit, **widths)
    assert ops.moe_error(ops.SCRATCH.current(dev, "moe_prefill")) == 0, "prefill set its error word"
    return out


@pytest.fixture(scope="module")
def small(dev):
    bits = [3, 2, 4, 3, 2, 2, 3, 4, 2, 3, 3, 2, 4, 2, 3, 2]
    return Layer(dev, 16, 512, 256, bits, seed=23)


@pytest.mark.parametrize("tokens", [1, 5, 17, 40, 130])
@pytest.mark.parametrize("routing", ["uniform", "zipf"])
def test_prefill_against_oracle(small, tokens, routing):
    print(f"prefill {routing} tokens={tokens}", flush=True)
    if routing == "uniform":
        ids, w = synth.routing(tokens, 16, 6, seed=800 + tokens)
    else:
        ids, w = synth.zipf_routing(tokens, 16, 6, seed=801 + tokens)
    x = synth.activations(tokens, 512, seed=802 + tokens)
    got = run_prefill(small, x, ids, w).cpu().numpy()
    assert_close(got, small.ref(x, ids, w), what=f"prefill {routing} T={tokens}")


@pytest.mark.parametrize("tokens", [9, 70])
def test_prefill_other_widths(dev, tokens):
    """Experts at 1, 5, 6, 7 and 8 bits: one GEMM launch per width, the
    one-multiply decode at 5, 6 and 7 bits, tiles with and without a second
    16-row block (70 tokens over 8 experts gives tiles past 16 rows)."""
    print(f"prefill other widths tokens={tokens}", flush=True)
    layer = Layer(dev, 8, 512, 256, [5, 6, 7, 1, 8, 5, 7, 6], seed=31)
    ids, w = synth.zipf_routing(tokens, 8, 6, seed=830 + tokens)
    x = synth.activations(tokens, 512, seed=831 + tokens)
    got = run_prefill(layer, x, ids, w).cpu().numpy()
    assert_close(got, layer.ref(x, ids, w), what=f"prefill widths 1/5/6/7/8 T={tokens}")


@pytest.mark.parametrize("hidden", [1280, 2304])
def test_prefill_hidden_not_a_multiple_of_512(dev, hidden):
    """A hidden size that is a multiple of 256 but not of 512: the input
    rotation's last 512-column wave is half full (its lanes past the row
    store nothing), and the down GEMM has an odd number of 256-column
    blocks."""
    print(f"prefill hidden={hidden}", flush=True)
    layer = Layer(dev, 6, hidden, 256, [3, 2, 3, 2, 4, 3], seed=36)
    ids, w = synth.zipf_routing(21, 6, 4, seed=840)
    x = synth.activations(21, hidden, seed=841)
    got = run_prefill(layer, x, ids, w).cpu().numpy()
    assert_close(got, layer.ref(x, ids, w), what=f"prefill hidden {hidden}")


def test_prefill_hot_expert_many_tiles(small):
    """Every token routes to expert 3 (4 tiles of 32 rows + a partial one) and
    to one other expert; duplicate ids within a row count twice."""
    T = 150
    rng = np.random.default_rng(4)
    ids = np.stack([np.array([3, rng.integers(0, 16), 3, rng.integers(0, 16)]) for _ in range(T)]).astype(np.int32)
    w = rng.random((T, 4)).astype(np.float32)
    w /= w.sum(axis=1, keepdims=True)          # routing weights are normalised per token
    x = synth.activations(T, 512, seed=805)
    got = run_prefill(small, x, ids, w).cpu().numpy()
    assert_close(got, small.ref(x, ids, w), what="hot expert")


def test_prefill_wide_tiles_bitwise_narrow(small):
    """Experts with more than 32 rows run wide tiles (up to 64 rows, each
    decoded step applied to four 16-row blocks, half of each tile's columns per
    lane): expert 3 (3-bit) gets 300 rows (four full wide tiles and a 44-row
    one), expert 5 (2-bit) 150 (two full ones and a 22-row narrow tile),
    expert 7 (4-bit) about 40 (one partial wide tile).  The same tokens in
    5-token calls give no expert more than 10 rows, so only narrow tiles run;
    every output row is bitwise the same either way, and both meet the oracle
    bar."""
    import torch

    T = 150
    rng = np.random.default_rng(14)
    others = np.array([0, 1, 2, 4, 6, 8, 9, 10, 11, 12, 13, 14, 15])
    ids = np.zeros((T, 4), np.int32)
    ids[:, 0], ids[:, 1], ids[:, 2] = 3, 5, 3
    ids[:, 3] = np.where(np.arange(T) < 40, 7, others[rng.integers(0, len(others), T)])
    w = rng.random((T, 4)).astype(np.float32)
    w /= w.sum(axis=1, keepdims=True)
    x = synth.activations(T, 512, seed=815)
    print("prefill wide tiles vs 5-token slices", flush=True)
    whole = run_prefill(small, x, ids, w)
    sliced = torch.cat([run_prefill(small, x[i:i + 5], ids[i:i + 5], w[i:i + 5]) for i in range(0, T, 5)])
    torch.cuda.synchronize()
    assert torch.equal(whole, sliced), "wide tiles changed a row's result"
    assert_close(whole.cpu().numpy(), small.ref(x, ids, w), what="wide tiles")
    # against the weights the kernels use (exact sums of the codebook addends)
    mae, rel = assert_close(whole.cpu().numpy(), small.ref(x, ids, w, exact_addends=True), max_abs=4e-3, rel=1e-4,
                            what="wide tiles (exact addends)")
    print(f"wide tiles against exact addends: max-abs {mae:.3e} rel-L2 {rel:.3e}", flush=True)


@pytest.mark.parametrize("tokens", [700, 1400])
def test_prefill_k_split_by_pair_count(small, tokens):
    """The GEMMs split K in two parts below 4096 (down) and 8192 (gate/up)
    (token, slot) pairs and run it whole above: 700 tokens x top-6 (4200 pairs)
    splits only the gate/up GEMM, 1400 tokens (8400 pairs) neither."""
    print(f"prefill k-split tokens={tokens}", flush=True)
    ids, w = synth.zipf_routing(tokens, 16, 6, seed=850 + tokens)
    x = synth.activations(tokens, 512, seed=851 + tokens)
    got = run_prefill(small, x, ids, w).cpu().numpy()
    assert_close(got, small.ref(x, ids, w), what=f"prefill T={tokens}")


def test_prefill_at_the_pair_limit(small):
    """The largest call one prefill launch sequence takes: 8192 tokens at
    top-8, 65536 (token, slot) pairs, about 4096 rows per expert (64 wide tiles
    each), K whole in both GEMMs."""
    T = 8192
    print(f"prefill at the pair limit T={T} top-8", flush=True)
    ids, w = synth.routing(T, 16, 8, seed=860)
    x = synth.activations(T, 512, seed=861)
    got = run_prefill(small, x, ids, w).cpu().numpy()
    assert_close(got, small.ref(x, ids, w), what="prefill 65536 pairs")


def test_prefill_invalid_ids_and_zero_rows(small):
    T = 33
    rng = np.random.default_rng(6)
    ids = rng.integers(-3, 20, size=(T, 5)).astype(np.int32)
    ids[7] = -1                       # a token routed nowhere: exact zero
    w = rng.random((T, 5)).astype(np.float32)
    w /= w.sum(axis=1, keepdims=True)
    x = synth.activations(T, 512, seed=806)
    got = run_prefill(small, x, ids, w).cpu().numpy()
    assert np.all(got[7] == 0.0)
    assert_close(got, small.ref(x, ids, w), what="invalid ids")


@pytest.mark.parametrize("x_dtype,out_dtype", [("fp16", "bf16"), ("bf16", "fp16"), ("bf16", "fp32")])
def test_prefill_dtypes(small, dev, x_dtype, out_dtype):
    import torch

    dt = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}
    T = 24
    ids, w = synth.zipf_routing(T, 16, 6, seed=807)
    x = synth.activations(T, 512, seed=808)
    xd = to_dev(x, dev).to(dt[x_dtype])
    got = run_prefill(small, xd, ids, w, out_dtype=dt[out_dtype]).float().cpu().numpy()
    x16 = xd.to(torch.float16).cpu().numpy()
    ref = small.ref(x16, ids, w)
    # a 16-bit output adds its own rounding (half an ulp: 2^-11 fp16, 2^-9 bf16)
    slack = {"fp32": 0.0, "fp16": 1e-3, "bf16": 4e-3}[out_dtype]
    assert_close(got, ref, max_abs=2e-2 + 8 * slack, rel=1e-3 + slack, what=f"{x_dtype}->{out_dtype}")


def test_prefill_shared_expert_slot(dev):
    layer = Layer(dev, 13, 512, 256, [3, 2] * 6 + [6], seed=34)
    T = 45
    ids, w = synth.zipf_routing(T, 12, 8, seed=809)
    ids9 = np.concatenate([ids, np.full((T, 1), 12, np.int32)], axis=1)
    w9 = np.concatenate([w, np.ones((T, 1), np.float32)], axis=1)
    x = synth.activations(T, 512, seed=810)
    got = run_prefill(layer, x, ids9, w9).cpu().numpy()
    assert_close(got, layer.ref(x, ids9, w9), what="routed + shared, prefill")


def test_prefill_uniform_width_and_repeat(dev):
    import torch

    layer = Layer(dev, 8, 256, 512, [2] * 8, seed=35)
    T = 70
    ids, w = synth.routing(T, 8, 3, seed=811)
    x = synth.activations(T, 256, seed=812)
    a = run_prefill(layer, x, ids, w, uniform=True)
    b = run_prefill(layer, x, ids, w, uniform=True)
    torch.cuda.synchronize()
    assert torch.equal(a, b), "prefill is not bitwise repeatable"
    assert_close(a.cpu().numpy(), layer.ref(x, ids, w), what="uniform K2")


def test_prefill_matches_decode_at_full_shape(dev):
    """256 experts, top-8, hidden 4096, intermediate 2048, 3/2-bit: 48 tokens in
    one prefill call against three 16-row decode launches, row by row."""
    from tests.test_gpu_moe import Layer as L

    print("prefill vs decode at the full layer shape", flush=True)
    layer = L(dev, 256, 4096, 2048, synth.mixed_bits(256), seed=2)
    T = 48
    ids, w = synth.zipf_routing(T, 256, 8, seed=813)
    x = synth.activations(T, 4096, seed=814)
    pre = run_prefill(layer, x, ids, w).cpu().numpy()
    dec = np.concatenate([layer.run(x[i:i + 16], ids[i:i + 16], w[i:i + 16]).cpu().numpy() for i in (0, 16, 32)])
    # The two paths add the gate/up sums in different fp32 orders (split-K
    # parts), which can flip an fp16 rounding of the activation by one ulp
    # (~5e-4 of that element) before the down projection: rel-L2 5e-4, half the
    # parity bar.  Both paths meet the oracle bar on their own (tests above).
    for r in range(T):
        assert rel_l2(pre[r], dec[r]) < 5e-4, f"row {r}: prefill and decode differ"
