"""bench.py on the CPU: the one-GPU refusal, argument errors, and the
algorithmic byte counts the roofline divides by (checked against the bytes of
the actual synthetic tensors, not against the formula)."""

from __future__ import annotations

import os
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402
from dsv4_carve_amd import synth  # noqa: E402


def _run(*args):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], capture_output=True, text=True,
                          timeout=120, cwd=ROOT)


def test_more_than_one_gpu_is_refused_with_a_message():
    r = _run("--gpus", "2")
    assert r.returncode == 2 and "one GPU" in r.stderr and not r.stdout.strip()


def test_unknown_extra_leg_is_an_error():
    r = _run("--extra", "sweep,nope")
    assert r.returncode == 2 and "nope" in r.stderr


@pytest.mark.parametrize("bits", [2, 3, 4, 6])
def test_expert_bytes_equal_the_tensors(bits):
    h, i = 512, 256
    ex = synth.expert(0, h, i, bits, seed=1)
    nbytes = sum(ex[p][t].nbytes for p in ("gate", "up", "down") for t in ("trellis", "suh", "svh"))
    assert bench.expert_bytes(h, i, bits) == nbytes


def test_step_bytes_count_each_distinct_valid_expert_once():
    h, i = 512, 256
    bits = [2, 3, 2, 3]
    ids = np.array([[0, 1, 1], [1, 3, -1], [7, 0, 3]])          # 0, 1, 3 valid; -1 and 7 are not
    want = sum(bench.expert_bytes(h, i, bits[e]) for e in (0, 1, 3)) + 3 * h * (2 + 4)
    assert bench.step_bytes(ids, bits, h, i) == want
