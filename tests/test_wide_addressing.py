"""CPU check of the wide prefill tiles' window addressing (csrc/exl3_prefill.hpp
load_tile_rot, mma_tile_wide; csrc/exl3_gemv.hpp win16): a lane of column
parity p holds its tile rotated by p 32-element blocks, loads only the even
blocks of the rotated stream and the last word before each, and reads each of
its 128 windows at the position the even columns' windows have.  Every window
read that way must be the stream's own window (the oracle's bit-serial
window) of the element the tile permutation puts at (k, 2m + p).  The GPU
test test_prefill_wide_tiles_bitwise_narrow checks the kernel itself."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as O


def _words(tile16: np.ndarray) -> list[int]:
    u = tile16.astype(np.uint16).astype(np.uint32)
    return [int(u[2 * i] | (u[2 * i + 1] << 16)) for i in range(len(u) // 2)]


def _rotated_buffer(words: list[int], bits: int, p: int) -> dict[int, int]:
    """The words load_tile_rot writes: rotated block 0 (bits words from word
    p * bits), the word before it, and rotated blocks 2, 4, 6 with the word
    before each."""
    nw = 8 * bits
    buf = {i: words[p * bits + i] for i in range(bits)}
    buf[nw - 1] = words[bits - 1] if p else words[nw - 1]
    for b in (2, 4, 6):
        for i in range(bits + 1):
            buf[b * bits - 1 + i] = words[p * bits + b * bits - 1 + i]
    return buf


def _win16(buf: dict[int, int], bits: int, t: int) -> int:
    """The kernel's window read: a window inside a word is a field of it, a
    window across words i-1, i a field of the funnel (W[i-1]:W[i]) >> 16."""
    nb, nw = 256 * bits, 8 * bits
    e0 = ((t + 1) * bits) % nb
    e = e0 if e0 else nb
    i1 = (e - 1) >> 5
    o = e - 32 * i1
    if o >= 16:
        return (buf[i1] >> (32 - o)) & 0xFFFF
    mid = ((buf[(i1 + nw - 1) % nw] << 16) | (buf[i1] >> 16)) & 0xFFFFFFFF
    return (mid >> (16 - o)) & 0xFFFF


@pytest.mark.parametrize("bits", range(1, 9))
def test_wide_lane_windows_are_stream_windows(bits):
    rng = np.random.default_rng(100 + bits)
    for _ in range(3):
        tile = rng.integers(-32768, 32768, size=16 * bits, dtype=np.int64).astype(np.int16)
        words = _words(tile)
        for p in (0, 1):
            buf = _rotated_buffer(words, bits, p)
            for r in range(4):
                for i in range(8):
                    n = 2 * (i >> 1) + 8 * (i & 1)          # the even column this lane's windows sit at
                    t0 = 32 * (n & 7) + 8 * r + 4 * (n >> 3)
                    for q in range(4):
                        k = 2 * r + (q & 1) + 8 * (q >> 1)
                        t = O.tile_t(k, n + p)
                        assert t == t0 + q + 32 * p
                        assert _win16(buf, bits, t0 + q) == O.window(tile, bits, t), (bits, p, n, r, q)
