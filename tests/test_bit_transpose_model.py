"""A lane-by-lane model of the transposed packed-bit operand of
gemm_narrow_bits_t (csrc/synapse.hip): the row order a lane loads, the
5-stage butterfly across lanes (partner lane l ^ D inside each half-wave,
rotate by the lane's own amount, bit-field insert with the lane's own
mask), and the expansion of a transposed word into the bf16 MFMA
fragment (mask, 24-bit multiply by 0x3F80).  The model must give, for every
lane, group and fragment pair, the 0/1 values of the rows that the 32x32x16
MFMA's A layout assigns to that slot (lane l: row l % 32 of the tile, k =
8 (l / 32) + [0, 8) of each 16-k group), so the kernel's bits are those of a
plain 0/1 operand.  CPU only."""

from __future__ import annotations

import numpy as np
import pytest

MASK = {16: 0x0000FFFF, 8: 0x00FF00FF, 4: 0x0F0F0F0F, 2: 0x33333333, 1: 0x55555555}
LANES = np.arange(64)


def rho(lane):
    """The row of a 64-row block that lane loads."""
    j = lane & 31
    return 16 * ((j & 15) >> 2) + 2 * (j & 3) + (j >> 4) + 8 * (lane >> 5)


def rotr(v, s):
    s %= 32
    return ((v >> s) | (v << (32 - s))) & 0xFFFFFFFF if s else v


def butterfly(words, order=(16, 8, 4, 2, 1), rho_fn=rho, flip_rotate=False):
    """words[r]: bit c = S[r, c].  Returns the 64 lanes' words after the
    stages (lane l, l ^ D partners inside each half-wave)."""
    w = [int(words[rho_fn(lane)]) for lane in range(64)]
    for D in order:
        partner = [w[(lane & 32) | ((lane & 31) ^ D)] for lane in range(64)]
        new = []
        for lane in range(64):
            top = (lane & D) == 0
            rot = (32 - D if top else D) if not flip_rotate else (D if top else 32 - D)
            keep = MASK[D] if top else ~MASK[D] & 0xFFFFFFFF
            q = rotr(partner[lane], rot)
            new.append((w[lane] & keep) | (q & ~keep & 0xFFFFFFFF))
        w = new
    return w


def fragment(x):
    """Per lane, per group q (0-3), the 8 bf16 bit patterns of its A slots."""
    out = np.zeros((64, 4, 8), dtype=np.int64)
    for lane in range(64):
        for q in range(4):
            xb = x[lane] >> 8 if q >= 2 else x[lane]
            for i in range(4):
                bp = (4 * q + i) & 7
                masked = xb & (0x10001 << bp)
                assert masked < (1 << 24), "the multiply is a 24-bit one"
                d = masked * (0x3F80 >> bp)
                out[lane, q, 2 * i] = d & 0xFFFF
                out[lane, q, 2 * i + 1] = d >> 16
    return out


def expected(S):
    """The MFMA A layout: lane l, group q, slot s holds row 16 q + 8 (l / 32) +
    s of column l % 32."""
    out = np.zeros((64, 4, 8), dtype=np.int64)
    for q in range(4):
        for s in range(8):
            rows = 16 * q + 8 * (LANES >> 5) + s
            out[:, q, s] = np.where(S[rows, LANES & 31] != 0, 0x3F80, 0)
    return out


def words_of(S):
    return [sum(int(S[r, c]) << c for c in range(32)) for r in range(64)]


@pytest.mark.parametrize("seed", range(6))
def test_lane_model_gives_the_mfma_fragments(seed):
    rng = np.random.default_rng(seed)
    density = (0.5, 0.1, 0.9, 0.02, 0.98, 0.5)[seed]
    S = (rng.random((64, 32)) < density).astype(np.uint8)
    frag = fragment(butterfly(words_of(S)))
    np.testing.assert_array_equal(frag, expected(S))


def test_lane_model_single_bits():
    # every one-hot block: exactly one slot of one lane holds 1.0
    for r in range(64):
        for c in range(32):
            S = np.zeros((64, 32), dtype=np.uint8)
            S[r, c] = 1
            np.testing.assert_array_equal(fragment(butterfly(words_of(S))), expected(S))


def test_plausible_mistakes_are_caught():
    rng = np.random.default_rng(7)
    S = (rng.random((64, 32)) < 0.5).astype(np.uint8)
    ref = expected(S)
    # rows loaded in plain order, the rotate turned the wrong way, a stage
    # order that skips a stage: each gives other fragments
    plain = lambda lane: lane
    assert not np.array_equal(fragment(butterfly(words_of(S), rho_fn=plain)), ref)
    assert not np.array_equal(fragment(butterfly(words_of(S), flip_rotate=True)), ref)
    assert not np.array_equal(fragment(butterfly(words_of(S), order=(16, 8, 4, 2))), ref)
