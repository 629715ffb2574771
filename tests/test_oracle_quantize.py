"""Pins of the oracle's int8 side output (quantize_x, kernels/quantize.h:10-25)
and of the host mirror's bookkeeping of it (ops/HipBase.scala:117-214).

The reference has no CPU form and no golden vectors for this quantization;
its GPU tests hold the fused norms equal to a separate quantize_x launch
(gpuTest/.../FusedOpsTests.scala:96-176). The oracle's restatement is pinned
here by what fixes the formula: a hand-worked block, the extreme value of a
block mapping to +-127, every value within half a step of its code, ties
going away from zero (roundf, not round-to-even), xs = xd * sum(codes), and
zero and NaN blocks."""

import numpy as np
import pytest
import torch

from drift_amd import ops as d
from oracle import oracle as o


def test_worked_block():
    x = np.arange(32, dtype=np.float32)
    xq, xd, xs = o.quantize_x(x)
    step = np.float32(31) / np.float32(127)
    assert xd[0] == step
    # i / (31 / 127) = 4.097 i: 1 -> 4, 2 -> 8, 3 -> 12, 16 -> 65.55 -> 66, 31 -> 127
    assert [int(xq[i]) for i in (0, 1, 2, 3, 16, 31)] == [0, 4, 8, 12, 66, 127]
    assert xs[0] == step * np.float32(int(xq.astype(np.int64).sum()))


def test_extremes_map_to_127_and_codes_are_nearest():
    rng = np.random.default_rng(5)
    x = (rng.standard_normal(32 * 500) * rng.uniform(1e-3, 1e3, 32 * 500)).astype(np.float32)
    xq, xd, xs = o.quantize_x(x)
    blocks = x.reshape(-1, 32).astype(np.float64)
    codes = xq.reshape(-1, 32).astype(np.int64)
    amax = np.abs(blocks).max(axis=1)
    assert np.all(np.abs(codes).max(axis=1) == 127)
    assert np.all(codes[np.arange(len(codes)), np.abs(blocks).argmax(axis=1)] ==
                  127 * np.sign(blocks[np.arange(len(blocks)), np.abs(blocks).argmax(axis=1)]))
    # xd is amax / 127 rounded once to float
    assert np.all(np.abs(xd.astype(np.float64) - amax / 127) <= np.spacing(xd).astype(np.float64) / 2)
    # each code is the nearest step to its value (the quotient is rounded to
    # float first, so within half a step and one float ulp of it)
    err = np.abs(blocks - codes * xd[:, None].astype(np.float64))
    assert np.all(err <= xd[:, None] * (0.5 + 2 ** -20))
    assert np.array_equal(xs, xd * codes.sum(axis=1).astype(np.float32))


def test_ties_round_away_from_zero():
    # amax = 127 / 16, so xd = 1/16 exactly and (k + 1/2) / 16 is a tie
    halves = (np.arange(1, 31) + 0.5) / 16
    x = np.concatenate([[127 / 16, -0.5 / 16], halves]).astype(np.float32)
    xq, xd, _ = o.quantize_x(x)
    assert xd[0] == np.float32(1 / 16)
    assert xq[1] == -1  # -0.5 goes to -1, not to -0
    assert np.array_equal(xq[2:].astype(np.int64), np.arange(1, 31) + 1)
    xq, _, _ = o.quantize_x(-x)
    assert np.array_equal(xq[2:].astype(np.int64), -(np.arange(1, 31) + 1))


def test_zero_and_nan_blocks():
    x = np.zeros(64, np.float32)
    x[32 + 5] = np.nan
    x[32 + 9] = 2.0
    x[32] = np.nan
    xq, xd, xs = o.quantize_x(x)
    assert np.all(xq[:32] == 0) and xd[0] == 0 and xs[0] == 0
    # fmaxf skips the NaNs: amax 2, the NaNs' codes 0
    assert xd[1] == np.float32(2) / np.float32(127)
    assert xq[32 + 9] == 127 and xq[32 + 5] == 0 and xq[32] == 0 and xs[1] == xd[1] * 127


def test_partial_blocks_are_refused():
    with pytest.raises(ValueError, match="whole blocks"):
        o.quantize_x(np.zeros(40, np.float32))


# ---------------------------------------------------------------- bookkeeping (host only)

def test_side_output_bookkeeping():
    hip = d.HipOps()
    out = torch.zeros((4, 2048), dtype=torch.float32)
    # no int8 product has run: nothing is quantized as written
    assert hip.quantizedTarget(out, 2048) == (None, (None, None, None))
    hip.quantizesX = True
    target, pointers = hip.quantizedTarget(out, 2048)
    assert target is not None and all(p is not None for p in pointers)
    assert target.codes().numel() == 8192 and target.scales().numel() == 256 and target.sums().numel() == 256
    # codes, then scales, then sums, in one buffer
    assert target.scales().data_ptr() - target.codes().data_ptr() == 8192
    assert target.sums().data_ptr() - target.scales().data_ptr() == 4 * 256
    hip.deviceWrites += 1  # the launch that writes out
    hip.wroteQuantized(target)
    rows = hip.quantizedInput(out[1:3], 2, 2048)
    assert rows is not None
    codes, scales, sums = rows
    assert codes.data_ptr() == target.codes().data_ptr() + 2048 and codes.numel() == 4096
    assert scales.data_ptr() == target.scales().data_ptr() + 4 * 64 and scales.numel() == 128
    assert sums.numel() == 128
    # not whole blocks from a block boundary, past the end, or another type: no
    assert hip.quantizedInput(out.view(-1)[16:], 1, 2048) is None
    assert hip.quantizedInput(out[3:], 2, 2048) is None
    assert hip.quantizedInput(out.to(torch.bfloat16), 1, 2048) is None
    # any later write makes it stale
    hip.wrote()
    assert hip.quantizedInput(out, 4, 2048) is None
    # too many values, a BF16 out or rows not of whole blocks: not eligible
    assert hip.quantizedTarget(torch.zeros((9, 16384)), 16384)[0] is None
    assert hip.quantizedTarget(torch.zeros((4, 2048), dtype=torch.bfloat16), 2048)[0] is None
    assert hip.quantizedTarget(torch.zeros((4, 48)), 48)[0] is None
