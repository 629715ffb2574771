"""Pins the oracle's ConvRot decoding (CPU only): ConvRot.rotate
(tensor/ConvRot.scala:20-50) and CpuBase.rotatedRows (ops/CpuBase.scala:
40-81).

The reference's fixtures for it (comfy_quant.safetensors and its expected
weights) are Git LFS pointers in the checkout, so the checks restate what
their generator (runner/fixtures/comfy_quant.py) computes, independently of
the loops under test:
- the rotation is the explicit 256 x 256 matrix, the Kronecker fourth power
  of [[1, 1, 1, -1], [1, 1, -1, 1], [1, -1, 1, 1], [-1, 1, 1, 1]] / 2
  (comfy_quant.py:39-45): exactly on small integers, to rounding on normals;
- it is its own inverse (ComfyQuantTests.scala:99-106, the same seed);
- its rounding is the rounds' order (strides 1, 4, 16, 64, sums left to
  right), written here as digit-axis passes over a [4, 4, 4, 4] view;
- the 4-bit levels are clip(round(codebook[code] * e4m3(relative)), -127,
  127) times the row scale (comfy_quant.py:95-108), e4m3 pinned to torch's
  float8_e4m3fn over all 256 codes.
"""

import numpy as np
import pytest
import torch

from oracle import oracle as o
from tests.helpers import comparison

F = np.float32


def hadamard():
    h4 = np.ones((4, 4)) - 2 * np.eye(4)[::-1]
    h = np.array([[1.0]])
    while h.shape[0] < 256:
        h = np.kron(h, h4)
    return h / 16.0


H = hadamard()


def test_the_matrix_is_symmetric_orthogonal():
    assert np.array_equal(H, H.T) and np.allclose(H @ H, np.eye(256), atol=1e-12)


def test_rotation_is_the_matrix_exactly_on_small_integers():
    x = np.random.default_rng(1).integers(-8, 9, (3, 512)).astype(F)
    want = (x.reshape(3, 2, 256).astype(np.float64) @ H).reshape(3, 512)
    assert np.array_equal(o.convrot_rotate(x), want.astype(F))


def test_rotation_is_the_matrix_to_rounding():
    x = np.random.default_rng(2).standard_normal((4, 1024)).astype(F)
    want = (x.reshape(4, 4, 256).astype(np.float64) @ H).reshape(4, 1024)
    assert np.abs(o.convrot_rotate(x) - want).max() < 1e-5


def test_rotation_is_its_own_inverse():
    # ComfyQuantTests.scala:99-106: Random(3) gaussians, Tolerance(1e-3, 1e-3)
    # apart once, Tolerance(1e-5, 1e-4) together twice
    values = o.java_gaussian(3, 512)
    once = o.convrot_rotate(values)
    assert not comparison(values, once, absolute=1e-3, relative=1e-3)[0]
    assert comparison(values, o.convrot_rotate(once), absolute=1e-5, relative=1e-4)[0]


def staged(x):
    """The rounds as passes along the base-4 digits of the column, digit 0
    (stride 1) first, float32, each half summed left to right."""
    x = x.astype(F).reshape(-1, 4, 4, 4, 4)  # [group, d3, d2, d1, d0]
    for axis in (4, 3, 2, 1):
        a, b, c, d = (np.take(x, k, axis=axis) for k in range(4))
        half = (((a + b) + c) + d) * F(0.5)
        x = np.stack([half - d, half - c, half - b, half - a], axis=axis)
    return x.reshape(-1)


def test_rotation_rounds_as_the_rounds_order():
    x = np.random.default_rng(3).standard_normal(256 * 64).astype(F) * F(3.7)
    got = o.convrot_rotate(x)
    assert np.array_equal(got.view(np.uint32), staged(x).view(np.uint32))
    # a round order the other way round rounds differently somewhere
    reverse = x.reshape(-1, 4, 4, 4, 4).transpose(0, 4, 3, 2, 1).reshape(-1)
    other = staged(reverse).reshape(-1, 4, 4, 4, 4).transpose(0, 4, 3, 2, 1).reshape(-1)
    assert not np.array_equal(got.view(np.uint32), other.view(np.uint32))


def test_e4m3_is_torchs_float8_e4m3fn():
    codes = np.arange(256, dtype=np.uint8)
    want = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    got = np.array([o.f8e4m3(c) for c in codes], F)
    nan = np.isnan(want)
    assert list(np.flatnonzero(nan)) == [0x7F, 0xFF] and np.isnan(got[nan]).all()
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_int8_levels_are_codes_times_the_row_scale():
    r = o.random_rotated(5, 256, np.random.default_rng(4))
    want = r.codes.view(np.int8).astype(F) * r.scales[:, None]
    assert np.array_equal(r.levels(), want)
    one = o.random_rotated(2, 256, np.random.default_rng(5), one_scale=True)
    assert np.array_equal(one.levels(), one.codes.view(np.int8).astype(F) * one.scales[0])


@pytest.mark.parametrize("group_size", [16, 32, 128])
def test_four_bit_levels_follow_the_fixture_generator(group_size):
    rows, cols = 3, 512
    r = o.random_rotated(rows, cols, np.random.default_rng(6), four_bit=True, group_size=group_size)
    raw = r.codes.astype(np.int32)
    codes = np.empty((rows, cols), np.int32)
    codes[:, 0::2] = raw & 0xF
    codes[:, 1::2] = (raw >> 4) & 0xF
    e4m3 = torch.from_numpy(r.relative.copy()).view(torch.float8_e4m3fn).float().numpy()
    values = r.codebook[codes].reshape(rows, -1, group_size) * e4m3[:, :, None]
    int8 = np.clip(np.round(values), -127, 127).astype(F)
    assert (np.abs(np.round(values)) > 127).any(), "the clamp is exercised"
    want = (int8 * r.scales.reshape(rows, 1, 1)).reshape(rows, cols)
    assert np.array_equal(r.levels(), want)
    # and the weight is those levels unrotated, as the generator's expected file
    unrotated = (want.reshape(rows, -1, 256).astype(np.float64) @ H).reshape(rows, cols)
    assert comparison(unrotated, r.rows_of(), absolute=1e-4, relative=1e-5)[0]


def test_nan_relative_scales_spread_over_their_group():
    r = o.random_rotated(2, 512, np.random.default_rng(7), four_bit=True, group_size=32)
    r.relative[1, 9] = 0x7F  # row 1, columns 288-319: the second group of 256
    rows = r.rows_of()
    assert np.isnan(rows[1, 256:]).all() and np.isfinite(rows[1, :256]).all() and np.isfinite(rows[0]).all()


def test_embedding_is_the_rows_rounded_to_bf16():
    r = o.random_rotated(9, 768, np.random.default_rng(8))
    ids = np.array([4, 0, 8, 4], np.int32)
    want = o.from_bf16(o.to_bf16(r.rows_of()[ids]))
    assert np.array_equal(r.embedding(ids), want)
    assert np.array_equal(r.rows_of(4, 1), r.rows_of()[4:5])  # a later row alone is the same row
    with pytest.raises(ValueError, match="token id 9 outside the table"):
        r.embedding([1, 9])
