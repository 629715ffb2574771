"""ConvRot's rotated linears on the GPU against the oracle (ops/CpuBase.scala:
40-81, tensor/ConvRot.scala:20-50): the embedding gather to F32 and BF16
(ops/HipLinear.scala:54-92) and the whole-weight decode to BF16
(ops/HipBase.scala:276-311), int8_tensorwise and asym_w4a8_int8. Bit-exact:
the F32 gather is the BF16 value widened, as the CPU gathers; NaN outputs
(from a NaN relative scale) are compared as NaN."""

import numpy as np
import pytest
import torch

from drift_amd import ops as d
from oracle import oracle as o
from tests.helpers import DEV, assert_bits, dev_i32, host_bits, host_f32, step

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hip():
    return d.HipOps()


def device_table(hip, r: o.Rotated, offset: int = 0) -> d.RotatedTable:
    """The oracle's weight on the device, its codes `offset` bytes past a
    256-byte boundary."""
    raw = r.codes.reshape(-1)
    flat = torch.zeros(raw.size + offset, dtype=torch.int8, device=DEV)
    flat[offset:] = torch.from_numpy(raw.view(np.int8).copy()).to(DEV)
    codes = flat[offset:].view(r.codes.shape)
    levels = None
    if r.codebook is not None:
        levels = d.ConvRotLevels(torch.from_numpy(r.codebook).to(DEV), torch.from_numpy(r.relative).to(DEV),
                                 r.group_size)
    return hip.rotated(codes, d.ConvRotParts(torch.from_numpy(r.scales).to(DEV), levels))


def same_bits(want_bits, got_bits, what):
    """Bit-exact, a NaN matching a NaN."""
    want_bits, got_bits = np.asarray(want_bits).ravel(), np.asarray(got_bits).ravel()
    wide = want_bits.dtype == np.uint32
    exp_mask, man_mask = (0x7F800000, 0x7FFFFF) if wide else (0x7F80, 0x7F)
    nan = ((want_bits & exp_mask) == exp_mask) & ((want_bits & man_mask) != 0)
    got_nan = ((got_bits & exp_mask) == exp_mask) & ((got_bits & man_mask) != 0)
    assert np.array_equal(nan, got_nan), f"{what}: NaNs differ"
    assert_bits(want_bits[~nan], got_bits[~nan], what)


CASES = [
    # (name, four_bit, group_size, one_scale)
    ("int8 row scales", False, 0, False),
    ("int8 one scale", False, 0, True),
    ("4-bit groups of 16", True, 16, False),
    ("4-bit groups of 32", True, 32, False),
    ("4-bit groups of 64", True, 64, False),
    ("4-bit groups of 128", True, 128, False),
    ("4-bit groups of 512", True, 512, False),
]


@pytest.mark.parametrize("name,four_bit,group_size,one_scale", CASES)
@pytest.mark.parametrize("out_type", ["f32", "bf16"])
def test_embedding(hip, name, four_bit, group_size, one_scale, out_type):
    rows, cols = 41, 1024
    r = o.random_rotated(rows, cols, np.random.default_rng(31), four_bit, group_size or 32, one_scale)
    table = device_table(hip, r)
    ids = np.random.default_rng(32).integers(0, rows, 37).astype(np.int32)  # 148 groups: a partial wave
    ids[:3] = [0, rows - 1, 0]
    step(f"rotated embedding {name} -> {out_type}, {ids.size} rows of {cols}")
    want = r.embedding(ids)
    dtype = torch.float32 if out_type == "f32" else torch.bfloat16
    out = torch.empty((ids.size, cols), dtype=dtype, device=DEV)
    hip.embedding(table, dev_i32(ids), out)
    if out_type == "f32":
        same_bits(want.view(np.uint32), host_f32(out).view(np.uint32), f"{name} f32")
    else:
        same_bits(o.to_bf16(want), host_bits(out), f"{name} bf16")


# every case at every shape whose rows its groups divide
DEQUANTIZE_CASES = [case + (shape,) for case in CASES for shape in [(1, 256), (23, 768), (64, 3072)]
                    if not case[1] or shape[1] % case[2] == 0]


@pytest.mark.parametrize("name,four_bit,group_size,one_scale,shape", DEQUANTIZE_CASES,
                         ids=[f"{c[0]} [{c[4][0]},{c[4][1]}]" for c in DEQUANTIZE_CASES])
def test_dequantize(hip, name, four_bit, group_size, one_scale, shape):
    rows, cols = shape
    r = o.random_rotated(rows, cols, np.random.default_rng(41 + cols), four_bit, group_size or 32, one_scale)
    table = device_table(hip, r)
    step(f"rotated dequantize {name} [{rows}, {cols}]")
    out = torch.empty((rows, cols), dtype=torch.bfloat16, device=DEV)
    hip.convert(table, out)
    same_bits(r.dequantize_bf16(), host_bits(out), f"{name} dequantize")


@pytest.mark.parametrize("four_bit", [False, True])
@pytest.mark.parametrize("offset", [1, 4, 8])
def test_codes_at_any_alignment(hip, four_bit, offset):
    rows, cols = 7, 512
    r = o.random_rotated(rows, cols, np.random.default_rng(51 + offset), four_bit, 64)
    table = device_table(hip, r, offset)
    step(f"rotated dequantize, {'4-bit' if four_bit else 'int8'} codes {offset} bytes off 16")
    out = torch.empty((rows, cols), dtype=torch.bfloat16, device=DEV)
    hip.dequantize(table, out)
    same_bits(r.dequantize_bf16(), host_bits(out), f"offset {offset}")
    ids = np.array([6, 1, 3], np.int32)
    got = torch.empty((3, cols), dtype=torch.float32, device=DEV)
    hip.embedding(table, dev_i32(ids), got)
    same_bits(r.embedding(ids).view(np.uint32), host_f32(got).view(np.uint32), f"offset {offset} embedding")


@pytest.mark.parametrize("group_size", [32, 64, 256])
def test_nan_relative_scales_and_codebooks(hip, group_size):
    rows, cols = 6, 512
    r = o.random_rotated(rows, cols, np.random.default_rng(61), True, group_size)
    per_row = cols // group_size
    r.relative[2, 3 * per_row // 16] = 0x7F  # row 2, first group of 256: NaN
    r.relative[5, per_row - 1] = 0xFF  # row 5, second group
    r.relative[4, 0] = 0x00  # a zero relative scale: an infinite entry's level is NaN
    table = device_table(hip, r)
    step("rotated dequantize with NaN relative scales")
    out = torch.empty((rows, cols), dtype=torch.bfloat16, device=DEV)
    hip.dequantize(table, out)
    want = r.dequantize_bf16()
    assert np.isnan(o.from_bf16(want[2, :256])).all() and np.isnan(o.from_bf16(want[5, 256:])).all()
    same_bits(want, host_bits(out), "NaN relative")
    # an infinite codebook entry times a finite scale is infinite, clamped to 127
    r.codebook[3] = np.inf
    r.codebook[9] = np.nan
    table = device_table(hip, r)
    step("rotated dequantize with a non-finite codebook")
    hip.dequantize(table, out)
    same_bits(r.dequantize_bf16(), host_bits(out), "non-finite codebook")


@pytest.mark.parametrize("four_bit,group_size", [(False, 0), (True, 32), (True, 64)])
def test_tiny_row_scales(hip, four_bit, group_size):
    # Row scales down to the float's smallest steps, where the rotation's
    # halves round: a wave holding such a row takes the two roundings, the
    # rest the fma form. Rows of 1,024 columns, four to a wave: rows 0-23
    # tiny, 24 at the boundary 2^-122 and 25 zero (a wave of the fma form),
    # 47 tiny in a wave of ordinary rows. The fma form would differ from
    # the oracle here (3 to 5 rows' BF16 values in each case, checked on the
    # CPU).
    rows, cols = 48, 1024
    rng = np.random.default_rng(95)
    r = o.random_rotated(rows, cols, rng, four_bit, group_size or 32)
    tiny = rows // 2
    r.scales[:tiny] = (rng.uniform(1, 2, tiny) * 2.0 ** rng.integers(-149, -118, tiny)).astype(np.float32)
    r.scales[tiny] = 2.0 ** -122
    r.scales[tiny + 1] = 0.0
    r.scales[-1] = 1e-40
    table = device_table(hip, r)
    step(f"rotated dequantize {'4-bit' if four_bit else 'int8'} with tiny row scales")
    out = torch.empty((rows, cols), dtype=torch.bfloat16, device=DEV)
    hip.dequantize(table, out)
    same_bits(r.dequantize_bf16(), host_bits(out), "tiny scales")
    ids = rng.integers(0, rows, 64).astype(np.int32)
    got = torch.empty((64, cols), dtype=torch.float32, device=DEV)
    hip.embedding(table, dev_i32(ids), got)
    same_bits(r.embedding(ids).view(np.uint32), host_f32(got).view(np.uint32), "tiny scales embedding")


def test_ids_outside_the_weight_give_zero_rows(hip):
    rows, cols = 5, 512
    r = o.random_rotated(rows, cols, np.random.default_rng(71), True, 32)
    table = device_table(hip, r)
    ids = np.array([1, -1, 5, 4, 1 << 30], np.int32)
    bad = torch.zeros(1, dtype=torch.int32, device=DEV)
    out = torch.full((ids.size, cols), 7.0, dtype=torch.float32, device=DEV)
    step("rotated embedding with ids outside the weight")
    hip.embedding(table, dev_i32(ids), out, bad)
    got = host_f32(out)
    assert np.array_equal(got[[0, 3]], r.embedding(ids[[0, 3]]))
    assert not got[[1, 2, 4]].any() and int(bad.item()) == 1


def test_a_large_weight(hip):
    # a DiT linear's shape: [3072, 3072] 4-bit, and 8192 int8 rows of 4096 gathered
    r = o.random_rotated(3072, 3072, np.random.default_rng(81), True, 64)
    table = device_table(hip, r)
    step("rotated dequantize 4-bit [3072, 3072]")
    out = torch.empty((3072, 3072), dtype=torch.bfloat16, device=DEV)
    hip.dequantize(table, out)
    sample = np.random.default_rng(82).choice(3072, 96, replace=False)
    got = host_bits(out).reshape(3072, 3072)
    for row in sample:
        assert_bits(o.to_bf16(r.rows_of(int(row), 1)[0]), got[row], f"row {row}")
    r8 = o.random_rotated(1000, 4096, np.random.default_rng(83))
    table8 = device_table(hip, r8)
    ids = np.random.default_rng(84).integers(0, 1000, 8192).astype(np.int32)
    step("rotated embedding int8 8192 ids of [1000, 4096]")
    out8 = torch.empty((8192, 4096), dtype=torch.bfloat16, device=DEV)
    hip.embedding(table8, dev_i32(ids), out8)
    rows = o.to_bf16(r8.rows_of())
    assert_bits(rows[ids], host_bits(out8), "8192 ids")
    step("rotated dequantize int8 [1000, 4096]")
    whole = torch.empty((1000, 4096), dtype=torch.bfloat16, device=DEV)
    hip.dequantize(table8, whole)
    assert_bits(rows, host_bits(whole), "int8 [1000, 4096]")
