"""The Q8_0 embedding gather on the GPU: bit-exact against the oracle, F32 and
BF16 outputs, every code and scale class, ids refused by the reference, rows
of an odd number of blocks (2-byte aligned) and tables at a 2-byte offset.

The reference has no GPU test of this gather (SmallOpsTests covers F32 tables
only, OpsComparisonCoverageTests.scala:102-123), and its gguf-py golden for
Q8_0 decoding is a Git LFS pointer in the reference checkout; the oracle's
decode is pinned by closed form instead (tests/test_oracle_pins.py)."""

import numpy as np
import pytest
import torch

from drift_amd import ops as d
from oracle import oracle as o
from drift_amd import _lib
from tests.helpers import DEV, assert_bits, dev_i32, host_bits, host_f32, step

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hip():
    return d.HipOps()


def table_on_device(table, cols):
    return d.Q8_0Table(torch.from_numpy(np.ascontiguousarray(table)).to(DEV), cols)


@pytest.mark.parametrize("vocab,cols,count", [(2048, 4096, 300), (100, 32, 50), (300, 96, 77), (64, 8192, 9),
                                              (50, 4160, 13), (10, 256, 1), (40, 8192 + 96, 70)])
def test_gather_matches_oracle_bit_for_bit(hip, vocab, cols, count):
    rng = np.random.default_rng(vocab + cols)
    table = o.q8_0_table(vocab, cols, rng)
    ids = rng.integers(0, vocab, count).astype(np.int32)
    dt = table_on_device(table, cols)
    want = o.embedding_q8_0(table, vocab, cols, ids)
    step(f"Q8_0 gather f32 vocab {vocab} cols {cols} count {count}")
    out = torch.empty((count, cols), dtype=torch.float32, device=DEV)
    hip.embedding(dt, dev_i32(ids), out)
    assert_bits(want.view(np.uint32), host_f32(out).view(np.uint32), what="f32")
    step(f"Q8_0 gather bf16 vocab {vocab} cols {cols} count {count}")
    outb = torch.empty((count, cols), dtype=torch.bfloat16, device=DEV)
    hip.embedding(dt, dev_i32(ids), outb)
    assert_bits(o.to_bf16(want), host_bits(outb), what="bf16")


def test_every_code_and_scale_class(hip):
    # all 256 codes against zero, subnormal, normal, negative, largest,
    # infinite and NaN scales
    scales = np.array([0.0, -0.0, 2 ** -24, 3 * 2 ** -24, 6.1e-5, 1e-3, 0.0123, -0.5, 1.0, 65504.0, -65504.0,
                       np.inf, -np.inf], np.float16)
    scale_bits = np.concatenate([scales.view(np.uint16), np.array([0x7E00, 0xFE01, 0x7C01], np.uint16)])
    codes = np.arange(-128, 128, dtype=np.int32).astype(np.int8).view(np.uint8).reshape(8, 32)
    rows = []
    for bits in scale_bits:
        blocks = [np.concatenate([np.array([bits], np.uint16).view(np.uint8), c]) for c in codes]
        rows.append(np.concatenate(blocks))
    table = np.stack(rows)
    vocab, cols = table.shape[0], 256
    ids = np.arange(vocab, dtype=np.int32)[::-1].copy()
    want = o.embedding_q8_0(table, vocab, cols, ids)
    dt = table_on_device(table, cols)
    step("Q8_0 gather, every code and scale class")
    out = torch.empty((vocab, cols), dtype=torch.float32, device=DEV)
    hip.embedding(dt, dev_i32(ids), out)
    assert_bits(want.view(np.uint32), host_f32(out).view(np.uint32), what="f32 classes")
    outb = torch.empty((vocab, cols), dtype=torch.bfloat16, device=DEV)
    hip.embedding(dt, dev_i32(ids), outb)
    assert_bits(o.to_bf16(want), host_bits(outb), what="bf16 classes")


def test_ids_outside_the_table(hip):
    # the CPU refuses them (ops/CpuLinear.scala:20-23); the kernel writes a
    # zero row and raises the flag
    rng = np.random.default_rng(7)
    table = o.q8_0_table(20, 128, rng)
    ids = np.array([3, -1, 19, 20, 5, 2 ** 31 - 1], np.int32)
    flag = torch.zeros(1, dtype=torch.int32, device=DEV)
    out = torch.full((6, 128), 7.0, dtype=torch.float32, device=DEV)
    step("Q8_0 gather, ids outside the table")
    hip.embedding(table_on_device(table, 128), dev_i32(ids), out, badId=flag)
    got = host_f32(out)
    assert int(flag.item()) == 1
    assert np.all(got[[1, 3, 5]] == 0)
    good = np.array([0, 2, 4])
    assert np.array_equal(got[good], o.embedding_q8_0(table, 20, 128, ids[good]))
    flag.zero_()
    hip.embedding(table_on_device(table, 128), dev_i32(ids[good]), out[:3], badId=flag)
    assert int(flag.item()) == 0


def test_table_at_a_two_byte_offset(hip):
    # the bytes of a mapped table need not start on a 4-byte boundary
    rng = np.random.default_rng(11)
    vocab, cols = 97, 4096
    table = o.q8_0_table(vocab, cols, rng)
    flat = torch.zeros(table.size + 2, dtype=torch.uint8, device=DEV)
    shifted = flat[2:].view(vocab, -1)
    shifted.copy_(torch.from_numpy(table).to(DEV))
    assert shifted.data_ptr() % 4 == 2
    ids = rng.integers(0, vocab, 200).astype(np.int32)
    want = o.embedding_q8_0(table, vocab, cols, ids)
    step("Q8_0 gather, table at a 2-byte offset")
    outb = torch.empty((200, cols), dtype=torch.bfloat16, device=DEV)
    hip.embedding(d.Q8_0Table(shifted, cols), dev_i32(ids), outb)
    assert_bits(o.to_bf16(want), host_bits(outb), what="bf16 shifted table")


def test_table_at_an_odd_address_is_refused(hip):
    flat = torch.zeros(34 * 4 + 1, dtype=torch.uint8, device=DEV)
    out = torch.empty((1, 32), dtype=torch.float32, device=DEV)
    with pytest.raises(_lib.HipError, match="2-byte aligned"):
        hip.embedding(d.Q8_0Table(flat[1:].view(4, 34), 32), dev_i32(np.zeros(1, np.int32)), out)


def test_outputs_past_two_to_the_31_values(hip):
    # 525,313 ids of 4096 values: the output's last rows lie past 2^31 values
    # (4.3 GB of BF16), so its offsets need 64 bits; sampled rows checked
    vocab, cols = 1000, 4096
    count = (1 << 31) // cols + 1025
    rng = np.random.default_rng(77)
    table = o.q8_0_table(vocab, cols, rng)
    ids = rng.integers(0, vocab, count).astype(np.int32)
    step(f"Q8_0 gather of {count} ids x {cols} to BF16 (past 2^31 output values)")
    out = torch.empty((count, cols), dtype=torch.bfloat16, device=DEV)
    hip.embedding(table_on_device(table, cols), dev_i32(ids), out)
    rows = np.array([0, 1, count // 2, (1 << 31) // cols - 1, (1 << 31) // cols, count - 2, count - 1])
    got = host_bits(out[torch.from_numpy(rows).to(DEV)])
    del out
    assert_bits(o.embedding_q8_0_bf16(table, vocab, cols, ids[rows]), got, what="rows past 2^31 values")
