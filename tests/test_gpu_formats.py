"""The embedding gather and the whole-table decode of every storage type the
runner's GPU backend reads (kernels/matvec.hip:942-954: Q4_0, Q5_1, Q8_0,
Q4_K, Q5_K, Q6_K, IQ4_NL, IQ4_XS, ROCmFP4 dual and fast, and the dense F32,
F16, BF16; plus Q4_1 and Q5_0, which the reference decodes on the CPU), on
the GPU against the oracle's decoders. Bit-exact: F32 outputs are the
decoders' float arithmetic, BF16 and F16 its result rounded to nearest even.
Tables are random blocks with finite scales (NaN scales are out: their NaN
bits follow the hardware)."""

import numpy as np
import pytest
import torch

from drift_amd import _lib
from drift_amd import ops as d
from oracle import oracle as o
from tests.helpers import DEV, assert_bits, dev_i32, host_bits, host_f32, step

pytestmark = pytest.mark.gpu

NAMES = sorted(o.FORMATS)


@pytest.fixture(scope="module")
def hip():
    return d.HipOps()


def table_of(name, vocab, cols, seed):
    rng = np.random.default_rng(seed)
    raw = o.quant_table(name, vocab, cols, rng)
    dev = torch.from_numpy(np.ascontiguousarray(raw)).to(DEV)
    return raw, d.StoredTable(dev, d.STORAGE_TYPES[name], cols)


@pytest.mark.parametrize("name", NAMES)
@pytest.mark.parametrize("out_type", ["f32", "bf16"])
def test_embedding_every_storage_type(hip, name, out_type):
    values = d.STORAGE_TYPES[name].values
    cols = 512 if values == 256 else 96 if values == 32 else 40
    vocab = 37
    raw, table = table_of(name, vocab, cols, 11)
    ids = np.random.default_rng(12).integers(0, vocab, 53).astype(np.int32)
    ids[:3] = [0, vocab - 1, 0]
    step(f"embedding {name} -> {out_type}, rows of {cols}")
    want = o.embedding(name, raw, vocab, cols, ids)
    if out_type == "f32":
        out = torch.empty((ids.size, cols), dtype=torch.float32, device=DEV)
        hip.embedding(table, dev_i32(ids), out)
        assert_bits(want.view(np.uint32), host_f32(out).view(np.uint32), what=f"{name} f32")
    else:
        out = torch.empty((ids.size, cols), dtype=torch.bfloat16, device=DEV)
        hip.embedding(table, dev_i32(ids), out)
        assert_bits(o.to_bf16(want), host_bits(out), what=f"{name} bf16")


@pytest.mark.parametrize("name", NAMES)
@pytest.mark.parametrize("out_type", ["bf16", "f16"])
def test_dequantize_every_storage_type(hip, name, out_type):
    values = d.STORAGE_TYPES[name].values
    cols = 768 if values == 256 else 160 if values == 32 else 64
    rows = 29
    raw, table = table_of(name, rows, cols, 21)
    step(f"dequantize {name} -> {out_type} [{rows}, {cols}]")
    want = o.embedding(name, raw, rows, cols, np.arange(rows, dtype=np.int32))
    out = torch.empty((rows, cols), dtype=torch.bfloat16 if out_type == "bf16" else torch.float16, device=DEV)
    hip.dequantize(table, out)
    expected = o.to_bf16(want) if out_type == "bf16" else want.astype(np.float16).view(np.uint16)
    assert_bits(expected, host_bits(out), what=f"{name} dequantize {out_type}")


# every block format: those that decode rows of whole runs staged in LDS
# (Q4_K, Q5_K, IQ4_NL, ROCmFP4), and those that decode them a chunk a thread
# by row
RUN_FORMATS = [n for n in NAMES if d.STORAGE_TYPES[n].values > 1]


@pytest.mark.parametrize("name", RUN_FORMATS)
@pytest.mark.parametrize("cols", [2048, 6144])
def test_rows_of_whole_runs(hip, name, cols):
    # rows of whole runs of 2048 values (8 blocks of 256 or 64 of 32), the
    # table on a 16-byte boundary: the run decoder where the format takes it,
    # for the gather (with ids outside the table: zero rows and the flag) and
    # the whole-table decode
    vocab = 19
    raw, table = table_of(name, vocab, cols, 41 + cols)
    assert table.data.data_ptr() % 16 == 0
    ids = np.random.default_rng(cols).integers(0, vocab, 23).astype(np.int32)
    ids[:2] = [vocab - 1, 0]
    bad_ids = ids.copy()
    bad_ids[[5, 11]] = [-1, vocab]
    step(f"embedding {name} rows of {cols}, ids outside the table")
    want = o.embedding(name, raw, vocab, cols, ids)
    want[[5, 11]] = 0.0
    bad = torch.zeros(1, dtype=torch.int32, device=DEV)
    out = torch.empty((ids.size, cols), dtype=torch.float32, device=DEV)
    hip.embedding(table, dev_i32(bad_ids), out, bad)
    assert_bits(want.view(np.uint32), host_f32(out).view(np.uint32), what=f"{name} f32 rows of {cols}")
    assert int(bad.item()) == 1
    out = torch.empty((ids.size, cols), dtype=torch.bfloat16, device=DEV)
    hip.embedding(table, dev_i32(ids), out)
    want = o.embedding(name, raw, vocab, cols, ids)
    assert_bits(o.to_bf16(want), host_bits(out), what=f"{name} bf16 rows of {cols}")
    step(f"dequantize {name} [{vocab}, {cols}] to bf16 and f16")
    whole = o.embedding(name, raw, vocab, cols, np.arange(vocab, dtype=np.int32))
    for dtype, expected in ((torch.bfloat16, o.to_bf16(whole)), (torch.float16, whole.astype(np.float16).view(np.uint16))):
        out = torch.empty((vocab, cols), dtype=dtype, device=DEV)
        hip.dequantize(table, out)
        assert_bits(expected, host_bits(out), what=f"{name} dequantize {dtype} rows of {cols}")


@pytest.mark.parametrize("name", RUN_FORMATS)
def test_runs_off_a_16_byte_boundary(hip, name):
    # the same rows from a table 8 bytes past a 16-byte boundary: the
    # chunk-a-thread decoder by row, with the same result
    vocab, cols = 7, 2048
    raw, _ = table_of(name, vocab, cols, 77)
    t = d.STORAGE_TYPES[name]
    flat = torch.zeros(raw.size + 8, dtype=torch.uint8, device=DEV)
    flat[8:] = torch.from_numpy(np.ascontiguousarray(raw).reshape(-1)).to(DEV)
    table = d.StoredTable(flat[8:].view(vocab, t.rowBytes(cols)), t, cols)
    assert table.data.data_ptr() % 16 == 8
    ids = np.array([3, 0, 6, 3], np.int32)
    step(f"embedding {name} rows of {cols} from a table 8 bytes off a 16-byte boundary")
    out = torch.empty((ids.size, cols), dtype=torch.float32, device=DEV)
    hip.embedding(table, dev_i32(ids), out)
    want = o.embedding(name, raw, vocab, cols, ids)
    assert_bits(want.view(np.uint32), host_f32(out).view(np.uint32), what=f"{name} f32 off 16")


@pytest.mark.parametrize("name", NAMES)
def test_more_rows_than_a_grid_column(hip, name):
    # 65,543 ids, more rows than the by-row grid's 65,535: the
    # one-dimensional decoders (the one-block-a-half-wave decoder for the
    # 256-value formats), every value of the output against the oracle
    values = d.STORAGE_TYPES[name].values
    cols = 256 if values > 1 else 40
    vocab = 23
    raw, table = table_of(name, vocab, cols, 91)
    ids = np.random.default_rng(92).integers(0, vocab, 65543).astype(np.int32)
    ids[[0, -1]] = [vocab - 1, 0]
    step(f"embedding {name} -> bf16, {ids.size} ids of {cols} values")
    out = torch.empty((ids.size, cols), dtype=torch.bfloat16, device=DEV)
    hip.embedding(table, dev_i32(ids), out)
    rows = o.to_bf16(o.embedding(name, raw, vocab, cols, np.arange(vocab, dtype=np.int32)))
    assert_bits(rows[ids], host_bits(out), what=f"{name} {ids.size} rows")


@pytest.mark.parametrize("name", ["Q4_K", "IQ4_NL", "Q4_0_ROCMFP4_FAST"])
def test_ids_outside_the_table_give_zero_rows(hip, name):
    values = d.STORAGE_TYPES[name].values
    cols = 256 if values == 256 else 64
    raw, table = table_of(name, 5, cols, 3)
    ids = np.array([1, -1, 5, 4], np.int32)
    step(f"embedding {name} with ids outside the table")
    bad = torch.zeros(1, dtype=torch.int32, device=DEV)
    out = torch.empty((4, cols), dtype=torch.float32, device=DEV)
    hip.embedding(table, dev_i32(ids), out, bad)
    got = host_f32(out)
    want = o.embedding(name, raw, 5, cols, ids[[0, 3]])
    assert np.array_equal(got[[0, 3]], want) and not got[[1, 2]].any()
    assert int(bad.item()) == 1


def test_misaligned_tables_are_refused(hip):
    cols = 256
    flat = torch.zeros(144 * 3 + 4, dtype=torch.uint8, device=DEV)
    shifted = d.StoredTable(flat[4:].view(3, 144), d.STORAGE_TYPES["Q4_K"], cols)
    out = torch.empty((1, cols), dtype=torch.float32, device=DEV)
    step("embedding Q4_K from a table 4 bytes off an 8-byte boundary")
    with pytest.raises(_lib.HipError, match="8-byte aligned"):
        hip.embedding(shifted, dev_i32(np.zeros(1, np.int32)), out)


@pytest.mark.parametrize("name", ["F32", "F16", "BF16"])
@pytest.mark.parametrize("cols", [1, 3, 100])
def test_dense_tables_of_any_width(hip, name, cols):
    # gather_rows_f32 (kernels/elementwise.hip:89-93) takes any width; so do
    # the dense types here, through their per-value path
    vocab = 19
    raw, table = table_of(name, vocab, cols, 31 + cols)
    ids = np.random.default_rng(32).integers(-1, vocab + 1, 45).astype(np.int32)
    step(f"embedding {name} rows of {cols}")
    good = (ids >= 0) & (ids < vocab)
    want = np.zeros((ids.size, cols), np.float32)
    want[good] = o.embedding(name, raw, vocab, cols, ids[good])
    out = torch.empty((ids.size, cols), dtype=torch.float32, device=DEV)
    bad = torch.zeros(1, dtype=torch.int32, device=DEV)
    hip.embedding(table, dev_i32(ids), out, bad)
    assert_bits(want.view(np.uint32), host_f32(out).view(np.uint32), what=f"{name} width {cols}")
    assert int(bad.item()) == int((~good).any())
    bf = torch.empty((ids.size, cols), dtype=torch.bfloat16, device=DEV)
    hip.embedding(table, dev_i32(ids), bf)
    assert_bits(o.to_bf16(want), host_bits(bf), what=f"{name} width {cols} bf16")
    dense = torch.empty((vocab, cols), dtype=torch.float16, device=DEV)
    hip.dequantize(table, dense)
    full = o.embedding(name, raw, vocab, cols, np.arange(vocab, dtype=np.int32))
    assert_bits(full.astype(np.float16).view(np.uint16), host_bits(dense), what=f"{name} width {cols} f16")
