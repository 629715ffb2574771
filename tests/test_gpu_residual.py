"""The gated residuals and per-row modulation on the GPU
(ops/CpuElementwise.scala:40-85): gatedAdd (one gate vector, or per-sample
gates), modulateChunks, gatedAddChunk and rowGatedAdd, F32 and BF16,
bit-exact against the oracle. Each value is computed in double and rounded
once, as the CPU reference does, so there is no tolerance to allow.

Shapes cover the chunked path (rows of whole 16-byte chunks), the
one-value-per-thread path (rows that are not, or unaligned tensors), in
place, and the Video DiT block's [65520, 3072] checked on sampled rows."""

import numpy as np
import pytest
import torch

from drift_amd import ops as d
from oracle import oracle as o
from tests.helpers import DEV, assert_bits, dev_bf16, dev_f32, gaussian, host_bits, host_f32, step

pytestmark = pytest.mark.gpu

SHAPES = [(1, 8), (3, 3072), (7, 96), (5, 100), (64, 128), (2, 4104), (33, 12)]


@pytest.fixture(scope="module")
def hip():
    return d.HipOps()


def device(dtype, a, offset=False):
    """a on the device as `dtype`; with offset, one element past an aligned
    start, so the tensor is not 16-byte aligned."""
    t = dev_f32(a) if dtype == "f32" else dev_bf16(o.to_bf16(a))
    if not offset:
        return t
    flat = torch.empty(t.numel() + 1, dtype=t.dtype, device=DEV)
    view = flat[1:].view(t.shape)
    view.copy_(t)
    return view


def seen(dtype, a):
    """a as the kernel reads it (bf16 inputs rounded)."""
    return a if dtype == "f32" else o.from_bf16(o.to_bf16(a))


def check(dtype, expected_f32, got, what):
    if dtype == "f32":
        assert_bits(np.asarray(expected_f32, np.float32).view(np.uint32), host_f32(got).view(np.uint32), what=what)
    else:
        assert_bits(o.to_bf16(expected_f32), host_bits(got), what=what)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("offset", [False, True])
def test_gated_add(hip, dtype, shape, offset):
    rows, cols = shape
    x, y, gate = gaussian(1, shape, 2.0), gaussian(2, shape), gaussian(3, cols, 0.5)
    step(f"gatedAdd {dtype} {shape} offset {offset}")
    xd, yd = device(dtype, x, offset), device(dtype, y)
    hip.gatedAdd(xd, yd, dev_f32(gate))
    check(dtype, o.gated_add(seen(dtype, x), seen(dtype, y), gate), xd, f"gatedAdd {dtype} {shape}")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("rows,per", [(10, 4), (64, 32), (7, 7)])
def test_gated_add_per_sample(hip, dtype, rows, per):
    cols = 3072
    samples = -(-rows // per)
    x, y, gates = gaussian(4, (rows, cols), 2.0), gaussian(5, (rows, cols)), gaussian(6, (samples, cols), 0.5)
    step(f"gatedAdd {dtype} [{rows},{cols}] per-sample gates, {per} rows per sample")
    xd = device(dtype, x)
    hip.gatedAdd(xd, device(dtype, y), dev_f32(gates), rowsPerSample=per)
    check(dtype, o.gated_add(seen(dtype, x), seen(dtype, y), gates, rows_per_sample=per), xd, "gatedAdd samples")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("chunks,shift,scale", [(6, 0, 1), (6, 3, 4), (2, 1, 0)])
def test_modulate_chunks(hip, dtype, shape, chunks, shift, scale):
    rows, channels = shape
    x, table = gaussian(7, shape, 3.0), gaussian(8, (rows, chunks * channels), 0.3)
    want = o.modulate_chunks(seen(dtype, x), table, shift, scale)
    step(f"modulateChunks {dtype} {shape} chunks {chunks} shift {shift} scale {scale}")
    out = torch.empty(shape, dtype=torch.float32 if dtype == "f32" else torch.bfloat16, device=DEV)
    hip.modulateChunks(device(dtype, x), dev_f32(table), shift, scale, out)
    check(dtype, want, out, f"modulateChunks {dtype} {shape}")
    step(f"modulateChunks {dtype} {shape} in place")
    xd = device(dtype, x, offset=True)
    hip.modulateChunks(xd, dev_f32(table), shift, scale, xd)
    check(dtype, want, xd, f"modulateChunks {dtype} {shape} in place")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("gate", [2, 5])
def test_gated_add_chunk(hip, dtype, shape, gate):
    rows, channels = shape
    x, y, table = gaussian(9, shape, 2.0), gaussian(10, shape), gaussian(11, (rows, 6 * channels), 0.5)
    step(f"gatedAddChunk {dtype} {shape} gate {gate}")
    xd = device(dtype, x)
    hip.gatedAddChunk(xd, device(dtype, y), dev_f32(table), gate)
    check(dtype, o.gated_add_chunk(seen(dtype, x), seen(dtype, y), table, gate), xd, f"gatedAddChunk {dtype}")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("offset", [False, True])
def test_row_gated_add(hip, dtype, shape, offset):
    rows, cols = shape
    x, y, gate = gaussian(12, shape, 2.0), gaussian(13, shape), gaussian(14, rows, 0.5)
    step(f"rowGatedAdd {dtype} {shape} offset {offset}")
    xd = device(dtype, x, offset)
    hip.rowGatedAdd(xd, device(dtype, y), dev_f32(gate))
    check(dtype, o.row_gated_add(seen(dtype, x), seen(dtype, y), gate), xd, f"rowGatedAdd {dtype} {shape}")


def test_the_video_block_shapes(hip):
    # x [2 x 32760, 3072] bf16: gated residual with per-sample gates, and
    # per-row modulation with a [rows, 6 x 3072] table; sampled rows checked
    rows, cols, per = 65520, 3072, 32760
    g = torch.Generator(device=DEV)
    g.manual_seed(21)
    x = torch.randn((rows, cols), generator=g, device=DEV).to(torch.bfloat16)
    y = torch.randn((rows, cols), generator=g, device=DEV).to(torch.bfloat16)
    gates = (0.5 * torch.randn((2, cols), generator=g, device=DEV)).float()
    table = (0.3 * torch.randn((rows, 6 * cols), generator=g, device=DEV)).float()
    sample = np.concatenate([np.arange(4), [32759, 32760, 32761], np.random.default_rng(3).integers(0, rows, 40),
                             [rows - 1]])
    xs, ys = host_bits(x[sample]), host_bits(y[sample])
    step("gatedAdd bf16 [65520, 3072], two samples")
    hip.gatedAdd(x, y, gates, rowsPerSample=per)
    gate_rows = host_f32(gates)[sample // per]
    want = np.stack([o.gated_add(o.from_bf16(xs[i:i + 1]), o.from_bf16(ys[i:i + 1]), gate_rows[i])[0]
                     for i in range(len(sample))])
    assert_bits(o.to_bf16(want), host_bits(x[sample]), what="C5 gatedAdd")
    step("modulateChunks bf16 [65520, 3072] with a [65520, 18432] table")
    xs = host_bits(x[sample])
    out = torch.empty_like(x)
    hip.modulateChunks(x, table, 3, 4, out)
    want = o.modulate_chunks(o.from_bf16(xs), host_f32(table[sample]), 3, 4)
    assert_bits(o.to_bf16(want), host_bits(out[sample]), what="C5 modulateChunks")
    step("gatedAddChunk bf16 [65520, 3072]")
    hip.gatedAddChunk(x, out, table, 5)
    want = o.gated_add_chunk(o.from_bf16(xs), o.from_bf16(host_bits(out[sample])), host_f32(table[sample]), 5)
    assert_bits(o.to_bf16(want), host_bits(x[sample]), what="C5 gatedAddChunk")
