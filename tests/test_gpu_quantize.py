"""The int8 side output on the GPU (the runner's quantize_x form,
kernels/quantize.h:10-25).

- drift_quantize_x is bit-exact against the oracle, F32 and BF16 inputs,
  on the chunked path and on the one-value-per-lane path that unaligned
  inputs or codes take.
- The side output the norms and `gated` write equals quantize_x over what
  they wrote, bit for bit, on the fused path and on the fallback (a
  quantize_x launch after the write): the reference's own bar
  (gpuTest/.../FusedOpsTests.scala:96-176).
- Through HipOps: once an int8 product has quantized its input, a norm's or
  gated's F32 output is quantized as it is written and an int8 product reads
  that instead of quantizing again (ops/HipBase.scala:156-214,
  ops/HipLinear.scala:142-143)."""

import ctypes

import numpy as np
import pytest
import torch

from drift_amd import _lib
from drift_amd import ops as d
from oracle import oracle as o
from tests.helpers import DEV, assert_bits, dev_bf16, dev_f32, gaussian, host_bits, host_f32, step

pytestmark = pytest.mark.gpu


def stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


class Side:
    """Device buffers for the side output of n values; `shift` moves the codes
    off their alignment (one byte) to force the one-value-per-lane path."""

    def __init__(self, n, shift=0):
        self.raw = torch.full((n + 16,), 0x55, dtype=torch.int8, device=DEV)
        self.xq = self.raw[shift:shift + n]
        self.xd = torch.full((n // 32,), 7.0, dtype=torch.float32, device=DEV)
        self.xs = torch.full((n // 32,), 7.0, dtype=torch.float32, device=DEV)

    def args(self):
        return ptr(self.xq), ptr(self.xd), ptr(self.xs)

    def check(self, values, what):
        """Equal, bit for bit, to the oracle's quantize_x of `values` (F32)."""
        xq, xd, xs = o.quantize_x(values)
        torch.cuda.synchronize()
        assert_bits(xq.view(np.uint8), self.xq.cpu().numpy().view(np.uint8), what=f"{what} codes")
        assert_bits(xd.view(np.uint32), host_f32(self.xd).view(np.uint32), what=f"{what} scales")
        assert_bits(xs.view(np.uint32), host_f32(self.xs).view(np.uint32), what=f"{what} sums")


def awkward_blocks(blocks, seed):
    """Blocks of mixed magnitude, with a zero block, a block of ties (xd a
    power of two) and a block holding NaNs."""
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((blocks, 32)) * 10.0 ** rng.uniform(-3, 3, (blocks, 1))).astype(np.float32)
    if blocks >= 4:
        x[1] = 0
        x[2] = np.concatenate([[127 / 16, -0.5 / 16], (np.arange(1, 31) + 0.5) / 16])
        x[3, [0, 7]] = np.nan
    return x.ravel()


@pytest.mark.parametrize("blocks", [1, 7, 4099])
@pytest.mark.parametrize("shift", [(0, 0), (1, 0), (0, 1)], ids=["aligned", "x_offset", "codes_offset"])
def test_quantize_x_f32(blocks, shift):
    x = awkward_blocks(blocks, blocks)
    step(f"quantize_x f32 {blocks} blocks, offsets {shift}")
    flat = torch.zeros(x.size + 4, dtype=torch.float32, device=DEV)
    flat[shift[0]:shift[0] + x.size] = dev_f32(x)
    side = Side(x.size, shift[1])
    _lib.call("drift_quantize_x_f32", ptr(flat[shift[0]:]), *side.args(), blocks, stream())
    side.check(x, "quantize_x f32")


@pytest.mark.parametrize("blocks", [1, 5, 4099])
@pytest.mark.parametrize("shift", [(0, 0), (1, 0), (0, 1)], ids=["aligned", "x_offset", "codes_offset"])
def test_quantize_x_bf16(blocks, shift):
    bits = o.to_bf16(awkward_blocks(blocks, 100 + blocks))
    step(f"quantize_x bf16 {blocks} blocks, offsets {shift}")
    flat = torch.zeros(bits.size + 8, dtype=torch.bfloat16, device=DEV)
    flat[shift[0]:shift[0] + bits.size] = dev_bf16(bits)
    side = Side(bits.size, shift[1])
    _lib.call("drift_quantize_x_bf16", ptr(flat[shift[0]:]), *side.args(), blocks, stream())
    side.check(o.from_bf16(bits), "quantize_x bf16")


def written(out):
    """What out holds, as F32."""
    return host_f32(out) if out.dtype == torch.float32 else o.from_bf16(host_bits(out))


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("rows,cols", [(1, 4096), (3, 2048), (64, 4096), (5, 96), (2, 8192), (1000, 64)])
@pytest.mark.parametrize("residual", [False, True])
def test_rms_norm_side_output(dtype, rows, cols, residual):
    x = gaussian(rows * cols, (rows, cols), 2.0)
    y = gaussian(rows + cols, (rows, cols), 1.0) if residual else None
    w = (1 + 0.1 * gaussian(7, cols)).astype(np.float32)
    make = dev_f32 if dtype == "f32" else (lambda a: dev_bf16(o.to_bf16(a)))
    for path in ("fused", "unaligned out", "unaligned codes"):
        step(f"rmsNorm {dtype} [{rows},{cols}] residual {residual}, side output {path}")
        xd = make(x)
        yd = None if y is None else make(y)
        flat = torch.empty(rows * cols + 8, dtype=xd.dtype, device=DEV)
        out = (flat[1:1 + rows * cols] if path == "unaligned out" else flat[:rows * cols]).view(rows, cols)
        side = Side(rows * cols, 1 if path == "unaligned codes" else 0)
        _lib.call(f"drift_rms_norm_{dtype}", ptr(xd), ptr(yd), ptr(dev_f32(w)), ptr(out), rows, cols, 1e-6, 0.0, 1,
                  *side.args(), stream())
        side.check(written(out), f"rmsNorm {dtype} {path}")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("n", [32, 14336, 8 * 14336, 64 * 14336])
@pytest.mark.parametrize("kind", [0, 1])
def test_gated_side_output(dtype, n, kind):
    g = gaussian(n + kind, n, 2.0)
    u = gaussian(n + 9, n, 1.0)
    make = dev_f32 if dtype == "f32" else (lambda a: dev_bf16(o.to_bf16(a)))
    for path in ("fused", "in place", "unaligned codes"):
        step(f"gated {dtype} kind {kind} n {n}, side output {path}")
        gd, ud = make(g), make(u)
        out = gd if path == "in place" else torch.empty_like(gd)
        side = Side(n, 1 if path == "unaligned codes" else 0)
        _lib.call(f"drift_gated_{dtype}", ptr(gd), ptr(ud), ptr(out), n, kind, *side.args(), stream())
        side.check(written(out), f"gated {dtype} {path}")


# ---------------------------------------------------------------- through HipOps

HIDDEN = 2048


def same(fused, separate, what):
    torch.cuda.synchronize()
    for name, a, b in zip(("codes", "scales", "sums"), fused, separate):
        assert torch.equal(a.view(torch.int8) if a.dtype == torch.int8 else a.view(torch.int32),
                           b.view(torch.int8) if b.dtype == torch.int8 else b.view(torch.int32)), f"{what} {name}"


@pytest.mark.parametrize("t", [1, 3])
def test_products_read_what_the_writer_quantized(t):
    # FusedOpsTests.scala:96-176 without the product itself: the quantized
    # input an int8 product would read of a norm's (or gated's) output equals
    # quantize_x of a copy of it
    hip = d.HipOps()
    norm = dev_f32(1 + 0.1 * gaussian(3, HIDDEN))
    step(f"HipOps side output flow, {t} rows")
    assert hip.quantizedInput(dev_f32(gaussian(4, (t, HIDDEN))), t, HIDDEN) is None
    hip.productInput(dev_f32(gaussian(4, (t, HIDDEN))), t, HIDDEN)  # a first product quantizes x itself
    assert hip.quantizesX

    def check(label, out, k):
        fused = hip.quantizedInput(out, out.numel() // k, k)
        assert fused is not None, f"{label}: not quantized as written"
        copy = out.clone()
        hip.wrote()
        assert hip.quantizedInput(out, out.numel() // k, k) is None
        separate = hip.productInput(copy, copy.numel() // k, k)
        same(fused, separate, label)
        side = o.quantize_x(host_f32(out))
        assert np.array_equal(side[0], fused[0].cpu().numpy()), label

    out = torch.empty((t, HIDDEN), dtype=torch.float32, device=DEV)
    hip.rmsNorm(dev_f32(gaussian(5, (t, HIDDEN))), norm, 1e-6, 0.0, out)
    check(f"rmsNorm, {t} rows", out, HIDDEN)
    out = torch.empty((t, HIDDEN), dtype=torch.float32, device=DEV)
    hip.addRmsNorm(dev_f32(gaussian(6, (t, HIDDEN))), dev_f32(gaussian(7, (t, HIDDEN))), d.RowNorm(norm, 1e-6, 0.0, out))
    check(f"addRmsNorm, {t} rows", out, HIDDEN)
    out = torch.empty((t, 2 * HIDDEN), dtype=torch.float32, device=DEV)
    hip.gated(d.Activation.Sigmoid, dev_f32(gaussian(11, (t, 2 * HIDDEN))), dev_f32(gaussian(12, (t, 2 * HIDDEN))),
              out)
    check(f"gated, {t} rows", out, 2 * HIDDEN)
    # BF16 outputs, as the reference's F32-only rule has it, are not
    outb = torch.empty((t, HIDDEN), dtype=torch.bfloat16, device=DEV)
    hip.rmsNorm(dev_bf16(o.to_bf16(gaussian(5, (t, HIDDEN)))), norm, 1e-6, 0.0, outb)
    assert hip.quantizedInput(outb, t, HIDDEN) is None
