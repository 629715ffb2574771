"""RMSNorm, LayerNorm, modulate and AdaLN on the GPU against the oracle.

Shapes are the reference's awkward ones (SmallOpsTests.scala:22-29,
HipOpsTests.scala:87-110) plus the decode (C2) and diffusion (C5) widths;
inputs 3 N(0,1) as SmallOpsTests.scala:50-54 draws them."""

import numpy as np
import pytest
import torch

from drift_amd import ops as d
from oracle import oracle as o
from tests.helpers import (DEV, assert_bf16, assert_f32, bf16_input, dev_bf16, dev_f32, gaussian, host_bits,
                           host_f32, step)

pytestmark = pytest.mark.gpu

SHAPES = [(1, 1), (3, 7), (2, 255), (5, 4097), (17, 2560), (1, 2048), (64, 2560), (3, 64), (9, 3072), (2, 8192),
          (1, 16384), (2, 20000)]


@pytest.fixture(scope="module")
def hip():
    return d.HipOps()


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("offset", [0.0, 1.0])
def test_rms_norm_f32(hip, shape, offset):
    step(f"rmsNorm f32 {shape} offset {offset}")
    x = gaussian(1, shape, 3.0)
    w = gaussian(2, shape[-1])
    out = torch.empty(shape, dtype=torch.float32, device=DEV)
    hip.rmsNorm(dev_f32(x), dev_f32(w), 1e-6, offset, out)
    assert_f32(o.rms_norm(x, w, 1e-6, offset), host_f32(out), what=f"rmsNorm {shape}")


@pytest.mark.parametrize("shape", [(1, 4096), (8, 4096), (64, 4096), (3, 7), (5, 4097), (17, 2560), (2, 16384)])
def test_rms_norm_bf16(hip, shape):
    step(f"rmsNorm bf16 {shape}")
    xb = bf16_input(gaussian(3, shape))
    w = (1 + 0.1 * gaussian(4, shape[-1])).astype(np.float32)
    out = torch.empty(shape, dtype=torch.bfloat16, device=DEV)
    hip.rmsNorm(dev_bf16(xb), dev_f32(w), 1e-5, 0.0, out)
    assert_bf16(o.rms_norm_bf16(xb, w, 1e-5), host_bits(out), what=f"rmsNorm bf16 {shape}")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("shape", [(3, 7), (4, 4096), (3, 6144), (2, 16384), (600, 1024)])
def test_add_rms_norm(hip, dtype, shape):
    step(f"addRmsNorm {dtype} {shape}")
    x, y = gaussian(5, shape), gaussian(6, shape)
    w = gaussian(7, shape[-1])
    if dtype == "f32":
        xd, yd = dev_f32(x), dev_f32(y)
        out = torch.empty(shape, dtype=torch.float32, device=DEV)
        hip.addRmsNorm(xd, yd, d.RowNorm(dev_f32(w), 1e-6, 0.0, out))
        summed, want = o.rms_norm(x, w, 1e-6, 0.0, y=y)
        assert np.array_equal(host_f32(xd), summed), "x += y is the F32 sum"
        assert_f32(want, host_f32(out), what="addRmsNorm")
    else:
        xb, yb = bf16_input(x), bf16_input(y)
        xd = dev_bf16(xb)
        out = torch.empty(shape, dtype=torch.bfloat16, device=DEV)
        hip.addRmsNorm(xd, dev_bf16(yb), d.RowNorm(dev_f32(w), 1e-6, 0.0, out))
        summed, want = o.rms_norm_bf16(xb, w, 1e-6, y_bits=yb)
        assert np.array_equal(host_bits(xd), summed), "x += y rounds the F32 sum to bf16"
        assert_bf16(want, host_bits(out), what="addRmsNorm bf16")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("cols", [1, 3, 16, 32])
def test_rms_norm_narrow_rows(hip, dtype, cols):
    # rows of at most 32 values (a pixel's channels; the reference's
    # rms_norm_narrow_f32): a thread per row, the row summed in order, so the
    # result is the oracle's to the last bit; with a residual too
    rows = 70001
    step(f"rmsNorm {dtype} narrow [{rows}, {cols}]")
    x, y = gaussian(21, (rows, cols), 3.0), gaussian(22, (rows, cols))
    w = gaussian(23, cols)
    if dtype == "f32":
        out = torch.empty((rows, cols), dtype=torch.float32, device=DEV)
        hip.rmsNorm(dev_f32(x), dev_f32(w), 1e-6, 0.5, out)
        assert np.array_equal(host_f32(out), o.rms_norm(x, w, 1e-6, 0.5)), "narrow rmsNorm f32"
        xd = dev_f32(x)
        hip.addRmsNorm(xd, dev_f32(y), d.RowNorm(dev_f32(w), 1e-6, 0.0, out))
        summed, want = o.rms_norm(x, w, 1e-6, 0.0, y=y)
        assert np.array_equal(host_f32(xd), summed) and np.array_equal(host_f32(out), want), "narrow addRmsNorm"
    else:
        xb, yb = bf16_input(x), bf16_input(y)
        out = torch.empty((rows, cols), dtype=torch.bfloat16, device=DEV)
        hip.rmsNorm(dev_bf16(xb), dev_f32(w), 1e-6, 0.0, out)
        assert np.array_equal(host_bits(out), o.rms_norm_bf16(xb, w, 1e-6)), "narrow rmsNorm bf16"


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("cols", [1024, 2048, 4096, 5120, 12288, 16384, 32768])
def test_rms_norm_does_not_depend_on_the_batch(hip, dtype, cols):
    # a row normed alone (a decode step's token) and inside a prefill batch
    # gives the same bits (ops/HipNormalisation.scala:82-88 asks this of the
    # reference's kernel); a few rows take the 8- and 16-wave groups, a batch
    # the 4-wave group
    rows = 2048
    step(f"rmsNorm {dtype} [{rows}, {cols}] against its rows one at a time")
    x = gaussian(31, (rows, cols), 2.0)
    w = (1 + 0.1 * gaussian(32, cols)).astype(np.float32)
    if dtype == "f32":
        xs, tt, host = dev_f32(x), torch.float32, host_f32
    else:
        xs, tt, host = dev_bf16(bf16_input(x)), torch.bfloat16, host_bits
    batch = torch.empty((rows, cols), dtype=tt, device=DEV)
    hip.rmsNorm(xs, dev_f32(w), 1e-6, 0.0, batch)
    for r in (0, 1, 777, rows - 1):
        alone = torch.empty((1, cols), dtype=tt, device=DEV)
        hip.rmsNorm(xs[r:r + 1], dev_f32(w), 1e-6, 0.0, alone)
        got, want = host(alone)[0], host(batch)[r]
        assert np.array_equal(got.view(np.uint8), want.view(np.uint8)), f"row {r}"
    few = torch.empty((7, cols), dtype=tt, device=DEV)
    hip.rmsNorm(xs[100:107], dev_f32(w), 1e-6, 0.0, few)
    assert np.array_equal(host(few).view(np.uint8), host(batch)[100:107].view(np.uint8)), "rows 100-106"


# (rows, groups, width) of the group norm, one case for each way the library
# splits a row: a thread per narrow row (<= 32 values), the scalar path
# (widths not whole 16-byte chunks), a wave or a 4-wave group per row in a
# batch, and the 8- or 16-wave group a few long rows take
GROUP_SHAPES = [(300, 2, 16), (41, 3, 3), (9, 3, 37), (64, 4, 512), (33, 2, 4096), (1, 2, 4096), (2, 3, 8192),
                (3, 4, 2560)]


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("rows,groups,width", GROUP_SHAPES)
def test_group_rms_norm(hip, dtype, rows, groups, width):
    # groupRmsNorm (ops/HipNormalisation.scala:133-158): rms_norm over rows x
    # groups rows of `width`, row r weighted by weight row r % groups
    step(f"groupRmsNorm {dtype} [{rows}, {groups} x {width}]")
    x = gaussian(41, (rows, groups * width), 2.0)
    w = (1 + 0.1 * gaussian(42, groups * width)).astype(np.float32)
    want_rows = (rows * groups, width)
    if dtype == "f32":
        out = torch.empty((rows, groups * width), dtype=torch.float32, device=DEV)
        hip.groupRmsNorm(dev_f32(x), dev_f32(w), groups, 1e-6, 0.25, out)
        want = o.rms_norm(x.reshape(want_rows), w.reshape(groups, width), 1e-6, 0.25, weight_rows=groups)
        assert_f32(want.reshape(rows, -1), host_f32(out), what="groupRmsNorm")
    else:
        xb = bf16_input(x)
        out = torch.empty((rows, groups * width), dtype=torch.bfloat16, device=DEV)
        hip.groupRmsNorm(dev_bf16(xb), dev_f32(w), groups, 1e-5, 0.0, out)
        want = o.rms_norm_bf16(xb.reshape(want_rows), w.reshape(groups, width), 1e-5, weight_rows=groups)
        assert_bf16(want.reshape(rows, -1), host_bits(out), what="groupRmsNorm bf16")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("rows,groups,width", GROUP_SHAPES)
def test_weight_rows_with_a_residual(hip, dtype, rows, groups, width):
    # rms_norm's weight_rows with y through the C ABI: x += y written back,
    # then row r of the sum normed with weight row r % weight_rows
    step(f"rms_norm {dtype} weight_rows {groups} with y, [{rows * groups}, {width}]")
    shape = (rows * groups, width)
    x, y = gaussian(43, shape), gaussian(44, shape)
    w = gaussian(45, (groups, width))
    entry = f"drift_rms_norm_{dtype}"
    wd = dev_f32(w)  # every device tensor held until the launch has run
    if dtype == "f32":
        xd, yd = dev_f32(x), dev_f32(y)
        out = torch.empty(shape, dtype=torch.float32, device=DEV)
        hip._launch(entry, d._ptr(xd), d._ptr(yd), d._ptr(wd), d._ptr(out), shape[0], width, 1e-6, 0.0, groups,
                    None, None, None)
        summed, want = o.rms_norm(x, w, 1e-6, 0.0, y=y, weight_rows=groups)
        assert np.array_equal(host_f32(xd), summed), "x += y is the F32 sum"
        assert_f32(want, host_f32(out), what="weight_rows with y")
    else:
        xb, yb = bf16_input(x), bf16_input(y)
        xd, yd = dev_bf16(xb), dev_bf16(yb)
        out = torch.empty(shape, dtype=torch.bfloat16, device=DEV)
        hip._launch(entry, d._ptr(xd), d._ptr(yd), d._ptr(wd), d._ptr(out), shape[0], width, 1e-6, 0.0, groups,
                    None, None, None)
        summed, want = o.rms_norm_bf16(xb, w, 1e-6, y_bits=yb, weight_rows=groups)
        assert np.array_equal(host_bits(xd), summed), "x += y rounds the F32 sum to bf16"
        assert_bf16(want, host_bits(out), what="weight_rows with y, bf16")


def test_rms_norm_in_place_and_zero_rows(hip):
    step("rmsNorm in place, zero row")
    x = gaussian(8, (6, 512))
    x[2] = 0
    w = gaussian(9, 512)
    xd = dev_f32(x)
    hip.rmsNorm(xd, dev_f32(w), 1e-6, 0.0, xd)
    got = host_f32(xd)
    assert_f32(o.rms_norm(x, w, 1e-6), got, what="in place")
    assert np.all(got[2] == 0)


@pytest.mark.parametrize("shape", [(1, 1), (3, 7), (2, 255), (5, 4097), (17, 2560), (1, 2048), (4, 3072)])
@pytest.mark.parametrize("affine", [(False, False), (True, False), (False, True), (True, True)])
def test_layer_norm_f32(hip, shape, affine):
    step(f"layerNorm f32 {shape} {affine}")
    x = gaussian(1, shape, 3.0)
    w = gaussian(2, shape[-1], 3.0) if affine[0] else None
    b = gaussian(3, shape[-1], 3.0) if affine[1] else None
    out = torch.empty(shape, dtype=torch.float32, device=DEV)
    hip.layerNorm(dev_f32(x), None if w is None else dev_f32(w), None if b is None else dev_f32(b), 1e-5, out)
    assert_f32(o.layer_norm(x, w, b, 1e-5), host_f32(out), what=f"layerNorm {shape}")


@pytest.mark.parametrize("shape", [(5, 64), (3, 6144), (3, 7), (2, 4097)])
def test_modulate_f32(hip, shape):
    # SmallOpsTests.scala:242-256 shapes
    step(f"modulate f32 {shape}")
    x = gaussian(1, shape, 3.0)
    s, sh = gaussian(2, shape[-1], 3.0), gaussian(3, shape[-1], 3.0)
    out = torch.empty(shape, dtype=torch.float32, device=DEV)
    hip.modulate(dev_f32(x), dev_f32(s), dev_f32(sh), out)
    assert_f32(o.modulate(x, s, sh), host_f32(out), what=f"modulate {shape}")


@pytest.mark.parametrize("rows,cols,samples", [(2 * 60, 3072, 2), (7, 64, 1), (3 * 17, 1536, 3), (10, 4097, 2),
                                               (6, 8, 3), (4, 12288, 2)])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_layer_norm_modulate(hip, rows, cols, samples, dtype):
    step(f"layerNormModulate {dtype} [{rows}, {cols}] x {samples} samples")
    per = -(-rows // samples)
    x = gaussian(11, (rows, cols))
    s = (0.1 * gaussian(12, (samples, cols))).astype(np.float32)
    sh = (0.1 * gaussian(13, (samples, cols))).astype(np.float32)
    if dtype == "f32":
        out = torch.empty((rows, cols), dtype=torch.float32, device=DEV)
        hip.layerNormModulate(dev_f32(x), dev_f32(s), dev_f32(sh), 1e-6, out, per)
        assert_f32(o.layer_norm_modulate(x, s, sh, per, 1e-6), host_f32(out), what="AdaLN f32")
    else:
        xb = bf16_input(x)
        out = torch.empty((rows, cols), dtype=torch.bfloat16, device=DEV)
        hip.layerNormModulate(dev_bf16(xb), dev_f32(s), dev_f32(sh), 1e-6, out, per)
        assert_bf16(o.layer_norm_modulate_bf16(xb, s, sh, per, 1e-6), host_bits(out), what="AdaLN bf16")


def test_layer_norm_modulate_in_place_bf16(hip):
    step("layerNormModulate bf16 in place")
    x = gaussian(14, (8, 3072))
    s = (0.1 * gaussian(15, (2, 3072))).astype(np.float32)
    sh = (0.1 * gaussian(16, (2, 3072))).astype(np.float32)
    xb = bf16_input(x)
    xd = dev_bf16(xb)
    hip.layerNormModulate(xd, dev_f32(s), dev_f32(sh), 1e-6, xd, 4)
    assert_bf16(o.layer_norm_modulate_bf16(xb, s, sh, 4, 1e-6), host_bits(xd), what="AdaLN in place")
