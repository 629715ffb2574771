"""Activations, gated activations and conversions on the GPU against the
oracle: every kind on the reference's shapes (SmallOpsTests.scala:90-114),
the tails where the reference's double arithmetic is itself quantized, IEEE
specials, and the decode SwiGLU (C2)."""

import numpy as np
import pytest
import torch

from drift_amd import ops as d
from oracle import oracle as o
from tests.helpers import (DEV, assert_bf16, assert_bits, assert_f32, bf16_input, dev_bf16, dev_f32, gaussian,
                           host_bits, host_f32, step)

pytestmark = pytest.mark.gpu

SHAPES = [(1, 1), (3, 7), (2, 255), (5, 4097), (17, 2560), (1, 2048)]
KINDS = list(d.Activation)
SPECIALS = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-30, -1e-30, 80.0, -80.0, 100.0, -100.0, 3e38, -3e38,
                     1e-40, -1e-40], np.float32)


@pytest.fixture(scope="module")
def hip():
    return d.HipOps()


@pytest.mark.parametrize("kind", KINDS)
def test_activation_f32(hip, kind):
    for shape in SHAPES:
        step(f"activation f32 {kind.name} {shape}")
        x = gaussian(1, shape, 3.0)
        out = torch.empty(shape, dtype=torch.float32, device=DEV)
        hip.activation(kind, dev_f32(x), out)
        assert_f32(o.activation(int(kind), x), host_f32(out), what=f"{kind.name} {shape}")


@pytest.mark.parametrize("kind", KINDS)
def test_activation_bf16(hip, kind):
    for shape in SHAPES + [(64, 3072)]:
        step(f"activation bf16 {kind.name} {shape}")
        xb = bf16_input(gaussian(2, shape, 3.0))
        out = torch.empty(shape, dtype=torch.bfloat16, device=DEV)
        hip.activation(kind, dev_bf16(xb), out)
        assert_bf16(o.activation_bf16(int(kind), xb), host_bits(out), what=f"{kind.name} bf16 {shape}")


@pytest.mark.parametrize("kind", [d.Activation.GeluTanh, d.Activation.GeluErf])
def test_gelu_tails_follow_the_reference(hip, kind):
    # below about -7 the reference's 1 + tanh(u) (1 + erf) is a whole number of
    # 2^-53 steps, and exactly 0 further out
    x = np.linspace(-14, -4, 20001).astype(np.float32)
    step(f"{kind.name} tail f32")
    out = torch.empty_like(dev_f32(x))
    hip.activation(kind, dev_f32(x), out)
    assert_f32(o.activation(int(kind), x), host_f32(out), what=f"{kind.name} tail")
    step(f"{kind.name} tail bf16")
    xb = bf16_input(x)
    outb = torch.empty(x.shape, dtype=torch.bfloat16, device=DEV)
    hip.activation(kind, dev_bf16(xb), outb)
    assert_bf16(o.activation_bf16(int(kind), xb), host_bits(outb), what=f"{kind.name} tail bf16")


@pytest.mark.parametrize("kind", KINDS)
def test_activation_specials_and_scale(hip, kind):
    step(f"activation specials {kind.name}")
    out = torch.empty(SPECIALS.shape, dtype=torch.float32, device=DEV)
    hip.activation(kind, dev_f32(SPECIALS), out)
    assert_f32(o.activation(int(kind), SPECIALS), host_f32(out), what=f"{kind.name} specials")
    # scaledActivation: the scale multiplies the value first (a power of two: exact in float too)
    x = gaussian(3, (4, 100), 3.0)
    hip.scaledActivation(kind, 0.5, dev_f32(x), out2 := torch.empty((4, 100), device=DEV))
    assert_f32(o.activation(int(kind), x, 0.5), host_f32(out2), what=f"{kind.name} scaled")


@pytest.mark.parametrize("kind", KINDS)
def test_gated(hip, kind):
    for shape in SHAPES:
        step(f"gated f32 {kind.name} {shape}")
        g, u = gaussian(1, shape, 3.0), gaussian(2, shape, 3.0)
        out = torch.empty(shape, dtype=torch.float32, device=DEV)
        hip.gated(kind, dev_f32(g), dev_f32(u), out)
        assert_f32(o.gated(int(kind), g, u), host_f32(out), what=f"gated {kind.name} {shape}")
        step(f"gated bf16 {kind.name} {shape}")
        gb, ub = bf16_input(g), bf16_input(u)
        outb = torch.empty(shape, dtype=torch.bfloat16, device=DEV)
        hip.gated(kind, dev_bf16(gb), dev_bf16(ub), outb)
        assert_bf16(o.gated_bf16(int(kind), gb, ub), host_bits(outb), what=f"gated bf16 {kind.name} {shape}")


@pytest.mark.parametrize("batch", [1, 8, 64])
def test_swiglu_decode_shape_in_place(hip, batch):
    # C2: silu(g) * u on gate/up [B, 14336] ~ N(0,1), out aliasing gate as
    # models/DenseDecoder.scala:927 calls it
    step(f"SwiGLU bf16 [{batch}, 14336] in place")
    gb = bf16_input(gaussian(20 + batch, (batch, 14336)))
    ub = bf16_input(gaussian(30 + batch, (batch, 14336)))
    gd = dev_bf16(gb)
    hip.gated(d.Activation.Silu, gd, dev_bf16(ub), gd)
    assert_bf16(o.gated_bf16(0, gb, ub), host_bits(gd), what="SwiGLU")


def test_activation_unaligned_and_ragged(hip):
    # a view starting one element in: the scalar path
    step("activation unaligned view")
    x = gaussian(4, 1001, 3.0)
    base = dev_f32(x)
    out = torch.empty(1001, dtype=torch.float32, device=DEV)
    hip.activation(d.Activation.GeluTanh, base[1:], out[1:])
    assert_f32(o.activation(1, x[1:]), host_f32(out)[1:], what="unaligned")


def test_convert_round_trips(hip):
    # ReferenceOpsTests.scala:184-213 and SmallOpsTests.scala:104-114
    values = np.concatenate([np.array([1, 1 + 2 ** -8, 1 + 3 * 2 ** -8, 65504, -0.5], np.float32),
                             gaussian(5, 4096, 3.0), SPECIALS,
                             np.array([0x7F800001, 0xFF812345, 0x7FC00000], np.uint32).view(np.float32)])
    step("convert f32 <-> bf16")
    x = dev_f32(values)
    b = torch.empty(values.shape, dtype=torch.bfloat16, device=DEV)
    hip.convert(x, b)
    assert_bits(o.to_bf16(values), host_bits(b), what="f32 -> bf16")
    back = torch.empty(values.shape, dtype=torch.float32, device=DEV)
    hip.convert(b, back)
    assert_bits(o.from_bf16(o.to_bf16(values)).view(np.uint32), host_f32(back).view(np.uint32), what="bf16 -> f32")
    step("convert f32 <-> f16")
    finite = values[~np.isnan(values)]
    h = torch.empty(finite.shape, dtype=torch.float16, device=DEV)
    hip.convert(dev_f32(finite), h)
    assert_bits(o.to_f16(finite), host_bits(h), what="f32 -> f16")
    back16 = torch.empty(finite.shape, dtype=torch.float32, device=DEV)
    hip.convert(h, back16)
    assert_bits(o.from_f16(o.to_f16(finite)).view(np.uint32), host_f32(back16).view(np.uint32), what="f16 -> f32")
    step("convert odd length, scalar path")
    odd = gaussian(6, 1003)
    bo = torch.empty(1003, dtype=torch.bfloat16, device=DEV)
    hip.convert(dev_f32(odd), bo)
    assert_bits(o.to_bf16(odd), host_bits(bo), what="odd length")


def test_convert_fp8_e4m3_to_f32(hip):
    # the reference's conversion code 4 (ops/HipBase.scala:268-274): every
    # E4M3 "fn" byte, as uint8 or torch's float8_e4m3fn, against the
    # oracle's DType.F8E4M3 decode (pinned to torch's float8_e4m3fn)
    codes = np.tile(np.arange(256, dtype=np.uint8), 5)
    want = np.array([o.f8e4m3(c) for c in codes], np.float32)
    nan = np.isnan(want)
    for source in (torch.from_numpy(codes).to(DEV), torch.from_numpy(codes).to(DEV).view(torch.float8_e4m3fn)):
        step(f"convert {source.dtype} -> f32")
        out = torch.empty(codes.size, dtype=torch.float32, device=DEV)
        hip.convert(source, out)
        got = host_f32(out)
        assert np.array_equal(np.isnan(got), nan)
        assert_bits(want[~nan].view(np.uint32), got[~nan].view(np.uint32), what="fp8 e4m3")
