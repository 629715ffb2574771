"""Tensors past 2^31 values on the GPU: GELU-tanh, gatedAdd, AdaLN and
RMSNorm over a little more than 2^31 values (4.3 GB of BF16 a tensor), so the
offsets of the last rows need 64 bits. The rows before, across and after
value 2^31, and the first and last, are checked against the oracle at the
bars of the small cases: 1 bf16 ulp for the activation and the norms, exact
for gatedAdd (one rounding of the F32 result, as the reference's convert)."""

import numpy as np
import pytest
import torch

from drift_amd import ops as d
from oracle import oracle as o
from tests.helpers import DEV, assert_bf16, assert_bits, host_bits, step

pytestmark = pytest.mark.gpu

LIMIT = 1 << 31


@pytest.fixture(scope="module")
def hip():
    return d.HipOps()


@pytest.fixture(autouse=True)
def release():
    yield
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def shape_past(cols):
    """Rows of `cols` values past 2^31 values, and the rows to check: the
    first two, the three around value 2^31 and the last two."""
    rows = LIMIT // cols + 2
    mid = LIMIT // cols
    return rows, np.array([0, 1, mid - 1, mid, mid + 1, rows - 2, rows - 1])


def bf16_normal(shape, seed, scale=1.0):
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    return (scale * torch.randn(shape, generator=g, device=DEV, dtype=torch.bfloat16)).to(torch.bfloat16)


def rows_of(t, rows):
    return host_bits(t[torch.from_numpy(rows).to(DEV)])


def test_gelu_tanh_in_place(hip):
    cols = 4096
    rows, check = shape_past(cols)
    step(f"GELU-tanh bf16 in place over [{rows}, {cols}]")
    x = bf16_normal((rows, cols), 501, 3.0)
    before = rows_of(x, check)
    hip.activation(d.Activation.GeluTanh, x, x)
    assert_bf16(o.activation_bf16(int(d.Activation.GeluTanh), before), rows_of(x, check), what="GELU past 2^31")


def test_gated_add(hip):
    cols = 4096
    rows, check = shape_past(cols)
    step(f"gatedAdd bf16 over [{rows}, {cols}], two samples")
    x, y = bf16_normal((rows, cols), 502), bf16_normal((rows, cols), 503)
    per = -(-rows // 2)
    gate = (0.5 * torch.randn((2, cols), generator=torch.Generator(device=DEV).manual_seed(504), device=DEV)).float()
    xb, yb, g = rows_of(x, check), rows_of(y, check), gate.cpu().numpy()
    hip.gatedAdd(x, y, gate, per)
    want = np.stack([o.gated_add(o.from_bf16(xb[i:i + 1]), o.from_bf16(yb[i:i + 1]), g[r // per])[0]
                     for i, r in enumerate(check)])
    assert_bits(o.to_bf16(want), rows_of(x, check), what="gatedAdd past 2^31")


def test_adaln(hip):
    cols = 3072
    rows, check = shape_past(cols)
    step(f"AdaLN bf16 over [{rows}, {cols}], two samples")
    x = bf16_normal((rows, cols), 505)
    out = torch.empty_like(x)
    per = -(-rows // 2)
    gen = torch.Generator(device=DEV).manual_seed(506)
    scale = (0.1 * torch.randn((2, cols), generator=gen, device=DEV)).float()
    shift = (0.1 * torch.randn((2, cols), generator=gen, device=DEV)).float()
    xb = rows_of(x, check)
    hip.layerNormModulate(x, scale, shift, 1e-6, out, per)
    s, sh = scale.cpu().numpy(), shift.cpu().numpy()
    want = np.concatenate([o.layer_norm_modulate_bf16(xb[i:i + 1], s[r // per], sh[r // per], 1, 1e-6)
                           for i, r in enumerate(check)])
    assert_bf16(want, rows_of(out, check), what="AdaLN past 2^31")


def test_rms_norm(hip):
    cols = 4096
    rows, check = shape_past(cols)
    step(f"RMSNorm bf16 over [{rows}, {cols}]")
    x = bf16_normal((rows, cols), 507)
    out = torch.empty_like(x)
    w = (1 + 0.1 * torch.randn(cols, generator=torch.Generator(device=DEV).manual_seed(508), device=DEV)).float()
    xb = rows_of(x, check)
    hip.rmsNorm(x, w, 1e-5, 0.0, out)
    assert_bf16(o.rms_norm_bf16(xb, w.cpu().numpy(), 1e-5), rows_of(out, check), what="RMSNorm past 2^31")
