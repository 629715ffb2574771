"""Tensors past 2^31 values on the GPU: GELU-tanh, gatedAdd, AdaLN, RMSNorm,
3-D RoPE and the QK norm+RoPE over a little more than 2^31 values (4.3 GB of
BF16 a tensor), so the offsets of the last rows need 64 bits. The rows
before, across and after value 2^31, and the first and last, are checked
against the oracle at the bars of the small cases: 1 bf16 ulp for the
activation, the norms and the rotations, exact for gatedAdd (one rounding of
the F32 result, as the reference's convert)."""

import numpy as np
import pytest
import torch

from drift_amd import ops as d
from oracle import oracle as o
from tests.helpers import DEV, assert_bf16, assert_bits, dev_f32, dev_i32, host_bits, step

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


def test_rope_3d_in_place(hip):
    # the C5 grid (21 x 30 x 52, 24 heads of 128), wrapped 21 times
    heads, dim = 24, 128
    tokens, check = shape_past(heads * dim)
    step(f"rope3d bf16 in place over [{tokens}, {heads}, {dim}]")
    x = bf16_normal((tokens, heads, dim), 509)
    before = rows_of(x, check)
    hip.rope3d(x, 21, 30, 52, x)
    want = np.concatenate([o.rope_3d_bf16(before[i:i + 1], 21, 30, 52, token_offset=int(t))
                           for i, t in enumerate(check)])
    assert_bf16(want, rows_of(x, check), what="rope3d past 2^31")


def test_query_key_norm_rope_in_place(hip):
    # Qwen3's heads (32 and 8 of 128) at positions 0 .. tokens - 1: the
    # queries past 2^31 values, angles up to half a million radians
    heads, kv, dim = 32, 8, 128
    tokens, check = shape_past(heads * dim)
    step(f"queryKeyNormRope bf16 in place over {tokens} tokens of {heads} + {kv} heads")
    q, k = bf16_normal((tokens, heads, dim), 510), bf16_normal((tokens, kv, dim), 511)
    rng = np.random.default_rng(512)
    qw = (1 + 0.1 * rng.standard_normal(dim)).astype(np.float32)
    kw = (1 + 0.1 * rng.standard_normal(dim)).astype(np.float32)
    rope = d.Rope(1e6, dim, d.RopeLayout.Neox)
    norms = d.QueryKeyNorms(dev_f32(qw), dev_f32(kw), 1e-6, 0.0, rope)
    positions = np.arange(tokens, dtype=np.int32)
    qb, kb = rows_of(q, check), rows_of(k, check)
    hip.queryKeyNormRope(q, k, norms, dev_i32(positions), q, k)
    want_q, want_k = o.qk_norm_rope_bf16(qb, kb, qw, kw, positions[check], 1e-6, 0.0, 1e6, dim)
    assert_bf16(want_q, rows_of(q, check), what="queries past 2^31")
    assert_bf16(want_k, rows_of(k, check), what="keys")
