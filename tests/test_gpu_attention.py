"""Attention inputs on the GPU against the oracle: the paged F16 cache write,
splitHalves, and attentionInputs (a gated query's split, per-head RMS norms,
rope and the cache write in one launch), in the reference's fused test case
(FusedOpsTests.scala:406-499: 16 heads, 2 key heads of 256, rotary 64 with
interleaved mRoPE, tokens crossing a page) and at Qwen3's shape, gated and
dense, F32 and BF16.

Bars: the cache write and splitHalves are bit-exact (they only move and
round values); rotated queries are held to the F32 bar or 1 bf16 ulp; the
keys in the cache, the F32 rope result rounded to F16, to 1 F16 ulp (the
rounding of a value within the F32 bar); gates and cached values exactly."""

import numpy as np
import pytest
import torch

from drift_amd import ops as d
from oracle import oracle as o
from tests.helpers import (DEV, assert_bf16, assert_bits, assert_f32, bf16_input, dev_bf16, dev_f32, dev_i32,
                           gaussian, host_bits, host_f32, step)

pytestmark = pytest.mark.gpu

PAGE = 16


@pytest.fixture(scope="module")
def hip():
    return d.HipOps()


def f16_ulps(expected, actual) -> np.ndarray:
    e = np.asarray(expected, np.uint16).astype(np.int64).ravel()
    a = np.asarray(actual, np.uint16).astype(np.int64).ravel()
    oe = np.where(e & 0x8000, -(e & 0x7FFF), e)
    oa = np.where(a & 0x8000, -(a & 0x7FFF), a)
    return np.abs(oe - oa)


def cache(pages, kv, dim, fill_seed):
    """A cache filled with seeded garbage, and its bits as the oracle's start."""
    rng = np.random.default_rng(fill_seed)
    keys = rng.integers(0, 0x7000, pages * PAGE * kv * dim).astype(np.uint16)  # finite halves
    values = rng.integers(0, 0x7000, pages * kv * dim * PAGE).astype(np.uint16)
    c = d.KvCache.allocate(pages, PAGE, kv, dim, DEV)
    c.keys.copy_(torch.from_numpy(keys.view(np.int16)).view(torch.float16).reshape(c.keys.shape))
    c.values.copy_(torch.from_numpy(values.view(np.int16)).view(torch.float16).reshape(c.values.shape))
    return c, keys, values


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("tokens,kv,dim,start", [(1, 8, 128, 14), (37, 2, 128, 5), (5, 3, 72, 30), (1, 1, 8, 0)])
def test_cache_write(hip, dtype, tokens, kv, dim, start):
    step(f"cacheWrite {dtype} {tokens} tokens, {kv} heads of {dim}, start {start}")
    pages = -(-(start + tokens) // PAGE) + 1
    table = np.random.default_rng(tokens).permutation(pages).astype(np.int32)
    k = gaussian(1, (tokens, kv, dim), 2.0)
    v = gaussian(2, (tokens, kv, dim), 2.0)
    if dtype == "bf16":
        kb, vb = bf16_input(k), bf16_input(v)
        k, v = o.from_bf16(kb), o.from_bf16(vb)
        kd, vd = dev_bf16(kb), dev_bf16(vb)
    else:
        kd, vd = dev_f32(k), dev_f32(v)
    c, keys0, values0 = cache(pages, kv, dim, 7)
    bad = torch.zeros(1, dtype=torch.int32, device=DEV)
    hip.cacheWrite(kd, vd, c, dev_i32(table), start, bad)
    want_k, want_v = o.cache_write(k, v, keys0, values0, table, PAGE, start)
    assert_bits(want_k, host_bits(c.keys), what="cached keys")
    assert_bits(want_v, host_bits(c.values), what="cached values")
    assert int(bad.item()) == 0


def test_cache_write_skips_a_page_outside_the_cache(hip):
    step("cacheWrite with a page-table entry past the cache")
    tokens, kv, dim, start = 20, 2, 64, 10  # positions 10..29 on pages 0 and 1
    table = np.array([1, 9], np.int32)  # page 9 does not exist (2 pages)
    k, v = gaussian(3, (tokens, kv, dim)), gaussian(4, (tokens, kv, dim))
    c, keys0, values0 = cache(2, kv, dim, 8)
    bad = torch.zeros(1, dtype=torch.int32, device=DEV)
    hip.cacheWrite(dev_f32(k), dev_f32(v), c, dev_i32(table), start, bad)
    # positions 10..15 land on page 1; 16..29 would be on page 9 and are dropped
    want_k, want_v = o.cache_write(k[:6], v[:6], keys0, values0, table, PAGE, start)
    assert_bits(want_k, host_bits(c.keys), what="keys")
    assert_bits(want_v, host_bits(c.values), what="values")
    assert int(bad.item()) == 1


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("shape", [(4, 3, 256), (7, 10), (1, 1, 16), (33, 2, 12)])
def test_split_halves(hip, dtype, shape):
    step(f"splitHalves {dtype} {shape}")
    x = gaussian(5, shape)
    half = shape[:-1] + (shape[-1] // 2,)
    if dtype == "bf16":
        xb = bf16_input(x)
        first = torch.empty(half, dtype=torch.bfloat16, device=DEV)
        second = torch.empty_like(first)
        hip.splitHalves(dev_bf16(xb), first, second)
        f, s = np.split(xb, 2, axis=-1)
        assert_bits(f, host_bits(first), what="first")
        assert_bits(s, host_bits(second), what="second")
    else:
        first = torch.empty(half, dtype=torch.float32, device=DEV)
        second = torch.empty_like(first)
        hip.splitHalves(dev_f32(x), first, second)
        f, s = o.split_halves(x)
        assert np.array_equal(f, host_f32(first)) and np.array_equal(s, host_f32(second))


REFERENCE_ROPE = d.Rope(1e7, 64, d.RopeLayout.Neox, d.RopeSections.Interleaved(11, 11, 10))
QWEN3_ROPE = d.Rope(1e6, 128, d.RopeLayout.Neox, d.RopeSections.Single())


def shifted(values: np.ndarray, shift: int) -> torch.Tensor:
    """values on the device, starting `shift` floats into their buffer."""
    return dev_f32(np.concatenate([np.full(shift, 7.0, np.float32), values]))[shift:]


def run_attention_inputs(hip, dtype, t, heads, kv, dim, rope, start, table, pages, gated, seed, offset=0.0,
                         weight_shift=0):
    rng = np.random.default_rng(seed)
    width = 2 * dim if gated else dim
    qg = (2 * rng.standard_normal((t, heads, width))).astype(np.float32)
    k = (2 * rng.standard_normal((t, kv, dim))).astype(np.float32)
    v = rng.standard_normal((t, kv, dim)).astype(np.float32)
    qw = (1 + 0.1 * rng.standard_normal(dim)).astype(np.float32)
    kw = (1 + 0.1 * rng.standard_normal(dim)).astype(np.float32)
    count = rope.sections.positionsPerToken
    positions = np.array([start + i % t + i // t for i in range(count * t)], np.int32)
    positions = positions.reshape(count, t) if count > 1 else positions
    c, keys0, values0 = cache(pages, kv, dim, seed + 1)
    norms = d.QueryKeyNorms(shifted(qw, weight_shift), shifted(kw, 2 * weight_shift), 1e-6, offset, rope)
    bf = dtype == "bf16"
    if bf:
        qgb, kb, vb = bf16_input(qg), bf16_input(k), bf16_input(v)
        qg, k, v = o.from_bf16(qgb), o.from_bf16(kb), o.from_bf16(vb)
        dev, tt = dev_bf16, torch.bfloat16
        inputs = (dev(qgb), dev(kb), dev(vb))
    else:
        dev, tt = dev_f32, torch.float32
        inputs = (dev(qg), dev(k), dev(v))
    rotated = torch.empty((t, heads, dim), dtype=tt, device=DEV)
    bad = torch.zeros(1, dtype=torch.int32, device=DEV)
    if gated:
        queries, gate = torch.empty_like(rotated), torch.empty_like(rotated)
        rotated_keys = torch.empty((t, kv, dim), dtype=tt, device=DEV)
        hip.attentionInputs(inputs[0], inputs[1], inputs[2], norms, dev_i32(positions), c, dev_i32(table), start,
                            queries, gate, rotated_keys, rotated, bad)
    else:
        gate = None
        hip.queryKeyNormRopeCache(inputs[0], inputs[1], inputs[2], norms, dev_i32(positions), c, dev_i32(table),
                                  start, rotated, bad)
    want_q, want_gate, want_k, want_v = o.attention_inputs(
        qg, k, v, qw, kw, 1e-6, offset, positions, rope.theta, rope.rotaryDimensions, keys0, values0, table, PAGE,
        start, int(rope.layout), rope.sections.code, rope.sections.sizes, gated)
    what = f"{dtype} {t} tokens"
    if bf:
        assert_bf16(o.to_bf16(want_q), host_bits(rotated), what=f"rotated queries {what}")
        if gated:
            assert_bits(o.to_bf16(want_gate), host_bits(gate), what=f"gate {what}")
    else:
        assert_f32(want_q, host_f32(rotated), what=f"rotated queries {what}")
        if gated:
            assert np.array_equal(want_gate, host_f32(gate)), f"gate {what}"
    ulps = f16_ulps(want_k, host_bits(c.keys))
    assert ulps.max() <= 1, f"cached keys {what}: {int((ulps > 1).sum())} beyond 1 F16 ulp"
    assert_bits(want_v, host_bits(c.values), what=f"cached values {what}")
    assert int(bad.item()) == 0


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("t", [1, 3])
def test_attention_inputs_reference_case(hip, dtype, t):
    step(f"attentionInputs {dtype}, the reference's fused case, {t} tokens")
    run_attention_inputs(hip, dtype, t, 16, 2, 256, REFERENCE_ROPE, 14, np.array([3, 0, 2, 1], np.int32), 4, True,
                         60 + t)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("t,gated", [(1, True), (5, True), (64, True), (1, False), (40, False)])
def test_attention_inputs_qwen3_shape(hip, dtype, t, gated):
    step(f"attentionInputs {dtype} Qwen3 heads 32/8 of 128, {t} tokens, gated {gated}")
    start = 9
    pages = -(-(start + t) // PAGE) + 2
    table = np.random.default_rng(t).permutation(pages).astype(np.int32)
    run_attention_inputs(hip, dtype, t, 32, 8, 128, QWEN3_ROPE, start, table, pages, gated, 90 + t)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("gated", [True, False])
def test_attention_inputs_with_a_weight_offset(hip, dtype, gated):
    # norms of (weight + 1), as a Gemma-style model passes them: the body
    # that adds the offset
    t, start = 19, 3
    step(f"attentionInputs {dtype} Qwen3 heads with a weight offset of 1, gated {gated}")
    pages = -(-(start + t) // PAGE) + 1
    table = np.random.default_rng(7).permutation(pages).astype(np.int32)
    run_attention_inputs(hip, dtype, t, 32, 8, 128, QWEN3_ROPE, start, table, pages, gated, 150, offset=1.0)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("heads,kv,dim,gated", [(8, 3, 64, True), (4, 5, 32, False), (6, 1, 16, True)])
def test_attention_inputs_small_heads(hip, dtype, heads, kv, dim, gated):
    # value tiles of several key heads, the last tile's heads cut short
    t, start = 37, 5
    step(f"attentionInputs {dtype} heads {heads}/{kv} of {dim}, {t} tokens, gated {gated}")
    pages = -(-(start + t) // PAGE) + 1
    table = np.random.default_rng(dim).permutation(pages).astype(np.int32)
    rope = d.Rope(1e4, dim, d.RopeLayout.Neox, d.RopeSections.Single())
    run_attention_inputs(hip, dtype, t, heads, kv, dim, rope, start, table, pages, gated, 120 + dim)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("heads,kv,dim", [(16, 3, 128), (64, 16, 64), (32, 9, 128)])
def test_attention_inputs_key_heads_by_the_group(hip, dtype, heads, kv, dim):
    # no gate, whole waves of query heads; key heads that fill part of a
    # wave's group, two groups, a group and a part
    t, start = 29, 7
    step(f"attentionInputs {dtype} heads {heads}/{kv} of {dim}, {t} tokens")
    pages = -(-(start + t) // PAGE) + 1
    table = np.random.default_rng(heads + kv).permutation(pages).astype(np.int32)
    rope = d.Rope(1e6, dim, d.RopeLayout.Neox, d.RopeSections.Single())
    run_attention_inputs(hip, dtype, t, heads, kv, dim, rope, start, table, pages, False, 170 + kv)


def test_attention_inputs_flag_a_page_outside_the_cache(hip):
    step("attentionInputs with a page-table entry past the cache")
    t, heads, kv, dim = 4, 4, 2, 128
    c, keys0, values0 = cache(1, kv, dim, 3)
    qg = gaussian(6, (t, heads, 2 * dim))
    k, v = gaussian(7, (t, kv, dim)), gaussian(8, (t, kv, dim))
    w = dev_f32(np.ones(dim, np.float32))
    norms = d.QueryKeyNorms(w, w, 1e-6, 0.0, QWEN3_ROPE)
    table = dev_i32(np.array([5], np.int32))
    bad = torch.zeros(1, dtype=torch.int32, device=DEV)
    out = [torch.empty((t, heads, dim), device=DEV) for _ in range(3)]
    hip.attentionInputs(dev_f32(qg), dev_f32(k), dev_f32(v), norms, dev_i32(np.arange(t, dtype=np.int32)), c, table,
                        0, out[0], out[1], torch.empty((t, kv, dim), device=DEV), out[2], bad)
    assert int(bad.item()) == 1
    assert_bits(keys0, host_bits(c.keys), what="keys untouched")
    assert_bits(values0, host_bits(c.values), what="values untouched")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("gated", [True, False])
def test_attention_inputs_with_weights_off_a_16_byte_boundary(hip, dtype, gated):
    # norm weights 4 and 8 bytes into their buffers: the fast body reads
    # weights as 16-byte loads, so these take the general kernel
    t, start = 21, 5
    step(f"attentionInputs {dtype} Qwen3 heads, norm weights off a 16-byte boundary, gated {gated}")
    pages = -(-(start + t) // PAGE) + 1
    table = np.random.default_rng(9).permutation(pages).astype(np.int32)
    run_attention_inputs(hip, dtype, t, 32, 8, 128, QWEN3_ROPE, start, table, pages, gated, 170, weight_shift=1)
