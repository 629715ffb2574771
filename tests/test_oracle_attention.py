"""Pins the oracle's attention-input pieces (CPU only): splitHalves, the paged
F16 cache write and the attentionInputs composition.

The reference's own checks of these are GPU tests of fused against separate
launches (runner/gpuTest/src/drift/runner/FusedOpsTests.scala:406-499); its
CPU forms are ops/CpuLayout.scala:137-143 and ops/CpuAttention.scala:163-210.
Here the oracle is held to known answers worked by hand, to numpy's own
float16 rounding (an independent F32 -> F16 routine), and to invariants a
slip in an index would break: every cache slot the tokens own holds its
value, every other slot is untouched, and the layouts are the reference's
(keys [pages, page_size, heads, D], values transposed within a page).
"""

import numpy as np
import pytest

from oracle import oracle as o

PAGE = 16


def test_split_halves_known_answer():
    x = np.arange(2 * 3 * 8, dtype=np.float32).reshape(2, 3, 8)
    first, second = o.split_halves(x)
    assert first.shape == second.shape == (2, 3, 4)
    assert first[1, 2].tolist() == [40, 41, 42, 43] and second[1, 2].tolist() == [44, 45, 46, 47]
    assert np.array_equal(np.concatenate([first, second], axis=-1), x)


def test_cache_place_hand_worked():
    # page table [3, 0, 2, 1]: position 14 is page 3 offset 14; position 16 page 0 offset 0
    table = np.array([3, 0, 2, 1])
    key, value = o.cache_place(table, PAGE, 14, 2, 8, 1, 5)
    assert key == ((3 * 16 + 14) * 2 + 1) * 8 + 5
    assert value == ((3 * 2 + 1) * 8 + 5) * 16 + 14
    key, value = o.cache_place(table, PAGE, 16, 2, 8, 0, 0)
    assert (key, value) == (0, 0)


def test_cache_write_layout_against_numpy_float16():
    rng = np.random.default_rng(3)
    tokens, kv, d, pages, start = 5, 2, 8, 4, 14  # positions 14..18 cross from page 3 to page 0
    table = np.array([3, 0, 2, 1], np.int32)
    k = rng.standard_normal((tokens, kv, d)).astype(np.float32)
    v = rng.standard_normal((tokens, kv, d)).astype(np.float32)
    keys0 = rng.integers(0, 1 << 16, pages * PAGE * kv * d).astype(np.uint16)
    values0 = rng.integers(0, 1 << 16, pages * kv * d * PAGE).astype(np.uint16)
    keys, values = o.cache_write(k, v, keys0, values0, table, PAGE, start)
    K = keys.reshape(pages, PAGE, kv, d)
    V = values.reshape(pages, kv, d, PAGE)
    owned_k = np.zeros(K.shape, bool)
    owned_v = np.zeros(V.shape, bool)
    for t in range(tokens):
        page, offset = table[(start + t) // PAGE], (start + t) % PAGE
        assert np.array_equal(K[page, offset], k[t].astype(np.float16).view(np.uint16))
        assert np.array_equal(V[page, :, :, offset], v[t].astype(np.float16).view(np.uint16))
        owned_k[page, offset] = True
        owned_v[page, :, :, offset] = True
    assert np.array_equal(K[~owned_k], keys0.reshape(K.shape)[~owned_k]), "slots no token owns are untouched"
    assert np.array_equal(V[~owned_v], values0.reshape(V.shape)[~owned_v])


def test_f16_rounding_agrees_with_numpy_at_ties_and_limits():
    # ties to even at the half-ulp, subnormals, the overflow threshold
    x = np.array([1 + 2 ** -11, 1 + 3 * 2 ** -11, 2 ** -24, 2 ** -25, 3 * 2 ** -26, 65504, 65519.99, 65520, -0.0,
                  1e-8, -6.1e-5], np.float32)
    with np.errstate(over="ignore"):
        assert np.array_equal(o.to_f16(x), x.astype(np.float16).view(np.uint16))


def _inputs(rng, t, heads, kv, d, gated=True):
    qg = rng.standard_normal((t, heads, 2 * d if gated else d)).astype(np.float32)
    k = rng.standard_normal((t, kv, d)).astype(np.float32)
    v = rng.standard_normal((t, kv, d)).astype(np.float32)
    qw = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    kw = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    return qg, k, v, qw, kw


@pytest.mark.parametrize("t", [1, 3])
def test_attention_inputs_composition(t):
    # the reference's fused test case: 16 heads, 2 key heads of 256, rotary 64
    # NeoX with interleaved mRoPE (11, 11, 10), theta 1e7, start 14 across a page
    rng = np.random.default_rng(60 + t)
    heads, kv, d, pages, start = 16, 2, 256, 4, 14
    table = np.array([3, 0, 2, 1], np.int32)
    qg, k, v, qw, kw = _inputs(rng, t, heads, kv, d)
    positions = np.array([start + i % t + i // t for i in range(3 * t)], np.int32)
    keys0 = np.zeros(pages * PAGE * kv * d, np.uint16)
    values0 = np.zeros(pages * kv * d * PAGE, np.uint16)
    args = (1e-6, 0.0, positions, 1e7, 64, keys0, values0, table, PAGE, start, o.NEOX, o.INTERLEAVED_MROPE,
            (11, 11, 10))
    rq, gate, keys, values = o.attention_inputs(qg, k, v, qw, kw, *args)
    assert np.array_equal(gate, qg[..., d:]), "the gate is the second half, untouched"
    # the dense form on the query halves gives the same queries and cache
    rq2, none, keys2, values2 = o.attention_inputs(np.ascontiguousarray(qg[..., :d]), k, v, qw, kw, *args,
                                                   gated=False)
    assert none is None and np.array_equal(rq, rq2) and np.array_equal(keys, keys2)
    assert np.array_equal(values, values2)
    # the cache holds the rotated keys rounded to F16 (numpy's rounding), the values likewise
    _, rk = o.qk_norm_rope(qg[..., :d], k, qw, kw, positions, 1e-6, 0.0, 1e7, 64, o.NEOX, o.INTERLEAVED_MROPE,
                           (11, 11, 10))
    K = keys.reshape(pages, PAGE, kv, d)
    V = values.reshape(pages, kv, d, PAGE)
    for i in range(t):
        page, offset = table[(start + i) // PAGE], (start + i) % PAGE
        assert np.array_equal(K[page, offset], rk[i].astype(np.float16).view(np.uint16))
        assert np.array_equal(V[page, :, :, offset], v[i].astype(np.float16).view(np.uint16))
    # partial rotary: values past the 64 rotary dimensions are only normed
    qn = o.rms_norm(qg[..., :d].reshape(t * heads, d), qw, 1e-6).reshape(t, heads, d)
    assert np.array_equal(rq[..., 64:], qn[..., 64:])
