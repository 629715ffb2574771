"""Pins of the oracle's gated residuals and per-row modulation
(ops/CpuElementwise.scala:40-85). The reference's CPU and GPU forms of these
are uncompared in its own suite (OpsComparisonCoverageTests.scala:102-123);
they are pinned here by exact sums, by reducing each to an operation pinned
elsewhere (modulate, gatedAdd) when the tables hold the same row everywhere,
and by chunk tables whose chunks are told apart by value."""

import numpy as np
import pytest

from oracle import oracle as o


def gaussian(seed, shape, scale=1.0):
    return (scale * np.random.default_rng(seed).standard_normal(shape)).astype(np.float32)


def test_gated_add_exact_cases():
    x = np.arange(-8, 8, dtype=np.float32).reshape(2, 8)
    y = np.full((2, 8), 3.0, np.float32)
    assert np.array_equal(o.gated_add(x, y, np.zeros(8, np.float32)), x)
    assert np.array_equal(o.gated_add(x, y, np.ones(8, np.float32)), x + 3)
    gate = np.arange(8, dtype=np.float32) / 4
    assert np.array_equal(o.gated_add(x, y, gate), x + 3 * gate)
    # one rounding of x + g*y: 1 + 2^-24 * 1 stays 1 only if the sum rounds once
    one = np.ones((1, 1), np.float32)
    tiny = np.full((1, 1), 2.0 ** -24, np.float32)
    half_up = o.gated_add(one, tiny, np.array([1.5], np.float32))  # 1 + 1.5 * 2^-24 -> 1 + 2^-23
    assert half_up[0, 0] == np.float32(1 + 2.0 ** -23)


def test_gated_add_per_sample_rows():
    x, y = gaussian(1, (10, 16)), gaussian(2, (10, 16))
    gates = gaussian(3, (3, 16))
    got = o.gated_add(x, y, gates, rows_per_sample=4)
    for s, (lo, hi) in enumerate([(0, 4), (4, 8), (8, 10)]):
        assert np.array_equal(got[lo:hi], o.gated_add(x[lo:hi], y[lo:hi], gates[s]))


def test_row_gated_add_is_gated_add_with_a_constant_gate():
    x, y = gaussian(4, (6, 24)), gaussian(5, (6, 24))
    g = gaussian(6, 6)
    got = o.row_gated_add(x, y, g)
    for r in range(6):
        assert np.array_equal(got[r:r + 1], o.gated_add(x[r:r + 1], y[r:r + 1], np.full(24, g[r], np.float32)))


def test_chunk_tables_reduce_to_vector_operations():
    rows, channels, chunks = 5, 12, 6
    x, y = gaussian(7, (rows, channels), 3.0), gaussian(8, (rows, channels))
    vectors = gaussian(9, (chunks, channels), 0.5)
    table = np.tile(vectors.reshape(1, -1), (rows, 1))
    assert np.array_equal(o.modulate_chunks(x, table, 0, 1), o.modulate(x, vectors[1], vectors[0]))
    assert np.array_equal(o.modulate_chunks(x, table, 3, 4), o.modulate(x, vectors[4], vectors[3]))
    assert np.array_equal(o.gated_add_chunk(x, y, table, 2), o.gated_add(x, y, vectors[2]))
    assert np.array_equal(o.gated_add_chunk(x, y, table, 5), o.gated_add(x, y, vectors[5]))


def test_chunks_and_rows_are_told_apart():
    rows, channels, chunks = 3, 4, 6
    # chunk k of row r holds 10 r + k everywhere
    table = np.array([[10 * r + k for k in range(chunks) for _ in range(channels)] for r in range(rows)], np.float32)
    x = np.ones((rows, channels), np.float32)
    y = np.full((rows, channels), 2.0, np.float32)
    for gate in range(chunks):
        got = o.gated_add_chunk(x, y, table, gate)
        assert np.array_equal(got, 1 + 2 * (10 * np.arange(rows)[:, None] + gate) * np.ones((1, channels)))
    got = o.modulate_chunks(x, table, 1, 4)  # x * (1 + scale) + shift
    assert np.array_equal(got, (1 + 10 * np.arange(rows)[:, None] + 4) + (10 * np.arange(rows)[:, None] + 1) +
                          np.zeros((1, channels)))


def test_modulate_chunks_zero_table_is_identity():
    x = gaussian(10, (4, 32), 5.0)
    assert np.array_equal(o.modulate_chunks(x, np.zeros((4, 64), np.float32), 0, 1), x)


def test_bad_tables_are_refused():
    x = np.zeros((3, 4), np.float32)
    with pytest.raises(ValueError):
        o.modulate_chunks(x, np.zeros((3, 10), np.float32), 0, 1)
    with pytest.raises(ValueError):
        o.gated_add_chunk(x, x, np.zeros((3, 8), np.float32), 2)
    with pytest.raises(ValueError):
        o.row_gated_add(x, x, np.zeros(2, np.float32))
    with pytest.raises(ValueError):
        o.gated_add(x, x, np.zeros((2, 4), np.float32), rows_per_sample=1)
