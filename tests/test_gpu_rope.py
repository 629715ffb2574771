"""RoPE kernels on the GPU against the oracle: the reference's seven rope
configurations (SmallOpsTests.scala:450-500), rope from tables, Wan's 3-D rope
with in-kernel angles, and per-head query/key RMSNorm fused with rope.

The reference holds its own GPU rope to 1e-2 absolute because its kernel's
powf differs from the CPU's pow (SmallOpsTests.scala:480-485); these kernels
take the inverse frequencies the CPU's way and turn in double, so they are
held to the F32 and BF16 bars instead."""

import numpy as np
import pytest
import torch

from drift_amd import ops as d
from oracle import oracle as o
from tests.helpers import (DEV, assert_bf16, assert_f32, bf16_input, dev_bf16, dev_f32, dev_i32, gaussian,
                           host_bits, host_f32, step)

pytestmark = pytest.mark.gpu

R = d.RopeSections
REFERENCE_ROPES = [
    d.Rope(1e4, 128, d.RopeLayout.Neox, R.Single()),
    d.Rope(1e4, 128, d.RopeLayout.Interleaved, R.Single()),
    d.Rope(1e7, 64, d.RopeLayout.Neox, R.Single()),
    d.Rope(1e7, 64, d.RopeLayout.Neox, R.Contiguous(11, 11, 10)),
    d.Rope(1e7, 64, d.RopeLayout.Neox, R.Interleaved(11, 11, 10)),
    d.Rope(1e3, 128, d.RopeLayout.Interleaved, R.Axes([16, 24, 24])),
    d.Rope(2e3, 128, d.RopeLayout.Interleaved, R.Axes([16, 16, 16, 16])),
]


def oracle_rope(x, positions, rope: d.Rope):
    return o.rope(x, positions, rope.theta, rope.rotaryDimensions, int(rope.layout), rope.sections.code,
                  rope.sections.sizes)


def reference_case(rope: d.Rope):
    dimension = 256 if rope.rotaryDimensions == 64 else 128
    shape = (37, 3, dimension)
    count = rope.sections.positionsPerToken
    positions = ((np.arange(count * 37) * 131) % 4096).astype(np.int32)
    if count > 1:
        positions = positions.reshape(count, 37)
    return shape, positions


@pytest.fixture(scope="module")
def hip():
    return d.HipOps()


@pytest.mark.parametrize("index", range(len(REFERENCE_ROPES)))
def test_reference_rope_configurations(hip, index):
    rope = REFERENCE_ROPES[index]
    shape, positions = reference_case(rope)
    x = gaussian(1, shape, 3.0)
    step(f"rope f32 {rope}")
    out = torch.empty(shape, dtype=torch.float32, device=DEV)
    hip.rope(dev_f32(x), dev_i32(positions), rope, out)
    assert_f32(oracle_rope(x, positions, rope), host_f32(out), what=f"rope {index}")
    step(f"rope bf16 {rope}")
    xb = bf16_input(x)
    outb = torch.empty(shape, dtype=torch.bfloat16, device=DEV)
    hip.rope(dev_bf16(xb), dev_i32(positions), rope, outb)
    assert_bf16(o.to_bf16(oracle_rope(o.from_bf16(xb), positions, rope)), host_bits(outb), what=f"rope bf16 {index}")


def test_rope_tables_follow_the_configuration(hip):
    # the library keeps the inverse frequencies of its last four rope
    # configurations per host thread: alternating between six (each theta,
    # rotary width and section split a different table) twice over, every
    # call must use its own
    step("rope f32 over six configurations, twice")
    ropes = REFERENCE_ROPES[:2] + REFERENCE_ROPES[3:5] + REFERENCE_ROPES[5:7]
    x = gaussian(3, (37, 3, 256), 2.0)
    for round_ in range(2):
        for index, rope in enumerate(ropes):
            dimension = 256 if rope.rotaryDimensions == 64 else 128
            shape, positions = reference_case(rope)
            xs = np.ascontiguousarray(x[:, :, :dimension])
            out = torch.empty(shape, dtype=torch.float32, device=DEV)
            hip.rope(dev_f32(xs), dev_i32(positions), rope, out)
            assert_f32(oracle_rope(xs, positions, rope), host_f32(out), what=f"round {round_}, rope {index}")


@pytest.mark.parametrize("shape,rotary,layout", [((5, 2, 6), 2, 0), ((4, 3, 10), 6, 1), ((3, 2, 7), 4, 0),
                                                 ((6, 5, 96), 48, 0), ((2, 1, 512), 512, 1)])
def test_rope_odd_shapes_and_in_place(hip, shape, rotary, layout):
    step(f"rope f32 {shape} rotary {rotary} layout {layout}, in place")
    x = gaussian(2, shape, 3.0)
    p = ((np.arange(shape[0]) * 977) % 40000).astype(np.int32)
    rope = d.Rope(1e4, rotary, d.RopeLayout(layout))
    xd = dev_f32(x)
    hip.rope(xd, dev_i32(p), rope, xd)
    assert_f32(oracle_rope(x, p, rope), host_f32(xd), what="rope in place")


def test_c1_rms_norm_then_rope_seed_0(hip):
    # C1: RMSNorm (eps 1e-6) on x[8, 2048] ~ N(0,1), weight ~ N(1, 0.1); NeoX
    # RoPE (theta 1e4) on Q[8, 16, 128] at positions 0..7; inputs from
    # TestData.gaussian's generator (java.util.Random) with seed 0.
    step("C1 rmsNorm + rope f32, seed 0")
    draws = o.java_gaussian(0, 8 * 2048 + 2048 + 8 * 16 * 128)
    x = draws[:8 * 2048].reshape(8, 2048)
    w = (1 + 0.1 * draws[8 * 2048:9 * 2048]).astype(np.float32)
    q = draws[9 * 2048:].reshape(8, 16, 128)
    out = torch.empty((8, 2048), dtype=torch.float32, device=DEV)
    hip.rmsNorm(dev_f32(x), dev_f32(w), 1e-6, 0.0, out)
    assert_f32(o.rms_norm(x, w, 1e-6), host_f32(out), what="C1 rmsNorm")
    rope = d.Rope(1e4, 128, d.RopeLayout.Neox)
    p = np.arange(8, dtype=np.int32)
    rq = torch.empty((8, 16, 128), dtype=torch.float32, device=DEV)
    hip.rope(dev_f32(q), dev_i32(p), rope, rq)
    assert_f32(oracle_rope(q, p, rope), host_f32(rq), what="C1 rope")


@pytest.mark.parametrize("halves", [False, True])
@pytest.mark.parametrize("per_head", [False, True])
@pytest.mark.parametrize("shape,pairs", [((7, 3, 128), 64), ((5, 2, 128), 48), ((4, 3, 10), 3)])
def test_rope_table(hip, halves, per_head, shape, pairs):
    tokens, heads, dim = shape
    table_shape = (tokens, heads, pairs) if per_head else (tokens, pairs)
    angles = np.random.default_rng(3).uniform(-40, 40, table_shape)
    cos, sin = np.cos(angles).astype(np.float32), np.sin(angles).astype(np.float32)
    x = gaussian(4, shape, 3.0)
    step(f"ropeTable f32 {shape} pairs {pairs} halves {halves} per_head {per_head}")
    out = torch.empty(shape, dtype=torch.float32, device=DEV)
    hip.ropeTable(dev_f32(x), dev_f32(cos), dev_f32(sin), out, halves)
    assert_f32(o.rope_table(x, cos, sin, halves), host_f32(out), what="ropeTable")
    step(f"ropeTable bf16 {shape}")
    xb = bf16_input(x)
    outb = torch.empty(shape, dtype=torch.bfloat16, device=DEV)
    hip.ropeTable(dev_bf16(xb), dev_f32(cos), dev_f32(sin), outb, halves)
    assert_bf16(o.to_bf16(o.rope_table(o.from_bf16(xb), cos, sin, halves)), host_bits(outb), what="ropeTable bf16")


# tokens of 1 to 18 chunks a lane (bf16: 1 to 72 heads of 128), each
# wave-per-token variant, and heads of 126 (not whole chunks)
@pytest.mark.parametrize("grid,heads,dim,samples", [((3, 4, 5), 2, 128, 2), ((1, 1, 9), 3, 128, 1),
                                                    ((2, 3, 7), 4, 64, 3), ((2, 2, 3), 2, 126, 1),
                                                    ((1, 1, 1), 1, 128, 2), ((2, 3, 5), 4, 128, 2),
                                                    ((3, 2, 2), 16, 128, 1), ((1, 2, 3), 64, 128, 1),
                                                    ((1, 2, 2), 72, 128, 1)])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_rope_3d(hip, grid, heads, dim, samples, dtype):
    frames, rows, cols = grid
    tokens = samples * frames * rows * cols
    x = gaussian(5, (tokens, heads, dim), 3.0)
    step(f"rope3d {dtype} grid {grid} heads {heads} dim {dim} samples {samples}")
    if dtype == "f32":
        out = torch.empty(x.shape, dtype=torch.float32, device=DEV)
        hip.rope3d(dev_f32(x), frames, rows, cols, out)
        assert_f32(o.rope_3d(x, frames, rows, cols), host_f32(out), what="rope3d")
    else:
        xb = bf16_input(x)
        xd = dev_bf16(xb)
        hip.rope3d(xd, frames, rows, cols, xd)  # in place
        assert_bf16(o.rope_3d_bf16(xb, frames, rows, cols), host_bits(xd), what="rope3d bf16")


def test_rope_3d_c5_grid_window(hip):
    # C5's grid (21 x 30 x 52, 24 heads of 128): a window of tokens across the
    # first sample's last frame into the second sample's first, by offset
    step("rope3d bf16 on the C5 grid, tokens 31000..34999")
    x = gaussian(6, (4000, 24, 128))
    xb = bf16_input(x)
    out = torch.empty(x.shape, dtype=torch.bfloat16, device=DEV)
    hip.rope3d(dev_bf16(xb), 21, 30, 52, out, tokenOffset=31000)
    assert_bf16(o.rope_3d_bf16(xb, 21, 30, 52, token_offset=31000), host_bits(out), what="C5 window")


QK_CASES = [
    # (tokens, heads, kv_heads, dim, rope)
    (64, 32, 8, 128, d.Rope(1e6, 128, d.RopeLayout.Neox)),                   # Qwen3 (C3) shape
    (33, 16, 2, 256, d.Rope(1e7, 256, d.RopeLayout.Neox)),
    (17, 8, 8, 64, d.Rope(1e4, 64, d.RopeLayout.Interleaved)),
    (9, 4, 2, 128, d.Rope(1e6, 128, d.RopeLayout.Neox, R.Contiguous(24, 20, 20))),
    (9, 4, 2, 256, d.Rope(1e7, 64, d.RopeLayout.Neox)),                      # partial rotary: generic kernel
    (9, 3, 1, 80, d.Rope(1e4, 80, d.RopeLayout.Interleaved)),                # 80 values: generic kernel
    (5, 6, 0, 128, d.Rope(1e6, 128, d.RopeLayout.Neox)),                     # no key heads
    # two groups of heads a wave, the key waves' second group part-filled or empty
    (19, 16, 12, 128, d.Rope(1e6, 128, d.RopeLayout.Neox)),
    (11, 32, 4, 64, d.Rope(1e4, 64, d.RopeLayout.Interleaved)),
    # the grid's query waves first and its key waves after them: odd token
    # counts, one token, 1, 2 or 3 query waves a token; bf16 heads of 128 and
    # 64, F32 heads of 128; no query heads at all
    (7, 32, 8, 128, d.Rope(1e6, 128, d.RopeLayout.Neox)),
    (1, 32, 8, 128, d.Rope(1e6, 128, d.RopeLayout.Neox)),
    (9, 16, 8, 128, d.Rope(1e6, 128, d.RopeLayout.Neox)),
    (5, 48, 8, 128, d.Rope(1e4, 128, d.RopeLayout.Interleaved)),
    (13, 8, 4, 128, d.Rope(1e6, 128, d.RopeLayout.Neox)),
    (6, 64, 16, 64, d.Rope(1e4, 64, d.RopeLayout.Interleaved)),
    (5, 0, 8, 128, d.Rope(1e6, 128, d.RopeLayout.Neox)),
]


@pytest.mark.parametrize("case", range(len(QK_CASES)))
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_query_key_norm_rope(hip, case, dtype):
    tokens, heads, kv, dim, rope = QK_CASES[case]
    q = gaussian(7, (tokens, heads, dim))
    k = gaussian(8, (tokens, kv, dim))
    qw = (1 + 0.1 * gaussian(9, dim)).astype(np.float32)
    kw = (1 + 0.1 * gaussian(10, dim)).astype(np.float32)
    count = rope.sections.positionsPerToken
    p = ((np.arange(count * tokens) * 131) % 4096).astype(np.int32)
    p = p if count == 1 else p.reshape(count, tokens)
    args = (qw, kw, p, 1e-6, 0.0, rope.theta, rope.rotaryDimensions, int(rope.layout), rope.sections.code,
            rope.sections.sizes)
    norms = d.QueryKeyNorms(dev_f32(qw), dev_f32(kw), 1e-6, 0.0, rope)
    step(f"queryKeyNormRope {dtype} case {case}: {tokens} x ({heads} + {kv}) x {dim} {rope}")
    if dtype == "f32":
        rq = torch.empty(q.shape, dtype=torch.float32, device=DEV)
        rk = torch.empty(k.shape, dtype=torch.float32, device=DEV)
        hip.queryKeyNormRope(dev_f32(q), dev_f32(k), norms, dev_i32(p), rq, rk)
        wq, wk = o.qk_norm_rope(q, k, *args)
        assert_f32(wq, host_f32(rq), what="queries")
        assert_f32(wk, host_f32(rk), what="keys")
    else:
        qb, kb = bf16_input(q), bf16_input(k)
        qd, kd = dev_bf16(qb), dev_bf16(kb)
        hip.queryKeyNormRope(qd, kd, norms, dev_i32(p), qd, kd)  # in place
        wq, wk = o.qk_norm_rope_bf16(qb, kb, *args)
        assert_bf16(wq, host_bits(qd), what="queries bf16")
        assert_bf16(wk, host_bits(kd), what="keys bf16")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_query_key_norm_rope_zero_epsilon(hip, dtype):
    # epsilon 0 takes the inverse square root that handles a zero mean: a
    # zero head's 1 / sqrt(0) is infinite and 0 times it NaN, as in the
    # reference's double arithmetic; the other heads are normed as usual
    tokens, heads, kv, dim = 6, 16, 4, 128
    rope = d.Rope(1e6, 128, d.RopeLayout.Neox)
    q = gaussian(31, (tokens, heads, dim))
    k = gaussian(32, (tokens, kv, dim))
    q[1, 3] = 0.0
    q[4, 15] = 0.0
    k[2, 1] = 0.0
    qw = (1 + 0.1 * gaussian(33, dim)).astype(np.float32)
    kw = (1 + 0.1 * gaussian(34, dim)).astype(np.float32)
    p = ((np.arange(tokens) * 131) % 4096).astype(np.int32)
    args = (qw, kw, p, 0.0, 0.0, rope.theta, rope.rotaryDimensions, int(rope.layout), rope.sections.code,
            rope.sections.sizes)
    norms = d.QueryKeyNorms(dev_f32(qw), dev_f32(kw), 0.0, 0.0, rope)
    step(f"queryKeyNormRope {dtype}, epsilon 0, zero heads")
    if dtype == "f32":
        rq = torch.empty(q.shape, dtype=torch.float32, device=DEV)
        rk = torch.empty(k.shape, dtype=torch.float32, device=DEV)
        hip.queryKeyNormRope(dev_f32(q), dev_f32(k), norms, dev_i32(p), rq, rk)
        wq, wk = o.qk_norm_rope(q, k, *args)
        assert np.isnan(wq[1, 3]).all() and np.isnan(wk[2, 1]).all()
        assert_f32(wq, host_f32(rq), what="queries")
        assert_f32(wk, host_f32(rk), what="keys")
    else:
        qb, kb = bf16_input(q), bf16_input(k)
        rq = torch.empty(q.shape, dtype=torch.bfloat16, device=DEV)
        rk = torch.empty(k.shape, dtype=torch.bfloat16, device=DEV)
        hip.queryKeyNormRope(dev_bf16(qb), dev_bf16(kb), norms, dev_i32(p), rq, rk)
        wq, wk = o.qk_norm_rope_bf16(qb, kb, *args)
        assert_bf16(wq, host_bits(rq), what="queries bf16")
        assert_bf16(wk, host_bits(rk), what="keys bf16")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("far,offset", [(True, 0.0), (False, 1.0), (True, 1.0)])
def test_query_key_norm_rope_far_positions_and_weight_offsets(hip, dtype, far, offset):
    # positions whose angles pass 2^20 (pair 0 turns by the position itself)
    # take the library's sincos instead of the reduced one; a weight offset
    # (norms of 1 + w) takes the body that adds it
    tokens, heads, kv, dim = 24, 8, 2, 128
    rope = d.Rope(1e6, 128, d.RopeLayout.Neox)
    q = gaussian(21, (tokens, heads, dim))
    k = gaussian(22, (tokens, kv, dim))
    qw = (0.1 * gaussian(23, dim)).astype(np.float32)
    kw = (0.1 * gaussian(24, dim)).astype(np.float32)
    if far:
        p = np.array([0, 1, 1048575, 1048576, 1048577, 2000003, 3 << 20, 16777215, 12345678, 7, 999999, 1 << 23,
                      5000000, 65536, 4095, 2097151, 2097152, 8388607, 9000001, 31, 131071, 1 << 22, 123456, 6000000],
                     np.int32)
    else:
        p = ((np.arange(tokens) * 131) % 4096).astype(np.int32)
    args = (qw, kw, p, 1e-6, offset, rope.theta, rope.rotaryDimensions, int(rope.layout), rope.sections.code,
            rope.sections.sizes)
    norms = d.QueryKeyNorms(dev_f32(qw), dev_f32(kw), 1e-6, offset, rope)
    step(f"queryKeyNormRope {dtype}, positions {'past 2^20' if far else 'below 4096'}, weight offset {offset}")
    if dtype == "f32":
        rq = torch.empty(q.shape, dtype=torch.float32, device=DEV)
        rk = torch.empty(k.shape, dtype=torch.float32, device=DEV)
        hip.queryKeyNormRope(dev_f32(q), dev_f32(k), norms, dev_i32(p), rq, rk)
        wq, wk = o.qk_norm_rope(q, k, *args)
        assert_f32(wq, host_f32(rq), what="queries")
        assert_f32(wk, host_f32(rk), what="keys")
    else:
        qb, kb = bf16_input(q), bf16_input(k)
        rq = torch.empty(q.shape, dtype=torch.bfloat16, device=DEV)
        rk = torch.empty(k.shape, dtype=torch.bfloat16, device=DEV)
        hip.queryKeyNormRope(dev_bf16(qb), dev_bf16(kb), norms, dev_i32(p), rq, rk)
        wq, wk = o.qk_norm_rope_bf16(qb, kb, *args)
        assert_bf16(wq, host_bits(rq), what="queries bf16")
        assert_bf16(wk, host_bits(rk), what="keys bf16")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_query_key_norm_rope_with_weights_off_a_16_byte_boundary(hip, dtype):
    # norm weights that start 4 bytes into a buffer (a slice): the fast body
    # reads weights as 16-byte loads, so these take the general kernel
    tokens, heads, kv, dim = 16, 32, 8, 128
    rope = d.Rope(1e6, 128, d.RopeLayout.Neox)
    q = gaussian(31, (tokens, heads, dim))
    k = gaussian(32, (tokens, kv, dim))
    qw = (1 + 0.1 * gaussian(33, dim)).astype(np.float32)
    kw = (1 + 0.1 * gaussian(34, dim)).astype(np.float32)
    p = np.arange(tokens, dtype=np.int32)
    qw_at = dev_f32(np.concatenate([[7.0], qw]).astype(np.float32))[1:]
    kw_at = dev_f32(np.concatenate([[7.0, 7.0, 7.0], kw]).astype(np.float32))[3:]
    assert qw_at.data_ptr() % 16 == 4 and kw_at.data_ptr() % 16 == 12
    args = (qw, kw, p, 1e-6, 0.0, rope.theta, rope.rotaryDimensions, int(rope.layout), rope.sections.code,
            rope.sections.sizes)
    norms = d.QueryKeyNorms(qw_at, kw_at, 1e-6, 0.0, rope)
    step(f"queryKeyNormRope {dtype}, norm weights 4 and 12 bytes past a 16-byte boundary")
    if dtype == "f32":
        rq = torch.empty(q.shape, dtype=torch.float32, device=DEV)
        rk = torch.empty(k.shape, dtype=torch.float32, device=DEV)
        hip.queryKeyNormRope(dev_f32(q), dev_f32(k), norms, dev_i32(p), rq, rk)
        torch.cuda.synchronize()
        wq, wk = o.qk_norm_rope(q, k, *args)
        assert_f32(wq, host_f32(rq), what="queries")
        assert_f32(wk, host_f32(rk), what="keys")
    else:
        qb, kb = bf16_input(q), bf16_input(k)
        rq = torch.empty(q.shape, dtype=torch.bfloat16, device=DEV)
        rk = torch.empty(k.shape, dtype=torch.bfloat16, device=DEV)
        hip.queryKeyNormRope(dev_bf16(qb), dev_bf16(kb), norms, dev_i32(p), rq, rk)
        torch.cuda.synchronize()
        wq, wk = o.qk_norm_rope_bf16(qb, kb, *args)
        assert_bf16(wq, host_bits(rq), what="queries bf16")
        assert_bf16(wk, host_bits(rk), what="keys bf16")
