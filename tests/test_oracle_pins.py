"""Pins the CPU oracle before any kernel is checked against it.

Each check comes from outside the oracle's own formulas: the reference's
known-answer tests (runner/test/src/drift/runner/CpuOpsTests.scala,
ReferenceOpsTests.scala), independent library routines (torch float64,
numpy float16, math.erf), closed forms and invariants chosen so that a
plausible slip (a dropped term, a wrong pair or partner, a transposed
operand, a wrong rounding) fails at least one of them.
"""

import math

import numpy as np
import pytest
import torch

from oracle import oracle as o


def comparison_passes(expected, actual, absolute, relative):
    """tensor/Comparison.scala:32-74: |a - e| <= abs + rel |e|; NaN and
    infinities pass only against the same."""
    e = np.asarray(expected, np.float64).ravel()
    a = np.asarray(actual, np.float64).ravel()
    nan = np.isnan(e) | np.isnan(a)
    inf = np.isinf(e) | np.isinf(a)
    ok = np.where(nan, np.isnan(e) & np.isnan(a),
                  np.where(inf, e == a, np.abs(a - e) <= absolute + relative * np.abs(e)))
    return bool(ok.all())


def ulps_f32(a, b):
    """Distance in float32 ulps (on the ordered integer line)."""
    ia = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    ib = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    ia = np.where(ia < 0, -(ia & 0x7FFFFFFF), ia)
    ib = np.where(ib < 0, -(ib & 0x7FFFFFFF), ib)
    return np.abs(ia - ib)


def rng(seed):
    return np.random.default_rng(seed)


# ------------------------------------------------------------------ inputs

def test_java_gaussian_matches_java_util_random():
    # new java.util.Random(0).nextGaussian(), five draws (published values)
    expected = [0.8025330637390305, -0.9015460884175122, 2.080920790428163, 0.7637707684364019,
                0.9845745328825128]
    assert np.array_equal(o.java_gaussian(0, 5), np.array(expected, np.float32))


# ------------------------------------------------------------------ RMSNorm

def test_rms_norm_hand_worked_rows():
    # CpuOpsTests.scala:25-43
    x = np.array([[1, 2, 3, 4], [2, -2, 2, -2]], np.float32)
    w = np.array([1, 1, 1, 2], np.float32)
    r = math.sqrt(7.5)
    expected = np.array([1 / r, 2 / r, 3 / r, 8 / r, 1, -1, 1, -2], np.float32)
    assert comparison_passes(expected, o.rms_norm(x, w, 0.0), 1e-6, 1e-6)


def test_rms_norm_zero_row_stays_zero():
    # CpuOpsTests.scala:44-57
    out = o.rms_norm(np.zeros((1, 3), np.float32), np.ones(3, np.float32), 1e-6)
    assert np.all(out == 0)


@pytest.mark.parametrize("shape", [(1, 1), (3, 7), (2, 255), (5, 4097), (17, 2560), (8, 2048)])
def test_rms_norm_against_torch_float64(shape):
    x = (3 * rng(1).standard_normal(shape)).astype(np.float32)
    w = rng(2).standard_normal(shape[-1]).astype(np.float32)
    for offset in (0.0, 1.0):
        ref = torch.nn.functional.rms_norm(torch.from_numpy(x).double(), (shape[-1],),
                                           torch.from_numpy(w).double() + offset, eps=1e-6)
        got = o.rms_norm(x, w, 1e-6, offset)
        assert ulps_f32(got, ref.float().numpy()).max() <= 1


def test_rms_norm_invariants():
    x = rng(3).standard_normal((4, 64)).astype(np.float32)
    w = rng(4).standard_normal(64).astype(np.float32)
    # scale invariance: doubling x is exact in float, so eps = 0 gives the same bits
    assert np.array_equal(o.rms_norm(2 * x, w, 0.0), o.rms_norm(x, w, 0.0))
    # Gemma's offset of 1 with zero weights: unit root mean square
    unit = o.rms_norm(x, np.zeros(64, np.float32), 0.0, 1.0)
    assert np.allclose(np.sqrt((unit.astype(np.float64) ** 2).mean(axis=1)), 1.0, atol=1e-6)


def test_add_rms_norm_and_weight_rows():
    x = rng(5).standard_normal((6, 32)).astype(np.float32)
    y = rng(6).standard_normal((6, 32)).astype(np.float32)
    w = rng(7).standard_normal((3, 32)).astype(np.float32)
    summed, out = o.rms_norm(x, w, 1e-5, 0.0, y=y, weight_rows=3)
    assert np.array_equal(summed, (x.astype(np.float64) + y).astype(np.float32))
    for r in range(6):
        assert np.array_equal(out[r], o.rms_norm(summed[r:r + 1], w[r % 3], 1e-5)[0])


# ------------------------------------------------------------------ LayerNorm / AdaLN

def test_layer_norm_zero_mean_unit_variance():
    # ReferenceOpsTests.scala:88-97
    out = o.layer_norm(np.array([[1, 2, 3, 6]], np.float32), None, None, 0.0).astype(np.float64)
    assert abs(out.sum()) < 1e-6
    assert abs((out * out).sum() / 4 - 1) < 1e-6


@pytest.mark.parametrize("affine", [(False, False), (True, False), (False, True), (True, True)])
def test_layer_norm_against_torch_float64(affine):
    x = (3 * rng(8).standard_normal((17, 2560))).astype(np.float32)
    w = rng(9).standard_normal(2560).astype(np.float32) if affine[0] else None
    b = rng(10).standard_normal(2560).astype(np.float32) if affine[1] else None
    ref = torch.nn.functional.layer_norm(
        torch.from_numpy(x).double(), (2560,), None if w is None else torch.from_numpy(w).double(),
        None if b is None else torch.from_numpy(b).double(), eps=1e-5)
    assert ulps_f32(o.layer_norm(x, w, b, 1e-5), ref.float().numpy()).max() <= 1


def test_layer_norm_shift_invariance_and_plain_modulate():
    x = rng(11).standard_normal((4, 3072)).astype(np.float32)
    plain = o.layer_norm(x, None, None, 1e-6)
    shifted = o.layer_norm(x + np.float32(8.0), None, None, 1e-6)
    assert np.abs(plain - shifted).max() < 1e-5
    zeros = np.zeros(3072, np.float32)
    assert np.array_equal(o.modulate(plain, zeros, zeros), plain)


def test_modulate_closed_form():
    x = rng(12).standard_normal((5, 64)).astype(np.float32)
    s = rng(13).standard_normal(64).astype(np.float32)
    sh = rng(14).standard_normal(64).astype(np.float32)
    expected = (x.astype(np.float64) * (1 + s.astype(np.float64)) + sh).astype(np.float32)
    assert np.array_equal(o.modulate(x, s, sh), expected)


def test_layer_norm_modulate_uses_each_samples_rows():
    x = rng(15).standard_normal((6, 48)).astype(np.float32)
    s = (0.1 * rng(16).standard_normal((2, 48))).astype(np.float32)
    sh = (0.1 * rng(17).standard_normal((2, 48))).astype(np.float32)
    out = o.layer_norm_modulate(x, s, sh, 3, 1e-6)
    normed = o.layer_norm(x, None, None, 1e-6)
    assert np.array_equal(out[:3], o.modulate(normed[:3], s[0], sh[0]))
    assert np.array_equal(out[3:], o.modulate(normed[3:], s[1], sh[1]))


# ------------------------------------------------------------------ activations

def test_erf_against_abramowitz_stegun():
    # ReferenceOpsTests.scala:33-46 (A&S table 7.1)
    for x, e in [(0.0, 0.0), (0.5, 0.5204998778), (1.0, 0.8427007929), (2.0, 0.9953222650),
                 (3.0, 0.9999779095)]:
        assert abs(o.erf(x) - e) < 1e-9
        assert abs(o.erf(-x) + e) < 1e-9


def test_erf_against_libm():
    # the reference documents its erf as good to about 1e-15 (ops/CpuOps.scala:26-28);
    # its series gives up a few more ulps just below 2.5
    for x in np.linspace(-6, 6, 1201):
        assert abs(o.erf(float(x)) - math.erf(float(x))) < 1e-14


def test_activations_at_known_points():
    # ReferenceOpsTests.scala:47-72
    x = np.array([-1, 0, 2], np.float32)
    e = math.e
    assert comparison_passes([-1 / (1 + e), 0, 2 / (1 + math.exp(-2))], o.activation(o.SILU, x), 1e-7, 0)
    assert comparison_passes([1 / (1 + e), 0.5, 1 / (1 + math.exp(-2))], o.activation(o.SIGMOID, x), 1e-7, 0)
    exact_gelu = [-0.1586552539, 0, 1.9544997361]
    assert comparison_passes(exact_gelu, o.activation(o.GELU_ERF, x), 1e-7, 0)
    assert comparison_passes(exact_gelu, o.activation(o.GELU_TANH, x), 1e-3, 0)


def test_activations_against_torch_float64():
    x = (3 * rng(18).standard_normal(20000)).astype(np.float32)
    t = torch.from_numpy(x).double()
    F = torch.nn.functional
    refs = {
        o.SILU: F.silu(t),
        o.GELU_TANH: F.gelu(t, approximate="tanh"),
        o.GELU_ERF: F.gelu(t),
        o.SIGMOID: torch.sigmoid(t),
        o.SITU: 4 * torch.tanh(t / 4) * torch.sigmoid(t),
    }
    # Below about -5, 1 + tanh(u) keeps few bits in double and the result
    # depends on how the libm rounds tanh's last bit: pinned separately.
    conditioned = x > -5
    for kind, ref in refs.items():
        got, want = o.activation(kind, x), ref.float().numpy()
        assert ulps_f32(got[conditioned], want[conditioned]).max() <= 1, kind


def test_gelu_tanh_deep_tail_uses_correctly_rounded_tanh():
    # 0.5 v (1 + tanh(u)) with tanh(u) rounded to the nearest double: in the
    # tail 1 + tanh(u) is a multiple of 2^-53, and 0 once tanh rounds to -1.
    mpmath = pytest.importorskip("mpmath")
    mpmath.mp.prec = 200
    x = np.linspace(-12, -5, 701).astype(np.float32)
    k = math.sqrt(2 / math.pi)
    expected = []
    for v in x.astype(np.float64):
        u = k * (v + 0.044715 * v * v * v)
        t = float(mpmath.tanh(mpmath.mpf(u)))  # rounded to nearest double
        expected.append(np.float32(0.5 * v * (1 + t)))
    assert np.array_equal(o.activation(o.GELU_TANH, x), np.array(expected, np.float32))


def test_activation_input_scale_multiplies_in_double():
    x = rng(19).standard_normal(1000).astype(np.float32)
    scale = np.float32(0.37)
    expected = np.array([o.activate(o.GELU_TANH, float(scale) * float(v)) for v in x]).astype(np.float32)
    assert np.array_equal(o.activation(o.GELU_TANH, x, float(scale)), expected)


def test_gated_against_torch_float64():
    g = (3 * rng(20).standard_normal(5000)).astype(np.float32)
    u = (3 * rng(21).standard_normal(5000)).astype(np.float32)
    tg, tu = torch.from_numpy(g).double(), torch.from_numpy(u).double()
    F = torch.nn.functional
    assert ulps_f32(o.gated(o.SILU, g, u), (F.silu(tg) * tu).float().numpy()).max() <= 1
    conditioned = g > -5  # the GELU-tanh tail is pinned on its own above
    geglu = o.gated(o.GELU_TANH, g, u)[conditioned]
    assert ulps_f32(geglu, (F.gelu(tg, approximate="tanh") * tu).float().numpy()[conditioned]).max() <= 1
    situ = 4 * torch.tanh(tg / 4) * torch.sigmoid(tg) * 25 * torch.tanh(tu / 25)
    assert ulps_f32(o.gated(o.SITU, g, u), situ.float().numpy()).max() <= 1


# ------------------------------------------------------------------ RoPE

def test_rope_hand_worked_pairs():
    # ReferenceOpsTests.scala:98-131: theta 100, one head of 4, position 1
    x = np.array([[[1, 1, 0, 0]]], np.float32)
    p = np.array([1], np.int32)
    a0, a1 = 1.0, 0.1
    inter = o.rope(x, p, 100.0, 4, o.INTERLEAVED)
    assert comparison_passes([math.cos(a0) - math.sin(a0), math.sin(a0) + math.cos(a0), 0, 0], inter, 1e-6, 0)
    neox = o.rope(x, p, 100.0, 4, o.NEOX)
    assert comparison_passes([math.cos(a0), math.cos(a1), math.sin(a0), math.sin(a1)], neox, 1e-6, 0)


def test_rope_partial_and_position_zero():
    # ReferenceOpsTests.scala:132-154
    values = np.array([[[1, 2, 3, 4, 5, 6]]], np.float32)
    out = o.rope(values, np.array([7], np.int32), 1e4, 2, o.NEOX)
    assert np.array_equal(out[..., 2:], values[..., 2:])
    assert np.array_equal(o.rope(values, np.array([0], np.int32), 1e4, 6, o.NEOX), values)


def test_mrope_with_equal_positions_is_plain_rope():
    # ReferenceOpsTests.scala:155-183
    x = o.java_gaussian(1, 128).reshape(2, 1, 64)
    plain = o.rope(x, np.array([5, 9], np.int32), 1e6, 64, o.NEOX)
    equal = np.array([5, 9, 5, 9, 5, 9], np.int32)
    for sections in (o.CONTIGUOUS, o.INTERLEAVED_MROPE):
        assert np.array_equal(o.rope(x, equal, 1e6, 64, o.NEOX, sections, (11, 11, 10)), plain)


def test_rope_inverse_frequency_within_an_ulp_of_float64():
    for theta, rotary in [(1e4, 128), (1e6, 128), (1e7, 64), (100.0, 4)]:
        for pair in range(rotary // 2):
            exact = np.float64(theta) ** (-2.0 * pair / rotary)
            got = o.rope_inverse_frequency(pair, rotary, theta)
            assert ulps_f32(np.float32(got), np.float32(exact)) <= 1
    # axes: each axis' pair j of n turns by theta^(-j/n); a new axis starts at 1
    sizes = (16, 24, 24)
    for pair, j, n in [(0, 0, 16), (15, 15, 16), (16, 0, 24), (39, 23, 24), (40, 0, 24), (63, 23, 24)]:
        got = o.rope_inverse_frequency(pair, 128, 1e3, o.AXES, sizes)
        assert ulps_f32(np.float32(got), np.float32(1e3 ** (-j / n))) <= 1


def test_neox_is_interleaved_on_permuted_values():
    # NeoX pairs (i, i + half); interleaved pairs (2i, 2i + 1): the same turn
    # once the values are permuted, bit for bit.
    x = rng(22).standard_normal((9, 3, 128)).astype(np.float32)
    p = ((np.arange(9) * 131) % 4096).astype(np.int32)
    perm = np.empty(128, np.int64)
    perm[0::2] = np.arange(64)
    perm[1::2] = np.arange(64) + 64
    neox = o.rope(x, p, 1e4, 128, o.NEOX)
    inter = o.rope(x[..., perm], p, 1e4, 128, o.INTERLEAVED)
    assert np.array_equal(neox[..., perm], inter)


def test_rope_preserves_pair_norms_and_inverts():
    x = rng(23).standard_normal((5, 2, 64)).astype(np.float32)
    p = np.array([3, 100, 1000, 4095, 77], np.int32)
    out = o.rope(x, p, 1e4, 64, o.INTERLEAVED).astype(np.float64)
    xin = x.astype(np.float64)
    assert np.allclose(out[..., 0::2] ** 2 + out[..., 1::2] ** 2, xin[..., 0::2] ** 2 + xin[..., 1::2] ** 2,
                       rtol=1e-6, atol=1e-6)
    back = o.rope(out.astype(np.float32), -p, 1e4, 64, o.INTERLEAVED)
    assert np.abs(back - x).max() < 1e-5


def test_rope_table_agrees_with_rope_and_copies_the_tail():
    x = rng(24).standard_normal((7, 3, 128)).astype(np.float32)
    p = ((np.arange(7) * 131) % 4096).astype(np.int32)
    inv = np.array([o.rope_inverse_frequency(i, 96, 1e4) for i in range(48)], np.float32)
    angles = (p[:, None].astype(np.float32) * inv[None, :]).astype(np.float64)
    cos, sin = np.cos(angles).astype(np.float32), np.sin(angles).astype(np.float32)
    for halves, layout in [(False, o.INTERLEAVED), (True, o.NEOX)]:
        table = o.rope_table(x, cos, sin, halves)
        direct = o.rope(x, p, 1e4, 96, layout)
        assert np.abs(table - direct).max() < 1e-5
        assert np.array_equal(table[..., 96:], x[..., 96:])
        per_head = o.rope_table(x, np.repeat(cos[:, None], 3, 1), np.repeat(sin[:, None], 3, 1), halves)
        assert np.array_equal(per_head, table)


# ------------------------------------------------------------------ Wan 3-D RoPE

def test_wan_pairs():
    # models/Wan.scala:35-41: d - 4 floor(d/6), 2 floor(d/6), 2 floor(d/6), halved
    assert o.wan_pairs(128) == (22, 21, 21)
    assert o.wan_pairs(64) == (12, 10, 10)


def test_wan_angles_closed_form_and_special_grids():
    frames, rows, cols = 3, 4, 5
    cos, sin = o.wan_angles(frames, rows, cols)
    t = np.arange(frames * rows * cols)
    pos = [t // (rows * cols), t // cols % rows, t % cols]
    pairs = (22, 21, 21)
    start = 0
    for axis, n in enumerate(pairs):
        for j in range(n):
            angle = pos[axis] / 10000.0 ** (2.0 * j / (2 * n))
            assert ulps_f32(cos[:, start + j], np.cos(angle).astype(np.float32)).max() <= 1
            assert ulps_f32(sin[:, start + j], np.sin(angle).astype(np.float32)).max() <= 1
        start += n
    # a 1 x 1 x W grid turns only the column pairs; 1 x 1 x 1 is the identity
    cos, sin = o.wan_angles(1, 1, 9)
    assert np.all(cos[:, :43] == 1) and np.all(sin[:, :43] == 0)
    x = rng(25).standard_normal((1, 2, 128)).astype(np.float32)
    assert np.array_equal(o.rope_3d(x, 1, 1, 1), x)
    # the column pairs of a 1 x 1 x W grid: interleaved RoPE on values 86.. by col / theta^(2j/42)
    x = rng(26).standard_normal((9, 2, 128)).astype(np.float32)
    out = o.rope_3d(x, 1, 1, 9)
    assert np.array_equal(out[..., :86], x[..., :86])
    col = np.arange(9, dtype=np.float64)
    ang = col[:, None] / 10000.0 ** (2.0 * np.arange(21) / 42)
    a, b = x[..., 86::2].astype(np.float64), x[..., 87::2].astype(np.float64)
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    assert np.abs(out[..., 86::2] - (a * c - b * s)).max() < 1e-5
    assert np.abs(out[..., 87::2] - (a * s + b * c)).max() < 1e-5


def test_rope_3d_token_offset_wraps_the_grid():
    x = rng(27).standard_normal((10, 1, 128)).astype(np.float32)
    both = o.rope_3d(np.concatenate([x, x]), 2, 1, 5)
    assert np.array_equal(both[:10], both[10:])
    assert np.array_equal(o.rope_3d(x[4:], 2, 1, 5, token_offset=4), both[4:10])


# ------------------------------------------------------------------ conversions

def test_bf16_round_to_nearest_even_known_answers():
    # ReferenceOpsTests.scala:184-213
    values = np.array([1, 1 + 2 ** -8, 1 + 3 * 2 ** -8, 65504, -0.5], np.float32)
    back = o.from_bf16(o.to_bf16(values))
    assert np.array_equal(back, np.array([1, 1, 1 + 2 ** -6, 65536, -0.5], np.float32))
    assert np.array_equal(o.from_f16(o.to_f16(values)), values)


def test_bf16_nan_keeps_top_half_with_quiet_bit():
    # CpuOps.toBfloat16: NaN -> (bits >>> 16) | 0x40
    bits = np.array([0x7FC00000, 0x7F800001, 0xFF812345, 0x7FFFFFFF], np.uint32)
    expected = np.array([0x7FC0, 0x7FC0, 0xFFC1, 0x7FFF], np.uint16)
    assert np.array_equal(o.to_bf16(bits.view(np.float32)), expected)


def _f32_sample():
    r = rng(28)
    random_bits = r.integers(0, 2 ** 32, 4_000_000, dtype=np.uint64).astype(np.uint32)
    hi = r.integers(0, 2 ** 16, 200_000, dtype=np.uint64).astype(np.uint32) << 16
    ties = np.concatenate([hi | 0x7FFF, hi | 0x8000, hi | 0x8001, hi, hi | 0xFFFF])
    special = np.array([0, 0x80000000, 0x7F800000, 0xFF800000, 0x7F7FFFFF, 0x00000001, 0x007FFFFF,
                        0x7F7F8000, 0x7F7F7FFF], np.uint32)
    return np.concatenate([random_bits, ties, special]).view(np.float32)


def test_bf16_rounding_matches_torch_on_non_nan():
    x = _f32_sample()
    x = x[~np.isnan(x)]
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(o.to_bf16(x), ref)
    assert np.array_equal(o.from_bf16(ref), torch.from_numpy(ref.view(np.int16)).view(torch.bfloat16).float().numpy())


def test_f16_conversions_match_numpy():
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = codes.view(np.float16).astype(np.float32)
    got = o.from_f16(codes)
    finite = ~np.isnan(ref)
    assert np.array_equal(got[finite].view(np.uint32), ref[finite].view(np.uint32))
    assert np.all(np.isnan(got[~finite]))
    x = _f32_sample()
    x = x[~np.isnan(x)]
    with np.errstate(over="ignore"):
        assert np.array_equal(o.to_f16(x), x.astype(np.float16).view(np.uint16))


# ------------------------------------------------------------------ Q8_0 gather

def test_q8_0_gather_every_code_and_scale_class_exact():
    # every int8 code against scales that are zero, subnormal, normal, negative and the largest f16
    scales = np.array([0.0, -0.0, 2 ** -24, 3 * 2 ** -24, 6.1e-5, 1e-3, 0.0123, -0.5, 1.0, 65504.0, -65504.0],
                      np.float16)
    codes = np.arange(-128, 128, dtype=np.int32)
    blocks = []
    for s in scales:
        for chunk in codes.reshape(8, 32):
            blocks.append(np.concatenate([np.array([s], np.float16).view(np.uint8), chunk.astype(np.int8).view(np.uint8)]))
    cols = 32 * 8
    table = np.stack(blocks).reshape(len(scales), cols // 32 * 34)
    out = o.embedding_q8_0(table, len(scales), cols, np.arange(len(scales), dtype=np.int32))
    expected = codes.astype(np.float32)[None, :] * scales.astype(np.float32)[:, None]
    assert np.array_equal(out.view(np.uint32), expected.view(np.uint32))
    ref_bf16 = torch.from_numpy(expected).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(o.embedding_q8_0_bf16(table, len(scales), cols, np.arange(len(scales))), ref_bf16)


def test_q8_0_gather_random_rows_and_refused_ids():
    r = rng(29)
    table = o.q8_0_table(50, 256, r)
    ids = r.integers(0, 50, 40).astype(np.int32)
    out = o.embedding_q8_0(table, 50, 256, ids)
    blocks = table.reshape(50, 8, 34)
    d = blocks[:, :, 0:2].copy().view(np.float16).astype(np.float32)
    q = blocks[:, :, 2:].view(np.int8).astype(np.float32)
    expected = (q * d).reshape(50, 256)[ids]
    assert np.array_equal(out, expected)
    for bad in (-1, 50):
        with pytest.raises(ValueError, match="outside the table"):
            o.embedding_q8_0(table, 50, 256, np.array([0, bad], np.int32))


def test_f32_embedding_copies_rows():
    table = rng(30).standard_normal((10, 16)).astype(np.float32)
    assert np.array_equal(o.embedding_f32(table, [2, 0, 3]), table[[2, 0, 3]])
