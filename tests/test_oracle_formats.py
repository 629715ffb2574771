"""Pins the oracle's decoders of the runner's storage types (CPU only).

The reference checks its decoders against gguf-py goldens
(runner/test/src/drift/runner/DTypeTests.scala), which are Git LFS pointers in
the checkout, and gguf-py itself is not installed here. So each decoder is
held, bit for bit over random blocks, to an independent restatement of
ggml's own dequantize_row_* loops (ggml-quants.c: the published algorithm,
written here in numpy with its loop structure, not the Scala's per-element
formulas), plus hand-worked known answers. ROCmFP4's scale is pinned to the
OCP E4M3 definition; its codebook is the reference's table (no independent
source: the fork's rocmfp4.c is not in the checkout).
"""

import numpy as np
import pytest

from oracle import oracle as o

F = np.float32


def f16(lo, hi):
    return np.array([int(lo) | (int(hi) << 8)], np.uint16).view(np.float16).astype(F)[0]


def u32(b, at):
    return int(b[at]) | (int(b[at + 1]) << 8) | (int(b[at + 2]) << 16) | (int(b[at + 3]) << 24)


def ggml_q4_0(b):
    d = f16(b[0], b[1])
    qs = b[2:18].astype(np.int32)
    return np.concatenate([((qs & 0xF) - 8).astype(F) * d, ((qs >> 4) - 8).astype(F) * d])


def ggml_q4_1(b):
    d, m = f16(b[0], b[1]), f16(b[2], b[3])
    qs = b[4:20].astype(np.int32)
    return np.concatenate([(qs & 0xF).astype(F) * d + m, (qs >> 4).astype(F) * d + m])


def ggml_q5(b, with_min):
    d = f16(b[0], b[1])
    m = f16(b[2], b[3]) if with_min else None
    at = 4 if with_min else 2
    qh = u32(b, at)
    qs = b[at + 4:at + 20].astype(np.int32)
    y = np.empty(32, F)
    for j in range(16):
        xh0 = ((qh >> (j + 0)) << 4) & 0x10
        xh1 = (qh >> (j + 12)) & 0x10
        x0 = (qs[j] & 0x0F) | xh0
        x1 = (qs[j] >> 4) | xh1
        if with_min:
            y[j], y[j + 16] = F(x0) * d + m, F(x1) * d + m
        else:
            y[j], y[j + 16] = F(x0 - 16) * d, F(x1 - 16) * d
    return y


def ggml_q8_0(b):
    return b[2:34].view(np.int8).astype(F) * f16(b[0], b[1])


def get_scale_min_k4(j, q):
    if j < 4:
        return q[j] & 63, q[j + 4] & 63
    return (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4), (q[j + 4] >> 4) | ((q[j] >> 6) << 4)


def ggml_q4_k(b, five=False):
    d, dmin = f16(b[0], b[1]), f16(b[2], b[3])
    scales = b[4:16].astype(np.int32)
    qh = b[16:48].astype(np.int32) if five else None
    ql = b[48:176].astype(np.int32) if five else b[16:144].astype(np.int32)
    y = np.empty(256, F)
    u1, u2, is_, out = 1, 2, 0, 0
    for j in range(0, 256, 64):
        sc, m = get_scale_min_k4(is_ + 0, scales)
        d1, m1 = d * F(sc), dmin * F(m)
        sc, m = get_scale_min_k4(is_ + 1, scales)
        d2, m2 = d * F(sc), dmin * F(m)
        q = ql[(j // 64) * 32:(j // 64) * 32 + 32]
        for l in range(32):
            h1 = 16 if five and (qh[l] & u1) else 0
            h2 = 16 if five and (qh[l] & u2) else 0
            y[out + l] = d1 * F((q[l] & 0xF) + h1) - m1
            y[out + l + 32] = d2 * F((q[l] >> 4) + h2) - m2
        out += 64
        is_ += 2
        u1 <<= 2
        u2 <<= 2
    return y


def ggml_q6_k(b):
    ql, qh = b[0:128].astype(np.int32), b[128:192].astype(np.int32)
    sc = b[192:208].view(np.int8).astype(np.int32)
    d = f16(b[208], b[209])
    y = np.empty(256, F)
    for n in range(2):
        q_l, q_h, s, base = ql[64 * n:], qh[32 * n:], sc[8 * n:], 128 * n
        for l in range(32):
            is_ = l // 16
            q1 = ((q_l[l + 0] & 0xF) | (((q_h[l] >> 0) & 3) << 4)) - 32
            q2 = ((q_l[l + 32] & 0xF) | (((q_h[l] >> 2) & 3) << 4)) - 32
            q3 = ((q_l[l + 0] >> 4) | (((q_h[l] >> 4) & 3) << 4)) - 32
            q4 = ((q_l[l + 32] >> 4) | (((q_h[l] >> 6) & 3) << 4)) - 32
            y[base + l + 0] = d * F(s[is_ + 0]) * F(q1)
            y[base + l + 32] = d * F(s[is_ + 2]) * F(q2)
            y[base + l + 64] = d * F(s[is_ + 4]) * F(q3)
            y[base + l + 96] = d * F(s[is_ + 6]) * F(q4)
    return y


KVALUES = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], F)


def ggml_iq4_nl(b):
    d = f16(b[0], b[1])
    qs = b[2:18].astype(np.int32)
    return np.concatenate([d * KVALUES[qs & 0xF], d * KVALUES[qs >> 4]])


def ggml_iq4_xs(b):
    d = f16(b[0], b[1])
    scales_h = int(b[2]) | (int(b[3]) << 8)
    y = np.empty(256, F)
    for ib in range(8):
        ls = ((int(b[4 + ib // 2]) >> 4 * (ib % 2)) & 0xF) | (((scales_h >> 2 * ib) & 3) << 4)
        dl = d * F(ls - 32)
        qs = b[8 + 16 * ib:24 + 16 * ib].astype(np.int32)
        y[32 * ib:32 * ib + 16] = dl * KVALUES[qs & 0xF]
        y[32 * ib + 16:32 * ib + 32] = dl * KVALUES[qs >> 4]
    return y


def e4m3_unsigned(byte):
    """OCP FP8 E4M3 (bias 7) read as unsigned, its top bit unused; 0x7f is NaN."""
    e, m = int(byte) >> 3, int(byte) & 7
    return (m / 8) * 2.0 ** -6 if e == 0 else (1 + m / 8) * 2.0 ** (e - 7)


CODEBOOK = np.array([0, 1, 2, 3, 4, 6, 8, 10, 0, -1, -2, -3, -4, -6, -8, -10], F)


def rocm(b, fast):
    lo = F(e4m3_unsigned(b[16]) / 2) if b[16] <= 0x7E else F(0)
    hb = b[16] if fast else b[17]
    hi = F(e4m3_unsigned(hb) / 2) if hb <= 0x7E else F(0)
    qs = b[0:16].astype(np.int32)
    return np.concatenate([CODEBOOK[qs & 0xF] * lo, CODEBOOK[qs >> 4] * hi])


INDEPENDENT = {
    "Q4_0": ggml_q4_0, "Q4_1": ggml_q4_1, "Q5_0": lambda b: ggml_q5(b, False), "Q5_1": lambda b: ggml_q5(b, True),
    "Q8_0": ggml_q8_0, "Q4_K": ggml_q4_k, "Q5_K": lambda b: ggml_q4_k(b, True), "Q6_K": ggml_q6_k,
    "IQ4_NL": ggml_iq4_nl, "IQ4_XS": ggml_iq4_xs, "Q4_0_ROCMFP4": lambda b: rocm(b, False),
    "Q4_0_ROCMFP4_FAST": lambda b: rocm(b, True),
}


@pytest.mark.parametrize("name", sorted(INDEPENDENT))
def test_decoders_match_ggml_loops(name):
    rng = np.random.default_rng(sum(map(ord, name)))
    values, size = o.format_block(name)
    blocks = 24
    table = o.quant_table(name, 1, values * blocks, rng)[0]
    got = o.decode_row(name, table, values * blocks)
    want = np.concatenate([INDEPENDENT[name](table[b * size:(b + 1) * size]) for b in range(blocks)])
    assert np.array_equal(got.view(np.uint32), want.astype(F).view(np.uint32)), name


def test_dense_types():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((2, 16)).astype(F)
    assert np.array_equal(o.decode_row("F32", x[0].view(np.uint8), 16), x[0])
    h = x[1].astype(np.float16)
    assert np.array_equal(o.decode_row("F16", h.view(np.uint8), 16), h.astype(F))
    b = o.to_bf16(x[1])
    assert np.array_equal(o.decode_row("BF16", b.view(np.uint8), 16), o.from_bf16(b))


def test_known_answers():
    # Q4_0 block: d = 1.0 (0x3c00), bytes 0x9F: element 0 = 15 - 8, element 16 = 9 - 8
    b = np.zeros(18, np.uint8)
    b[0:2] = [0x00, 0x3C]
    b[2] = 0x9F
    y = o.decode_row("Q4_0", b, 32)
    assert y[0] == 7 and y[16] == 1 and y[1] == -8
    # Q4_K: scale j=5 takes its high bits from byte 1's top two, its low from byte 9's low nibble
    b = np.zeros(144, np.uint8)
    b[0:2] = [0x00, 0x3C]  # d = 1
    b[4 + 1] = 0b11000000  # top bits of the 6-bit scale of sub-block 5
    b[4 + 9] = 0x03        # low nibble of it: scale 0b110011 = 51
    b[16 + 64] = 0x20  # element 160 (sub-block 5, first) nibble: high nibble of byte 64 = 2
    y = o.decode_row("Q4_K", b, 256)
    assert y[160] == 51 * 2 and np.count_nonzero(y) == 1
    # IQ4_NL: nibble 8 maps to 1, nibble 0 to -127
    b = np.zeros(18, np.uint8)
    b[0:2] = [0x00, 0x40]  # d = 2
    b[2] = 0x08
    y = o.decode_row("IQ4_NL", b, 32)
    assert y[0] == 2 and y[16] == -254


@pytest.mark.parametrize("byte", [0x00, 0x01, 0x07, 0x08, 0x38, 0x3F, 0x7E, 0x7F, 0x80, 0xFF])
def test_rocmfp4_scale_is_half_an_unsigned_e4m3(byte):
    want = e4m3_unsigned(byte) / 2 if byte <= 0x7E else 0.0
    assert o.rocmfp4_half_scale(byte) == want
