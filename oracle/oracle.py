"""Test infrastructure only: numpy front end of the CPU oracle (cpu_ops.c).

The oracle restates the drift runner's CPU reference backend (`CpuOps`,
ops/CpuOps.scala) for the fused layer kernels' path. Tests compare the HIP
kernels with it, bench.py times it as the CPU baseline, and
__graft_entry__.smoke() checks one launch against it. The product never
imports this module.

Compositions for the bf16 configurations follow the reference's own bf16
path: `convert` BF16 -> F32 (tensor/DType.scala:99-102), the F32 op, then
`convert` F32 -> BF16 (ops/CpuMemory.scala:84-109, CpuOps.toBfloat16).
"""

from __future__ import annotations

import ctypes
import math
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libdrift_oracle.so")

SILU, GELU_TANH, GELU_ERF, SIGMOID, SITU = range(5)
NEOX, INTERLEAVED = 0, 1
SINGLE, CONTIGUOUS, INTERLEAVED_MROPE, AXES = range(4)


def build() -> str:
    """Compile cpu_ops.c with the Makefile beside it; return the library path."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int
_F32 = ctypes.c_float
_F64 = ctypes.c_double


def _declare(l: ctypes.CDLL) -> None:
    sig = {
        "oracle_format_block": (_I32, [_I32, _P, _P]),
        "oracle_rocmfp4_half_scale": (_F32, [_I32]),
        "oracle_decode_row": (_I32, [_I32, _P, _I64, _P]),
        "oracle_embedding": (_I64, [_I32, _P, _I64, _I64, _P, _I64, _P]),
        "oracle_to_bf16": (ctypes.c_uint16, [_F32]),
        "oracle_from_bf16": (_F32, [ctypes.c_uint16]),
        "oracle_f16_to_f32": (_F32, [ctypes.c_uint16]),
        "oracle_f32_to_f16": (ctypes.c_uint16, [_F32]),
        "oracle_f32_to_bf16_n": (None, [_P, _P, _I64]),
        "oracle_bf16_to_f32_n": (None, [_P, _P, _I64]),
        "oracle_f32_to_f16_n": (None, [_P, _P, _I64]),
        "oracle_f16_to_f32_n": (None, [_P, _P, _I64]),
        "oracle_erf": (_F64, [_F64]),
        "oracle_activate": (_F64, [_I32, _F64]),
        "oracle_activation": (None, [_I32, _F32, _P, _P, _I64]),
        "oracle_gated": (None, [_I32, _P, _P, _P, _I64]),
        "oracle_rms_norm": (None, [_P, _P, _P, _P, _I64, _I64, _F32, _F32, _I64]),
        "oracle_layer_norm": (None, [_P, _P, _P, _P, _I64, _I64, _F32]),
        "oracle_modulate": (None, [_P, _P, _P, _P, _I64, _I64]),
        "oracle_rope": (None, [_P, _P, _P, _I32, _I32, _I32, _I32, _F32, _I32, _I32, _P]),
        "oracle_rope_inverse_frequency": (_F32, [_I32, _I32, _F32, _I32, _P]),
        "oracle_rope_table": (None, [_P, _P, _P, _P, _I32, _I32, _I32, _I32, _I32, _I32]),
        "oracle_wan_pairs": (None, [_I32, _P]),
        "oracle_wan_angles": (None, [_I32, _I32, _I32, _I32, _F64, _P, _P]),
        "oracle_embedding_q8_0": (_I64, [_P, _I64, _I64, _P, _I64, _P]),
        "oracle_embedding_f32": (_I64, [_P, _I64, _I64, _P, _I64, _P]),
        "oracle_quantize_x": (None, [_P, _P, _P, _P, _I64]),
        "oracle_gated_add": (None, [_P, _P, _P, _I64, _I64, _I64]),
        "oracle_modulate_chunks": (None, [_P, _P, _P, _I64, _I64, _I64, _I64, _I64]),
        "oracle_gated_add_chunk": (None, [_P, _P, _P, _I64, _I64, _I64, _I64]),
        "oracle_row_gated_add": (None, [_P, _P, _P, _I64, _I64]),
        "oracle_f8e4m3": (_F32, [_I32]),
        "oracle_convrot_rotate": (None, [_P, _I64, _I64]),
        "oracle_convrot_levels": (None, [_P, _P, _I64, _P, _P, _I64, _I64, _I64, _I64, _P]),
        "oracle_convrot_rows": (None, [_P, _P, _I64, _P, _P, _I64, _I64, _I64, _I64, _P]),
        "oracle_convrot_embedding": (_I64, [_P, _P, _I64, _P, _P, _I64, _I64, _I64, _P, _I64, _P]),
    }
    for name, (restype, argtypes) in sig.items():
        fn = getattr(l, name)
        fn.restype = restype
        fn.argtypes = argtypes


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data


def _need(condition: bool, message: str) -> None:
    """Shapes are checked here, before the C loops index the arrays."""
    if not condition:
        raise ValueError(message)


def _c(a, dtype) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=dtype)


# ---------------------------------------------------------------- conversions

def to_bf16(x) -> np.ndarray:
    """F32 -> BF16 bits, CpuOps.toBfloat16 (ops/CpuOps.scala:52-57)."""
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().oracle_f32_to_bf16_n(_ptr(x), _ptr(out), x.size)
    return out


def from_bf16(bits) -> np.ndarray:
    """BF16 bits -> F32 (tensor/DType.scala:99-102)."""
    bits = _c(bits, np.uint16)
    out = np.empty(bits.shape, np.float32)
    lib().oracle_bf16_to_f32_n(_ptr(bits), _ptr(out), bits.size)
    return out


def to_f16(x) -> np.ndarray:
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().oracle_f32_to_f16_n(_ptr(x), _ptr(out), x.size)
    return out


def from_f16(bits) -> np.ndarray:
    """F16 bits -> F32, Float.float16ToFloat (tensor/LittleEndian.scala:45-46)."""
    bits = _c(bits, np.uint16)
    out = np.empty(bits.shape, np.float32)
    lib().oracle_f16_to_f32_n(_ptr(bits), _ptr(out), bits.size)
    return out


def erf(x: float) -> float:
    return lib().oracle_erf(x)


def activate(kind: int, v: float) -> float:
    return lib().oracle_activate(kind, v)


# ---------------------------------------------------------------- F32 ops

def activation(kind: int, x, input_scale: float = 1.0) -> np.ndarray:
    x = _c(x, np.float32)
    out = np.empty_like(x)
    lib().oracle_activation(kind, input_scale, _ptr(x), _ptr(out), x.size)
    return out


def gated(kind: int, gate, up) -> np.ndarray:
    gate, up = _c(gate, np.float32), _c(up, np.float32)
    _need(gate.shape == up.shape, f"gated: gate {gate.shape}, up {up.shape}")
    out = np.empty_like(gate)
    lib().oracle_gated(kind, _ptr(gate), _ptr(up), _ptr(out), gate.size)
    return out


def rms_norm(x, weight, eps: float, offset: float = 0.0, y=None, weight_rows: int = 1):
    """Returns `out`, or `(x + y, out)` when `y` is given (addRmsNorm)."""
    x = np.array(x, dtype=np.float32, copy=True, order="C")
    weight = _c(weight, np.float32)
    cols = x.shape[-1]
    rows = x.size // cols if cols else 0
    yy = None if y is None else _c(y, np.float32)
    _need(weight.size == weight_rows * cols, f"rms_norm: weight of {weight.size} for {weight_rows} rows of {cols}")
    _need(weight_rows >= 1 and rows % weight_rows == 0, f"rms_norm: {rows} rows in groups of {weight_rows}")
    _need(yy is None or yy.shape == x.shape, "rms_norm: y is not x's shape")
    out = np.empty_like(x)
    lib().oracle_rms_norm(_ptr(x), _ptr(yy), _ptr(weight), _ptr(out), rows, cols, eps, offset, weight_rows)
    return out if y is None else (x, out)


def layer_norm(x, weight=None, bias=None, eps: float = 1e-5) -> np.ndarray:
    x = _c(x, np.float32)
    w = None if weight is None else _c(weight, np.float32)
    b = None if bias is None else _c(bias, np.float32)
    cols = x.shape[-1]
    _need(all(v is None or v.size == cols for v in (w, b)), f"layer_norm: weight or bias not of {cols}")
    out = np.empty_like(x)
    lib().oracle_layer_norm(_ptr(x), _ptr(w), _ptr(b), _ptr(out), x.size // cols, cols, eps)
    return out


def modulate(x, scale, shift) -> np.ndarray:
    x = _c(x, np.float32)
    scale, shift = _c(scale, np.float32), _c(shift, np.float32)
    cols = x.shape[-1]
    _need(scale.size == cols and shift.size == cols, f"modulate: scale or shift not of {cols}")
    out = np.empty_like(x)
    lib().oracle_modulate(_ptr(x), _ptr(scale), _ptr(shift), _ptr(out), x.size // cols, cols)
    return out


def _sections(sizes) -> np.ndarray:
    s = np.zeros(4, np.int32)
    s[: len(sizes)] = sizes
    return s


def rope(x, positions, theta: float, rotary: int, layout: int = NEOX, sections: int = SINGLE, sizes=()):
    x = _c(x, np.float32)
    positions = _c(positions, np.int32)
    tokens, heads, dim = x.shape
    _need(rotary % 2 == 0 and 0 < rotary <= dim, f"rope: {rotary} rotary dimensions of {dim}")
    axes = {SINGLE: 1, CONTIGUOUS: 3, INTERLEAVED_MROPE: 3, AXES: len(sizes)}[sections]
    _need(sections != AXES or 2 * sum(sizes) >= rotary, f"rope: axes {tuple(sizes)} cover fewer than {rotary} dims")
    _need(positions.size >= axes * tokens, f"rope: {positions.size} positions for {axes} x {tokens} tokens")
    out = np.empty_like(x)
    lib().oracle_rope(_ptr(x), _ptr(positions), _ptr(out), tokens, heads, dim, rotary, theta, layout,
                      sections, _ptr(_sections(sizes)))
    return out


def rope_inverse_frequency(pair: int, rotary: int, theta: float, sections: int = SINGLE, sizes=()) -> float:
    return lib().oracle_rope_inverse_frequency(pair, rotary, theta, sections, _ptr(_sections(sizes)))


def rope_table(x, cosines, sines, halves: bool = False) -> np.ndarray:
    x = _c(x, np.float32)
    cosines, sines = _c(cosines, np.float32), _c(sines, np.float32)
    tokens, heads, dim = x.shape
    pairs = cosines.shape[-1]
    per_head = 1 if cosines.ndim == 3 else 0
    want = (tokens, heads, pairs) if per_head else (tokens, pairs)
    _need(cosines.shape == want and sines.shape == want,
          f"rope_table: tables {cosines.shape} and {sines.shape} for x {x.shape} (want {want})")
    _need(2 * pairs <= dim, f"rope_table: {pairs} pairs in heads of {dim}")
    out = np.empty_like(x)
    lib().oracle_rope_table(_ptr(x), _ptr(cosines), _ptr(sines), _ptr(out), tokens, heads, dim, pairs, per_head,
                            1 if halves else 0)
    return out


def wan_pairs(head_dim: int = 128):
    p = np.zeros(3, np.int32)
    lib().oracle_wan_pairs(head_dim, _ptr(p))
    return tuple(int(v) for v in p)


def wan_angles(frames: int, rows: int, cols: int, head_dim: int = 128, theta: float = 10000.0):
    tokens = frames * rows * cols
    cos = np.empty((tokens, head_dim // 2), np.float32)
    sin = np.empty((tokens, head_dim // 2), np.float32)
    lib().oracle_wan_angles(frames, rows, cols, head_dim, theta, _ptr(cos), _ptr(sin))
    return cos, sin


def embedding_q8_0(table, vocab: int, cols: int, ids) -> np.ndarray:
    table = _c(table, np.uint8)
    ids = _c(ids, np.int32)
    _need(cols % 32 == 0 and table.size == vocab * cols // 32 * 34,
          f"embedding_q8_0: {table.size} bytes for {vocab} rows of {cols}")
    out = np.empty((ids.size, cols), np.float32)
    bad = lib().oracle_embedding_q8_0(_ptr(table), vocab, cols, _ptr(ids), ids.size, _ptr(out))
    if bad >= 0:
        raise ValueError(f"token id {int(ids[bad])} outside the table")
    return out


def embedding_f32(table, ids) -> np.ndarray:
    table = _c(table, np.float32)
    ids = _c(ids, np.int32)
    vocab, cols = table.shape
    out = np.empty((ids.size, cols), np.float32)
    bad = lib().oracle_embedding_f32(_ptr(table), vocab, cols, _ptr(ids), ids.size, _ptr(out))
    if bad >= 0:
        raise ValueError(f"token id {int(ids[bad])} outside the table")
    return out


def gated_add(x, y, gate, rows_per_sample=None) -> np.ndarray:
    """x + gate * y per row (ops/CpuElementwise.scala:40-49), returned (x is
    not changed). gate [cols], or [samples, cols] with rows_per_sample."""
    out = np.array(x, dtype=np.float32, copy=True, order="C")
    y, gate = _c(y, np.float32), _c(gate, np.float32)
    _need(y.shape == out.shape and out.ndim >= 1, f"gated_add: x {out.shape}, y {y.shape}")
    cols = out.shape[-1]
    rows = out.size // cols
    per = rows if rows_per_sample is None else rows_per_sample
    _need(per > 0 and gate.size == -(-rows // per) * cols, f"gated_add: gate {gate.shape} for {out.shape}")
    lib().oracle_gated_add(_ptr(out), _ptr(y), _ptr(gate), rows, cols, per)
    return out


def _chunks(x, table, *indices):
    _need(x.ndim == 2 and table.ndim == 2 and table.shape[0] == x.shape[0] and table.shape[1] % x.shape[1] == 0,
          f"table {table.shape} for {x.shape}")
    chunks = table.shape[1] // x.shape[1]
    _need(all(0 <= i < chunks for i in indices), f"chunks {indices} of {chunks}")
    return x.shape[0], x.shape[1], chunks


def modulate_chunks(x, table, shift: int, scale: int) -> np.ndarray:
    """ops/CpuElementwise.scala:51-67."""
    x, table = _c(x, np.float32), _c(table, np.float32)
    rows, channels, chunks = _chunks(x, table, shift, scale)
    out = np.empty_like(x)
    lib().oracle_modulate_chunks(_ptr(x), _ptr(table), _ptr(out), rows, channels, chunks, shift, scale)
    return out


def gated_add_chunk(x, y, table, gate: int) -> np.ndarray:
    """ops/CpuElementwise.scala:69-79, returned."""
    out = np.array(x, dtype=np.float32, copy=True, order="C")
    y, table = _c(y, np.float32), _c(table, np.float32)
    _need(y.shape == out.shape, f"gated_add_chunk: x {out.shape}, y {y.shape}")
    rows, channels, chunks = _chunks(out, table, gate)
    lib().oracle_gated_add_chunk(_ptr(out), _ptr(y), _ptr(table), rows, channels, chunks, gate)
    return out


def row_gated_add(x, y, gate) -> np.ndarray:
    """ops/CpuElementwise.scala:81-85, returned."""
    out = np.array(x, dtype=np.float32, copy=True, order="C")
    y, gate = _c(y, np.float32), _c(gate, np.float32)
    _need(y.shape == out.shape and out.ndim == 2 and gate.size == out.shape[0],
          f"row_gated_add: x {out.shape}, y {y.shape}, gate {gate.shape}")
    lib().oracle_row_gated_add(_ptr(out), _ptr(y), _ptr(gate), out.shape[0], out.shape[1])
    return out


def quantize_x(x):
    """The int8 side output of `x` (flat, whole blocks of 32): codes xq
    (int8 [n]), scales xd and code sums xs (float32 [n / 32]),
    kernels/quantize.h:10-25."""
    x = _c(x, np.float32).ravel()
    _need(x.size % 32 == 0, f"quantize_x: {x.size} values are not whole blocks of 32")
    blocks = x.size // 32
    xq = np.empty(x.size, np.int8)
    xd = np.empty(blocks, np.float32)
    xs = np.empty(blocks, np.float32)
    lib().oracle_quantize_x(_ptr(x), _ptr(xq), _ptr(xd), _ptr(xs), blocks)
    return xq, xd, xs


# ---------------------------------------------------------------- bf16 compositions
# The reference has no bf16 kernels: its bf16 path is convert -> F32 op ->
# convert (ops/HipBase.scala:268-274, kernels/elementwise.hip:68-86).

def rms_norm_bf16(x_bits, weight, eps, offset=0.0, y_bits=None, weight_rows=1):
    x = from_bf16(x_bits)
    if y_bits is None:
        return to_bf16(rms_norm(x, weight, eps, offset, weight_rows=weight_rows))
    summed, out = rms_norm(x, weight, eps, offset, y=from_bf16(y_bits), weight_rows=weight_rows)
    return to_bf16(summed), to_bf16(out)


def activation_bf16(kind, x_bits, input_scale=1.0):
    return to_bf16(activation(kind, from_bf16(x_bits), input_scale))


def gated_bf16(kind, gate_bits, up_bits):
    return to_bf16(gated(kind, from_bf16(gate_bits), from_bf16(up_bits)))


def layer_norm_modulate(x, scale, shift, rows_per_sample: int, eps: float):
    """AdaLN as Wan runs it (models/Wan.scala:431-432): layerNorm without
    affine, F32 written, then modulate with each sample's scale and shift rows
    (`scale`, `shift` [samples, cols]) over that sample's rows."""
    x = _c(x, np.float32)
    scale, shift = np.atleast_2d(_c(scale, np.float32)), np.atleast_2d(_c(shift, np.float32))
    normed = layer_norm(x, None, None, eps)
    out = np.empty_like(normed)
    rows = normed.shape[0]
    for s in range(math.ceil(rows / rows_per_sample)):
        lo, hi = s * rows_per_sample, min(rows, (s + 1) * rows_per_sample)
        out[lo:hi] = modulate(normed[lo:hi], scale[s], shift[s])
    return out


def layer_norm_modulate_bf16(x_bits, scale, shift, rows_per_sample, eps):
    return to_bf16(layer_norm_modulate(from_bf16(x_bits), scale, shift, rows_per_sample, eps))


def qk_norm_rope(q, k, q_weight, k_weight, positions, eps, offset, theta, rotary, layout=NEOX,
                 sections=SINGLE, sizes=()):
    """The reference's composition for attention inputs
    (ops/AttentionOps.scala:87-107): per-head rmsNorm in place (F32 written),
    then rope of queries and keys. q [t, heads, D], k [t, kvHeads, D]."""
    q = _c(q, np.float32)
    k = _c(k, np.float32)
    t, heads, d = q.shape
    kv = k.shape[1]
    qn = rms_norm(q.reshape(t * heads, d), q_weight, eps, offset).reshape(t, heads, d)
    kn = rms_norm(k.reshape(t * kv, d), k_weight, eps, offset).reshape(t, kv, d)
    return (rope(qn, positions, theta, rotary, layout, sections, sizes),
            rope(kn, positions, theta, rotary, layout, sections, sizes))


def qk_norm_rope_bf16(q_bits, k_bits, q_weight, k_weight, positions, eps, offset, theta, rotary, layout=NEOX,
                      sections=SINGLE, sizes=()):
    rq, rk = qk_norm_rope(from_bf16(q_bits), from_bf16(k_bits), q_weight, k_weight, positions, eps, offset, theta,
                          rotary, layout, sections, sizes)
    return to_bf16(rq), to_bf16(rk)


def rope_3d(x, frames, rows, cols, theta=10000.0, token_offset=0):
    """Wan's 3-D RoPE (models/Wan.scala:324-361, :442-443): the angle tables
    of the frames x rows x cols grid, then ropeTable with adjacent pairs.
    x [tokens, heads, D]; token i sits at grid index token_offset + i."""
    x = _c(x, np.float32)
    tokens, heads, d = x.shape
    cos, sin = wan_angles(frames, rows, cols, d, theta)
    grid = frames * rows * cols
    index = (token_offset + np.arange(tokens)) % grid
    return rope_table(x, cos[index], sin[index], halves=False)


def rope_3d_bf16(x_bits, frames, rows, cols, theta=10000.0, token_offset=0):
    return to_bf16(rope_3d(from_bf16(x_bits), frames, rows, cols, theta, token_offset))


def embedding_q8_0_bf16(table, vocab, cols, ids):
    """The F32 gather converted to BF16: bit-exact by construction, since the
    product of an fp16 scale and an int8 code is exact in F32."""
    return to_bf16(embedding_q8_0(table, vocab, cols, ids))


# ---------------------------------------------------------------- storage types

# GGUF type ids of the storage types with decoders (tensor/DType.scala and the
# quant objects' ggmlId), and where each block keeps its f16 scales (for
# the test tables; ROCmFP4 keeps E4M3 scale bytes at 16 and 17 instead).
FORMATS = {"F32": 0, "F16": 1, "Q4_0": 2, "Q4_1": 3, "Q5_0": 6, "Q5_1": 7, "Q8_0": 8, "Q4_K": 12, "Q5_K": 13,
           "Q6_K": 14, "IQ4_NL": 20, "IQ4_XS": 23, "BF16": 30, "Q4_0_ROCMFP4": 100, "Q4_0_ROCMFP4_FAST": 101}
_F16_FIELDS = {"Q4_0": (0,), "Q4_1": (0, 2), "Q5_0": (0,), "Q5_1": (0, 2), "Q8_0": (0,), "Q4_K": (0, 2),
               "Q5_K": (0, 2), "Q6_K": (208,), "IQ4_NL": (0,), "IQ4_XS": (0,)}


def format_block(name: str):
    """(values, bytes) of a block of storage type `name`."""
    values, size = ctypes.c_int(), ctypes.c_int()
    _need(lib().oracle_format_block(FORMATS[name], ctypes.byref(values), ctypes.byref(size)) == 0, name)
    return values.value, size.value


def row_bytes(name: str, cols: int) -> int:
    values, size = format_block(name)
    _need(cols % values == 0, f"{cols} values are not whole {name} blocks of {values}")
    return cols // values * size


def rocmfp4_half_scale(byte: int) -> float:
    return lib().oracle_rocmfp4_half_scale(byte)


def decode_row(name: str, row, cols: int) -> np.ndarray:
    """One row's bytes decoded to F32, as DType.decode (tensor/DType.scala)."""
    row = _c(row, np.uint8)
    _need(row.size >= row_bytes(name, cols), f"{row.size} bytes for a {name} row of {cols}")
    out = np.empty(cols, np.float32)
    lib().oracle_decode_row(FORMATS[name], _ptr(row), cols, _ptr(out))
    return out


def embedding(name: str, table, vocab: int, cols: int, ids) -> np.ndarray:
    """CpuLinear.embedding (ops/CpuLinear.scala:12-41): rows `ids` of a table
    of storage type `name` (its bytes, [vocab, row bytes]), as F32."""
    table = _c(table, np.uint8)
    ids = _c(ids, np.int32)
    _need(table.size >= vocab * row_bytes(name, cols), "table bytes")
    out = np.empty((ids.size, cols), np.float32)
    bad = lib().oracle_embedding(FORMATS[name], _ptr(table), vocab, cols, _ptr(ids), ids.size, _ptr(out))
    _need(bad == -1, f"token id {ids[bad] if bad >= 0 else '?'} outside the table")
    return out


def embedding_bf16(name: str, table, vocab: int, cols: int, ids) -> np.ndarray:
    return to_bf16(embedding(name, table, vocab, cols, ids))


def quant_table(name: str, rows: int, cols: int, rng: np.random.Generator) -> np.ndarray:
    """Random bytes of a [rows, cols] table of storage type `name` whose
    values are all finite: f16 scales uniform in +-[1e-3, 2e-2], ROCmFP4 scale
    bytes finite E4M3 codes, dense values random normals."""
    if name in ("F32", "F16", "BF16"):
        x = rng.standard_normal((rows, cols)).astype(np.float32)
        raw = {"F32": x, "F16": x.astype(np.float16), "BF16": to_bf16(x)}[name]
        return np.ascontiguousarray(raw).view(np.uint8).reshape(rows, -1)
    values, size = format_block(name)
    blocks = cols // values
    t = rng.integers(0, 256, (rows, blocks, size), dtype=np.uint8)
    for at in _F16_FIELDS.get(name, ()):
        d = (rng.uniform(1e-3, 2e-2, (rows, blocks)) * rng.choice([-1, 1], (rows, blocks))).astype(np.float16)
        t[:, :, at:at + 2] = d.view(np.uint8).reshape(rows, blocks, 2)
    if name.startswith("Q4_0_ROCMFP4"):
        t[:, :, 16:] = rng.integers(0, 0x7f, (rows, blocks, size - 16), dtype=np.uint8)
    return t.reshape(rows, blocks * size)


# ---------------------------------------------------------------- attention inputs

def split_halves(x):
    """CpuLayout.splitHalves (ops/CpuLayout.scala:137-143): rows [.., 2 d]
    into their first and second halves."""
    x = _c(x, np.float32)
    d = x.shape[-1] // 2
    return np.ascontiguousarray(x[..., :d]), np.ascontiguousarray(x[..., d:])


def cache_place(page_table, page_size: int, position: int, kv_heads: int, dim: int, head: int, d: int):
    """CpuAttention.cacheIndices (ops/CpuAttention.scala:163-179): the flat
    indices of (position, head, d) in the keys and in the values."""
    page = int(page_table[position // page_size])
    offset = position % page_size
    return (((page * page_size + offset) * kv_heads + head) * dim + d,
            ((page * kv_heads + head) * dim + d) * page_size + offset)


def cache_write(k, v, keys, values, page_table, page_size: int, start: int):
    """CpuAttention.cacheWrite (ops/CpuAttention.scala:181-210): keys and
    values [tokens, kv_heads, D] F32 into copies of the F16 cache (bits,
    keys [pages, page_size, kv_heads, D], values [pages, kv_heads, D,
    page_size]) at positions start .. start + tokens - 1; returns the copies.
    Every element's indices are cache_place's formula, taken over all
    (t, head, d) at once."""
    k, v = _c(k, np.float32), _c(v, np.float32)
    tokens, kv_heads, dim = k.shape
    keys, values = np.array(keys, np.uint16).reshape(-1), np.array(values, np.uint16).reshape(-1)
    position = start + np.arange(tokens, dtype=np.int64)[:, None, None]
    page = np.asarray(page_table, np.int64)[position // page_size]
    offset = position % page_size
    head = np.arange(kv_heads, dtype=np.int64)[None, :, None]
    d = np.arange(dim, dtype=np.int64)[None, None, :]
    keys[((page * page_size + offset) * kv_heads + head) * dim + d] = to_f16(k)
    values[((page * kv_heads + head) * dim + d) * page_size + offset] = to_f16(v)
    return keys, values


def attention_inputs(query_and_gate, k, v, q_norm, k_norm, eps, offset, positions, theta, rotary, keys, values,
                     page_table, page_size, start, layout=NEOX, sections=SINGLE, sizes=(), gated=True):
    """The reference's attentionInputs composition (ops/AttentionOps.scala:
    73-107): splitHalves of the gated query projection [t, heads, 2 D] (or,
    with gated False, plain queries [t, heads, D]), rmsNorm of each query and
    key head in place (F32 written), rope of both, cacheWrite of the rotated
    keys with the values. Returns (rotated queries, gate or None, keys,
    values), the cache as F16 bits."""
    k = _c(k, np.float32)
    if gated:
        queries, gate = split_halves(query_and_gate)
    else:
        queries, gate = _c(query_and_gate, np.float32), None
    rq, rk = qk_norm_rope(queries, k, q_norm, k_norm, positions, eps, offset, theta, rotary, layout, sections, sizes)
    keys, values = cache_write(rk, v, keys, values, page_table, page_size, start)
    return rq, gate, keys, values


def attention_inputs_bf16(qg_bits, k_bits, v_bits, q_norm, k_norm, eps, offset, positions, theta, rotary, keys,
                          values, page_table, page_size, start, layout=NEOX, sections=SINGLE, sizes=(), gated=True):
    """The bf16 composition: inputs converted to F32, the F32 op, queries and
    gate converted to BF16; the cache holds the F32 results rounded to F16."""
    rq, gate, keys, values = attention_inputs(from_bf16(qg_bits), from_bf16(k_bits), from_bf16(v_bits), q_norm,
                                              k_norm, eps, offset, positions, theta, rotary, keys, values,
                                              page_table, page_size, start, layout, sections, sizes, gated)
    return to_bf16(rq), None if gate is None else to_bf16(gate), keys, values


# ---------------------------------------------------------------- inputs

def java_gaussian(seed: int, count: int) -> np.ndarray:
    """TestData.gaussian (runner/test/src/drift/runner/TestData.scala:10-13):
    `scala.util.Random(seed).nextGaussian().toFloat`, i.e. java.util.Random's
    48-bit LCG and its polar Box-Muller. StrictMath.log is replaced by the C
    library's log; both are within an ulp in double, far below a float's."""
    mask = (1 << 48) - 1
    state = (seed ^ 0x5DEECE66D) & mask

    def nxt(bits):
        nonlocal state
        state = (state * 0x5DEECE66D + 0xB) & mask
        return state >> (48 - bits)

    def next_double():
        return ((nxt(26) << 27) + nxt(27)) * (1.0 / (1 << 53))

    out = np.empty(count, np.float32)
    spare = None
    for i in range(count):
        if spare is not None:
            out[i] = np.float32(spare)
            spare = None
            continue
        while True:
            v1 = 2 * next_double() - 1
            v2 = 2 * next_double() - 1
            s = v1 * v1 + v2 * v2
            if 0 < s < 1:
                break
        multiplier = math.sqrt(-2 * math.log(s) / s)
        spare = v2 * multiplier
        out[i] = np.float32(v1 * multiplier)
    return out


def q8_0_table(rows: int, cols: int, rng: np.random.Generator, scale_lo=1e-3, scale_hi=2e-2) -> np.ndarray:
    """A Q8_0 table: codes uniform in [-127, 127], fp16 scales uniform in
    [scale_lo, scale_hi], as bytes [rows, cols/32*34]."""
    blocks = rows * (cols // 32)
    raw = np.empty((blocks, 34), np.uint8)
    scales = rng.uniform(scale_lo, scale_hi, blocks).astype(np.float16)
    raw[:, 0:2] = scales.view(np.uint8).reshape(blocks, 2)
    raw[:, 2:] = rng.integers(-127, 128, (blocks, 32)).astype(np.int8).view(np.uint8)
    return raw.reshape(rows, cols // 32 * 34)


# ---------------------------------------------------------------- ConvRot rotated linears

CONVROT_GROUP = 256  # tensor/ConvRot.scala:13


def f8e4m3(code: int) -> float:
    """DType.F8E4M3 (tensor/DType.scala:105-115)."""
    return lib().oracle_f8e4m3(int(code))


def convrot_rotate(values, group: int = CONVROT_GROUP) -> np.ndarray:
    """ConvRot.rotate (tensor/ConvRot.scala:20-50) of a copy of `values`,
    every `group` of them."""
    out = _c(values, np.float32).copy()
    _need(out.size % group == 0, f"{out.size} values are not whole groups of {group}")
    lib().oracle_convrot_rotate(_ptr(out), out.size, group)
    return out.reshape(np.shape(values))


class Rotated:
    """A rotated linear [rows, cols] as a file holds it (ops/LinearOps.scala:
    21-33, ops/ConvRotParts.scala): `codes` uint8 [rows, cols] (int8
    codes) or [rows, cols / 2] (4-bit, with `codebook` F32 [16], `relative`
    fp8 bytes [rows, cols / group_size] and `group_size`), and `scales` F32
    [rows] (or [1] for int8 codes)."""

    def __init__(self, codes, scales, cols, codebook=None, relative=None, group_size=0):
        self.codes = _c(codes, np.uint8)
        self.scales = _c(scales, np.float32)
        self.cols, self.group_size = int(cols), int(group_size)
        self.codebook = None if codebook is None else _c(codebook, np.float32)
        self.relative = None if relative is None else _c(relative, np.uint8)
        self.rows = self.codes.shape[0]
        per_row = self.cols // 2 if self.codebook is not None else self.cols
        _need(self.codes.size == self.rows * per_row, "codes")
        if self.codebook is not None:
            _need(self.codebook.size == 16 and self.group_size > 0 and self.cols % self.group_size == 0, "levels")
            _need(self.relative.size == self.rows * (self.cols // self.group_size), "relative scales")

    def _args(self):
        return (_ptr(self.codes), _ptr(self.scales), self.scales.size, _ptr(self.codebook), _ptr(self.relative),
                self.group_size, self.cols)

    def levels(self, first: int = 0, count: int | None = None) -> np.ndarray:
        """The rows' values before their rotation (int8 level times scale)."""
        count = self.rows - first if count is None else count
        out = np.empty((count, self.cols), np.float32)
        lib().oracle_convrot_levels(*self._args(), first, count, _ptr(out))
        return out

    def rows_of(self, first: int = 0, count: int | None = None) -> np.ndarray:
        """CpuBase.rotatedRows (ops/CpuBase.scala:40-81): the F32 weight rows."""
        _need(self.cols % CONVROT_GROUP == 0, f"rotated: rows of {self.cols} columns")
        count = self.rows - first if count is None else count
        out = np.empty((count, self.cols), np.float32)
        lib().oracle_convrot_rows(*self._args(), first, count, _ptr(out))
        return out

    def embedding(self, ids) -> np.ndarray:
        """CpuLinear.embedding of a rotated table (ops/CpuLinear.scala:12-41):
        rows `ids` as the BF16 they hold, widened to F32."""
        ids = _c(ids, np.int32)
        out = np.empty((ids.size, self.cols), np.float32)
        bad = lib().oracle_convrot_embedding(*self._args()[:6], self.rows, self.cols, _ptr(ids), ids.size, _ptr(out))
        _need(bad == -1, f"token id {ids[bad] if bad >= 0 else '?'} outside the table")
        return out

    def dequantize_bf16(self) -> np.ndarray:
        """convert to BF16 (ops/HipMemory.scala:127-130): the rows rounded."""
        return to_bf16(self.rows_of())


def random_rotated(rows: int, cols: int, rng: np.random.Generator, four_bit: bool = False, group_size: int = 32,
                   one_scale: bool = False) -> Rotated:
    """A random rotated weight: int8 codes in [-128, 127] with scales uniform
    in [1e-4, 1e-2]; or 4-bit codes with a sorted codebook uniform in [-1, 1],
    positive relative scales 0x58..0x76 (16 to 240, so the int8 clamp is
    exercised) and row scales in [1e-4, 1e-3]."""
    if not four_bit:
        codes = rng.integers(0, 256, (rows, cols), dtype=np.uint8)
        scales = rng.uniform(1e-4, 1e-2, 1 if one_scale else rows).astype(np.float32)
        return Rotated(codes, scales, cols)
    codes = rng.integers(0, 256, (rows, cols // 2), dtype=np.uint8)
    codebook = np.sort(rng.uniform(-1, 1, 16)).astype(np.float32)
    relative = rng.integers(0x58, 0x77, (rows, cols // group_size), dtype=np.uint8)
    scales = rng.uniform(1e-4, 1e-3, rows).astype(np.float32)
    return Rotated(codes, scales, cols, codebook, relative, group_size)
