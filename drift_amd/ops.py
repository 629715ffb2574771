"""`HipOps`: the drift runner's operation interface for the fused layer
kernels' path, over libdrift_kernels.

It mirrors the runner's Scala `Ops` trait (runner/src/drift/runner/ops/Ops.scala:15-34)
for the methods on this path: same names, same argument meaning, and the
same shape and dtype rules, checked before any launch and refused with a
`ValueError` carrying the reference's message (the reference throws
IllegalArgumentException from `require`, ops/Ops.scala:36-93). Tensors are
torch tensors in device memory; `out` is written, never read, and may be an
input of the elementwise and row-wise operations.

Beyond the reference's F32 activations, the kernels take BF16 tensors
(torch.bfloat16) with F32 norm, modulation and rope vectors: the reference's
bf16 path is convert -> F32 op -> convert, which these produce in one pass.
Everything launches asynchronously on the current torch stream (or the
stream given to the constructor); nothing synchronizes.
"""

from __future__ import annotations

import ctypes
import enum
from dataclasses import dataclass, replace
from typing import Optional, Sequence, Tuple

import torch

from . import _lib

F32, BF16, F16, I32 = torch.float32, torch.bfloat16, torch.float16, torch.int32
_FLOAT_TYPES = (F32, BF16)


class Activation(enum.IntEnum):
    """ops/Activation.scala:6-20; the value is the kernels' `kind`."""
    Silu = 0
    GeluTanh = 1
    GeluErf = 2
    Sigmoid = 3
    Situ = 4


class RopeLayout(enum.IntEnum):
    """ops/Rope.scala:7-12."""
    Neox = 0
    Interleaved = 1


@dataclass(frozen=True)
class RopeSections:
    """ops/Rope.scala:14-37: which position each pair turns by."""
    code: int
    sizes: tuple = ()

    @staticmethod
    def Single() -> "RopeSections":
        return RopeSections(0)

    @staticmethod
    def Contiguous(temporal: int, height: int, width: int) -> "RopeSections":
        return RopeSections(1, (temporal, height, width))

    @staticmethod
    def Interleaved(temporal: int, height: int, width: int) -> "RopeSections":
        return RopeSections(2, (temporal, height, width))

    @staticmethod
    def Axes(pairs: Sequence[int]) -> "RopeSections":
        return RopeSections(3, tuple(pairs))

    @property
    def positionsPerToken(self) -> int:
        return 1 if self.code == 0 else (len(self.sizes) if self.code == 3 else 3)

    def launch_sizes(self) -> tuple:
        """`rope_f32`'s four section sizes (ops/HipAttention.scala:73-79)."""
        return tuple(self.sizes) + (0,) * (4 - len(self.sizes))


@dataclass(frozen=True)
class Rope:
    """ops/Rope.scala:39-46."""
    theta: float
    rotaryDimensions: int
    layout: RopeLayout = RopeLayout.Neox
    sections: RopeSections = RopeSections(0)


@dataclass
class RowNorm:
    """ops/RowNorm.scala:17-23: an RMS norm taken of a result as it is written."""
    weight: torch.Tensor
    epsilon: float
    weightOffset: float
    out: torch.Tensor


@dataclass
class QueryKeyNorms:
    """ops/RowNorm.scala:5-15: query and key RMS norms, then `rope`."""
    queryNorm: torch.Tensor
    keyNorm: torch.Tensor
    epsilon: float
    weightOffset: float
    rope: Rope


@dataclass
class KvCache:
    """ops/KvCache.scala:5-22: a paged cache of pages of `pageSize` tokens;
    keys F16 [pages, pageSize, kvHeads, headDimension], values F16 [pages,
    kvHeads, headDimension, pageSize] (transposed within a page)."""
    keys: torch.Tensor
    values: torch.Tensor
    pageSize: int

    def __post_init__(self):
        _require(self.pageSize % 16 == 0, f"pages of {self.pageSize} tokens: not a multiple of 16")
        _require(self.keys.dtype == F16 and self.values.dtype == F16, "the cache is F16")
        _require(self.keys.dim() == 4 and self.values.dim() == 4, "the cache's keys and values are 4-dimensional")
        self.pages, _, self.kvHeads, self.headDimension = (int(d) for d in self.keys.shape)
        _require(tuple(self.values.shape) == (self.pages, self.kvHeads, self.headDimension, self.pageSize),
                 f"cache values {_shape(self.values)} for keys {_shape(self.keys)}")

    @staticmethod
    def allocate(pages: int, pageSize: int, kvHeads: int, headDimension: int, device="cuda") -> "KvCache":
        """HipOps.allocateCache: the cache's two tensors, uninitialised."""
        return KvCache(torch.empty((pages, pageSize, kvHeads, headDimension), dtype=F16, device=device),
                       torch.empty((pages, kvHeads, headDimension, pageSize), dtype=F16, device=device), pageSize)


@dataclass(frozen=True)
class StorageType:
    """A table's storage type (tensor/DType.scala:14-66): `values` per block
    of `bytes`, its GGUF type id (the kernels' `format`), and the alignment
    its blocks' fields need."""
    name: str
    ggmlId: int
    values: int
    bytes: int
    align: int

    def rowBytes(self, cols: int) -> int:
        _require(cols % self.values == 0, f"{cols} elements are not whole {self.name} blocks of {self.values}")
        return cols // self.values * self.bytes


# tensor/DType.scala, GgmlQuants.scala:12-118, KQuants.scala:100-134,
# IQuants.scala:40-80, RocmFp4.scala:75-84: the types with gather kernels
# (kernels/matvec.hip:942-954), and F32, F16, BF16.
STORAGE_TYPES = {t.name: t for t in (
    StorageType("F32", 0, 1, 4, 16), StorageType("F16", 1, 1, 2, 16), StorageType("BF16", 30, 1, 2, 16),
    StorageType("Q4_0", 2, 32, 18, 2), StorageType("Q4_1", 3, 32, 20, 4), StorageType("Q5_0", 6, 32, 22, 2),
    StorageType("Q5_1", 7, 32, 24, 4), StorageType("Q8_0", 8, 32, 34, 2), StorageType("Q4_K", 12, 256, 144, 8),
    StorageType("Q5_K", 13, 256, 176, 8), StorageType("Q6_K", 14, 256, 210, 2),
    StorageType("IQ4_NL", 20, 32, 18, 2), StorageType("IQ4_XS", 23, 256, 136, 8),
    StorageType("Q4_0_ROCMFP4", 100, 32, 18, 2), StorageType("Q4_0_ROCMFP4_FAST", 101, 32, 17, 1))}


@dataclass
class StoredTable:
    """A table ([vocabulary, cols] values) as its stored bytes: a uint8
    tensor [vocabulary, row bytes] in storage type `dtype` (a GGUF tensor's
    data as it lies in the file)."""
    data: torch.Tensor
    dtype: StorageType
    cols: int

    @property
    def shape(self) -> tuple:
        return (self.data.shape[0], self.cols)


def Q8_0Table(data: torch.Tensor, cols: int) -> StoredTable:
    """A Q8_0 table: per 32 values an fp16 scale then 32 int8 codes
    (tensor/GgmlQuants.scala:104-118), [vocabulary, cols / 32 * 34] bytes."""
    return StoredTable(data, STORAGE_TYPES["Q8_0"], cols)


@dataclass(frozen=True)
class ConvRotLevels:
    """What makes an int8 level of a 4-bit code (ops/ConvRotParts.scala:5-13):
    the 16-level `codebook` (F32 [16]) and each row's `relative` scales (fp8
    E4M3 [rows, cols / groupSize], as uint8 bytes or float8_e4m3fn), one a
    `groupSize` columns."""
    codebook: torch.Tensor
    relative: torch.Tensor
    groupSize: int


@dataclass(frozen=True)
class ConvRotParts:
    """What a rotated linear's codes are decoded with
    (ops/ConvRotParts.scala:15-17): `scales` F32, one a row (or one for all,
    without `levels`), and a 4-bit linear's `levels`."""
    scales: torch.Tensor
    levels: Optional[ConvRotLevels] = None


CONVROT_GROUP = 256  # tensor/ConvRot.scala:13


@dataclass(frozen=True)
class RotatedTable:
    """A rotated linear [rows, cols] left where the file holds it
    (ops/LinearOps.scala:21-33 `rotated`): ComfyUI's int8_tensorwise codes
    (I8 [rows, cols], dtype CONVROT_I8) or asym_w4a8_int8's 4-bit codes (two
    a byte, [rows, cols / 2], dtype CONVROT_W4A8), seen as the weight they
    make with `parts` (tensor/ConvRot.scala:52-71)."""
    codes: torch.Tensor
    parts: ConvRotParts
    cols: int

    @property
    def dtype(self) -> str:
        return "CONVROT_I8" if self.parts.levels is None else "CONVROT_W4A8"

    @property
    def shape(self) -> tuple:
        return (self.codes.shape[0], self.cols)


@dataclass(frozen=True)
class QuantizedValues:
    """`values` F32 values at device address `address` that the launch
    numbered `written` also wrote quantized into `buffer`: codes (int8 per
    value), then scales, then code sums (F32 per block of 32)
    (ops/HipBase.scala:129-147). Blocks do not depend on rows, so any whole
    blocks within serve."""

    address: int
    values: int
    buffer: torch.Tensor
    written: int

    def codes(self, first: int = 0, count: Optional[int] = None) -> torch.Tensor:
        count = self.values - first if count is None else count
        return self.buffer.narrow(0, first, count)

    def scales(self, first: int = 0, count: Optional[int] = None) -> torch.Tensor:
        blocks = self.values // 32
        count = blocks - first if count is None else count
        return self.buffer.narrow(0, self.values + 4 * first, 4 * count).view(torch.float32)

    def sums(self, first: int = 0, count: Optional[int] = None) -> torch.Tensor:
        blocks = self.values // 32
        count = blocks - first if count is None else count
        return self.buffer.narrow(0, self.values + 4 * blocks + 4 * first, 4 * count).view(torch.float32)


# ------------------------------------------------------------------ checks
# object Ops (ops/Ops.scala:36-93) and the groups' checks.

def _require(condition: bool, message: str) -> None:
    if not condition:
        raise ValueError(message)


def _name(dtype) -> str:
    return {F32: "F32", BF16: "BF16", F16: "F16", I32: "I32", torch.int8: "I8", torch.uint8: "U8",
            torch.float8_e4m3fn: "F8_E4M3"}.get(dtype, str(dtype))


def _dims(shape) -> str:
    """A shape as the reference's Shape.toString writes it
    (tensor/Tensor.scala:12)."""
    return "[" + "×".join(str(d) for d in shape) + "]"


def _shape(t) -> str:
    return _dims(t.shape)


def requireF32(operation: str, *tensors) -> None:
    for t in tensors:
        _require(t.dtype == F32, f"{operation} takes F32, not {_name(t.dtype)}")


def requireSameShape(operation: str, *tensors) -> None:
    _require(len({tuple(t.shape) for t in tensors}) == 1,
             f"{operation} needs equal shapes, got {', '.join(_shape(t) for t in tensors)}")


def checkElementwise(operation: str, *tensors) -> None:
    """Same-shape operands of one float type (F32, or BF16 here)."""
    _require(tensors[0].dtype in _FLOAT_TYPES, f"{operation} takes F32 or BF16, not {_name(tensors[0].dtype)}")
    for t in tensors[1:]:
        _require(t.dtype == tensors[0].dtype,
                 f"{operation} takes one type, not {_name(tensors[0].dtype)} and {_name(t.dtype)}")
    requireSameShape(operation, *tensors)


def checkRowWise(operation: str, x, out, *rowVectors) -> int:
    """Returns the row count (ops/Ops.scala:76-92)."""
    checkElementwise(operation, x, out)
    _require(x.dim() >= 1, f"{operation} needs at least one dimension")
    for vector in rowVectors:
        requireF32(operation, vector)
        _require(tuple(vector.shape) == (x.shape[-1],), f"{operation}: {_shape(vector)} for rows of {x.shape[-1]}")
    return x.numel() // x.shape[-1] if x.shape[-1] else 0


def checkChunks(operation: str, x, table, out, *indices) -> tuple:
    """Returns (rows, C, chunks): x, out [rows, C], table F32
    [rows, chunks * C], every index a chunk (ops/ElementwiseOps.scala:55-76)."""
    checkElementwise(operation, x, out)
    requireF32(operation, table)
    _require(x.dim() == 2, f"{operation} takes [rows, C], not {_shape(x)}")
    rows, channels = x.shape
    width = table.shape[-1] if table.dim() else 0
    _require(table.dim() == 2 and table.shape[0] == rows and channels > 0 and width % channels == 0
             and all(0 <= i < width // channels for i in indices),
             f"{operation}: table {_shape(table)} for {_shape(x)}, chunks ArraySeq({', '.join(map(str, indices))})")
    return rows, channels, width // channels


def checkRowGatedAdd(x, y, gate) -> tuple:
    """Returns (rows, cols) (ops/ElementwiseOps.scala:79-92)."""
    checkElementwise("rowGatedAdd", x, y)
    requireF32("rowGatedAdd", gate)
    _require(x.dim() == 2, f"rowGatedAdd takes [rows, cols], not {_shape(x)}")
    rows, cols = x.shape
    _require(gate.numel() == rows, f"rowGatedAdd: gate {_shape(gate)} for {_shape(x)}")
    return rows, cols


def checkRope(x, positions, rope: Rope, out) -> tuple:
    """ops/AttentionOps.scala:185-223; returns (tokens, heads, headDimension)."""
    checkElementwise("rope", x, out)
    _require(x.dim() == 3, f"rope takes [tokens, heads, headDimension], got {_shape(x)}")
    tokens, heads, dimension = x.shape
    _require(positions.dtype == I32, f"rope positions are I32, not {_name(positions.dtype)}")
    if rope.sections.code == 3:
        pairs = rope.sections.sizes
        _require(len(pairs) <= 4 and all(p > 0 for p in pairs) and sum(pairs) * 2 == rope.rotaryDimensions,
                 f"rope: axes of {list(pairs)} pairs for {rope.rotaryDimensions} rotary values")
    count = rope.sections.positionsPerToken
    expected = (tokens,) if count == 1 else (count, tokens)
    _require(tuple(positions.shape) == expected,
             f"rope positions {_shape(positions)}, expected {_dims(expected)}")
    _require(rope.rotaryDimensions % 2 == 0 and rope.rotaryDimensions <= dimension,
             f"rope: {rope.rotaryDimensions} rotary dimensions in heads of {dimension}")
    return tokens, heads, dimension


def checkRopeTable(x, cosines, sines, out) -> tuple:
    """ops/AttentionOps.scala:129-151; returns (tokens, heads, D, pairs, perHead)."""
    checkElementwise("ropeTable", x, out)
    requireF32("ropeTable", cosines, sines)
    _require(x.dim() == 3, f"ropeTable takes [tokens, heads, D], not {_shape(x)}")
    tokens, heads, d = x.shape
    pairs = cosines.shape[-1]
    per_head = cosines.dim() == 3
    _require((tuple(cosines.shape) in ((tokens, pairs), (tokens, heads, pairs)))
             and sines.shape == cosines.shape and 2 * pairs <= d,
             f"ropeTable: tables {_shape(cosines)}, {_shape(sines)} for {_shape(x)}")
    return tokens, heads, d, pairs, per_head


def checkEmbedding(table, ids, out) -> None:
    """ops/LinearOps.scala:92-106."""
    shape = table.shape
    _require(len(shape) == 2, f"an embedding table is [vocabulary, D], not {list(shape)}")
    _require(ids.dtype == I32 and ids.dim() == 1,
             f"embedding ids are I32 [tokens], not {_name(ids.dtype)} {_shape(ids)}")
    _require(out.dtype in _FLOAT_TYPES, f"embedding takes F32 or BF16, not {_name(out.dtype)}")
    _require(tuple(out.shape) == (ids.shape[0], shape[-1]),
             f"embedding: out {_shape(out)} for {ids.shape[0]} rows of {shape[-1]}")


def checkRotated(codes, parts: ConvRotParts) -> RotatedTable:
    """Ops.checkRotated (ops/LinearOps.scala:121-157): the weight `codes`
    make with `parts`."""
    _require(codes.dtype == torch.int8 and codes.dim() == 2,
             f"rotated: {_name(codes.dtype)} codes {_shape(codes)}")
    n = codes.shape[0]
    k = codes.shape[1] * (1 if parts.levels is None else 2)
    _require(k % CONVROT_GROUP == 0, f"rotated: rows of {k} columns")
    scaleCount = parts.scales.numel()
    _require(parts.scales.dtype == F32 and (scaleCount == n or scaleCount == 1 and parts.levels is None),
             f"rotated: {scaleCount} {_name(parts.scales.dtype)} scales for {n} rows")
    l = parts.levels
    if l is not None:
        _require(l.groupSize > 0 and l.groupSize % 16 == 0 and k % l.groupSize == 0,
                 f"rotated: {k} columns in groups of {l.groupSize}")
        _require(l.codebook.dtype == F32 and l.codebook.numel() == 16,
                 f"rotated: a codebook {_name(l.codebook.dtype)} {_shape(l.codebook)}")
        _require(l.relative.dtype in (torch.uint8, torch.float8_e4m3fn) and
                 tuple(l.relative.shape) == (n, k // l.groupSize),
                 f"rotated: relative scales {_name(l.relative.dtype)} {_shape(l.relative)}")
    return RotatedTable(codes, parts, k)


def checkPageTable(pageTable, cache: KvCache, positions: int) -> None:
    """ops/AttentionOps.scala:243-256."""
    _require(pageTable.dtype == I32 and pageTable.dim() == 1,
             f"a page table is I32 [pages], not {_name(pageTable.dtype)} {_shape(pageTable)}")
    _require(pageTable.numel() * cache.pageSize >= positions,
             f"a page table of {pageTable.numel()} pages for {positions} positions")


def checkCacheWrite(k, v, cache: KvCache, pageTable, start: int) -> int:
    """ops/AttentionOps.scala:225-241; returns the token count."""
    checkElementwise("cacheWrite", k, v)
    _require(k.dim() == 3 and tuple(k.shape[1:]) == (cache.kvHeads, cache.headDimension),
             f"cacheWrite: {_shape(k)} into a cache of {cache.kvHeads} heads of {cache.headDimension}")
    tokens = int(k.shape[0])
    checkPageTable(pageTable, cache, start + tokens)
    return tokens


def checkSplitHalves(x, first, second) -> None:
    """ops/LayoutOps.scala:73-80 (F32, or BF16 here)."""
    checkElementwise("splitHalves", x)
    checkElementwise("splitHalves", first, second)
    _require(x.dtype == first.dtype, f"splitHalves takes one type, not {_name(x.dtype)} and {_name(first.dtype)}")
    _require(x.numel() == 2 * first.numel() and first.dim() >= 1 and x.shape[-1] == 2 * first.shape[-1],
             f"splitHalves: {_shape(x)} into {_shape(first)}")


# ops/HipBase.scala:268-274's codes (fp8 E4M3 bytes as uint8 or float8_e4m3fn)
_CONVERSIONS = {(F32, F16): 0, (F32, BF16): 1, (F16, F32): 2, (BF16, F32): 3, (torch.uint8, F32): 4,
                (torch.float8_e4m3fn, F32): 4}


def checkConvert(x, out) -> int:
    """ops/MemoryOps.scala:68-84: F32 to F16 or BF16, those to F32, and fp8
    E4M3 to F32."""
    requireSameShape("convert", x, out)
    kind = _CONVERSIONS.get((x.dtype, out.dtype))
    _require(kind is not None, f"convert: no conversion from {_name(x.dtype)} to {_name(out.dtype)}")
    return kind


def _on_device(operation: str, *tensors) -> None:
    for t in tensors:
        _require(t.is_cuda, f"{operation}: tensors live in device memory")
        _require(t.is_contiguous(), f"{operation}: tensors are dense row-major")


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _suffix(dtype) -> str:
    return "f32" if dtype == F32 else "bf16"


# ------------------------------------------------------------------ the backend

class HipOps:
    """The GPU backend of this path (the reference's HipOps, ops/HipOps.scala),
    launching libdrift_kernels on `stream` (default: torch's current stream)."""

    name = "hip"

    # At most this many values are quantized as they are written: a decode
    # step's inputs, not a prompt's (ops/HipBase.scala:150-154).
    QuantizedMaximumValues = 8 * 16384

    def __init__(self, stream: Optional[torch.cuda.Stream] = None):
        _lib.load()
        self.stream = stream
        self.onWork = lambda: None  # ops/Ops.scala:29-33
        # the int8 side output's bookkeeping (ops/HipBase.scala:117-214):
        # launches so far, whether int8 products ran, what was last written
        # quantized, and the buffers
        self.deviceWrites = 0
        self.quantizesX = False
        self._quantizedValues: Optional[QuantizedValues] = None
        self._quantizedBuffer: Optional[torch.Tensor] = None
        self._scratch: Optional[torch.Tensor] = None

    def _stream(self):
        s = self.stream if self.stream is not None else torch.cuda.current_stream()
        return ctypes.c_void_p(s.cuda_stream)

    def _launch(self, entry: str, *args) -> None:
        self.deviceWrites += 1
        self.onWork()
        _lib.call(entry, *args, self._stream())

    def wrote(self) -> None:
        """Counts a device write made outside these methods (a copy, a
        torch op): what was written quantized before it no longer serves, as
        every write the reference's backend makes counts
        (ops/HipMemory.scala:57,97,141,147)."""
        self.deviceWrites += 1

    # ---------------------------------------------------------------- int8 side output

    def quantizedTarget(self, out, cols: int) -> Tuple[Optional[QuantizedValues], tuple]:
        """Where a kernel writing `out` (rows of `cols`) also writes it
        quantized, when int8 products may read it, and the kernel's xq, xd,
        xs pointers (nulls when not): ops/HipBase.scala:156-190."""
        values = out.numel()
        eligible = (self.quantizesX and out.dtype == F32 and values <= self.QuantizedMaximumValues
                    and cols % 32 == 0)
        if not eligible:
            return None, (None, None, None)
        size = values + 8 * (values // 32)
        buffer = self._quantizedBuffer
        if buffer is None or buffer.numel() < size or buffer.device != out.device:
            buffer = torch.empty(max(size, 65536), dtype=torch.int8, device=out.device)
            self._quantizedBuffer = buffer
        target = QuantizedValues(out.data_ptr(), values, buffer, 0)
        return target, (_ptr(target.codes()), _ptr(target.scales()), _ptr(target.sums()))

    def wroteQuantized(self, target: Optional[QuantizedValues]) -> None:
        """After the launch that wrote `target` (ops/HipBase.scala:191-193)."""
        if target is not None:
            self._quantizedValues = replace(target, written=self.deviceWrites)

    def quantizedInput(self, x, m: int, k: int):
        """`m` rows of `x` (`k` wide) as the last launch wrote them quantized,
        if it did: (codes, scales, sums), ops/HipBase.scala:195-214."""
        q = self._quantizedValues
        if q is None or q.written != self.deviceWrites or x.dtype != F32:
            return None
        offset = x.data_ptr() - q.address
        first = offset // 4
        if offset >= 0 and offset % (4 * 32) == 0 and k % 32 == 0 and first + m * k <= q.values:
            return q.codes(first, m * k), q.scales(first // 32, m * k // 32), q.sums(first // 32, m * k // 32)
        return None

    def quantize(self, x, m: int, k: int):
        """`m` rows of `x` (`k` wide) quantized per 32 values into scratch
        memory by quantize_x: (codes, scales, sums). Marks that int8 products
        run, so the norms quantize as they write from now on
        (ops/HipLinear.scala:366-386)."""
        self.quantizesX = True
        _require(x.dtype in (F32, BF16) and (m * k) % 32 == 0 and x.numel() >= m * k,
                 f"quantize: {m} rows of {k} from {_shape(x)}")
        _on_device("quantize", x)
        blocks = m * k // 32
        size = m * k + 8 * blocks
        if self._scratch is None or self._scratch.numel() < size or self._scratch.device != x.device:
            self._scratch = torch.empty(max(size, 65536), dtype=torch.int8, device=x.device)
        q = QuantizedValues(0, m * k, self._scratch, 0)
        codes, scales, sums = q.codes(), q.scales(), q.sums()
        self._launch(f"drift_quantize_x_{_suffix(x.dtype)}", _ptr(x), _ptr(codes), _ptr(scales), _ptr(sums), blocks)
        return codes, scales, sums

    def productInput(self, x, m: int, k: int):
        """What an int8 product over `m` rows of `x` reads: the side output
        the launch that wrote x made, else x quantized now
        (ops/HipLinear.scala:142-143)."""
        found = self.quantizedInput(x, m, k)
        return found if found is not None else self.quantize(x, m, k)

    # ---------------------------------------------------------------- norms

    def rmsNorm(self, x, weight, epsilon: float, weightOffset: float, out) -> None:
        """`out = x / sqrt(mean(x^2) + epsilon) * (weight + weightOffset)`
        (ops/NormalisationOps.scala:30-45)."""
        rows = checkRowWise("rmsNorm", x, out, weight)
        _on_device("rmsNorm", x, weight, out)
        self._normRows(x, None, weight, epsilon, weightOffset, out, rows)

    def _normRows(self, x, y, weight, epsilon, weightOffset, out, rows) -> None:
        """rms_norm over `rows`, `y` added to x first when given, out
        quantized too when int8 products may read it
        (ops/HipNormalisation.scala:83-115). Rows of 32 or fewer values take
        the reference's narrow kernel there, which quantizes nothing."""
        cols = x.shape[-1]
        target, (xq, xd, xs) = self.quantizedTarget(out, cols) if cols > 32 else (None, (None, None, None))
        self._launch(f"drift_rms_norm_{_suffix(x.dtype)}", _ptr(x), _ptr(y), _ptr(weight), _ptr(out), rows, cols,
                     epsilon, weightOffset, 1, xq, xd, xs)
        self.wroteQuantized(target)

    def addRmsNorm(self, x, y, norm: RowNorm) -> None:
        """`x += y`, then `norm`'s RMS norm of x into its out, in one launch
        (ops/NormalisationOps.scala:42-45, ops/HipNormalisation.scala:117-131)."""
        checkElementwise("addRmsNorm", x, y)
        rows = checkRowWise("addRmsNorm", x, norm.out, norm.weight)
        _on_device("addRmsNorm", x, y, norm.weight, norm.out)
        self._normRows(x, y, norm.weight, norm.epsilon, norm.weightOffset, norm.out, rows)

    def groupRmsNorm(self, x, weight, groups: int, epsilon: float, weightOffset: float, out) -> None:
        """RMS norm of each of a row's `groups` equal parts on its own, with
        `weight` spanning the whole row ([groups × width])
        (ops/NormalisationOps.scala:46-58): rms_norm over rows × groups rows
        of width values, row r weighted by weight row r % groups, with no
        int8 side output (ops/HipNormalisation.scala:133-158)."""
        rows = checkRowWise("groupRmsNorm", x, out, weight)
        _require(groups > 0 and x.shape[-1] % groups == 0, f"{_shape(x)} in {groups} groups")
        _on_device("groupRmsNorm", x, weight, out)
        self._launch(f"drift_rms_norm_{_suffix(x.dtype)}", _ptr(x), None, _ptr(weight), _ptr(out), rows * groups,
                     x.shape[-1] // groups, epsilon, weightOffset, groups, None, None, None)

    def layerNorm(self, x, weight: Optional[torch.Tensor], bias: Optional[torch.Tensor], epsilon: float,
                  out) -> None:
        """ops/NormalisationOps.scala:74-80 (F32, as the reference's kernel)."""
        rows = checkRowWise("layerNorm", x, out, *[t for t in (weight, bias) if t is not None])
        requireF32("layerNorm", x)
        _on_device("layerNorm", x, out, *[t for t in (weight, bias) if t is not None])
        self._launch("drift_layer_norm_f32", _ptr(x), _ptr(weight), _ptr(bias), _ptr(out), rows, x.shape[-1],
                     epsilon)

    def modulate(self, x, scale, shift, out) -> None:
        """`out = x * (1 + scale) + shift` (ops/ElementwiseOps.scala:28), F32."""
        rows = checkRowWise("modulate", x, out, scale, shift)
        requireF32("modulate", x)
        _on_device("modulate", x, scale, shift, out)
        self._launch("drift_modulate_f32", _ptr(x), _ptr(scale), _ptr(shift), _ptr(out), rows, x.shape[-1])

    # ---------------------------------------------------------------- gated residuals

    def gatedAdd(self, x, y, gate, rowsPerSample: Optional[int] = None) -> None:
        """`x += gate * y` in place (ops/ElementwiseOps.scala:30-31). `gate` is
        F32 [cols], one vector for every row, as the reference's; or, beyond
        it, [samples, cols] with sample s's row for rows
        [s * rowsPerSample, (s + 1) * rowsPerSample)."""
        if gate.dim() <= 1:
            rows = checkRowWise("gatedAdd", x, y, gate)
            per = max(rows, 1)
        else:
            checkElementwise("gatedAdd", x, y)
            requireF32("gatedAdd", gate)
            cols = x.shape[-1]
            rows = x.numel() // cols if cols else 0
            _require(rowsPerSample is not None and rowsPerSample > 0, "gatedAdd: per-sample gates need rowsPerSample")
            samples = -(-rows // rowsPerSample)
            _require(gate.dim() == 2 and tuple(gate.shape) == (samples, cols),
                     f"gatedAdd: {_shape(gate)} for {samples} samples of rows of {cols}")
            per = rowsPerSample
        _on_device("gatedAdd", x, y, gate)
        self._launch(f"drift_gated_add_{_suffix(x.dtype)}", _ptr(x), _ptr(y), _ptr(gate), rows, x.shape[-1], per)

    def modulateChunks(self, x, table, shift: int, scale: int, out) -> None:
        """`out = x * (1 + table chunk scale) + table chunk shift`, x, out
        [rows, C], table F32 [rows, chunks * C] (ops/ElementwiseOps.scala:33-43)."""
        rows, channels, chunks = checkChunks("modulateChunks", x, table, out, shift, scale)
        _on_device("modulateChunks", x, table, out)
        self._launch(f"drift_modulate_chunks_{_suffix(x.dtype)}", _ptr(x), _ptr(table), _ptr(out), rows, channels,
                     chunks, shift, scale)

    def gatedAddChunk(self, x, y, table, gate: int) -> None:
        """`x += table chunk gate * y`, the tables as modulateChunks'
        (ops/ElementwiseOps.scala:45-46)."""
        rows, channels, chunks = checkChunks("gatedAddChunk", x, table, y, gate)
        _on_device("gatedAddChunk", x, y, table)
        self._launch(f"drift_gated_add_chunk_{_suffix(x.dtype)}", _ptr(x), _ptr(y), _ptr(table), rows, channels,
                     chunks, gate)

    def rowGatedAdd(self, x, y, gate) -> None:
        """`x[r] += gate[r] * y[r]`: one gate per row, gate F32 [rows]
        (ops/ElementwiseOps.scala:48-49)."""
        rows, cols = checkRowGatedAdd(x, y, gate)
        _on_device("rowGatedAdd", x, y, gate)
        self._launch(f"drift_row_gated_add_{_suffix(x.dtype)}", _ptr(x), _ptr(y), _ptr(gate), rows, cols)

    def layerNormModulate(self, x, scale, shift, epsilon: float, out, rowsPerSample: Optional[int] = None) -> None:
        """AdaLN in one launch: layerNorm(x, None, None, epsilon) then
        modulate with sample s's row of `scale` and `shift` ([samples, C])
        over that sample's rows (models/Wan.scala:431-432). x, out [rows, C]."""
        checkElementwise("layerNormModulate", x, out)
        requireF32("layerNormModulate", scale, shift)
        _require(x.dim() == 2, f"layerNormModulate takes [rows, C], not {_shape(x)}")
        rows, cols = x.shape
        scale2 = scale.reshape(-1, cols) if scale.dim() == 1 else scale
        _require(scale2.dim() == 2 and scale2.shape[1] == cols and tuple(shift.shape) == tuple(scale.shape),
                 f"layerNormModulate: scale {_shape(scale)}, shift {_shape(shift)} for rows of {cols}")
        samples = scale2.shape[0]
        per = rowsPerSample if rowsPerSample is not None else -(-rows // samples)
        _require(per > 0 and samples * per >= rows,
                 f"layerNormModulate: {samples} samples of {per} rows for {rows} rows")
        _on_device("layerNormModulate", x, scale, shift, out)
        self._launch(f"drift_layer_norm_modulate_{_suffix(x.dtype)}", _ptr(x), _ptr(scale), _ptr(shift), _ptr(out),
                     rows, cols, per, epsilon)

    # ---------------------------------------------------------------- activations

    def activation(self, kind: Activation, x, out) -> None:
        self.scaledActivation(kind, 1.0, x, out)

    def scaledActivation(self, kind: Activation, inputScale: float, x, out) -> None:
        """`out = kind(inputScale * x)` (ops/NormalisationOps.scala:10-19)."""
        checkElementwise("activation", x, out)
        _on_device("activation", x, out)
        self._launch(f"drift_activation_{_suffix(x.dtype)}", _ptr(x), _ptr(out), x.numel(), int(kind), inputScale)

    def gated(self, kind: Activation, gate, up, out) -> None:
        """`out = kind(gate) * up` (ops/NormalisationOps.scala:21-24)."""
        checkElementwise("gated", gate, up, out)
        _on_device("gated", gate, up, out)
        target, (xq, xd, xs) = self.quantizedTarget(out, out.shape[-1])
        self._launch(f"drift_gated_{_suffix(gate.dtype)}", _ptr(gate), _ptr(up), _ptr(out), gate.numel(), int(kind),
                     xq, xd, xs)
        self.wroteQuantized(target)

    # ---------------------------------------------------------------- rotary

    def rope(self, x, positions, rope: Rope, out) -> None:
        """ops/AttentionOps.scala:42-45."""
        tokens, heads, dimension = checkRope(x, positions, rope, out)
        _on_device("rope", x, positions, out)
        s = rope.sections.launch_sizes()
        self._launch(f"drift_rope_{_suffix(x.dtype)}", _ptr(x), _ptr(positions), _ptr(out), tokens, heads, dimension,
                     rope.rotaryDimensions, rope.theta, int(rope.layout), rope.sections.code, *s)

    def ropeTable(self, x, cosines, sines, out, halves: bool = False) -> None:
        """ops/AttentionOps.scala:25-40."""
        tokens, heads, d, pairs, per_head = checkRopeTable(x, cosines, sines, out)
        _on_device("ropeTable", x, cosines, sines, out)
        self._launch(f"drift_rope_table_{_suffix(x.dtype)}", _ptr(x), _ptr(cosines), _ptr(sines), _ptr(out), tokens,
                     heads, d, pairs, int(per_head), int(halves))

    def rope3d(self, x, frames: int, rows: int, columns: int, out, tokenOffset: int = 0,
               theta: float = 10000.0) -> None:
        """Wan's 3-D RoPE with the angles made in the kernel: what
        models/Wan.scala:324-361 tabulates and :442-443 applies, for a
        `frames x rows x columns` grid; token i of x is grid token
        (tokenOffset + i) mod (frames * rows * columns)."""
        checkElementwise("rope3d", x, out)
        _require(x.dim() == 3, f"rope3d takes [tokens, heads, D], not {_shape(x)}")
        _on_device("rope3d", x, out)
        tokens, heads, d = x.shape
        self._launch(f"drift_rope_3d_{_suffix(x.dtype)}", _ptr(x), _ptr(out), tokens, heads, d, frames, rows,
                     columns, tokenOffset, theta)

    def queryKeyNormRope(self, q, k, norms: QueryKeyNorms, positions, rotatedQueries, rotatedKeys) -> None:
        """Per-head RMS norms of queries and keys, then their rope, in one
        launch: the composition ops/AttentionOps.scala:87-107 runs as
        rmsNorm, rmsNorm, rope, rope. q [t, heads, D], k [t, kvHeads, D]."""
        checkElementwise("queryKeyNormRope", q, rotatedQueries)
        checkElementwise("queryKeyNormRope", k, rotatedKeys)
        _require(q.dtype == k.dtype, "queryKeyNormRope takes one type for queries and keys")
        _require(q.dim() == 3 and k.dim() == 3 and q.shape[0] == k.shape[0] and q.shape[2] == k.shape[2],
                 f"queryKeyNormRope: queries {_shape(q)}, keys {_shape(k)}")
        tokens, heads, d = q.shape
        kv = k.shape[1]
        checkRope(q, positions, norms.rope, rotatedQueries)
        for name, w in (("queryNorm", norms.queryNorm), ("keyNorm", norms.keyNorm)):
            requireF32("queryKeyNormRope", w)
            _require(tuple(w.shape) == (d,), f"queryKeyNormRope: {name} {_shape(w)} for heads of {d}")
        _on_device("queryKeyNormRope", q, k, rotatedQueries, rotatedKeys, norms.queryNorm, norms.keyNorm, positions)
        r = norms.rope
        self._launch(f"drift_qk_norm_rope_{_suffix(q.dtype)}", _ptr(q), _ptr(k), _ptr(rotatedQueries),
                     _ptr(rotatedKeys), _ptr(norms.queryNorm), _ptr(norms.keyNorm), _ptr(positions), tokens, heads,
                     kv, d, norms.epsilon, norms.weightOffset, r.rotaryDimensions, r.theta, int(r.layout),
                     r.sections.code, *r.sections.launch_sizes())

    # ---------------------------------------------------------------- attention inputs

    # attention.hip's ATTENTION_INPUT_DIMENSION (ops/HipAttention.scala:217-218)
    AttentionInputDimension = 512

    def cacheWrite(self, k, v, cache: KvCache, pageTable, start: int, badPage: Optional[torch.Tensor] = None) -> None:
        """Keys and values [tokens, kvHeads, D] into the cache at positions
        start .. start + tokens - 1 (ops/AttentionOps.scala:52-63). A page
        table entry outside the cache (which the reference fails on) writes
        nothing and sets `badPage` (int32 [1], device) to 1 when given."""
        tokens = checkCacheWrite(k, v, cache, pageTable, start)
        _on_device("cacheWrite", k, v, cache.keys, cache.values, pageTable)
        self._launch(f"drift_cache_write_{_suffix(k.dtype)}", _ptr(k), _ptr(v), _ptr(cache.keys), _ptr(cache.values),
                     _ptr(pageTable), pageTable.numel(), cache.pages, tokens, cache.kvHeads, cache.headDimension,
                     cache.pageSize, start, _ptr(badPage))

    def splitHalves(self, x, first, second) -> None:
        """Rows [.., 2 d] into their halves (ops/LayoutOps.scala:31)."""
        checkSplitHalves(x, first, second)
        _on_device("splitHalves", x, first, second)
        d = first.shape[-1]
        self._launch(f"drift_split_halves_{_suffix(x.dtype)}", _ptr(x), _ptr(first), _ptr(second), first.numel() // d,
                     d)

    def attentionInputs(self, queryAndGate, keys, values, norms: QueryKeyNorms, positions, cache: KvCache, pageTable,
                        start: int, queries, gate, rotatedKeys, rotatedQueries,
                        badPage: Optional[torch.Tensor] = None) -> None:
        """A gated attention's inputs in one launch (ops/AttentionOps.scala:
        66-107, ops/HipAttention.scala:144-215): the query halves of
        `queryAndGate` [t, heads, 2 D] normed and turned into
        `rotatedQueries`, the gate halves into `gate`, the keys normed,
        turned and written to `cache` with `values` at `start`. `queries` and
        `rotatedKeys` are the unfused steps' scratch, checked and not written,
        as the reference's fused launch leaves them."""
        t, heads, d = (int(n) for n in queries.shape) if queries.dim() == 3 else (0, 0, 0)
        _require(d <= self.AttentionInputDimension,
                 f"attentionInputs: heads of {d} values (at most {self.AttentionInputDimension} fused)")
        checkSplitHalves(queryAndGate, queries, gate)
        checkRope(queries, positions, norms.rope, rotatedQueries)
        checkRope(keys, positions, norms.rope, rotatedKeys)
        checkCacheWrite(rotatedKeys, values, cache, pageTable, start)
        self._attentionInputs(queryAndGate, keys, values, norms, positions, cache, pageTable, start, gate,
                              rotatedQueries, badPage)

    def queryKeyNormRopeCache(self, q, k, v, norms: QueryKeyNorms, positions, cache: KvCache, pageTable, start: int,
                              rotatedQueries, badPage: Optional[torch.Tensor] = None) -> None:
        """The dense decoders' attention inputs in one launch: per-head RMS
        norms of q [t, heads, D] and k [t, kvHeads, D], their rope, the
        queries into `rotatedQueries` and the keys, with the values v, into
        the cache at `start` (models/DenseDecoder.scala:834-863 runs rmsNorm,
        rmsNorm, rope, rope, cacheWrite)."""
        _require(q.dim() == 3 and q.shape[2] <= self.AttentionInputDimension,
                 f"queryKeyNormRopeCache: queries {_shape(q)}")
        checkRope(q, positions, norms.rope, rotatedQueries)
        checkRope(k, positions, norms.rope, k)
        checkCacheWrite(k, v, cache, pageTable, start)
        self._attentionInputs(q, k, v, norms, positions, cache, pageTable, start, None, rotatedQueries, badPage)

    def _attentionInputs(self, queryAndGate, keys, values, norms, positions, cache, pageTable, start, gate,
                         rotatedQueries, badPage) -> None:
        tokens, heads, d = (int(n) for n in rotatedQueries.shape)
        _require(tuple(keys.shape) == (tokens, cache.kvHeads, d),
                 f"attentionInputs: keys {_shape(keys)} for {tokens} tokens of heads of {d}")
        _require(queryAndGate.dtype == keys.dtype == values.dtype == rotatedQueries.dtype and
                 (gate is None or gate.dtype == keys.dtype),
                 "attentionInputs takes one type for queries, gate, keys and values")
        for name, w in (("queryNorm", norms.queryNorm), ("keyNorm", norms.keyNorm)):
            requireF32("attentionInputs", w)
            _require(tuple(w.shape) == (d,), f"attentionInputs: {name} {_shape(w)} for heads of {d}")
        tensors = [queryAndGate, keys, values, norms.queryNorm, norms.keyNorm, positions, cache.keys, cache.values,
                   pageTable, rotatedQueries] + ([] if gate is None else [gate])
        _on_device("attentionInputs", *tensors)
        r = norms.rope
        self._launch(f"drift_attention_inputs_{_suffix(keys.dtype)}", _ptr(queryAndGate), _ptr(keys), _ptr(values),
                     _ptr(norms.queryNorm), _ptr(norms.keyNorm), norms.epsilon, norms.weightOffset, _ptr(positions),
                     tokens, heads, cache.kvHeads, d, r.rotaryDimensions, r.theta, int(r.layout), r.sections.code,
                     *r.sections.launch_sizes(), _ptr(rotatedQueries), _ptr(gate), _ptr(cache.keys),
                     _ptr(cache.values), _ptr(pageTable), pageTable.numel(), cache.pages, cache.pageSize, start,
                     _ptr(badPage))

    # ---------------------------------------------------------------- embedding, convert

    def embedding(self, table, ids, out, badId: Optional[torch.Tensor] = None) -> None:
        """Rows `ids` of a table, decoded (ops/LinearOps.scala:16), into out
        F32 or BF16: a StoredTable, or a RotatedTable as the BF16 it holds
        (ops/HipLinear.scala:28,54-92). An id outside the table (which the
        reference refuses) gets a zero row and sets `badId` (int32 [1],
        device) to 1 when given."""
        checkEmbedding(table, ids, out)
        if isinstance(table, RotatedTable):
            self._rotated(f"drift_rotated_embedding_{_suffix(out.dtype)}", table, out, ids, badId)
            return
        t = self._checkStored("embedding", table)
        _require(table.cols % 8 == 0 or t.values == 1,
                 f"embedding: rows of {table.cols} values (quant kernels take multiples of 8)")
        _on_device("embedding", table.data, ids, out)
        vocab, cols = table.shape
        if t.name == "Q8_0":
            self._launch(f"drift_embedding_q8_0_{_suffix(out.dtype)}", _ptr(table.data), _ptr(ids), _ptr(out),
                         ids.shape[0], vocab, cols, _ptr(badId))
        else:
            self._launch(f"drift_embedding_{_suffix(out.dtype)}", _ptr(table.data), t.ggmlId, _ptr(ids), _ptr(out),
                         ids.shape[0], vocab, cols, _ptr(badId))

    def rotated(self, codes, parts: ConvRotParts) -> RotatedTable:
        """Ops.rotated (ops/LinearOps.scala:21-33): ComfyUI's rotated linear
        [N, K] left where the file holds it, `codes` I8 [N, K] or with
        `parts.levels` the 4-bit codes [N, K / 2], seen as the weight they
        make with `parts`; `embedding`, `dequantize` and `convert` decode it."""
        return checkRotated(codes, parts)

    def _rotated(self, entry: str, table: RotatedTable, out, ids=None, badId=None) -> None:
        table = checkRotated(table.codes, table.parts)
        p, l = table.parts, table.parts.levels
        _require(table.codes.is_contiguous() and p.scales.is_contiguous() and
                 (l is None or l.codebook.is_contiguous() and l.relative.is_contiguous()),
                 f"{entry}: codes, scales and levels must be contiguous")
        tensors = [table.codes, p.scales, out] + ([] if l is None else [l.codebook, l.relative]) + \
            ([] if ids is None else [ids])
        _on_device(entry, *tensors)
        rows, cols = table.shape
        head = (_ptr(table.codes), _ptr(p.scales), p.scales.numel(), None if l is None else _ptr(l.codebook),
                None if l is None else _ptr(l.relative), 0 if l is None else l.groupSize)
        if ids is None:
            self._launch(entry, *head, _ptr(out), rows, cols)
        else:
            self._launch(entry, *head, _ptr(ids), _ptr(out), ids.shape[0], rows, cols, _ptr(badId))

    def dequantize(self, table, out) -> None:
        """The whole table decoded into out [rows, cols], BF16 or F16, for
        the GEMM path (kernels/matvec.hip:801-827 dequantize, dequantize_bf16);
        a RotatedTable to BF16 (ops/HipBase.scala:276-311)."""
        if isinstance(table, RotatedTable):
            _require(out.dtype == BF16, f"convert: no conversion from {table.dtype} to {_name(out.dtype)}")
            _require(tuple(out.shape) == table.shape, f"convert: out {_shape(out)} for {_dims(table.shape)}")
            self._rotated("drift_rotated_dequantize_bf16", table, out)
            return
        t = self._checkStored("dequantize", table)
        _require(out.dtype in (BF16, F16), f"dequantize writes BF16 or F16, not {_name(out.dtype)}")
        _require(tuple(out.shape) == table.shape, f"dequantize: out {_shape(out)} for a table {_dims(table.shape)}")
        _require(table.cols % 8 == 0 or t.values == 1,
                 f"dequantize: rows of {table.cols} values (quant kernels take multiples of 8)")
        _on_device("dequantize", table.data, out)
        entry = "drift_dequantize_bf16" if out.dtype == BF16 else "drift_dequantize_f16"
        self._launch(entry, _ptr(table.data), t.ggmlId, _ptr(out), table.shape[0], table.cols)

    @staticmethod
    def _checkStored(operation: str, table: StoredTable) -> StorageType:
        _require(isinstance(table, StoredTable), f"{operation}: a table of stored bytes")
        t = table.dtype
        vocab, cols = table.shape
        _require(cols % t.values == 0, f"{cols} elements are not whole {t.name} blocks of {t.values}")
        _require(table.data.dtype == torch.uint8 and tuple(table.data.shape) == (vocab, t.rowBytes(cols)),
                 f"{operation}: {t.name} bytes {_shape(table.data)} for rows of {cols}")
        _require(table.data.is_contiguous(), f"{operation}: {t.name} bytes must be contiguous rows")
        return t

    def convert(self, x, out) -> None:
        """ops/MemoryOps.scala:46; a rotated linear converts to BF16
        (ops/HipMemory.scala:127-130)."""
        if isinstance(x, RotatedTable):
            self.dequantize(x, out)
            return
        kind = checkConvert(x, out)
        _on_device("convert", x, out)
        self._launch("drift_convert", _ptr(x), _ptr(out), x.numel(), kind)
