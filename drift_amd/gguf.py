"""GGUF files (versions 2 and 3, little-endian), read as the runner reads them
(runner/src/drift/runner/formats/Gguf.scala): metadata, tensor infos, then
the data section, each tensor at a multiple of `general.alignment`. The file
is memory-mapped; a tensor's bytes are a slice of the mapping until they are
copied to the device (`GgufFile.table`), for instance a model's Q8_0
`token_embd.weight` for `HipOps.embedding`.

GGUF lists dimensions innermost first (`ne[0]` is the row length); shapes
here are outermost first, reversed once, as the reference's `Shape`. The
reference's checks are kept, with its messages (raised as FormatError for its
FormatException): the magic and version, plausible counts, metadata value
types, a power-of-two alignment, at most 8 dimensions, rows of whole blocks,
aligned offsets within the data, each tensor's byte size agreeing with the
room the file gives it (Gguf.scala:262-285), and ROCmFP4's finite scale
bytes (tensor/RocmFp4.scala:64-73).
"""

from __future__ import annotations

import math
import mmap
import struct
import warnings
from dataclasses import dataclass
from typing import Dict, Optional, Tuple

import numpy as np

from .ops import STORAGE_TYPES, StoredTable


class FormatError(ValueError):
    """formats/StoredTensor.scala:57 FormatException."""


@dataclass(frozen=True)
class GgmlType:
    """A GGUF tensor type the runner decodes (tensor/DType.scala:168-193):
    values per block and bytes per block."""
    name: str
    ggmlId: int
    values: int
    bytes: int

    def byteSize(self, elements: int) -> int:
        if elements % self.values:
            raise FormatError(f"{elements} elements are not whole {self.name} blocks of {self.values}")
        size = elements // self.values * self.bytes
        if size > _INT64_MAX:
            raise FormatError(f"{elements} {self.name} elements do not fit 2^63 bytes")
        return size


# DType.all's GGUF types (tensor/DType.scala:168-193 and the quant objects).
GGML_TYPES = {t.ggmlId: t for t in (
    GgmlType("F32", 0, 1, 4), GgmlType("F16", 1, 1, 2), GgmlType("BF16", 30, 1, 2), GgmlType("I8", 24, 1, 1),
    GgmlType("I32", 26, 1, 4), GgmlType("I64", 27, 1, 8), GgmlType("Q4_0", 2, 32, 18), GgmlType("Q4_1", 3, 32, 20),
    GgmlType("Q5_0", 6, 32, 22), GgmlType("Q5_1", 7, 32, 24), GgmlType("Q8_0", 8, 32, 34),
    GgmlType("Q2_K", 10, 256, 84), GgmlType("Q3_K", 11, 256, 110), GgmlType("Q4_K", 12, 256, 144),
    GgmlType("Q5_K", 13, 256, 176), GgmlType("Q6_K", 14, 256, 210), GgmlType("IQ4_NL", 20, 32, 18),
    GgmlType("IQ4_XS", 23, 256, 136), GgmlType("Q4_0_ROCMFP4", 100, 32, 18),
    GgmlType("Q4_0_ROCMFP4_FAST", 101, 32, 17))}

# GGML's type ids the runner does not decode, named for the error (DType.scala:199-216).
UNSUPPORTED_NAMES = {9: "Q8_1", 15: "Q8_K", 16: "IQ2_XXS", 17: "IQ2_XS", 18: "IQ3_XXS", 19: "IQ1_S", 21: "IQ3_S",
                     22: "IQ2_S", 25: "I16", 28: "F64", 29: "IQ1_M", 34: "TQ1_0", 35: "TQ2_0", 39: "MXFP4"}

DEFAULT_ALIGNMENT = 32
_INT64_MAX = (1 << 63) - 1
_ROCM_SAMPLED_BLOCKS = 4096  # RocmFp4.scala:41-42


def type_of(ggml_id: int):
    """DType.fromGgmlId: the type, or the reason it is unsupported."""
    t = GGML_TYPES.get(ggml_id)
    if t is not None:
        return t, None
    name = UNSUPPORTED_NAMES.get(ggml_id)
    return None, (f"unknown GGML type id {ggml_id}" if name is None else f"GGML type {name} is not supported yet")


@dataclass(frozen=True)
class StoredTensor:
    """formats/StoredTensor.scala:9-38: a tensor's type, shape (outermost
    first) and where its bytes start in the whole file."""
    name: str
    dtype: GgmlType
    shape: Tuple[int, ...]
    fileOffset: int

    @property
    def byteSize(self) -> int:
        # exact integers: the dimensions of a crafted file can multiply past
        # an int64, which is refused
        elements = math.prod(int(d) for d in self.shape)
        if elements > _INT64_MAX:
            raise FormatError(f"{self.name} of {list(self.shape)} has more than 2^63 elements")
        return self.dtype.byteSize(elements)


class GgufFile:
    """A read GGUF file: `metadata` (key -> int, float, bool, str or list),
    `tensors` (name -> StoredTensor) and `unsupported` (name -> reason). The
    mapping stays open while the object lives, or until `close()`."""

    def __init__(self, source: str, version: int, metadata: dict, alignment: int, tensors: Dict[str, StoredTensor],
                 unsupported: Dict[str, str], buffer):
        self.source, self.version, self.metadata, self.alignment = source, version, metadata, alignment
        self.tensors, self.unsupported = tensors, unsupported
        self._buffer = buffer

    # GgufFile's typed getters (Gguf.scala:37-82)
    def _value(self, key: str):
        if key not in self.metadata:
            raise FormatError(f"{self.source} has no {key}")
        return self.metadata[key]

    def long(self, key: str) -> int:
        v = self._value(key)
        if isinstance(v, bool) or not isinstance(v, int) or not -(1 << 63) <= v < (1 << 63):
            raise FormatError(f"{self.source}: {key} is {v!r}")
        return v

    def double(self, key: str) -> float:
        v = self._value(key)
        if isinstance(v, bool) or not isinstance(v, (int, float)):
            raise FormatError(f"{self.source}: {key} is {v!r}")
        return float(v)

    def string(self, key: str) -> str:
        v = self._value(key)
        if not isinstance(v, str):
            raise FormatError(f"{self.source}: {key} is {v!r}")
        return v

    def boolean(self, key: str) -> bool:
        v = self._value(key)
        if not isinstance(v, bool):
            raise FormatError(f"{self.source}: {key} is {v!r}")
        return v

    def strings(self, key: str):
        v = self._value(key)
        if not isinstance(v, list) or not all(isinstance(x, str) for x in v):
            raise FormatError(f"{self.source}: {key} is {v!r}")
        return list(v)

    @property
    def architecture(self) -> str:
        return self.string("general.architecture")

    def __getitem__(self, name: str) -> StoredTensor:
        """TensorSource.apply (StoredTensor.scala:46-54)."""
        if name in self.tensors:
            return self.tensors[name]
        raise KeyError(f"{name}: {self.unsupported[name]}" if name in self.unsupported else f"no tensor {name}")

    def bytes(self, name: str) -> np.ndarray:
        """A tensor's bytes, a view of the mapping (not copied)."""
        t = self[name]
        return np.frombuffer(self._buffer, np.uint8, t.byteSize, t.fileOffset)

    def table(self, name: str, device="cuda") -> StoredTable:
        """A 2-D tensor ([rows, cols]) as a table on `device` for
        HipOps.embedding / dequantize: its bytes copied as they lie in the
        file, [rows, row bytes]."""
        import torch

        t = self[name]
        if len(t.shape) != 2:
            raise FormatError(f"{name} is {list(t.shape)}, not a table")
        if t.dtype.name not in STORAGE_TYPES:
            raise FormatError(f"{name}: {t.dtype.name} tables have no gather kernel")
        rows, cols = t.shape
        with warnings.catch_warnings():
            # the read-only mapping is only read, by the copy to the device
            warnings.filterwarnings("ignore", message="The given NumPy array is not writable")
            host = torch.from_numpy(self.bytes(name).reshape(rows, -1))
        data = host.to(device, copy=True)
        return StoredTable(data, STORAGE_TYPES[t.dtype.name], cols)

    def close(self) -> None:
        if isinstance(self._buffer, mmap.mmap):
            self._buffer.close()


def open_gguf(path: str) -> GgufFile:
    """Gguf.open: maps the file and reads it."""
    with open(path, "rb") as f:
        size = f.seek(0, 2)
        if size == 0:
            raise FormatError(f"{path}: truncated at byte 0 (needs 8 more)")
        buffer = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
    try:
        return read(buffer, path)
    except Exception:
        buffer.close()
        raise


def read(buffer, source: str = "<bytes>") -> GgufFile:
    """Gguf.read: the whole file's bytes (bytes, bytearray or mmap)."""
    return _Reader(buffer, source).read()


class _Reader:
    def __init__(self, buffer, source: str):
        self.b, self.source, self.position = buffer, source, 0
        self.size = len(buffer)

    def fail(self, message: str):
        raise FormatError(f"{self.source}: {message}")

    def need(self, n: int) -> None:
        if n < 0 or self.position + n > self.size:
            self.fail(f"truncated at byte {self.position} (needs {n} more)")

    def take(self, fmt: str):
        n = struct.calcsize(fmt)
        self.need(n)
        v = struct.unpack_from(fmt, self.b, self.position)[0]
        self.position += n
        return v

    def count(self, what: str) -> int:
        """A count or a length: a u64 that must fit what follows it."""
        v = self.take("<q")
        if v < 0 or v > self.size:
            self.fail(f"{what} of {v} is not plausible")
        return v

    def text(self) -> str:
        n = self.count("string length")
        self.need(n)
        s = bytes(self.b[self.position:self.position + n]).decode("utf-8", errors="replace")
        self.position += n
        return s

    def value(self, kind: int):
        simple = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 10: "<Q", 11: "<q", 12: "<d"}
        if kind in simple:
            return self.take(simple[kind])
        if kind == 7:
            return self.take("<B") != 0
        if kind == 8:
            return self.text()
        if kind == 9:
            element = self.take("<I")
            n = self.count("array length")
            return [self.value(element) for _ in range(n)]
        self.fail(f"unknown metadata value type {kind}")

    def read(self) -> GgufFile:
        self.need(8)
        if bytes(self.b[0:4]) != b"GGUF":
            self.fail("not a GGUF file")
        self.position = 4
        version = self.take("<I")
        if version not in (2, 3):
            self.fail("big-endian GGUF is not supported" if version > 0xFFFF
                      else f"GGUF version {version} is not supported")
        tensor_count = self.count("tensor count")
        metadata_count = self.count("metadata count")
        metadata = {}
        for _ in range(metadata_count):
            key = self.text()
            metadata[key] = self.value(self.take("<I"))
        alignment = metadata.get("general.alignment", None)
        if alignment is None:
            alignment = DEFAULT_ALIGNMENT
        elif isinstance(alignment, bool) or not isinstance(alignment, int) or alignment <= 0 or \
                alignment & (alignment - 1):
            self.fail(f"general.alignment is {alignment!r}")
        infos = []
        for _ in range(tensor_count):
            name = self.text()
            rank = self.take("<I")
            if rank > 8:
                self.fail(f"{name} has {rank} dimensions")
            dims = [self.count(f"{name} dimension") for _ in range(rank)]
            type_id, offset = self.take("<I"), self.take("<q")
            # an offset before the data section would place the tensor over
            # the header (the reference's bounds-checked slice refuses it)
            if offset < 0:
                self.fail(f"{name} starts at offset {offset}, before the data section")
            infos.append((name, dims, type_id, offset))
        data_start = (self.position + alignment - 1) // alignment * alignment
        data_bytes = self.size - data_start
        if data_bytes < 0:
            self.fail("truncated before the data section")
        described: Dict[str, Tuple[Optional[StoredTensor], Optional[str]]] = {}
        for name, dims, type_id, offset in infos:
            t, reason = type_of(type_id)
            if t is None:
                described[name] = (None, reason)
                continue
            if dims and dims[0] % t.values != 0:
                self.fail(f"{name}: rows of {dims[0]} are not whole {t.name} blocks")
            if offset % alignment != 0:
                self.fail(f"{name} is not aligned to {alignment}")
            if offset > data_bytes:
                self.fail(f"{name} runs past the end of the file")
            tensor = StoredTensor(name, t, tuple(reversed(dims)), data_start + offset)
            try:
                size = tensor.byteSize
            except FormatError as e:
                self.fail(str(e))
            if offset + size > data_bytes:
                self.fail(f"{name} runs past the end of the file")
            described[name] = (tensor, None)
        self.check_spans(infos, described, data_bytes, alignment)
        tensors = {n: t for n, (t, _) in described.items() if t is not None}
        for t in tensors.values():
            self.rejects(t)
        unsupported = {n: r for n, (_, r) in described.items() if r is not None}
        return GgufFile(self.source, version, metadata, alignment, tensors, unsupported, self.b)

    def check_spans(self, infos, described, data_bytes: int, alignment: int) -> None:
        """Gguf.checkSpans (Gguf.scala:262-285): each tensor's byte size and
        the room to the next tensor agree up to the alignment padding."""
        by_offset = sorted(infos, key=lambda i: i[3])
        for index, (name, _, _, offset) in enumerate(by_offset):
            tensor, _ = described[name]
            if tensor is None:
                continue
            end = by_offset[index + 1][3] if index + 1 < len(by_offset) else data_bytes
            room = end - offset
            if room < tensor.byteSize or room - tensor.byteSize >= alignment:
                self.fail(f"{name} is {tensor.dtype.name} {list(tensor.shape)}, {tensor.byteSize} bytes, "
                          f"but the file gives it {room}")

    def rejects(self, t: StoredTensor) -> None:
        """RocmFp4's check that a tensor's scale bytes are finite E4M3 codes."""
        if not t.dtype.name.startswith("Q4_0_ROCMFP4"):
            return
        offsets = (16, 17) if t.dtype.name == "Q4_0_ROCMFP4" else (16,)
        blocks = min(t.byteSize // t.dtype.bytes, _ROCM_SAMPLED_BLOCKS)
        # a copy: a view left on the mapping would keep a refused file's
        # mapping from closing
        data = np.frombuffer(self.b, np.uint8, blocks * t.dtype.bytes, t.fileOffset).reshape(blocks, -1).copy()
        scales = data[:, list(offsets)]
        bad = np.flatnonzero(scales.reshape(-1) > 0x7E)  # the first in byte order, as the reference scans
        if bad.size:
            block, which = divmod(int(bad[0]), len(offsets))
            where = block * t.dtype.bytes + offsets[which]
            self.fail(f"{t.name}: scale byte 0x{int(scales[block, which]):02x} at byte {where} is not a finite "
                      f"unsigned E4M3, so this is not {t.dtype.name}")


def write(path: str, metadata: dict, tensors: Dict[str, Tuple[str, Tuple[int, ...], np.ndarray]],
          alignment: int = DEFAULT_ALIGNMENT, version: int = 3) -> None:
    """Writes a GGUF file: `metadata` key -> value (int as i64 unless it is
    a bool, float as f64, str, or a list of str), `tensors` name -> (type
    name, shape outermost first, bytes). For building test files and tables."""
    ids = {t.name: t.ggmlId for t in GGML_TYPES.values()}
    out = bytearray(b"GGUF")
    out += struct.pack("<IQQ", version, len(tensors), len(metadata) + (alignment != DEFAULT_ALIGNMENT))

    def text(s: str):
        b = s.encode()
        return struct.pack("<Q", len(b)) + b

    def value(v):
        if isinstance(v, bool):
            return struct.pack("<IB", 7, int(v))
        if isinstance(v, int):
            return struct.pack("<Iq", 11, v)
        if isinstance(v, float):
            return struct.pack("<Id", 12, v)
        if isinstance(v, str):
            return struct.pack("<I", 8) + text(v)
        if isinstance(v, list):
            return struct.pack("<IIQ", 9, 8, len(v)) + b"".join(text(x) for x in v)
        raise TypeError(v)

    items = list(metadata.items())
    if alignment != DEFAULT_ALIGNMENT:
        items.append(("general.alignment", struct.pack("<II", 4, alignment)))
    for key, v in items:
        out += text(key) + (v if isinstance(v, bytes) else value(v))
    offset = 0
    layout = []
    for name, (type_name, shape, data) in tensors.items():
        raw = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
        out += text(name) + struct.pack("<I", len(shape)) + b"".join(struct.pack("<Q", d) for d in reversed(shape))
        out += struct.pack("<Iq", ids[type_name], offset)
        layout.append(raw)
        offset = (offset + raw.size + alignment - 1) // alignment * alignment
    out += b"\0" * ((-len(out)) % alignment)
    for i, raw in enumerate(layout):
        out += raw.tobytes()
        if i + 1 < len(layout):
            out += b"\0" * ((-raw.size) % alignment)
    with open(path, "wb") as f:
        f.write(out)
