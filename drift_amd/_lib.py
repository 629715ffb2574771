"""Loads libdrift_kernels.so (the C ABI declared in include/drift_kernels.h)
and declares every entry point's signature for ctypes.

There is no fallback: if the library is not built, importing the ops fails
with a message that says how to build it.
"""

from __future__ import annotations

import ctypes
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
LIBRARY = os.path.join(HERE, "libdrift_kernels.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "drift_kernels.h")

_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_F32 = ctypes.c_float
_F64 = ctypes.c_double

# Argument types of every entry point, in the header's order.
SIGNATURES = {
    "drift_abi_version": (_I32, []),
    "drift_error_string": (ctypes.c_char_p, [_I32]),
    "drift_last_error": (ctypes.c_char_p, []),
    "drift_quantize_x_f32": (_I32, [_P, _P, _P, _P, _I64, _P]),
    "drift_quantize_x_bf16": (_I32, [_P, _P, _P, _P, _I64, _P]),
    "drift_rms_norm_f32": (_I32, [_P, _P, _P, _P, _I64, _I32, _F32, _F32, _I32, _P, _P, _P, _P]),
    "drift_rms_norm_bf16": (_I32, [_P, _P, _P, _P, _I64, _I32, _F32, _F32, _I32, _P, _P, _P, _P]),
    "drift_layer_norm_f32": (_I32, [_P, _P, _P, _P, _I64, _I32, _F32, _P]),
    "drift_modulate_f32": (_I32, [_P, _P, _P, _P, _I64, _I32, _P]),
    "drift_layer_norm_modulate_f32": (_I32, [_P, _P, _P, _P, _I64, _I32, _I64, _F32, _P]),
    "drift_layer_norm_modulate_bf16": (_I32, [_P, _P, _P, _P, _I64, _I32, _I64, _F32, _P]),
    "drift_gated_add_f32": (_I32, [_P, _P, _P, _I64, _I32, _I64, _P]),
    "drift_gated_add_bf16": (_I32, [_P, _P, _P, _I64, _I32, _I64, _P]),
    "drift_modulate_chunks_f32": (_I32, [_P, _P, _P, _I64, _I32, _I32, _I32, _I32, _P]),
    "drift_modulate_chunks_bf16": (_I32, [_P, _P, _P, _I64, _I32, _I32, _I32, _I32, _P]),
    "drift_gated_add_chunk_f32": (_I32, [_P, _P, _P, _I64, _I32, _I32, _I32, _P]),
    "drift_gated_add_chunk_bf16": (_I32, [_P, _P, _P, _I64, _I32, _I32, _I32, _P]),
    "drift_row_gated_add_f32": (_I32, [_P, _P, _P, _I64, _I32, _P]),
    "drift_row_gated_add_bf16": (_I32, [_P, _P, _P, _I64, _I32, _P]),
    "drift_activation_f32": (_I32, [_P, _P, _I64, _I32, _F32, _P]),
    "drift_activation_bf16": (_I32, [_P, _P, _I64, _I32, _F32, _P]),
    "drift_gated_f32": (_I32, [_P, _P, _P, _I64, _I32, _P, _P, _P, _P]),
    "drift_gated_bf16": (_I32, [_P, _P, _P, _I64, _I32, _P, _P, _P, _P]),
    "drift_rope_f32": (_I32, [_P, _P, _P, _I32, _I32, _I32, _I32, _F32, _I32, _I32, _I32, _I32, _I32, _I32, _P]),
    "drift_rope_bf16": (_I32, [_P, _P, _P, _I32, _I32, _I32, _I32, _F32, _I32, _I32, _I32, _I32, _I32, _I32, _P]),
    "drift_rope_table_f32": (_I32, [_P, _P, _P, _P, _I32, _I32, _I32, _I32, _I32, _I32, _P]),
    "drift_rope_table_bf16": (_I32, [_P, _P, _P, _P, _I32, _I32, _I32, _I32, _I32, _I32, _P]),
    "drift_rope_3d_f32": (_I32, [_P, _P, _I64, _I32, _I32, _I32, _I32, _I32, _I64, _F64, _P]),
    "drift_rope_3d_bf16": (_I32, [_P, _P, _I64, _I32, _I32, _I32, _I32, _I32, _I64, _F64, _P]),
    "drift_qk_norm_rope_f32": (_I32, [_P, _P, _P, _P, _P, _P, _P, _I32, _I32, _I32, _I32, _F32, _F32, _I32, _F32,
                                      _I32, _I32, _I32, _I32, _I32, _I32, _P]),
    "drift_qk_norm_rope_bf16": (_I32, [_P, _P, _P, _P, _P, _P, _P, _I32, _I32, _I32, _I32, _F32, _F32, _I32, _F32,
                                       _I32, _I32, _I32, _I32, _I32, _I32, _P]),
    "drift_cache_write_f32": (_I32, [_P, _P, _P, _P, _P, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _P, _P]),
    "drift_cache_write_bf16": (_I32, [_P, _P, _P, _P, _P, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _P, _P]),
    "drift_split_halves_f32": (_I32, [_P, _P, _P, _I64, _I32, _P]),
    "drift_split_halves_bf16": (_I32, [_P, _P, _P, _I64, _I32, _P]),
    "drift_attention_inputs_f32": (_I32, [_P, _P, _P, _P, _P, _F32, _F32, _P, _I32, _I32, _I32, _I32, _I32, _F32,
                                          _I32, _I32, _I32, _I32, _I32, _I32, _P, _P, _P, _P, _P, _I32, _I32, _I32,
                                          _I32, _P, _P]),
    "drift_attention_inputs_bf16": (_I32, [_P, _P, _P, _P, _P, _F32, _F32, _P, _I32, _I32, _I32, _I32, _I32, _F32,
                                           _I32, _I32, _I32, _I32, _I32, _I32, _P, _P, _P, _P, _P, _I32, _I32, _I32,
                                           _I32, _P, _P]),
    "drift_embedding_q8_0_f32": (_I32, [_P, _P, _P, _I64, _I64, _I32, _P, _P]),
    "drift_embedding_q8_0_bf16": (_I32, [_P, _P, _P, _I64, _I64, _I32, _P, _P]),
    "drift_embedding_f32": (_I32, [_P, _I32, _P, _P, _I64, _I64, _I32, _P, _P]),
    "drift_embedding_bf16": (_I32, [_P, _I32, _P, _P, _I64, _I64, _I32, _P, _P]),
    "drift_dequantize_bf16": (_I32, [_P, _I32, _P, _I64, _I32, _P]),
    "drift_dequantize_f16": (_I32, [_P, _I32, _P, _I64, _I32, _P]),
    "drift_rotated_embedding_f32": (_I32, [_P, _P, _I64, _P, _P, _I32, _P, _P, _I64, _I64, _I32, _P, _P]),
    "drift_rotated_embedding_bf16": (_I32, [_P, _P, _I64, _P, _P, _I32, _P, _P, _I64, _I64, _I32, _P, _P]),
    "drift_rotated_dequantize_bf16": (_I32, [_P, _P, _I64, _P, _P, _I32, _P, _I64, _I32, _P]),
    "drift_convert": (_I32, [_P, _P, _I64, _I32, _P]),
    "drift_read_sum_f32x4": (_I32, [_P, _I64, _P, _I32, _P]),
    "drift_stream_mix": (_I32, [_P, _I64, _P, _I64, _I32, _P]),
    "drift_row_probe": (_I32, [_P, _I64, _I32, _P, _I64, _P, _I32, _P]),
    "drift_wave_copy": (_I32, [_P, _I64, _P, _I64, _I32, _P]),
    "drift_block_copy": (_I32, [_P, _I64, _P, _I64, _I32, _I32, _P]),
    "drift_wave_row_probe": (_I32, [_P, _I64, _I32, _P, _I64, _P, _I32, _I32, _P]),
}

ABI_VERSION = 10


class NotBuilt(RuntimeError):
    pass


class HipError(RuntimeError):
    """A refused call or a failed launch: the HIP code and the library's reason."""

    def __init__(self, entry: str, code: int, reason: str):
        super().__init__(f"{entry}: HIP error {code}: {reason}")
        self.entry = entry
        self.code = code
        self.reason = reason


_lib = None


def header_entry_points() -> list[str]:
    """The entry points include/drift_kernels.h declares."""
    with open(HEADER) as f:
        text = f.read()
    return re.findall(r"^\s*(?:int|const char\*)\s+(drift_\w+)\s*\(", text, re.M)


def load() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIBRARY):
        raise NotBuilt(f"{LIBRARY} is not built: run `python -c 'import __graft_entry__ as g; g.build()'` "
                       f"or `make -C drift_amd/csrc`")
    lib = ctypes.CDLL(LIBRARY)
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    version = lib.drift_abi_version()
    if version != ABI_VERSION:
        raise NotBuilt(f"{LIBRARY} implements ABI {version}, this package expects {ABI_VERSION}: rebuild it")
    _lib = lib
    return lib


def call(name: str, *args) -> None:
    """Calls entry point `name`; raises HipError on a nonzero return."""
    lib = load()
    code = getattr(lib, name)(*args)
    if code != 0:
        reason = lib.drift_last_error().decode() or lib.drift_error_string(code).decode()
        raise HipError(name, code, reason)
