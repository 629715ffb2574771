"""The C++ host side (drift_amd/host, libdrift_ops.so) through its own test
program, tests/cpp/test_host.cpp: without a GPU, the shape and type refusals
with the reference's messages and a library refusal surfacing as a
HipException; on the GPU, operations launched through HipOps held to the
oracle's C functions."""

import os
import struct
import subprocess

import numpy as np
import pytest

from drift_amd import gguf
from oracle import oracle as o
from tests.test_gguf import crafted_files, header, model_file, one_tensor

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PROGRAM = os.path.join(ROOT, "tests", "cpp", "test_host")


def _sources():
    return [os.path.join(ROOT, "tests", "cpp", "test_host.cpp"), os.path.join(ROOT, "tests", "cpp", "comparison.hpp"),
            os.path.join(ROOT, "drift_amd", "host", "drift_ops.cpp"),
            os.path.join(ROOT, "drift_amd", "host", "drift_ops.hpp"),
            os.path.join(ROOT, "drift_amd", "host", "gguf.cpp"), os.path.join(ROOT, "drift_amd", "host", "gguf.hpp")]


def _program():
    """The built test program; made here (host code, seconds) when missing or
    older than its sources."""
    stale = not os.path.exists(PROGRAM) or any(
        os.path.getmtime(s) > os.path.getmtime(PROGRAM) for s in _sources())
    if stale:
        subprocess.run(["make", "-C", os.path.join(ROOT, "drift_amd", "host")], check=True)
        subprocess.run(["make", "-C", os.path.join(ROOT, "tests", "cpp")], check=True)
    return PROGRAM


def _run(mode):
    result = subprocess.run([_program(), mode], capture_output=True, text=True, timeout=120)
    print(result.stdout)
    assert result.returncode == 0, result.stdout + result.stderr
    assert " 0 failed" in result.stdout


def test_host_checks():
    _run("--checks")


@pytest.mark.gpu
def test_host_on_the_gpu():
    _run("--gpu")


def python_summary(path: str) -> list:
    """What tests/cpp/test_host.cpp --gguf prints, from the Python reader."""
    lines = [f"file {path}"]
    try:
        f = gguf.open_gguf(path)
    except gguf.FormatError as e:
        return lines + [f"refused {e}"]
    lines.append(f"version {f.version} alignment {f.alignment}")
    for name in sorted(f.tensors):
        t = f.tensors[name]
        lines.append(f"tensor {name} {t.dtype.name} [{','.join(map(str, t.shape))}] {t.fileOffset} {t.byteSize}")
    lines += [f"unsupported {name}: {f.unsupported[name]}" for name in sorted(f.unsupported)]
    f.close()
    return lines


def test_the_gguf_readers_agree(tmp_path):
    """The C++ reader (drift_amd/host/gguf.cpp) and the Python one read the
    same files to the same tensors, or refuse them with the same message."""
    files = []
    for alignment in (32, 64):
        model_file(tmp_path / f"model{alignment}.gguf", alignment=alignment)
        files.append(str(tmp_path / f"model{alignment}.gguf"))
    q8 = o.quant_table("Q8_0", 2, 64, np.random.default_rng(1)).tobytes()
    rocm = o.quant_table("Q4_0_ROCMFP4", 1, 64, np.random.default_rng(2))
    bad_rocm = rocm.copy()
    bad_rocm[0, 18 + 17] = 0x7F
    blobs = [b"", b"GGML" + bytes(20), header(version=4), header(version=0x03000000), b"GGUF\x03\x00",
             header(tensors=1 << 40),
             header(metadata=1) + struct.pack("<Q", 3) + b"key" + struct.pack("<I", 13),
             one_tensor(8, [64, 2], 0, q8), one_tensor(8, [48, 2], 0, q8), one_tensor(8, [64, 2], 8, q8),
             one_tensor(8, [64, 3], 0, q8), one_tensor(2, [64, 2], 0, q8),
             header(tensors=1) + struct.pack("<Q", 1) + b"t" + struct.pack("<I", 9),
             one_tensor(9, [32, 1], 0, bytes(36)), one_tensor(100, [64, 1], 0, rocm.tobytes()),
             one_tensor(100, [64, 1], 0, bad_rocm.tobytes())] + [blob for blob, _ in crafted_files()]
    for i, blob in enumerate(blobs):
        path = tmp_path / f"case{i}.gguf"
        path.write_bytes(blob)
        files.append(str(path))
    result = subprocess.run([_program(), "--gguf", *files], capture_output=True, text=True, timeout=120)
    assert result.returncode == 0, result.stderr
    want = [line for path in files for line in python_summary(path)]
    assert result.stdout.splitlines() == want
    assert sum(line.startswith("refused ") for line in want) == 20


def fnv1a(data: bytes) -> int:
    h = 1469598103934665603
    for b in data:
        h = ((h ^ b) * 1099511628211) & (2 ** 64 - 1)
    return h


@pytest.mark.gpu
def test_the_cpp_reader_s_table_gathers_on_the_gpu(tmp_path):
    path = str(tmp_path / "m.gguf")
    model_file(path, vocab=300, cols=512, rng=np.random.default_rng(9))
    ids = np.random.default_rng(10).integers(0, 300, 29).astype(np.int32)
    result = subprocess.run([_program(), "--gguf-embed", path, "token_embd.weight", *map(str, ids)],
                            capture_output=True, text=True, timeout=120)
    assert result.returncode == 0, result.stdout + result.stderr
    f = gguf.open_gguf(path)
    want = o.embedding_q8_0(f.bytes("token_embd.weight").reshape(300, -1), 300, 512, ids)
    f.close()
    assert result.stdout.strip() == f"embedding {fnv1a(np.ascontiguousarray(want, np.float32).tobytes())}"
