"""The GGUF reader (drift_amd/gguf.py) against the reference reader's rules
(runner/src/drift/runner/formats/Gguf.scala): files written here with a
Q8_0 token_embd table and other tensors read back with their metadata,
reversed shapes and bytes, and each of the reference's refusals. The
reference's GGUF fixtures are Git LFS pointers, so the files are built by
this test (the writer follows the GGUF v3 layout the reader checks).
A GPU test gathers rows of the file's table and compares them with the
oracle's decoding of the same bytes."""

import struct

import numpy as np
import pytest
import torch

from drift_amd import gguf
from drift_amd import ops as d
from oracle import oracle as o
from tests.helpers import DEV, host_bits, step


def model_file(path, vocab=64, cols=256, rng=None, alignment=32):
    rng = rng or np.random.default_rng(0)
    tensors = {
        "token_embd.weight": ("Q8_0", (vocab, cols), o.quant_table("Q8_0", vocab, cols, rng)),
        "output_norm.weight": ("F32", (cols,), rng.standard_normal(cols).astype(np.float32)),
        "blk.0.ffn_down.weight": ("Q4_K", (8, cols), o.quant_table("Q4_K", 8, cols, rng)),
        "blk.0.attn_q.weight": ("IQ4_XS", (4, cols), o.quant_table("IQ4_XS", 4, cols, rng)),
    }
    metadata = {"general.architecture": "qwen3", "qwen3.embedding_length": cols, "qwen3.rope.freq_base": 1e6,
                "tokenizer.ggml.tokens": [f"t{i}" for i in range(vocab)], "general.flag": True}
    gguf.write(str(path), metadata, tensors, alignment=alignment)
    return tensors, metadata


def test_reads_back_what_it_was_given(tmp_path):
    tensors, metadata = model_file(tmp_path / "m.gguf")
    f = gguf.open_gguf(str(tmp_path / "m.gguf"))
    assert f.version == 3 and f.alignment == 32 and f.architecture == "qwen3"
    assert f.long("qwen3.embedding_length") == 256 and f.double("qwen3.rope.freq_base") == 1e6
    assert f.strings("tokenizer.ggml.tokens")[5] == "t5" and f.boolean("general.flag") is True
    for name, (type_name, shape, data) in tensors.items():
        t = f[name]
        assert t.dtype.name == type_name and t.shape == shape and t.fileOffset % 32 == 0
        assert np.array_equal(f.bytes(name), np.ascontiguousarray(data).view(np.uint8).reshape(-1))
    with pytest.raises(gguf.FormatError, match="has no general.name"):
        f.string("general.name")
    with pytest.raises(gguf.FormatError, match="is 'qwen3'"):
        f.long("general.architecture")
    f.close()


def test_a_larger_alignment_is_kept(tmp_path):
    model_file(tmp_path / "a.gguf", alignment=64)
    f = gguf.open_gguf(str(tmp_path / "a.gguf"))
    assert f.alignment == 64 and all(t.fileOffset % 64 == 0 for t in f.tensors.values())


def header(version=3, tensors=0, metadata=0):
    return b"GGUF" + struct.pack("<IQQ", version, tensors, metadata)


@pytest.mark.parametrize("blob,message", [
    (b"GGML" + bytes(20), "not a GGUF file"),
    (header(version=4), "GGUF version 4 is not supported"),
    (header(version=0x03000000), "big-endian GGUF is not supported"),
    (b"GGUF\x03\x00", "truncated at byte 0"),
    (header(tensors=1 << 40), "tensor count of 1099511627776 is not plausible"),
    (header(metadata=1) + struct.pack("<Q", 3) + b"key" + struct.pack("<I", 13), "unknown metadata value type 13"),
])
def test_refusals_of_the_header(blob, message):
    with pytest.raises(gguf.FormatError, match=message):
        gguf.read(blob, "x")


def one_tensor(type_id, dims, offset, data, alignment=32):
    head = header(tensors=1) + struct.pack("<Q", 1) + b"t" + struct.pack("<I", len(dims))
    head += b"".join(struct.pack("<Q", x) for x in dims) + struct.pack("<Iq", type_id, offset)
    head += b"\0" * ((-len(head)) % alignment)
    return head + data


def test_refusals_of_the_tensors():
    q8 = o.quant_table("Q8_0", 2, 64, np.random.default_rng(1)).tobytes()  # 136 bytes
    assert gguf.read(one_tensor(8, [64, 2], 0, q8), "x")["t"].shape == (2, 64)
    with pytest.raises(gguf.FormatError, match="rows of 48 are not whole Q8_0 blocks"):
        gguf.read(one_tensor(8, [48, 2], 0, q8), "x")
    with pytest.raises(gguf.FormatError, match="t is not aligned to 32"):
        gguf.read(one_tensor(8, [64, 2], 8, q8), "x")
    with pytest.raises(gguf.FormatError, match="t runs past the end of the file"):
        gguf.read(one_tensor(8, [64, 3], 0, q8), "x")
    # Q8_0 bytes read as Q4_0: 72 bytes against 136 of room
    with pytest.raises(gguf.FormatError, match=r"t is Q4_0 \[2, 64\], 72 bytes, but the file gives it 136"):
        gguf.read(one_tensor(2, [64, 2], 0, q8), "x")
    with pytest.raises(gguf.FormatError, match="has 9 dimensions"):
        gguf.read(header(tensors=1) + struct.pack("<Q", 1) + b"t" + struct.pack("<I", 9), "x")


def crafted_files():
    """Files whose tensor records point outside the data or overflow: a
    negative offset (over the header, down to -2^63), an aligned offset just
    below 2^63 (data start + offset would overflow an int64) and dimensions
    whose product passes 2^63, each with the message both readers give."""
    q8 = o.quant_table("Q8_0", 2, 64, np.random.default_rng(1)).tobytes()
    rocm = o.quant_table("Q4_0_ROCMFP4", 1, 64, np.random.default_rng(2)).tobytes()
    big = [64] + [1 << 10] * 6 + [1 << 4]  # 2^6 * 2^60 * 2^4 = 2^70 values, each dimension within the file's size
    return [
        (one_tensor(8, [64, 2], -6528, q8), "t starts at offset -6528, before the data section"),
        (one_tensor(100, [64, 1], -32, rocm), "t starts at offset -32, before the data section"),
        (one_tensor(8, [64, 2], -(1 << 63), q8), "t starts at offset -9223372036854775808, before the data section"),
        (one_tensor(8, [64, 2], ((1 << 63) - 1) // 32 * 32, q8), "t runs past the end of the file"),
        (one_tensor(8, [64, 2], ((1 << 63) - 1) // 32 * 32 - 32 * 1024, q8), "t runs past the end of the file"),
        (one_tensor(8, big, 0, q8 + bytes(1 << 16)), r"t of \[16, 1024, 1024, 1024, 1024, 1024, 1024, 64\] has "
                                                    r"more than 2\^63 elements"),
        # 2^61 F32 values fit an int64, their 2^63 bytes do not
        (one_tensor(0, [1 << 16, 1 << 16, 1 << 16, 1 << 13], 0, bytes(1 << 17)),
         r"2305843009213693952 F32 elements do not fit 2\^63 bytes"),
    ]


def test_refusals_of_crafted_offsets_and_sizes():
    for blob, message in crafted_files():
        with pytest.raises(gguf.FormatError, match=message):
            gguf.read(blob, "x")


def test_unsupported_types_fail_only_when_asked_for():
    f = gguf.read(one_tensor(9, [32, 1], 0, bytes(36)), "x")  # Q8_1
    assert "t" not in f.tensors and f.unsupported["t"] == "GGML type Q8_1 is not supported yet"
    with pytest.raises(KeyError, match="GGML type Q8_1 is not supported yet"):
        f["t"]


def test_rocmfp4_scale_bytes_must_be_finite():
    good = o.quant_table("Q4_0_ROCMFP4", 1, 64, np.random.default_rng(2))
    assert gguf.read(one_tensor(100, [64, 1], 0, good.tobytes()), "x")["t"].dtype.name == "Q4_0_ROCMFP4"
    bad = good.copy()
    bad[0, 18 + 17] = 0x7F
    with pytest.raises(gguf.FormatError, match="scale byte 0x7f at byte 35 is not a finite unsigned E4M3"):
        gguf.read(one_tensor(100, [64, 1], 0, bad.tobytes()), "x")
    # the first bad byte in file order names the error, whichever scale it is
    bad[0, 16] = 0x80
    with pytest.raises(gguf.FormatError, match="scale byte 0x80 at byte 16 "):
        gguf.read(one_tensor(100, [64, 1], 0, bad.tobytes()), "x")


@pytest.mark.gpu
def test_the_files_embedding_table_gathers_on_the_gpu(tmp_path):
    tensors, _ = model_file(tmp_path / "m.gguf", vocab=300, cols=512, rng=np.random.default_rng(9))
    f = gguf.open_gguf(str(tmp_path / "m.gguf"))
    step("GGUF token_embd.weight Q8_0 [300, 512] gathered to BF16")
    table = f.table("token_embd.weight", DEV)
    assert table.shape == (300, 512) and table.dtype.name == "Q8_0"
    ids = np.random.default_rng(10).integers(0, 300, 77).astype(np.int32)
    out = torch.empty((77, 512), dtype=torch.bfloat16, device=DEV)
    d.HipOps().embedding(table, torch.from_numpy(ids).to(DEV), out)
    want = o.embedding_q8_0_bf16(f.bytes("token_embd.weight").reshape(300, -1), 300, 512, ids)
    assert np.array_equal(host_bits(out), want)
    step("GGUF blk.0.ffn_down.weight Q4_K [8, 512] decoded to BF16")
    k = f.table("blk.0.ffn_down.weight", DEV)
    dense = torch.empty((8, 512), dtype=torch.bfloat16, device=DEV)
    d.HipOps().dequantize(k, dense)
    want_k = o.embedding_bf16("Q4_K", f.bytes("blk.0.ffn_down.weight").reshape(8, -1), 8, 512, np.arange(8))
    assert np.array_equal(host_bits(dense), want_k)
    f.close()
