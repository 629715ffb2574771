"""HipOps' shape and dtype rules on the host: the reference's checks
(ops/Ops.scala:36-93, ops/AttentionOps.scala:129-223, ops/LinearOps.scala:92-106,
ops/MemoryOps.scala:68-84) refuse the same calls with the same messages,
before anything is launched. CPU tensors only: a call that passed the shape
rules would stop at "tensors live in device memory"."""

import pytest
import torch

from drift_amd import ops as d


@pytest.fixture(scope="module")
def hip():
    return d.HipOps()


def f32(*shape):
    return torch.zeros(shape, dtype=torch.float32)


def bf16(*shape):
    return torch.zeros(shape, dtype=torch.bfloat16)


def test_mismatched_shapes_are_refused(hip):
    # CpuOpsTests.scala:58-70
    with pytest.raises(ValueError, match="equal shapes"):
        hip.gated(d.Activation.Silu, f32(2), f32(3), f32(2))


def test_row_vectors_must_match_rows(hip):
    with pytest.raises(ValueError, match=r"rmsNorm: \[3\] for rows of 4"):
        hip.rmsNorm(f32(2, 4), f32(3), 1e-6, 0.0, f32(2, 4))
    with pytest.raises(ValueError, match="takes F32, not BF16"):
        hip.rmsNorm(f32(2, 4), bf16(4), 1e-6, 0.0, f32(2, 4))
    with pytest.raises(ValueError, match="one type"):
        hip.rmsNorm(bf16(2, 4), f32(4), 1e-6, 0.0, f32(2, 4))
    with pytest.raises(ValueError, match=r"modulate: \[5\] for rows of 4"):
        hip.modulate(f32(2, 4), f32(4), f32(5), f32(2, 4))
    # groupRmsNorm (ops/HipNormalisation.scala:141-142): weights span the row
    with pytest.raises(ValueError, match=r"groupRmsNorm: \[2\] for rows of 4"):
        hip.groupRmsNorm(f32(2, 4), f32(2), 2, 1e-6, 0.0, f32(2, 4))
    with pytest.raises(ValueError, match=r"^\[2×6\] in 4 groups$"):
        hip.groupRmsNorm(f32(2, 6), f32(6), 4, 1e-6, 0.0, f32(2, 6))


def test_rope_rules(hip):
    rope = d.Rope(1e4, 128, d.RopeLayout.Neox)
    with pytest.raises(ValueError, match="rope takes"):
        hip.rope(f32(4, 128), torch.zeros(4, dtype=torch.int32), rope, f32(4, 128))
    with pytest.raises(ValueError, match="positions are I32, not F32"):
        hip.rope(f32(4, 2, 128), f32(4), rope, f32(4, 2, 128))
    with pytest.raises(ValueError, match=r"positions \[4\], expected \[3×4\]"):
        mrope = d.Rope(1e6, 64, d.RopeLayout.Neox, d.RopeSections.Contiguous(11, 11, 10))
        hip.rope(f32(4, 2, 128), torch.zeros(4, dtype=torch.int32), mrope, f32(4, 2, 128))
    with pytest.raises(ValueError, match="axes of"):
        axes = d.Rope(1e3, 128, d.RopeLayout.Interleaved, d.RopeSections.Axes([16, 24, 23]))
        hip.rope(f32(4, 2, 128), torch.zeros(3, 4, dtype=torch.int32), axes, f32(4, 2, 128))
    with pytest.raises(ValueError, match="130 rotary dimensions in heads of 128"):
        hip.rope(f32(4, 2, 128), torch.zeros(4, dtype=torch.int32), d.Rope(1e4, 130), f32(4, 2, 128))


def test_rope_table_rules(hip):
    with pytest.raises(ValueError, match="ropeTable: tables"):
        hip.ropeTable(f32(4, 2, 128), f32(4, 65), f32(4, 65), f32(4, 2, 128))
    with pytest.raises(ValueError, match="ropeTable: tables"):
        hip.ropeTable(f32(4, 2, 128), f32(3, 64), f32(3, 64), f32(4, 2, 128))


def test_embedding_rules(hip):
    table = d.Q8_0Table(torch.zeros(10, 68, dtype=torch.uint8), 64)
    with pytest.raises(ValueError, match="ids are I32"):
        hip.embedding(table, torch.zeros(3, dtype=torch.int64), f32(3, 64))
    with pytest.raises(ValueError, match=r"out \[3×32\] for 3 rows of 64"):
        hip.embedding(table, torch.zeros(3, dtype=torch.int32), f32(3, 32))


def test_convert_rules(hip):
    with pytest.raises(ValueError, match="no conversion from BF16 to F16"):
        hip.convert(bf16(4), torch.zeros(4, dtype=torch.float16))


def test_host_tensors_are_refused_before_launch(hip):
    with pytest.raises(ValueError, match="device memory"):
        hip.rmsNorm(f32(2, 4), f32(4), 1e-6, 0.0, f32(2, 4))


def test_gated_residual_rules(hip):
    # ops/ElementwiseOps.scala:55-92, ops/Ops.scala:76-92
    with pytest.raises(ValueError, match=r"gatedAdd: \[3\] for rows of 4"):
        hip.gatedAdd(f32(2, 4), f32(2, 4), f32(3))
    with pytest.raises(ValueError, match="equal shapes"):
        hip.gatedAdd(f32(2, 4), f32(3, 4), f32(4))
    with pytest.raises(ValueError, match="rowsPerSample"):
        hip.gatedAdd(f32(4, 4), f32(4, 4), f32(2, 4))
    with pytest.raises(ValueError, match=r"gatedAdd: \[3×4\] for 2 samples"):
        hip.gatedAdd(f32(4, 4), f32(4, 4), f32(3, 4), rowsPerSample=2)
    with pytest.raises(ValueError, match=r"modulateChunks takes \[rows, C\], not \[2×2×4\]"):
        hip.modulateChunks(f32(2, 2, 4), f32(2, 24), 0, 1, f32(2, 2, 4))
    with pytest.raises(ValueError, match=r"modulateChunks: table \[2×10\] for \[2×4\], chunks ArraySeq\(0, 1\)"):
        hip.modulateChunks(f32(2, 4), f32(2, 10), 0, 1, f32(2, 4))
    with pytest.raises(ValueError, match=r"gatedAddChunk: table \[2×24\] for \[2×4\], chunks ArraySeq\(6\)"):
        hip.gatedAddChunk(f32(2, 4), f32(2, 4), f32(2, 24), 6)
    with pytest.raises(ValueError, match="takes F32, not BF16"):
        hip.gatedAddChunk(f32(2, 4), f32(2, 4), bf16(2, 24), 2)
    with pytest.raises(ValueError, match=r"rowGatedAdd takes \[rows, cols\], not \[8\]"):
        hip.rowGatedAdd(f32(8), f32(8), f32(1))
    with pytest.raises(ValueError, match=r"rowGatedAdd: gate \[3\] for \[2×4\]"):
        hip.rowGatedAdd(f32(2, 4), f32(2, 4), f32(3))
    # a call that passes the rules stops at the device check
    with pytest.raises(ValueError, match="device memory"):
        hip.gatedAddChunk(f32(2, 4), f32(2, 4), f32(2, 24), 5)


def f16(*shape):
    return torch.zeros(shape, dtype=torch.float16)


def i32(*shape):
    return torch.zeros(shape, dtype=torch.int32)


def test_the_cache_and_its_writes_are_checked(hip):
    # ops/KvCache.scala:12-20: pages of a multiple of 16 tokens, F16
    with pytest.raises(ValueError, match="pages of 10 tokens: not a multiple of 16"):
        d.KvCache(f16(4, 10, 2, 8), f16(4, 2, 8, 10), 10)
    with pytest.raises(ValueError, match="the cache is F16"):
        d.KvCache(f32(4, 16, 2, 8), f16(4, 2, 8, 16), 16)
    cache = d.KvCache(f16(4, 16, 2, 8), f16(4, 2, 8, 16), 16)
    # ops/AttentionOps.scala:225-256
    with pytest.raises(ValueError, match=r"cacheWrite: \[3×3×8\] into a cache of 2 heads of 8"):
        hip.cacheWrite(f32(3, 3, 8), f32(3, 3, 8), cache, i32(4), 0)
    with pytest.raises(ValueError, match="a page table of 1 pages for 19 positions"):
        hip.cacheWrite(f32(3, 2, 8), f32(3, 2, 8), cache, i32(1), 16)
    with pytest.raises(ValueError, match="a page table is I32"):
        hip.cacheWrite(f32(3, 2, 8), f32(3, 2, 8), cache, f32(4), 0)
    with pytest.raises(ValueError, match="equal shapes"):
        hip.cacheWrite(f32(3, 2, 8), f32(2, 2, 8), cache, i32(4), 0)
    with pytest.raises(ValueError, match="tensors live in device memory"):
        hip.cacheWrite(f32(3, 2, 8), f32(3, 2, 8), cache, i32(4), 0)


def test_split_halves_and_attention_inputs_are_checked(hip):
    with pytest.raises(ValueError, match=r"splitHalves: \[2×10\] into \[2×4\]"):
        hip.splitHalves(f32(2, 10), f32(2, 4), f32(2, 4))
    cache = d.KvCache(f16(4, 16, 2, 8), f16(4, 2, 8, 16), 16)
    norms = d.QueryKeyNorms(f32(8), f32(8), 1e-6, 0.0, d.Rope(1e4, 8))
    t, heads = 3, 4
    args = lambda qg, queries: (qg, f32(t, 2, 8), f32(t, 2, 8), norms, i32(t), cache, i32(4), 0, queries,
                                f32(t, heads, 8), f32(t, 2, 8), f32(t, heads, 8))
    with pytest.raises(ValueError, match="splitHalves"):
        hip.attentionInputs(*args(f32(t, heads, 8), f32(t, heads, 8)))
    with pytest.raises(ValueError, match="at most 512 fused"):
        hip.attentionInputs(*args(f32(t, heads, 1024), f32(t, heads, 1024)))
    with pytest.raises(ValueError, match="rope positions"):
        hip.attentionInputs(f32(t, heads, 16), f32(t, 2, 8), f32(t, 2, 8), norms, i32(t + 1), cache, i32(4), 0,
                            f32(t, heads, 8), f32(t, heads, 8), f32(t, 2, 8), f32(t, heads, 8))
    with pytest.raises(ValueError, match="tensors live in device memory"):
        hip.attentionInputs(*args(f32(t, heads, 16), f32(t, heads, 8)))


def test_rotated_weights_are_checked_as_checkRotated_does(hip):
    codes = torch.zeros((4, 256), dtype=torch.int8)
    scales = torch.ones(4)
    t = hip.rotated(codes, d.ConvRotParts(scales))
    assert t.shape == (4, 256) and t.dtype == "CONVROT_I8"
    assert hip.rotated(codes, d.ConvRotParts(torch.ones(1))).shape == (4, 256)
    with pytest.raises(ValueError, match=r"rotated: U8 codes \[4×256\]"):
        hip.rotated(codes.view(torch.uint8), d.ConvRotParts(scales))
    with pytest.raises(ValueError, match="rotated: rows of 200 columns"):
        hip.rotated(torch.zeros((4, 200), dtype=torch.int8), d.ConvRotParts(scales))
    with pytest.raises(ValueError, match="rotated: 3 F32 scales for 4 rows"):
        hip.rotated(codes, d.ConvRotParts(torch.ones(3)))
    levels = d.ConvRotLevels(torch.zeros(16), torch.zeros((4, 16), dtype=torch.uint8), 32)
    four = hip.rotated(torch.zeros((4, 256), dtype=torch.int8), d.ConvRotParts(scales, levels))
    assert four.shape == (4, 512) and four.dtype == "CONVROT_W4A8"
    with pytest.raises(ValueError, match="rotated: 1 F32 scales for 4 rows"):
        hip.rotated(torch.zeros((4, 256), dtype=torch.int8), d.ConvRotParts(torch.ones(1), levels))
    with pytest.raises(ValueError, match="rotated: 512 columns in groups of 24"):
        hip.rotated(torch.zeros((4, 256), dtype=torch.int8), d.ConvRotParts(scales, d.ConvRotLevels(
            torch.zeros(16), torch.zeros((4, 16), dtype=torch.uint8), 24)))
    with pytest.raises(ValueError, match=r"rotated: a codebook F32 \[8\]"):
        hip.rotated(torch.zeros((4, 256), dtype=torch.int8), d.ConvRotParts(scales, d.ConvRotLevels(
            torch.zeros(8), torch.zeros((4, 16), dtype=torch.uint8), 32)))
    with pytest.raises(ValueError, match=r"rotated: relative scales U8 \[4×8\]"):
        hip.rotated(torch.zeros((4, 256), dtype=torch.int8), d.ConvRotParts(scales, d.ConvRotLevels(
            torch.zeros(16), torch.zeros((4, 8), dtype=torch.uint8), 32)))
    with pytest.raises(ValueError, match="embedding: out \\[3×256\\] for 2 rows of 256"):
        hip.embedding(t, torch.zeros(2, dtype=torch.int32), torch.empty((3, 256)))
    with pytest.raises(ValueError, match="convert: no conversion from CONVROT_I8 to F32"):
        hip.convert(t, torch.empty((4, 256)))
