"""The streaming probes the benchmark's ceilings come from: the reference's
read_sum_f32x4 (runner/kernels/bandwidth.hip:5-20) sums what it reads, and
stream_mix writes every chunk it is given, whatever the mix of read and
write blocks, checked here against numpy on small sizes."""

import ctypes

import numpy as np
import pytest
import torch

from drift_amd import _lib
from tests.helpers import DEV, step

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n4,blocks", [(1, 1), (1000, 3), (4096, 4), (1 << 20, 2048), (1 << 20, 1024)])
def test_read_sum_sums_what_it_reads(n4, blocks):
    step(f"read_sum_f32x4 over {n4} float4 values, {blocks} blocks")
    values = np.random.default_rng(n4).integers(-8, 9, 4 * n4).astype(np.float32)  # sums exact in float
    x = torch.from_numpy(values).to(DEV)
    partials = torch.full((blocks,), np.nan, dtype=torch.float32, device=DEV)
    _lib.call("drift_read_sum_f32x4", ctypes.c_void_p(x.data_ptr()), n4, ctypes.c_void_p(partials.data_ptr()),
              blocks, None)
    got = partials.cpu().numpy()
    assert np.all(np.isfinite(got)), "every block writes its partial"
    assert got.astype(np.float64).sum() == values.astype(np.float64).sum()


@pytest.mark.parametrize("reads,writes,per", [(1, 1, 1), (1000, 3000, 2), (35651, 67108, 4), (0, 513, 1),
                                              (2, 70000, 2), (90000, 5, 4)])
def test_stream_mix_reads_all_and_writes_all(reads, writes, per):
    # every written chunk holds its pattern (its index, its place in the
    # lane, 0x5eed); the reads, whose values are not all ones, leave chunk 0
    # alone
    step(f"stream_mix {reads} chunks read, {writes} written, {per} a lane")
    src = torch.full((max(reads, 1), 4), 7, dtype=torch.int32, device=DEV)
    dst = torch.zeros((writes, 4), dtype=torch.int32, device=DEV)
    _lib.call("drift_stream_mix", ctypes.c_void_p(src.data_ptr()), reads, ctypes.c_void_p(dst.data_ptr()), writes,
              per, None)
    got = dst.cpu().numpy().view(np.uint32)
    i = np.arange(writes, dtype=np.uint64)
    assert np.array_equal(got[:, 0], (i & 0xFFFFFFFF).astype(np.uint32))
    assert np.array_equal(got[:, 1], (i >> np.uint64(32)).astype(np.uint32))
    assert np.array_equal(got[:, 2], ((i // 256) % per).astype(np.uint32))
    assert np.all(got[:, 3] == 0x5EED)


@pytest.mark.parametrize("rows,row_chunks,count,out_chunks", [(5, 1, 3, 1), (40, 272, 17, 512), (9, 256, 8, 300),
                                                              (300, 512, 64, 1000), (3, 100, 1, 3)])
def test_row_probe_writes_what_each_row_holds(rows, row_chunks, count, out_chunks):
    # thread i of the block for id t XORs row chunks i and i + 256 (those in
    # the row) and stores that, its first word XORed with the chunk index,
    # into every chunk j = i (mod 256) of out row t; ids outside the table
    # are clamped into it
    step(f"row_probe {count} ids into {rows} rows of {row_chunks} chunks, {out_chunks} out")
    rng = np.random.default_rng(rows + row_chunks)
    table = rng.integers(0, 2**32, (rows, row_chunks, 4), dtype=np.uint64).astype(np.uint32)
    ids = rng.integers(-2, rows + 2, count).astype(np.int32)
    dt = torch.from_numpy(table.view(np.int32)).to(DEV)
    di = torch.from_numpy(ids).to(DEV)
    out = torch.zeros((count, out_chunks, 4), dtype=torch.int32, device=DEV)
    _lib.call("drift_row_probe", ctypes.c_void_p(dt.data_ptr()), rows, row_chunks, ctypes.c_void_p(di.data_ptr()),
              count, ctypes.c_void_p(out.data_ptr()), out_chunks, None)
    got = out.cpu().numpy().view(np.uint32)
    want = np.zeros((count, out_chunks, 4), dtype=np.uint32)
    for t, id_ in enumerate(np.clip(ids, 0, rows - 1)):
        folded = np.zeros((256, 4), dtype=np.uint32)
        for i in range(256):
            for k in (i, i + 256):
                if k < row_chunks:
                    folded[i] ^= table[id_, k]
        j = np.arange(out_chunks)
        want[t] = folded[j % 256]
        want[t, :, 0] ^= j.astype(np.uint32)
    assert np.array_equal(got, want)


def _fold_rows(chunks: np.ndarray, r0: int, r1: int) -> np.ndarray:
    """What wave_part leaves in each lane: the XOR of chunks r0 + lane + 64 k below r1."""
    folded = np.zeros((64, 4), dtype=np.uint32)
    for i in range(r0, r1):
        folded[(i - r0) % 64] ^= chunks[i]
    return folded


def _wave_out(folded: np.ndarray, w0: int, w1: int) -> np.ndarray:
    """Chunks [w0, w1) as a wave writes them: lane (j - w0) % 64's fold, word 0 XOR (j - w0)."""
    j = np.arange(w1 - w0)
    out = folded[j % 64].copy()
    out[:, 0] ^= j.astype(np.uint32)
    return out


@pytest.mark.parametrize("reads,writes,per,block", [(1, 1, 1, 1), (1000, 3000, 2, 1), (35651, 67108, 8, 1),
                                                    (0, 513, 1, 1), (2, 7000, 2, 1), (9000, 5, 4, 1), (4096, 4096, 4, 1),
                                                    (1000, 3000, 2, 8), (35651, 67108, 1, 16), (9000, 5, 4, 2),
                                                    (4096, 4096, 4, 4), (1, 1, 1, 8)])
def test_wave_copy_folds_each_waves_reads_into_its_writes(reads, writes, per, block):
    # wave b reads [b r, (b + 1) r) and writes [b w, (b + 1) w), r and w the
    # even shares over max(reads, writes) / (64 per) waves, rounded up, in
    # blocks of `block` waves (drift_block_copy; 1: drift_wave_copy)
    step(f"wave_copy {reads} chunks read, {writes} written, {per} a lane, {block} waves a block")
    rng = np.random.default_rng(reads + 7 * writes)
    chunks = rng.integers(0, 2**32, (max(reads, 1), 4), dtype=np.uint64).astype(np.uint32)
    src = torch.from_numpy(chunks.view(np.int32)).to(DEV)
    dst = torch.zeros((writes, 4), dtype=torch.int32, device=DEV)
    if block == 1:
        _lib.call("drift_wave_copy", ctypes.c_void_p(src.data_ptr()), reads, ctypes.c_void_p(dst.data_ptr()), writes,
                  per, None)
    else:
        _lib.call("drift_block_copy", ctypes.c_void_p(src.data_ptr()), reads, ctypes.c_void_p(dst.data_ptr()),
                  writes, per, block, None)
    got = dst.cpu().numpy().view(np.uint32)
    waves = max(-(-reads // (64 * per)), -(-writes // (64 * per)))
    r, w = -(-reads // waves), -(-writes // waves)
    want = np.zeros((writes, 4), dtype=np.uint32)
    for b in range(waves):
        w0, w1 = b * w, min(b * w + w, writes)
        if w0 < w1:
            want[w0:w1] = _wave_out(_fold_rows(chunks, b * r, min(b * r + r, reads)), w0, w1)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("rows,row_chunks,count,out_chunks,slices", [(5, 1, 3, 1, 1), (40, 272, 17, 512, 4),
                                                                     (9, 256, 8, 300, 2), (300, 512, 64, 1000, 2),
                                                                     (3, 100, 1, 3, 3), (50, 272, 33, 512, 1)])
def test_wave_row_probe_folds_each_slice(rows, row_chunks, count, out_chunks, slices):
    # wave s of id t folds row chunks [s r, (s + 1) r) of row ids[t] (clamped)
    # into output chunks [s o, (s + 1) o) of row t
    step(f"wave_row_probe {count} ids into {rows} rows of {row_chunks} chunks, {out_chunks} out, {slices} waves a row")
    rng = np.random.default_rng(rows + row_chunks + slices)
    table = rng.integers(0, 2**32, (rows, row_chunks, 4), dtype=np.uint64).astype(np.uint32)
    ids = rng.integers(-2, rows + 2, count).astype(np.int32)
    dt = torch.from_numpy(table.view(np.int32)).to(DEV)
    di = torch.from_numpy(ids).to(DEV)
    out = torch.zeros((count, out_chunks, 4), dtype=torch.int32, device=DEV)
    _lib.call("drift_wave_row_probe", ctypes.c_void_p(dt.data_ptr()), rows, row_chunks, ctypes.c_void_p(di.data_ptr()),
              count, ctypes.c_void_p(out.data_ptr()), out_chunks, slices, None)
    got = out.cpu().numpy().view(np.uint32)
    r, o = -(-row_chunks // slices), -(-out_chunks // slices)
    want = np.zeros((count, out_chunks, 4), dtype=np.uint32)
    for t, id_ in enumerate(np.clip(ids, 0, rows - 1)):
        for s in range(slices):
            w0, w1 = s * o, min(s * o + o, out_chunks)
            if w0 < w1:
                want[t, w0:w1] = _wave_out(_fold_rows(table[id_], s * r, min(s * r + r, row_chunks)), w0, w1)
    assert np.array_equal(got, want)
