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
