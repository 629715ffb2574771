"""The oracle's front end refuses shapes its C loops would index past: a
rope table shorter than the tokens, positions for fewer tokens or axes, and
weights, scales or Q8_0 bytes of the wrong size."""

import numpy as np
import pytest

from oracle import oracle as o


def test_short_rope_table_is_refused():
    x = np.zeros((10, 2, 8), np.float32)
    cos = np.ones((9, 4), np.float32)
    with pytest.raises(ValueError, match="rope_table"):
        o.rope_table(x, cos, cos)
    assert o.rope_table(x, np.ones((10, 4), np.float32), np.zeros((10, 4), np.float32)).shape == x.shape


def test_rope_positions_cover_every_axis():
    x = np.zeros((5, 1, 8), np.float32)
    with pytest.raises(ValueError, match="positions"):
        o.rope(x, np.zeros(4, np.int32), 1e4, 8)
    with pytest.raises(ValueError, match="positions"):
        o.rope(x, np.zeros(5, np.int32), 1e4, 8, sections=o.CONTIGUOUS, sizes=(2, 1, 1))
    with pytest.raises(ValueError, match="axes"):
        o.rope(x, np.zeros(10, np.int32), 1e4, 8, sections=o.AXES, sizes=(1, 1))
    o.rope(x, np.zeros(15, np.int32), 1e4, 8, sections=o.CONTIGUOUS, sizes=(2, 1, 1))


def test_wrong_sized_operands_are_refused():
    x = np.zeros((4, 8), np.float32)
    with pytest.raises(ValueError, match="rms_norm"):
        o.rms_norm(x, np.ones(7, np.float32), 1e-6)
    with pytest.raises(ValueError, match="rms_norm"):
        o.rms_norm(x, np.ones(24, np.float32), 1e-6, weight_rows=3)
    with pytest.raises(ValueError, match="layer_norm"):
        o.layer_norm(x, np.ones(9, np.float32))
    with pytest.raises(ValueError, match="modulate"):
        o.modulate(x, np.ones(8, np.float32), np.ones(4, np.float32))
    with pytest.raises(ValueError, match="gated"):
        o.gated(0, x, x[:2])
    with pytest.raises(ValueError, match="embedding_q8_0"):
        o.embedding_q8_0(np.zeros(67, np.uint8), 2, 32, np.zeros(1, np.int32))
