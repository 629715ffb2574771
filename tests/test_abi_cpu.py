"""The C ABI without a GPU: the library loads, exports every entry point the
header declares, and refuses bad geometry before it would launch anything
(each call here fails validation, so nothing reaches the device)."""

import ctypes

import pytest

from drift_amd import _lib


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def test_header_and_library_agree(lib):
    declared = _lib.header_entry_points()
    assert len(declared) == len(set(declared)) >= 20
    assert set(declared) == set(_lib.SIGNATURES), "the ctypes table and the header differ"
    for name in declared:
        assert hasattr(lib, name), f"{name} is not exported"


def test_version_and_error_text(lib):
    assert lib.drift_abi_version() == _lib.ABI_VERSION == 10
    assert lib.drift_error_string(0).decode().lower().startswith("no error")
    assert lib.drift_error_string(1)


NULL = None


def refused(lib, name, *args):
    code = getattr(lib, name)(*args)
    return code == 1 and lib.drift_last_error().decode()


def test_norms_refuse_bad_geometry(lib):
    p = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    no_q = (NULL, NULL, NULL)
    assert "rows of 0 values" in refused(lib, "drift_rms_norm_f32", p, NULL, p, p, 4, 0, 1e-6, 0.0, 1, *no_q, NULL)
    assert "-1 rows" in refused(lib, "drift_rms_norm_bf16", p, NULL, p, p, -1, 8, 1e-6, 0.0, 1, *no_q, NULL)
    assert "weight rows" in refused(lib, "drift_rms_norm_f32", p, NULL, p, p, 4, 8, 1e-6, 0.0, 0, *no_q, NULL)
    assert "null" in refused(lib, "drift_rms_norm_f32", NULL, NULL, p, p, 4, 8, 1e-6, 0.0, 1, *no_q, NULL)
    assert "rows per sample" in refused(lib, "drift_layer_norm_modulate_bf16", p, p, p, p, 4, 8, 0, 1e-6, NULL)
    assert "null scale or shift" in refused(lib, "drift_layer_norm_modulate_f32", p, NULL, p, p, 4, 8, 2, 1e-6, NULL)
    # empty input: success, nothing launched
    assert lib.drift_rms_norm_f32(NULL, NULL, NULL, NULL, 0, 8, 1e-6, 0.0, 1, *no_q, NULL) == 0
    assert lib.drift_layer_norm_f32(NULL, NULL, NULL, NULL, 0, 8, 1e-6, NULL) == 0


def test_elementwise_refuses_bad_arguments(lib):
    p = ctypes.c_void_p(16)
    assert "no activation 5" in refused(lib, "drift_activation_f32", p, p, 10, 5, 1.0, NULL)
    assert "no activation -1" in refused(lib, "drift_gated_bf16", p, p, p, 10, -1, NULL, NULL, NULL, NULL)
    assert "no conversion 7" in refused(lib, "drift_convert", p, ctypes.c_void_p(32), 10, 7, NULL)
    assert "no conversion 5" in refused(lib, "drift_convert", p, ctypes.c_void_p(32), 10, 5, NULL)
    assert "same buffer" in refused(lib, "drift_convert", p, p, 10, 0, NULL)
    assert lib.drift_activation_bf16(NULL, NULL, 0, 1, 1.0, NULL) == 0


def test_rope_refuses_what_checkRope_refuses(lib):
    p = ctypes.c_void_p(16)
    args = lambda rotary, sections, s: (p, p, p, 4, 2, 128, rotary, 1e4, 0, sections, *s, NULL)
    # ops/AttentionOps.scala:201-221: even rotary within the head, axes summing to it
    assert "rotary" in refused(lib, "drift_rope_f32", *args(127, 0, (0, 0, 0, 0)))
    assert "rotary" in refused(lib, "drift_rope_f32", *args(130, 0, (0, 0, 0, 0)))
    assert "axes" in refused(lib, "drift_rope_bf16", *args(128, 3, (16, 24, 23, 0)))
    assert "axes" in refused(lib, "drift_rope_bf16", *args(128, 3, (32, 0, 32, 0)))
    assert "no layout" in refused(lib, "drift_rope_f32", p, p, p, 4, 2, 128, 128, 1e4, 2, 0, 0, 0, 0, 0, NULL)
    assert "heads of 1024" in refused(lib, "drift_rope_f32", p, p, p, 4, 2, 1024, 128, 1e4, 0, 0, 0, 0, 0, 0, NULL)
    assert "pairs in heads" in refused(lib, "drift_rope_table_f32", p, p, p, p, 4, 2, 128, 65, 0, 0, NULL)
    assert "grid" in refused(lib, "drift_rope_3d_bf16", p, p, 10, 2, 128, 0, 3, 4, 0, 1e4, NULL)
    assert "too narrow" in refused(lib, "drift_rope_3d_f32", p, p, 10, 2, 4, 1, 1, 1, 0, 1e4, NULL)
    assert "key heads" in refused(lib, "drift_qk_norm_rope_bf16", p, p, p, p, p, p, p, 4, 2, -1, 128, 1e-6, 0.0,
                                  128, 1e6, 0, 0, 0, 0, 0, 0, NULL)


def test_embedding_refuses_partial_blocks(lib):
    p = ctypes.c_void_p(16)
    assert "whole Q8_0 blocks" in refused(lib, "drift_embedding_q8_0_bf16", p, p, p, 4, 10, 48, NULL, NULL)
    assert "not 16-byte aligned" in refused(lib, "drift_embedding_q8_0_f32", p, p, ctypes.c_void_p(18), 4, 10, 64,
                                            NULL, NULL)


def test_side_output_refuses_partial_blocks(lib):
    p = ctypes.c_void_p(16)
    q = (ctypes.c_void_p(64), ctypes.c_void_p(128), ctypes.c_void_p(256))
    assert "whole blocks of 32" in refused(lib, "drift_rms_norm_f32", p, NULL, p, p, 4, 48, 1e-6, 0.0, 1, *q, NULL)
    assert "whole blocks of 32" in refused(lib, "drift_gated_f32", p, p, p, 40, 0, *q, NULL)
    assert "xd or xs" in refused(lib, "drift_gated_bf16", p, p, p, 64, 0, q[0], NULL, q[2], NULL)
    assert "4-byte aligned" in refused(lib, "drift_rms_norm_bf16", p, NULL, p, p, 2, 64, 1e-6, 0.0, 1, q[0],
                                       ctypes.c_void_p(130), q[2], NULL)
    assert "null xq" in refused(lib, "drift_quantize_x_f32", p, NULL, q[1], q[2], 4, NULL)
    assert "-2 blocks" in refused(lib, "drift_quantize_x_bf16", p, q[0], q[1], q[2], -2, NULL)
    assert lib.drift_quantize_x_f32(NULL, NULL, NULL, NULL, 0, NULL) == 0


def test_gated_residuals_refuse_bad_geometry(lib):
    p = ctypes.c_void_p(16)
    assert "rows per sample" in refused(lib, "drift_gated_add_f32", p, p, p, 4, 8, 0, NULL)
    assert "rows of 0 values" in refused(lib, "drift_gated_add_bf16", p, p, p, 4, 0, 4, NULL)
    assert "chunk 6 of 6" in refused(lib, "drift_modulate_chunks_f32", p, p, p, 4, 8, 6, 0, 6, NULL)
    assert "chunk -1 of 6" in refused(lib, "drift_gated_add_chunk_bf16", p, p, p, 4, 8, 6, -1, NULL)
    assert "0 chunks per row" in refused(lib, "drift_modulate_chunks_bf16", p, p, p, 4, 8, 0, 0, 0, NULL)
    assert "-3 rows" in refused(lib, "drift_row_gated_add_f32", p, p, p, -3, 8, NULL)
    assert "null operand" in refused(lib, "drift_row_gated_add_bf16", p, NULL, p, 3, 8, NULL)
    assert lib.drift_gated_add_f32(NULL, NULL, NULL, 0, 8, 1, NULL) == 0


def test_attention_inputs_refuse_what_the_cache_checks_refuse(lib):
    p = ctypes.c_void_p(16)
    # cache_write(k, v, keys, values, table, table_pages, cache_pages, tokens, kv_heads, d, page_size, start, bad)
    cw = lambda *g: (p, p, p, p, p, *g, NULL, NULL)
    # KvCache: pages of a multiple of 16 tokens (ops/KvCache.scala:14-17)
    assert "multiple of 16" in refused(lib, "drift_cache_write_f32", *cw(4, 4, 3, 2, 128, 10, 0))
    # checkPageTable: the table covers start + tokens (ops/AttentionOps.scala:243-256)
    assert "page table of 1 pages for 20 positions" in refused(lib, "drift_cache_write_bf16", *cw(1, 4, 6, 2, 128, 16, 14))
    assert "start -1" in refused(lib, "drift_cache_write_f32", *cw(4, 4, 3, 2, 128, 16, -1))
    assert lib.drift_cache_write_f32(NULL, NULL, NULL, NULL, NULL, 4, 4, 0, 2, 128, 16, 0, NULL, NULL) == 0
    assert "rows of 2 x 0" in refused(lib, "drift_split_halves_f32", p, p, p, 4, 0, NULL)
    assert lib.drift_split_halves_bf16(NULL, NULL, NULL, 0, 8, NULL) == 0
    ai = lambda heads, kv, d, rotary, page_size, table_pages, start: (
        p, p, p, p, p, 1e-6, 0.0, p, 3, heads, kv, d, rotary, 1e7, 0, 0, 0, 0, 0, 0, p, p, p, p, p, table_pages, 4,
        page_size, start, NULL, NULL)
    assert "rotary" in refused(lib, "drift_attention_inputs_f32", *ai(16, 2, 256, 257, 16, 4, 14))
    assert "heads of 1024" in refused(lib, "drift_attention_inputs_bf16", *ai(16, 2, 1024, 64, 16, 4, 14))
    assert "multiple of 16" in refused(lib, "drift_attention_inputs_f32", *ai(16, 2, 256, 64, 8, 4, 14))
    assert "page table" in refused(lib, "drift_attention_inputs_f32", *ai(16, 2, 256, 64, 16, 1, 14))
    assert "key heads" in refused(lib, "drift_attention_inputs_bf16", *ai(16, -2, 256, 64, 16, 4, 14))


def test_rotated_tables_refuse_what_checkRotated_refuses(lib):
    p, out = ctypes.c_void_p(16), ctypes.c_void_p(256)
    book = ctypes.c_void_p(64)
    ids = ctypes.c_void_p(128)
    assert "rows of 200 columns" in refused(lib, "drift_rotated_dequantize_bf16", p, p, 4, NULL, NULL, 0, out, 4,
                                            200, NULL)
    assert "3 scales for 4 rows" in refused(lib, "drift_rotated_dequantize_bf16", p, p, 3, NULL, NULL, 0, out, 4,
                                            256, NULL)
    # one scale for all is int8's only: 4-bit weights take one a row
    assert "1 scales for 4 rows" in refused(lib, "drift_rotated_dequantize_bf16", p, p, 1, book, p, 32, out, 4,
                                            256, NULL)
    assert "256 columns in groups of 24" in refused(lib, "drift_rotated_dequantize_bf16", p, p, 4, book, p, 24, out,
                                                    4, 256, NULL)
    assert "null codes" in refused(lib, "drift_rotated_dequantize_bf16", p, p, 4, book, NULL, 32, out, 4, 256, NULL)
    assert "16-byte aligned" in refused(lib, "drift_rotated_embedding_bf16", p, p, 4, NULL, NULL, 0, ids,
                                        ctypes.c_void_p(8), 3, 4, 256, NULL, NULL)
    assert "empty weight" in refused(lib, "drift_rotated_embedding_f32", p, p, 0, NULL, NULL, 0, ids, out, 3, 0,
                                     256, NULL, NULL)
    assert "null ids" in refused(lib, "drift_rotated_embedding_f32", p, p, 4, NULL, NULL, 0, NULL, out, 3, 4, 256,
                                 NULL, NULL)
    assert lib.drift_rotated_embedding_bf16(NULL, NULL, 4, NULL, NULL, 0, NULL, NULL, 0, 4, 256, NULL, NULL) == 0


def test_probes_refuse_bad_geometry(lib):
    p = ctypes.c_void_p(16)
    assert "0 blocks" in refused(lib, "drift_read_sum_f32x4", p, 100, p, 0, NULL)
    assert "not 16-byte aligned" in refused(lib, "drift_read_sum_f32x4", ctypes.c_void_p(8), 100, p, 4, NULL)
    assert "at least one written" in refused(lib, "drift_stream_mix", p, 10, p, 0, 1, NULL)
    assert "3 a lane" in refused(lib, "drift_stream_mix", p, 10, p, 10, 3, NULL)
    assert "null" in refused(lib, "drift_stream_mix", NULL, 10, p, 10, 1, NULL)
    assert "rows of 513 chunks (1 to 512)" in refused(lib, "drift_row_probe", p, 10, 513, p, 4, p, 8, NULL)
    assert "0 rows" in refused(lib, "drift_row_probe", p, 0, 16, p, 4, p, 8, NULL)
    assert "null" in refused(lib, "drift_row_probe", p, 10, 16, NULL, 4, p, 8, NULL)
    assert "not 16-byte aligned" in refused(lib, "drift_row_probe", p, 10, 16, p, 4, ctypes.c_void_p(8), 8, NULL)


def test_wave_probes_refuse_bad_geometry(lib):
    p = ctypes.c_void_p(16)
    assert "at least one written" in refused(lib, "drift_wave_copy", p, 10, p, 0, 1, NULL)
    assert "3 a lane" in refused(lib, "drift_wave_copy", p, 10, p, 10, 3, NULL)
    assert "16 a lane" in refused(lib, "drift_wave_copy", p, 10, p, 10, 16, NULL)
    assert "null" in refused(lib, "drift_wave_copy", NULL, 10, p, 10, 1, NULL)
    assert "not 16-byte aligned" in refused(lib, "drift_wave_copy", p, 10, ctypes.c_void_p(8), 10, 1, NULL)
    assert "3 waves a block" in refused(lib, "drift_block_copy", p, 10, p, 10, 1, 3, NULL)
    assert "32 waves a block" in refused(lib, "drift_block_copy", p, 10, p, 10, 1, 32, NULL)
    assert "0 waves a block" in refused(lib, "drift_block_copy", p, 10, p, 10, 1, 0, NULL)
    assert "at least one written" in refused(lib, "drift_block_copy", p, 10, p, 0, 1, 8, NULL)
    assert "at most 512 chunks" in refused(lib, "drift_wave_row_probe", p, 10, 1025, p, 4, p, 8, 2, NULL)
    assert "at most 512 chunks" in refused(lib, "drift_wave_row_probe", p, 10, 16, p, 4, p, 600, 1, NULL)
    assert "0 waves a row" in refused(lib, "drift_wave_row_probe", p, 10, 16, p, 4, p, 8, 0, NULL)
    assert "null" in refused(lib, "drift_wave_row_probe", p, 10, 16, NULL, 4, p, 8, 1, NULL)
    assert "not 16-byte aligned" in refused(lib, "drift_wave_row_probe", p, 10, 16, p, 4, ctypes.c_void_p(8), 8, 1,
                                            NULL)
    assert lib.drift_wave_row_probe(NULL, 10, 16, NULL, 0, NULL, 8, 1, NULL) == 0
