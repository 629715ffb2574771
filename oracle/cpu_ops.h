/*
 * Test infrastructure only: the CPU oracle the HIP kernels are checked
 * against. It restates the drift runner's reference backend (`CpuOps`, plain
 * Scala loops accumulating in double) in C, operation by operation, so that a
 * kernel's output can be compared with what the reference computes on the
 * same inputs. Nothing in the product links or calls it; only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.
 *
 * Conventions (as the reference's): activations are F32, computed per element
 * in double and rounded once to float when written (ops/CpuBase.scala:18-30);
 * sums over a row are sequential left folds in double
 * (`(0L until n).map(...).sum`). Every function cites the reference lines it
 * follows.
 */
#ifndef DRIFT_ORACLE_CPU_OPS_H
#define DRIFT_ORACLE_CPU_OPS_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- conversions: ops/CpuOps.scala:52-57, tensor/DType.scala:99-102,
 *      tensor/LittleEndian.scala:45-46 ---- */
uint16_t oracle_to_bf16(float value);
float oracle_from_bf16(uint16_t bits);
float oracle_f16_to_f32(uint16_t bits);
uint16_t oracle_f32_to_f16(float value);
void oracle_f32_to_bf16_n(const float* x, uint16_t* out, int64_t n);
void oracle_bf16_to_f32_n(const uint16_t* x, float* out, int64_t n);
void oracle_f32_to_f16_n(const float* x, uint16_t* out, int64_t n);
void oracle_f16_to_f32_n(const uint16_t* x, float* out, int64_t n);

/* ---- ops/CpuOps.scala:26-50 ---- */
double oracle_erf(double x);

/* ---- ops/CpuNormalisation.scala:11-41 (kinds: ops/Activation.scala:6-20) ---- */
double oracle_activate(int kind, double v);
void oracle_activation(int kind, float input_scale, const float* x, float* out, int64_t n);
void oracle_gated(int kind, const float* gate, const float* up, float* out, int64_t n);

/* ---- ops/CpuElementwise.scala:9-13 (add), ops/CpuNormalisation.scala:53-71
 *      (rmsNorm), ops/NormalisationOps.scala:42-45 (addRmsNorm) ----
 * With `y`, x += y first (written back), then the norm of x into out. Row r
 * uses weight row r % weight_rows. */
void oracle_rms_norm(float* x, const float* y, const float* weight, float* out, int64_t rows, int64_t cols,
                     float eps, float offset, int64_t weight_rows);

/* ---- ops/CpuNormalisation.scala:128-151; weight, bias nullable ---- */
void oracle_layer_norm(const float* x, const float* weight, const float* bias, float* out, int64_t rows,
                       int64_t cols, float eps);

/* ---- ops/CpuElementwise.scala:33-38 ---- */
void oracle_modulate(const float* x, const float* scale, const float* shift, float* out, int64_t rows,
                     int64_t cols);

/* ---- ops/CpuAttention.scala:89-146 (rope), ops/Rope.scala:7-46 ----
 * sections: 0 single, 1 contiguous mRoPE, 2 interleaved mRoPE, 3 axes;
 * s[4] the section sizes in pairs. Positions are [positions_per_token, tokens]. */
void oracle_rope(const float* x, const int32_t* positions, float* out, int tokens, int heads, int dim, int rotary,
                 float theta, int layout, int sections, const int32_t* s);
/* the inverse frequency of pair `pair`, as the CPU computes it (float) */
float oracle_rope_inverse_frequency(int pair, int rotary, float theta, int sections, const int32_t* s);

/* ---- ops/CpuAttention.scala:53-87 (ropeTable) ---- */
void oracle_rope_table(const float* x, const float* cosines, const float* sines, float* out, int tokens, int heads,
                       int dim, int pairs, int per_head, int halves);

/* ---- models/Wan.scala:35-41 (pairs per axis), :324-361 (angle tables) ----
 * cos/sin [frames*rows*cols, head_dim/2], theta as Wan's 10000.0. */
void oracle_wan_pairs(int head_dim, int32_t* pairs3);
void oracle_wan_angles(int frames, int rows, int cols, int head_dim, double theta, float* cosines, float* sines);

/* ---- ops/CpuLinear.scala:12-41, tensor/GgmlQuants.scala:104-118 ----
 * Q8_0 rows of `cols` values (cols/32 blocks of 34 bytes). Returns the index
 * of the first id outside [0, vocab) (the reference refuses it), or -1. */
int64_t oracle_embedding_q8_0(const uint8_t* table, int64_t vocab, int64_t cols, const int32_t* ids, int64_t count,
                              float* out);
/* ---- storage types by their GGUF type ids (tensor/DType.scala and the
 * quant objects): decoders restating each decodeBlock in float. ---- */
enum {
  ORACLE_F32 = 0,
  ORACLE_F16 = 1,
  ORACLE_Q4_0 = 2,
  ORACLE_Q4_1 = 3,
  ORACLE_Q5_0 = 6,
  ORACLE_Q5_1 = 7,
  ORACLE_Q8_0 = 8,
  ORACLE_Q4_K = 12,
  ORACLE_Q5_K = 13,
  ORACLE_Q6_K = 14,
  ORACLE_IQ4_NL = 20,
  ORACLE_IQ4_XS = 23,
  ORACLE_BF16 = 30,
  ORACLE_ROCMFP4 = 100,
  ORACLE_ROCMFP4_FAST = 101
};
/* Values and bytes of a block; -1 for an unknown format. */
int oracle_format_block(int format, int* block_values, int* block_bytes);
float oracle_rocmfp4_half_scale(int byte);
/* A row of `cols` values (whole blocks); -1 if not. */
int oracle_decode_row(int format, const uint8_t* row, int64_t cols, float* out);
/* ops/CpuLinear.scala:12-41: the first id outside [0, vocab), -1 if none,
 * -2 for a bad format or partial blocks. */
int64_t oracle_embedding(int format, const uint8_t* table, int64_t vocab, int64_t cols, const int32_t* ids,
                         int64_t count, float* out);
/* ---- F32 tables: ops/CpuLinear.scala:12-41 with DType.F32 ---- */
int64_t oracle_embedding_f32(const float* table, int64_t vocab, int64_t cols, const int32_t* ids, int64_t count,
                             float* out);

/* ---- gated residuals and per-row modulation: ops/CpuElementwise.scala:40-86 ----
 * In place on x [rows, cols] (gatedAdd, gatedAddChunk, rowGatedAdd) or into
 * out (modulateChunks); tables are [rows, chunks * cols]. gatedAdd's gate is
 * [ceil(rows / rows_per_sample), cols] (rows_per_sample = rows: the
 * reference's one vector). */
void oracle_gated_add(float* x, const float* y, const float* gate, int64_t rows, int64_t cols,
                      int64_t rows_per_sample);
void oracle_modulate_chunks(const float* x, const float* table, float* out, int64_t rows, int64_t channels,
                            int64_t chunks, int64_t shift, int64_t scale);
void oracle_gated_add_chunk(float* x, const float* y, const float* table, int64_t rows, int64_t channels,
                            int64_t chunks, int64_t gate);
void oracle_row_gated_add(float* x, const float* y, const float* gate, int64_t rows, int64_t cols);

/* ---- the int8 side output: kernels/quantize.h:10-25 (quantize_block),
 *      kernels/matvec.hip:392-397 (quantize_x) ----
 * Per block b of 32 consecutive values: xd[b] = max|x| / 127 (float
 * division), xq[32 b + i] = (int8) roundf(x / xd[b]) (0 where xd[b] is 0 or
 * the quotient is NaN), xs[b] = xd[b] * (float) sum of the block's codes. */
void oracle_quantize_x(const float* x, int8_t* xq, float* xd, float* xs, int64_t blocks);

/* ---- ConvRot's rotated linears: tensor/ConvRot.scala, ops/CpuBase.scala:40-81 ---- */
float oracle_f8e4m3(int code);
void oracle_convrot_rotate(float* values, int64_t length, int64_t group);
/* codebook NULL: int8 codes [rows, cols]; else 4-bit codes [rows, cols / 2]
 * with relative fp8 [rows, cols / group_size]. */
void oracle_convrot_levels(const uint8_t* codes, const float* scales, int64_t scale_count, const float* codebook,
                           const uint8_t* relative, int64_t group_size, int64_t cols, int64_t first, int64_t count,
                           float* out);
void oracle_convrot_rows(const uint8_t* codes, const float* scales, int64_t scale_count, const float* codebook,
                         const uint8_t* relative, int64_t group_size, int64_t cols, int64_t first, int64_t count,
                         float* out);
int64_t oracle_convrot_embedding(const uint8_t* codes, const float* scales, int64_t scale_count,
                                 const float* codebook, const uint8_t* relative, int64_t group_size, int64_t rows,
                                 int64_t cols, const int32_t* ids, int64_t count, float* out);

#ifdef __cplusplus
}
#endif
#endif
