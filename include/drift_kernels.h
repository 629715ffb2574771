/*
 * libdrift_kernels: the drift runner's fused layer kernels for MI355X
 * (gfx950, CDNA4, wave64), behind a plain C ABI.
 *
 * Every entry point
 *   - takes device pointers and sizes, and the HIP stream to launch on
 *     (`stream` is a hipStream_t; NULL is the default stream);
 *   - validates its arguments on the host before launching and returns
 *     hipErrorInvalidValue (1) for bad geometry, with the reason in
 *     drift_last_error();
 *   - launches asynchronously: it never synchronizes and never allocates;
 *   - returns 0 (hipSuccess) or the HIP error of the launch. It never aborts.
 *
 * Element types: F32 is float; BF16 is uint16_t holding the top half of an
 * F32, rounded to nearest even from float results (NaN keeps its top half with
 * the quiet bit set), as the runner's CpuOps.toBfloat16
 * (runner/src/drift/runner/ops/CpuOps.scala:52-57). Norm, modulation and
 * rope vectors are F32; positions and ids are int32.
 *
 * Arithmetic follows the runner's CPU reference (`CpuOps`): statistics,
 * normalisation, modulation and rotations in double (full rate on CDNA4),
 * activations in float through forms that keep their relative accuracy.
 *
 * Aliasing: `out` may be the same buffer as `x` (or `gate`) for every entry
 * point, rope ones included (each lane reads a pair before it writes it).
 * Partially overlapping buffers are not supported.
 *
 * Each declaration names the reference interface it replaces (paths under
 * the reference's runner/).
 */
#ifndef DRIFT_KERNELS_H
#define DRIFT_KERNELS_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DRIFT_ABI_VERSION 10

/* Activation kinds: src/drift/runner/ops/Activation.scala:6-20. */
enum {
  DRIFT_SILU = 0,
  DRIFT_GELU_TANH = 1,
  DRIFT_GELU_ERF = 2,
  DRIFT_SIGMOID = 3,
  DRIFT_SITU = 4
};

/* RoPE layouts and sections: src/drift/runner/ops/Rope.scala:7-46. */
enum { DRIFT_ROPE_NEOX = 0, DRIFT_ROPE_INTERLEAVED = 1 };
enum {
  DRIFT_SECTIONS_SINGLE = 0,
  DRIFT_SECTIONS_CONTIGUOUS = 1,
  DRIFT_SECTIONS_INTERLEAVED = 2,
  DRIFT_SECTIONS_AXES = 3
};

/* Storage types of tables, by their GGUF type ids (the ggmlId of
 * src/drift/runner/tensor/DType.scala, GgmlQuants.scala, KQuants.scala,
 * IQuants.scala, RocmFp4.scala). */
enum {
  DRIFT_F32 = 0,
  DRIFT_F16 = 1,
  DRIFT_Q4_0 = 2,
  DRIFT_Q4_1 = 3,
  DRIFT_Q5_0 = 6,
  DRIFT_Q5_1 = 7,
  DRIFT_Q8_0 = 8,
  DRIFT_Q4_K = 12,
  DRIFT_Q5_K = 13,
  DRIFT_Q6_K = 14,
  DRIFT_IQ4_NL = 20,
  DRIFT_IQ4_XS = 23,
  DRIFT_BF16 = 30,
  DRIFT_Q4_0_ROCMFP4 = 100,
  DRIFT_Q4_0_ROCMFP4_FAST = 101
};

/* Conversions: the reference's codes, src/drift/runner/ops/HipBase.scala:
 * 268-274 (kernels/elementwise.hip:68-86), so a caller passes the kind it
 * passed before. */
enum {
  DRIFT_F32_TO_F16 = 0,
  DRIFT_F32_TO_BF16 = 1,
  DRIFT_F16_TO_F32 = 2,
  DRIFT_BF16_TO_F32 = 3,
  DRIFT_F8E4M3_TO_F32 = 4
};

/* The ABI version this library implements (DRIFT_ABI_VERSION). */
int drift_abi_version(void);
/* A HIP error code's text. */
const char* drift_error_string(int code);
/* Why the calling thread's last refused call was refused ("" if none). */
const char* drift_last_error(void);

/* ---------------------------------------------------------------- int8 side output
 * The runner's int8 products read their input x quantized per block of 32
 * consecutive values: codes xq[32 b + i] = round-half-away(x / xd[b]) (0 where
 * xd[b] is 0), xd[b] = max |x| / 127 over the block, xs[b] = xd[b] * the sum
 * of its codes (kernels/quantize.h:6-25). The norms and `gated` write it as
 * they write `out` when given a non-null xq (then xd and xs non-null and
 * 4-byte aligned, and the values whole blocks); for BF16 outputs it describes
 * the rounded values out holds. It equals drift_quantize_x over `out`, bit for
 * bit, as the reference's fused norms equal quantize_x
 * (gpuTest/.../FusedOpsTests.scala:96-176).
 *
 * drift_quantize_x: `blocks` blocks of x quantized on their own. Replaces
 * kernels/matvec.hip:392-397 quantize_x as launched by
 * src/drift/runner/ops/HipLinear.scala:366-386. */
int drift_quantize_x_f32(const float* x, int8_t* xq, float* xd, float* xs, int64_t blocks, void* stream);
int drift_quantize_x_bf16(const uint16_t* x, int8_t* xq, float* xd, float* xs, int64_t blocks, void* stream);

/* ---------------------------------------------------------------- RMSNorm
 * out = x / sqrt(mean(x^2) + eps) * (weight[r % weight_rows] + offset), per
 * row of `cols`. With `y` (nullable), x += y is written back first
 * (addRmsNorm). weight is F32 [weight_rows, cols]. With `xq` (nullable), the
 * int8 side output of out, above (cols a multiple of 32).
 * Replaces kernels/norm.hip:15-41 rms_norm_f32 as launched by
 * src/drift/runner/ops/HipNormalisation.scala:57-131 (rmsNorm, normRows,
 * addRmsNorm); the CPU definition is ops/CpuNormalisation.scala:53-71. */
int drift_rms_norm_f32(float* x, const float* y, const float* weight, float* out, int64_t rows, int32_t cols,
                       float eps, float offset, int32_t weight_rows, int8_t* xq, float* xd, float* xs,
                       void* stream);
/* BF16 x, y, out; F32 weight. The reference's bf16 path is
 * convert -> rms_norm_f32 -> convert (kernels/elementwise.hip:68-86). */
int drift_rms_norm_bf16(uint16_t* x, const uint16_t* y, const float* weight, uint16_t* out, int64_t rows,
                        int32_t cols, float eps, float offset, int32_t weight_rows, int8_t* xq, float* xd, float* xs,
                        void* stream);

/* ---------------------------------------------------------------- LayerNorm, AdaLN
 * out = (x - mean) / sqrt(var + eps) * weight + bias; weight, bias nullable.
 * Replaces kernels/norm.hip:63-80 layer_norm_f32
 * (ops/HipNormalisation.scala:217-238; CPU ops/CpuNormalisation.scala:128-151). */
int drift_layer_norm_f32(const float* x, const float* weight, const float* bias, float* out, int64_t rows,
                         int32_t cols, float eps, void* stream);

/* out = x * (1 + scale[c]) + shift[c]. Replaces kernels/elementwise.hip:97-103
 * modulate_f32 (ops/HipElementwise.scala:77-89; CPU ops/CpuElementwise.scala:33-38). */
int drift_modulate_f32(const float* x, const float* scale, const float* shift, float* out, int64_t rows,
                       int32_t cols, void* stream);

/* AdaLN in one pass: layerNorm without affine (its F32 result), then
 * modulate with sample s's rows of scale and shift ([samples, cols] F32),
 * sample s being rows [s * rows_per_sample, (s + 1) * rows_per_sample).
 * Replaces the pair layerNorm(x, None, None, eps) + modulate(...) that
 * src/drift/runner/models/Wan.scala:431-432,470-471,482-488 launch one sample
 * at a time. */
int drift_layer_norm_modulate_f32(const float* x, const float* scale, const float* shift, float* out,
                                  int64_t rows, int32_t cols, int64_t rows_per_sample, float eps, void* stream);
int drift_layer_norm_modulate_bf16(const uint16_t* x, const float* scale, const float* shift, uint16_t* out,
                                   int64_t rows, int32_t cols, int64_t rows_per_sample, float eps,
                                   void* stream);

/* ---------------------------------------------------------------- gated residuals
 * The steps either side of a diffusion block's modulated norms, in place on
 * x [rows, cols] (F32, or BF16 with F32 gates and tables); every value is
 * computed in double and rounded once, as the CPU reference does
 * (ops/CpuElementwise.scala:40-86).
 *
 * x[r][c] += gate[r / rows_per_sample][c] * y[r][c], gate F32
 * [ceil(rows / rows_per_sample), cols]; rows_per_sample = rows is the
 * reference's one gate vector. Replaces kernels/elementwise.hip:105-108
 * gated_add_f32 (ops/HipElementwise.scala:91-102). */
int drift_gated_add_f32(float* x, const float* y, const float* gate, int64_t rows, int32_t cols,
                        int64_t rows_per_sample, void* stream);
int drift_gated_add_bf16(uint16_t* x, const uint16_t* y, const float* gate, int64_t rows, int32_t cols,
                         int64_t rows_per_sample, void* stream);
/* out[r][c] = x[r][c] * (1 + table[r][scale][c]) + table[r][shift][c], table
 * F32 [rows, chunks * channels]; out may be x. Replaces
 * kernels/elementwise.hip:110-121 modulate_chunks_f32
 * (ops/HipElementwise.scala:104-126). */
int drift_modulate_chunks_f32(const float* x, const float* table, float* out, int64_t rows, int32_t channels,
                              int32_t chunks, int32_t shift, int32_t scale, void* stream);
int drift_modulate_chunks_bf16(const uint16_t* x, const float* table, uint16_t* out, int64_t rows, int32_t channels,
                               int32_t chunks, int32_t shift, int32_t scale, void* stream);
/* x[r][c] += table[r][gate][c] * y[r][c], the tables as modulate_chunks'.
 * Replaces kernels/elementwise.hip:123-130 gated_add_chunk_f32
 * (ops/HipElementwise.scala:128-143). */
int drift_gated_add_chunk_f32(float* x, const float* y, const float* table, int64_t rows, int32_t channels,
                              int32_t chunks, int32_t gate, void* stream);
int drift_gated_add_chunk_bf16(uint16_t* x, const uint16_t* y, const float* table, int64_t rows, int32_t channels,
                               int32_t chunks, int32_t gate, void* stream);
/* x[r][c] += gate[r] * y[r][c], gate F32 [rows]. Replaces
 * kernels/elementwise.hip:132-138 row_gated_add_f32
 * (ops/HipElementwise.scala:145-157). */
int drift_row_gated_add_f32(float* x, const float* y, const float* gate, int64_t rows, int32_t cols, void* stream);
int drift_row_gated_add_bf16(uint16_t* x, const uint16_t* y, const float* gate, int64_t rows, int32_t cols,
                             void* stream);

/* ---------------------------------------------------------------- activations
 * out = kind(scale * x), elementwise over n values. Replaces
 * kernels/elementwise.hip:31-53 activation_f32 (ops/HipNormalisation.scala:14-30;
 * CPU ops/CpuNormalisation.scala:11-35). */
int drift_activation_f32(const float* x, float* out, int64_t n, int32_t kind, float scale, void* stream);
int drift_activation_bf16(const uint16_t* x, uint16_t* out, int64_t n, int32_t kind, float scale, void* stream);

/* out = kind(gate) * up (SiTU soft-caps up as 25 tanh(up / 25)); with `xq`
 * (nullable), the int8 side output of out (n a multiple of 32). Replaces
 * kernels/elementwise.hip:46-65 gated_f32 (ops/HipNormalisation.scala:32-47;
 * CPU ops/CpuNormalisation.scala:22-41). */
int drift_gated_f32(const float* gate, const float* up, float* out, int64_t n, int32_t kind, int8_t* xq,
                    float* xd, float* xs, void* stream);
int drift_gated_bf16(const uint16_t* gate, const uint16_t* up, uint16_t* out, int64_t n, int32_t kind,
                     int8_t* xq, float* xd, float* xs, void* stream);

/* ---------------------------------------------------------------- RoPE
 * x, out [tokens, heads, head_dim]; positions int32 [positions_per_token,
 * tokens] (1 for SINGLE, 3 for mRoPE, the number of nonzero s for AXES).
 * Pair i turns by position * theta^(-2i/rotary) (AXES: pair j of an axis of
 * n pairs by theta^(-j/n)); the inverse frequency is the CPU's: pow in
 * double, rounded to float, then a float reciprocal; the angle is their
 * float product; the turn is in double. Values from `rotary` on are copied.
 * Replaces kernels/rope.hip:6-15 rope_f32 with kernels/rope.h:20-51
 * (ops/HipAttention.scala:74-104; CPU ops/CpuAttention.scala:89-146; checks
 * ops/AttentionOps.scala:185-223). */
int drift_rope_f32(const float* x, const int32_t* positions, float* out, int32_t tokens, int32_t heads,
                   int32_t head_dim, int32_t rotary, float theta, int32_t layout, int32_t sections, int32_t s0,
                   int32_t s1, int32_t s2, int32_t s3, void* stream);
int drift_rope_bf16(const uint16_t* x, const int32_t* positions, uint16_t* out, int32_t tokens, int32_t heads,
                    int32_t head_dim, int32_t rotary, float theta, int32_t layout, int32_t sections, int32_t s0,
                    int32_t s1, int32_t s2, int32_t s3, void* stream);

/* RoPE from F32 tables cosines, sines [tokens, pairs] (or [tokens, heads,
 * pairs] with per_head): adjacent pairs (2m, 2m+1), or with `halves` pairs
 * (m, m + pairs); values past 2 pairs copied. Replaces
 * kernels/rope.hip:17-55 rope_table_f32 / rope_table_halves_f32
 * (ops/HipAttention.scala:45-71; CPU ops/CpuAttention.scala:53-87). */
int drift_rope_table_f32(const float* x, const float* cosines, const float* sines, float* out, int32_t tokens,
                         int32_t heads, int32_t head_dim, int32_t pairs, int32_t per_head, int32_t halves,
                         void* stream);
int drift_rope_table_bf16(const uint16_t* x, const float* cosines, const float* sines, uint16_t* out,
                          int32_t tokens, int32_t heads, int32_t head_dim, int32_t pairs, int32_t per_head,
                          int32_t halves, void* stream);

/* Wan's 3-D RoPE with its angles made in the kernel: token i of x sits at
 * grid index g = (token_offset + i) mod (frames * grid_rows * grid_cols) of a
 * frames x grid_rows x grid_cols grid; its pairs split into frame, row and
 * column pairs (head_dim - 4 floor(head_dim/6), 2 floor(head_dim/6),
 * 2 floor(head_dim/6) values) turning by axis position /
 * theta^(2 index / (2 pairs_axis)), the angle in double, cos and sin rounded to
 * float as the host tables are; adjacent pairs. Replaces the host table build
 * of src/drift/runner/models/Wan.scala:324-361 plus the ropeTable launches at
 * :442-443. */
int drift_rope_3d_f32(const float* x, float* out, int64_t tokens, int32_t heads, int32_t head_dim, int32_t frames,
                      int32_t grid_rows, int32_t grid_cols, int64_t token_offset, double theta, void* stream);
int drift_rope_3d_bf16(const uint16_t* x, uint16_t* out, int64_t tokens, int32_t heads, int32_t head_dim,
                       int32_t frames, int32_t grid_rows, int32_t grid_cols, int64_t token_offset, double theta,
                       void* stream);

/* Per-head RMSNorm of queries and keys fused with their RoPE: q [tokens,
 * heads, head_dim], k [tokens, kv_heads, head_dim], each head row normed with
 * q_weight / k_weight ([head_dim] F32, + offset) as rmsNorm does, the F32
 * result then turned as rope does. Outputs q_out, k_out like q, k (they may
 * be q, k). Replaces the composition of ops/AttentionOps.scala:87-107 (rmsNorm
 * of each head in place, then rope of queries and keys) that
 * src/drift/runner/models/DenseDecoder.scala:834-855 runs as four launches, and
 * the norm+rope part of kernels/attention.hip:495-536 attention_inputs. */
int drift_qk_norm_rope_f32(const float* q, const float* k, float* q_out, float* k_out, const float* q_weight,
                           const float* k_weight, const int32_t* positions, int32_t tokens, int32_t heads,
                           int32_t kv_heads, int32_t head_dim, float eps, float offset, int32_t rotary, float theta,
                           int32_t layout, int32_t sections, int32_t s0, int32_t s1, int32_t s2, int32_t s3,
                           void* stream);
int drift_qk_norm_rope_bf16(const uint16_t* q, const uint16_t* k, uint16_t* q_out, uint16_t* k_out,
                            const float* q_weight, const float* k_weight, const int32_t* positions, int32_t tokens,
                            int32_t heads, int32_t kv_heads, int32_t head_dim, float eps, float offset,
                            int32_t rotary, float theta, int32_t layout, int32_t sections, int32_t s0, int32_t s1,
                            int32_t s2, int32_t s3, void* stream);

/* ---------------------------------------------------------------- attention inputs
 * The paged KV cache (src/drift/runner/ops/KvCache.scala:5-22): keys F16
 * (IEEE half bits in uint16_t) [cache_pages, page_size, kv_heads, head_dim],
 * values F16 [cache_pages, kv_heads, head_dim, page_size] (transposed within
 * a page); page_table (int32, table_pages entries) maps position / page_size
 * to a page, position start + t holding token t. page_size must be a
 * multiple of 16 (KvCache's rule) and table_pages * page_size >= start +
 * tokens (ops/AttentionOps.scala:243-256). A page-table entry outside
 * [0, cache_pages) writes nothing for its tokens and, when `bad_page`
 * (device int32, nullable) is given, sets *bad_page = 1; the CPU reference
 * fails on such an entry. F32 values are rounded to F16 to nearest even, as
 * Float.floatToFloat16 does (F16 NaN payloads are the hardware's). */

/* Keys and values [tokens, kv_heads, head_dim] into the cache at positions
 * start .. start + tokens - 1. Replaces kernels/attention.hip:480-493
 * cache_write (ops/HipAttention.scala cacheWrite; CPU
 * ops/CpuAttention.scala:181-210). */
int drift_cache_write_f32(const float* k, const float* v, uint16_t* keys, uint16_t* values,
                          const int32_t* page_table, int32_t table_pages, int32_t cache_pages, int32_t tokens,
                          int32_t kv_heads, int32_t head_dim, int32_t page_size, int32_t start, int32_t* bad_page,
                          void* stream);
int drift_cache_write_bf16(const uint16_t* k, const uint16_t* v, uint16_t* keys, uint16_t* values,
                           const int32_t* page_table, int32_t table_pages, int32_t cache_pages, int32_t tokens,
                           int32_t kv_heads, int32_t head_dim, int32_t page_size, int32_t start, int32_t* bad_page,
                           void* stream);

/* The halves of each row: x [rows, 2 d] into first and second [rows, d].
 * Replaces kernels/linear_attention.hip:298-307 split_halves (CPU
 * ops/CpuLayout.scala:137-143). */
int drift_split_halves_f32(const float* x, float* first, float* second, int64_t rows, int32_t d, void* stream);
int drift_split_halves_bf16(const uint16_t* x, uint16_t* first, uint16_t* second, int64_t rows, int32_t d,
                            void* stream);

/* A gated attention's inputs in one launch: each query head's row of
 * query_and_gate [tokens, heads, 2 head_dim] is its query then its output
 * gate (copied to gate [tokens, heads, head_dim]); the query is RMS-normed
 * with q_norm (+ offset), as rmsNorm writes it in F32, and turned by the rope
 * into queries [tokens, heads, head_dim]; each key head of k [tokens,
 * kv_heads, head_dim] is normed with k_norm and turned, and written with its
 * values v to the cache as cache_write does. With gate NULL, query_and_gate
 * holds plain queries [tokens, heads, head_dim] (the dense decoders'
 * norm + rope + cache write). Outputs may not alias inputs. Replaces
 * kernels/attention.hip:495-536 attention_inputs (ops/HipAttention.scala:
 * 144-215), the composition of ops/AttentionOps.scala:73-107 (splitHalves,
 * rmsNorm, rmsNorm, rope, rope, cacheWrite). */
int drift_attention_inputs_f32(const float* query_and_gate, const float* k, const float* v, const float* q_norm,
                               const float* k_norm, float eps, float offset, const int32_t* positions,
                               int32_t tokens, int32_t heads, int32_t kv_heads, int32_t head_dim, int32_t rotary,
                               float theta, int32_t layout, int32_t sections, int32_t s0, int32_t s1, int32_t s2,
                               int32_t s3, float* queries, float* gate, uint16_t* keys, uint16_t* values,
                               const int32_t* page_table, int32_t table_pages, int32_t cache_pages, int32_t page_size,
                               int32_t start, int32_t* bad_page, void* stream);
int drift_attention_inputs_bf16(const uint16_t* query_and_gate, const uint16_t* k, const uint16_t* v,
                                const float* q_norm, const float* k_norm, float eps, float offset,
                                const int32_t* positions, int32_t tokens, int32_t heads, int32_t kv_heads,
                                int32_t head_dim, int32_t rotary, float theta, int32_t layout, int32_t sections,
                                int32_t s0, int32_t s1, int32_t s2, int32_t s3, uint16_t* queries, uint16_t* gate,
                                uint16_t* keys, uint16_t* values, const int32_t* page_table, int32_t table_pages,
                                int32_t cache_pages, int32_t page_size, int32_t start, int32_t* bad_page,
                                void* stream);

/* ---------------------------------------------------------------- embedding
 * Rows `ids` of a Q8_0 table ([vocab, cols], cols a multiple of 32: per 32
 * values a 34-byte block, fp16 scale d then 32 int8 codes), decoded as
 * float(code) * d (exact in F32), into out [count, cols]. An id outside
 * [0, vocab) gets a row of zeros and, when `bad_id` (device int32, nullable)
 * is given, sets *bad_id = 1; the CPU reference refuses such an id. The
 * table must be 2-byte aligned and `out` 16-byte aligned.
 * Replaces kernels/matvec.hip:830-839,894-897 gather_q8_0
 * (ops/HipLinear.scala:21-52; CPU ops/CpuLinear.scala:12-41 with
 * tensor/GgmlQuants.scala:104-118). BF16 output is bit-exact against
 * convert(embedding F32). */
int drift_embedding_q8_0_f32(const uint8_t* table, const int32_t* ids, float* out, int64_t count, int64_t vocab,
                             int32_t cols, int32_t* bad_id, void* stream);
int drift_embedding_q8_0_bf16(const uint8_t* table, const int32_t* ids, uint16_t* out, int64_t count,
                              int64_t vocab, int32_t cols, int32_t* bad_id, void* stream);

/* Rows `ids` of a table of storage type `format` ([vocab, cols] values, each
 * row whole blocks: 32 values for the 32-value quants, 256 for the K-quants
 * and IQ4_XS, cols a multiple of 8; dense F32, F16, BF16 rows of any width),
 * decoded as the type's decoder in the reference does (bit-exact, BF16 the
 * F32 value rounded to nearest even), into out [count, cols]. The table must
 * be aligned to its blocks' fields (2 bytes for Q4_0, Q5_0, Q8_0, Q6_K,
 * IQ4_NL, ROCmFP4; 4 for Q4_1, Q5_1; 8 for Q4_K, Q5_K, IQ4_XS; 1 for ROCmFP4
 * fast) and out 16-byte aligned; dense tables need only their elements
 * aligned (16-byte aligned ones with rows of multiples of 8 take 16-byte
 * loads). Ids outside [0, vocab) as drift_embedding_q8_0 (which Q8_0
 * tables take). Replaces kernels/matvec.hip:830-839 gather<T> and its
 * gather_<q> instances (:891-897, :942-954) and elementwise.hip:89-93
 * gather_rows_f32 (ops/HipLinear.scala:21-52; CPU ops/CpuLinear.scala:12-41). */
int drift_embedding_f32(const void* table, int32_t format, const int32_t* ids, float* out, int64_t count,
                        int64_t vocab, int32_t cols, int32_t* bad_id, void* stream);
int drift_embedding_bf16(const void* table, int32_t format, const int32_t* ids, uint16_t* out, int64_t count,
                         int64_t vocab, int32_t cols, int32_t* bad_id, void* stream);

/* A whole table of storage type `format` ([rows, cols]) decoded into out
 * [rows, cols] as BF16 (nearest even) or F16 (IEEE half bits, nearest even),
 * for the GEMM path. Same layout rules as drift_embedding_f32. Replaces
 * kernels/matvec.hip:814-827 dequantize_bf16<T> and :801-812 dequantize<T>
 * (their dequantize_bf16_<q> and dequantize_<q> instances, :891-893). */
int drift_dequantize_bf16(const void* table, int32_t format, uint16_t* out, int64_t rows, int32_t cols,
                          void* stream);
int drift_dequantize_f16(const void* table, int32_t format, uint16_t* out, int64_t rows, int32_t cols,
                         void* stream);

/* ConvRot's rotated linears read where the file holds them (ComfyUI's
 * int8_tensorwise and asym_w4a8_int8 under convrot, ops/LinearOps.scala:
 * 21-33 `rotated`, tensor/ConvRot.scala): a weight [rows, cols] (cols a
 * multiple of 256) whose every 256 columns are the int8 levels times the
 * normalized regular Hadamard matrix.
 * - codebook NULL (int8_tensorwise): codes int8 [rows, cols]; scales F32,
 *   scale_count = rows (one a row) or 1 (one for all); relative and
 *   group_size unused.
 * - codebook F32 [16] (asym_w4a8_int8): codes [rows, cols / 2], two 4-bit
 *   codes a byte, the even column in the low nibble; a level is
 *   clamp(rint(codebook[code] * e4m3(relative)), -127, 127) (a NaN stays
 *   NaN, as the CPU's min and max keep it), relative fp8 E4M3 bytes [rows,
 *   cols / group_size] (group_size a positive multiple of 16 dividing cols);
 *   scales F32 [rows], scale_count = rows.
 * Values are the CPU's bit for bit (ops/CpuBase.scala:40-81): the level
 * times the row's scale in float, rotated in float in ConvRot.rotate's
 * order. Codes may lie at any alignment (16-byte aligned ones are read with
 * 16-byte loads); scales and codebook 4-byte aligned; out 16-byte aligned.
 *
 * drift_rotated_embedding_*: rows `ids` into out [count, cols] as the BF16
 * the weight holds (F32: those BF16 values widened, as
 * ops/CpuLinear.scala:24-29 gathers). An id outside [0, rows) gets zeros and
 * sets *bad_id = 1 when `bad_id` is given (the CPU refuses it). Replaces
 * kernels/convrot.hip:90-94,116-121 convrot_gather_f32_i8/_w4a8
 * (ops/HipLinear.scala:54-92).
 * drift_rotated_dequantize_bf16: the whole weight into out [rows, cols]
 * BF16 for the GEMM path. Replaces kernels/convrot.hip:84-88,109-114
 * convrot_dequantize_bf16_i8/_w4a8 (ops/HipBase.scala:276-311, the convert
 * of ops/HipMemory.scala:127-130). */
int drift_rotated_embedding_f32(const void* codes, const float* scales, int64_t scale_count, const float* codebook,
                                const uint8_t* relative, int32_t group_size, const int32_t* ids, float* out,
                                int64_t count, int64_t rows, int32_t cols, int32_t* bad_id, void* stream);
int drift_rotated_embedding_bf16(const void* codes, const float* scales, int64_t scale_count, const float* codebook,
                                 const uint8_t* relative, int32_t group_size, const int32_t* ids, uint16_t* out,
                                 int64_t count, int64_t rows, int32_t cols, int32_t* bad_id, void* stream);
int drift_rotated_dequantize_bf16(const void* codes, const float* scales, int64_t scale_count, const float* codebook,
                                  const uint8_t* relative, int32_t group_size, uint16_t* out, int64_t rows,
                                  int32_t cols, void* stream);

/* ---------------------------------------------------------------- convert
 * Elementwise type conversion of n values (kinds above: F32 to F16 and BF16
 * to nearest even, F16 and BF16 to F32 exactly, fp8 E4M3 "fn" bytes to F32
 * as tensor/DType.scala:105-115 decodes them). Replaces
 * kernels/elementwise.hip:68-86 convert (CPU ops/CpuMemory.scala:84-109). */
int drift_convert(const void* x, void* out, int64_t n, int32_t kind, void* stream);

/* ---------------------------------------------------------------- bandwidth probes
 * drift_read_sum_f32x4: a streaming read of n4 float4 values (16-byte
 * aligned x); block b writes the sum of the values it read to partials[b],
 * for `blocks` blocks of 256 threads (at most 2^20). Each lane reads four
 * float4 per pass over the grid, so blocks >= n4 / 1024 read everything in
 * one pass. Replaces kernels/bandwidth.hip:5-20 read_sum_f32x4
 * (runner/gpuTest/src/drift/runner/MemoryBandwidth.scala:37-52 launches it
 * with 2048 blocks).
 * drift_stream_mix: the read/write mix of a fused kernel, for its ceiling:
 * read_chunks 16-byte chunks of src read and write_chunks (at least 1) of
 * dst written, by 256-thread blocks that each read or write 256 x
 * per_thread (1, 2 or 4) consecutive chunks, read and write blocks
 * interleaved evenly in dispatch order; src and dst 16-byte aligned. dst
 * gets a pattern of the chunk index (and its chunk 0 the fold of what a
 * read block read, should that be all ones). No counterpart in the
 * reference: its probe reads only. */
int drift_read_sum_f32x4(const float* x, int64_t n4, float* partials, int32_t blocks, void* stream);
int drift_stream_mix(const void* src, int64_t read_chunks, void* dst, int64_t write_chunks, int32_t per_thread,
                     void* stream);
/* drift_row_probe: a gather's bytes in a gather's pattern, for its ceiling:
 * a 256-thread block per id reads the whole row ids[t] of a table of `rows`
 * rows of row_chunks (1 to 512) 16-byte chunks (ids clamped into the
 * table), and writes out_chunks chunks to row t of out, thread i's chunks
 * holding the XOR of the row chunks i and i + 256 it read (the first word
 * also XORed with the chunk index). table and out 16-byte aligned. No
 * counterpart in the reference. */
int drift_row_probe(const void* table, int64_t rows, int32_t row_chunks, const int32_t* ids, int64_t count, void* out,
                    int32_t out_chunks, void* stream);
/* drift_wave_copy: a fused kernel's read/write mix in its own shape, for its
 * ceiling: one-wave blocks, wave b reading chunks [b r, (b + 1) r) of src and
 * then writing chunks [b w, (b + 1) w) of dst (r and w the even shares of
 * read_chunks and write_chunks over max(read_chunks, write_chunks) / (64
 * per_lane) waves, rounded up; per_lane 1, 2, 4 or 8; at least one chunk
 * written). Each lane's written chunks hold the XOR of the chunks it read,
 * the first word also XORed with the chunk's place in the wave's share; src
 * and dst 16-byte aligned. No counterpart in the reference.
 * drift_block_copy: the same waves in blocks of waves_per_block waves (1, 2,
 * 4, 8 or 16; 1 is drift_wave_copy), wave w of block k being wave
 * k waves_per_block + w: the shape of the kernels that take several waves a
 * block. No counterpart in the reference.
 * drift_wave_row_probe: a gather's bytes in the gather's own shape: `slices`
 * one-wave blocks per id, wave s of id t reading chunks [s r, (s + 1) r) of
 * table row ids[t] (clamped into the table; r = row_chunks / slices rounded
 * up, at most 512) and writing chunks [s o, (s + 1) o) of out row t (o =
 * out_chunks / slices rounded up, at most 512), each lane's chunks holding
 * the XOR of what it read as in drift_wave_copy. No counterpart in the
 * reference. */
int drift_wave_copy(const void* src, int64_t read_chunks, void* dst, int64_t write_chunks, int32_t per_lane,
                    void* stream);
int drift_block_copy(const void* src, int64_t read_chunks, void* dst, int64_t write_chunks, int32_t per_lane,
                     int32_t waves_per_block, void* stream);
int drift_wave_row_probe(const void* table, int64_t rows, int32_t row_chunks, const int32_t* ids, int64_t count,
                         void* out, int32_t out_chunks, int32_t slices, void* stream);

#ifdef __cplusplus
}
#endif
#endif
