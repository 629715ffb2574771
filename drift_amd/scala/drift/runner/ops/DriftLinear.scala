package drift.runner.ops

import drift.runner.tensor.*

import java.lang.foreign.*

/** HipLinear's table gathers as libdrift_kernels downcalls
  * (ops/HipLinear.scala:21-92), and the bodies of two of its private members,
  * which the trait's own code reaches:
  *   - `quantize` (ops/HipLinear.scala:366-386) becomes `quantizeX(x, m, k)`;
  *   - `halfGemm`'s dequantize launch (ops/HipLinear.scala:443-455) becomes
  *     `dequantizeWeight(weight, target, wide, n, k)`.
  * Those two are one-line edits inside HipLinear: a private member cannot be
  * overridden.
  */
private[ops] trait DriftLinear extends HipLinear with DriftBase {

  /** Rows `ids` of a table, decoded into out: Q8_0 by its own entry point,
    * every other storage type by its GGUF type id, a rotated linear by
    * ConvRot's. An id outside the table writes a zero row; the reference's
    * checks refuse such ids on the host before any launch.
    */
  override def embedding(table: Tensor, ids: Tensor, out: Tensor): Unit = {
    Ops.checkEmbedding(table, ids, out)
    require(integerX.contains(table.dtype), s"no kernels for ${table.dtype} tables yet")
    val count: Long = ids.shape.elementCount
    val vocab: Long = table.shape.dimensions.head
    val cols: Int = table.shape.last.toInt
    if (ConvRot.stored(table.dtype)) {
      val parts = partsOf(table)
      val (codebook, relative, groupSize) = levelsOf(parts)
      val scaleCount: Long = parts.scales.shape.elementCount
      downcall(entry("drift_rotated_embedding", out))(
        (drift.rotatedEmbedding(bf16(out)).invokeExact(pointer(table), pointer(parts.scales), scaleCount, codebook,
          relative, groupSize, pointer(ids), pointer(out), count, vocab, cols, MemorySegment.NULL,
          DefaultStream): Int)
      )
    } else {
      require(cols % 8 == 0 || table.dtype.blockElements == 1,
        s"embedding: rows of $cols values (the block decoders take multiples of 8)")
      if (table.dtype == GgmlQuants.Q8_0)
        downcall(entry("drift_embedding_q8_0", out))(
          (drift.embeddingQ8_0(bf16(out)).invokeExact(pointer(table), pointer(ids), pointer(out), count, vocab, cols,
            MemorySegment.NULL, DefaultStream): Int)
        )
      else {
        val format: Int = ggmlIdOf(table.dtype)
        downcall(entry("drift_embedding", out))(
          (drift.embedding(bf16(out)).invokeExact(pointer(table), format, pointer(ids), pointer(out), count, vocab,
            cols, MemorySegment.NULL, DefaultStream): Int)
        )
      }
    }
  }

  private def ggmlIdOf(dtype: DType): Int =
    dtype.ggmlId.getOrElse(throw new IllegalArgumentException(s"$dtype has no GGUF type id"))

  /** `m` rows of `x` (`k` wide) quantized per 32 values into scratch memory:
    * codes, then scales, then sums, as `quantize` lays them out; marks that
    * int8 products run, so the norms quantize as they write from now on.
    */
  protected def quantizeX(x: Tensor, m: Int, k: Int): (MemorySegment, MemorySegment, MemorySegment) = {
    quantizesX = true
    val values = m.toLong * k
    val blocks: Long = values / 32
    val codes = scratch(0, values + 8 * blocks)
    val (scales, sums) = (offset(codes, values), offset(codes, values + 4 * blocks))
    downcall(entry("drift_quantize_x", x))(
      (drift.quantizeX(bf16(x)).invokeExact(pointer(x), codes, scales, sums, blocks, DefaultStream): Int)
    )
    (codes, scales, sums)
  }

  /** `n` rows of `k` values of a stored weight decoded at `target`, to BF16
    * when `wide`, else F16: the GEMM path's weight.
    */
  protected def dequantizeWeight(weight: Tensor, target: MemorySegment, wide: Boolean, n: Int, k: Int): Unit = {
    val format: Int = ggmlIdOf(weight.dtype)
    val rows: Long = n.toLong
    if (wide)
      downcall("drift_dequantize_bf16")(
        (drift.dequantizeBf16.invokeExact(pointer(weight), format, target, rows, k, DefaultStream): Int)
      )
    else
      downcall("drift_dequantize_f16")(
        (drift.dequantizeF16.invokeExact(pointer(weight), format, target, rows, k, DefaultStream): Int)
      )
  }
}
