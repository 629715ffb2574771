package drift.runner.ops

import drift.runner.tensor.*

import java.lang.foreign.*

/** HipElementwise's modulations and gated residuals as libdrift_kernels
  * downcalls (ops/HipElementwise.scala:77-157), and Wan's AdaLN in one
  * launch. `maxAbs`, `add`, `mul`, `scale` and `addRow` stay as they are.
  */
private[ops] trait DriftElementwise extends HipElementwise with DriftBase {

  override def modulate(x: Tensor, scale: Tensor, shift: Tensor, out: Tensor): Unit = {
    val rows = Ops.checkRowWise("modulate", x, out, scale, shift)
    val cols: Int = x.shape.last.toInt
    downcall("drift_modulate_f32")(
      (drift.modulateF32.invokeExact(pointer(x), pointer(scale), pointer(shift), pointer(out), rows, cols,
        DefaultStream): Int)
    )
  }

  /** One gate vector for every row: the whole tensor is one sample. */
  override def gatedAdd(x: Tensor, y: Tensor, gate: Tensor): Unit = {
    val rows = Ops.checkRowWise("gatedAdd", x, y, gate)
    val cols: Int = x.shape.last.toInt
    val rowsPerSample: Long = math.max(rows, 1L)
    downcall(entry("drift_gated_add", x))(
      (drift.gatedAdd(bf16(x)).invokeExact(pointer(x), pointer(y), pointer(gate), rows, cols, rowsPerSample,
        DefaultStream): Int)
    )
  }

  override def modulateChunks(x: Tensor, table: Tensor, shift: Int, scale: Int, out: Tensor): Unit = {
    val (rows, channels, chunks) = Ops.checkChunks("modulateChunks", x, table, out, shift, scale)
    downcall(entry("drift_modulate_chunks", x))(
      (drift.modulateChunks(bf16(x)).invokeExact(pointer(x), pointer(table), pointer(out), rows, channels, chunks,
        shift, scale, DefaultStream): Int)
    )
  }

  override def gatedAddChunk(x: Tensor, y: Tensor, table: Tensor, gate: Int): Unit = {
    val (rows, channels, chunks) = Ops.checkChunks("gatedAddChunk", x, table, y, gate)
    downcall(entry("drift_gated_add_chunk", x))(
      (drift.gatedAddChunk(bf16(x)).invokeExact(pointer(x), pointer(y), pointer(table), rows, channels, chunks, gate,
        DefaultStream): Int)
    )
  }

  override def rowGatedAdd(x: Tensor, y: Tensor, gate: Tensor): Unit = {
    val (rows, cols) = Ops.checkRowGatedAdd(x, y, gate)
    downcall(entry("drift_row_gated_add", x))(
      (drift.rowGatedAdd(bf16(x)).invokeExact(pointer(x), pointer(y), pointer(gate), rows, cols,
        DefaultStream): Int)
    )
  }

  /** Wan's AdaLN in one launch: `layerNorm(x, None, None, epsilon)` then
    * `modulate` by `scale` and `shift` (models/Wan.scala:431-432), x and out
    * `[rows, C]`. `scale` and `shift` are one `[C]` row for every row, or
    * `[samples, C]` with sample s's row for rows
    * `[s × rowsPerSample, (s + 1) × rowsPerSample)`, so a batch of samples
    * takes one launch.
    */
  def layerNormModulate(x: Tensor, scale: Tensor, shift: Tensor, epsilon: Float, out: Tensor,
                        rowsPerSample: Option[Long] = None): Unit = {
    Ops.checkElementwise("layerNormModulate", x, out)
    Ops.requireF32("layerNormModulate", scale, shift)
    require(x.shape.rank == 2, s"layerNormModulate takes [rows, C], not ${x.shape}")
    val Seq(rows, width) = x.shape.dimensions
    require(scale.shape == shift.shape && scale.shape.last == width && scale.shape.rank <= 2,
      s"layerNormModulate: scale ${scale.shape}, shift ${shift.shape} for rows of $width")
    val samples = scale.shape.elementCount / width
    val per: Long = rowsPerSample.getOrElse((rows + samples - 1) / samples)
    require(per > 0 && samples * per >= rows, s"layerNormModulate: $samples samples of $per rows for $rows rows")
    val cols: Int = width.toInt
    downcall(entry("drift_layer_norm_modulate", x))(
      (drift.layerNormModulate(bf16(x)).invokeExact(pointer(x), pointer(scale), pointer(shift), pointer(out), rows,
        cols, per, epsilon, DefaultStream): Int)
    )
  }
}
