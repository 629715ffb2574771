package drift.runner.ops

import drift.runner.tensor.*

import java.lang.foreign.*

/** HipNormalisation's norms and activations as libdrift_kernels downcalls
  * (ops/HipNormalisation.scala:14-158, 217-238). The library picks its own
  * grid for every row width, so the narrow-row kernel and its branch go;
  * `softmax`, `groupNorm` and `gatedRmsNorm` stay as they are.
  */
private[ops] trait DriftNormalisation extends HipNormalisation with DriftBase {

  override def scaledActivation(kind: Activation, inputScale: Float, x: Tensor, out: Tensor): Unit = {
    Ops.checkElementwise("activation", x, out)
    val count: Long = out.shape.elementCount
    downcall(entry("drift_activation", x))(
      (drift.activation(bf16(x)).invokeExact(pointer(x), pointer(out), count, kind.code, inputScale,
        DefaultStream): Int)
    )
  }

  override def gated(kind: Activation, gate: Tensor, up: Tensor, out: Tensor): Unit = {
    Ops.checkElementwise("gated", gate, up, out)
    val (target, quantized) = quantizedTarget(out, out.shape.last)
    val (xq, xd, xs) = sideOutput(quantized)
    val count: Long = out.shape.elementCount
    downcall(entry("drift_gated", out))(
      (drift.gated(bf16(out)).invokeExact(pointer(gate), pointer(up), pointer(out), count, kind.code, xq, xd, xs,
        DefaultStream): Int)
    )
    wroteQuantized(target)
  }

  override def rmsNorm(x: Tensor, weight: Tensor, epsilon: Float, weightOffset: Float, out: Tensor): Unit = {
    val rows = Ops.checkRowWise("rmsNorm", x, out, weight)
    normRowsOnce(x, None, weight, epsilon, weightOffset, out, rows)
  }

  /** `x += y` first when `y` is given, then the RMS norm of every row into
    * out, in one launch; `out` also quantized when int8 products may read it
    * (rows of more than 32 values: the reference's narrow rows quantize
    * nothing).
    */
  private def normRowsOnce(x: Tensor, y: Option[Tensor], weight: Tensor, epsilon: Float, weightOffset: Float,
                           out: Tensor, rows: Long): Unit = {
    val cols: Int = x.shape.last.toInt
    val (target, (xq, xd, xs)) =
      if (cols > 32) {
        val (written, quantized) = quantizedTarget(out, cols)
        (written, sideOutput(quantized))
      } else (None, (MemorySegment.NULL, MemorySegment.NULL, MemorySegment.NULL))
    downcall(entry("drift_rms_norm", x))(
      (drift.rmsNorm(bf16(x)).invokeExact(pointer(x), optional(y), pointer(weight), pointer(out), rows, cols, epsilon,
        weightOffset, 1, xq, xd, xs, DefaultStream): Int)
    )
    wroteQuantized(target)
  }

  /** One launch for every width: the library adds y to x as it norms. */
  override def addRmsNorm(x: Tensor, y: Tensor, norm: RowNorm): Unit = {
    Ops.checkElementwise("addRmsNorm", x, y)
    val rows = Ops.checkRowWise("addRmsNorm", x, norm.out, norm.weight)
    normRowsOnce(x, Some(y), norm.weight, norm.epsilon, norm.weightOffset, norm.out, rows)
  }

  /** rms_norm over rows × groups rows of a group's width, row r weighted by
    * weight row r % groups, with no int8 side output
    * (ops/HipNormalisation.scala:133-158).
    */
  override def groupRmsNorm(x: Tensor, weight: Tensor, groups: Int, epsilon: Float, weightOffset: Float,
                            out: Tensor): Unit = {
    val rows = Ops.checkRowWise("groupRmsNorm", x, out, weight)
    require(x.shape.last % groups == 0, s"${x.shape} in $groups groups")
    val width: Int = (x.shape.last / groups).toInt
    val groupRows: Long = rows * groups
    downcall(entry("drift_rms_norm", x))(
      (drift.rmsNorm(bf16(x)).invokeExact(pointer(x), MemorySegment.NULL, pointer(weight), pointer(out), groupRows,
        width, epsilon, weightOffset, groups, MemorySegment.NULL, MemorySegment.NULL, MemorySegment.NULL,
        DefaultStream): Int)
    )
  }

  override def layerNorm(x: Tensor, weight: Option[Tensor], bias: Option[Tensor], epsilon: Float,
                         out: Tensor): Unit = {
    val rows = Ops.checkRowWise("layerNorm", x, out, (weight ++ bias).toSeq*)
    val cols: Int = x.shape.last.toInt
    downcall("drift_layer_norm_f32")(
      (drift.layerNormF32.invokeExact(pointer(x), optional(weight), optional(bias), pointer(out), rows, cols, epsilon,
        DefaultStream): Int)
    )
  }
}
