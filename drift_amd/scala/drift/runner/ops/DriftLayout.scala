package drift.runner.ops

import drift.runner.tensor.*

/** HipLayout's split of a gated attention's query rows into their halves as
  * a libdrift_kernels downcall (ops/HipLayout.scala:143-157). The rest of
  * the trait stays as it is.
  */
private[ops] trait DriftLayout extends HipLayout with DriftBase {

  override def splitHalves(x: Tensor, first: Tensor, second: Tensor): Unit = {
    Ops.checkSplitHalves(x, first, second)
    val d: Int = first.shape.last.toInt
    val rows: Long = first.shape.elementCount / d
    downcall(entry("drift_split_halves", x))(
      (drift.splitHalves(bf16(x)).invokeExact(pointer(x), pointer(first), pointer(second), rows, d,
        DefaultStream): Int)
    )
  }
}
