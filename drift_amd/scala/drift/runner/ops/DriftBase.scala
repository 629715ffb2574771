package drift.runner.ops

import drift.runner.native.*
import drift.runner.native.KernelArgument.*
import drift.runner.tensor.*

import java.lang.foreign.*

/** What the libdrift_kernels traits build on: the library, a downcall's
  * bookkeeping, and the two HipBase members that other traits reach through
  * it. Mixed into `HipOps` after the `Hip*` traits, so the `Drift*`
  * overrides are the members that run.
  *
  * A downcall counts as a launch counts (ops/HipBase.scala:216-227): one
  * device write, then `onWork`. The int8 side output's bookkeeping
  * (`quantizedTarget`, `wroteQuantized`, ops/HipBase.scala:156-193) is kept
  * as it is: its pointers go to the entry points' `xq`, `xd`, `xs`.
  *
  * `convertAt` and `dequantizeRotated` (ops/HipBase.scala:262-311) become
  * `drift_convert` and `drift_rotated_dequantize_bf16` here, so
  * `HipMemory.convert` and the GEMM path's conversions
  * (ops/HipLinear.scala:410-469) take them with no change of their own.
  */
private[ops] trait DriftBase extends HipBase {

  /** libdrift_kernels, loaded once per process. */
  protected def drift: DriftKernels

  /** The default stream, where the runner launches everything. */
  protected val DefaultStream: MemorySegment = MemorySegment.NULL

  /** One downcall: counted as a launch, then made, its code checked. With
    * `DRIFT_HIP_TRACE` set it is timed as `HipRuntime.launch` times a kernel
    * (native/HipRuntime.scala:318,358-362): from before the call until the
    * device has finished it, recorded under the entry point's name in the
    * per-kernel table printed at exit.
    */
  protected def downcall(name: => String)(call: => Int): Unit = {
    deviceWrites += 1
    onWork()
    if (HipRuntime.Trace.on) {
      val from = System.nanoTime()
      drift.check(name, call)
      hip.synchronize()
      HipRuntime.Trace.record(name, System.nanoTime() - from)
    } else drift.check(name, call)
  }

  /** Whether `tensor` takes an entry point's BF16 form. */
  protected def bf16(tensor: Tensor): Boolean = tensor.dtype == DType.BF16

  /** The name of the form of `stem` that `tensor` takes, for a failure's
    * message.
    */
  protected def entry(stem: String, tensor: Tensor): String =
    if (bf16(tensor)) s"${stem}_bf16" else s"${stem}_f32"

  protected def optional(tensor: Option[Tensor]): MemorySegment =
    tensor.fold(MemorySegment.NULL)(pointer)

  /** The addresses `quantizedTarget` hands out, as the entry points take
    * them: codes, scales, sums (all null when no int8 product reads `out`).
    */
  protected def sideOutput(arguments: Seq[KernelArgument]): (MemorySegment, MemorySegment, MemorySegment) =
    arguments match {
      case Seq(Pointer(xq), Pointer(xd), Pointer(xs)) => (xq, xd, xs)
      case other => throw new IllegalStateException(s"side output arguments $other")
    }

  /** A rotated weight's codebook, relative scales and group size; nulls and
    * 0 for int8 codes.
    */
  protected def levelsOf(parts: ConvRotParts): (MemorySegment, MemorySegment, Int) =
    parts.levels match {
      case Some(levels) => (pointer(levels.codebook), pointer(levels.relative), levels.groupSize)
      case None => (MemorySegment.NULL, MemorySegment.NULL, 0)
    }

  override protected def convertAt(from: MemorySegment, to: MemorySegment, count: Long, code: Int): Unit =
    downcall("drift_convert")((drift.convert.invokeExact(from, to, count, code, DefaultStream): Int))

  override protected def dequantizeRotated(weight: Tensor, to: MemorySegment): Unit = {
    val parts = partsOf(weight)
    val (codebook, relative, groupSize) = levelsOf(parts)
    val rows: Long = weight.shape.dimensions.head
    val cols: Int = weight.shape.last.toInt
    val scaleCount: Long = parts.scales.shape.elementCount
    downcall("drift_rotated_dequantize_bf16")(
      (drift.rotatedDequantizeBf16.invokeExact(pointer(weight), pointer(parts.scales), scaleCount, codebook, relative,
        groupSize, to, rows, cols, DefaultStream): Int)
    )
  }
}
