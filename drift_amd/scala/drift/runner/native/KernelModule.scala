package drift.runner.native

import java.lang.foreign.{Arena, MemorySegment}

/** A code object built from `runner/kernels/<name>.hip`, served as the
  * resource `kernels/<name>.hsaco`, the same class and members the runner's
  * backend uses (native/KernelModule.scala:8-33), with one change: the code
  * object is loaded the first time one of its functions is looked up, not
  * when the module is made.
  *
  * `HipBase` makes all ten modules when the backend is built
  * (ops/HipBase.scala:71-75,328-336). They are built for gfx1151 only
  * (build.mill:292-318), so on an MI355X (gfx950) an eager load fails in
  * `hipModuleLoadData` before any operation runs. With libdrift_kernels the
  * fused layer operations never look these modules up, so the backend builds
  * on gfx950 and runs them; an operation that does reach a module there
  * (the matrix-vector products, attention, convolutions) fails on its first
  * launch, naming the module and the device's missing code. Those kernels
  * must not be built for gfx950 as they are: several assume 32-lane waves
  * (kernels/matvec.hip:30-31, kernels/quantize.h:14,20) and attention uses
  * RDNA's wmma instructions (kernels/attention.hip:41-42).
  *
  * `close` unloads only a module that was loaded.
  */
final class KernelModule(hip: HipRuntime, val name: String) extends AutoCloseable {

  private val arena = Arena.ofShared()
  private var handle = Option.empty[MemorySegment]

  private def module: MemorySegment = synchronized {
    handle.getOrElse {
      val resource = s"/kernels/$name.hsaco"
      val bytes = Option(getClass.getResourceAsStream(resource)) match {
        case Some(stream) =>
          try stream.readAllBytes()
          finally stream.close()
        case None => throw new IllegalStateException(s"kernel module $resource is not built")
      }
      val image = arena.allocate(bytes.length.toLong, 64)
      MemorySegment.copy(MemorySegment.ofArray(bytes), 0, image, 0, bytes.length)
      val loaded =
        try hip.loadModule(image)
        catch {
          case e: HipException =>
            throw new IllegalStateException(
              s"kernel module $name has no code for this GPU (it is built for gfx1151; on MI355X only the " +
                "libdrift_kernels operations run)",
              e
            )
        }
      handle = Some(loaded)
      loaded
    }
  }

  def function(functionName: String): KernelFunction = hip.function(module, functionName)

  def close(): Unit = synchronized {
    handle.foreach(hip.unloadModule)
    handle = None
    arena.close()
  }
}
