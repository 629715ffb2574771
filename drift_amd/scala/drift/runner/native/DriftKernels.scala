package drift.runner.native

import java.lang.foreign.*
import java.lang.foreign.ValueLayout.*
import java.lang.invoke.MethodHandle
import java.nio.file.Path

/** libdrift_kernels, the fused layer kernels for MI355X (gfx950), bound
  * through FFM as `HipRuntime` binds libamdhip64
  * (native/HipRuntime.scala:56-71): by hand, each binding repeating the C
  * signature of `include/drift_kernels.h`.
  *
  * Every kernel entry point takes device pointers, sizes and a `hipStream_t`
  * (`MemorySegment.NULL`, the default stream, which is where the runner
  * launches), checks its arguments on the host, launches, and returns 0 or a
  * HIP error code; `check` turns a nonzero code into a `HipException` with
  * the library's reason. The library neither allocates nor synchronizes.
  *
  * Most entry points have an F32 and a BF16 form with the same arguments
  * (`Twins`); the BF16 form takes `uint16_t*` tensors, which are addresses
  * here like any other.
  */
final class DriftKernels(path: Path) {

  import DriftKernels.*

  private val linker = Linker.nativeLinker()
  private val library = SymbolLookup.libraryLookup(path, Arena.global())

  private def find(name: String): MemorySegment =
    library
      .find(name)
      .orElseThrow(() => new IllegalStateException(s"$name is not in $path"))

  private def bind(name: String, arguments: MemoryLayout*): MethodHandle =
    linker.downcallHandle(find(name), FunctionDescriptor.of(JAVA_INT, arguments*))

  /** `<stem>_f32` and `<stem>_bf16`, which take the same arguments. */
  private def twins(stem: String, arguments: MemoryLayout*): Twins =
    Twins(bind(s"${stem}_f32", arguments*), bind(s"${stem}_bf16", arguments*))

  private val P = ADDRESS

  private val lastError =
    linker.downcallHandle(find("drift_last_error"), FunctionDescriptor.of(ADDRESS))
  private val abiVersion =
    linker.downcallHandle(find("drift_abi_version"), FunctionDescriptor.of(JAVA_INT))

  locally {
    val version = (abiVersion.invokeExact(): Int)
    require(version == AbiVersion, s"$path implements ABI $version, the runner binds ABI $AbiVersion")
  }

  // ------------------------------------------------------------ norms, activations
  val quantizeX = twins("drift_quantize_x", P, P, P, P, JAVA_LONG, P)
  val rmsNorm = twins("drift_rms_norm", P, P, P, P, JAVA_LONG, JAVA_INT, JAVA_FLOAT, JAVA_FLOAT, JAVA_INT, P, P, P, P)
  val layerNormF32 = bind("drift_layer_norm_f32", P, P, P, P, JAVA_LONG, JAVA_INT, JAVA_FLOAT, P)
  val modulateF32 = bind("drift_modulate_f32", P, P, P, P, JAVA_LONG, JAVA_INT, P)
  val layerNormModulate = twins("drift_layer_norm_modulate", P, P, P, P, JAVA_LONG, JAVA_INT, JAVA_LONG, JAVA_FLOAT, P)
  val activation = twins("drift_activation", P, P, JAVA_LONG, JAVA_INT, JAVA_FLOAT, P)
  val gated = twins("drift_gated", P, P, P, JAVA_LONG, JAVA_INT, P, P, P, P)

  // ------------------------------------------------------------ gated residuals
  val gatedAdd = twins("drift_gated_add", P, P, P, JAVA_LONG, JAVA_INT, JAVA_LONG, P)
  val modulateChunks = twins("drift_modulate_chunks", P, P, P, JAVA_LONG, JAVA_INT, JAVA_INT, JAVA_INT, JAVA_INT, P)
  val gatedAddChunk = twins("drift_gated_add_chunk", P, P, P, JAVA_LONG, JAVA_INT, JAVA_INT, JAVA_INT, P)
  val rowGatedAdd = twins("drift_row_gated_add", P, P, P, JAVA_LONG, JAVA_INT, P)

  // ------------------------------------------------------------ rotary positions
  val rope = twins("drift_rope", P, P, P, JAVA_INT, JAVA_INT, JAVA_INT, JAVA_INT, JAVA_FLOAT, JAVA_INT, JAVA_INT,
    JAVA_INT, JAVA_INT, JAVA_INT, JAVA_INT, P)
  val ropeTable = twins("drift_rope_table", P, P, P, P, JAVA_INT, JAVA_INT, JAVA_INT, JAVA_INT, JAVA_INT, JAVA_INT, P)
  val rope3d = twins("drift_rope_3d", P, P, JAVA_LONG, JAVA_INT, JAVA_INT, JAVA_INT, JAVA_INT, JAVA_INT, JAVA_LONG,
    JAVA_DOUBLE, P)
  val qkNormRope = twins("drift_qk_norm_rope", P, P, P, P, P, P, P, JAVA_INT, JAVA_INT, JAVA_INT, JAVA_INT, JAVA_FLOAT,
    JAVA_FLOAT, JAVA_INT, JAVA_FLOAT, JAVA_INT, JAVA_INT, JAVA_INT, JAVA_INT, JAVA_INT, JAVA_INT, P)

  // ------------------------------------------------------------ attention inputs
  val cacheWrite = twins("drift_cache_write", P, P, P, P, P, JAVA_INT, JAVA_INT, JAVA_INT, JAVA_INT, JAVA_INT, JAVA_INT,
    JAVA_INT, P, P)
  val splitHalves = twins("drift_split_halves", P, P, P, JAVA_LONG, JAVA_INT, P)
  val attentionInputs = twins("drift_attention_inputs", P, P, P, P, P, JAVA_FLOAT, JAVA_FLOAT, P, JAVA_INT, JAVA_INT,
    JAVA_INT, JAVA_INT, JAVA_INT, JAVA_FLOAT, JAVA_INT, JAVA_INT, JAVA_INT, JAVA_INT, JAVA_INT, JAVA_INT, P, P, P, P,
    P, JAVA_INT, JAVA_INT, JAVA_INT, JAVA_INT, P, P)

  // ------------------------------------------------------------ tables
  val embeddingQ8_0 = twins("drift_embedding_q8_0", P, P, P, JAVA_LONG, JAVA_LONG, JAVA_INT, P, P)
  // any storage type the runner reads, by its GGUF type id
  val embedding = twins("drift_embedding", P, JAVA_INT, P, P, JAVA_LONG, JAVA_LONG, JAVA_INT, P, P)
  val dequantizeBf16 = bind("drift_dequantize_bf16", P, JAVA_INT, P, JAVA_LONG, JAVA_INT, P)
  val dequantizeF16 = bind("drift_dequantize_f16", P, JAVA_INT, P, JAVA_LONG, JAVA_INT, P)
  // ConvRot's rotated linears: codes, scales, their count, codebook and
  // relative scales (NULL for int8 codes), group size, ...
  val rotatedEmbedding = twins("drift_rotated_embedding", P, P, JAVA_LONG, P, P, JAVA_INT, P, P, JAVA_LONG, JAVA_LONG,
    JAVA_INT, P, P)
  val rotatedDequantizeBf16 = bind("drift_rotated_dequantize_bf16", P, P, JAVA_LONG, P, P, JAVA_INT, P, JAVA_LONG,
    JAVA_INT, P)
  val convert = bind("drift_convert", P, P, JAVA_LONG, JAVA_INT, P)

  // ------------------------------------------------------------ bandwidth probes
  val readSumF32x4 = bind("drift_read_sum_f32x4", P, JAVA_LONG, P, JAVA_INT, P)
  val streamMix = bind("drift_stream_mix", P, JAVA_LONG, P, JAVA_LONG, JAVA_INT, P)
  val rowProbe = bind("drift_row_probe", P, JAVA_LONG, JAVA_INT, P, JAVA_LONG, P, JAVA_INT, P)
  val waveCopy = bind("drift_wave_copy", P, JAVA_LONG, P, JAVA_LONG, JAVA_INT, P)
  val blockCopy = bind("drift_block_copy", P, JAVA_LONG, P, JAVA_LONG, JAVA_INT, JAVA_INT, P)
  val waveRowProbe = bind("drift_wave_row_probe", P, JAVA_LONG, JAVA_INT, P, JAVA_LONG, P, JAVA_INT, JAVA_INT, P)

  /** A downcall's result: a nonzero code becomes a HipException carrying the
    * library's reason (as HipRuntime.check does, native/HipRuntime.scala:123-130).
    * `name` is by name: only a failure builds it.
    */
  def check(name: => String, code: Int): Unit =
    if (code != 0) {
      val text = (lastError.invokeExact(): MemorySegment)
      val reason =
        if (text == MemorySegment.NULL) "unknown"
        else text.reinterpret(Long.MaxValue).getString(0)
      throw new HipException(name, code, reason)
    }
}

object DriftKernels {

  /** `DRIFT_ABI_VERSION` of the header these bindings repeat. */
  val AbiVersion = 10

  /** Where the runner's build puts the library: the resource
    * `lib/libdrift_kernels.so` of the runner's jar (the `driftKernels` task
    * of drift_amd/scala/build.mill.drift, beside the `kernels` task's code
    * objects).
    */
  val Resource = "/lib/libdrift_kernels.so"

  /** The library the runner loads: the file `-Ddrift.kernels=<path>` names,
    * else the jar's resource, copied to a temporary file (a shared library
    * is mapped from a file, not from a jar entry) that is removed at exit.
    */
  def default(): DriftKernels =
    sys.props.get("drift.kernels").map(_.trim).filter(_.nonEmpty) match {
      case Some(path) => new DriftKernels(Path.of(path))
      case None =>
        val stream = Option(classOf[DriftKernels].getResourceAsStream(Resource)).getOrElse(
          throw new IllegalStateException(s"$Resource is not built: build the runner with the driftKernels task")
        )
        val file = java.nio.file.Files.createTempFile("libdrift_kernels", ".so")
        file.toFile.deleteOnExit()
        try java.nio.file.Files.copy(stream, file, java.nio.file.StandardCopyOption.REPLACE_EXISTING)
        finally stream.close()
        new DriftKernels(file)
    }

  /** An entry point's F32 and BF16 forms. The header's enumerations are the
    * runner's own codes: `Activation.code`, `RopeLayout.code`,
    * `RopeSections.code`, the conversion codes (ops/HipBase.scala:268-274)
    * and the GGUF type ids pass as they are.
    */
  final case class Twins(f32: MethodHandle, bf16: MethodHandle) {
    def apply(bf16Values: Boolean): MethodHandle = if (bf16Values) bf16 else f32
  }
}
