package drift.runner.ops

import drift.runner.tensor.*

import java.lang.foreign.*

/** HipAttention's rotary positions, cache write and attention inputs as
  * libdrift_kernels downcalls (ops/HipAttention.scala:45-218), and two
  * fused launches the models' sequences can take instead: Wan's 3-D rope
  * with its angles made in the kernel, and the dense decoders' per-head norms
  * and ropes. `shortAttention`, `attention` and the rest stay as they are.
  */
private[ops] trait DriftAttention extends HipAttention with DriftBase {

  /** The four section sizes the rope entry points take. */
  private def sectionSizes(rope: Rope): (Int, Int, Int, Int) = rope.sections match {
    case RopeSections.Single => (0, 0, 0, 0)
    case RopeSections.Contiguous(t, h, w) => (t, h, w, 0)
    case RopeSections.Interleaved(t, h, w) => (t, h, w, 0)
    case RopeSections.Axes(pairs) =>
      val Seq(a, b, c, d) = pairs.padTo(4, 0)
      (a, b, c, d)
  }

  override def rope(x: Tensor, positions: Tensor, rope: Rope, out: Tensor): Unit = {
    val (tokens, heads, dimension) = Ops.checkRope(x, positions, rope, out)
    val (s0, s1, s2, s3) = sectionSizes(rope)
    downcall(entry("drift_rope", x))(
      (drift.rope(bf16(x)).invokeExact(pointer(x), pointer(positions), pointer(out), tokens, heads, dimension,
        rope.rotaryDimensions, rope.theta, rope.layout.code, rope.sections.code, s0, s1, s2, s3,
        DefaultStream): Int)
    )
  }

  override def ropeTable(x: Tensor, cosines: Tensor, sines: Tensor, out: Tensor, halves: Boolean): Unit = {
    val (tokens, heads, d, pairs, perHead) = Ops.checkRopeTable(x, cosines, sines, out)
    val perHeadCode: Int = if (perHead) 1 else 0
    val halvesCode: Int = if (halves) 1 else 0
    downcall(entry("drift_rope_table", x))(
      (drift.ropeTable(bf16(x)).invokeExact(pointer(x), pointer(cosines), pointer(sines), pointer(out), tokens, heads,
        d, pairs, perHeadCode, halvesCode, DefaultStream): Int)
    )
  }

  /** Wan's 3-D rope with the angles made in the kernel: what
    * models/Wan.scala:324-361 tabulates on the host and :442-443 applies by
    * `ropeTable`, for a `frames × rows × columns` grid; token i of x
    * `[tokens, heads, D]` is grid token (tokenOffset + i) mod the grid's
    * tokens. No table to build or upload.
    */
  def rope3d(x: Tensor, frames: Int, rows: Int, columns: Int, out: Tensor, tokenOffset: Long = 0L,
             theta: Double = 10000.0): Unit = {
    Ops.checkElementwise("rope3d", x, out)
    require(x.shape.rank == 3, s"rope3d takes [tokens, heads, D], not ${x.shape}")
    val Seq(tokens, heads, d) = x.shape.dimensions
    val (headCount, dimension) = (heads.toInt, d.toInt)
    downcall(entry("drift_rope_3d", x))(
      (drift.rope3d(bf16(x)).invokeExact(pointer(x), pointer(out), tokens, headCount, dimension, frames, rows, columns,
        tokenOffset, theta, DefaultStream): Int)
    )
  }

  /** Per-head RMS norms of queries `[t, heads, D]` and keys `[t, kvHeads, D]`
    * and then their rope, in one launch: what models/DenseDecoder.scala:834-855
    * runs as rmsNorm, rmsNorm, rope, rope. q and k are read, not written.
    */
  def queryKeyNormRope(q: Tensor, k: Tensor, norms: QueryKeyNorms, positions: Tensor, rotatedQueries: Tensor,
                       rotatedKeys: Tensor): Unit = {
    Ops.checkElementwise("queryKeyNormRope", q, rotatedQueries)
    Ops.checkElementwise("queryKeyNormRope", k, rotatedKeys)
    val (tokens, heads, d) = Ops.checkRope(q, positions, norms.rope, rotatedQueries)
    val (_, kvHeads, _) = Ops.checkRope(k, positions, norms.rope, rotatedKeys)
    checkHeadNorms("queryKeyNormRope", norms, d)
    val rope = norms.rope
    val (s0, s1, s2, s3) = sectionSizes(rope)
    downcall(entry("drift_qk_norm_rope", q))(
      (drift.qkNormRope(bf16(q)).invokeExact(pointer(q), pointer(k), pointer(rotatedQueries), pointer(rotatedKeys),
        pointer(norms.queryNorm), pointer(norms.keyNorm), pointer(positions), tokens, heads, kvHeads, d,
        norms.epsilon, norms.weightOffset, rope.rotaryDimensions, rope.theta, rope.layout.code, rope.sections.code,
        s0, s1, s2, s3, DefaultStream): Int)
    )
  }

  private def checkHeadNorms(operation: String, norms: QueryKeyNorms, d: Int): Unit =
    Seq("queryNorm" -> norms.queryNorm, "keyNorm" -> norms.keyNorm).foreach { (name, weight) =>
      Ops.requireF32(operation, weight)
      require(weight.shape == Shape.of(d), s"$operation: $name ${weight.shape} for heads of $d")
    }

  override def cacheWrite(k: Tensor, v: Tensor, cache: KvCache, pageTable: Tensor, start: Int): Unit = {
    val tokens = Ops.checkCacheWrite(k, v, cache, pageTable, start)
    val tablePages: Int = pageTable.shape.elementCount.toInt
    downcall(entry("drift_cache_write", k))(
      (drift.cacheWrite(bf16(k)).invokeExact(pointer(k), pointer(v), pointer(cache.keys), pointer(cache.values),
        pointer(pageTable), tablePages, cache.pages, tokens, cache.kvHeads, cache.headDimension, cache.pageSize, start,
        MemorySegment.NULL, DefaultStream): Int)
    )
  }

  /** `attention.hip`'s ATTENTION_INPUT_DIMENSION, the widest head the fused
    * launch takes (ops/HipAttention.scala:217-218).
    */
  private val FusedHeadDimension = 512

  override def attentionInputs(queryAndGate: Tensor, keys: Tensor, values: Tensor, norms: QueryKeyNorms,
                               positions: Tensor, cache: KvCache, pageTable: Tensor, start: Int, queries: Tensor,
                               gate: Tensor, rotatedKeys: Tensor, rotatedQueries: Tensor): Unit = {
    val Seq(_, _, d) = queries.shape.dimensions
    if (d > FusedHeadDimension)
      super.attentionInputs(queryAndGate, keys, values, norms, positions, cache, pageTable, start, queries, gate,
        rotatedKeys, rotatedQueries)
    else {
      Ops.checkSplitHalves(queryAndGate, queries, gate)
      Ops.checkRope(queries, positions, norms.rope, rotatedQueries)
      Ops.checkRope(keys, positions, norms.rope, rotatedKeys)
      Ops.checkCacheWrite(rotatedKeys, values, cache, pageTable, start)
      inputsOnce(queryAndGate, keys, values, norms, positions, cache, pageTable, start, pointer(gate), rotatedQueries)
    }
  }

  /** The dense decoders' attention inputs in one launch: per-head norms of
    * q and k, their rope, the queries into `rotatedQueries` and the keys,
    * with the values v, into the cache at `start`
    * (models/DenseDecoder.scala:834-863 runs rmsNorm, rmsNorm, rope, rope,
    * cacheWrite).
    */
  def queryKeyNormRopeCache(q: Tensor, k: Tensor, v: Tensor, norms: QueryKeyNorms, positions: Tensor,
                            cache: KvCache, pageTable: Tensor, start: Int, rotatedQueries: Tensor): Unit = {
    require(q.shape.rank == 3 && q.shape.last <= FusedHeadDimension, s"queryKeyNormRopeCache: queries ${q.shape}")
    Ops.checkRope(q, positions, norms.rope, rotatedQueries)
    Ops.checkRope(k, positions, norms.rope, k)
    Ops.checkCacheWrite(k, v, cache, pageTable, start)
    inputsOnce(q, k, v, norms, positions, cache, pageTable, start, MemorySegment.NULL, rotatedQueries)
  }

  /** The fused launch; `gateAddress` null writes no gate (the dense decoders'
    * queries have none).
    */
  private def inputsOnce(queryAndGate: Tensor, keys: Tensor, values: Tensor, norms: QueryKeyNorms,
                         positions: Tensor, cache: KvCache, pageTable: Tensor, start: Int,
                         gateAddress: MemorySegment, rotatedQueries: Tensor): Unit = {
    val Seq(t, h, dimension) = rotatedQueries.shape.dimensions
    val (tokens, heads, d) = (t.toInt, h.toInt, dimension.toInt)
    require(keys.shape == Shape.of(t, cache.kvHeads, dimension),
      s"attentionInputs: keys ${keys.shape} for $tokens tokens of heads of $d")
    checkHeadNorms("attentionInputs", norms, d)
    val rope = norms.rope
    val (s0, s1, s2, s3) = sectionSizes(rope)
    val tablePages: Int = pageTable.shape.elementCount.toInt
    downcall(entry("drift_attention_inputs", keys))(
      (drift.attentionInputs(bf16(keys)).invokeExact(pointer(queryAndGate), pointer(keys), pointer(values),
        pointer(norms.queryNorm), pointer(norms.keyNorm), norms.epsilon, norms.weightOffset, pointer(positions),
        tokens, heads, cache.kvHeads, d, rope.rotaryDimensions, rope.theta, rope.layout.code, rope.sections.code,
        s0, s1, s2, s3, pointer(rotatedQueries), gateAddress, pointer(cache.keys), pointer(cache.values), pointer(pageTable),
        tablePages, cache.pages, cache.pageSize, start, MemorySegment.NULL, DefaultStream): Int)
    )
  }
}
