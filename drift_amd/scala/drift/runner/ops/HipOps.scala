package drift.runner.ops

import drift.runner.native.{DriftKernels, HipRuntime}

/** The GPU backend with libdrift_kernels: the `Hip*` traits as they are,
  * then the `Drift*` traits, whose overrides replace those traits' launches
  * with downcalls (the linearization puts them last, so theirs are the
  * members that run). The one change to the runner's `HipOps`
  * (ops/HipOps.scala:8-20) is the `drift` library and the six traits.
  */
final class HipOps(
    protected val hip: HipRuntime,
    protected val inputs: MatVecInputs,
    protected val drift: DriftKernels
) extends HipBase
    with HipMemory
    with HipElementwise
    with HipNormalisation
    with HipLinear
    with HipExperts
    with HipAttention
    with HipConvolution
    with HipLayout
    with HipSequence
    with DriftBase
    with DriftNormalisation
    with DriftElementwise
    with DriftLinear
    with DriftAttention
    with DriftLayout
