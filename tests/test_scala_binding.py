"""The Scala FFM binding (drift_amd/scala) against the C ABI, read as text:
no JDK is installed here, so these checks stand in for the compiler and the
first downcalls.

- every `bind("drift_…", …)` and `twins("drift_…", …)` layout list matches the
  entry point's argument types in drift_amd/_lib.py (which test_abi_cpu holds
  to the library), and every kernel entry point is bound;
- every `invokeExact` call is ascribed, `(h.invokeExact(…): Int)`, the form
  native/HipRuntime.scala:127,149-188 uses: without it Scala types the
  signature-polymorphic call as returning Object and the JVM throws
  WrongMethodTypeException on the first call; and no `.asInstanceOf` is left;
- every `invokeExact` on a binding passes as many arguments as its layout
  has, addresses where the layout has ADDRESS and values elsewhere, each
  value of the layout's type (read from its declaration, or the return type
  of the reference's check that made it), the stream last.
"""

import glob
import os
import re

import pytest

from drift_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SCALA = os.path.join(ROOT, "drift_amd", "scala")
BINDING = os.path.join(SCALA, "drift", "runner", "native", "DriftKernels.scala")

LAYOUTS = {"P": _lib._P, "ADDRESS": _lib._P, "JAVA_INT": _lib._I32, "JAVA_LONG": _lib._I64,
           "JAVA_FLOAT": _lib._F32, "JAVA_DOUBLE": _lib._F64}

# the entry points that are not kernels: bound on their own in DriftKernels
SERVICE = {"drift_abi_version", "drift_last_error", "drift_error_string"}

# arguments that are addresses: pointer(t), optional(t), nulls, the stream,
# and the MemorySegment locals the traits name
ADDRESS_ARGUMENT = re.compile(r"^(pointer\(|optional\(|MemorySegment\.NULL$|DefaultStream$|"
                              r"(xq|xd|xs|codebook|relative|gateAddress|to|from|target|codes|scales|sums)$)")


def sources():
    files = sorted(glob.glob(os.path.join(SCALA, "**", "*.scala"), recursive=True))
    assert files, "no Scala sources"
    return {f: open(f).read() for f in files}


def strip_comments(text):
    text = re.sub(r"/\*.*?\*/", lambda m: " " * len(m.group(0)), text, flags=re.S)
    return re.sub(r"//[^\n]*", "", text)


def call_arguments(text, open_at):
    """The top-level arguments of the call whose '(' is at open_at, and the
    index just past its ')'."""
    assert text[open_at] == "("
    depth, start, args, i = 0, open_at + 1, [], open_at
    quote = False
    while True:
        c = text[i]
        if c == '"':
            quote = not quote
        elif not quote:
            if c in "([{":
                depth += 1
            elif c in ")]}":
                depth -= 1
                if depth == 0:
                    last = text[start:i].strip()
                    if last:
                        args.append(last)
                    return args, i + 1
            elif c == "," and depth == 1:
                args.append(text[start:i].strip())
                start = i + 1
        i += 1


def bindings():
    """{val name: (kind, C name or stem, [layout tokens])} from DriftKernels."""
    text = strip_comments(open(BINDING).read())
    found = {}
    for m in re.finditer(r"\bval (\w+) = (bind|twins)\(", text):
        args, _ = call_arguments(text, m.end() - 1)
        name = args[0].strip('"')
        found[m.group(1)] = (m.group(2), name, args[1:])
    return found


def expected(kind, name):
    return [name] if kind == "bind" else [f"{name}_f32", f"{name}_bf16"]


def test_every_layout_matches_the_c_abi():
    found = bindings()
    assert len(found) >= 25
    for val, (kind, name, layout) in found.items():
        for entry in expected(kind, name):
            assert entry in _lib.SIGNATURES, f"{val}: {entry} is not an entry point"
            restype, argtypes = _lib.SIGNATURES[entry]
            assert restype == _lib._I32
            got = [LAYOUTS[token] for token in layout]
            assert got == argtypes, f"{val} ({entry}): layout {layout} against {argtypes}"


def test_every_kernel_entry_point_is_bound():
    bound = {entry for kind, name, _ in bindings().values() for entry in expected(kind, name)}
    missing = sorted(set(_lib.SIGNATURES) - SERVICE - bound)
    assert not missing, f"not bound in DriftKernels.scala: {missing}"


def test_the_abi_version_is_the_librarys():
    text = open(BINDING).read()
    assert re.search(r"val AbiVersion = (\d+)", text).group(1) == str(_lib.ABI_VERSION)


def test_no_cast_of_a_downcall_result():
    texts = list(sources().values()) + [open(os.path.join(ROOT, "INTEGRATION.md")).read()]
    for text in texts:
        assert ".asInstanceOf" not in text


def invoke_calls():
    """(file, handle expression, arguments, text after the call, the text of
    the method holding it) of every invokeExact in the Scala sources."""
    calls = []
    for path, raw in sources().items():
        text = strip_comments(raw)
        for m in re.finditer(r"invokeExact\(", text):
            args, end = call_arguments(text, m.end() - 1)
            head = text[:m.start()]
            handle = re.search(r"([\w.]+(\((?:[^()]|\([^()]*\))*\))?)\.$", head)
            method = head[head.rfind("def "):] if "def " in head else head
            calls.append((os.path.relpath(path, ROOT), handle.group(1) if handle else "?", args, text[end:end + 20],
                          method))
    return calls


def test_every_downcall_is_ascribed():
    calls = invoke_calls()
    assert len(calls) >= 25
    for path, handle, _, after, _ in calls:
        assert re.match(r"\s*:\s*(Int|MemorySegment)\s*\)", after), f"{path}: {handle}.invokeExact is not ascribed"


SCALA_TYPE = {"JAVA_INT": "Int", "JAVA_LONG": "Long", "JAVA_FLOAT": "Float", "JAVA_DOUBLE": "Double"}

# what the reference's helpers return (ops/AttentionOps.scala:129-233,
# ops/ElementwiseOps.scala:57-90, ops/Ops.scala:76-94) and this binding's own
RETURNS = {"Ops.checkChunks": ["Long", "Int", "Int"], "Ops.checkRowGatedAdd": ["Long", "Int"],
           "Ops.checkRope": ["Int", "Int", "Int"], "Ops.checkRopeTable": ["Int", "Int", "Int", "Int", "Boolean"],
           "Ops.checkRowWise": ["Long"], "Ops.checkCacheWrite": ["Int"], "sectionSizes": ["Int"] * 4,
           "levelsOf": ["MemorySegment", "MemorySegment", "Int"]}

# members of the reference's case classes and enums
MEMBERS = {"rope.rotaryDimensions": "Int", "rope.theta": "Float", "rope.layout.code": "Int",
           "rope.sections.code": "Int", "cache.pages": "Int", "cache.kvHeads": "Int", "cache.headDimension": "Int",
           "cache.pageSize": "Int", "norms.epsilon": "Float", "norms.weightOffset": "Float", "kind.code": "Int"}


def declared_types(method):
    """{name: Scala type} of a method's parameters and vals, where the text
    or the helpers' return types fix them."""
    types = {}
    for name, t in re.findall(r"\b(\w+)\s*:\s*(Int|Long|Float|Double|Boolean)\b", method):
        types[name] = t
    for names, call in re.findall(r"val \(([\w, ]+)\) = ([\w.]+)\(", method):
        if call in RETURNS:
            for name, t in zip([n.strip() for n in names.split(",")], RETURNS[call]):
                types[name] = t
    for name, call in re.findall(r"val (\w+) = ([\w.]+)\(", method):
        if call in RETURNS:
            types[name] = RETURNS[call][0]
    for names in re.findall(r"val Seq\(([\w, ]+)\) = [\w.]+\.shape\.dimensions", method):
        for name in names.split(","):
            types[name.strip()] = "Long"
    for names, values in re.findall(r"val \(([\w, ]+)\) = \(([^()]*(?:\([^()]*\)[^()]*)*)\)", method):
        for name, value in zip(names.split(","), values.split(",")):
            suffix = re.search(r"\.to(Int|Long)$", value.strip())
            if suffix:
                types[name.strip()] = suffix.group(1)
    return types


def value_type(arg, types):
    if re.fullmatch(r"\d+", arg):
        return "Int"
    if re.fullmatch(r"\d+L", arg):
        return "Long"
    return types.get(arg) or MEMBERS.get(arg)


def test_every_downcall_passes_its_layout():
    found = bindings()
    checked = 0
    for path, handle, args, _, method in invoke_calls():
        m = re.match(r"drift\.(\w+)(\(.*\))?$", handle)
        if not m:
            continue  # the binding's own service calls
        val = m.group(1)
        assert val in found, f"{path}: drift.{val} is not a binding"
        kind, name, layout = found[val]
        assert (m.group(2) is not None) == (kind == "twins"), f"{path}: drift.{val} picks a form iff it has two"
        assert len(args) == len(layout), f"{path}: drift.{val} takes {len(layout)} arguments, given {len(args)}"
        types = declared_types(method)
        for i, (arg, token) in enumerate(zip(args, layout)):
            address = LAYOUTS[token] == _lib._P
            assert bool(ADDRESS_ARGUMENT.match(arg)) == address, \
                f"{path}: drift.{val} argument {i} `{arg}` where the layout has {token}"
            if not address:
                # the call site's static types are the downcall's types: each
                # value's type must be known and be the layout's
                assert value_type(arg, types) == SCALA_TYPE[token], \
                    f"{path}: drift.{val} argument {i} `{arg}` is {value_type(arg, types)}, the layout has {token}"
        assert args[-1] == "DefaultStream", f"{path}: drift.{val} runs on the default stream"
        checked += 1
    assert checked >= 25


@pytest.mark.parametrize("stem", ["drift_rms_norm", "drift_attention_inputs", "drift_qk_norm_rope"])
def test_twins_take_the_same_arguments(stem):
    assert _lib.SIGNATURES[f"{stem}_f32"] == _lib.SIGNATURES[f"{stem}_bf16"]


MILL = os.path.join(SCALA, "driftKernels.mill")
MAKEFILE = os.path.join(ROOT, "drift_amd", "csrc", "Makefile")
MODULE = os.path.join(SCALA, "drift", "runner", "native", "KernelModule.scala")
BASE = os.path.join(SCALA, "drift", "runner", "ops", "DriftBase.scala")


def make_variable(name):
    """A Makefile variable's words (one assignment, continuation lines joined)."""
    text = open(MAKEFILE).read().replace("\\\n", " ")
    value = re.search(rf"^{name}\s*:?=\s*(.*)$", text, re.M).group(1)
    return value.split()


def test_the_build_task_puts_the_library_where_the_binding_loads_it():
    # the task writes <dest>/lib/libdrift_kernels.so and serves <dest> as a
    # resource root: the jar's resource /lib/libdrift_kernels.so, which
    # DriftKernels.default() copies out and loads
    mill = strip_comments(open(MILL).read())
    assert re.search(r'val out = Task\.dest / "lib"', mill)
    assert re.search(r'out / "libdrift_kernels\.so"', mill)
    assert re.search(r"PathRef\(Task\.dest\)", mill)
    assert re.search(r"super\.resources\(\) :\+ kernels\(\) :\+ driftKernels\(\)", mill)
    binding = strip_comments(open(BINDING).read())
    assert re.search(r'val Resource = "/lib/libdrift_kernels\.so"', binding)
    assert "getResourceAsStream(Resource)" in binding
    assert 'sys.props.get("drift.kernels")' in binding


def test_the_build_task_compiles_what_the_makefile_compiles():
    mill = strip_comments(open(MILL).read())
    listed = re.search(r"driftSources = Seq\(([^)]*)\)", mill).group(1)
    assert re.findall(r'"([^"]+)"', listed) == make_variable("SOURCES")
    flags = re.findall(r'"([^"]+)"', re.search(r"driftFlags = Seq\(([^)]*)\)", mill).group(1))
    make_flags = [f.replace("$(ARCH)", "gfx950") for f in make_variable("FLAGS")]
    for flag in ("--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off"):
        assert flag in flags and flag in make_flags, flag
    # packed FP32 off in both: -Xclang -target-feature -Xclang -packed-fp32-ops
    for words in (flags, make_flags):
        i = words.index("-packed-fp32-ops")
        assert words[i - 3:i] == ["-Xclang", "-target-feature", "-Xclang"]


def test_kernel_modules_load_on_first_lookup():
    # the runner's modules are made when the backend is built
    # (ops/HipBase.scala:71-75,328-336) but hold no code for gfx950: the
    # replacement KernelModule loads one only inside `module`, which only
    # `function` reaches, and `close` unloads only a loaded one
    text = strip_comments(open(MODULE).read())
    assert re.search(r"final class KernelModule\(hip: HipRuntime, val name: String\) extends AutoCloseable", text)
    body = text[text.index("private def module"):]
    module_def = body[:body.index("def function")]
    assert text.count("hip.loadModule(") == 1 and "hip.loadModule(" in module_def
    assert re.search(r"def function\(functionName: String\): KernelFunction = hip\.function\(module, functionName\)",
                     text)
    close = text[text.index("def close()"):]
    assert "handle.foreach(hip.unloadModule)" in close and "module" not in close.replace("unloadModule", "")
    # nothing outside `module` touches the code object
    outside = text.replace(module_def, "")
    assert "loadModule(" not in outside.replace("unloadModule", "")


def test_traced_downcalls_record_their_time():
    # DRIFT_HIP_TRACE times every launch by name (native/HipRuntime.scala:318,
    # 358-362); a downcall records under its entry point's name after the
    # device has finished it
    text = strip_comments(open(BASE).read())
    downcall = text[text.index("protected def downcall"):]
    downcall = downcall[:downcall.index("\n  }\n")]
    assert "HipRuntime.Trace.on" in downcall
    traced = downcall[downcall.index("HipRuntime.Trace.on"):downcall.index("} else")]
    order = [traced.index(s) for s in ("System.nanoTime()", "drift.check(name, call)", "hip.synchronize()",
                                       "HipRuntime.Trace.record(name, System.nanoTime() - from)")]
    assert order == sorted(order)
    assert "drift.check(name, call)" in downcall[downcall.index("} else"):]
