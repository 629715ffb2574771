"""Shared pieces of the GPU parity tests: device tensors from the oracle's
numpy arrays and back, and the tolerances the kernels are held to.

Tolerances (the stated bars):
- F32 outputs: tensor/Comparison.scala's rule |a - e| <= abs + rel |e| with
  rel 1e-5 and abs 1e-6 (the reference's `Close`, SmallOpsTests.scala:66),
  and the stated fp32 bar, 1e-5 relative with no absolute slack:
  |a - e| <= 1e-5 max(|e|, 2^-126) (the floor only for subnormal and zero
  expectations, whose ulps are wider than 1e-5 of them);
- BF16 outputs: at most 1 bf16 ulp from the oracle's bf16 (its F32 result
  rounded with CpuOps.toBfloat16), NaN where the oracle has NaN;
- gathers and conversions: bit-exact.
"""

from __future__ import annotations

import os
import sys

import numpy as np
import torch

from oracle import oracle as o

DEV = "cuda:0"


def step(message: str) -> None:
    """Names the case about to run on the GPU, flushed first."""
    print(f"[gpu] {message}", flush=True)
    sys.stdout.flush()


def dev_f32(a) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(DEV)


def dev_bf16(bits) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits, np.uint16).view(np.int16)).view(torch.bfloat16).to(DEV)


def dev_i32(a) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, np.int32)).to(DEV)


def host_f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().numpy().astype(np.float32, copy=False)


def host_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def bf16_input(values) -> np.ndarray:
    """f32 values rounded to bf16 bits (the inputs of the bf16 cases)."""
    return o.to_bf16(np.asarray(values, np.float32))


def comparison(expected, actual, absolute=1e-6, relative=1e-5):
    """(passed, mismatches, max abs, first index) as Comparison.of reports."""
    e = np.asarray(expected, np.float64).ravel()
    a = np.asarray(actual, np.float64).ravel()
    nan = np.isnan(e) | np.isnan(a)
    inf = np.isinf(e) | np.isinf(a)
    with np.errstate(invalid="ignore"):
        diff = np.abs(a - e)
        ok = np.where(nan, np.isnan(e) & np.isnan(a), np.where(inf, e == a, diff <= absolute + relative * np.abs(e)))
    bad = np.flatnonzero(~ok)
    finite = ~(nan | inf)
    return bad.size == 0, bad.size, float(diff[finite].max(initial=0.0)), (int(bad[0]) if bad.size else None)


F32_RELATIVE = 1e-5
F32_FLOOR = float(np.finfo(np.float32).tiny)  # 2^-126


def relative_errors(expected, actual) -> np.ndarray:
    """|a - e| / max(|e|, 2^-126) of the finite pairs (NaN and infinity are
    held to equality by `comparison`)."""
    e = np.asarray(expected, np.float64).ravel()
    a = np.asarray(actual, np.float64).ravel()
    finite = np.isfinite(e) & np.isfinite(a)
    return np.abs(a[finite] - e[finite]) / np.maximum(np.abs(e[finite]), F32_FLOOR)


def assert_f32(expected, actual, absolute=1e-6, relative=1e-5, what=""):
    passed, mismatches, max_abs, first = comparison(expected, actual, absolute, relative)
    assert passed, f"{what}: {mismatches} mismatches, first at {first}, max abs {max_abs:.3g}"
    rel = relative_errors(expected, actual)
    worst = float(rel.max(initial=0.0))
    record_f32(what, worst)
    assert worst <= F32_RELATIVE, (f"{what}: {int((rel > F32_RELATIVE).sum())} values beyond {F32_RELATIVE:g} "
                                   f"relative, worst {worst:.3g}")


def record_f32(what: str, worst: float) -> None:
    """Appends an F32 check's worst relative error to the file
    DRIFT_F32_ERRORS names, if any (the figures the design notes report)."""
    path = os.environ.get("DRIFT_F32_ERRORS")
    if path:
        with open(path, "a") as f:
            f.write(f"{os.environ.get('PYTEST_CURRENT_TEST', '?').split(' ')[0]}\t{what}\t{worst:.3e}\n")


def bf16_ulps(expected_bits, actual_bits) -> np.ndarray:
    """Distance in bf16 ulps on the ordered line; NaN against NaN is 0, NaN
    against a number is huge."""
    e = np.asarray(expected_bits, np.uint16).astype(np.int64).ravel()
    a = np.asarray(actual_bits, np.uint16).astype(np.int64).ravel()
    e_nan = ((e & 0x7F80) == 0x7F80) & ((e & 0x7F) != 0)
    a_nan = ((a & 0x7F80) == 0x7F80) & ((a & 0x7F) != 0)
    oe = np.where(e & 0x8000, -(e & 0x7FFF), e)
    oa = np.where(a & 0x8000, -(a & 0x7FFF), a)
    d = np.abs(oe - oa)
    return np.where(e_nan | a_nan, np.where(e_nan & a_nan, 0, 1 << 20), d)


def assert_bf16(expected_bits, actual_bits, max_ulps=1, what=""):
    u = bf16_ulps(expected_bits, actual_bits)
    bad = np.flatnonzero(u > max_ulps)
    assert bad.size == 0, (f"{what}: {bad.size} values beyond {max_ulps} bf16 ulp, first at {bad[0]} "
                           f"(expected {int(np.asarray(expected_bits).ravel()[bad[0]]):#06x}, "
                           f"got {int(np.asarray(actual_bits).ravel()[bad[0]]):#06x})")


def assert_bits(expected_bits, actual_bits, what=""):
    e = np.asarray(expected_bits).ravel()
    a = np.asarray(actual_bits).ravel()
    bad = np.flatnonzero(e != a)
    assert bad.size == 0, f"{what}: {bad.size} values differ, first at {bad[0]} ({e[bad[0]]:#x} vs {a[bad[0]]:#x})"


def gaussian(seed: int, shape, scale: float = 1.0) -> np.ndarray:
    return (scale * np.random.default_rng(seed).standard_normal(shape)).astype(np.float32)
