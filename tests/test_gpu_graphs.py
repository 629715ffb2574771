"""The entry points inside a HIP graph. The library allocates, synchronizes
and clears nothing when it launches, so a caller may capture its launches
(here through torch.cuda.graph: the host mirror launches on torch's current
stream). A decode step's and a prefill step's launches are captured once,
then replayed three times with new inputs copied in between; after each
replay every output, the int8 side output included, must equal bit for bit
what the same calls make eagerly on the same inputs."""

import numpy as np
import pytest
import torch

from drift_amd import ops as d
from oracle import oracle as o
from tests.helpers import DEV, step

pytestmark = pytest.mark.gpu

B, HIDDEN, INTER = 8, 4096, 14336
TOKENS, Q_HEADS, KV_HEADS, DIM = 64, 32, 8, 128
ROWS, COLS, PER_SAMPLE = 256, 3072, 128
VOCAB, IDS = 512, 37
R_ROWS, R_COLS = 40, 512


def inputs(seed: int) -> dict:
    """Fresh host values for every input of the captured steps."""
    rng = np.random.default_rng(seed)

    def bf16(shape, scale=1.0):
        bits = o.to_bf16((scale * rng.standard_normal(shape)).astype(np.float32))
        return torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16)

    def f32(shape, scale=1.0, offset=0.0):
        return torch.from_numpy((offset + scale * rng.standard_normal(shape)).astype(np.float32))

    codes = rng.integers(-127, 128, (R_ROWS, R_COLS)).astype(np.int8)
    return {
        "x": bf16((B, HIDDEN)), "w": f32(HIDDEN, 0.1, 1.0), "xf": f32((B, HIDDEN)),
        "gate": bf16((B, INTER)), "up": bf16((B, INTER)),
        "ax": bf16((ROWS, COLS)), "scale": f32((2, COLS), 0.1), "shift": f32((2, COLS), 0.1),
        "q": bf16((TOKENS, Q_HEADS, DIM)), "k": bf16((TOKENS, KV_HEADS, DIM)),
        "qw": f32(DIM, 0.1, 1.0), "kw": f32(DIM, 0.1, 1.0),
        "positions": torch.from_numpy(rng.integers(0, 4096, TOKENS).astype(np.int32)),
        "table": torch.from_numpy(o.q8_0_table(VOCAB, HIDDEN, rng)),
        "ids": torch.from_numpy(rng.integers(0, VOCAB, IDS).astype(np.int32)),
        "codes": torch.from_numpy(codes.view(np.int8)),
        "rscales": torch.from_numpy((1e-3 + 1e-3 * rng.random(R_ROWS)).astype(np.float32)),
    }


def outputs() -> dict:
    def empty(shape, dtype=torch.bfloat16):
        return torch.empty(shape, dtype=dtype, device=DEV)

    return {
        "norm": empty((B, HIDDEN)), "normf": empty((B, HIDDEN), torch.float32), "swiglu": empty((B, INTER)),
        "adaln": empty((ROWS, COLS)), "rq": empty((TOKENS, Q_HEADS, DIM)), "rk": empty((TOKENS, KV_HEADS, DIM)),
        "emb": empty((IDS, HIDDEN)), "rot": empty((R_ROWS, R_COLS)),
    }


def run(hip: d.HipOps, dev: dict, out: dict) -> None:
    """A decode step's launches (norm, SwiGLU, the F32 norm with its int8
    side output, the embedding gather) and a prefill step's (AdaLN, QK norm +
    RoPE, a rotated weight's decode)."""
    hip.rmsNorm(dev["x"], dev["w"], 1e-5, 0.0, out["norm"])
    hip.gated(d.Activation.Silu, dev["gate"], dev["up"], out["swiglu"])
    hip.rmsNorm(dev["xf"], dev["w"], 1e-6, 0.0, out["normf"])  # quantizes as it writes
    hip.embedding(d.Q8_0Table(dev["table"], HIDDEN), dev["ids"], out["emb"])
    hip.layerNormModulate(dev["ax"], dev["scale"], dev["shift"], 1e-6, out["adaln"], PER_SAMPLE)
    norms = d.QueryKeyNorms(dev["qw"], dev["kw"], 1e-6, 0.0, d.Rope(1e6, DIM, d.RopeLayout.Neox))
    hip.queryKeyNormRope(dev["q"], dev["k"], norms, dev["positions"], out["rq"], out["rk"])
    weight = hip.rotated(dev["codes"], d.ConvRotParts(dev["rscales"]))
    hip.convert(weight, out["rot"])


def bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.uint8).numpy()


def test_decode_and_prefill_steps_replay_in_a_graph():
    step("decode and prefill launches captured in a HIP graph, replayed 3 times")
    eager, captured = d.HipOps(), d.HipOps()
    eager.quantizesX = captured.quantizesX = True  # int8 products follow: the F32 norm quantizes
    dev = {name: t.to(DEV) for name, t in inputs(1).items()}
    graph_out, eager_out = outputs(), outputs()
    # a first eager run sizes the side output's buffer before the capture
    run(captured, dev, graph_out)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run(captured, dev, graph_out)
    torch.cuda.synchronize()
    for replay in range(3):
        fresh = inputs(10 + replay)
        for name, t in fresh.items():
            dev[name].copy_(t.to(DEV))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = {name: bits(t) for name, t in graph_out.items()}
        got_side = bits(captured._quantizedBuffer[: eager_side_size()])
        run(eager, dev, eager_out)
        torch.cuda.synchronize()
        for name, t in eager_out.items():
            assert np.array_equal(got[name], bits(t)), f"replay {replay}: {name} differs from the eager launch"
        assert np.array_equal(got_side, bits(eager._quantizedBuffer[: eager_side_size()])), \
            f"replay {replay}: the int8 side output differs"


def eager_side_size() -> int:
    """Bytes of the side output of the F32 norm's B x HIDDEN values."""
    values = B * HIDDEN
    return values + 8 * (values // 32)
