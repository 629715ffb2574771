"""Benchmark of the drift runner's fused layer kernels on one MI355X.

A step is one pass of the path over its configurations, every kernel once:
  C2  decode bf16: RMSNorm [B, 4096] and SwiGLU [B, 14336], B = 1, 8, 64
      decode F32 with the int8 side output the products read: RMSNorm
      [B, 4096] and SwiGLU [B, 14336], B = 1, 64
  C3  prefill bf16: per-head RMSNorm + NeoX RoPE, Q [4096, 32, 128], K [4096, 8, 128]; and
      the same with V [4096, 8, 128], keys and values written to a paged F16 KV cache
  C4  Q8_0 gather of 8192 ids from [151936, 4096] to bf16
  C5  Video DiT block bf16: AdaLN [65520, 3072], GELU-tanh in place, 3-D RoPE
      Q [65520, 24, 128] on the 21 x 30 x 52 grid; the gated residual with
      per-sample gates, per-row modulation and gated residual from a
      [65520, 6 x 3072] F32 table, and a per-head gate over [65520 x 24, 128]
  Weights decoded to bf16 for the GEMM path: a Q4_K GGUF weight [14336, 4096],
      and ComfyUI's rotated linears (ConvRot, int8 and 4-bit codes) [13824, 5120]
Inputs are synthetic (seeded device generators) and resident in HBM. Each
kernel rotates through buffer sets totalling more than 512 MB, so the 256 MB
Infinity Cache cannot hold what the next launch reads.

The timed region replays, kernel by kernel (largest first, so that no short
kernel is timed while the clocks rise after the decode kernels' idle gaps),
a HIP graph holding that kernel's K launches (K of one, then K of the next), so no
kernel reads what the kernel before it left in the Infinity Cache or pays
for the dirty lines it left there, and no host call sits between launches.
Every call is checked by the Ops layer beforehand; the graphs capture the
C-ABI calls those checks produced. The same launches made one by one from
Python are timed too (`us_eager`), and `host_us_per_call` is the C++ host
cost of one call of each entry point (drift_amd/host/launch_cost).

Printed: one JSON line. `value` is the step's algorithmic bytes (the reads
and writes of the tensors each op names) over the step's wall time;
`kernels` has each kernel's HIP-event times: `us_step`, its K-launch
replay's span over K in the timed step; `us_replay`, the median over five
replays; and `us`, the launch inside a graph: `us_replay` less the fixed
start every replay pays between the event before it and its first launch
(`graph_start_us`, measured in the run with a one-block launch in graphs
of K and 4 K launches: about 12 us, 0.6 us a launch at K = 20; the kernel
trace shows the same gap before every kernel's graph). Then GB/s (from
`us`), fraction of the 8 TB/s HBM peak, fraction of its ceiling and
rows/s;
`ceilings` holds, for each long kernel, the fastest probe moving its bytes
in its read:write mix with nothing else (drift_stream_mix: blocks that only
read or only write; drift_wave_copy: one-wave blocks each reading its share
and then writing its share, the kernels' own shape and the tighter at the
prefill sizes; drift_block_copy: the same waves in 512-thread blocks, the
shape of the ops that read F32 table rows), for the gather also its own pattern with no decode
(drift_row_probe and drift_wave_row_probe: the rows its ids name read, its
output written, by a block or by 1 to 8 waves an id; `frac_of_row_probe`), the
reference's streaming read (drift_read_sum_f32x4) over 1 GiB, and the
per-launch floor of a graph replay (`launch_floor`: one block writing one
16-byte chunk), which the decode shapes' few microseconds sit on. A probe's
launches fall into two or three durations by clock and memory state, so
each kernel is also replayed in alternation with its best probe
(`ceilings[k]["matched"]`, and `frac_of_probe_matched`: the ratio of their
median replays under the same conditions, the start taken out of both);
every probe's `us` is taken the same way;
`roofline` is the dominant kernel's; `cpu_baseline` is the CPU reference
arithmetic (the oracle) timed on a bounded sample of the same work on this
host's cores, scaled to the whole step. With `--formats`, `formats` holds
every storage type's decode of a [14336, 4096] weight to bf16, each against
its probe in alternation (not part of the step or `value`).
"""

from __future__ import annotations

import argparse
import ctypes
import faulthandler
import json
import math
import os
import statistics
import sys
import time
import subprocess
from concurrent.futures import ThreadPoolExecutor
from typing import Optional

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from drift_amd import _lib  # noqa: E402
from drift_amd import ops as d  # noqa: E402

HBM_PEAK_GBS = 8000.0
MATCHED_ROUNDS = 7  # alternations of each kernel with its probe
GRAPH_ROUNDS = 5  # replays of each kernel's graph: the first is the timed step
LONG = 4  # the graph start's long graph holds LONG x K launches
START_MS = 0.0  # a graph replay's fixed start (graph_start); 0 with --no-graph-start
STEPS = 20  # launches a graph holds (--steps)
MALL_BYTES = 512 << 20
DEV = "cuda:0"


class Kernel:
    """One fused kernel at one configuration: its launch over buffer set i,
    its algorithmic bytes (and how many of them are reads) and rows per
    launch, and a CPU reference leg."""

    def __init__(self, name, config, bytes_per_call, rows, launch, sets=1, read_bytes=None):
        self.name, self.config = name, config
        self.sets = sets
        self.calls = []
        self.bytes, self.rows = bytes_per_call, rows
        self.read_bytes = bytes_per_call // 2 if read_bytes is None else read_bytes
        self.launch = launch
        self.cpu = None  # (sample description, seconds for the sample, fraction of a call the sample is)
        self.cpu_all = None  # (threads, seconds for the same sample split across them)
        self.graph_ms = None  # a K-launch replay's span over K, its fixed start included (median over the rounds)
        self.step_ms = None  # the same in the timed step's replay
        self.matched_ms = None  # the same, in alternation with its probe (median replay)
        self.eager_ms = None  # average launch, each made from Python through ctypes
        self.ceiling = None  # the stream probe at this kernel's bytes and read/write mix

    def prepare(self, ops: "Prepared") -> None:
        """Runs the Ops checks of every buffer set's call and keeps the C-ABI
        call each produces."""
        lib = _lib.load()
        for i in range(self.sets):
            ops.kept = None
            self.launch(i)
            if ops.kept is None:
                raise RuntimeError(f"{self.name}: the launch made no C-ABI call")
            entry, args = ops.kept
            self.calls.append((entry, getattr(lib, entry), args))

    @property
    def launch_ms(self) -> float:
        """Average launch inside the graph: the median replay's span over K
        with the replay's fixed start (START_MS) taken out."""
        return self.graph_ms - START_MS / STEPS

    @property
    def matched_launch_ms(self) -> float:
        return self.matched_ms - START_MS / STEPS

    def fire(self, i: int, stream) -> None:
        entry, fn, args = self.calls[i % len(self.calls)]
        code = fn(*args, stream)
        if code != 0:
            raise _lib.HipError(entry, code, _lib.load().drift_last_error().decode())


class Prepared(d.HipOps):
    """The Ops layer with its checks, keeping the call each method would make
    (without its stream) instead of making it."""

    kept = None

    def _launch(self, entry: str, *args) -> None:
        self.onWork()
        self.kept = (entry, args)


def sets_for(bytes_per_call: int, floor: int = 2, cap: int = 64) -> int:
    """Buffer sets to rotate through so the sets total more than 512 MB (the
    decode shapes are capped: a decode step's activations do sit in cache)."""
    return min(cap, max(floor, math.ceil(MALL_BYTES / max(bytes_per_call, 1)) + 1))


def gen(seed):
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    return g


def randn_bf16(shape, seed, scale=1.0):
    return (scale * torch.randn(shape, generator=gen(seed), device=DEV)).to(torch.bfloat16)


def _side(side, values):
    """Pointers to the codes, scales and sums of a side-output buffer."""
    base = side.data_ptr()
    return (ctypes.c_void_p(base), ctypes.c_void_p(base + values), ctypes.c_void_p(base + values + 4 * (values // 32)))


def side_args(x, y, w, out, rows, cols, side):
    return (ctypes.c_void_p(x.data_ptr()), None if y is None else ctypes.c_void_p(y.data_ptr()),
            ctypes.c_void_p(w.data_ptr()), ctypes.c_void_p(out.data_ptr()), rows, cols, 1e-5, 0.0, 1,
            *_side(side, rows * cols))


def gated_side_args(g, u, out, n, side):
    return (ctypes.c_void_p(g.data_ptr()), ctypes.c_void_p(u.data_ptr()), ctypes.c_void_p(out.data_ptr()), n, 0,
            *_side(side, n))


def make_kernels(hip: d.HipOps):
    kernels = []

    # C2 decode: RMSNorm bf16 [B, 4096] (w f32, eps 1e-5) and SwiGLU [B, 14336]
    for b in (1, 8, 64):
        nbytes = 2 * b * 4096 * 2 + 4096 * 4
        n = sets_for(nbytes, 8, 8)
        xs = [randn_bf16((b, 4096), 10 + i) for i in range(n)]
        outs = [torch.empty_like(xs[0]) for _ in range(n)]
        w = (1 + 0.1 * torch.randn(4096, generator=gen(1), device=DEV)).float()
        kernels.append(Kernel(f"rms_norm_bf16_b{b}", f"C2 RMSNorm bf16 [{b},4096] eps 1e-5", nbytes, b,
                              lambda i, xs=xs, outs=outs, w=w: hip.rmsNorm(xs[i % len(xs)], w, 1e-5, 0.0,
                                                                           outs[i % len(outs)]), sets=n,
                              read_bytes=b * 4096 * 2 + 4096 * 4))
        nbytes = 3 * b * 14336 * 2
        n = sets_for(nbytes, 8, 8)
        gs = [randn_bf16((b, 14336), 100 + i) for i in range(n)]
        us = [randn_bf16((b, 14336), 200 + i) for i in range(n)]
        os_ = [torch.empty_like(gs[0]) for _ in range(n)]
        kernels.append(Kernel(f"swiglu_bf16_b{b}", f"C2 SwiGLU bf16 [{b},14336]", nbytes, b,
                              lambda i, gs=gs, us=us, os_=os_: hip.gated(d.Activation.Silu, gs[i % len(gs)],
                                                                         us[i % len(us)], os_[i % len(os_)]),
                              sets=n, read_bytes=2 * b * 14336 * 2))

    # The int8 side output for the decode products: F32 RMSNorm [B, 4096] and
    # SwiGLU [B, 14336] writing their output quantized too (codes 1 B per
    # value, scale and code sum 8 B per 32 values)
    for b in (1, 64):
        n = sets_for(b * 4096 * 9, 8, 8)
        xs = [(0.5 * torch.randn((b, 4096), generator=gen(800 + i), device=DEV)) for i in range(n)]
        outs = [torch.empty_like(xs[0]) for _ in range(n)]
        sides = [torch.empty(b * 4096 + 8 * (b * 4096 // 32), dtype=torch.int8, device=DEV) for _ in range(n)]
        w = (1 + 0.1 * torch.randn(4096, generator=gen(7), device=DEV)).float()
        nbytes = b * 4096 * (4 + 4 + 1) + 8 * (b * 4096 // 32) + 4096 * 4
        kernels.append(Kernel(f"rms_norm_q8_f32_b{b}", f"RMSNorm f32 [{b},4096] + int8 side output", nbytes, b,
                              lambda i, xs=xs, outs=outs, sides=sides, w=w, b=b: hip._launch(
                                  "drift_rms_norm_f32", *side_args(xs[i % len(xs)], None, w, outs[i % len(outs)], b,
                                                                   4096, sides[i % len(sides)])), sets=n,
                              read_bytes=b * 4096 * 4 + 4096 * 4))
        n = sets_for(b * 14336 * 13, 8, 8)
        gs = [(0.5 * torch.randn((b, 14336), generator=gen(900 + i), device=DEV)) for i in range(n)]
        us = [(0.5 * torch.randn((b, 14336), generator=gen(950 + i), device=DEV)) for i in range(n)]
        os_ = [torch.empty_like(gs[0]) for _ in range(n)]
        sides = [torch.empty(b * 14336 + 8 * (b * 14336 // 32), dtype=torch.int8, device=DEV) for _ in range(n)]
        nbytes = b * 14336 * (4 + 4 + 4 + 1) + 8 * (b * 14336 // 32)
        kernels.append(Kernel(f"swiglu_q8_f32_b{b}", f"SwiGLU f32 [{b},14336] + int8 side output", nbytes, b,
                              lambda i, gs=gs, us=us, os_=os_, sides=sides, b=b: hip._launch(
                                  "drift_gated_f32", *gated_side_args(gs[i % len(gs)], us[i % len(us)],
                                                                      os_[i % len(os_)], b * 14336,
                                                                      sides[i % len(sides)])), sets=n,
                              read_bytes=2 * b * 14336 * 4))

    # C3 prefill: per-head RMSNorm (eps 1e-6) + NeoX RoPE (theta 1e6)
    t, hq, hk, dim = 4096, 32, 8, 128
    nbytes = 2 * (t * (hq + hk) * dim * 2) + t * 4 + 2 * dim * 4
    n = sets_for(nbytes)
    qs = [randn_bf16((t, hq, dim), 300 + i) for i in range(n)]
    ks = [randn_bf16((t, hk, dim), 400 + i) for i in range(n)]
    rqs = [torch.empty_like(qs[0]) for _ in range(n)]
    rks = [torch.empty_like(ks[0]) for _ in range(n)]
    qw = (1 + 0.1 * torch.randn(dim, generator=gen(2), device=DEV)).float()
    kw = (1 + 0.1 * torch.randn(dim, generator=gen(3), device=DEV)).float()
    positions = torch.arange(t, dtype=torch.int32, device=DEV)
    norms = d.QueryKeyNorms(qw, kw, 1e-6, 0.0, d.Rope(1e6, 128, d.RopeLayout.Neox))
    kernels.append(Kernel("qk_norm_rope_bf16", "C3 per-head RMSNorm + NeoX RoPE bf16 Q[4096,32,128] K[4096,8,128]",
                          nbytes, t,
                          lambda i, n=n: hip.queryKeyNormRope(qs[i % n], ks[i % n], norms, positions, rqs[i % n],
                                                              rks[i % n]), sets=n,
                          read_bytes=t * (hq + hk) * dim * 2 + t * 4 + 2 * dim * 4))

    # The same prefill through the dense decoders' whole attention-input step:
    # per-head norms, NeoX rope, and keys and values into the paged F16 cache
    # (pages of 16 tokens, a shuffled page table)
    vs = [randn_bf16((t, hk, dim), 450 + i) for i in range(n)]
    pages = t // 16
    caches = [d.KvCache.allocate(pages, 16, hk, dim, DEV) for _ in range(n)]
    tables = [torch.randperm(pages, generator=gen(460 + i), device=DEV).to(torch.int32) for i in range(n)]
    nbytes_ai = t * (2 * hq + 4 * hk) * dim * 2 + t * 4 + 2 * dim * 4 + pages * 4
    kernels.append(Kernel("attention_inputs_bf16", "C3 with the KV-cache write: norms + NeoX RoPE of Q[4096,32,128] "
                          "K[4096,8,128] bf16, K and V[4096,8,128] into a paged F16 cache", nbytes_ai, t,
                          lambda i, n=n: hip.queryKeyNormRopeCache(qs[i % n], ks[i % n], vs[i % n], norms, positions,
                                                                   caches[i % n], tables[i % n], 0, rqs[i % n]),
                          sets=n, read_bytes=t * (hq + 2 * hk) * dim * 2 + t * 4 + 2 * dim * 4 + pages * 4))

    # C4: Q8_0 gather, 8192 ids from [151936, 4096] to bf16
    vocab, cols, count = 151936, 4096, 8192
    blocks = cols // 32
    table = torch.empty((vocab, blocks, 34), dtype=torch.uint8, device=DEV)
    g = gen(4)
    for lo in range(0, vocab, 16384):
        hi = min(vocab, lo + 16384)
        table[lo:hi, :, 2:] = torch.randint(-127, 128, (hi - lo, blocks, 32), generator=g, device=DEV,
                                            dtype=torch.int32).to(torch.int8).view(torch.uint8)
        sc = (1e-3 + (2e-2 - 1e-3) * torch.rand((hi - lo, blocks), generator=g, device=DEV)).half()
        table[lo:hi, :, 0:2] = sc.view(torch.uint8).view(hi - lo, blocks, 2)
    q8 = d.Q8_0Table(table.view(vocab, blocks * 34), cols)
    nbytes = count * blocks * 34 + count * 4 + count * cols * 2
    # id sets enough that the rows they name total more than 512 MB: fewer
    # sets would re-read rows the 256 MB MALL still holds from earlier sets
    n = sets_for(count * blocks * 34)
    idss = [torch.randint(0, vocab, (count,), generator=gen(500 + i), device=DEV, dtype=torch.int32)
            for i in range(n)]
    gouts = [torch.empty((count, cols), dtype=torch.bfloat16, device=DEV) for _ in range(n)]
    kernels.append(Kernel("embedding_q8_0_bf16", "C4 Q8_0 gather 8192 ids from [151936,4096] to bf16", nbytes,
                          count, lambda i, n=n: hip.embedding(q8, idss[i % n], gouts[i % n]), sets=n,
                          read_bytes=count * blocks * 34 + count * 4))

    # C5: Video DiT block, x [2 * 32760, 3072]
    rows, width, per = 2 * 32760, 3072, 32760
    n = 2
    xs5 = [randn_bf16((rows, width), 600 + i) for i in range(n)]
    outs5 = [torch.empty_like(xs5[0]) for _ in range(n)]
    shift = (0.1 * torch.randn((2, width), generator=gen(5), device=DEV)).float()
    scale = (0.1 * torch.randn((2, width), generator=gen(6), device=DEV)).float()
    nbytes = 2 * rows * width * 2 + 2 * 2 * width * 4
    kernels.append(Kernel("adaln_bf16", "C5 AdaLN LN(eps 1e-6)*(1+scale)+shift bf16 [65520,3072]", nbytes, rows,
                          lambda i, n=n: hip.layerNormModulate(xs5[i % n], scale, shift, 1e-6, outs5[i % n], per),
                          sets=n, read_bytes=rows * width * 2 + 2 * 2 * width * 4))
    nbytes = 2 * rows * width * 2
    kernels.append(Kernel("gelu_tanh_bf16", "C5 GELU-tanh bf16 in place [65520,3072]", nbytes, rows,
                          lambda i, n=n: hip.activation(d.Activation.GeluTanh, outs5[i % n], outs5[i % n]),
                          sets=n, read_bytes=rows * width * 2))
    qs5 = [randn_bf16((rows, 24, 128), 700 + i) for i in range(n)]
    rq5 = [torch.empty_like(qs5[0]) for _ in range(n)]
    nbytes = 2 * rows * 24 * 128 * 2
    kernels.append(Kernel("rope_3d_bf16", "C5 3-D RoPE bf16 Q[65520,24,128] grid 21x30x52 theta 1e4", nbytes, rows,
                          lambda i, n=n: hip.rope3d(qs5[i % n], 21, 30, 52, rq5[i % n]), sets=n,
                          read_bytes=rows * 24 * 128 * 2))

    # The same block's gated residuals and per-row modulation (bf16 x, F32
    # gates and tables): x += gate[sample] * y; out = x * (1 + t[r][4]) +
    # t[r][3] and x += t[r][5] * y over a [65520, 6 x 3072] table; and the
    # per-head gate x[r] += g[r] * y[r] over [65520 x 24, 128]
    ys5 = [randn_bf16((rows, width), 650 + i) for i in range(n)]
    gates = (0.5 * torch.randn((2, width), generator=gen(8), device=DEV)).float()
    nbytes = rows * width * 6 + 2 * width * 4
    kernels.append(Kernel("gated_add_bf16", "C5 gated residual x += gate[sample] * y bf16 [65520,3072]", nbytes, rows,
                          lambda i, n=n: hip.gatedAdd(xs5[i % n], ys5[i % n], gates, per), sets=n,
                          read_bytes=rows * width * 4 + 2 * width * 4))
    table = torch.empty((rows, 6 * width), dtype=torch.float32, device=DEV)
    for lo in range(0, rows, 8192):
        table[lo:lo + 8192] = 0.3 * torch.randn((min(8192, rows - lo), 6 * width), generator=gen(9), device=DEV)
    # in place, as every caller of the reference's modulateChunks runs it
    # (models/Pid.scala:755,811, models/MageVae.scala:603)
    nbytes = rows * width * (2 + 2 + 4 + 4)
    kernels.append(Kernel("modulate_chunks_bf16", "C5 per-row modulation x = x*(1+t[r][4])+t[r][3] in place, bf16 "
                          "[65520,3072], t F32 [65520,18432]", nbytes, rows,
                          lambda i, n=n: hip.modulateChunks(xs5[i % n], table, 3, 4, xs5[i % n]), sets=n,
                          read_bytes=rows * width * 10))
    nbytes = rows * width * (2 + 2 + 2 + 4)
    kernels.append(Kernel("gated_add_chunk_bf16", "C5 per-row gated residual x += t[r][5] * y bf16 [65520,3072]",
                          nbytes, rows, lambda i, n=n: hip.gatedAddChunk(xs5[i % n], ys5[i % n], table, 5), sets=n,
                          read_bytes=rows * width * 8))
    heads = rows * 24
    head_gates = torch.rand(heads, generator=gen(10), device=DEV).float()
    nbytes = heads * 128 * 6 + heads * 4
    kernels.append(Kernel("row_gated_add_bf16", "per-head gate x[r] += g[r] * y[r] bf16 [65520*24,128]", nbytes, heads,
                          lambda i, n=n: hip.rowGatedAdd(qs5[i % n].view(heads, 128), rq5[i % n].view(heads, 128),
                                                         head_gates), sets=n,
                          read_bytes=heads * 128 * 4 + heads * 4))

    # Weights decoded for the GEMM path: a Q4_K GGUF weight [14336, 4096] to
    # bf16, and ComfyUI's rotated linears (int8 codes, and 4-bit codes with
    # fp8 scales a 64 columns) of a DiT FFN [13824, 5120] to bf16
    rows_k, cols_k = 14336, 4096
    nbytes = rows_k * cols_k // 256 * 144 + rows_k * cols_k * 2
    n = sets_for(nbytes)
    q4k = []
    for i in range(n):
        raw = torch.randint(0, 256, (rows_k, cols_k // 256, 144), generator=gen(1000 + i), device=DEV,
                            dtype=torch.int32).to(torch.uint8)
        dm = (1e-3 + 1e-2 * torch.rand((rows_k, cols_k // 256, 2), generator=gen(1100 + i), device=DEV)).half()
        raw[:, :, 0:4] = dm.view(torch.uint8).view(rows_k, cols_k // 256, 4)
        q4k.append(d.StoredTable(raw.view(rows_k, -1), d.STORAGE_TYPES["Q4_K"], cols_k))
    kouts = [torch.empty((rows_k, cols_k), dtype=torch.bfloat16, device=DEV) for _ in range(n)]
    kernels.append(Kernel("dequantize_q4_k_bf16", "Q4_K weight [14336,4096] decoded to bf16", nbytes, rows_k,
                          lambda i, n=n: hip.dequantize(q4k[i % n], kouts[i % n]), sets=n,
                          read_bytes=rows_k * cols_k // 256 * 144))
    rows_r, cols_r, group = 13824, 5120, 64
    for four in (False, True):
        code_bytes = rows_r * cols_r // (2 if four else 1)
        nbytes = code_bytes + rows_r * 4 + rows_r * cols_r * 2 + (rows_r * cols_r // group if four else 0)
        n = sets_for(nbytes)
        weights = []
        for i in range(n):
            codes = torch.randint(-128, 128, (rows_r, cols_r // (2 if four else 1)), generator=gen(1200 + i),
                                  device=DEV, dtype=torch.int32).to(torch.int8)
            scales = (1e-4 + 1e-3 * torch.rand(rows_r, generator=gen(1300 + i), device=DEV)).float()
            levels = None
            if four:
                book = torch.sort(2 * torch.rand(16, generator=gen(1400 + i), device=DEV) - 1).values.float()
                rel = torch.randint(0x58, 0x77, (rows_r, cols_r // group), generator=gen(1500 + i), device=DEV,
                                    dtype=torch.int32).to(torch.uint8)
                levels = d.ConvRotLevels(book, rel, group)
            weights.append(hip.rotated(codes, d.ConvRotParts(scales, levels)))
        routs = [torch.empty((rows_r, cols_r), dtype=torch.bfloat16, device=DEV) for _ in range(n)]
        name = "rotated_dequantize_w4a8_bf16" if four else "rotated_dequantize_i8_bf16"
        what = "4-bit (fp8 scales a 64 columns)" if four else "int8"
        kernels.append(Kernel(name, f"ConvRot rotated linear, {what} codes [13824,5120] decoded to bf16", nbytes,
                              rows_r, lambda i, n=n, w=weights, o_=routs: hip.convert(w[i % n], o_[i % n]), sets=n,
                              read_bytes=nbytes - rows_r * cols_r * 2))
    return kernels


# ------------------------------------------------------------------ CPU baseline

def format_kernels(hip: d.HipOps) -> list:
    """Every storage type's whole-table decode to bf16 (the GEMM path's
    dequantize) at the Q4_K weight's shape [14336, 4096]: random bytes with
    each block's leading fp16 fields set to small positive scales, buffer
    sets past the MALL. Timed only with --formats, outside the step."""
    rows, cols = 14336, 4096
    kernels = []
    for name, t in d.STORAGE_TYPES.items():
        row_bytes = t.rowBytes(cols)
        nbytes = rows * row_bytes + rows * cols * 2
        n = sets_for(nbytes)
        tables = []
        for i in range(n):
            g = gen(2000 + i)
            raw = torch.randint(0, 256, (rows, row_bytes), generator=g, device=DEV, dtype=torch.int32).to(torch.uint8)
            if t.values > 1 and name != "Q6_K":  # Q6_K keeps its scale last
                blocks = raw.view(rows, cols // t.values, t.bytes)
                scales = (1e-3 + 1e-2 * torch.rand((rows, cols // t.values, 2), generator=g, device=DEV)).half()
                blocks[:, :, 0:4] = scales.view(torch.uint8).view(rows, cols // t.values, 4)
            tables.append(d.StoredTable(raw, t, cols))
        outs = [torch.empty((rows, cols), dtype=torch.bfloat16, device=DEV) for _ in range(n)]
        kernels.append(Kernel(f"dequantize_{name.lower()}_bf16", f"{name} weight [14336,4096] decoded to bf16", nbytes,
                              rows, lambda i, n=n, ts=tables, os_=outs: hip.dequantize(ts[i % n], os_[i % n]), sets=n,
                              read_bytes=rows * row_bytes))
    return kernels


def time_formats(hip: d.HipOps, lib, steps: int, warmup: int) -> dict:
    """--formats: each storage type's decode timed from a graph and against
    its best stream probe in alternation."""
    kernels = format_kernels(hip)
    for k in kernels:
        k.prepare(hip)
    probes = {k.name: ceiling_probes(k, lib) for k in kernels}
    time_graphs(kernels, steps, warmup)
    time_graphs([p for group in probes.values() for p in group], steps, warmup)
    for k in kernels:
        k.ceiling = min(probes[k.name], key=lambda p: p.graph_ms)
    time_matched([[k, k.ceiling] for k in kernels], steps, MATCHED_ROUNDS)
    out = {}
    for k in kernels:
        gbs = k.bytes / (k.launch_ms * 1e-3) / 1e9
        out[k.name] = {"config": k.config, "us": round(k.launch_ms * 1e3, 2),
                       "us_replay": round(k.graph_ms * 1e3, 2), "bytes": k.bytes, "GB_s": round(gbs, 1),
                       "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
                       "probe_us": round(k.ceiling.matched_launch_ms * 1e3, 2),
                       "frac_of_probe_matched": round(k.ceiling.matched_launch_ms / k.matched_launch_ms, 4)}
    for k in kernels:
        k.calls = []
    for group in probes.values():
        for p in group:
            p.buffers = None
    torch.cuda.synchronize()
    return out


def host_cpu() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def host_threads() -> int:
    """Host threads for the all-cores leg: this process's CPUs, at most 16
    (one GPU's share of an 8-GPU node's host cores)."""
    return max(1, min(16, len(os.sched_getaffinity(0))))


def cpu_baseline(kernels, budget_s: float):
    """The oracle (the reference's CPU arithmetic, restated in C) on a bounded
    sample of each kernel's work, scaled to the whole launch: rows are
    independent in every op, so time grows with rows. Two legs: one core, as
    the reference's serial loops run, and the same rows split across the
    host's threads (the oracle's C loops release the GIL)."""
    from oracle import oracle as o

    rng = np.random.default_rng(0)

    def bits(shape):
        return o.to_bf16(rng.standard_normal(shape).astype(np.float32))

    w4096 = (1 + 0.1 * rng.standard_normal(4096)).astype(np.float32)
    w128 = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    sc = (0.1 * rng.standard_normal((1, 3072))).astype(np.float32)
    # the C4 table at its full size, [151936, 4096] (661 MB), so the gather
    # reads rows the host caches do not hold, as the GPU's does: codes random
    # bytes, scales fp16 in [1e-3, 2e-2]
    vocab = 151936
    table = np.frombuffer(rng.bytes(vocab * 128 * 34), np.uint8).reshape(vocab * 128, 34).copy()
    table[:, 0:2] = rng.uniform(1e-3, 2e-2, vocab * 128).astype(np.float16).view(np.uint8).reshape(-1, 2)
    table = table.reshape(vocab, 128 * 34)

    def rms(units):
        x = bits((units, 4096))
        return lambda: o.rms_norm_bf16(x, w4096, 1e-5)

    def swiglu(units):
        g, u = bits((units, 14336)), bits((units, 14336))
        return lambda: o.gated_bf16(0, g, u)

    def rms_q8(units):
        x = rng.standard_normal((units, 4096)).astype(np.float32)
        return lambda: o.quantize_x(o.rms_norm(x, w4096, 1e-5))

    def swiglu_q8(units):
        g, u = rng.standard_normal((units, 14336)).astype(np.float32), rng.standard_normal((units, 14336)).astype(
            np.float32)
        return lambda: o.quantize_x(o.gated(0, g, u))

    def qk(units):
        q, k = bits((units, 32, 128)), bits((units, 8, 128))
        p = np.arange(units, dtype=np.int32)
        return lambda: o.qk_norm_rope_bf16(q, k, w128, w128, p, 1e-6, 0.0, 1e6, 128)

    def attention_inputs(units):
        q, k, v = bits((units, 32, 128)), bits((units, 8, 128)), bits((units, 8, 128))
        p = np.arange(units, dtype=np.int32)
        pages = -(-units // 16)
        keys, values = np.zeros(pages * 16 * 8 * 128, np.uint16), np.zeros(pages * 8 * 128 * 16, np.uint16)
        table = rng.permutation(pages).astype(np.int32)
        return lambda: o.attention_inputs_bf16(q, k, v, w128, w128, 1e-6, 0.0, p, 1e6, 128, keys, values, table, 16,
                                               0, gated=False)

    def gather(units):
        ids = rng.integers(0, vocab, units).astype(np.int32)
        return lambda: o.embedding_q8_0_bf16(table, vocab, 4096, ids)

    def adaln(units):
        x = bits((units, 3072))
        return lambda: o.layer_norm_modulate_bf16(x, sc, sc, units, 1e-6)

    def gelu(units):
        x = bits((units, 3072))
        return lambda: o.activation_bf16(1, x)

    g3072 = (0.5 * rng.standard_normal(3072)).astype(np.float32)

    def gated_add(units):
        x, y = o.from_bf16(bits((units, 3072))), o.from_bf16(bits((units, 3072)))
        return lambda: o.to_bf16(o.gated_add(x, y, g3072))

    def modulate_chunks(units):
        x = o.from_bf16(bits((units, 3072)))
        t = (0.3 * rng.standard_normal((units, 6 * 3072))).astype(np.float32)
        return lambda: o.to_bf16(o.modulate_chunks(x, t, 3, 4))

    def gated_add_chunk(units):
        x, y = o.from_bf16(bits((units, 3072))), o.from_bf16(bits((units, 3072)))
        t = (0.3 * rng.standard_normal((units, 6 * 3072))).astype(np.float32)
        return lambda: o.to_bf16(o.gated_add_chunk(x, y, t, 5))

    def row_gated_add(units):
        x, y = o.from_bf16(bits((units, 128))), o.from_bf16(bits((units, 128)))
        g = rng.random(units).astype(np.float32)
        return lambda: o.to_bf16(o.row_gated_add(x, y, g))

    cos, sin = o.wan_angles(21, 30, 52)  # Wan keeps a grid's tables (models/Wan.scala:324-330)

    def rope3d(units):
        # token i of the 2-sample batch is grid token i mod 32760
        x = o.from_bf16(bits((units, 24, 128)))
        index = np.arange(units) % cos.shape[0]
        c, s = cos[index], sin[index]
        return lambda: o.to_bf16(o.rope_table(x, c, s))

    q4k_table = o.quant_table("Q4_K", 64, 4096, rng)

    def dequantize_q4_k(units):
        table = np.concatenate([q4k_table] * math.ceil(units / 64))[:units]
        return lambda: o.embedding_bf16("Q4_K", table, units, 4096, np.arange(units, dtype=np.int32))

    def rotated(four):
        def make(units):
            r = o.random_rotated(units, 5120, rng, four, 64)
            return lambda: r.dequantize_bf16()
        return make

    work = {}
    for b in (1, 8, 64):
        work[f"rms_norm_bf16_b{b}"] = (rms, b, "rows")
        work[f"swiglu_bf16_b{b}"] = (swiglu, b, "rows")
    for b in (1, 64):
        work[f"rms_norm_q8_f32_b{b}"] = (rms_q8, b, "rows")
        work[f"swiglu_q8_f32_b{b}"] = (swiglu_q8, b, "rows")
    work.update({"qk_norm_rope_bf16": (qk, 4096, "tokens"), "attention_inputs_bf16": (attention_inputs, 4096, "tokens"),
                 "embedding_q8_0_bf16": (gather, 8192, "ids"),
                 "adaln_bf16": (adaln, 65520, "rows"), "gelu_tanh_bf16": (gelu, 65520, "rows"),
                 "rope_3d_bf16": (rope3d, 65520, "tokens"), "gated_add_bf16": (gated_add, 65520, "rows"),
                 "modulate_chunks_bf16": (modulate_chunks, 65520, "rows"),
                 "gated_add_chunk_bf16": (gated_add_chunk, 65520, "rows"),
                 "row_gated_add_bf16": (row_gated_add, 65520 * 24, "head rows"),
                 "dequantize_q4_k_bf16": (dequantize_q4_k, 14336, "rows"),
                 "rotated_dequantize_i8_bf16": (rotated(False), 13824, "rows"),
                 "rotated_dequantize_w4a8_bf16": (rotated(True), 13824, "rows")})
    # Each kernel gets 2/3 of budget_s / (kernels) seconds on one core: a sample of
    # up to the whole launch's units, run once untimed and then again until
    # that time is spent; the per-run time is what scales to the whole
    # launch. The all-cores leg gets the other third.
    target = budget_s * 2 / 3 / max(len(kernels), 1)
    threads = host_threads()
    for k in kernels:
        make, total, unit = work[k.name]
        probe = min(total, 8)
        fn = make(probe)
        t0 = time.perf_counter()
        fn()
        per_unit = (time.perf_counter() - t0) / probe
        units = int(min(total, max(probe, target / 2 / max(per_unit, 1e-9))))
        fn = make(units)
        fn()  # untimed: the first run's fresh output pages fault in
        runs, spent = 0, 0.0
        while runs == 0 or spent < target:
            t0 = time.perf_counter()
            fn()
            spent += time.perf_counter() - t0
            runs += 1
        k.cpu = (f"{units} of {total} {unit}, {runs} runs", spent / runs, units / total)
        del fn
        t = max(1, min(threads, units))
        parts = [make(units // t + (1 if i < units % t else 0)) for i in range(t)]
        with ThreadPoolExecutor(t) as pool:
            for done in [pool.submit(part) for part in parts]:
                done.result()
            runs, spent = 0, 0.0
            while runs == 0 or spent < target / 2:
                t0 = time.perf_counter()
                for done in [pool.submit(part) for part in parts]:
                    done.result()
                spent += time.perf_counter() - t0
                runs += 1
        k.cpu_all = (t, spent / runs)


# ------------------------------------------------------------------ ceilings

def ceiling_probes(k: Kernel, lib) -> list:
    """The probes moving k's read and write bytes with nothing else, over
    buffer sets totalling more than 512 MB like the kernel's: the stream
    probe (drift_stream_mix: 256-thread blocks that only read or only write,
    1, 2 or 4 chunks a lane), the one-wave probe (drift_wave_copy: each
    one-wave block reading its share and then writing its share, 1, 2, 4 or
    8 chunks a lane, the shape most fused kernels take) and the same waves in
    512-thread blocks (drift_block_copy, 1, 2 or 4 chunks a lane). The
    fastest is k's ceiling."""
    reads = -(-k.read_bytes // 16)
    writes = -(-(k.bytes - k.read_bytes) // 16)
    n = sets_for(16 * (reads + writes))
    buffers = [(torch.empty(max(reads, 1) * 16, dtype=torch.uint8, device=DEV).fill_(7),
                torch.empty(writes * 16, dtype=torch.uint8, device=DEV)) for _ in range(n)]
    probes = []
    for entry, shape, lanes, extra in (("drift_stream_mix", "stream_mix", (1, 2, 4), ()),
                                       ("drift_wave_copy", "wave_copy", (1, 2, 4, 8), ()),
                                       ("drift_block_copy", "block_copy_8_waves", (1, 2, 4), (8,))):
        for per in lanes:
            probe = Kernel(f"ceiling of {k.name}", f"{shape}: {reads} chunks read, {writes} written, {per} a lane",
                           16 * (reads + writes), k.rows, None, n, read_bytes=16 * reads)
            probe.per_lane = per
            probe.shape = shape
            probe.buffers = buffers
            for src, dst in buffers:
                probe.calls.append((entry, getattr(lib, entry),
                                    (ctypes.c_void_p(src.data_ptr()), reads, ctypes.c_void_p(dst.data_ptr()), writes,
                                     per) + extra))
            probes.append(probe)
    return probes


def row_probes(k: Kernel, lib) -> list:
    """The gather's own pattern with no decode: each of k's launches (table,
    ids, out, count, vocab, cols, bad_id) becomes, with the same ids and
    outputs, a 256-thread block per id reading the whole Q8_0 row the id
    names and writing the row's BF16 bytes (drift_row_probe), or 1, 2, 4 or
    8 one-wave blocks per id each reading its slice of the row and writing
    its slice of the output (drift_wave_row_probe; the gather itself takes 4
    waves a row). Random rows of a table larger than the cache come from
    scattered DRAM pages, which the contiguous probes do not measure."""
    probes = []
    for slices in (0, 1, 2, 4, 8):
        what = ("a 256-thread block per id" if slices == 0 else f"{slices} one-wave blocks per id")
        probe = Kernel(f"row probe of {k.name}", f"rows of the gather's table read at its ids, its output written: "
                       f"{what}", k.bytes, k.rows, None, k.sets, read_bytes=k.read_bytes)
        probe.slices = slices
        for _, _, (table, ids, out, count, vocab, cols, _) in k.calls:
            row_bytes = cols // 32 * 34
            if row_bytes % 16 or table.value % 16:
                return []
            if slices == 0:
                probe.calls.append(("drift_row_probe", lib.drift_row_probe,
                                    (table, vocab, row_bytes // 16, ids, count, out, cols * 2 // 16)))
            else:
                probe.calls.append(("drift_wave_row_probe", lib.drift_wave_row_probe,
                                    (table, vocab, row_bytes // 16, ids, count, out, cols * 2 // 16, slices)))
        probes.append(probe)
    return probes


def floor_probe(lib) -> Kernel:
    """The per-launch floor of a graph replay: drift_stream_mix writing one
    16-byte chunk (one block of 256 threads) and reading nothing. The decode
    shapes (C2) move tens of kilobytes: their time is this floor plus their
    own dependent chain (loads, a row reduction, the stores)."""
    dsts = [torch.empty(16, dtype=torch.uint8, device=DEV) for _ in range(2)]
    probe = Kernel("launch_floor", "drift_stream_mix writing one 16-byte chunk, nothing read: one block of 256 "
                   "threads", 16, 1, None, 2, read_bytes=0)
    probe.buffers = dsts
    for dst in dsts:
        probe.calls.append(("drift_stream_mix", lib.drift_stream_mix, (None, 0, ctypes.c_void_p(dst.data_ptr()), 1, 1)))
    return probe


def read_probe(lib, gib_bytes: int, blocks: int, name: str) -> Kernel:
    """The reference's streaming read (drift_read_sum_f32x4) over gib_bytes."""
    x = torch.ones(gib_bytes // 4, dtype=torch.float32, device=DEV)
    partials = torch.empty(blocks, dtype=torch.float32, device=DEV)
    probe = Kernel(name, f"read_sum_f32x4 over {gib_bytes >> 20} MiB, {blocks} blocks of 256", gib_bytes, 1, None, 1,
                   read_bytes=gib_bytes)
    probe.buffers = [(x, partials)]
    probe.calls.append(("drift_read_sum_f32x4", lib.drift_read_sum_f32x4,
                        (ctypes.c_void_p(x.data_ptr()), gib_bytes // 16, ctypes.c_void_p(partials.data_ptr()), blocks)))
    return probe


def capture(k: Kernel, first: int, launches: int):
    """A HIP graph of k's launches over buffer sets first, first + 1, ..."""
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        captured = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        for i in range(launches):
            k.fire(first + i, captured)
    return g


def graph_start(floor: Kernel, steps: int, rounds: int = 7) -> float:
    """The fixed start every graph replay pays between the event before it
    and its first launch, in ms: `floor`'s launch (one block writing 16
    bytes) in a graph of `steps` launches and in one of LONG x `steps`,
    replayed back to back after an untimed replay, `rounds` times. A launch
    of it costs the same at every position of a graph, so each round's
    start is (LONG t_K - t_long) / (LONG - 1); the median is returned. The
    kernel trace shows the same gap before every kernel's graph (17.5-18 us
    from one graph's last kernel to the next graph's first, whatever the
    kernels), so one start is subtracted from every kernel's replay."""
    stream = torch.cuda.current_stream()
    here = ctypes.c_void_p(stream.cuda_stream)
    for i in range(2):
        floor.fire(i, here)
    torch.cuda.synchronize()
    short, long = capture(floor, 0, steps), capture(floor, 0, LONG * steps)
    short.replay()
    long.replay()
    torch.cuda.synchronize()
    starts = []
    for _ in range(rounds):
        a, b, c = (torch.cuda.Event(enable_timing=True) for _ in range(3))
        short.replay()
        a.record(stream)
        short.replay()
        b.record(stream)
        long.replay()
        c.record(stream)
        torch.cuda.synchronize()
        starts.append((LONG * a.elapsed_time(b) - b.elapsed_time(c)) / (LONG - 1))
    del short, long
    return max(statistics.median(starts), 0.0)


def time_graphs(kernels, steps: int, warmup: int, rounds: int = 1) -> float:
    """Each kernel's `steps` launches captured in a HIP graph (rotating its
    buffer sets), replayed with one event pair around the replay on the
    replaying stream: the average launch is the span over `steps`, with no
    host call in it. The first round of replays (every kernel once, in
    order) is the timed region: its wall time is returned and each kernel's
    figure in it kept as `step_ms`. Further rounds, after it, replay the same
    graphs in the same order; `graph_ms` is each kernel's median over all
    rounds, so one slow replay does not stand for the kernel."""
    stream = torch.cuda.current_stream()
    here = ctypes.c_void_p(stream.cuda_stream)
    graphs = []
    for k in kernels:
        for i in range(warmup):
            k.fire(i, here)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            captured = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
            for i in range(steps):
                k.fire(warmup + i, captured)
        graphs.append(g)
    torch.cuda.synchronize()
    for g in graphs:
        g.replay()
    torch.cuda.synchronize()
    times = [[] for _ in kernels]
    wall = None
    for r in range(rounds):
        events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in kernels]
        t0 = time.perf_counter()
        for g, (start, end) in zip(graphs, events):
            start.record(stream)
            g.replay()
            end.record(stream)
        torch.cuda.synchronize()
        if r == 0:
            wall = time.perf_counter() - t0
        for j, (start, end) in enumerate(events):
            times[j].append(start.elapsed_time(end) / steps)
    for k, t in zip(kernels, times):
        k.step_ms = t[0]
        k.graph_ms = statistics.median(t)
    del graphs
    return wall


def time_matched(groups, steps: int, rounds: int) -> None:
    """Each group (a kernel, then its probes) replayed from captured graphs in
    turn, `rounds` times, one event pair around each replay: a kernel and its
    probes see the same clocks and memory state, which change from launch to
    launch (a probe's launches at one size fall into two or three
    durations). Sets `matched_ms` on each to its median replay's average
    launch."""
    stream = torch.cuda.current_stream()
    here = ctypes.c_void_p(stream.cuda_stream)
    for group in groups:
        graphs = []
        for k in group:
            for i in range(2):
                k.fire(i, here)
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                captured = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
                for i in range(steps):
                    k.fire(i, captured)
            graphs.append(g)
        for g in graphs:
            g.replay()
        torch.cuda.synchronize()
        events = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in group]
                  for _ in range(rounds)]
        for r in range(rounds):
            for g, (start, end) in zip(graphs, events[r]):
                start.record(stream)
                g.replay()
                end.record(stream)
        torch.cuda.synchronize()
        for j, k in enumerate(group):
            k.matched_ms = statistics.median(events[r][j][0].elapsed_time(events[r][j][1]) for r in range(rounds)) / steps
        del graphs


def time_eager(kernels, steps: int) -> None:
    """The same launches made one by one from Python through ctypes, as a
    caller without graphs makes them: for launches shorter than the host's
    call, the span includes the host."""
    stream = torch.cuda.current_stream()
    here = ctypes.c_void_p(stream.cuda_stream)
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in kernels]
    torch.cuda.synchronize()
    for k, (start, end) in zip(kernels, events):
        start.record(stream)
        for i in range(steps):
            k.fire(i, here)
        end.record(stream)
    torch.cuda.synchronize()
    for k, (start, end) in zip(kernels, events):
        k.eager_ms = start.elapsed_time(end) / steps


def host_call_cost() -> Optional[dict]:
    """Host microseconds per C-ABI call, from drift_amd/host/launch_cost (a
    C++ loop of 1000 calls of each entry point at its benchmark shape)."""
    program = os.path.join(ROOT, "drift_amd", "host", "launch_cost")
    if not os.path.exists(program):
        return None
    done = subprocess.run([program], capture_output=True, text=True, timeout=120)
    if done.returncode != 0:
        raise RuntimeError(f"launch_cost failed: {done.stdout}{done.stderr}")
    return json.loads(done.stdout.strip().splitlines()[-1])


# ------------------------------------------------------------------ main

def main():
    faulthandler.enable()  # a crash in native code prints the Python stack
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--cpu-budget", type=float, default=24.0, help="seconds of CPU reference work, about")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--only", default="", help="comma-separated kernel names to run (profiling)")
    ap.add_argument("--formats", action="store_true",
                    help="also time every storage type's decode to bf16 (outside the step), reported in 'formats'")
    ap.add_argument("--no-graph-start", action="store_true",
                    help="no long graph: the graph start is not measured, per-kernel us is the K-launch replay's span "
                         "over K (for counter passes: rocprofv3 --pmc has ended in a segmentation fault of its own "
                         "thread in an 80-launch graph)")
    ap.add_argument("--no-host", action="store_true",
                    help="skip the host cost per call (a child process that launches kernels of its own: profilers "
                         "tracing this process would trace it too)")
    args = ap.parse_args()
    global START_MS, STEPS
    STEPS = args.steps
    if args.gpus != 1:
        print(f"bench.py: this path runs on one GPU; --gpus {args.gpus} is not supported "
              f"(rows shard across GPUs with no exchange, so N GPUs do N times the work)", file=sys.stderr)
        sys.exit(2)

    torch.cuda.set_device(0)
    lib = _lib.load()
    hip = Prepared()
    kernels = make_kernels(hip)
    if args.only:
        keep = set(args.only.split(","))
        kernels = [k for k in kernels if k.name in keep]
    for k in kernels:
        k.prepare(hip)
    # the ceilings: the stream probe at each long kernel's bytes and mix, and
    # the reference's streaming read over 1 GiB (its 2048 blocks, and one pass)
    probes = {}
    for k in kernels:
        if k.bytes >= (8 << 20):
            probes[k.name] = ceiling_probes(k, lib)
    rows_probes = {}
    for k in kernels:
        if k.name == "embedding_q8_0_bf16":
            p = row_probes(k, lib)
            if p:
                rows_probes[k.name] = p
    reads = [] if args.only else [read_probe(lib, 1 << 30, 2048, "read_sum_1gib_2048_blocks"),
                                  read_probe(lib, 1 << 30, (1 << 30) // 16 // 1024, "read_sum_1gib_one_pass")]
    floors = [] if args.only else [floor_probe(lib)]
    torch.cuda.synchronize()

    # kernels: graph replays (kernel time) and Python-driven launches (what a
    # caller without graphs sees); the probes: graph replays
    # largest first: after an idle gap the clocks take some milliseconds to
    # rise, and a 17 us kernel timed right after the decode kernels' short
    # launches ran 25% slower than the same kernel after a long one
    largest_first = sorted(kernels, key=lambda k: k.bytes, reverse=True)
    wall = time_graphs(largest_first, args.steps, args.warmup, rounds=GRAPH_ROUNDS)
    time_eager(largest_first, args.steps)
    # the fixed start of a graph replay, which every kernel's and probe's
    # replay span carries (taken out of each `us`)
    if not args.no_graph_start:
        START_MS = graph_start(floor_probe(lib), args.steps)
    time_graphs([p for group in probes.values() for p in group] + [p for group in rows_probes.values() for p in group]
                + reads + floors, args.steps, args.warmup)
    ceilings = {}
    for k in kernels:
        if k.name not in probes:
            continue
        best = min(probes[k.name], key=lambda p: p.graph_ms)
        k.ceiling = best
        gbs = best.bytes / (best.launch_ms * 1e-3) / 1e9
        ceilings[k.name] = {"read_bytes": best.read_bytes, "write_bytes": best.bytes - best.read_bytes,
                            "probe": best.shape, "chunks_a_lane": best.per_lane, "us": round(best.launch_ms * 1e3, 2),
                            "us_replay": round(best.graph_ms * 1e3, 2),
                            "GB_s": round(gbs, 1), "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
                            "us_by_probe": {f"{p.shape} {p.per_lane} a lane": round(p.launch_ms * 1e3, 2)
                                            for p in probes[k.name]}}
    # each kernel against its best probe (and the gather against its best row
    # probe) under the same conditions, in alternation
    best_rows = {name: min(group, key=lambda p: p.graph_ms) for name, group in rows_probes.items()}
    groups = [[k, k.ceiling] + ([best_rows[k.name]] if k.name in best_rows else []) for k in kernels
              if k.ceiling is not None]
    time_matched(groups, args.steps, MATCHED_ROUNDS)
    for group in groups:
        k, probe = group[0], group[1]
        matched = {"rounds": MATCHED_ROUNDS, "us": round(k.matched_launch_ms * 1e3, 2),
                   "probe_us": round(probe.matched_launch_ms * 1e3, 2),
                   "frac_of_probe": round(probe.matched_launch_ms / k.matched_launch_ms, 4),
                   "us_replay": round(k.matched_ms * 1e3, 2),
                   "probe_us_replay": round(probe.matched_ms * 1e3, 2)}
        if len(group) > 2:
            matched["row_probe_us"] = round(group[2].matched_launch_ms * 1e3, 2)
            matched["frac_of_row_probe"] = round(group[2].matched_launch_ms / k.matched_launch_ms, 4)
        ceilings[k.name]["matched"] = matched
    for name, group in rows_probes.items():
        p = best_rows[name]
        gbs = p.bytes / (p.launch_ms * 1e-3) / 1e9
        ceilings[name]["row_probe"] = {"us": round(p.launch_ms * 1e3, 2), "GB_s": round(gbs, 1),
                                       "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4), "what": p.config,
                                       "us_by_shape": {("block per id" if q.slices == 0 else f"{q.slices} waves per id"):
                                                       round(q.launch_ms * 1e3, 2) for q in group}}
    for r in reads:
        gbs = r.bytes / (r.launch_ms * 1e-3) / 1e9
        ceilings[r.name] = {"bytes": r.bytes, "us": round(r.launch_ms * 1e3, 2), "GB_s": round(gbs, 1),
                            "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4), "what": r.config}
    for f in floors:
        ceilings[f.name] = {"us": round(f.launch_ms * 1e3, 2), "us_replay": round(f.graph_ms * 1e3, 2),
                            "what": f.config}
    for group in probes.values():
        for p in group:
            p.buffers = None
    for r in reads + floors:
        r.buffers = None
    probes = reads = rows_probes = floors = None
    torch.cuda.synchronize()

    # A plain device copy of one C5 tensor (402.6 MB read + 402.6 MB
    # written) into two destinations in turn: the known-size kernel that
    # rocprofv3's FETCH_SIZE and WRITE_SIZE counts are scaled by.
    stream = torch.cuda.current_stream()
    copy_elems = 65520 * 3072
    src = torch.empty(copy_elems, dtype=torch.bfloat16, device=DEV).fill_(1.0)
    dsts = [torch.empty_like(src) for _ in range(2)]
    for i in range(2):
        dsts[i].copy_(src)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for i in range(10):
        dsts[i % 2].copy_(src)
    end.record(stream)
    torch.cuda.synchronize()
    copy_ms = start.elapsed_time(end) / 10
    copy_gbs = 2 * copy_elems * 2 / (copy_ms * 1e-3) / 1e9
    del src, dsts

    host = None if args.only or args.no_host else host_call_cost()
    formats = time_formats(hip, lib, args.steps, args.warmup) if args.formats else None

    if not args.no_cpu:
        cpu_baseline(kernels, args.cpu_budget)

    step_bytes = sum(k.bytes for k in kernels)
    ms_per_step = wall * 1e3 / args.steps
    table = {}
    for k in kernels:
        avg = k.launch_ms
        gbs = k.bytes / (avg * 1e-3) / 1e9
        table[k.name] = {
            "config": k.config, "us": round(avg * 1e3, 2), "us_replay": round(k.graph_ms * 1e3, 2),
            "us_step": round(k.step_ms * 1e3, 2),
            "us_eager": round(k.eager_ms * 1e3, 2), "bytes": k.bytes,
            "GB_s": round(gbs, 1), "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
            "rows_per_s": round(k.rows / (avg * 1e-3), 1),
        }
        if k.name in ceilings:
            table[k.name]["frac_of_ceiling"] = round(gbs / ceilings[k.name]["GB_s"], 4)
            table[k.name]["frac_of_probe_matched"] = ceilings[k.name]["matched"]["frac_of_probe"]
            if "row_probe" in ceilings[k.name]:
                table[k.name]["frac_of_row_probe"] = round(gbs / ceilings[k.name]["row_probe"]["GB_s"], 4)
    # the roofline kernel's launches as the timed step replayed them
    dominant = max(kernels, key=lambda k: k.graph_ms)
    dom_avg = dominant.step_ms
    achieved = dominant.bytes / (dom_avg * 1e-3) / 1e9
    # HBM bytes per launch are not measured in this run (counters need a
    # profiler pass of their own): they come from the committed counter
    # passes, and the line says which
    traffic = traffic_source = None
    traffic_file = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(traffic_file):
        with open(traffic_file) as f:
            counted = json.load(f)
        traffic = counted.get(dominant.name)
        traffic_source = (f"profiles/traffic.json: {counted.get('_how', 'rocprofv3 FETCH_SIZE and WRITE_SIZE passes')}"
                          f" ({counted.get('_date', 'date not recorded')}), not this run")
    line = {
        "metric": "achieved HBM GB/s and % of MI355X peak per fused kernel; rows/sec at 1 GPU",
        "value": round(step_bytes / (ms_per_step * 1e-3) / 1e9, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded device generators), resident in HBM; buffer sets rotated past the 256 MB MALL",
        "config": {
            "workload": "drift fused layer kernels, one pass over C2 (decode B=1,8,64; F32 with int8 side output "
                        "B=1,64), C3 (prefill QK norm+RoPE, and with the paged KV-cache write), C4 (Q8_0 gather), "
                        "C5 (Video DiT AdaLN, GELU-tanh, 3-D RoPE, gated residuals, per-row modulation), and "
                        "weights decoded to bf16 (Q4_K [14336,4096]; ConvRot int8 and 4-bit [13824,5120])",
            "step_bytes": step_bytes,
            "parallelism": "single GPU",
            "timing": "each kernel's K launches replayed from a captured HIP graph, one event pair per kernel "
                      "(the timed step, value); per-kernel us: the median replay's span over K less graph_start_us / K",
        },
        "graph_start_us": {"us": round(START_MS * 1e3, 2),
                           "what": "the fixed start of a graph replay, between the event before it and its first "
                                   "launch: a one-block launch in graphs of K and 4K launches, median of 7 pairs; "
                                   "each kernel's and probe's us is its K-launch replay's span less this, over K"},
        "kernels": table,
        "ceilings": ceilings,
        "formats": formats,
        "hbm_copy_reference": {"GB_s": round(copy_gbs, 1), "frac_hbm_peak": round(copy_gbs / HBM_PEAK_GBS, 4),
                               "what": "torch copy_ of 402.6 MB (read + write)"},
        "host_us_per_call": host,
        "roofline": {
            "kernel": dominant.name, "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
            "traffic_source": traffic_source,
            "algorithmic_bytes_per_launch": dominant.bytes, "avg_launch_us": round(dom_avg * 1e3, 2),
        },
    }
    if not args.no_cpu and all(k.cpu and k.cpu_all for k in kernels):
        one_core_s = sum(k.cpu[1] / k.cpu[2] for k in kernels)
        all_cores_s = sum(k.cpu_all[1] / k.cpu[2] for k in kernels)
        line["cpu_baseline"] = {
            "value": round(step_bytes / all_cores_s / 1e9, 4), "unit": "GB/s", "cores": host_threads(),
            "kind": "port",
            "sample": "each kernel timed on a sample of its rows (the C4 ids gather from a full-size "
                      "[151936, 4096] table) and scaled to the whole launch: "
                      + "; ".join(f"{k.name}: {k.cpu[0]}, {k.cpu[1]:.4f} s a run on 1 core, "
                                  f"{k.cpu_all[1]:.4f} s on {k.cpu_all[0]}" for k in kernels),
            "step_seconds": round(all_cores_s, 3),
            "single_core": {"value": round(step_bytes / one_core_s / 1e9, 4), "cores": 1,
                            "step_seconds": round(one_core_s, 2)},
            "host": f"{host_cpu()}, {os.cpu_count()} CPUs visible, {host_threads()} used",
        }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
