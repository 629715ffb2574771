"""The benchmark configurations at full size (decode C2, prefill C3, gather C4,
Video DiT C5), made on the device from seeded generators, and every value
of every output compared with the oracle. Rows are independent in every one
of these ops, so the oracle runs over contiguous ranges of rows on threads
(its C loops release the GIL): a few seconds for the largest output."""

from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest
import torch

from drift_amd import ops as d
from oracle import oracle as o
from tests.helpers import DEV, assert_bf16, assert_bits, host_bits, step

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hip():
    return d.HipOps()


def device_bf16(shape, seed, scale=1.0):
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    return (scale * torch.randn(shape, generator=g, device=DEV)).to(torch.bfloat16)


def by_ranges(check, first, end, parts=16):
    """check(lo, hi) over `parts` contiguous ranges of [first, end) on
    threads; a failing range raises."""
    bounds = np.linspace(first, end, parts + 1).astype(np.int64)
    with ThreadPoolExecutor(parts) as pool:
        for done in [pool.submit(check, int(lo), int(hi)) for lo, hi in zip(bounds[:-1], bounds[1:]) if hi > lo]:
            done.result()


def test_c2_decode_rms_norm_and_swiglu(hip):
    for batch in (1, 8, 64):
        step(f"C2 rmsNorm bf16 [{batch}, 4096] eps 1e-5")
        x = device_bf16((batch, 4096), 100 + batch)
        w = (1 + 0.1 * torch.randn(4096, generator=torch.Generator().manual_seed(batch))).float()
        out = torch.empty_like(x)
        hip.rmsNorm(x, w.to(DEV), 1e-5, 0.0, out)
        assert_bf16(o.rms_norm_bf16(host_bits(x), w.numpy(), 1e-5), host_bits(out), what="C2 rmsNorm")
        step(f"C2 SwiGLU bf16 [{batch}, 14336]")
        g, u = device_bf16((batch, 14336), 200 + batch), device_bf16((batch, 14336), 300 + batch)
        s = torch.empty_like(g)
        hip.gated(d.Activation.Silu, g, u, s)
        assert_bf16(o.gated_bf16(0, host_bits(g), host_bits(u)), host_bits(s), what="C2 SwiGLU")


def test_c3_prefill_query_key_norm_rope(hip):
    step("C3 queryKeyNormRope bf16 Q[4096, 32, 128] K[4096, 8, 128] theta 1e6 eps 1e-6")
    q, k = device_bf16((4096, 32, 128), 1), device_bf16((4096, 8, 128), 2)
    gen = torch.Generator().manual_seed(3)
    qw = (1 + 0.1 * torch.randn(128, generator=gen)).float()
    kw = (1 + 0.1 * torch.randn(128, generator=gen)).float()
    positions = torch.arange(4096, dtype=torch.int32, device=DEV)
    rope = d.Rope(1e6, 128, d.RopeLayout.Neox)
    rq, rk = torch.empty_like(q), torch.empty_like(k)
    hip.queryKeyNormRope(q, k, d.QueryKeyNorms(qw.to(DEV), kw.to(DEV), 1e-6, 0.0, rope), positions, rq, rk)
    qh, kh, gq, gk = host_bits(q), host_bits(k), host_bits(rq), host_bits(rk)
    tokens = np.arange(4096, dtype=np.int32)

    def check(lo, hi):
        wq, wk = o.qk_norm_rope_bf16(qh[lo:hi], kh[lo:hi], qw.numpy(), kw.numpy(), tokens[lo:hi], 1e-6, 0.0, 1e6, 128)
        assert_bf16(wq, gq[lo:hi], what=f"C3 queries of tokens {lo}..{hi}")
        assert_bf16(wk, gk[lo:hi], what=f"C3 keys of tokens {lo}..{hi}")

    by_ranges(check, 0, 4096)


def test_c4_q8_0_gather_full_table(hip):
    vocab, cols, count = 151936, 4096, 8192
    step(f"C4 Q8_0 table [{vocab}, {cols}] on device, gather {count} ids to bf16")
    g = torch.Generator(device=DEV)
    g.manual_seed(5)
    data = torch.empty((vocab, cols // 32, 34), dtype=torch.uint8, device=DEV)
    data[:, :, 2:] = torch.randint(-127, 128, (vocab, cols // 32, 32), generator=g, device=DEV,
                                   dtype=torch.int32).to(torch.int8).view(torch.uint8)
    scales = (1e-3 + (2e-2 - 1e-3) * torch.rand((vocab, cols // 32), generator=g, device=DEV)).half()
    data[:, :, 0:2] = scales.view(torch.uint8).view(vocab, cols // 32, 2)
    table = d.Q8_0Table(data.view(vocab, cols // 32 * 34), cols)
    ids = torch.randint(0, vocab, (count,), generator=g, device=DEV, dtype=torch.int32)
    out = torch.empty((count, cols), dtype=torch.bfloat16, device=DEV)
    hip.embedding(table, ids, out)
    # the table's rows the ids name, in id order, then every output row
    all_ids = ids.cpu().numpy()
    unique = np.unique(all_ids)
    sub = table.data[torch.from_numpy(unique).to(DEV).long()].cpu().numpy()
    local = np.searchsorted(unique, all_ids).astype(np.int32)
    got = host_bits(out)

    def check(lo, hi):
        assert_bits(o.embedding_q8_0_bf16(sub, unique.size, cols, local[lo:hi]), got[lo:hi], what=f"C4 rows {lo}..{hi}")

    by_ranges(check, 0, count)


def test_c5_dit_block(hip):
    rows, cols, per = 2 * 32760, 3072, 32760
    step("C5 AdaLN bf16 [65520, 3072] eps 1e-6 with per-sample shift/scale [2, 3072]")
    x = device_bf16((rows, cols), 7)
    gen = torch.Generator().manual_seed(8)
    shift = (0.1 * torch.randn((2, cols), generator=gen)).float()
    scale = (0.1 * torch.randn((2, cols), generator=gen)).float()
    out = torch.empty_like(x)
    hip.layerNormModulate(x, scale.to(DEV), shift.to(DEV), 1e-6, out, per)
    xs, got = host_bits(x), host_bits(out)
    del x
    # every row against the oracle with its own sample's shift and scale
    for sample in (0, 1):
        def check(lo, hi, s=sample):
            want = o.layer_norm_modulate_bf16(xs[lo:hi], scale.numpy()[s], shift.numpy()[s], hi - lo, 1e-6)
            assert_bf16(want, got[lo:hi], what=f"C5 AdaLN rows {lo}..{hi}")

        by_ranges(check, sample * per, (sample + 1) * per)
    del xs
    step("C5 GELU-tanh bf16 in place [65520, 3072]")
    hip.activation(d.Activation.GeluTanh, out, out)
    after = host_bits(out)
    del out

    def check_gelu(lo, hi):
        assert_bf16(o.activation_bf16(1, got[lo:hi]), after[lo:hi], what=f"C5 GELU rows {lo}..{hi}")

    by_ranges(check_gelu, 0, rows)
    del got, after
    step("C5 3-D RoPE bf16 Q[65520, 24, 128] on the 21 x 30 x 52 grid")
    qx = device_bf16((rows, 24, 128), 10)
    rq = torch.empty_like(qx)
    hip.rope3d(qx, 21, 30, 52, rq)
    qh, gr = host_bits(qx), host_bits(rq)

    def check_rope(lo, hi):
        want = o.rope_3d_bf16(qh[lo:hi], 21, 30, 52, token_offset=lo)
        assert_bf16(want, gr[lo:hi], what=f"C5 rope tokens {lo}..{hi}")

    by_ranges(check_rope, 0, rows)
