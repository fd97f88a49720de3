"""Exact visible-token counts on every benchmarked shape, through the C ABI.

With q = k = 0 every visible key gets the same weight, so (definitions of
src/portable_gpu_ops.cpp:30-31; known-answer pattern of
tests/ascend_ops_tests.cpp:21,44):
  * LSE = ln(n) exactly up to the last fp32 rounding, n = visible keys of the
    row (end-aligned causal: len - qlen + i + 1; non-causal: len).  One key
    dropped or added moves LSE by ~1/n, 3e-5 at n = 32768: the 1e-5 bound
    pins n exactly on every split boundary and last partial block.
  * out = mean of the visible V rows.  V of token t, kv head g is the one-hot
    vector e_{(t + 7g) mod 128}, so out[d] = (#visible t with t = d - 7g
    mod 128) / n: the residue counts show which tokens were read, not only
    how many.  Slots past a sequence's end and the dummy page hold ones in
    every dim, so a stale read moves every element.
fp16 runs compare out at 2e-3 relative (a missing key moves one element by
128/n >= 3.9e-3 at n = 32768); bf16 runs at the attention tolerance 1e-2.
"""

import math

import numpy as np
import pytest
import torch

import feattn
from feattn import workloads as W

pytestmark = pytest.mark.gpu
LSE_EXACT = 1e-5


def visible_counts(b, causal):
    """n per query row (int64 [rows])."""
    n = np.zeros(b.rows, dtype=np.int64)
    for s in range(b.batch):
        L, ln = b.qlens[s], b.lens[s]
        i = np.arange(L)
        n[b.qo[s]:b.qo[s + 1]] = (ln - L + i + 1) if causal else ln
    return n


def residue_v_cache(b, dtype):
    """V cache: token t of every sequence, kv head g -> one-hot at (t + 7g) % 128;
    every other slot (stale tail of the last page, unused and dummy pages) all ones."""
    vc = np.ones((b.cache_slots, b.hkv, 128), dtype=np.float16)  # 0 and 1 are exact in both 16-bit types
    g = np.arange(b.hkv)
    for s in range(b.batch):
        ln = b.lens[s]
        t = np.arange(ln)
        table = np.asarray(b.tables[s], dtype=np.int64)
        slot = table[t // b.page] * b.page + t % b.page
        vc[slot] = 0.0
        d = (t[:, None] + 7 * g[None, :]) % 128
        vc[slot[:, None], g[None, :], d] = 1.0
    return torch.from_numpy(vc.reshape(b.blocks + 1, b.page, b.hkv, 128)).to(dtype)


def expected_out(b, n, rows):
    """out[r, h, d] for the chosen rows (float64 [len(rows), hq, 128])."""
    G = b.group
    h = np.arange(b.hq)
    d = np.arange(128)
    r = (d[None, :] - 7 * (h[:, None] // G)) % 128          # [hq, 128] first token of the class
    nn = n[rows][:, None, None]
    cnt = np.where(r[None] < nn, (nn - 1 - r[None]) // 128 + 1, 0)
    return cnt / nn


def run_case(dev, b, causal, dtype, plan_pages=None):
    dt = torch.bfloat16 if dtype == "bf16" else torch.float16
    q = torch.zeros(b.rows, b.hq, 128, dtype=dt, device=dev)
    kc = torch.zeros(b.blocks + 1, b.page, b.hkv, 128, dtype=dt, device=dev)
    vc = residue_v_cache(b, dt).to(dev)
    plan = feattn.Plan(b.hq, b.hkv, 128, b.page, b.batch, plan_pages or b.max_pages(), dt == torch.bfloat16,
                       b.blocks)
    plan.prepare(b.qo, b.kv, b.pages, b.last, b.batch, b.rows)
    out = torch.full_like(q, float("nan"))
    lse = torch.full((b.rows, b.hq), float("nan"), device=dev)
    plan.run(q, kc, vc, out, causal=causal, lse=lse)
    torch.cuda.synchronize()
    plan.close()
    n = visible_counts(b, causal)
    want_lse = torch.from_numpy(np.log(n.astype(np.float64))).float()[:, None].expand(b.rows, b.hq)
    lse = lse.cpu()
    err_lse = (lse - want_lse).abs().max().item()
    assert err_lse <= LSE_EXACT, f"LSE off by {err_lse:.3g} (count pin 1e-5)"
    # out: every row for small batches, a strided sample of up to 2048 rows otherwise
    rows = np.arange(b.rows) if b.rows <= 2048 else np.unique(np.linspace(0, b.rows - 1, 2048).astype(np.int64))
    got = out.cpu()[torch.from_numpy(rows)].double().numpy()
    want = expected_out(b, n, rows)
    rtol = 2e-3 if dtype == "f16" else 1e-2
    bad = np.abs(got - want) > rtol * want + 1e-6
    assert not bad.any(), f"{int(bad.sum())} out elements off, first at {np.argwhere(bad)[0].tolist()}"
    return err_lse


SHAPES = {
    "decode8b": (lambda: W.qwen3_8b_decode(), True),
    "long16x32k": (lambda: W.long_decode(), True),
    "prefill8b": (lambda: W.qwen3_8b_prefill(), True),
    "dflash": (lambda: W.dflash_block(), False),
    "mixed30b": (lambda: W.qwen3_30b_mixed(), True),
}


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("name", list(SHAPES))
def test_exact_counts_full_shapes(dev, name, dtype):
    make, causal = SHAPES[name]
    b = make()
    run_case(dev, b, causal, dtype)


@pytest.mark.parametrize("causal", [True, False])
def test_exact_counts_prefill_chunks_non_causal_and_causal(dev, causal):
    """Chunks and verify rows with both masks: every chunk boundary against
    the 64-token tile and 16-token page grids."""
    b = W.make_batch(32, 8, starts=[0, 15, 16, 17, 63, 64, 65, 1000, 2047],
                     qlens=[1, 2, 3, 64, 65, 127, 129, 300, 33], seed=77, extra_pages=2)
    run_case(dev, b, causal, "f16")


@pytest.mark.parametrize("hq,hkv", [(16, 2), (24, 6), (40, 8), (8, 8), (24, 8), (48, 8), (128, 8), (64, 2),
                                    (128, 1), (32, 16), (64, 16), (32, 32)])
def test_exact_counts_head_layouts(dev, hq, hkv):
    """Head layouts whose decode workgroups hold 2 or 1 wavefronts (hkv = 2,
    6, 1), decode shares held by two or four workgroups of 8 wavefronts
    (hkv = 16, 32), non-power-of-two groups (3, 5, 6) and groups of 16 to
    128 query heads per kv head (a row alone fills a decode or a tile item),
    decode and chunk rows mixed."""
    b = W.make_batch(hq, hkv, starts=[4095, 0, 777, 5000, 31], qlens=[1, 1, 1, 2, 90], seed=hq + hkv,
                     extra_pages=1)
    run_case(dev, b, True, "f16")


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("hq,hkv", [(32, 8), (32, 4), (24, 6)])
def test_exact_counts_short_blocks(dev, causal, hq, hkv):
    """Blocks of rows just past the decode kernel's 32 columns per kv head
    (one to two decode widths: DFlash and verify blocks, on the tile kernel),
    with both masks, next to single decode rows and a longer chunk."""
    G = hq // hkv
    rmax = 32 // G
    b = W.make_batch(hq, hkv, starts=[5000, 900, 3000, 17, 40, 12000, 100],
                     qlens=[1, rmax + 1, 2 * rmax, 2 * rmax, 1, rmax + 2, 300], seed=hq * hkv,
                     extra_pages=2)
    run_case(dev, b, causal, "f16")


@pytest.mark.parametrize("page", [32, 64, 128])
@pytest.mark.parametrize("causal", [True, False])
def test_exact_counts_page_sizes(dev, page, causal):
    """Larger pages: lengths ending just before, on and just after page
    boundaries, decode rows and chunks, so every page-index shift and the
    last partial page are pinned exactly."""
    b = W.make_batch(32, 8, starts=[page - 2, page - 1, page, 3 * page + 1, 5000, 700],
                     qlens=[1, 1, 1, 2, 1, 100], seed=page, page=page, extra_pages=2)
    run_case(dev, b, causal, "f16")


def test_counts_single_128k_sequence(dev):
    """One 131072-token decode row (and a 6-token one) spread over every
    decode share: about 256 pieces whose partials one merge folds in 32
    batches of 8.  At n = 131072 a single token moves LSE by 7.6e-6, under
    the 1e-5 bound, so this pins the count to within a token (and any lost
    or doubled piece by far)."""
    b = W.make_batch(32, 8, starts=[131071, 5], qlens=[1, 1], seed=128, extra_pages=1)
    counts = feattn.describe(b.hq, b.hkv, 128, b.page, b.batch, b.max_pages(), b.blocks, b.qo, b.kv,
                             b.pages, b.last, b.batch, b.rows)
    assert counts[3] >= 128  # the long row is cut into that many partial rows at least
    run_case(dev, b, True, "f16")


@pytest.mark.parametrize("causal", [True, False])
def test_exact_counts_long_chunks(dev, causal):
    """An 8192-row chunk from an empty cache (row i sees exactly i + 1 keys
    when causal) beside a 2048-row chunk over a 3000-token prefix: diagonal
    tiles, splits and merges across many tile items."""
    b = W.make_batch(32, 8, starts=[0, 3000], qlens=[8192, 2048], seed=81, extra_pages=1)
    run_case(dev, b, causal, "f16")


# Batches whose tile work is the equal cut of the tile stream (the
# longest-first list would split their chunks): one- and two-block chunks
# over long prefixes, 5, 4 and 16 kv heads, one query head per kv head, one
# kv head for 128 query heads (a chunk is one row), and 16-row blocks; every
# piece boundary falls inside a chunk.
STREAM_CUT = {
    "chunks_32_8": (32, 8, [6000, 9000, 300], [200, 64, 40]),
    "chunks_40_5": (40, 5, [7000, 2500, 12000], [48, 20, 33]),
    "chunks_8_8": (8, 8, [9000, 4000], [300, 130]),
    "chunks_32_16": (32, 16, [10000, 3000, 5000], [100, 70, 17]),
    "blocks_32_8": (32, 8, [3000, 7000, 11000, 1500, 9000, 5000], [16] * 6),
    "rows_128_1": (128, 1, [9000, 3000], [40, 20]),
    "chunks_64_4": (64, 4, [12000, 800], [50, 30]),
}


def stream_cut_taken(b, causal):
    """True when the tile list is laid out as the equal cut: kv heads in
    runs 0..hkv-1 repeating, kv head 0's pieces following the tile stream,
    and some chunk cut into consecutive pieces."""
    items = [it for it in feattn.dump(b.hq, b.hkv, 128, b.page, b.batch, b.max_pages(), b.blocks, b.qo, b.kv,
                                      b.pages, b.last, b.batch, b.rows, causal) if it[0] == 1]
    heads = [it[4] for i, it in enumerate(items) if i == 0 or it[4] != items[i - 1][4]]
    if heads != list(range(b.hkv)) * (len(heads) // b.hkv):
        return False
    k0 = [it for it in items if it[4] == 0]
    if not any((a[1], a[2]) == (c[1], c[2]) for a, c in zip(k0, k0[1:])):
        return False
    return all((c[1], c[2], c[5]) == ((a[1], a[2], a[6]) if a[6] < c[6] and (a[1], a[2]) == (c[1], c[2])
                                      else (c[1], c[2], 0)) for a, c in zip(k0, k0[1:]))


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("name", list(STREAM_CUT))
def test_exact_counts_tile_stream_cut(dev, name, causal):
    hq, hkv, starts, qlens = STREAM_CUT[name]
    b = W.make_batch(hq, hkv, starts=starts, qlens=qlens, seed=hq + hkv + 5, extra_pages=1)
    assert stream_cut_taken(b, causal)
    run_case(dev, b, causal, "f16")
