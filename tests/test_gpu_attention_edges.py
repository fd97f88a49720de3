"""GPU edge cases of fe_attn_run against the oracle: page sizes other than
16, page-boundary lengths (len 1, len = page, len = page + 1, a chunk with no
prefix), an empty batch, stale or poisoned cache slots outside every visible
range (they must not leak into results: the reference kernel reads only
visible tokens), plan capacity limits, and scores far outside the range of
an exponential (a dominant first token, scores rising or falling by ~10 in
log2 units every 48 tokens, natural-log LSE up to ~300).  Tolerance as in
test_gpu_attention.py: |a-b| <= 1e-2 + 1e-2*|b|, LSE within 1e-3."""

import math

import pytest
import torch

import feattn
from feattn import workloads as W
from test_gpu_known_counts import stream_cut_taken
from oracle import aten_attention as A

pytestmark = pytest.mark.gpu


def run(b, q, kc, vc, causal, dev, max_pages=None):
    plan = feattn.Plan(b.hq, b.hkv, 128, b.page, max(1, b.batch), max_pages or b.max_pages(),
                       q.dtype == torch.bfloat16, b.blocks)
    plan.prepare(b.qo, b.kv, b.pages, b.last, b.batch, b.rows)
    qd, kd, vd = q.to(dev), kc.to(dev), vc.to(dev)
    out = torch.zeros_like(qd)
    lse = torch.full((b.rows, b.hq), float("nan"), device=dev)
    plan.run(qd, kd, vd, out, causal=causal, lse=lse)
    torch.cuda.synchronize()
    plan.close()
    return out.cpu(), lse.cpu()


def check(out, lse, want_out, want_lse):
    torch.testing.assert_close(out.float(), want_out.float(), atol=1e-2, rtol=1e-2)
    torch.testing.assert_close(lse, want_lse, atol=1e-3, rtol=0)


@pytest.mark.parametrize("page", [32, 64, 256])
@pytest.mark.parametrize("causal", [True, False])
def test_page_sizes(dev, page, causal):
    b = W.make_batch(32, 8, starts=[page - 1, page, 3 * page + 5, 0, 2 * page - 3],
                     qlens=[1, 1, 40, page + 3, 4], seed=page, extra_pages=2)
    q, kc, vc = W.make_tensors(b, seed=page)
    out, lse = run(b, q, kc, vc, causal, dev)
    want_out, want_lse = A.run(b, q, kc, vc, causal)
    check(out, lse, want_out, want_lse)


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_page_boundary_lengths(dev, dtype):
    """len 1, len = page, len = page + 1, a 16-row chunk with no prefix, a
    chunk ending exactly on a page boundary, one 64-token tile exactly."""
    b = W.make_batch(32, 8, starts=[0, 15, 16, 0, 16, 63, 0], qlens=[1, 1, 1, 16, 16, 1, 64], seed=5)
    q, kc, vc = W.make_tensors(b, seed=5, dtype=dtype)
    for causal in (True, False):
        out, lse = run(b, q, kc, vc, causal, dev)
        want_out, want_lse = A.run(b, q, kc, vc, causal)
        check(out, lse, want_out, want_lse)
    # a single visible token: softmax weight 1, out = v, lse = scaled score
    r = b.qo[0]
    v0 = vc[b.tables[0][0], 0].float().repeat_interleave(4, 0)
    out, lse = run(b, q, kc, vc, True, dev)
    torch.testing.assert_close(out[r].float(), v0, atol=1e-2, rtol=1e-2)
    k0 = kc[b.tables[0][0], 0].float().repeat_interleave(4, 0)
    want_lse0 = (q[r].float() * k0).sum(-1) / math.sqrt(128)
    torch.testing.assert_close(lse[r], want_lse0, atol=1e-3, rtol=0)


def test_empty_batch_is_a_no_op(dev):
    plan = feattn.Plan(32, 8, 128, 16, 4, 8, True, 16)
    plan.prepare([0], [0], [], [], 0, 0)
    q = torch.zeros(1, 32, 128, dtype=torch.bfloat16, device=dev)
    kc = torch.zeros(17, 16, 8, 128, dtype=torch.bfloat16, device=dev)
    out = torch.full_like(q, 7.0)
    plan.run(q, kc, kc, out, causal=True)
    torch.cuda.synchronize()
    assert (out == 7.0).all()
    plan.close()


@pytest.mark.parametrize("causal", [True, False])
def test_stale_slots_do_not_leak(dev, causal):
    """Every cache slot outside the visible ranges (the rest of each last
    page, unused pool pages, the dummy page) holds NaN; the results must be
    those of a cache holding zeros there."""
    b = W.make_batch(32, 8, starts=[700, 5, 33, 0, 2000], qlens=[1, 3, 50, 20, 16], seed=9, extra_pages=6)
    q, kc, vc = W.make_tensors(b, seed=9)
    live = torch.zeros(b.blocks + 1, b.page, dtype=torch.bool)
    for s in range(b.batch):
        for t in range(b.lens[s]):
            live[b.tables[s][t // b.page], t % b.page] = True
    kz, vz = kc.clone(), vc.clone()
    kz[~live] = 0
    vz[~live] = 0
    kn, vn = kc.clone(), vc.clone()
    kn[~live] = float("nan")
    vn[~live] = float("nan")
    out, lse = run(b, q, kn, vn, causal, dev)
    assert torch.isfinite(out.float()).all() and torch.isfinite(lse).all()
    want_out, want_lse = A.run(b, q, kz, vz, causal)
    check(out, lse, want_out, want_lse)


def test_capacity_limits(dev):
    """max_batch sequences at the longest context the plan admits
    ((max_pages - 1) * page tokens) run; one token more is refused."""
    max_pages = 9
    ctx = (max_pages - 1) * 16
    b = W.make_batch(32, 8, starts=[ctx - 1] * 3, qlens=[1] * 3, seed=2)
    q, kc, vc = W.make_tensors(b, seed=2)
    out, lse = run(b, q, kc, vc, True, dev, max_pages=max_pages)
    want_out, want_lse = A.run(b, q, kc, vc, True, max_pages=max_pages)
    check(out, lse, want_out, want_lse)
    plan = feattn.Plan(32, 8, 128, 16, 3, max_pages, True, b.blocks)
    too_long = W.make_batch(32, 8, starts=[ctx] * 3, qlens=[1] * 3, seed=2)
    with pytest.raises(RuntimeError):
        plan.prepare(too_long.qo, too_long.kv, too_long.pages, too_long.last, 3, 3)
    four = W.make_batch(32, 8, starts=[10] * 4, qlens=[1] * 4, seed=2)
    with pytest.raises(RuntimeError):
        plan.prepare(four.qo, four.kv, four.pages, four.last, 4, 4)
    plan.close()



@pytest.mark.parametrize("hq,hkv,starts,qlens", [
    # 4 query heads per kv head: 16-row blocks (64 columns) beside narrow rows
    (32, 8, [3000, 40, 700, 5000, 16], [16, 1, 9, 12, 3]),
    # 8 per kv head, 3 kv heads: 64-, 40-, 8- and 56-column items
    (24, 3, [2000, 100, 900, 17], [8, 5, 1, 7]),
    # one kv head with 64 query heads: a single row is 64 columns
    (64, 1, [4000, 33, 1500], [1, 1, 1]),
])
@pytest.mark.parametrize("causal", [True, False])
def test_many_columns_per_kv_head(dev, hq, hkv, starts, qlens, causal):
    """(row, head) column counts per kv head around the decode kernel's
    limit of 32: 33..64-column items run as tile items beside decode items,
    with an odd kv head count and with a single kv head."""
    b = W.make_batch(hq, hkv, starts=starts, qlens=qlens, seed=hq + hkv, extra_pages=1)
    q, kc, vc = W.make_tensors(b, seed=hq)
    out, lse = run(b, q, kc, vc, causal, dev)
    want_out, want_lse = A.run(b, q, kc, vc, causal)
    check(out, lse, want_out, want_lse)


def test_graph_keeps_captured_decode_variant(dev):
    """A graph captured on 8-row verify items (32 columns per kv head: the
    two-block decode variant) replays single rows correctly and refuses
    16-row blocks (tile work, which the captured decode-only step does not
    launch); a graph captured on single rows refuses 8-row items afterwards
    (reference refusal of layout changes: src/flashinfer_attention.cu:32)."""
    hq, hkv, blocks = 32, 8, 700
    kc = torch.zeros(blocks + 1, 16, hkv, 128, dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    q = torch.zeros(64, hq, 128, dtype=torch.bfloat16, device=dev)
    out = torch.zeros_like(q)
    lse = torch.zeros(64, hq, device=dev)
    plan = feattn.Plan(hq, hkv, 128, 16, 4, 200, True, blocks)

    def load(bb, seed):
        qq, kk, vv = W.make_tensors(bb, seed=seed)
        kc.copy_(kk.to(dev))
        vc.copy_(vv.to(dev))
        q.zero_()
        q[:bb.rows].copy_(qq.to(dev))
        plan.prepare(bb.qo, bb.kv, bb.pages, bb.last, bb.batch, bb.rows, graph=True)
        return qq, kk, vv

    verify = W.make_batch(hq, hkv, starts=[900, 2000, 40, 1200], qlens=[8] * 4, seed=1, pool=blocks)
    load(verify, 1)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        plan.run(q, kc, vc, out, causal=True, lse=lse)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        plan.run(q, kc, vc, out, causal=True, lse=lse)
    steps = [W.make_batch(hq, hkv, starts=[3000, 5, 700, 1800], qlens=[1] * 4, seed=2, pool=blocks), verify]
    for seed, bb in enumerate(steps, start=2):
        qq, kk, vv = load(bb, seed)
        graph.replay()
        torch.cuda.synchronize()
        want_out, want_lse = A.run(bb, qq, kk, vv, True)
        check(out[:bb.rows].cpu(), lse[:bb.rows].cpu(), want_out, want_lse)
    blocks16 = W.make_batch(hq, hkv, starts=[300, 1500, 60, 2500], qlens=[16] * 4, seed=3, pool=blocks)
    with pytest.raises(RuntimeError):
        plan.prepare(blocks16.qo, blocks16.kv, blocks16.pages, blocks16.last, blocks16.batch, blocks16.rows,
                     graph=True)
    plan.close()

    narrow = feattn.Plan(hq, hkv, 128, 16, 4, 200, True, blocks)
    one = W.make_batch(hq, hkv, starts=[30, 60], qlens=[1, 1], seed=4, pool=blocks)
    narrow.prepare(one.qo, one.kv, one.pages, one.last, one.batch, one.rows, graph=True)
    with pytest.raises(RuntimeError):
        narrow.prepare(verify.qo, verify.kv, verify.pages, verify.last, verify.batch, verify.rows, graph=True)
    narrow.close()


@pytest.mark.parametrize("hq,hkv,qlen", [(32, 8, 16), (32, 8, 11), (32, 4, 8), (64, 8, 8)])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_block_items_vs_oracle(dev, hq, hkv, qlen, causal, dtype):
    """33..64-column items (16-row DFlash blocks, 8-row items with 8 heads per
    kv head) beside single rows, over a split 20000-token context, a block
    that is its whole context and short ones."""
    b = W.make_batch(hq, hkv, starts=[20000, 3000, 16, 700, 0], qlens=[qlen, qlen, qlen, 1, qlen],
                     seed=qlen + hkv, extra_pages=1)
    q, kc, vc = W.make_tensors(b, seed=qlen, dtype=dtype)
    out, lse = run(b, q, kc, vc, causal, dev)
    want_out, want_lse = A.run(b, q, kc, vc, causal)
    check(out, lse, want_out, want_lse)


def test_graph_captured_on_blocks(dev):
    """A graph captured on 16-row blocks (tile work, no decode rows) replays
    other block batches and single-row batches, each matching the oracle,
    and refuses 8-row items, which need the wider decode variant than the
    one captured (reference refusal of layout changes:
    src/flashinfer_attention.cu:32).  The two block batches are planned one
    by the longest-first list and one by the equal cut of the tile stream,
    so the replays switch between the two share layouts."""
    hq, hkv, blocks = 32, 8, 900
    kc = torch.zeros(blocks + 1, 16, hkv, 128, dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    q = torch.zeros(64, hq, 128, dtype=torch.bfloat16, device=dev)
    out = torch.zeros_like(q)
    lse = torch.zeros(64, hq, device=dev)
    plan = feattn.Plan(hq, hkv, 128, 16, 4, 250, True, blocks)

    def load(bb, seed):
        qq, kk, vv = W.make_tensors(bb, seed=seed)
        kc.copy_(kk.to(dev))
        vc.copy_(vv.to(dev))
        q.zero_()
        q[:bb.rows].copy_(qq.to(dev))
        plan.prepare(bb.qo, bb.kv, bb.pages, bb.last, bb.batch, bb.rows, graph=True)
        return qq, kk, vv

    first = W.make_batch(hq, hkv, starts=[900, 2000, 40, 1200], qlens=[16] * 4, seed=1, pool=blocks)
    load(first, 1)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        plan.run(q, kc, vc, out, causal=False, lse=lse)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        plan.run(q, kc, vc, out, causal=False, lse=lse)
    steps = [first,
             W.make_batch(hq, hkv, starts=[3500, 5, 700, 1800], qlens=[16] * 4, seed=2, pool=blocks),
             W.make_batch(hq, hkv, starts=[3000, 5, 700, 1800], qlens=[1] * 4, seed=3, pool=blocks)]
    assert not stream_cut_taken(steps[0], False) and stream_cut_taken(steps[1], False)
    for seed, bb in enumerate(steps, start=1):
        qq, kk, vv = load(bb, seed)
        graph.replay()
        torch.cuda.synchronize()
        want_out, want_lse = A.run(bb, qq, kk, vv, False)
        check(out[:bb.rows].cpu(), lse[:bb.rows].cpu(), want_out, want_lse)
    eight = W.make_batch(hq, hkv, starts=[100, 2500, 60], qlens=[8, 8, 8], seed=4, pool=blocks)
    with pytest.raises(RuntimeError):
        plan.prepare(eight.qo, eight.kv, eight.pages, eight.last, eight.batch, eight.rows, graph=True)
    plan.close()


def test_back_to_back_prepares_without_host_sync(dev):
    """One plan prepared for two different batches in turn, each prepare
    followed by its attention call, 12 times with no host synchronisation:
    a prepare rewrites the plan's pinned staging image only after the
    previous prepare's staging kernel has read it, so every call sees its
    own metadata.  Each call writes its own output buffer; all match the
    oracle afterwards."""
    hq, hkv, blocks = 32, 8, 1200
    a = W.make_batch(hq, hkv, starts=[3000, 17, 900, 2500], qlens=[1, 1, 5, 1], seed=61, pool=blocks)
    b = W.make_batch(hq, hkv, starts=[64, 4000, 1200], qlens=[40, 1, 16], seed=62, pool=blocks)
    # one K/V pool serves both batches: their pages come from the same pool of `blocks`
    q, kc, vc = W.make_tensors(a, seed=61)
    qd, kd, vd = q.to(dev), kc.to(dev), vc.to(dev)
    qb = torch.randn(b.rows, hq, 128, generator=torch.Generator().manual_seed(62)).to(torch.bfloat16)
    qbd = qb.to(dev)
    plan = feattn.Plan(hq, hkv, 128, 16, 4, 300, True, blocks)
    outs = []
    for i in range(12):
        bb, qq = (a, qd) if i % 2 == 0 else (b, qbd)
        plan.prepare(bb.qo, bb.kv, bb.pages, bb.last, bb.batch, bb.rows)
        out = torch.empty_like(qq)
        lse = torch.empty(bb.rows, hq, device=dev)
        plan.run(qq, kd, vd, out, causal=True, lse=lse)
        outs.append((bb, out, lse))
    torch.cuda.synchronize()
    plan.close()
    want = {id(a): A.run(a, q, kc, vc, True), id(b): A.run(b, qb, kc, vc, True)}
    for bb, out, lse in outs:
        check(out.cpu(), lse.cpu(), *want[id(bb)])


def test_prepare_refuses_a_capturing_stream(dev):
    """prepare_plan on a capturing stream returns FE_EINVAL before enqueuing
    anything; the capture ends with an empty graph, and the plan still holds
    the metadata of its previous prepare."""
    a = W.make_batch(32, 8, starts=[100, 40], qlens=[1, 3], seed=71)
    b = W.make_batch(32, 8, starts=[900, 5], qlens=[2, 1], seed=72)
    q, kc, vc = W.make_tensors(a, seed=71)
    qd, kd, vd = q.to(dev), kc.to(dev), vc.to(dev)
    plan = feattn.Plan(32, 8, 128, 16, 2, max(a.max_pages(), b.max_pages()), True, a.blocks)
    plan.prepare(a.qo, a.kv, a.pages, a.last, a.batch, a.rows)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, capture_error_mode="thread_local"):
        with pytest.raises(RuntimeError, match="capturing"):
            plan.prepare(b.qo, b.kv, b.pages, b.last, b.batch, b.rows)
    torch.cuda.synchronize()
    out = torch.zeros_like(qd)
    lse = torch.empty(a.rows, 32, device=dev)
    plan.run(qd, kd, vd, out, causal=True, lse=lse)
    torch.cuda.synchronize()
    plan.close()
    check(out.cpu(), lse.cpu(), *A.run(a, q, kc, vc, True))


def test_misaligned_tensors_are_refused(dev):
    """q, the K/V caches and out move in 16-byte pieces: a view starting 8
    bytes into its storage is refused before any launch, and the aligned
    call that follows still matches the oracle."""
    b = W.make_batch(32, 8, starts=[100, 40], qlens=[1, 3], seed=31)
    q, kc, vc = W.make_tensors(b, seed=31)
    plan = feattn.Plan(b.hq, b.hkv, 128, b.page, b.batch, b.max_pages(), True, b.blocks)
    plan.prepare(b.qo, b.kv, b.pages, b.last, b.batch, b.rows)
    qd, kd, vd = q.to(dev), kc.to(dev), vc.to(dev)
    out = torch.zeros_like(qd)
    n = qd.numel()
    shifted = torch.zeros(n + 8, dtype=qd.dtype, device=dev)[4:4 + n].view_as(qd)
    shifted.copy_(qd)
    with pytest.raises(RuntimeError, match="aligned"):
        plan.run(shifted, kd, vd, out, causal=True)
    with pytest.raises(RuntimeError, match="aligned"):
        plan.run(qd, kd, vd, torch.zeros(n + 8, dtype=qd.dtype, device=dev)[4:4 + n].view_as(qd), causal=True)
    lse = torch.zeros(b.rows, b.hq, device=dev)
    plan.run(qd, kd, vd, out, causal=True, lse=lse)
    torch.cuda.synchronize()
    plan.close()
    want_out, want_lse = A.run(b, q, kc, vc, True)
    check(out.cpu(), lse.cpu(), want_out, want_lse)


@pytest.mark.parametrize("causal", [True, False])
def test_null_lse_gives_the_same_output(dev, causal):
    """The reference's attention has no LSE output (its call passes none):
    with lse = NULL every kernel (decode, tile, both merges) must write the
    same output bits as with an LSE buffer.  The batch splits decode
    sequences (long contexts) and tile items (a long chunk)."""
    b = W.make_batch(32, 8, starts=[9000, 40, 6000, 0], qlens=[1, 1, 3, 600], seed=31, extra_pages=1)
    q, kc, vc = W.make_tensors(b, seed=31)
    counts = feattn.describe(b.hq, b.hkv, 128, b.page, b.batch, b.max_pages(), b.blocks, b.qo, b.kv,
                             b.pages, b.last, b.batch, b.rows)
    assert counts[2] > 0  # some rows are merged from split partials
    plan = feattn.Plan(b.hq, b.hkv, 128, b.page, b.batch, b.max_pages(), True, b.blocks)
    plan.prepare(b.qo, b.kv, b.pages, b.last, b.batch, b.rows)
    qd, kd, vd = q.to(dev), kc.to(dev), vc.to(dev)
    with_lse = torch.zeros_like(qd)
    lse = torch.full((b.rows, b.hq), float("nan"), device=dev)
    plan.run(qd, kd, vd, with_lse, causal=causal, lse=lse)
    no_lse = torch.zeros_like(qd)
    plan.run(qd, kd, vd, no_lse, causal=causal, lse=None)
    torch.cuda.synchronize()
    plan.close()
    assert torch.equal(with_lse.view(torch.int16), no_lse.view(torch.int16))
    want_out, want_lse = A.run(b, q, kc, vc, causal)
    check(no_lse.cpu(), lse.cpu(), want_out, want_lse)


def test_pool_beyond_4_gib(dev):
    """K/V caches of 140001 pages each (4.6 GB at hkv 8, 32 KB per page) with
    every page of the batch past the first 4 GiB, so each K/V address and
    store offset needs more than 32 bits: decode rows, a 16-row block and a
    prefill chunk (both masks) against the oracle on a compact copy of the
    pages, then the batch's new K/V rows stored at their slots and read back
    bit-exact."""
    hq, hkv, page, pool = 32, 8, 16, 140000
    compact = W.make_batch(hq, hkv, starts=[3000, 700, 0, 1500], qlens=[1, 16, 300, 1], seed=81)
    q, kc, vc = W.make_tensors(compact, seed=81)
    base = pool - compact.blocks - 1  # compact page p is page base + p of the large pool
    assert base * page * hkv * 128 * 2 > 1 << 32
    big = W.build_metadata(W.Batch(hq=hq, hkv=hkv, page=page, blocks=pool, starts=list(compact.starts),
                                   qlens=list(compact.qlens),
                                   tables=[[base + p for p in t] for t in compact.tables]))
    kd = torch.empty((pool + 1, page, hkv, 128), dtype=torch.bfloat16, device=dev)
    vd = torch.empty_like(kd)
    kd[base:base + compact.blocks + 1].copy_(kc.to(dev))
    vd[base:base + compact.blocks + 1].copy_(vc.to(dev))
    qd = q.to(dev)
    plan = feattn.Plan(hq, hkv, 128, page, big.batch, big.max_pages(), True, big.blocks)
    plan.prepare(big.qo, big.kv, big.pages, big.last, big.batch, big.rows)
    for causal in (True, False):
        out = torch.zeros_like(qd)
        lse = torch.full((big.rows, hq), float("nan"), device=dev)
        plan.run(qd, kd, vd, out, causal=causal, lse=lse)
        torch.cuda.synchronize()
        check(out.cpu(), lse.cpu(), *A.run(compact, q, kc, vc, causal))
    plan.close()
    gen = torch.Generator().manual_seed(82)
    k_new = torch.randn(big.rows, hkv, 128, generator=gen).to(torch.bfloat16)
    v_new = torch.randn(big.rows, hkv, 128, generator=gen).to(torch.bfloat16)
    slots = torch.from_numpy(big.slots)
    assert int(slots.min()) >= base * page
    feattn.store(k_new.to(dev), v_new.to(dev), kd, vd, slots.to(dev), big.rows, hkv * 128, True, (pool + 1) * page)
    torch.cuda.synchronize()
    kflat, vflat = kd.view(-1, hkv, 128), vd.view(-1, hkv, 128)
    sd = slots.to(dev)
    assert torch.equal(kflat[sd].cpu(), k_new) and torch.equal(vflat[sd].cpu(), v_new)
    del kd, vd, kflat, vflat
    torch.cuda.empty_cache()


def test_two_plans_on_two_streams(dev):
    """Two plans (a decode batch and a prefill batch, different shapes) are
    prepared and run on two streams at once, three times in a row; both
    results match the oracle.  Plans share no state, so streams may run
    them concurrently."""
    dec = W.make_batch(32, 8, starts=[3000, 40, 700, 1500], qlens=[1, 1, 1, 1], seed=21, extra_pages=1)
    pre = W.make_batch(16, 4, starts=[0, 300], qlens=[200, 90], seed=22, extra_pages=1)
    jobs = []
    for b, causal, seed in ((dec, True, 21), (pre, True, 22)):
        q, kc, vc = W.make_tensors(b, seed=seed)
        plan = feattn.Plan(b.hq, b.hkv, 128, b.page, b.batch, b.max_pages(), True, b.blocks)
        want = A.run(b, q, kc, vc, causal)
        jobs.append(dict(b=b, plan=plan, causal=causal, want=want, q=q.to(dev), kc=kc.to(dev), vc=vc.to(dev),
                         out=torch.zeros(b.rows, b.hq, 128, dtype=torch.bfloat16, device=dev),
                         lse=torch.zeros(b.rows, b.hq, device=dev), st=torch.cuda.Stream()))
    torch.cuda.synchronize()
    for _ in range(3):
        for j in jobs:
            b = j["b"]
            with torch.cuda.stream(j["st"]):
                j["out"].zero_()
                j["plan"].prepare(b.qo, b.kv, b.pages, b.last, b.batch, b.rows, stream=j["st"])
                j["plan"].run(j["q"], j["kc"], j["vc"], j["out"], causal=j["causal"], lse=j["lse"], stream=j["st"])
    torch.cuda.synchronize()
    for j in jobs:
        check(j["out"].cpu(), j["lse"].cpu(), *j["want"])
        j["plan"].close()


def _extreme_scores(b, pattern, dtype, seed):
    """Positive q and k in [0.5, 1), k scaled by a function of the token's
    logical position, so that every score is positive and its size is set by
    the position: "rising" steps up by ~10 (log2 units) every 48 tokens,
    "falling" steps down (both capped at 40x, which keeps the fp32 sums of
    the scores exact to ~1e-4), "sink" puts token 0 ~480x above the rest."""
    _, _, vc = W.make_tensors(b, seed=seed, dtype=dtype)
    g = torch.Generator().manual_seed(seed + 99)
    q = torch.rand((b.rows, b.hq, 128), generator=g) * 0.5 + 0.5
    k = torch.rand(vc.shape, generator=g) * 0.5 + 0.5
    pos = torch.zeros(vc.shape[0], vc.shape[1])
    for s in range(b.batch):
        for t in range(b.lens[s]):
            pos[b.tables[s][t // b.page], t % b.page] = t
    pos = pos.view(vc.shape[0], vc.shape[1], 1, 1)
    if pattern == "rising":
        scale = (1.0 + torch.floor(pos / 48)).clamp(max=40.0)
    elif pattern == "falling":
        scale = (1.0 + torch.floor((pos.max() - pos) / 48)).clamp(max=40.0)
    else:
        scale = torch.where(pos == 0, torch.tensor(24.0), torch.tensor(0.05))
    dt = torch.bfloat16 if dtype == "bf16" else torch.float16
    return q.to(dt), (k * scale).to(dt), vc


@pytest.mark.parametrize("pattern", ["rising", "falling", "sink"])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_extreme_scores(dev, pattern, causal, dtype):
    """Decode rows, a 200-row chunk, a 16-row block and a split long context
    whose scores exceed the exponential's range by far: the running maximum
    must be raised (with l and o rescaled) as often and as far as the scores
    demand, and tokens far below it must not disturb the result."""
    b = W.make_batch(32, 8, starts=[2000, 0, 700, 30, 20000], qlens=[1, 200, 16, 1, 1], seed=5)
    q, kc, vc = _extreme_scores(b, pattern, dtype, seed=7)
    want_out, want_lse = A.run(b, q, kc, vc, causal)
    assert float(want_lse.max()) > 150.0  # far past exp's range without the maximum taken out
    out, lse = run(b, q, kc, vc, causal, dev)
    check(out, lse, want_out, want_lse)
