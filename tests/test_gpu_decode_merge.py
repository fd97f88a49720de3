"""The decode kernel's own merge of split sequences (the last of a
sequence's workgroups to store its partials merges them, through the L2 its
XCD shares or, for sequences whose pieces span XCDs, with device-scope
release / acquire) against the merge-kernel path, which a plan created with
FEATTN_MERGE_KERNEL=1 takes: outputs and LSE must be bit-identical (both
fold the same partials in the same order with the same arithmetic), and
repeated runs of one plan must give the same bits (the per-sequence arrival
counters return to zero after every launch).  Parity of the decode path
with the oracle is covered by the attention suites."""

import os

import pytest
import torch

import feattn
from feattn import workloads as W

pytestmark = pytest.mark.gpu


def make_cache(b, dev, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    shape = (b.blocks + 1, b.page, b.hkv, 128)
    kc = torch.randn(shape, generator=g, device=dev).to(torch.bfloat16)
    vc = torch.randn(shape, generator=g, device=dev).to(torch.bfloat16)
    q = torch.randn(b.rows, b.hq, 128, generator=g, device=dev).to(torch.bfloat16)
    return q, kc, vc


def runs(b, q, kc, vc, merge_kernel, n=1, causal=True):
    old = os.environ.get("FEATTN_MERGE_KERNEL")
    os.environ["FEATTN_MERGE_KERNEL"] = "1" if merge_kernel else "0"
    try:
        plan = feattn.Plan(b.hq, b.hkv, 128, b.page, b.batch, b.max_pages(), True, b.blocks)
    finally:
        if old is None:
            del os.environ["FEATTN_MERGE_KERNEL"]
        else:
            os.environ["FEATTN_MERGE_KERNEL"] = old
    plan.prepare(b.qo, b.kv, b.pages, b.last, b.batch, b.rows)
    res = []
    for _ in range(n):
        out = torch.zeros_like(q)
        lse = torch.full((b.rows, b.hq), float("nan"), device=q.device)
        plan.run(q, kc, vc, out, causal=causal, lse=lse)
        torch.cuda.synchronize()
        res.append((out.cpu(), lse.cpu()))
    plan.close()
    return res


def batches():
    return {
        "headline_64x": W.qwen3_8b_decode(),                       # 64 split, 7 across XCD groups
        "long_16x32k": W.long_decode(batch=16),                    # 16 pieces per sequence
        "mixed30b": W.qwen3_30b_mixed(),                           # decode beside tile items
        "hkv16": W.make_batch(64, 16, starts=[3000, 700, 9000, 1], qlens=[1, 2, 1, 1], seed=9),
        "hkv6": W.make_batch(24, 6, starts=list(range(100, 6100, 300)), qlens=[1] * 20, seed=10),
        "hkv1_189x": W.make_batch(8, 1, starts=[5000, 20, 12000], qlens=[1, 4, 1], seed=11),
        "verify_rows": W.make_batch(32, 8, starts=[4000, 2500, 7000, 300], qlens=[8, 3, 8, 1], seed=12),
    }


@pytest.mark.parametrize("name", list(batches()))
def test_inline_merge_matches_merge_kernel(dev, name):
    b = batches()[name]
    recs, _ = feattn.decode_merges(b.hq, b.hkv, 128, b.page, b.batch, b.max_pages(), b.blocks,
                                   b.qo, b.kv, b.pages, b.last, b.batch, b.rows)
    assert any(r[2] > 0 for r in recs), "no split decode sequence in this batch"
    print(f"[decode merge] {name}: {sum(r[2] > 0 for r in recs)} split, "
          f"{sum(r[3] for r in recs)} across XCD groups", flush=True)
    q, kc, vc = make_cache(b, dev, seed=len(name))
    inline = runs(b, q, kc, vc, merge_kernel=False, n=3)
    (want_out, want_lse), = runs(b, q, kc, vc, merge_kernel=True)
    assert not torch.isnan(want_lse).any()
    for out, lse in inline:
        assert torch.equal(out.view(torch.int16), want_out.view(torch.int16))
        assert torch.equal(lse, want_lse)
