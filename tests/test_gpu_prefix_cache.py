"""Serving through the page allocator's prefix cache on the GPU
(BlockManager::probe / publish, src/scheduler.cpp:6-29, as CudaModel::prepare
hands the tables to prepare_plan, src/cuda_model.cpp:131-142).

Prompts share a stem.  Each sequence probes the cache, RoPE-appends only the
tokens past its cached prefix into pages of its own, attends over the shared
pages, and publishes what it computed; then one decode step runs all of them
in one batch.  A hit must be invisible: every output row and LSE is
bit-identical to a run without the cache in which each sequence first
recomputes the same prefix into pages of its own (the compared calls have the
same shapes, so the same plan; only page ids differ), the K/V each sequence
sees are bit-identical, and the cached run matches the oracle and, when oracle/_ref is
built, the reference's own ATen attention (tolerance: |a-b| <= 1e-2 +
1e-2*|b| on outputs, 1e-3 on the natural-log LSE)."""

import math

import numpy as np
import pytest
import torch

import feattn
from feattn import workloads as W
from oracle import aten_attention as A
from oracle import ref_lib

pytestmark = pytest.mark.gpu
HQ, HKV, PAGE, DIM, VOCAB = 32, 8, 16, 128, 64
POOL = 420
MAX_LEN = 1400


def prompts():
    rng = np.random.default_rng(2024)
    stem = rng.integers(0, VOCAB, 1000).tolist()
    tail = lambda n: rng.integers(0, VOCAB, n).tolist()
    first = stem + tail(300)
    return {
        1: first,                    # computes everything, publishes 81 pages
        2: stem + tail(37),          # hits the stem's 62 whole pages
        3: stem[:500] + tail(800),   # hits 31 pages
        4: list(first),              # the same prompt: 81 pages, 4 tokens left
    }


def embeddings(dtype, dev):
    g = torch.Generator().manual_seed(77)
    t = torch.bfloat16 if dtype == "bf16" else torch.float16
    mk = lambda h: torch.randn(VOCAB, h, DIM, generator=g).to(t).to(dev)
    return mk(HQ), mk(HKV), mk(HKV)


def serve(caching, cut, dtype, dev, oracle_checks=None):
    """Prefill every prompt (from its cached prefix when `caching`, else in
    two chunks split where the cached run's prefix ended), then one decode
    step for all.  Returns the compared outputs, the allocator and caches."""
    eq, ek, ev = embeddings(dtype, dev)
    bf16 = dtype == "bf16"
    rope = W.rope_table(MAX_LEN, 1e6).to(dev)
    kc = torch.zeros(POOL + 1, PAGE, HKV, DIM, dtype=eq.dtype, device=dev)
    vc = torch.zeros_like(kc)
    blocks = feattn.Blocks(POOL, PAGE, caching)
    plan = feattn.Plan(HQ, HKV, DIM, PAGE, 4, math.ceil(MAX_LEN / PAGE) + 1, bf16, POOL)
    toks = {s: list(p) for s, p in prompts().items()}
    got, starts = {}, {}

    def step(seqs, begins, ends, key):
        for s, e in zip(seqs, ends):
            assert blocks.ensure(s, e)
        b = W.build_metadata(W.Batch(hq=HQ, hkv=HKV, page=PAGE, blocks=POOL, starts=list(begins),
                                     qlens=[e - st for st, e in zip(begins, ends)],
                                     tables=[blocks.table(s) for s in seqs]))
        ids = torch.tensor([toks[s][p] for s, st, e in zip(seqs, begins, ends) for p in range(st, e)], device=dev)
        q, k, v = eq[ids].contiguous(), ek[ids].contiguous(), ev[ids].contiguous()
        pos = torch.from_numpy(b.positions).to(dev)
        slots = torch.from_numpy(b.slots).to(dev)
        feattn.rope_append(q, k, v, kc, vc, pos, slots, rope, b.rows, HQ, HKV, DIM, bf16, MAX_LEN,
                           b.cache_slots)
        plan.prepare(b.qo, b.kv, b.pages, b.last, b.batch, b.rows)
        out = torch.zeros_like(q)
        lse = torch.full((b.rows, HQ), float("nan"), device=dev)
        plan.run(q, kc, vc, out, causal=True, lse=lse)
        torch.cuda.synchronize()
        got[key] = (out.cpu(), lse.cpu())
        if oracle_checks is not None:
            oracle_checks.append((key, b, q.clone(), out.cpu(), lse.cpu()))
        for s, e in zip(seqs, ends):
            blocks.publish(s, toks[s], e)

    for s in sorted(toks):
        c = blocks.probe(s, toks[s])
        starts[s] = c
        if caching:
            step([s], [c], [len(toks[s])], ("prefill", s))
        else:
            if cut[s] > 0:
                step([s], [0], [cut[s]], ("prefix", s))
            step([s], [cut[s]], [len(toks[s])], ("prefill", s))
    seqs = sorted(toks)
    begins = [len(toks[s]) for s in seqs]
    rng = np.random.default_rng(5)
    for s in seqs:  # the sampled token of each sequence (src/scheduler.cpp:94-99)
        toks[s].append(int(rng.integers(0, VOCAB)))
    step(seqs, begins, [b + 1 for b in begins], ("decode", 0))
    plan.close()
    return got, starts, blocks, toks, kc, vc


def kv_of(blocks, seq, n, cache):
    t = blocks.table(seq)
    idx = torch.tensor([t[p // PAGE] * PAGE + p % PAGE for p in range(n)])
    return cache.reshape(-1, HKV, DIM)[idx.to(cache.device)].cpu()


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_prefix_cache_hits_are_invisible(dev, dtype):
    checks = []
    shared, cut, blocks, toks, kc, vc = serve(True, None, dtype, dev, checks)
    assert cut == {1: 0, 2: 992, 3: 496, 4: 1296}
    st = blocks.stats()
    assert st["prefix_hit_requests"] == 3 and st["prefix_cached_blocks"] == 62 + 31 + 81
    # shared pages really are shared: seq 4's table starts with seq 1's 81 pages
    assert blocks.table(4)[:81] == blocks.table(1)[:81]
    private, cut2, pblocks, _, pkc, pvc = serve(False, cut, dtype, dev)
    assert cut2 == {1: 0, 2: 0, 3: 0, 4: 0} and pblocks.stats()["prefix_new_blocks"] == 0
    assert not set(pblocks.table(4)) & set(pblocks.table(1))
    for key, (out, lse) in shared.items():
        pout, plse = private[key]
        assert torch.equal(out, pout), key
        assert torch.equal(lse, plse), key
    for s in toks:
        n = len(toks[s])
        assert torch.equal(kv_of(blocks, s, n, kc), kv_of(pblocks, s, n, pkc)), s
        assert torch.equal(kv_of(blocks, s, n, vc), kv_of(pblocks, s, n, pvc)), s
    kcc, vcc = kc.cpu(), vc.cpu()
    for key, b, q, out, lse in checks:
        want_out, want_lse = A.run(b, q.cpu(), kcc, vcc, True)
        torch.testing.assert_close(out.float(), want_out.float(), atol=1e-2, rtol=1e-2, msg=str(key))
        torch.testing.assert_close(lse, want_lse, atol=1e-3, rtol=0, msg=str(key))
        if ref_lib.available():
            # the reference's own create_plan / prepare_plan / attention
            # (src/portable_gpu_ops.cpp:18-44) on the same device tensors
            ref = ref_lib.attention(b, q, kc, vc, True).cpu()
            torch.testing.assert_close(out.float(), ref.float(), atol=1e-2, rtol=1e-2, msg=str(key))
    blocks.close()
    pblocks.close()
