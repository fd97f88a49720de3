"""fe_attn_run_noalloc (attention with no device allocation) against the plan
entry points fe_attn_plan_prepare + fe_attn_run on the same inputs: the same
work lists and kernels, so out and LSE must match bit for bit.  Two calls in
a row share the library's device scratch; the second is smaller (fewer
sequences, other heads, dtype and mask), so anything it read from the first
call's leftovers would show."""

import ctypes

import numpy as np
import pytest
import torch

import feattn
from feattn import workloads as W
from test_gpu_known_counts import stream_cut_taken

pytestmark = pytest.mark.gpu


def both_paths(dev, b, causal, dtype, seed):
    dt = torch.bfloat16 if dtype == "bf16" else torch.float16
    q = W.randn_bf16((b.rows, b.hq, 128), seed, dtype, device=dev).to(dt)
    kc = W.randn_bf16((b.blocks + 1, b.page, b.hkv, 128), seed + 1, dtype, device=dev).to(dt)
    vc = W.randn_bf16((b.blocks + 1, b.page, b.hkv, 128), seed + 2, dtype, device=dev).to(dt)
    bf16 = dt == torch.bfloat16
    out_p = torch.full_like(q, float("nan"))
    lse_p = torch.full((b.rows, b.hq), float("nan"), device=dev)
    plan = feattn.Plan(b.hq, b.hkv, 128, b.page, b.batch, b.max_pages(), bf16, b.blocks)
    plan.prepare(b.qo, b.kv, b.pages, b.last, b.batch, b.rows)
    plan.run(q, kc, vc, out_p, causal=causal, lse=lse_p)
    torch.cuda.synchronize()
    plan.close()
    out_n = torch.full_like(q, float("nan"))
    lse_n = torch.full((b.rows, b.hq), float("nan"), device=dev)
    feattn.run_noalloc(q, kc, vc, out_n, b.qo, b.kv, b.pages, b.last, b.batch, b.rows, b.hq, b.hkv, 128,
                       b.page, b.blocks, bf16, causal=causal, lse=lse_n)
    torch.cuda.synchronize()
    assert not torch.isnan(out_p.float()).any() and not torch.isnan(lse_p).any()
    assert torch.equal(out_n.view(torch.int16), out_p.view(torch.int16))
    assert torch.equal(lse_n.view(torch.int32), lse_p.view(torch.int32))


def test_noalloc_matches_plan_path_twice_second_smaller(dev):
    # decode rows with split-KV (30000 and 4095 tokens), chunks on the tile
    # kernel, merge rows: every kernel of the path and every scratch region
    big = W.make_batch(32, 8, starts=[30000, 4095, 777, 0, 1000, 12], qlens=[1, 1, 1, 300, 129, 3], seed=31,
                       extra_pages=2)
    both_paths(dev, big, True, "bf16", 500)
    small = W.make_batch(16, 2, starts=[200, 64], qlens=[5, 1], seed=32, extra_pages=1)
    assert small.rows < big.rows and small.batch < big.batch
    both_paths(dev, small, False, "f16", 600)


def test_noalloc_stream_cut_batch_small_then_big(dev):
    """A batch planned by the equal cut of the tile stream (chunks split into
    consecutive pieces with partial rows), run after a smaller call and
    before one: the smaller call's metadata and partial rows are overwritten
    by the bigger call's, and the next small call reads none of them."""
    small = W.make_batch(16, 2, starts=[200, 64], qlens=[5, 1], seed=33, extra_pages=1)
    both_paths(dev, small, True, "bf16", 700)
    cut = W.make_batch(32, 8, starts=[6000, 9000, 300], qlens=[200, 64, 40], seed=45, extra_pages=1)
    assert stream_cut_taken(cut, True) and stream_cut_taken(cut, False)
    both_paths(dev, cut, True, "bf16", 710)
    both_paths(dev, cut, False, "f16", 720)
    both_paths(dev, small, False, "bf16", 730)


def test_noalloc_refuses_a_capturing_stream(dev):
    """Under stream capture the call returns FE_EINVAL before enqueuing
    anything (its metadata copy would read released host memory on every
    replay); the capture ends with an empty graph."""
    b = W.make_batch(32, 8, starts=[100, 40], qlens=[1, 3], seed=9)
    q = torch.zeros(b.rows, 32, 128, dtype=torch.bfloat16, device=dev)
    kc = torch.zeros(b.blocks + 1, 16, 8, 128, dtype=torch.bfloat16, device=dev)
    out = torch.full_like(q, float("nan"))
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, capture_error_mode="thread_local"):
        with pytest.raises(RuntimeError, match="capturing"):
            feattn.run_noalloc(q, kc, kc, out, b.qo, b.kv, b.pages, b.last, b.batch, b.rows, 32, 8, 128, 16,
                               b.blocks, True)
    torch.cuda.synchronize()
    assert torch.isnan(out.float()).all()
    # the stream is usable afterwards
    feattn.run_noalloc(q, kc, kc, out, b.qo, b.kv, b.pages, b.last, b.batch, b.rows, 32, 8, 128, 16, b.blocks,
                       True)
    torch.cuda.synchronize()
    assert not torch.isnan(out.float()).any()


def test_noalloc_rejects_calls_beyond_its_scratch(dev):
    """A page table of 13M entries (52 MB) cannot fit the 48 MiB scratch: the
    call fails on the host with FE_ECAPACITY and launches nothing."""
    lib = feattn.lib()
    npg = 13_000_000
    qo = np.array([0, 1], dtype=np.int32)
    kv = np.array([0, npg], dtype=np.int32)
    pages = np.zeros(npg, dtype=np.int32)
    last = np.array([16], dtype=np.int32)
    q = torch.zeros(1, 32, 128, dtype=torch.bfloat16, device=dev)
    kc = torch.zeros(2, 16, 8, 128, dtype=torch.bfloat16, device=dev)
    out = torch.full_like(q, float("nan"))
    p32 = lambda a: a.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))
    rc = lib.fe_attn_run_noalloc(q.data_ptr(), kc.data_ptr(), kc.data_ptr(), out.data_ptr(), None, 1, p32(qo),
                                 p32(kv), p32(pages), p32(last), 1, 1, 32, 8, 128, 16, 1, 1,
                                 torch.cuda.current_stream().cuda_stream)
    assert rc == feattn.FE_ECAPACITY
    assert b"scratch" in lib.fe_attn_last_error()
    torch.cuda.synchronize()
    assert torch.isnan(out.float()).all()


def test_noalloc_rejects_bad_arguments(dev):
    """The plan entry points' checks hold without a plan: head size,
    alignment, negative batch and invalid metadata are refused on the host
    with FE_EINVAL before any launch."""
    b = W.make_batch(32, 8, starts=[100, 40], qlens=[1, 3], seed=9)
    q = torch.zeros(b.rows, 32, 128, dtype=torch.bfloat16, device=dev)
    kc = torch.zeros(b.blocks + 1, 16, 8, 128, dtype=torch.bfloat16, device=dev)
    out = torch.full_like(q, float("nan"))

    def call(**kw):
        args = dict(q=q, k_cache=kc, v_cache=kc, out=out, qo=b.qo, kv=b.kv, pages=b.pages, last=b.last,
                    batch=b.batch, rows=b.rows, hq=32, hkv=8, dim=128, page=16, blocks=b.blocks, bf16=True)
        args.update(kw)
        return feattn.run_noalloc(**args)

    with pytest.raises(RuntimeError, match="error -1"):
        call(dim=64)
    with pytest.raises(RuntimeError, match="error -1"):
        call(q=q.view(-1)[4:].view(-1)[: q.numel() - 8])  # 8 bytes past the allocation start
    with pytest.raises(RuntimeError, match="error -1"):
        call(batch=-1)
    bad_last = list(b.last)
    bad_last[0] = 17
    with pytest.raises(RuntimeError, match="error -1"):
        call(last=bad_last)
    torch.cuda.synchronize()
    assert torch.isnan(out.float()).all()
