"""GPU side of the host driver: the RoPE table kernel (src/cuda_model.cpp:44-47)
against closed forms and the float32 CPU table, and a multi-step serving
sequence driven the way the reference's model runner drives it
(src/cuda_model.cpp:131-142, 94-95): page allocator -> per-step metadata ->
fused RoPE + KV append -> paged attention, every step checked against the
oracle (bit-exact for the append, 1e-2 abs / 1e-2 rel for attention outputs,
1e-3 for the log-sum-exp)."""

import numpy as np
import pytest
import torch

import feattn
from feattn import workloads as W
from oracle import aten_attention as A
from oracle import rope_store as R

pytestmark = pytest.mark.gpu


def u16(t):
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


def from_u16(a, dt, shape):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(dt).reshape(shape)


def device_table(dev, max_len, dim, theta):
    t = torch.full((max_len, dim), float("nan"), device=dev)
    feattn.rope_table(t, max_len, dim, theta)
    torch.cuda.synchronize()
    return t.cpu()


@pytest.mark.parametrize("dim,theta", [(128, 1e6), (128, 1e4), (64, 5e5)])
def test_rope_table_closed_forms(dev, dim, theta):
    t = device_table(dev, 4096, dim, theta).double()
    half = dim // 2
    # position 0: cos = 1, sin = 0 in every column
    assert torch.equal(t[0, :half], torch.ones(half, dtype=torch.float64))
    assert torch.equal(t[0, half:], torch.zeros(half, dtype=torch.float64))
    # column 0 has frequency 1: (cos p, sin p)
    p = torch.arange(4096, dtype=torch.float64)
    assert torch.allclose(t[:, 0], p.cos(), atol=2e-6, rtol=0)
    assert torch.allclose(t[:, half], p.sin(), atol=2e-6, rtol=0)
    # position 1: frequencies theta^(-2i/dim), first half cos, second half sin
    inv = torch.tensor([theta ** (-(2 * i) / dim) for i in range(half)], dtype=torch.float64)
    assert torch.allclose(t[1, :half], inv.cos(), atol=2e-6, rtol=0)
    assert torch.allclose(t[1, half:], inv.sin(), atol=2e-6, rtol=0)
    # unit circle everywhere
    assert torch.allclose(t[:, :half] ** 2 + t[:, half:] ** 2, torch.ones(4096, half, dtype=torch.float64),
                          atol=1e-6, rtol=0)


def test_rope_table_matches_cpu_float32(dev):
    """Same float32 formula on the CPU; positions up to 40960 (Qwen3
    max_position_embeddings).  A one-ulp difference in a frequency moves
    p * inv by at most ~2.4e-7 * p, hence the position-scaled bound."""
    n = 40960
    got = device_table(dev, n, 128, 1e6)
    want = W.rope_table(n, 1e6)
    bound = 1e-6 + 3e-7 * torch.arange(n, dtype=torch.float32).unsqueeze(1)
    assert ((got - want).abs() <= bound).all()


HQ, HKV, PAGE, POOL, MAX_LEN = 32, 8, 16, 64, 256


class Runner:
    """A miniature of the reference's per-step loop on one plan and one
    persistent pair of KV caches (device and oracle copies)."""

    def __init__(self, dev, dtype):
        self.dev, self.dt, self.bf16 = dev, dtype, dtype == torch.bfloat16
        self.blocks = feattn.Blocks(POOL, PAGE)
        self.table_d = torch.empty(MAX_LEN, 128, device=dev)
        feattn.rope_table(self.table_d, MAX_LEN, 128, 1e6)
        self.table = self.table_d.cpu()
        gen = torch.Generator().manual_seed(17)
        shape = (POOL + 1, PAGE, HKV, 128)        # page POOL is the padding page
        self.kc = torch.randn(shape, generator=gen).to(dtype)
        self.vc = torch.randn(shape, generator=gen).to(dtype)
        self.kc_d, self.vc_d = self.kc.to(dev), self.vc.to(dev)
        self.plan = feattn.Plan(HQ, HKV, 128, PAGE, 8, MAX_LEN // PAGE + 1, self.bf16, POOL)
        self.gen = torch.Generator().manual_seed(29)

    def step(self, seqs, starts, rows, count=None, entry_rows=0, causal=True):
        for s, st, r in zip(seqs, starts, rows):
            assert self.blocks.ensure(s, st + r)
        tables = [self.blocks.table(s) for s in seqs]
        m = feattn.prepare_metadata(starts, rows, tables, PAGE, MAX_LEN, count=count, entry_rows=entry_rows,
                                    dummy_page=POOL)
        n, batch = len(m["positions"]), len(m["last"])
        q = torch.randn(n, HQ, 128, generator=self.gen).to(self.dt)
        k = torch.randn(n, HKV, 128, generator=self.gen).to(self.dt)
        v = torch.randn(n, HKV, 128, generator=self.gen).to(self.dt)
        pos, slots = torch.from_numpy(m["positions"]), torch.from_numpy(m["slots"])
        cslots = (POOL + 1) * PAGE
        wq, wkc, wvc = R.rope_append(u16(q), u16(k), u16(v), u16(self.kc), u16(self.vc), pos.numpy(),
                                     slots.numpy(), self.table.numpy(), n, HQ, HKV, 128, self.bf16, MAX_LEN,
                                     cslots)
        qd = q.to(self.dev)
        feattn.rope_append(qd, k.to(self.dev), v.to(self.dev), self.kc_d, self.vc_d, pos.to(self.dev),
                           slots.to(self.dev), self.table_d, n, HQ, HKV, 128, self.bf16, MAX_LEN, cslots)
        self.plan.prepare(m["qo"].tolist(), m["kv"].tolist(), m["pages"].tolist(), m["last"].tolist(), batch, n)
        out = torch.zeros_like(qd)
        lse = torch.full((n, HQ), float("nan"), device=self.dev)
        self.plan.run(qd, self.kc_d, self.vc_d, out, causal=causal, lse=lse)
        torch.cuda.synchronize()
        assert np.array_equal(u16(qd), wq)
        assert np.array_equal(u16(self.kc_d).reshape(cslots, -1), wkc)
        assert np.array_equal(u16(self.vc_d).reshape(cslots, -1), wvc)
        self.kc = from_u16(wkc, self.dt, self.kc.shape)
        self.vc = from_u16(wvc, self.dt, self.vc.shape)
        pad = batch - len(seqs)
        b = W.Batch(hq=HQ, hkv=HKV, page=PAGE, blocks=POOL, starts=list(starts) + [0] * pad,
                    qlens=list(rows) + [entry_rows] * pad, tables=tables + [[POOL]] * pad,
                    qo=m["qo"].tolist(), kv=m["kv"].tolist(), pages=m["pages"].tolist(), last=m["last"].tolist())
        want_out, want_lse = A.run(b, from_u16(wq, self.dt, q.shape), self.kc, self.vc, causal,
                                   max_pages=MAX_LEN // PAGE + 1)
        torch.testing.assert_close(out.cpu().float(), want_out.float(), atol=1e-2, rtol=1e-2)
        torch.testing.assert_close(lse.cpu(), want_lse, atol=1e-3, rtol=0)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_serving_steps_vs_oracle(dev, dtype):
    r = Runner(dev, dtype)
    prompt = {0: 40, 1: 5, 2: 100, 3: 17}
    # chunked prefill: sequence 2 gets 60 of its 100 prompt tokens
    r.step([0, 1, 2, 3], [0, 0, 0, 0], [40, 5, 60, 17])
    r.step([2], [60], [40])                                   # rest of the prompt over a 60-token prefix
    lens = dict(prompt)
    for _ in range(3):                                        # decode, bucket 4: no padding
        r.step([0, 1, 2, 3], [lens[s] for s in range(4)], [1] * 4, count=4, entry_rows=1)
        lens = {s: n + 1 for s, n in lens.items()}
    r.blocks.release(1)                                       # sequence 1 finishes; its page is recycled last
    del lens[1]
    # FIFO pool: pages 0..12 went out in order (3 + 1 + 4 + 2, then 3 more for
    # sequence 2); sequence 1's page 3 is now behind 13..63
    assert r.blocks.table(0) == [0, 1, 2] and r.blocks.table(2) == [4, 5, 6, 7, 10, 11, 12]
    assert r.blocks.ensure(4, 30) and r.blocks.table(4) == [13, 14]
    r.step([4], [0], [30])
    lens[4] = 30
    live = [0, 2, 4]
    bucket = next(b for b in feattn.graph_buckets(8) if b >= len(live))
    assert bucket == 4
    r.step(live, [lens[s] for s in live], [1] * 3, count=bucket, entry_rows=1)   # one padding entry
    lens = {s: lens[s] + 1 for s in lens}
    # speculative verify: 4 rows per sequence, padded with 4-row entries
    r.step(live, [lens[s] for s in live], [4] * 3, count=bucket, entry_rows=4)
    # block (non-causal) attention over the same rows, as the drafter runs it
    r.step(live, [lens[s] + 4 for s in live], [16] * 3, count=bucket, entry_rows=16, causal=False)
    for s in (0, 2, 3, 4):
        r.blocks.release(s)
    assert r.blocks.used() == 0
    r.plan.close()
