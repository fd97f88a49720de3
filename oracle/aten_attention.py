"""ORACLE (test infrastructure only): LibTorch-CPU restatement of the
reference's ATen attention path, src/portable_gpu_ops.cpp.

The reference runs these ATen ops on at::kCUDA; here the same op sequence
runs on the CPU:
  * create_plan   (:23-25)  cache_slots = (blocks+1)*page,
                            max_context = (max_pages-1)*page
  * prepare_plan  (:27-38)  gather indices over max_context per sequence and
                            [rows, max_context] causal / full masks
  * attention     (:39-44)  per sequence: index_select -> repeat_interleave
                            (GQA) -> fp32 bmm / sqrt(dim) -> masked_fill(-inf)
                            -> softmax -> bmm -> copy_ (round to bf16/fp16)
The natural-log log-sum-exp of the masked logits is an added output (the
reference has none; see src/flashinfer_attention.cu:38 lse=nullptr).

Pinned by tests/test_oracle_attention.py against: the closed-form known
answers of tests/ascend_ops_tests.cpp:21,44,49-51,62-65 (uniform softmax ->
mean of visible V rows), GQA head permutation, and the float64 brute force in
oracle/brute.py on randomized tiny shapes.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Sequence

import torch


@dataclass
class RefPlan:
    hq: int
    hkv: int
    dim: int
    page: int
    max_batch: int
    max_pages: int
    bf16: bool
    cache_slots: int
    max_context: int
    batch: int = 0
    rows: int = 0
    qo: Sequence[int] = ()
    indices: torch.Tensor = None
    causal_mask: torch.Tensor = None
    full_mask: torch.Tensor = None


def create_plan(hq, hkv, dim, page, max_batch, max_pages, bf16, blocks) -> RefPlan:
    """portable_gpu_ops.cpp:23-25."""
    return RefPlan(hq, hkv, dim, page, max_batch, max_pages, bf16,
                   cache_slots=(blocks + 1) * page, max_context=(max_pages - 1) * page)


def prepare_plan(p: RefPlan, qo, kv, pages, last, batch: int, rows: int) -> None:
    """portable_gpu_ops.cpp:27-38: indices[b][t] = t < len ?
    pages[kv[b] + t/page]*page + t%page : cache_slots - 1;
    causal[r][t] = t <= len - qlen + (r - qo[b]); full[r][t] = t < len."""
    if batch > p.max_batch:
        raise RuntimeError("reference attention batch out of range")
    mc = p.max_context
    indices = torch.full((batch, mc), p.cache_slots - 1, dtype=torch.int64)
    causal = torch.zeros((rows, mc), dtype=torch.bool)
    full = torch.zeros((rows, mc), dtype=torch.bool)
    t = torch.arange(mc, dtype=torch.int64)
    for b in range(batch):
        length = (kv[b + 1] - kv[b] - 1) * p.page + last[b]
        qrows = qo[b + 1] - qo[b]
        if length < qrows or length > mc:
            raise RuntimeError("reference attention context out of range")
        tv = t[:length]
        pg = torch.tensor(list(pages[kv[b]:kv[b + 1]]), dtype=torch.int64)
        indices[b, :length] = pg[tv // p.page] * p.page + tv % p.page
        r = torch.arange(qo[b], qo[b + 1], dtype=torch.int64)
        full[qo[b]:qo[b + 1]] = (t < length).unsqueeze(0)
        causal[qo[b]:qo[b + 1]] = t.unsqueeze(0) <= (length - qrows + (r - qo[b])).unsqueeze(1)
    p.indices, p.causal_mask, p.full_mask = indices, causal, full
    p.batch, p.rows, p.qo = batch, rows, list(qo[:batch + 1])


def attention(p: RefPlan, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, out: torch.Tensor,
              causal: bool, lse: torch.Tensor = None) -> None:
    """portable_gpu_ops.cpp:39-44 on CPU tensors; writes `out` (and `lse`,
    natural log, [rows, hq]) for the rows of every sequence."""
    query = q.reshape(p.rows, p.hq, p.dim)
    keys = k.reshape(p.cache_slots, p.hkv, p.dim)
    values = v.reshape(p.cache_slots, p.hkv, p.dim)
    o = out.view(p.rows, p.hq, p.dim)
    g = p.hq // p.hkv
    for b in range(p.batch):
        lo, hi = p.qo[b], p.qo[b + 1]
        if hi == lo:
            continue
        key = keys.index_select(0, p.indices[b]).repeat_interleave(g, 1).permute(1, 2, 0)
        value = values.index_select(0, p.indices[b]).repeat_interleave(g, 1).permute(1, 0, 2)
        x = query[lo:hi].permute(1, 0, 2).to(torch.float32)
        logits = torch.bmm(x, key.to(torch.float32)) / math.sqrt(float(p.dim))
        mask = (p.causal_mask if causal else p.full_mask)[lo:hi].unsqueeze(0)
        logits.masked_fill_(mask.logical_not(), -math.inf)
        if lse is not None:
            lse[lo:hi] = torch.logsumexp(logits, -1).permute(1, 0)
        result = torch.bmm(torch.softmax(logits, -1), value.to(torch.float32).contiguous())
        o[lo:hi].copy_(result.permute(1, 0, 2))


def run(batch, q, kc, vc, causal: bool, max_pages: int = None, want_lse: bool = True):
    """Convenience: plan + prepare + attention for a feattn.workloads.Batch
    on CPU tensors.  Returns (out, lse)."""
    mp = max_pages if max_pages is not None else batch.max_pages()
    p = create_plan(batch.hq, batch.hkv, q.shape[-1], batch.page, max(1, batch.batch), mp,
                    q.dtype == torch.bfloat16, batch.blocks)
    prepare_plan(p, batch.qo, batch.kv, batch.pages, batch.last, batch.batch, batch.rows)
    out = torch.zeros_like(q)
    lse = torch.full((batch.rows, batch.hq), float("nan"), dtype=torch.float32) if want_lse else None
    attention(p, q, kc, vc, out, causal, lse)
    return out, lse
