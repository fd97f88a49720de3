"""Seeded synthetic paged-attention workloads.

Host metadata follows the reference's per-step builder, CudaModel::prepare
(src/cuda_model.cpp:131-142): a sequence with `start` cached tokens and `rows`
new query rows has positions start..start+rows-1, write slots
blocks[pos // page] * page + pos % page, contributes `rows` to the query CSR
(qo), ceil(len / page) page ids to the page CSR (kv, pages) with
len = start + rows, and last = (len - 1) % page + 1.  The KV caches have
blocks + 1 pages; page id `blocks` is the padding ("dummy") page
(src/cuda_model.cpp:60,115).

Tensor contents are i.i.d. N(0, 1) drawn from one seeded CPU generator per
stream (lengths, permutation, q, k, v) so the GPU path and the oracle see the
same bytes.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import List, Optional, Sequence

import numpy as np

PAGE = 16
HEAD_DIM = 128


@dataclass
class Batch:
    hq: int
    hkv: int
    page: int
    blocks: int                 # number of real pages; page id `blocks` is the dummy page
    starts: List[int]           # cached tokens before this step, per sequence
    qlens: List[int]            # query rows per sequence this step
    tables: List[List[int]]     # page table (block list) per sequence
    qo: List[int] = field(default_factory=list)
    kv: List[int] = field(default_factory=list)
    pages: List[int] = field(default_factory=list)
    last: List[int] = field(default_factory=list)
    positions: Optional[np.ndarray] = None   # int64 [rows]
    slots: Optional[np.ndarray] = None       # int64 [rows]

    @property
    def batch(self) -> int:
        return len(self.qlens)

    @property
    def rows(self) -> int:
        return self.qo[-1] if self.qo else 0

    @property
    def lens(self) -> List[int]:
        return [s + q for s, q in zip(self.starts, self.qlens)]

    @property
    def group(self) -> int:
        return self.hq // self.hkv

    @property
    def cache_slots(self) -> int:
        return (self.blocks + 1) * self.page

    def max_pages(self) -> int:
        """Plan capacity as the reference sizes it: ceil(max_len / page) + 1
        (src/cuda_model.cpp:118)."""
        return max(1, math.ceil(max(self.lens, default=1) / self.page)) + 1


def build_metadata(b: Batch) -> Batch:
    """CudaModel::prepare (src/cuda_model.cpp:131-142) for real sequences."""
    qo, kv, pages, last, pos, slots = [0], [0], [], [], [], []
    for start, rows, table in zip(b.starts, b.qlens, b.tables):
        length = start + rows
        for j in range(rows):
            p = start + j
            if p // b.page >= len(table):
                raise ValueError("page table does not cover the write slot")
            pos.append(p)
            slots.append(table[p // b.page] * b.page + p % b.page)
        qo.append(qo[-1] + rows)
        n = (length + b.page - 1) // b.page
        if n > len(table):
            raise ValueError("page table does not cover the context")
        pages.extend(table[:n])
        kv.append(len(pages))
        last.append((length - 1) % b.page + 1)
    b.qo, b.kv, b.pages, b.last = qo, kv, pages, last
    b.positions = np.asarray(pos, dtype=np.int64)
    b.slots = np.asarray(slots, dtype=np.int64)
    return b


def make_batch(hq: int, hkv: int, starts: Sequence[int], qlens: Sequence[int], seed: int,
               page: int = PAGE, pool: Optional[int] = None, extra_pages: int = 0) -> Batch:
    """Assigns pages from a seeded random permutation of a pool of `pool`
    pages (default: exactly the pages the batch needs) in sequence order."""
    import torch

    need = [math.ceil((s + q) / page) for s, q in zip(starts, qlens)]
    total = sum(need) + extra_pages
    pool = total if pool is None else pool
    if pool < total:
        raise ValueError("page pool too small")
    g = torch.Generator().manual_seed(seed * 7919 + 1)
    perm = torch.randperm(pool, generator=g).tolist()
    tables, off = [], 0
    for n in need:
        tables.append(perm[off:off + n])
        off += n
    b = Batch(hq=hq, hkv=hkv, page=page, blocks=pool, starts=list(starts), qlens=list(qlens),
              tables=tables)
    return build_metadata(b)


def make_shared_prefix_batch(hq: int, hkv: int, groups, seed: int, page: int = PAGE,
                             extra_pages: int = 0) -> Batch:
    """Page tables that share pages across sequences, as a prefix-cache hit
    produces them: BlockManager::probe (src/scheduler.cpp:6-17) hands every
    sequence whose leading tokens match a published prefix the same page ids
    for those whole pages, and the sequence's later pages come from the free
    list (src/scheduler.cpp:31-33).  `groups` is a list of
    (prefix_pages, [(start, qlen), ...]): each sequence of a group reuses the
    group's prefix_pages page ids for its first prefix_pages * page tokens
    and gets pages of its own for the rest.  Shared pages are never written
    (src/scheduler.cpp:10), so start >= prefix_pages * page.  Page ids come
    from one seeded permutation of the pool, shared prefixes first."""
    import torch

    seqs, own_need, pre_need = [], [], 0
    for npre, members in groups:
        pre_need += npre
        for start, qlen in members:
            if start < npre * page:
                raise ValueError("a shared prefix page would be written")
            seqs.append((start, qlen))
            own_need.append(math.ceil((start + qlen) / page) - npre)
    pool = pre_need + sum(own_need) + extra_pages
    g = torch.Generator().manual_seed(seed * 7919 + 3)
    perm = torch.randperm(pool, generator=g).tolist()
    off, k, tables = pre_need, 0, []
    pre_off = 0
    for npre, members in groups:
        prefix = perm[pre_off:pre_off + npre]
        pre_off += npre
        for _ in members:
            tables.append(prefix + perm[off:off + own_need[k]])
            off += own_need[k]
            k += 1
    b = Batch(hq=hq, hkv=hkv, page=page, blocks=pool, starts=[s for s, _ in seqs],
              qlens=[q for _, q in seqs], tables=tables)
    return build_metadata(b)


def randn_bf16(shape, seed: int, dtype="bf16", device="cpu"):
    """N(0,1) fp32 from a seeded generator, rounded to bf16/fp16 (RNE)."""
    import torch

    if device == "cpu":
        g = torch.Generator().manual_seed(seed)
        x = torch.randn(shape, generator=g, dtype=torch.float32)
    else:
        g = torch.Generator(device=device).manual_seed(seed)
        x = torch.randn(shape, generator=g, dtype=torch.float32, device=device)
    return x.to(torch.bfloat16 if dtype == "bf16" else torch.float16)


def make_tensors(b: Batch, seed: int, dtype="bf16", device="cpu"):
    """q [rows, hq, 128]; k/v caches [blocks+1, page, hkv, 128], every slot
    (stale and dummy ones included) filled with N(0,1)."""
    q = randn_bf16((b.rows, b.hq, HEAD_DIM), seed * 3 + 11, dtype, device)
    kc = randn_bf16((b.blocks + 1, b.page, b.hkv, HEAD_DIM), seed * 3 + 12, dtype, device)
    vc = randn_bf16((b.blocks + 1, b.page, b.hkv, HEAD_DIM), seed * 3 + 13, dtype, device)
    return q, kc, vc


def rope_table(max_positions: int, theta: float, dim: int = HEAD_DIM):
    """fp32 cos|sin table as built at model init (src/cuda_model.cpp:44-47),
    computed on the CPU in float32: inv = 1 / theta^(arange(0,d,2)/d),
    freqs = arange(max_len) x inv, table = cat(cos(freqs), sin(freqs))."""
    import torch

    inv = 1.0 / torch.pow(torch.tensor(theta, dtype=torch.float32),
                          torch.arange(0, dim, 2, dtype=torch.float32) / dim)
    freqs = torch.arange(max_positions, dtype=torch.float32).unsqueeze(1) * inv.unsqueeze(0)
    return torch.cat([freqs.cos(), freqs.sin()], 1).contiguous()


# ---------------------------------------------------------------------------
# The five workload configurations (seeded).
# ---------------------------------------------------------------------------

def _rng(seed):
    return np.random.default_rng(seed)


def qwen3_06b_decode(seed: int = 1) -> Batch:
    """16 q heads / 8 kv heads; 4 sequences x 512 cached tokens (the decode
    row included); pages from randperm(256) of a 256-page pool."""
    return make_batch(16, 8, starts=[511] * 4, qlens=[1] * 4, seed=seed, pool=256)


def qwen3_8b_decode(seed: int = 2, batch: int = 64, lo: int = 512, hi: int = 4096) -> Batch:
    """32 q heads / 8 kv heads; 64 sequences, context ~ U{512..4096}; pool =
    pages needed + 1 padding page."""
    ctx = _rng(seed).integers(lo, hi + 1, size=batch).tolist()
    return make_batch(32, 8, starts=[c - 1 for c in ctx], qlens=[1] * batch, seed=seed,
                      extra_pages=1)


def qwen3_8b_prefill(seed: int = 3, nseq: int = 8, budget: int = 8192, min_chunk: int = 64,
                     max_prefix: int = 2048) -> Batch:
    """Chunked prefill: 8 sequences, cached prefix ~ U{0..2048}; chunk lengths
    >= 64 summing to the 8192-token batch budget (64 each plus a seeded
    multinomial split of the rest)."""
    r = _rng(seed)
    prefix = r.integers(0, max_prefix + 1, size=nseq).tolist()
    rest = budget - nseq * min_chunk
    extra = r.multinomial(rest, np.full(nseq, 1.0 / nseq)).tolist()
    chunks = [min_chunk + e for e in extra]
    return make_batch(32, 8, starts=prefix, qlens=chunks, seed=seed, extra_pages=1)


def qwen3_30b_mixed(seed: int = 4, ndec: int = 256, lo: int = 1024, hi: int = 8192,
                    npre: int = 2, chunk: int = 1024, prefix: int = 4096) -> Batch:
    """32 q heads / 4 kv heads: 256 decode sequences (context ~ U{1024..8192})
    and 2 chunked prefills of 1024 tokens over 4096 cached, one shared pool."""
    ctx = _rng(seed).integers(lo, hi + 1, size=ndec).tolist()
    starts = [c - 1 for c in ctx] + [prefix] * npre
    qlens = [1] * ndec + [chunk] * npre
    return make_batch(32, 4, starts=starts, qlens=qlens, seed=seed, extra_pages=1)


def dflash_block(seed: int = 5, batch: int = 32, block: int = 16, lo: int = 2048,
                 hi: int = 16384) -> Batch:
    """DFlash block verify: 16-row draft blocks attending non-causally to
    themselves plus a context ~ U{2048..16384}."""
    ctx = _rng(seed).integers(lo, hi + 1, size=batch).tolist()
    return make_batch(32, 8, starts=ctx, qlens=[block] * batch, seed=seed, extra_pages=1)


def long_decode(seed: int = 6, batch: int = 16, ctx: int = 32768) -> Batch:
    """Long-context decode: 16 sequences x 32768 tokens."""
    return make_batch(32, 8, starts=[ctx - 1] * batch, qlens=[1] * batch, seed=seed,
                      extra_pages=1)


# ---------------------------------------------------------------------------
# Algorithmic work units (visible key positions only; page padding excluded).
# ---------------------------------------------------------------------------

def kv_bytes_per_token(hkv: int, elem: int = 2) -> int:
    return 2 * hkv * HEAD_DIM * elem


def visible_pairs(b: Batch, causal: bool) -> int:
    """Sum over query rows of visible keys: causal chunk of L over prefix P
    gives L*P + L(L+1)/2; non-causal gives L*(P+L)."""
    tot = 0
    for start, L in zip(b.starts, b.qlens):
        if causal:
            tot += L * start + L * (L + 1) // 2
        else:
            tot += L * (start + L)
    return tot


def attention_flops(b: Batch, causal: bool) -> int:
    """4 * hq * 128 per visible (row, key) pair (QK^T and PV)."""
    return 4 * b.hq * HEAD_DIM * visible_pairs(b, causal)


def decode_bytes(b: Batch, elem: int = 2) -> int:
    """sum_b ctx_b * KVB + q in + o out + 4 B per page id read."""
    kvb = kv_bytes_per_token(b.hkv, elem)
    ctx = sum(b.lens)
    q_o = 2 * b.rows * b.hq * HEAD_DIM * elem
    page_ids = 4 * sum(math.ceil(l / b.page) for l in b.lens)
    return ctx * kvb + q_o + page_ids


def norm_rope_append_bytes(b: Batch, elem: int = 2) -> int:
    """Fused q/k norm + RoPE + append per new token: the q|k|v projection
    row read, q written, k and v cache writes, pos and slot reads, the cos|sin
    row read (the two 128-element weights stay in cache)."""
    per_row = ((b.hq + 2 * b.hkv) * HEAD_DIM * elem + b.hq * HEAD_DIM * elem + 2 * b.hkv * HEAD_DIM * elem
               + 16 + HEAD_DIM * 4)
    return b.rows * per_row


def rope_bytes(b: Batch, elem: int = 2) -> int:
    """In-place RoPE of the new tokens (fe_rope): q and k read and written,
    the pos read, the cos|sin row read: per new token."""
    return b.rows * (2 * (b.hq + b.hkv) * HEAD_DIM * elem + 8 + HEAD_DIM * 4)


def store_bytes(b: Batch, elem: int = 2) -> int:
    """Paged store of the new tokens (fe_store): k and v read, k and v cache
    writes, the slot read: per new token."""
    return b.rows * (4 * b.hkv * HEAD_DIM * elem + 8)


def rope_append_bytes(b: Batch, elem: int = 2) -> int:
    """q read+write, k and v read, k and v cache writes, pos and slot reads,
    the cos|sin row read: per new token."""
    per_row = (2 * b.hq * HEAD_DIM * elem + 4 * b.hkv * HEAD_DIM * elem + 16
               + HEAD_DIM * 4)
    return b.rows * per_row
