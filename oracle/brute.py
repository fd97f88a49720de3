"""ORACLE (test infrastructure only): float64 brute-force paged attention.

Straight from the definition in the reference's interface comment and ATen
statement (src/portable_gpu_ops.cpp:30-31,39-44): for each sequence b, row i,
head h, key t visible if t <= len - qlen + i (causal) or t < len (full);
logits = q . k / sqrt(dim); output = softmax-weighted V; lse = log-sum-exp.
Scalar Python loops over the page table, no torch kernels, so it checks the
torch-CPU restatement independently.  Tiny shapes only.
"""

from __future__ import annotations

import math

import numpy as np


def attention(qo, kv, pages, last, batch, page, q, kc, vc, hq, hkv, causal):
    """q: float64 [rows, hq, d]; kc, vc: float64 [blocks+1, page, hkv, d].
    Returns (out float64 [rows, hq, d], lse float64 [rows, hq])."""
    rows = q.shape[0]
    d = q.shape[2]
    g = hq // hkv
    out = np.zeros_like(q)
    lse = np.full((rows, hq), np.nan)
    for b in range(batch):
        length = (kv[b + 1] - kv[b] - 1) * page + last[b]
        qlen = qo[b + 1] - qo[b]
        for i in range(qlen):
            r = qo[b] + i
            limit = length - qlen + i if causal else length - 1
            for h in range(hq):
                kh = h // g
                logits = []
                vals = []
                for t in range(limit + 1):
                    pg = pages[kv[b] + t // page]
                    off = t % page
                    kvec = kc[pg, off, kh]
                    logits.append(float(np.dot(q[r, h], kvec)) / math.sqrt(d))
                    vals.append(vc[pg, off, kh])
                mx = max(logits)
                w = [math.exp(x - mx) for x in logits]
                s = sum(w)
                out[r, h] = sum(wi * vi for wi, vi in zip(w, vals)) / s
                lse[r, h] = mx + math.log(s)
    return out, lse
