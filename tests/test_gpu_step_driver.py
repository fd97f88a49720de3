"""The C++ caller in tests/cpp/step_driver.cpp drives libfeattn.so through
the reference's fe::cuda:: signatures the way src/cuda_model.cpp does (page
allocator with its prefix cache, per-step metadata, q/k RMSNorm + RoPE +
paged append and paged attention per layer, an eager prefill step, a request
that reuses a published prefix's pages, then decode steps replayed from a
captured HIP graph with a padded bucket).  It writes every input and output;
this test replays the same sequence on the oracle: allocator decisions,
metadata and caches bit-exact, attention outputs within 1e-2 abs / 1e-2
rel."""

import os
import struct
import subprocess

import numpy as np
import pytest
import torch

import feattn
from feattn import workloads as W
from oracle import aten_attention as A
from oracle import norm_ops as N
from oracle import step_metadata as S

pytestmark = pytest.mark.gpu

DRIVER = os.path.join(os.path.dirname(feattn.LIB_PATH), "fe_step_driver")
HQ, HKV, D, PAGE, POOL, MAX_LEN, LAYERS = 32, 8, 128, 16, 64, 256, 2
QKV = (HQ + 2 * HKV) * D
CSLOTS = (POOL + 1) * PAGE
DTYPES = {0: np.uint16, 1: np.int32, 2: np.int64, 3: np.float32}


def read_records(path):
    rec = {}
    with open(path, "rb") as f:
        assert f.read(8) == b"FESTEP01"
        while True:
            head = f.read(4)
            if not head:
                return rec
            (n,) = struct.unpack("<I", head)
            name = f.read(n).decode()
            dtype, nd = struct.unpack("<II", f.read(8))
            dims = struct.unpack(f"<{nd}Q", f.read(8 * nd))
            dt = np.dtype(DTYPES[dtype])
            count = int(np.prod(dims)) if dims else 1
            rec[name] = np.frombuffer(f.read(count * dt.itemsize), dtype=dt).reshape(dims)


def bf(a, shape=None):
    t = torch.from_numpy(np.array(a, dtype=np.uint16).view(np.int16)).view(torch.bfloat16)
    return t if shape is None else t.reshape(shape)


def check_step(r, tag, starts, qlens, tables, count, entry_rows):
    """Metadata of one step against oracle.step_metadata (exact)."""
    want = S.prepare(starts, qlens, tables, PAGE, MAX_LEN, count=count, entry_rows=entry_rows, dummy_page=POOL)
    for key in ("qo", "kv", "pages", "last", "positions", "slots"):
        assert r[f"{tag}_{key}"].tolist() == want[key], (tag, key)
    return want


def attention_oracle(m, starts, qlens, tables, q_rows, kc, vc):
    b = W.Batch(hq=HQ, hkv=HKV, page=PAGE, blocks=POOL, starts=starts, qlens=qlens, tables=tables,
                qo=m["qo"], kv=m["kv"], pages=m["pages"], last=m["last"])
    out, _ = A.run(b, q_rows, bf(kc, (POOL + 1, PAGE, HKV, D)), bf(vc, (POOL + 1, PAGE, HKV, D)), True,
                   max_pages=MAX_LEN // PAGE + 1, want_lse=False)
    return out


def test_cpp_step_driver_vs_oracle(dev, tmp_path):
    assert os.path.exists(DRIVER), "fe_step_driver is not built (make -C flashengine.cpp_amd)"
    path = str(tmp_path / "steps.bin")
    res = subprocess.run([DRIVER, path], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stderr
    assert res.stdout.strip().endswith("ok")
    r = read_records(path)
    assert r["buckets"].tolist() == S.graph_buckets(4) == [1, 2, 4]
    table = r["rope_table"]
    blocks = S.Blocks(POOL, PAGE, caching=True)
    ids, lens = [1, 2, 3], [40, 5, 17]
    tokens = {i: r[f"tokens{i}"].tolist() for i in ids}
    kc = [np.zeros((CSLOTS, HKV * D), np.uint16) for _ in range(LAYERS)]
    vc = [np.zeros((CSLOTS, HKV * D), np.uint16) for _ in range(LAYERS)]

    def layer(l, qkv, m, rows, starts, qlens, tables, got_out, got_q=None):
        q, kc[l], vc[l] = N.norm_rope_append(qkv, QKV, r[f"qn{l}"], r[f"kn{l}"], 1e-6, kc[l], vc[l],
                                             np.asarray(m["positions"]), np.asarray(m["slots"]), table, rows,
                                             HQ, HKV, True, MAX_LEN, CSLOTS)
        if got_q is not None:
            assert np.array_equal(got_q.reshape(q.shape), q)
        want = attention_oracle(m, starts, qlens, tables, bf(q, (rows, HQ, D)), kc[l], vc[l])
        torch.testing.assert_close(bf(got_out, (rows, HQ, D)).float(), want.float(), atol=1e-2, rtol=1e-2)

    # step 0: eager prefill of the prompts, then their full pages published
    for i, n in zip(ids, lens):
        assert blocks.probe(i, tokens[i]) == 0
        assert blocks.ensure(i, n)
    tables = [blocks.tables[i] for i in ids]
    m = check_step(r, "s0", [0, 0, 0], lens, tables, 3, 0)
    rows = sum(lens)
    for l in range(LAYERS):
        layer(l, r[f"s0_l{l}_qkv"], m, rows, [0, 0, 0], lens, tables, r[f"s0_l{l}_out"], r[f"s0_l{l}_q"])
    for i, n in zip(ids, lens):
        blocks.publish(i, tokens[i], n)
    # a request sharing sequence 1's first 36 tokens: two shared pages, its
    # last 8 rows computed over them (src/scheduler.cpp:6-17)
    t4 = r["tokens4"].tolist()
    assert t4[:36] == tokens[1][:36] and len(t4) == 40
    cached = blocks.probe(4, t4)
    assert cached == 32 == r["p_cached"][0]
    assert blocks.ensure(4, 40)
    t4_table = blocks.tables[4]
    assert t4_table[:2] == blocks.tables[1][:2] and t4_table[2] not in blocks.tables[1]
    m = check_step(r, "p", [32], [8], [t4_table], 1, 0)
    for l in range(LAYERS):
        layer(l, r[f"p_l{l}_qkv"], m, 8, [32], [8], [t4_table], r[f"p_l{l}_out"], r[f"p_l{l}_q"])
    blocks.forget(4)
    st = blocks.stats()
    assert r["prefix_stats"].tolist() == [st[k] for k in (
        "prefix_requests", "prefix_hit_requests", "prefix_cached_blocks", "prefix_new_blocks",
        "prefix_resident_blocks", "prefix_evictions")] == [4, 1, 2, 3, 3, 0]
    # decode steps 1-3 through the graph of bucket 4 (one padding entry)
    for step in (1, 2, 3):
        starts = list(lens)
        lens = [n + 1 for n in lens]
        for i, n in zip(ids, lens):
            assert blocks.ensure(i, n)
        tables = [blocks.tables[i] for i in ids]
        m = check_step(r, f"s{step}", starts, [1, 1, 1], tables, 4, 1)
        qkv = r[f"s{step}_qkv"].reshape(LAYERS, 4 * QKV)
        out = r[f"s{step}_out"]
        for l in range(LAYERS):
            layer(l, qkv[l], m, 4, starts + [0], [1, 1, 1, 1], tables + [[POOL]], out[l])
    for l in range(LAYERS):
        assert np.array_equal(r[f"final_kc{l}"].reshape(CSLOTS, -1), kc[l])
        assert np.array_equal(r[f"final_vc{l}"].reshape(CSLOTS, -1), vc[l])
