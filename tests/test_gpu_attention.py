"""GPU parity of fe_attn_run (decode, chunked prefill, DFlash block, mixed,
split-KV) against the oracle, the golden fixture, closed-form known answers
and, when oracle/_ref is built, the reference's own ATen attention on the
same device tensors.  Tolerance (bf16/fp16 outputs): |a-b| <= 1e-2 + 1e-2*|b|;
natural-log LSE: |a-b| <= 1e-3."""

import hashlib
import math
import os

import numpy as np
import pytest
import torch

import feattn
from feattn import workloads as W
from oracle import aten_attention as A
from oracle import ref_lib

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
ATOL = RTOL = 1e-2
LSE_TOL = 1e-3


def hip_attention(b, q, kc, vc, causal, dev, max_pages=None, plan=None):
    bf16 = q.dtype == torch.bfloat16
    own = plan is None
    if own:
        plan = feattn.Plan(b.hq, b.hkv, 128, b.page, max(1, b.batch), max_pages or b.max_pages(),
                           bf16, b.blocks)
    plan.prepare(b.qo, b.kv, b.pages, b.last, b.batch, b.rows)
    qd, kd, vd = q.to(dev), kc.to(dev), vc.to(dev)
    out = torch.zeros_like(qd)
    lse = torch.full((b.rows, b.hq), float("nan"), device=dev)
    plan.run(qd, kd, vd, out, causal=causal, lse=lse)
    torch.cuda.synchronize()
    if own:
        plan.close()
    return out.cpu(), lse.cpu()


def check(out, lse, want_out, want_lse, rows=None):
    if rows is not None:
        out, lse, want_out, want_lse = out[rows], lse[rows], want_out[rows], want_lse[rows]
    torch.testing.assert_close(out.float(), want_out.float(), atol=ATOL, rtol=RTOL)
    torch.testing.assert_close(lse, want_lse, atol=LSE_TOL, rtol=0)


def sub_batch(b, seqs):
    """The chosen sequences of `b` with their page tables (same cache)."""
    sb = W.Batch(hq=b.hq, hkv=b.hkv, page=b.page, blocks=b.blocks,
                 starts=[b.starts[s] for s in seqs], qlens=[b.qlens[s] for s in seqs],
                 tables=[b.tables[s] for s in seqs])
    W.build_metadata(sb)
    rows = torch.cat([torch.arange(b.qo[s], b.qo[s + 1]) for s in seqs])
    return sb, rows


def test_golden_decode_qwen3_06b(dev):
    g = np.load(os.path.join(GOLDEN, "decode_qwen3_06b.npz"))
    b = W.qwen3_06b_decode(seed=int(g["seed"]))
    q, kc, vc = W.make_tensors(b, seed=int(g["seed"]))
    sha = lambda t: hashlib.sha256(t.contiguous().view(torch.uint8).numpy().tobytes()).hexdigest()
    assert sha(kc) == str(g["kc_sha"])
    out, lse = hip_attention(b, q, kc, vc, True, dev)
    want = torch.from_numpy(g["out"].view(np.int16)).view(torch.bfloat16)
    check(out, lse, want, torch.from_numpy(g["lse"]))


CASES = [
    # hq, hkv, starts, qlens
    (32, 8, [511, 0, 3000, 17, 64], [1, 1, 1, 1, 1]),
    (32, 8, [100, 2000, 5], [4, 2, 3]),                      # verify rows (4 x 4 = 16 columns)
    (32, 8, [0, 700, 31], [300, 129, 64]),                   # chunked prefill
    (32, 4, [900, 1, 4096, 1023], [1, 1, 1024, 1]),          # mixed decode + prefill, GQA 8
    (16, 8, [10, 400], [33, 1]),                             # GQA 2
    (8, 8, [130, 0], [7, 50]),                               # MHA
    (40, 8, [60, 250], [1, 90]),                             # GQA 5 (non power of two)
    (16, 2, [1000, 5, 300, 64], [1, 1, 3, 1]),               # hkv 2: 2-wavefront decode workgroups
    (24, 6, [2000, 17, 90, 4000], [1, 2, 40, 1]),            # hkv 6: 2-wavefront decode workgroups
    (24, 8, [700, 2000, 33, 5], [1, 10, 11, 50]),            # GQA 3: 30-column decode items, 33-column tile items
    (48, 8, [900, 17, 3000], [5, 6, 1]),                     # GQA 6
    (128, 8, [1000, 64, 2500], [2, 3, 1]),                   # GQA 16: 2 rows fill a decode item
    (64, 2, [1500, 40], [1, 2]),                             # GQA 32
    (128, 1, [800, 20], [1, 2]),                             # GQA 128: one row is a whole tile item
    (32, 16, [1200, 3, 600], [1, 9, 70]),                    # hkv 16: a decode share spans two workgroups
    (32, 8, [6000, 9000, 300], [200, 64, 40]),               # tile stream cut: one- and two-block chunks
    (40, 5, [7000, 2500, 12000], [48, 20, 33]),              # tile stream cut over 102 shares per kv head
    (32, 8, [3000, 7000, 11000, 1500], [16, 16, 16, 16]),    # tile stream cut: 16-row blocks
]


@pytest.mark.parametrize("case", range(len(CASES)))
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_ragged_batches_vs_oracle(dev, case, causal, dtype):
    hq, hkv, starts, qlens = CASES[case]
    b = W.make_batch(hq, hkv, starts=starts, qlens=qlens, seed=100 + case, extra_pages=3)
    q, kc, vc = W.make_tensors(b, seed=case, dtype=dtype)
    want_out, want_lse = A.run(b, q, kc, vc, causal)
    out, lse = hip_attention(b, q, kc, vc, causal, dev)
    check(out, lse, want_out, want_lse)


def test_uniform_softmax_known_answer(dev):
    """q = 0: every visible key has the same weight; out = mean of visible V."""
    b = W.make_batch(32, 8, starts=[0, 37, 1000], qlens=[70, 1, 16], seed=3)
    q = torch.zeros(b.rows, 32, 128, dtype=torch.bfloat16)
    _, kc, vc = W.make_tensors(b, seed=3)
    out, lse = hip_attention(b, q, kc, vc, True, dev)
    for s in range(b.batch):
        for i in (0, b.qlens[s] - 1):
            r = b.qo[s] + i
            n = b.lens[s] - b.qlens[s] + i + 1
            idx = [b.tables[s][t // 16] * 16 + t % 16 for t in range(n)]
            mean = vc.reshape(-1, 8, 128)[idx].float().mean(0).repeat_interleave(4, 0)
            torch.testing.assert_close(out[r].float(), mean, atol=ATOL, rtol=RTOL)
            assert torch.allclose(lse[r], torch.full((32,), math.log(n)), atol=LSE_TOL)


def test_causal_prefix_known_answer(dev):
    """v_t = t + 1 in every dim, q = k = 0: chunk row i over a prefix of P
    tokens is (P + i + 2) / 2 (tests/ascend_ops_tests.cpp:62-65 pattern)."""
    P, L = 1000, 200
    b = W.make_batch(32, 8, starts=[P], qlens=[L], seed=4)
    q = torch.zeros(L, 32, 128, dtype=torch.bfloat16)
    kc = torch.zeros(b.blocks + 1, 16, 8, 128, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    for t in range(P + L):
        vc[b.tables[0][t // 16], t % 16] = float(t + 1)
    out, _ = hip_attention(b, q, kc, vc, True, dev)
    want = torch.tensor([(P + i + 2) / 2 for i in range(L)]).view(L, 1, 1).expand(L, 32, 128)
    # bf16 V values above 256 are rounded to multiples of 2-8; compare at their resolution
    torch.testing.assert_close(out.float(), want, atol=4.0, rtol=1e-2)
    ref, _ = A.run(b, q, kc, vc, True)
    check(out, torch.zeros(L, 32), ref, torch.zeros(L, 32))


def test_split_kv_long_context(dev):
    b = W.long_decode(batch=3, ctx=32768)
    q, kc, vc = W.make_tensors(b, seed=6)
    counts = feattn.describe(b.hq, b.hkv, 128, 16, b.batch, b.max_pages(), b.blocks, b.qo, b.kv,
                             b.pages, b.last, b.batch, b.rows)
    assert counts[2] == 3  # split + merged
    out, lse = hip_attention(b, q, kc, vc, True, dev)
    want_out, want_lse = A.run(b, q, kc, vc, True)
    check(out, lse, want_out, want_lse)


@pytest.mark.parametrize("name", ["decode8b", "prefill8b", "mixed30b", "dflash_bf16", "dflash_f16", "long16"])
def test_full_size_configs_sampled(dev, name, err_report):
    """The full-size workloads run in one call; a seeded sample of sequences
    is recomputed by the oracle.  The largest errors are reported in the
    session summary (headroom under the tolerance)."""
    causal, dtype = True, "bf16"
    if name == "decode8b":
        b, pick = W.qwen3_8b_decode(), [0, 17, 40, 63]
    elif name == "long16":
        # 16 x 32768: every sequence is cut into several split-KV pieces
        b, pick = W.long_decode(), [0, 7, 15]
    elif name == "prefill8b":
        b, pick = W.qwen3_8b_prefill(), [0, 5]
    elif name == "mixed30b":
        b, pick = W.qwen3_30b_mixed(ndec=256), [0, 100, 255, 256, 257]
    else:
        b, pick = W.dflash_block(), [0, 9, 31]
        causal, dtype = False, ("bf16" if name.endswith("bf16") else "f16")
    q, kc, vc = W.make_tensors(b, seed=7, dtype=dtype, device=dev)
    out, lse = hip_attention(b, q, kc, vc, causal, dev)
    sb, rows = sub_batch(b, pick)
    want_out, want_lse = A.run(sb, q.cpu()[rows], kc.cpu(), vc.cpu(), causal)
    err_report(name, out[rows], lse[rows], want_out, want_lse)
    check(out[rows], lse[rows], want_out, want_lse)
    assert torch.isfinite(out.float()).all()
    if ref_lib.available():
        # the reference's own create_plan / prepare_plan / attention
        # (src/portable_gpu_ops.cpp:18-44) on the same sampled sequences and
        # the same device caches
        ref = ref_lib.attention(sb, q[rows.to(dev)].contiguous(), kc, vc, causal).cpu()
        err_report(name + "_ref", out[rows], None, ref, None)
        torch.testing.assert_close(out[rows].float(), ref.float(), atol=ATOL, rtol=RTOL)


# Sequences sharing their leading pages, as prefix-cache hits leave them
# (BlockManager::probe, src/scheduler.cpp:6-17; tests/host_tests.cpp:35-36):
# (shared prefix pages, [(cached tokens, query rows), ...]) per group.
SHARED = [
    # decode rows and a 16-row block over one 3200-token prefix
    (200, [(3205, 1), (3900, 1), (3200, 1), (3300, 16), (4500, 1)]),
    # chunks over one 1024-token prefix (tile kernel), and a decode row
    (64, [(1024, 100), (1061, 300), (2000, 1), (1024, 64)]),
    # two 32K decode rows sharing 2000 pages: split-KV pieces read the same pages
    (2000, [(32767, 1), (32767, 1)]),
]


def shared_prefix_batch(hq=32, hkv=8):
    return W.make_shared_prefix_batch(hq, hkv, SHARED, seed=77, extra_pages=2)


def test_shared_prefix_tables_share_pages():
    """The generator's tables reuse page ids across sequences (the prefix)
    and nowhere else; no sequence writes a shared page."""
    b = shared_prefix_batch()
    seen = {}
    for s, t in enumerate(b.tables):
        for i, p in enumerate(t):
            seen.setdefault(p, []).append((s, i))
    shared = {p: v for p, v in seen.items() if len(v) > 1}
    assert len(shared) == 200 + 64 + 2000
    assert all(len({i for _, i in v}) == 1 for v in shared.values())  # same position in every table
    for s in range(b.batch):
        for r in range(b.qo[s], b.qo[s + 1]):
            assert b.slots[r] // 16 not in shared


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_shared_prefix_pages_vs_oracle(dev, causal, dtype):
    """Decode, block, chunk and split-KV work over page tables that share
    pages across sequences, against the oracle."""
    b = shared_prefix_batch()
    counts = feattn.describe(b.hq, b.hkv, 128, 16, b.batch, b.max_pages(), b.blocks, b.qo, b.kv,
                             b.pages, b.last, b.batch, b.rows)
    assert counts[0] > 0 and counts[1] > 0 and counts[2] > 0  # decode, tile and merged (split) rows
    q, kc, vc = W.make_tensors(b, seed=78, dtype=dtype)
    want_out, want_lse = A.run(b, q, kc, vc, causal)
    out, lse = hip_attention(b, q, kc, vc, causal, dev)
    check(out, lse, want_out, want_lse)


def test_deterministic(dev):
    b = W.make_batch(32, 8, starts=[5000, 10, 300], qlens=[1, 100, 16], seed=12)
    q, kc, vc = W.make_tensors(b, seed=12)
    o1, l1 = hip_attention(b, q, kc, vc, True, dev)
    o2, l2 = hip_attention(b, q, kc, vc, True, dev)
    assert torch.equal(o1, o2) and torch.equal(l1, l2)


def test_graph_capture_replay_with_new_metadata(dev):
    """rope_append + attention captured once (prepare outside capture,
    reference src/cuda_model.cpp:150-157); replays after prepares with
    different lengths and page tables match eager runs, replay after replay."""
    hq, hkv, nseq = 32, 8, 4
    blocks = 600
    plan = feattn.Plan(hq, hkv, 128, 16, nseq, 130, True, blocks)
    kc = torch.zeros(blocks + 1, 16, hkv, 128, dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    q = torch.zeros(nseq, hq, 128, dtype=torch.bfloat16, device=dev)
    k = torch.zeros(nseq, hkv, 128, dtype=torch.bfloat16, device=dev)
    v = torch.zeros_like(k)
    pos = torch.zeros(nseq, dtype=torch.int64, device=dev)
    slots = torch.full((nseq,), -1, dtype=torch.int64, device=dev)
    table = W.rope_table(4096, 1e6).to(dev)
    out = torch.zeros_like(q)
    lse = torch.zeros(nseq, hq, device=dev)

    def step_meta(seed):
        r = np.random.default_rng(seed)
        starts = r.integers(0, 2000, size=nseq).tolist()
        bb = W.make_batch(hq, hkv, starts=starts, qlens=[1] * nseq, seed=seed, pool=blocks)
        return bb

    def body():
        feattn.rope_append(q, k, v, kc, vc, pos, slots, table, nseq, hq, hkv, 128, True, 4096,
                           (blocks + 1) * 16)
        plan.run(q, kc, vc, out, causal=True, lse=lse)

    def load_step(bb, seed):
        g = torch.Generator(device=dev).manual_seed(seed)
        kc.copy_(torch.randn(kc.shape, generator=g, device=dev).to(torch.bfloat16))
        vc.copy_(torch.randn(vc.shape, generator=g, device=dev).to(torch.bfloat16))
        for t in (q, k, v):
            t.copy_(torch.randn(t.shape, generator=g, device=dev).to(torch.bfloat16))
        pos.copy_(torch.from_numpy(bb.positions))
        slots.copy_(torch.from_numpy(bb.slots))
        plan.prepare(bb.qo, bb.kv, bb.pages, bb.last, bb.batch, bb.rows, graph=True)

    bb = step_meta(0)
    load_step(bb, 0)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        body()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        body()
    for it in range(1, 5):
        bb = step_meta(it)
        load_step(bb, it)
        graph.replay()
        torch.cuda.synchronize()
        got_out, got_lse = out.clone(), lse.clone()
        load_step(bb, it)
        body()
        torch.cuda.synchronize()
        assert torch.equal(got_out, out) and torch.equal(got_lse, lse), it
    plan.close()


@pytest.mark.skipif(not ref_lib.available(), reason="oracle/_ref not built")
@pytest.mark.parametrize("causal", [True, False])
def test_matches_reference_aten_on_device(dev, causal):
    """The reference's own create_plan / prepare_plan / attention
    (src/portable_gpu_ops.cpp) on the same device tensors."""
    for seed, (hq, hkv, starts, qlens) in enumerate([(16, 8, [511] * 4, [1] * 4),
                                                     (32, 8, [0, 300, 2000], [200, 1, 16])]):
        b = W.make_batch(hq, hkv, starts=starts, qlens=qlens, seed=seed, extra_pages=1)
        q, kc, vc = W.make_tensors(b, seed=seed, device=dev)
        ref = ref_lib.attention(b, q, kc, vc, causal).cpu()
        out, _ = hip_attention(b, q, kc, vc, causal, dev)
        torch.testing.assert_close(out.float(), ref.float(), atol=ATOL, rtol=RTOL)


@pytest.mark.skipif(not ref_lib.available(), reason="oracle/_ref not built")
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_shared_prefix_pages_vs_reference_aten(dev, causal, dtype, err_report):
    """Page tables sharing prefix pages through the reference's own ATen
    attention (src/portable_gpu_ops.cpp:27-44) on the same device tensors."""
    b = shared_prefix_batch()
    q, kc, vc = W.make_tensors(b, seed=79, dtype=dtype, device=dev)
    ref = ref_lib.attention(b, q, kc, vc, causal).cpu()
    out, _ = hip_attention(b, q, kc, vc, causal, dev)
    err_report(f"shared_{dtype}_{'c' if causal else 'nc'}_ref", out, None, ref, None)
    torch.testing.assert_close(out.float(), ref.float(), atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("seed", range(16))
def test_random_batches_vs_oracle(dev, seed):
    """Seeded random ragged batches (the planner's random-batch generator:
    head layout, decode rows, short blocks, longer chunks, prefixes up to
    6000 tokens) through both masks against the oracle; between them they
    take the longest-first list, the stream cut, split and unsplit rows."""
    from test_planner import HEAD_LAYOUTS

    rng = np.random.default_rng(1000 + seed)
    hq, hkv = HEAD_LAYOUTS[seed % len(HEAD_LAYOUTS)]
    batch = int(rng.integers(1, 9))
    qlens, starts = [], []
    for _ in range(batch):
        kind = rng.integers(0, 3)
        qlens.append(int(1 if kind == 0 else rng.integers(2, 33) if kind == 1 else rng.integers(33, 161)))
        starts.append(int(rng.integers(0, 6001)))
    b = W.make_batch(hq, hkv, starts=starts, qlens=qlens, seed=seed, extra_pages=int(rng.integers(0, 3)))
    q, kc, vc = W.make_tensors(b, seed=500 + seed)
    for causal in (True, False):
        want_out, want_lse = A.run(b, q, kc, vc, causal)
        out, lse = hip_attention(b, q, kc, vc, causal, dev)
        check(out, lse, want_out, want_lse)
