"""Pins the ATen restatement (oracle/aten_attention.py) before it is trusted:
closed-form known answers (reference tests/ascend_ops_tests.cpp:21,44,49-51,
62-65), GQA head permutation, float64 brute force, and the golden fixture."""

import hashlib
import math
import os

import numpy as np
import pytest
import torch

from feattn import workloads as W
from oracle import aten_attention as A
from oracle import brute

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def fill_rows(kc, b, values_of_token):
    """Writes per-token values (broadcast over heads and dims) into the cache
    at each sequence's slots."""
    for s, table in enumerate(b.tables):
        for t in range(b.lens[s]):
            pg, off = table[t // b.page], t % b.page
            kc[pg, off] = values_of_token(s, t)


def test_uniform_softmax_mean_of_visible_rows():
    b = W.make_batch(8, 4, starts=[0, 9, 40], qlens=[5, 1, 17], seed=11)
    q = torch.zeros(b.rows, 8, 128, dtype=torch.bfloat16)
    kc = torch.zeros(b.blocks + 1, 16, 4, 128, dtype=torch.bfloat16)
    vc = torch.randn(b.blocks + 1, 16, 4, 128).to(torch.bfloat16)
    for causal in (True, False):
        out, lse = A.run(b, q, kc, vc, causal)
        for s in range(b.batch):
            for i in range(b.qlens[s]):
                r = b.qo[s] + i
                n = b.lens[s] - b.qlens[s] + i + 1 if causal else b.lens[s]
                toks = [(b.tables[s][t // 16], t % 16) for t in range(n)]
                mean = torch.stack([vc[p, o].float() for p, o in toks]).mean(0)  # [hkv, d]
                want = mean.repeat_interleave(2, 0)
                torch.testing.assert_close(out[r].float(), want, atol=1e-2, rtol=1e-2)
                assert torch.allclose(lse[r], torch.full((8,), math.log(n)), atol=1e-5)


def test_causal_known_answer_over_prefix():
    """v_t = t + 1, q = k = 0: chunk row i over prefix P -> (P + i + 2) / 2."""
    P, L = 37, 21
    b = W.make_batch(2, 1, starts=[P], qlens=[L], seed=5)
    q = torch.zeros(L, 2, 128, dtype=torch.bfloat16)
    kc = torch.zeros(b.blocks + 1, 16, 1, 128, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    fill_rows(vc, b, lambda s, t: float(t + 1))
    out, _ = A.run(b, q, kc, vc, True)
    for i in range(L):
        assert torch.allclose(out[i].float(), torch.full((2, 128), (P + i + 2) / 2), rtol=4e-3)


def test_ragged_isolation():
    """Two sequences of 3 and 13 rows with no prefix: no row reads the other
    sequence's V (ascend_ops_tests.cpp:49-51)."""
    b = W.make_batch(2, 1, starts=[0, 0], qlens=[3, 13], seed=6)
    q = torch.zeros(16, 2, 128, dtype=torch.bfloat16)
    kc = torch.zeros(b.blocks + 1, 16, 1, 128, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    fill_rows(vc, b, lambda s, t: float(t + 1) if s == 0 else 100.0 + t)
    out, _ = A.run(b, q, kc, vc, True)
    for r in range(16):
        want = (r + 2) / 2 if r < 3 else 100.0 + (r - 3) / 2
        assert abs(out[r, 0, 0].float().item() - want) <= 0.5 + 4e-3 * want


def test_noncausal_block_sees_whole_block():
    C, n = 40, 16
    b = W.make_batch(4, 2, starts=[C], qlens=[n], seed=8)
    q = torch.zeros(n, 4, 128, dtype=torch.bfloat16)
    kc = torch.zeros(b.blocks + 1, 16, 2, 128, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    fill_rows(vc, b, lambda s, t: float(t + 1))
    out, lse = A.run(b, q, kc, vc, False)
    want = (C + n + 1) / 2
    assert torch.allclose(out.float(), torch.full_like(out.float(), want), rtol=4e-3)
    assert torch.allclose(lse, torch.full_like(lse, math.log(C + n)), atol=1e-5)


def test_gqa_head_permutation():
    b = W.make_batch(8, 2, starts=[30, 3], qlens=[1, 6], seed=9)
    q, kc, vc = W.make_tensors(b, seed=9)
    perm = torch.tensor([1, 3, 0, 2, 6, 4, 7, 5])  # within groups {0..3}, {4..7}
    out, lse = A.run(b, q, kc, vc, True)
    out2, lse2 = A.run(b, q[:, perm].contiguous(), kc, vc, True)
    assert torch.equal(out2, out[:, perm])
    assert torch.equal(lse2, lse[:, perm])


@pytest.mark.parametrize("seed", [0, 1, 2])
@pytest.mark.parametrize("causal", [True, False])
def test_against_float64_brute_force(seed, causal):
    r = np.random.default_rng(seed)
    hkv = int(r.choice([1, 2, 4]))
    hq = hkv * int(r.choice([1, 2, 4]))
    n = int(r.integers(1, 4))
    qlens = [int(x) for x in r.integers(1, 20, size=n)]
    starts = [int(x) for x in r.integers(0, 50, size=n)]
    b = W.make_batch(hq, hkv, starts=starts, qlens=qlens, seed=seed, extra_pages=2)
    q, kc, vc = W.make_tensors(b, seed=seed)
    out, lse = A.run(b, q, kc, vc, causal)
    bo, bl = brute.attention(b.qo, b.kv, b.pages, b.last, b.batch, b.page, q.double().numpy(),
                             kc.double().numpy(), vc.double().numpy(), hq, hkv, causal)
    # the oracle rounds its fp32 result to bf16 once: <= half a bf16 ulp
    np.testing.assert_allclose(out.float().numpy(), bo, atol=2e-3, rtol=4e-3)
    np.testing.assert_allclose(lse.numpy(), bl, atol=1e-5, rtol=0)


def test_golden_decode_fixture():
    g = np.load(os.path.join(GOLDEN, "decode_qwen3_06b.npz"))
    b = W.qwen3_06b_decode(seed=int(g["seed"]))
    assert b.qo == g["qo"].tolist() and b.pages == g["pages"].tolist()
    q, kc, vc = W.make_tensors(b, seed=int(g["seed"]))
    sha = lambda t: hashlib.sha256(t.contiguous().view(torch.uint8).numpy().tobytes()).hexdigest()
    assert sha(q) == str(g["q_sha"]) and sha(kc) == str(g["kc_sha"]) and sha(vc) == str(g["vc_sha"])
    out, lse = A.run(b, q, kc, vc, True)
    want = torch.from_numpy(g["out"].view(np.int16)).view(torch.bfloat16)
    torch.testing.assert_close(out.float(), want.float(), atol=1e-2, rtol=1e-2)
    np.testing.assert_allclose(lse.numpy(), g["lse"], atol=1e-4)


def test_prepare_rejects_like_reference():
    p = A.create_plan(4, 2, 128, 16, 1, 3, True, 8)
    with pytest.raises(RuntimeError):
        A.prepare_plan(p, [0, 1, 2], [0, 1, 2], [0, 1], [1, 1], 2, 2)  # batch > max_batch
    with pytest.raises(RuntimeError):
        A.prepare_plan(p, [0, 5], [0, 1], [0], [3], 1, 5)  # len 3 < 5 rows
