"""Writes the golden fixtures under tests/golden/ from the oracle.

    python tests/golden/make_golden.py

Fixtures (small; inputs are regenerated from their seeds and checked by
SHA-256, so only metadata, digests and expected outputs are stored):
  decode_qwen3_06b.npz   4 x 512-token decode, 16/8 heads, randperm(256) pool:
                         expected out (bf16 bits) and natural-log LSE from the
                         ATen restatement, cross-checked here against the
                         float64 brute force before writing.
  rope_bf16.npz / rope_f16.npz
                         rope of 6 rows x (4 q + 2 k heads) x 128 at mixed
                         positions of a theta = 1e6 table: expected bits.
"""

import hashlib
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [ROOT, os.path.join(ROOT, "flashengine.cpp_amd")]

from feattn import workloads as W  # noqa: E402
from oracle import aten_attention, brute, rope_store  # noqa: E402


def digest(t: torch.Tensor) -> str:
    return hashlib.sha256(t.contiguous().view(torch.uint8).numpy().tobytes()).hexdigest()


def decode_fixture():
    b = W.qwen3_06b_decode(seed=1)
    q, kc, vc = W.make_tensors(b, seed=1)
    out, lse = aten_attention.run(b, q, kc, vc, causal=True)
    bo, bl = brute.attention(b.qo, b.kv, b.pages, b.last, b.batch, b.page, q.double().numpy(),
                             kc.double().numpy(), vc.double().numpy(), b.hq, b.hkv, True)
    assert np.abs(out.float().numpy() - bo).max() < 1e-2
    assert np.abs(lse.numpy() - bl).max() < 1e-4
    np.savez_compressed(
        os.path.join(HERE, "decode_qwen3_06b.npz"),
        seed=1, qo=b.qo, kv=b.kv, pages=b.pages, last=b.last, blocks=b.blocks, hq=b.hq,
        hkv=b.hkv, q_sha=digest(q), kc_sha=digest(kc), vc_sha=digest(vc),
        out=out.view(torch.int16).numpy().view(np.uint16), lse=lse.numpy())


def rope_fixture(bf16: bool):
    rows, hq, hkv, dim = 6, 4, 2, 128
    g = torch.Generator().manual_seed(42)
    dt = torch.bfloat16 if bf16 else torch.float16
    q = (torch.randn(rows, hq, dim, generator=g) * 3).to(dt)
    k = (torch.randn(rows, hkv, dim, generator=g) * 3).to(dt)
    table = W.rope_table(40000, 1e6)
    pos = np.array([0, 1, 17, 4095, 32767, 39999], np.int64)
    u16 = lambda t: t.view(torch.int16).numpy().view(np.uint16)
    q2, k2 = rope_store.rope(u16(q), u16(k), pos, table.numpy(), rows, hq, hkv, dim, bf16, 40000)
    name = "rope_bf16.npz" if bf16 else "rope_f16.npz"
    np.savez_compressed(os.path.join(HERE, name), q=u16(q), k=u16(k), pos=pos,
                        table_rows=table.numpy()[pos], q_out=q2, k_out=k2)


if __name__ == "__main__":
    decode_fixture()
    rope_fixture(True)
    rope_fixture(False)
    print("golden fixtures written")
