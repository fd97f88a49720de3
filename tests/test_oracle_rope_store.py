"""Pins the numpy RoPE / store restatement (oracle/rope_store.py)."""

import os

import numpy as np
import pytest
import torch

from feattn import workloads as W
from oracle import rope_store as R

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def u16(t):
    return t.view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("bf16", [True, False])
def test_rounding_matches_torch_conversion(bf16):
    g = torch.Generator().manual_seed(0)
    f = torch.randn(200000, generator=g) * torch.exp(torch.randn(200000, generator=g) * 4)
    # exact ties of the 16-bit grids
    ties = (torch.arange(1, 5000, dtype=torch.int32) << 15 | 0x3F800000).view(torch.float32) \
        if bf16 else torch.tensor([1 + 2 ** -11, 1 + 3 * 2 ** -11, 2 ** -24 * 1.5, 65520.0])
    f = torch.cat([f, ties, torch.tensor([0.0, -0.0, float("inf"), -float("inf"), 1e-40])])
    dt = torch.bfloat16 if bf16 else torch.float16
    assert np.array_equal(R.from_f32(f.numpy(), bf16), u16(f.to(dt)))
    back = R.to_f32(u16(f.to(dt)), bf16)
    assert np.array_equal(back, f.to(dt).float().numpy())


@pytest.mark.parametrize("bf16", [True, False])
def test_identity_and_quarter_turn(bf16):
    rows, hq, hkv, d = 3, 2, 1, 128
    dt = torch.bfloat16 if bf16 else torch.float16
    q = u16(torch.randn(rows, hq, d).to(dt))
    k = u16(torch.randn(rows, hkv, d).to(dt))
    pos = np.array([0, 1, 2])
    ident = np.concatenate([np.ones((3, 64)), np.zeros((3, 64))], 1).astype(np.float32)
    q2, k2 = R.rope(q, k, pos, ident, rows, hq, hkv, d, bf16, 3)
    assert np.array_equal(q2, q) and np.array_equal(k2, k)
    quarter = np.concatenate([np.zeros((3, 64)), np.ones((3, 64))], 1).astype(np.float32)
    q3, _ = R.rope(q, k, pos, quarter, rows, hq, hkv, d, bf16, 3)
    neg = R.from_f32(-R.to_f32(q[..., 64:], bf16), bf16)
    assert np.array_equal(q3[..., :64], neg) and np.array_equal(q3[..., 64:], q[..., :64])


@pytest.mark.parametrize("bf16", [True, False])
def test_matches_aten_op_sequence(bf16):
    """Same values as the reference's ATen statement of rope
    (portable_gpu_ops.cpp:50-53) evaluated with torch on the CPU."""
    rows, hq, hkv, d = 9, 4, 2, 128
    dt = torch.bfloat16 if bf16 else torch.float16
    q = (torch.randn(rows, hq, d) * 5).to(dt)
    k = (torch.randn(rows, hkv, d) * 5).to(dt)
    table = W.rope_table(5000, 1e6)
    pos = torch.tensor([0, 3, 99, 4999, 1000, 7, 7, 2500, 1])
    allr = table.index_select(0, pos).unsqueeze(1)
    cs, sn = allr[..., :64], allr[..., 64:]

    def aten(x):
        v = x.float()
        a, b = v[..., :64], v[..., 64:]
        return torch.cat([a * cs - b * sn, b * cs + a * sn], 2).to(dt)

    q2, k2 = R.rope(u16(q), u16(k), pos.numpy(), table.numpy(), rows, hq, hkv, d, bf16, 5000)
    assert np.array_equal(q2, u16(aten(q)))
    assert np.array_equal(k2, u16(aten(k)))


def test_rotation_round_trip():
    rows, d = 4, 128
    x = torch.randn(rows, 1, d)
    q = u16(x.to(torch.bfloat16))
    k = q.copy()
    theta = np.random.default_rng(0).uniform(-3, 3, size=(rows, 64)).astype(np.float32)
    fwd = np.concatenate([np.cos(theta), np.sin(theta)], 1).astype(np.float32)
    bwd = np.concatenate([np.cos(theta), -np.sin(theta)], 1).astype(np.float32)
    pos = np.arange(rows)
    q2, _ = R.rope(q, k, pos, fwd, rows, 1, 1, d, True, rows)
    q3, _ = R.rope(q2, k, pos, bwd, rows, 1, 1, d, True, rows)
    np.testing.assert_allclose(R.to_f32(q3, True), R.to_f32(q, True), atol=0.05, rtol=0.02)


def test_invalid_positions_left_unchanged():
    q = u16(torch.randn(2, 1, 128).to(torch.bfloat16))
    k = q.copy()
    table = W.rope_table(4, 1e6).numpy()
    q2, _ = R.rope(q, k, np.array([-1, 4]), table, 2, 1, 1, 128, True, 4)
    assert np.array_equal(q2, q)


def test_store_skips_padding_and_leaves_other_slots():
    width, slots_n = 16, 48
    kc = np.arange(slots_n * width, dtype=np.uint16).reshape(slots_n, width)
    vc = kc[::-1].copy()
    k = np.full((4, width), 7, np.uint16)
    v = np.full((4, width), 9, np.uint16)
    slots = np.array([3, -1, 47, 20])
    kc2, vc2 = R.store(k, v, kc, vc, slots, 4, width, slots_n)
    for s in range(slots_n):
        if s in (3, 47, 20):
            assert (kc2[s] == 7).all() and (vc2[s] == 9).all()
        else:
            assert np.array_equal(kc2[s], kc[s]) and np.array_equal(vc2[s], vc[s])


@pytest.mark.parametrize("name,bf16", [("rope_bf16.npz", True), ("rope_f16.npz", False)])
def test_golden_rope_fixture(name, bf16):
    g = np.load(os.path.join(GOLDEN, name))
    table = np.zeros((40000, 128), np.float32)
    table[g["pos"]] = g["table_rows"]
    q2, k2 = R.rope(g["q"], g["k"], g["pos"], table, 6, 4, 2, 128, bf16, 40000)
    assert np.array_equal(q2, g["q_out"]) and np.array_equal(k2, g["k_out"])
