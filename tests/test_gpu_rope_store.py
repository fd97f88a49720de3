"""GPU parity of fe_rope / fe_store / fe_rope_append against the oracle
(bit-exact), and against the reference's own ATen ops when oracle/_ref is
built."""

import os

import numpy as np
import pytest
import torch

import feattn
from feattn import workloads as W
from oracle import ref_lib
from oracle import rope_store as R

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def u16(t):
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


def dtype_of(bf16):
    return torch.bfloat16 if bf16 else torch.float16


@pytest.mark.parametrize("bf16", [True, False])
def test_rope_golden(dev, bf16):
    g = np.load(os.path.join(GOLDEN, "rope_bf16.npz" if bf16 else "rope_f16.npz"))
    table = torch.zeros(40000, 128)
    table[torch.from_numpy(g["pos"])] = torch.from_numpy(g["table_rows"])
    dt = dtype_of(bf16)
    q = torch.from_numpy(g["q"].view(np.int16)).view(dt).to(dev)
    k = torch.from_numpy(g["k"].view(np.int16)).view(dt).to(dev)
    pos = torch.from_numpy(g["pos"]).to(dev)
    feattn.rope(q, k, pos, table.to(dev), 6, 4, 2, 128, bf16, 40000)
    torch.cuda.synchronize()
    assert np.array_equal(u16(q), g["q_out"]) and np.array_equal(u16(k), g["k_out"])


@pytest.mark.parametrize("bf16", [True, False])
@pytest.mark.parametrize("hq,hkv,rows", [(32, 8, 333), (16, 8, 5), (40, 8, 64)])
def test_rope_bit_exact(dev, bf16, hq, hkv, rows):
    dt = dtype_of(bf16)
    gen = torch.Generator().manual_seed(rows + hq)
    q = (torch.randn(rows, hq, 128, generator=gen) * 4).to(dt)
    k = (torch.randn(rows, hkv, 128, generator=gen) * 4).to(dt)
    table = W.rope_table(8192, 1e6)
    pos = torch.randint(0, 8192, (rows,), generator=gen)
    pos[0] = -1  # out of range: row left unchanged
    pos[-1] = 8192
    want_q, want_k = R.rope(u16(q), u16(k), pos.numpy(), table.numpy(), rows, hq, hkv, 128, bf16,
                            8192)
    qd, kd = q.to(dev), k.to(dev)
    feattn.rope(qd, kd, pos.to(dev), table.to(dev), rows, hq, hkv, 128, bf16, 8192)
    torch.cuda.synchronize()
    assert np.array_equal(u16(qd), want_q)
    assert np.array_equal(u16(kd), want_k)


def _plant_specials(t, seed):
    """Writes bf16 special values at seeded positions of t: NaNs with
    several payloads and signs (quiet and signalling), infinities, values
    whose rotation overflows, subnormals and signed zeros."""
    specials = [0x7FC0, 0x7FC1, 0x7F81, 0xFFC0, 0x7FFF, 0x7F80, 0xFF80, 0x7F7F, 0xFF7F, 0x0001, 0x8001,
                0x007F, 0x0000, 0x8000]
    flat = t.view(torch.int16).view(-1)
    gen = torch.Generator().manual_seed(seed)
    idx = torch.randperm(flat.numel(), generator=gen)[:8 * len(specials)]
    for j, i in enumerate(idx.tolist()):
        flat[i] = np.int16(np.uint16(specials[j % len(specials)]))
    return t


@pytest.mark.parametrize("hq,hkv,rows", [(32, 8, 61), (16, 8, 7)])
def test_rope_special_values_bit_exact(dev, hq, hkv, rows):
    """bf16 rounding of NaN (0x7fc0 whatever the payload), infinities,
    overflow and subnormals matches the oracle bit for bit, in fe_rope and
    in the fused append."""
    gen = torch.Generator().manual_seed(rows)
    q = _plant_specials((torch.randn(rows, hq, 128, generator=gen) * 4).to(torch.bfloat16), 1)
    k = _plant_specials((torch.randn(rows, hkv, 128, generator=gen) * 4).to(torch.bfloat16), 2)
    v = torch.randn(rows, hkv, 128, generator=gen).to(torch.bfloat16)
    table = W.rope_table(8192, 1e6)
    pos = torch.randint(0, 8192, (rows,), generator=gen)
    with np.errstate(all="ignore"):  # inf * 0 and overflow are the point here
        want_q, want_k = R.rope(u16(q), u16(k), pos.numpy(), table.numpy(), rows, hq, hkv, 128, True, 8192)
    qd, kd = q.to(dev), k.to(dev)
    feattn.rope(qd, kd, pos.to(dev), table.to(dev), rows, hq, hkv, 128, True, 8192)
    torch.cuda.synchronize()
    assert np.array_equal(u16(qd), want_q)
    assert np.array_equal(u16(kd), want_k)
    slots = torch.randperm(4 * rows, generator=gen)[:rows].clone()
    kc = torch.zeros(4 * rows, hkv, 128, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    with np.errstate(all="ignore"):
        wq, wkc, wvc = R.rope_append(u16(q), u16(k), u16(v), u16(kc), u16(vc), pos.numpy(), slots.numpy(),
                                     table.numpy(), rows, hq, hkv, 128, True, 8192, 4 * rows)
    qd, kcd, vcd = q.to(dev), kc.to(dev), vc.to(dev)
    feattn.rope_append(qd, k.to(dev), v.to(dev), kcd, vcd, pos.to(dev), slots.to(dev), table.to(dev), rows, hq,
                       hkv, 128, True, 8192, 4 * rows)
    torch.cuda.synchronize()
    assert np.array_equal(u16(qd), wq)
    assert np.array_equal(u16(kcd).reshape(wkc.shape), wkc)
    assert np.array_equal(u16(vcd).reshape(wvc.shape), wvc)


def test_rope_rejects_alias(dev):
    q = torch.zeros(2, 2, 128, dtype=torch.bfloat16, device=dev)
    pos = torch.zeros(2, dtype=torch.int64, device=dev)
    table = torch.zeros(4, 128, device=dev)
    with pytest.raises(RuntimeError, match="alias"):
        feattn.rope(q, q, pos, table, 2, 2, 2, 128, True, 4)


@pytest.mark.parametrize("width", [1024, 512, 36])
def test_store_with_sentinels(dev, width):
    """Padding rows (slot -1) are skipped; every other slot, and guard
    regions before and after the caches, stay untouched."""
    slots_n, rows = 200, 50
    gen = torch.Generator().manual_seed(width)
    slots = torch.randperm(slots_n, generator=gen)[:rows]
    slots[::7] = -1
    k = torch.randint(-30000, 30000, (rows, width), generator=gen, dtype=torch.int16)
    v = torch.randint(-30000, 30000, (rows, width), generator=gen, dtype=torch.int16)
    guard = 8 * width
    kc = torch.randint(-30000, 30000, (slots_n * width + 2 * guard,), generator=gen,
                       dtype=torch.int16)
    vc = kc.flip(0).clone()
    want_k, want_v = R.store(k.numpy().view(np.uint16), v.numpy().view(np.uint16),
                             kc[guard:-guard].numpy().view(np.uint16),
                             vc[guard:-guard].numpy().view(np.uint16), slots.numpy(), rows, width,
                             slots_n)
    kcd, vcd = kc.to(dev), vc.to(dev)
    feattn.store(k.to(dev), v.to(dev), kcd[guard:-guard], vcd[guard:-guard], slots.to(dev), rows,
                 width, True, slots_n)
    torch.cuda.synchronize()
    kcd, vcd = kcd.cpu(), vcd.cpu()
    assert torch.equal(kcd[:guard], kc[:guard]) and torch.equal(kcd[-guard:], kc[-guard:])
    assert torch.equal(vcd[:guard], vc[:guard]) and torch.equal(vcd[-guard:], vc[-guard:])
    assert np.array_equal(kcd[guard:-guard].numpy().view(np.uint16).reshape(slots_n, width), want_k)
    assert np.array_equal(vcd[guard:-guard].numpy().view(np.uint16).reshape(slots_n, width), want_v)


@pytest.mark.parametrize("bf16", [True, False])
def test_rope_append_matches_rope_then_store(dev, bf16):
    """Fused append == the reference's per-layer rope then store
    (src/cuda_model.cpp:94-95), bit for bit, on a chunked-prefill batch."""
    b = W.make_batch(32, 8, starts=[0, 100, 1000], qlens=[77, 16, 200], seed=21, extra_pages=3)
    dt = dtype_of(bf16)
    gen = torch.Generator().manual_seed(5)
    q = torch.randn(b.rows, 32, 128, generator=gen).to(dt)
    k = torch.randn(b.rows, 8, 128, generator=gen).to(dt)
    v = torch.randn(b.rows, 8, 128, generator=gen).to(dt)
    kc = torch.randn(b.blocks + 1, 16, 8, 128, generator=gen).to(dt)
    vc = torch.randn(b.blocks + 1, 16, 8, 128, generator=gen).to(dt)
    slots = torch.from_numpy(b.slots.copy())
    slots[5] = -1  # a padding row
    pos = torch.from_numpy(b.positions)
    table = W.rope_table(4096, 1e6)
    wq, wkc, wvc = R.rope_append(u16(q), u16(k), u16(v), u16(kc), u16(vc), pos.numpy(), slots.numpy(),
                                 table.numpy(), b.rows, 32, 8, 128, bf16, 4096, b.cache_slots)
    qd, kd, vd, kcd, vcd = (t.to(dev) for t in (q, k, v, kc, vc))
    feattn.rope_append(qd, kd, vd, kcd, vcd, pos.to(dev), slots.to(dev), table.to(dev), b.rows, 32,
                       8, 128, bf16, 4096, b.cache_slots)
    torch.cuda.synchronize()
    assert np.array_equal(u16(qd), wq)
    assert np.array_equal(u16(kcd).reshape(b.cache_slots, -1), wkc)
    assert np.array_equal(u16(vcd).reshape(b.cache_slots, -1), wvc)
    assert torch.equal(kd.cpu(), k) and torch.equal(vd.cpu(), v)  # inputs untouched


@pytest.mark.skipif(not ref_lib.available(), reason="oracle/_ref not built")
@pytest.mark.parametrize("bf16", [True, False])
def test_rope_store_match_reference_aten_on_device(dev, bf16):
    """The reference's own ATen rope and store (src/portable_gpu_ops.cpp:50-54)
    on the same device tensors: identical bits (store compared outside the
    dummy page, where the reference parks slot < 0 rows)."""
    b = W.make_batch(32, 8, starts=[3, 500], qlens=[40, 9], seed=31, extra_pages=1)
    dt = dtype_of(bf16)
    gen = torch.Generator().manual_seed(8)
    q = torch.randn(b.rows, 32, 128, generator=gen).to(dt).to(dev)
    k = torch.randn(b.rows, 8, 128, generator=gen).to(dt).to(dev)
    v = torch.randn(b.rows, 8, 128, generator=gen).to(dt).to(dev)
    pos = torch.from_numpy(b.positions).to(dev)
    slots = torch.from_numpy(b.slots.copy())
    slots[0] = -1
    slots = slots.to(dev)
    table = W.rope_table(1024, 1e6).to(dev)
    q1, k1, q2, k2 = q.clone(), k.clone(), q.clone(), k.clone()
    feattn.rope(q1, k1, pos, table, b.rows, 32, 8, 128, bf16, 1024)
    ref_lib.rope(q2, k2, pos, table, b.rows, 32, 8, 128, bf16, 1024)
    torch.cuda.synchronize()
    assert torch.equal(q1, q2) and torch.equal(k1, k2)
    kc1 = torch.zeros(b.blocks + 1, 16, 8, 128, dtype=dt, device=dev)
    vc1, kc2, vc2 = kc1.clone(), kc1.clone(), kc1.clone()
    feattn.store(k1, v, kc1, vc1, slots, b.rows, 1024, bf16, b.cache_slots)
    ref_lib.store(k1, v, kc2, vc2, slots, b.rows, 1024, bf16, b.cache_slots)
    torch.cuda.synchronize()
    assert torch.equal(kc1[:-1], kc2[:-1]) and torch.equal(vc1[:-1], vc2[:-1])


@pytest.mark.parametrize("bf16", [True, False])
def test_rope_append_full_prefill_step(dev, bf16):
    """The benchmarked chunked-prefill step: all 8192 new tokens of the
    8-sequence Qwen3-8B batch appended with RoPE (theta 1e6) in one call,
    bit-identical to fe_rope then fe_store on the device and to the oracle,
    with every slot outside the new tokens left untouched."""
    b = W.qwen3_8b_prefill()
    dt = dtype_of(bf16)
    gen = torch.Generator().manual_seed(9)
    q = torch.randn(b.rows, 32, 128, generator=gen).to(dt)
    k = torch.randn(b.rows, 8, 128, generator=gen).to(dt)
    v = torch.randn(b.rows, 8, 128, generator=gen).to(dt)
    kc = torch.randn(b.blocks + 1, 16, 8, 128, generator=gen).to(dt)
    vc = torch.randn(b.blocks + 1, 16, 8, 128, generator=gen).to(dt)
    pos, slots = torch.from_numpy(b.positions), torch.from_numpy(b.slots)
    table = W.rope_table(4096, 1e6)
    args = lambda *t: [x.to(dev) for x in t]
    qd, kd, vd, kcd, vcd, posd, slotsd, tabd = args(q, k, v, kc, vc, pos, slots, table)
    feattn.rope_append(qd, kd, vd, kcd, vcd, posd, slotsd, tabd, b.rows, 32, 8, 128, bf16, 4096, b.cache_slots)
    q2, k2, kc2, vc2 = args(q, k, kc, vc)  # fresh device copies of the unrotated inputs
    feattn.rope(q2, k2, posd, tabd, b.rows, 32, 8, 128, bf16, 4096)
    feattn.store(k2, vd, kc2, vc2, slotsd, b.rows, 8 * 128, bf16, b.cache_slots)
    torch.cuda.synchronize()
    assert torch.equal(qd, q2) and torch.equal(kcd, kc2) and torch.equal(vcd, vc2)
    wq, wkc, wvc = R.rope_append(u16(q), u16(k), u16(v), u16(kc), u16(vc), b.positions, b.slots,
                                 table.numpy(), b.rows, 32, 8, 128, bf16, 4096, b.cache_slots)
    assert np.array_equal(u16(qd), wq)
    assert np.array_equal(u16(kcd).reshape(b.cache_slots, -1), wkc)
    assert np.array_equal(u16(vcd).reshape(b.cache_slots, -1), wvc)
    untouched = np.ones(b.cache_slots, dtype=bool)
    untouched[b.slots] = False
    assert np.array_equal(u16(kcd).reshape(b.cache_slots, -1)[untouched], u16(kc).reshape(b.cache_slots, -1)[untouched])
