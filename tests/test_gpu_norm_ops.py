"""GPU parity of the per-token operators (include/fe_ops.h) against
oracle/norm_ops.py: RMSNorm and the fused q/k RMSNorm + RoPE + paged append
bit-exact (and the fused call bit-identical to fe_norm + fe_rope + fe_store),
acceptance on the reference's matrix pattern (tests/gpu_ops_tests.cpp:55-79:
sentinels around the output, eager and HIP-graph replays), SiLU-gated product
within one rounding step of the 16-bit type."""

import numpy as np
import pytest
import torch

import feattn
from feattn import workloads as W
from oracle import norm_ops as N
from oracle import rope_store as R

pytestmark = pytest.mark.gpu


def u16(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def dtype_of(bf16):
    return torch.bfloat16 if bf16 else torch.float16


@pytest.mark.parametrize("bf16", [True, False])
@pytest.mark.parametrize("width,residual", [(128, False), (128, True), (1000, False), (4096, True), (5120, False)])
def test_norm_bit_exact(dev, bf16, width, residual):
    dt = dtype_of(bf16)
    gen = torch.Generator().manual_seed(width + residual)
    rows = 37
    x = (torch.randn(rows, width, generator=gen) * 3).to(dt)
    r = torch.randn(rows, width, generator=gen).to(dt) if residual else None
    w = (1 + 0.1 * torch.randn(width, generator=gen)).to(dt)
    want, want_res = N.rms_norm(u16(x), u16(w), 1e-6, bf16, residual=u16(r) if residual else None)
    xd, wd = x.to(dev), w.to(dev)
    rd = r.to(dev) if residual else None
    out = torch.empty_like(xd)
    new_res = torch.empty_like(xd) if residual else None
    feattn.norm(xd, wd, out, rows, width, 1e-6, bf16, residual=rd, new_residual=new_res)
    torch.cuda.synchronize()
    assert np.array_equal(u16(out), want)
    if residual:
        assert np.array_equal(u16(new_res), want_res)
    # in place (output aliases x), as Net::forward's callers may do
    feattn.norm(xd, wd, xd, rows, width, 1e-6, bf16, residual=rd)
    torch.cuda.synchronize()
    assert np.array_equal(u16(xd), want)


def make_fused_case(bf16, rows, hq, hkv, row_stride, seed, cache_pages=64, max_pos=4096):
    dt = dtype_of(bf16)
    gen = torch.Generator().manual_seed(seed)
    buf = (torch.randn(rows * row_stride, generator=gen) * 2).to(dt)
    qw = (1 + 0.1 * torch.randn(128, generator=gen)).to(dt)
    kw = (1 + 0.1 * torch.randn(128, generator=gen)).to(dt)
    cache_slots = cache_pages * 16
    kc = torch.randn(cache_slots, hkv, 128, generator=gen).to(dt)
    vc = torch.randn(cache_slots, hkv, 128, generator=gen).to(dt)
    pos = torch.randint(0, max_pos, (rows,), generator=gen)
    pos[1] = -1
    pos[-1] = max_pos               # out of range: normalized, not rotated
    slots = torch.randperm(cache_slots, generator=gen)[:rows].clone()
    slots[2] = -1                   # padding row: no cache entry
    slots[3] = cache_slots          # out of range: skipped
    table = W.rope_table(max_pos, 1e6)
    return buf, qw, kw, kc, vc, pos, slots, table, cache_slots


@pytest.mark.parametrize("bf16", [True, False])
@pytest.mark.parametrize("rows,hq,hkv,extra", [(203, 32, 8, 0), (64, 16, 8, 0), (9, 40, 8, 64), (130, 32, 4, 0)])
def test_norm_rope_append_vs_oracle(dev, bf16, rows, hq, hkv, extra):
    row_stride = (hq + 2 * hkv) * 128 + extra
    buf, qw, kw, kc, vc, pos, slots, table, cs = make_fused_case(bf16, rows, hq, hkv, row_stride, rows + hq)
    wq, wkc, wvc = N.norm_rope_append(u16(buf), row_stride, u16(qw), u16(kw), 1e-6, u16(kc), u16(vc), pos.numpy(),
                                      slots.numpy(), table.numpy(), rows, hq, hkv, bf16, 4096, cs)
    q_out = torch.empty(rows, hq, 128, dtype=buf.dtype, device=dev)
    kcd, vcd = kc.to(dev), vc.to(dev)
    feattn.norm_rope_append(buf.to(dev), row_stride, qw.to(dev), kw.to(dev), 1e-6, q_out, kcd, vcd, pos.to(dev),
                            slots.to(dev), table.to(dev), rows, hq, hkv, bf16, 4096, cs)
    torch.cuda.synchronize()
    assert np.array_equal(u16(q_out), wq)
    assert np.array_equal(u16(kcd).reshape(cs, -1), wkc)      # untouched slots included
    assert np.array_equal(u16(vcd).reshape(cs, -1), wvc)


def test_norm_rope_append_special_values(dev):
    """bf16 projection rows holding NaNs (several payloads), infinities,
    the largest finite values and subnormals: every head, rotated or not,
    matches the oracle bit for bit (a NaN or infinity poisons its head's
    sum of squares; NaN results round to 0x7fc0)."""
    rows, hq, hkv = 47, 32, 8
    row_stride = (hq + 2 * hkv) * 128
    buf, qw, kw, kc, vc, pos, slots, table, cs = make_fused_case(True, rows, hq, hkv, row_stride, 11)
    specials = [0x7FC0, 0x7FC1, 0x7F81, 0xFFC0, 0x7FFF, 0x7F80, 0xFF80, 0x7F7F, 0xFF7F, 0x0001, 0x8001]
    flat = buf.view(torch.int16)
    gen = torch.Generator().manual_seed(12)
    for j, i in enumerate(torch.randperm(flat.numel(), generator=gen)[:6 * len(specials)].tolist()):
        flat[i] = np.int16(np.uint16(specials[j % len(specials)]))
    with np.errstate(all="ignore"):  # NaN and infinity arithmetic is the point here
        wq, wkc, wvc = N.norm_rope_append(u16(buf), row_stride, u16(qw), u16(kw), 1e-6, u16(kc), u16(vc),
                                          pos.numpy(), slots.numpy(), table.numpy(), rows, hq, hkv, True, 4096, cs)
    q_out = torch.empty(rows, hq, 128, dtype=buf.dtype, device=dev)
    kcd, vcd = kc.to(dev), vc.to(dev)
    feattn.norm_rope_append(buf.to(dev), row_stride, qw.to(dev), kw.to(dev), 1e-6, q_out, kcd, vcd, pos.to(dev),
                            slots.to(dev), table.to(dev), rows, hq, hkv, True, 4096, cs)
    torch.cuda.synchronize()
    assert (wq == 0x7FC0).any()  # the NaN path is exercised
    assert np.array_equal(u16(q_out), wq)
    assert np.array_equal(u16(kcd).reshape(cs, -1), wkc)
    assert np.array_equal(u16(vcd).reshape(cs, -1), wvc)


@pytest.mark.parametrize("bf16", [True, False])
def test_norm_rope_append_equals_unfused_sequence(dev, bf16):
    """Bit-identical to src/cuda_model.cpp:91-95 run as separate calls:
    norm(q), norm(k), rope(q, k), store(k, v)."""
    rows, hq, hkv = 150, 32, 8
    row_stride = (hq + 2 * hkv) * 128
    buf, qw, kw, kc, vc, pos, slots, table, cs = make_fused_case(bf16, rows, hq, hkv, row_stride, 7)
    b2 = buf.view(rows, hq + 2 * hkv, 128).to(dev)
    qwd, kwd, tabd, posd, slotsd = qw.to(dev), kw.to(dev), table.to(dev), pos.to(dev), slots.to(dev)
    q = torch.empty(rows, hq, 128, dtype=buf.dtype, device=dev)
    k = torch.empty(rows, hkv, 128, dtype=buf.dtype, device=dev)
    feattn.norm(b2[:, :hq].contiguous(), qwd, q, rows * hq, 128, 1e-6, bf16)
    feattn.norm(b2[:, hq:hq + hkv].contiguous(), kwd, k, rows * hkv, 128, 1e-6, bf16)
    feattn.rope(q, k, posd, tabd, rows, hq, hkv, 128, bf16, 4096)
    kc1, vc1 = kc.to(dev), vc.to(dev)
    feattn.store(k, b2[:, hq + hkv:].contiguous(), kc1, vc1, slotsd, rows, hkv * 128, bf16, cs)
    q2 = torch.empty_like(q)
    kc2, vc2 = kc.to(dev), vc.to(dev)
    feattn.norm_rope_append(buf.to(dev), row_stride, qwd, kwd, 1e-6, q2, kc2, vc2, posd, slotsd, tabd, rows, hq,
                            hkv, bf16, 4096, cs)
    torch.cuda.synchronize()
    assert torch.equal(q.view(torch.int16), q2.view(torch.int16))
    assert torch.equal(kc1.view(torch.int16), kc2.view(torch.int16))
    assert torch.equal(vc1.view(torch.int16), vc2.view(torch.int16))


@pytest.mark.parametrize("bf16", [True, False])
def test_draft_context_projection_layout(dev, bf16):
    """Net::project (src/cuda_model.cpp:102-107): per layer, k and v of a
    [rows][layers][2][hkv][128] projection; hq = 0, row stride over layers."""
    rows, layers, hkv = 48, 3, 8
    row_stride = layers * 2 * hkv * 128
    buf, _, kw, kc, vc, pos, slots, table, cs = make_fused_case(bf16, rows, 0, hkv, row_stride, 9)
    for lid in range(layers):
        off = lid * 2 * hkv * 128
        _, wkc, wvc = N.norm_rope_append(u16(buf)[off:], row_stride, None, u16(kw), 1e-6, u16(kc), u16(vc),
                                         pos.numpy(), slots.numpy(), table.numpy(), rows, 0, hkv, bf16, 4096, cs)
        kcd, vcd = kc.to(dev), vc.to(dev)
        feattn.norm_rope_append(buf.to(dev)[off:], row_stride, None, kw.to(dev), 1e-6, None, kcd, vcd, pos.to(dev),
                                slots.to(dev), table.to(dev), rows, 0, hkv, bf16, 4096, cs)
        torch.cuda.synchronize()
        assert np.array_equal(u16(kcd).reshape(cs, -1), wkc)
        assert np.array_equal(u16(vcd).reshape(cs, -1), wvc)


def test_accept_matrix_eager_and_graph(dev):
    """tests/gpu_ops_tests.cpp:55-79: draft = verify = 10 + j except
    verify[accepted] = 99 with accepted = (first + b) % (k + 1); 8 sentinel
    words on each side of the output stay untouched; the same launch replayed
    from a captured graph sees the new inputs."""
    checks = replays = 0
    for batch in (1, 2, 4, 8):
        for k in range(1, 16):
            draft = torch.zeros(batch, k, dtype=torch.int64, device=dev)
            verify = torch.zeros(batch, k + 1, dtype=torch.int64, device=dev)
            output = torch.full((batch * (k + 2) + 16,), -999, dtype=torch.int64, device=dev)
            run = lambda: feattn.accept(draft, verify, output[8:], batch, k)
            run()
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                run()
            for first in range(k + 1):
                acc = [(first + b) % (k + 1) for b in range(batch)]
                d = np.tile(10 + np.arange(k), (batch, 1))
                v = np.tile(10 + np.arange(k + 1), (batch, 1))
                for b in range(batch):
                    v[b, acc[b]] = 99
                draft.copy_(torch.from_numpy(d))
                verify.copy_(torch.from_numpy(v))
                want = N.accept(d, v).reshape(-1)
                for captured in (False, True):
                    output.fill_(-999)
                    if captured:
                        graph.replay()
                        replays += 1
                    else:
                        run()
                    ids = output.cpu().numpy()
                    assert (ids[:8] == -999).all() and (ids[8 + batch * (k + 2):] == -999).all()
                    assert np.array_equal(ids[8:8 + batch * (k + 2)], want)
                    for b in range(batch):
                        row = ids[8 + b * (k + 2):8 + (b + 1) * (k + 2)]
                        assert row[k + 1] == acc[b] + 1 and row[acc[b]] == 99
                        assert row[:acc[b]].tolist() == list(range(10, 10 + acc[b]))
                        checks += 1
            del graph
    assert checks == 2 * sum(b * (k + 1) for b in (1, 2, 4, 8) for k in range(1, 16)) and replays > 0


@pytest.mark.parametrize("bf16", [True, False])
def test_silu_mul_within_one_step(dev, bf16):
    dt = dtype_of(bf16)
    gen = torch.Generator().manual_seed(4)
    rows, width = 77, 1536
    gu = (torch.randn(rows, 2 * width, generator=gen) * 4).to(dt)
    want = N.silu_mul(u16(gu), bf16)
    out = torch.empty(rows, width, dtype=dt, device=dev)
    feattn.silu_mul(gu.to(dev), out, rows, width, bf16)
    torch.cuda.synchronize()
    got = u16(out)
    a = R.to_f32(got, bf16).astype(np.float64)
    b = R.to_f32(want, bf16).astype(np.float64)
    step = np.maximum(np.abs(a), np.abs(b)) * (2.0 ** -7 if bf16 else 2.0 ** -10) + (0 if bf16 else 2.0 ** -24)
    assert (np.abs(a - b) <= step).all()
    assert np.mean(got == want) > 0.99
