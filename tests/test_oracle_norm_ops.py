"""Pins oracle/norm_ops.py (RMSNorm, SiLU-gated product, greedy acceptance)
against exact arithmetic, hand-derived values, the reference's ATen formula
and the reference's own acceptance assertions."""

from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import norm_ops as N
from oracle.rope_store import from_f32, to_f32


def exact_round32(x: Fraction) -> np.float32:
    """Round a rational to the nearest float32, ties to even, by comparing
    exactly against the two float32 neighbours."""
    f = np.float32(float(x))          # within one float32 ulp of x
    cands = {f, np.nextafter(f, np.float32(np.inf)), np.nextafter(f, np.float32(-np.inf))}
    best = min(cands, key=lambda c: (abs(Fraction(float(c)) - x),
                                      int(np.array(c, np.float32).view(np.uint32)) & 1))
    return np.float32(best)


def test_fma32_matches_exact_rounding():
    rng = np.random.default_rng(0)
    a = (rng.standard_normal(400) * 2.0 ** rng.integers(-20, 20, 400)).astype(np.float32)
    b = (rng.standard_normal(400) * 2.0 ** rng.integers(-20, 20, 400)).astype(np.float32)
    c = (rng.standard_normal(400) * 2.0 ** rng.integers(-60, 40, 400)).astype(np.float32)
    got = N.fma32(a, b, c)
    for i in range(400):
        want = exact_round32(Fraction(float(a[i])) * Fraction(float(b[i])) + Fraction(float(c[i])))
        assert got[i] == want, i


def test_fma32_sticky_case():
    """a*a + c with a = 1 + 2^-12, c = 2^-60: the exact value lies just above
    the float32 midpoint 1 + 2^-11 + 2^-24, so it rounds up; a float64 sum
    lands on the midpoint and would round to even (down)."""
    a = np.float32(1 + 2.0 ** -12)
    c = np.float32(2.0 ** -60)
    assert np.float32(np.float64(a) * np.float64(a) + np.float64(c)) == np.float32(1 + 2.0 ** -11)
    assert N.fma32(np.array([a]), np.array([a]), np.array([c]))[0] == np.float32(1 + 2.0 ** -11 + 2.0 ** -23)


def test_tree_total_hand_derived():
    """v = [4096, 1 x 127]: squares 2^24 and 1.  Tree steps on position 0:
    s=64: 2^24 + 1 -> 2^24 (tie to even); s=32: + 2 -> 2^24+2; s=16: + 4;
    s=8: + 8; s=4: + 16; s=2: + 32; s=1: + 64  => 2^24 + 126.  (Sequential
    accumulation gives 2^24; the exact sum is 2^24 + 127.)"""
    v = np.ones((1, 128), np.float32)
    v[0, 0] = 4096
    assert N.sum_squares(v)[0] == np.float32(2 ** 24 + 126)


@pytest.mark.parametrize("width", [1, 7, 128, 256, 300, 1000, 4096])
def test_integer_squares_exact(width):
    """Small integers: every square and partial sum is exact, so the tree
    total equals the exact sum of squares -- no term dropped or doubled."""
    v = ((np.arange(width) * 5) % 11 - 5).astype(np.float32)[None, :]
    assert N.sum_squares(v)[0] == float(np.sum(v.astype(np.int64) ** 2))


@pytest.mark.parametrize("bf16", [True, False])
@pytest.mark.parametrize("c", [0.25, -2.0, 8.0])
def test_constant_row_closed_form(bf16, c):
    """x = c everywhere, eps = 0: mean(x^2) = c^2, scale = 1/|c| (a power of
    two), so out = sign(c) * w exactly."""
    width = 128
    x = from_f32(np.full((3, width), c, np.float32), bf16)
    w = from_f32(np.random.default_rng(1).standard_normal(width).astype(np.float32), bf16)
    out, new_res = N.rms_norm(x, w, 0.0, bf16)
    assert np.array_equal(to_f32(out, bf16), np.sign(c) * np.broadcast_to(to_f32(w, bf16), (3, width)))
    assert np.array_equal(new_res, x)


def _ulp_diff(a, b, bf16):
    """Distance in representable steps between two uint16 arrays of finite
    same-sign values."""
    fa, fb = to_f32(a, bf16).astype(np.float64), to_f32(b, bf16).astype(np.float64)
    step = np.maximum(np.abs(fa), np.abs(fb)) * (2.0 ** -7 if bf16 else 2.0 ** -10)
    return np.abs(fa - fb) / np.maximum(step, 1e-30)


@pytest.mark.parametrize("bf16", [True, False])
@pytest.mark.parametrize("width,residual", [(128, False), (4096, True), (1000, False)])
def test_matches_aten_formula_within_one_ulp(bf16, width, residual):
    """src/portable_gpu_ops.cpp:46-48 in torch float32 (another reduction
    order and rsqrt): the 16-bit outputs agree to one rounding step."""
    rng = np.random.default_rng(width)
    x = from_f32((rng.standard_normal((16, width)) * 3).astype(np.float32), bf16)
    r = from_f32(rng.standard_normal((16, width)).astype(np.float32), bf16) if residual else None
    w = from_f32((1 + rng.standard_normal(width) * 0.1).astype(np.float32), bf16)
    out, new_res = N.rms_norm(x, w, 1e-6, bf16, residual=r)
    v = torch.from_numpy(to_f32(x, bf16))
    if residual:
        v = v + torch.from_numpy(to_f32(r, bf16))
        assert np.array_equal(new_res, from_f32(v.numpy(), bf16))
    ref = v * torch.rsqrt((v * v).mean(-1, keepdim=True) + 1e-6) * torch.from_numpy(to_f32(w, bf16))
    want = from_f32(ref.numpy(), bf16)
    assert (_ulp_diff(out, want, bf16) <= 1.0 + 1e-9).all()
    assert np.mean(out == want) > 0.95


def test_scale_within_rsqrt_accuracy():
    """float64 brute force: scale = 1/sqrt(mean + eps) to within 1 ulp of
    float32 (the tree sum itself is within a few ulps of the exact sum)."""
    rng = np.random.default_rng(3)
    v = rng.standard_normal((64, 128)).astype(np.float32)
    total = N.sum_squares(v).astype(np.float64)
    exact = np.sum(v.astype(np.float64) ** 2, axis=-1)
    assert np.all(np.abs(total - exact) <= exact * 2.0 ** -20)
    ms = (N.sum_squares(v) / np.float32(128)).astype(np.float32) + np.float32(1e-6)
    scale = N.rsqrt(ms).astype(np.float64)
    assert np.all(np.abs(scale - 1 / np.sqrt(ms.astype(np.float64))) <= scale * 2.0 ** -23)


def test_accept_greedy_reference_assertions():
    # tests/host_tests.cpp:28-30: accept_greedy(draft, verify) returns the
    # accepted prefix plus the bonus token = out[0 .. m]
    for draft, verify, want in (([1, 2, 3], [1, 9, 8, 7], [1, 9]), ([1, 2], [1, 2, 3], [1, 2, 3]),
                                ([1], [9, 8], [9])):
        out = N.accept(np.array([draft]), np.array([verify]))[0]
        m1 = int(out[-1])
        assert out[:m1].tolist() == want
        assert out[:len(verify)].tolist() == verify


def test_accept_matrix_reference_pattern():
    # tests/host_tests.cpp:31 and tests/gpu_ops_tests.cpp:55-79: draft = verify
    # = 10 + j except verify[accepted] = 99
    for batch in (1, 2, 4, 8):
        for k in range(1, 16):
            for first in range(k + 1):
                d = np.tile(10 + np.arange(k), (batch, 1))
                v = np.tile(10 + np.arange(k + 1), (batch, 1))
                acc = [(first + b) % (k + 1) for b in range(batch)]
                for b in range(batch):
                    v[b, acc[b]] = 99
                out = N.accept(d, v)
                for b in range(batch):
                    assert out[b, k + 1] == acc[b] + 1 and out[b, acc[b]] == 99
                    assert out[b, :acc[b]].tolist() == (10 + np.arange(acc[b])).tolist()


@pytest.mark.parametrize("bf16", [True, False])
def test_silu_closed_forms_and_float64(bf16):
    x = np.array([0.0, 20.0, -20.0, 1.0, -1.0, 3.5], np.float32)
    up = np.array([5.0, 1.0, 1.0, 2.0, 2.0, -1.0], np.float32)
    gu = from_f32(np.concatenate([x, up])[None, :], bf16)
    out = to_f32(N.silu_mul(gu, bf16), bf16)[0]
    xf, uf = to_f32(gu, bf16)[0, :6].astype(np.float64), to_f32(gu, bf16)[0, 6:].astype(np.float64)
    assert out[0] == 0.0                                   # silu(0) = 0
    assert out[1] == to_f32(from_f32(np.float32(20.0), bf16), bf16)   # silu(20) = 20 to 1e-8
    assert abs(out[2]) < 1e-7                              # silu(-20) ~ -4e-8
    ref = xf / (1 + np.exp(-xf)) * uf
    # one rounding step of T (fp16 results below its normal range round to
    # multiples of 2^-24)
    tol = np.abs(ref) * (2.0 ** -7 if bf16 else 2.0 ** -10) + (1e-30 if bf16 else 2.0 ** -24)
    assert np.all(np.abs(out - ref) <= tol)
