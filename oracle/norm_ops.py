"""ORACLE (test infrastructure only): numpy restatement of the reference's
per-token operators around attention, bit-exact where the reference is.

  rms_norm      src/cuda_kernels.cu:11-17 (norm_kernel, 256 threads per row):
                v = x (+ residual); thread t accumulates v_j^2 for
                j = t, t+256, ... with one FMA per term (nvcc contracts
                `sum += value*value`); partial sums combined by the tree
                p[t] += p[t+s], s = 128 .. 1; scale = rsqrt(p[0]/width + eps);
                out = T(rn(rn(v*scale) * w)); new_residual = T(v).
                rsqrt is evaluated as 1 / sqrt in float64, rounded once to
                float32 (the reference calls the device's approximate rsqrtf,
                which this cannot reproduce; see the tests for the bound).
  silu_mul      src/cuda_kernels.cu:18: T(rn(x / (1 + exp(-x))) * up).
                numpy's float32 exp and the device expf may differ by an ulp,
                so this one is a tolerance oracle (1 ulp of T).
  accept        src/cuda_kernels.cu:25, src/portable_gpu_ops.cpp:56-58,
                src/scheduler.cpp:110 (accept_greedy): m = agreeing prefix
                length, out[0..k] = verify[0..k], out[k+1] = m + 1.
  norm_rope_append
                src/cuda_model.cpp:91-95: q = norm(q, qw), k = norm(k, kw),
                rope(q, k) (oracle.rope_store.rope), store(k, v).

Pinned by tests/test_oracle_norm_ops.py: the FMA emulation against exact
rational rounding (and a case where a plain double sum double-rounds), a
hand-derived tree total that differs from the sequential and the exact sum,
integer inputs whose sum of squares is exact (every term counted once),
constant rows (power-of-two scale: output = sign * weight exactly), the ATen
formula (src/portable_gpu_ops.cpp:46-48) within one ulp of T, the
reference's accept_greedy assertions (tests/host_tests.cpp:28-31) and
acceptance matrix (tests/gpu_ops_tests.cpp:55-79), and silu closed forms
plus a float64 evaluation.
"""

from __future__ import annotations

import numpy as np

from oracle.rope_store import from_f32, rope, store, to_f32

_THREADS = 256


def fma32(a: np.ndarray, b: np.ndarray, c: np.ndarray) -> np.ndarray:
    """Correctly rounded float32 fma(a, b, c) (round to nearest even).

    a*b is exact in float64 (24 + 24 bits); TwoSum gives s + e == a*b + c
    exactly; rounding s to float32 is then correct unless s is a float32
    midpoint and e != 0, in which case e decides the direction."""
    a64 = np.asarray(a, np.float32).astype(np.float64)
    b64 = np.asarray(b, np.float32).astype(np.float64)
    c64 = np.asarray(c, np.float32).astype(np.float64)
    p = a64 * b64
    s = p + c64
    bb = s - p
    e = (p - (s - bb)) + (c64 - bb)
    r = s.astype(np.float32)
    r64 = r.astype(np.float64)
    n = np.nextafter(r, np.where(s > r64, np.inf, -np.inf).astype(np.float32))
    mid = (r64 != s) & ((r64 + n.astype(np.float64)) * 0.5 == s)
    lo, hi = np.minimum(r, n), np.maximum(r, n)
    return np.where(mid & (e > 0), hi, np.where(mid & (e < 0), lo, r)).astype(np.float32)


def sum_squares(v: np.ndarray) -> np.ndarray:
    """Tree-ordered sum of squares over the last axis of float32 v."""
    v = np.asarray(v, np.float32)
    width = v.shape[-1]
    part = np.zeros(v.shape[:-1] + (_THREADS,), np.float32)
    for j in range(width):
        t = j % _THREADS
        part[..., t] = fma32(v[..., j], v[..., j], part[..., t])
    s = _THREADS // 2
    while s >= 1:
        part[..., :s] = part[..., :s] + part[..., s:2 * s]
        s //= 2
    return part[..., 0]


def rsqrt(x: np.ndarray) -> np.ndarray:
    return (1.0 / np.sqrt(np.asarray(x, np.float32).astype(np.float64))).astype(np.float32)


def rms_norm(x, weight, eps: float, bf16: bool, residual=None):
    """x, residual: uint16 [rows, width]; weight uint16 [width].  Returns
    (out, new_residual) as uint16."""
    v = to_f32(np.asarray(x, np.uint16), bf16)
    if residual is not None:
        v = (v + to_f32(np.asarray(residual, np.uint16), bf16)).astype(np.float32)
    width = v.shape[-1]
    total = sum_squares(v)
    ms = (total / np.float32(width)).astype(np.float32) + np.float32(eps)
    scale = rsqrt(ms.astype(np.float32))[..., None]
    w = to_f32(np.asarray(weight, np.uint16), bf16)
    out = ((v * scale).astype(np.float32) * w).astype(np.float32)
    return from_f32(out, bf16), from_f32(v, bf16)


def silu_mul(gu, bf16: bool):
    """gu uint16 [rows, 2*width] -> uint16 [rows, width]."""
    f = to_f32(np.asarray(gu, np.uint16), bf16)
    width = f.shape[-1] // 2
    x, up = f[..., :width], f[..., width:]
    with np.errstate(over="ignore"):
        sig = (x / (np.float32(1) + np.exp(-x)).astype(np.float32)).astype(np.float32)
    return from_f32((sig * up).astype(np.float32), bf16)


def accept(draft: np.ndarray, verify: np.ndarray) -> np.ndarray:
    """draft int64 [batch, k], verify [batch, k+1] -> out [batch, k+2]."""
    draft = np.asarray(draft, np.int64)
    verify = np.asarray(verify, np.int64)
    batch, k = draft.shape
    out = np.zeros((batch, k + 2), np.int64)
    for b in range(batch):
        m = 0
        while m < k and draft[b, m] == verify[b, m]:
            m += 1
        out[b, :k + 1] = verify[b]
        out[b, k + 1] = m + 1
    return out


def norm_rope_append(qkv, row_stride: int, qw, kw, eps: float, kc, vc, pos, slots, cache, rows: int,
                     hq: int, hkv: int, bf16: bool, max_positions: int, cache_slots: int):
    """qkv: flat uint16 buffer, row r's heads at r*row_stride.  Returns
    (q_out [rows, hq, 128], kc', vc' as [cache_slots, hkv*128])."""
    d = 128
    flat = np.asarray(qkv, np.uint16).reshape(-1)
    heads = np.stack([flat[r * row_stride:r * row_stride + (hq + 2 * hkv) * d] for r in range(rows)])
    heads = heads.reshape(rows, hq + 2 * hkv, d)
    q = heads[:, :hq].reshape(rows * hq, d)
    k = heads[:, hq:hq + hkv].reshape(rows * hkv, d)
    v = heads[:, hq + hkv:].reshape(rows, hkv * d)
    qn, _ = rms_norm(q, qw, eps, bf16) if hq else (q, None)
    kn, _ = rms_norm(k, kw, eps, bf16) if hkv else (k, None)
    q2, k2 = rope(qn.reshape(rows, hq, d), kn.reshape(rows, hkv, d), pos, cache, rows, hq, hkv, d, bf16,
                  max_positions)
    kc2, vc2 = store(k2.reshape(rows, hkv * d), v, kc, vc, slots, rows, hkv * d, cache_slots)
    return q2, kc2, vc2
