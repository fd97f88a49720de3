"""ORACLE (test infrastructure only): numpy restatement of the reference's
RoPE and paged-KV store, bit-exact.

  rope   src/cuda_kernels.cu:19-23 (also src/portable_gpu_ops.cpp:50-53):
         NeoX rotate-half on each (row, head, j < dim/2) in fp32 with every
         product and difference rounded separately (__fmul_rn / __fsub_rn /
         __fadd_rn in the CUDA kernel; separate tensor ops in ATen):
            x'_j        = rn(rn(a*c) - rn(b*s))
            x'_{j+d/2}  = rn(rn(b*c) + rn(a*s))
         with c = cache[pos*dim + j], s = cache[pos*dim + d/2 + j], then
         round-to-nearest-even back to bf16 / fp16.
  store  src/cuda_kernels.cu:24: kc[slot*W + c] = k[row*W + c] (same for v);
         rows with slot < 0 are skipped.  (The ATen variant,
         portable_gpu_ops.cpp:54, redirects them to the last dummy slot
         instead; the dummy page's contents are unspecified either way.)

numpy float32 ufuncs round every multiply and subtract separately (no
contraction), which is exactly the reference arithmetic.

Pinned by tests/test_oracle_rope_store.py: cos=1/sin=0 is the identity,
cos=0/sin=1 maps (a, b) -> (-b, a) (tests/ascend_ops_tests.cpp:35-36
pattern), fp32->bf16/fp16 rounding against torch's own conversions over
every 16-bit pattern's neighbourhood, rotation by theta then -theta within
rounding, and store against a brute-force slot loop with untouched slots
checked.
"""

from __future__ import annotations

import numpy as np


def bf16_to_f32(u16: np.ndarray) -> np.ndarray:
    return (u16.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(f: np.ndarray) -> np.ndarray:
    """Round to nearest even; NaN -> 0x7fc0 (c10::BFloat16's CPU rule)."""
    u = np.ascontiguousarray(f, dtype=np.float32).view(np.uint32)
    r = ((u + np.uint32(0x7FFF) + ((u >> 16) & np.uint32(1))) >> 16).astype(np.uint16)
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    r[nan] = 0x7FC0
    return r


def f16_to_f32(u16: np.ndarray) -> np.ndarray:
    return u16.view(np.float16).astype(np.float32)


def f32_to_f16(f: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):  # overflow to +-inf is the IEEE result
        return np.ascontiguousarray(f, dtype=np.float32).astype(np.float16).view(np.uint16)


def to_f32(u16: np.ndarray, bf16: bool) -> np.ndarray:
    return bf16_to_f32(u16) if bf16 else f16_to_f32(u16)


def from_f32(f: np.ndarray, bf16: bool) -> np.ndarray:
    return f32_to_bf16(f) if bf16 else f32_to_f16(f)


def rope(q: np.ndarray, k: np.ndarray, pos: np.ndarray, cache: np.ndarray, rows: int, hq: int,
         hkv: int, dim: int, bf16: bool, max_positions: int):
    """Returns rotated copies of q [rows, hq, dim] and k [rows, hkv, dim]
    (uint16 storage).  Rows whose position lies outside [0, max_positions)
    are returned unchanged (the library's documented behaviour; the
    reference reads out of bounds there)."""
    half = dim // 2
    cache = np.asarray(cache, dtype=np.float32).reshape(-1, dim)
    pos = np.asarray(pos, dtype=np.int64)
    ok = (pos >= 0) & (pos < max_positions)
    cs = np.zeros((rows, half), np.float32)
    sn = np.zeros((rows, half), np.float32)
    cs[ok] = cache[pos[ok], :half]
    sn[ok] = cache[pos[ok], half:]
    outs = []
    for x, heads in ((q, hq), (k, hkv)):
        x = np.array(x, dtype=np.uint16).reshape(rows, heads, dim)
        f = to_f32(x, bf16)
        a, b = f[..., :half], f[..., half:]
        c, s = cs[:, None, :], sn[:, None, :]
        na = (a * c).astype(np.float32) - (b * s).astype(np.float32)
        nb = (b * c).astype(np.float32) + (a * s).astype(np.float32)
        y = np.concatenate([from_f32(na, bf16), from_f32(nb, bf16)], axis=-1)
        y[~ok] = x[~ok]
        outs.append(y)
    return outs[0], outs[1]


def store(k: np.ndarray, v: np.ndarray, kc: np.ndarray, vc: np.ndarray, slots: np.ndarray,
          rows: int, width: int, cache_slots: int):
    """Returns updated copies of the caches (viewed as [cache_slots, width]);
    slot < 0 rows (padding) are skipped, as in the CUDA kernel."""
    kc2 = np.array(kc, dtype=np.uint16).reshape(cache_slots, width)
    vc2 = np.array(vc, dtype=np.uint16).reshape(cache_slots, width)
    k = np.asarray(k, dtype=np.uint16).reshape(rows, width)
    v = np.asarray(v, dtype=np.uint16).reshape(rows, width)
    for r in range(rows):
        s = int(slots[r])
        if s < 0 or s >= cache_slots:
            continue
        kc2[s] = k[r]
        vc2[s] = v[r]
    return kc2, vc2


def rope_append(q, k, v, kc, vc, pos, slots, cache, rows, hq, hkv, dim, bf16, max_positions,
                cache_slots):
    """The composition the reference performs per layer
    (src/cuda_model.cpp:94-95): rope(q, k) then store(k, v).  Returns
    (q', kc', vc')."""
    q2, k2 = rope(q, k, pos, cache, rows, hq, hkv, dim, bf16, max_positions)
    kc2, vc2 = store(k2, v, kc, vc, slots, rows, hkv * dim, cache_slots)
    return q2, kc2, vc2
