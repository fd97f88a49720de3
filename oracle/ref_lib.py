"""ORACLE (test infrastructure only): ctypes access to oracle/_ref/libref_aten_ops.so,
the reference's own ATen implementation of the attention boundary
(src/portable_gpu_ops.cpp) compiled by oracle/Makefile.  Its ATen ops run on
the torch device "cuda" (HIP on ROCm), so it is usable only where a GPU is.
"""

from __future__ import annotations

import ctypes
import os

REF_LIB = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_ref", "libref_aten_ops.so")
_L = None


def available() -> bool:
    return os.path.exists(REF_LIB)


def lib():
    global _L
    if _L is None:
        import torch  # noqa: F401  (LibTorch and its HIP backend first)

        L = ctypes.CDLL(REF_LIB)
        vp, i = ctypes.c_void_p, ctypes.c_int
        i32p = ctypes.POINTER(ctypes.c_int32)
        L.ref_last_error.restype = ctypes.c_char_p
        L.ref_create_plan.restype = vp
        L.ref_create_plan.argtypes = [i] * 8
        L.ref_destroy_plan.argtypes = [vp]
        L.ref_prepare_plan.argtypes = [vp, i32p, i32p, i32p, i32p, i, i, i, vp]
        L.ref_attention.argtypes = [vp, vp, vp, vp, vp, i, vp]
        L.ref_rope.argtypes = [vp, vp, vp, vp, i, i, i, i, i, vp, i]
        L.ref_store.argtypes = [vp, vp, vp, vp, vp, i, i, i, vp, i]
        for n in ("ref_destroy_plan", "ref_prepare_plan", "ref_attention", "ref_rope", "ref_store"):
            getattr(L, n).restype = i
        _L = L
    return _L


def _check(rc):
    if rc != 0:
        raise RuntimeError("reference ATen op failed: " + lib().ref_last_error().decode())


def _i32(v):
    return (ctypes.c_int32 * max(1, len(v)))(*v)


def attention(batch, q, kc, vc, causal: bool, max_pages: int = None):
    """Runs the reference's create_plan / prepare_plan / attention on device
    tensors; returns the output tensor."""
    import torch

    L = lib()
    mp = max_pages if max_pages is not None else batch.max_pages()
    plan = L.ref_create_plan(batch.hq, batch.hkv, q.shape[-1], batch.page, max(1, batch.batch), mp,
                             int(q.dtype == torch.bfloat16), batch.blocks)
    if not plan:
        _check(-1)
    try:
        s = torch.cuda.current_stream().cuda_stream
        _check(L.ref_prepare_plan(plan, _i32(batch.qo), _i32(batch.kv), _i32(batch.pages),
                                  _i32(batch.last), batch.batch, batch.rows, 0, s))
        out = torch.zeros_like(q)
        _check(L.ref_attention(plan, q.data_ptr(), kc.data_ptr(), vc.data_ptr(), out.data_ptr(),
                               int(causal), s))
        torch.cuda.synchronize()
        return out
    finally:
        L.ref_destroy_plan(plan)


def rope(q, k, pos, cache, rows, hq, hkv, dim, bf16, max_positions):
    import torch

    _check(lib().ref_rope(q.data_ptr(), k.data_ptr(), pos.data_ptr(), cache.data_ptr(), rows, hq, hkv,
                          dim, int(bf16), torch.cuda.current_stream().cuda_stream, max_positions))


def store(k, v, kc, vc, slots, rows, width, bf16, cache_slots):
    import torch

    _check(lib().ref_store(k.data_ptr(), v.data_ptr(), kc.data_ptr(), vc.data_ptr(), slots.data_ptr(),
                           rows, width, int(bf16), torch.cuda.current_stream().cuda_stream,
                           cache_slots))
