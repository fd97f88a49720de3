"""ctypes binding of libfeattn.so (the C ABI declared in include/fe_attn.h).

This is plumbing for the tests, the smoke check and the benchmark: torch
provides device memory and the current HIP stream, every computation runs in
the library's HIP kernels.  There is no fallback: if the library is missing,
:func:`lib` raises.

The functions mirror the reference's ``fe::cuda`` boundary
(include/fe/native_cuda.hpp:6-14): same names, same argument meaning, and a
failed call raises ``RuntimeError`` with the library's message, as the
reference's ``check()`` throws ``std::runtime_error``.
"""

from __future__ import annotations

import ctypes
import os
from typing import Optional, Sequence

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.environ.get("FEATTN_LIB") or os.path.join(PKG_DIR, "lib", "libfeattn.so")

FE_OK = 0
FE_EINVAL = -1
FE_ECAPACITY = -2
FE_EDEVICE = -3
FE_ENOMEM = -4

# Every extern "C" symbol of include/fe_attn.h.
C_SYMBOLS = (
    "fe_attn_plan_create",
    "fe_attn_plan_destroy",
    "fe_attn_plan_prepare",
    "fe_attn_run",
    "fe_rope",
    "fe_store",
    "fe_rope_append",
    "fe_attn_last_error",
    "fe_attn_plan_describe",
    "fe_attn_plan_dump",
    "fe_attn_version",
    "fe_attn_run_noalloc",
    "fe_attn_assign_shares",
)

# Every extern "C" symbol of include/fe_driver.h.
DRIVER_SYMBOLS = (
    "fe_graph_buckets",
    "fe_blocks_create",
    "fe_blocks_destroy",
    "fe_blocks_ensure",
    "fe_blocks_release",
    "fe_blocks_table",
    "fe_blocks_used",
    "fe_blocks_create_ex",
    "fe_blocks_forget",
    "fe_blocks_free_pages",
    "fe_blocks_set_prefix_hooks",
    "fe_blocks_probe",
    "fe_blocks_publish",
    "fe_blocks_prefix_stats",
    "fe_prepare_metadata",
    "fe_rope_table",
)

# Every extern "C" symbol of include/fe_ops.h.
OPS_SYMBOLS = (
    "fe_norm",
    "fe_silu_mul",
    "fe_accept",
    "fe_norm_rope_append",
)

_LIB: Optional[ctypes.CDLL] = None

_i32p = ctypes.POINTER(ctypes.c_int32)
_vp = ctypes.c_void_p
_int = ctypes.c_int


class PrefixStats(ctypes.Structure):
    """fe_prefix_stats (include/fe_driver.h)."""
    _fields_ = [(name, ctypes.c_int64) for name in (
        "requests", "hit_requests", "cached_blocks", "new_blocks", "resident_blocks", "evictions")]


def lib() -> ctypes.CDLL:
    """Loads libfeattn.so once.  torch is imported first so that the library
    binds to the HIP runtime torch already loaded (same SONAME)."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is not built; run `make -C flashengine.cpp_amd` "
            "or __graft_entry__.build() first")
    import torch  # noqa: F401  (HIP runtime first)

    L = ctypes.CDLL(LIB_PATH)
    L.fe_attn_last_error.restype = ctypes.c_char_p
    L.fe_attn_last_error.argtypes = []
    L.fe_attn_version.restype = ctypes.c_char_p
    L.fe_attn_version.argtypes = []
    L.fe_attn_plan_create.argtypes = [_int] * 8 + [ctypes.POINTER(_vp)]
    L.fe_attn_plan_destroy.argtypes = [_vp]
    L.fe_attn_plan_prepare.argtypes = [_vp, _i32p, _i32p, _i32p, _i32p, _int, _int, _int, _vp]
    L.fe_attn_run.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _int, _vp]
    L.fe_attn_run_noalloc.argtypes = [_vp] * 5 + [_int] + [_i32p] * 4 + [_int] * 8 + [_vp]
    L.fe_attn_assign_shares.argtypes = [_i32p, _int, _int, _int, _i32p, _i32p, ctypes.POINTER(_int)]
    L.fe_rope.argtypes = [_vp, _vp, _vp, _vp, _int, _int, _int, _int, _int, _vp, _int]
    L.fe_store.argtypes = [_vp, _vp, _vp, _vp, _vp, _int, _int, _int, _vp, _int]
    L.fe_rope_append.argtypes = [_vp] * 8 + [_int] * 7 + [_vp]
    L.fe_attn_plan_describe.argtypes = [_int] * 7 + [_i32p] * 4 + [_int, _int, _i32p]
    L.fe_attn_plan_dump.argtypes = [_int] * 7 + [_i32p] * 4 + [_int, _int, _int, _i32p, _int,
                                                             ctypes.POINTER(_int)]
    for name in C_SYMBOLS:
        getattr(L, name).restype = ctypes.c_char_p if name in (
            "fe_attn_last_error", "fe_attn_version") else _int
    _i64 = ctypes.c_int64
    _i64p = ctypes.POINTER(ctypes.c_int64)
    L.fe_graph_buckets.argtypes = [_i64, _i64p, _int, ctypes.POINTER(_int)]
    L.fe_blocks_create.argtypes = [_i64, _i64, ctypes.POINTER(_vp)]
    L.fe_blocks_destroy.argtypes = [_vp]
    L.fe_blocks_ensure.argtypes = [_vp, _i64, _i64, ctypes.POINTER(_int)]
    L.fe_blocks_release.argtypes = [_vp, _i64]
    L.fe_blocks_table.argtypes = [_vp, _i64, _i32p, _int, ctypes.POINTER(_int)]
    L.fe_blocks_used.argtypes = [_vp]
    L.fe_blocks_create_ex.argtypes = [_i64, _i64, _int, ctypes.POINTER(_vp)]
    L.fe_blocks_forget.argtypes = [_vp, _i64]
    L.fe_blocks_free_pages.argtypes = [_vp]
    L.fe_blocks_set_prefix_hooks.argtypes = [_vp, _vp, _vp, _vp]
    L.fe_blocks_probe.argtypes = [_vp, _i64, _i64p, _i64, _i64p]
    L.fe_blocks_publish.argtypes = [_vp, _i64, _i64p, _i64, _i64]
    L.fe_blocks_prefix_stats.argtypes = [_vp, ctypes.POINTER(PrefixStats)]
    L.fe_prepare_metadata.argtypes = ([_int, _i64p, _i32p, _i32p, _i32p, _int, _int, _int, _i64, ctypes.c_int32,
                                       _i64p, _i64p, _int, _i32p, _i32p, _i32p, _int, _i32p,
                                       ctypes.POINTER(_int), ctypes.POINTER(_int)])
    L.fe_rope_table.argtypes = [_vp, _int, _int, ctypes.c_double, _vp]
    for name in DRIVER_SYMBOLS:
        getattr(L, name).restype = _i64 if name in ("fe_blocks_used", "fe_blocks_free_pages") else _int
    _f = ctypes.c_float
    L.fe_norm.argtypes = [_vp] * 5 + [_int, _int, _f, _int, _vp]
    L.fe_silu_mul.argtypes = [_vp, _vp, _int, _int, _int, _vp]
    L.fe_accept.argtypes = [_vp, _vp, _vp, _int, _int, _vp]
    L.fe_norm_rope_append.argtypes = ([_vp, _i64, _vp, _vp, _f] + [_vp] * 6 + [_int] * 4 + [_int, _int, _int, _vp])
    for name in OPS_SYMBOLS:
        getattr(L, name).restype = _int
    _LIB = L
    return L


def _check(rc: int) -> None:
    if rc != FE_OK:
        msg = lib().fe_attn_last_error().decode(errors="replace")
        raise RuntimeError(f"feattn error {rc}: {msg}")


def _i32(values: Sequence[int]):
    if isinstance(values, ctypes.Array) and values._type_ is ctypes.c_int32:
        return values  # already converted (callers that prepare every step convert once)
    arr = (ctypes.c_int32 * max(1, len(values)))(*values)
    return arr


def _stream(stream) -> int:
    import torch

    if stream is None:
        return torch.cuda.current_stream().cuda_stream
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


def _ptr(t) -> Optional[int]:
    return None if t is None else t.data_ptr()


class Plan:
    """Owning wrapper of ``fe_attn_plan`` (reference: fe::cuda::AttentionPlan,
    created with create_plan's arguments, native_cuda.hpp:7)."""

    def __init__(self, hq: int, hkv: int, dim: int, page: int, max_batch: int,
                 max_pages: int, bf16: bool, blocks: int):
        self.hq, self.hkv, self.dim, self.page = hq, hkv, dim, page
        self.max_batch, self.max_pages, self.bf16, self.blocks = max_batch, max_pages, bf16, blocks
        handle = _vp()
        _check(lib().fe_attn_plan_create(hq, hkv, dim, page, max_batch, max_pages,
                                         int(bool(bf16)), blocks, ctypes.byref(handle)))
        self._h = handle
        self.rows = 0

    def prepare(self, qo: Sequence[int], kv: Sequence[int], pages: Sequence[int],
                last: Sequence[int], batch: int, rows: int, graph: bool = False,
                stream=None) -> None:
        """fe::cuda::prepare_plan (native_cuda.hpp:9): host CSR metadata."""
        _check(lib().fe_attn_plan_prepare(self._h, _i32(qo), _i32(kv), _i32(pages), _i32(last),
                                          batch, rows, int(bool(graph)), _stream(stream)))
        self.rows = rows

    def run(self, q, k_cache, v_cache, out, causal: bool = True, lse=None, stream=None) -> None:
        """fe::cuda::attention (native_cuda.hpp:10) plus the optional LSE output."""
        _check(lib().fe_attn_run(self._h, _ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(out),
                                 _ptr(lse), int(bool(causal)), _stream(stream)))

    def close(self) -> None:
        if getattr(self, "_h", None) is not None and self._h.value:
            lib().fe_attn_plan_destroy(self._h)
            self._h = _vp()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def run_noalloc(q, k_cache, v_cache, out, qo: Sequence[int], kv: Sequence[int], pages: Sequence[int],
                last: Sequence[int], batch: int, rows: int, hq: int, hkv: int, dim: int, page: int,
                blocks: int, bf16: bool, causal: bool = True, lse=None, stream=None) -> None:
    """Plan-free attention that allocates no device memory (fe_attn_run_noalloc):
    the results of Plan(...).prepare(...) followed by run(...)."""
    _check(lib().fe_attn_run_noalloc(_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(out), _ptr(lse),
                                     int(bool(causal)), _i32(qo), _i32(kv), _i32(pages), _i32(last),
                                     batch, rows, hq, hkv, dim, page, blocks, int(bool(bf16)),
                                     _stream(stream)))


def rope(q, k, pos, cache, rows: int, hq: int, hkv: int, dim: int, bf16: bool,
         max_positions: int, stream=None) -> None:
    """fe::cuda::rope (native_cuda.hpp:13), in place on q and k."""
    _check(lib().fe_rope(_ptr(q), _ptr(k), _ptr(pos), _ptr(cache), rows, hq, hkv, dim,
                         int(bool(bf16)), _stream(stream), max_positions))


def store(k, v, k_cache, v_cache, slots, rows: int, width: int, bf16: bool,
          cache_slots: int, stream=None) -> None:
    """fe::cuda::store (native_cuda.hpp:14): slot < 0 rows are skipped."""
    _check(lib().fe_store(_ptr(k), _ptr(v), _ptr(k_cache), _ptr(v_cache), _ptr(slots), rows,
                          width, int(bool(bf16)), _stream(stream), cache_slots))


def rope_append(q, k, v, k_cache, v_cache, pos, slots, cache, rows: int, hq: int, hkv: int,
                dim: int, bf16: bool, max_positions: int, cache_slots: int, stream=None) -> None:
    """Fused rope + store of the new tokens (q rotated in place)."""
    _check(lib().fe_rope_append(_ptr(q), _ptr(k), _ptr(v), _ptr(k_cache), _ptr(v_cache), _ptr(pos),
                                _ptr(slots), _ptr(cache), rows, hq, hkv, dim, int(bool(bf16)),
                                max_positions, cache_slots, _stream(stream)))


def describe(hq, hkv, dim, page, max_batch, max_pages, blocks, qo, kv, pages, last, batch, rows):
    """Host-only planner counts: (decode items, causal tile items, merge rows, partial rows)."""
    out = (ctypes.c_int32 * 4)()
    _check(lib().fe_attn_plan_describe(hq, hkv, dim, page, max_batch, max_pages, blocks, _i32(qo),
                                       _i32(kv), _i32(pages), _i32(last), batch, rows, out))
    return tuple(out)


def assign_shares(costs: Sequence[int], slots: int, fast: int = -1):
    """Host-only planner share assignment: (order, off) -- the input index of
    each item share by share, and the CSR offsets of the shares.  Shares
    below `fast` (when it is >= 0) take 3/2 of the others' work."""
    n = len(costs)
    order = (ctypes.c_int32 * max(1, n))()
    off = (ctypes.c_int32 * (min(slots, n) + 2))()
    ns = _int()
    _check(lib().fe_attn_assign_shares(_i32(costs), n, slots, fast, order, off, ctypes.byref(ns)))
    return list(order[:n]), list(off[:ns.value + 1])


def dump(hq, hkv, dim, page, max_batch, max_pages, blocks, qo, kv, pages, last, batch, rows,
         causal: bool):
    """Host-only planner work list: list of (kind, seq, q0, nq, kvh, t0, t1, part)."""
    n = _int()
    _check(lib().fe_attn_plan_dump(hq, hkv, dim, page, max_batch, max_pages, blocks, _i32(qo),
                                   _i32(kv), _i32(pages), _i32(last), batch, rows, int(causal),
                                   None, 0, ctypes.byref(n)))
    buf = (ctypes.c_int32 * (8 * max(1, n.value)))()
    _check(lib().fe_attn_plan_dump(hq, hkv, dim, page, max_batch, max_pages, blocks, _i32(qo),
                                   _i32(kv), _i32(pages), _i32(last), batch, rows, int(causal),
                                   buf, n.value, ctypes.byref(n)))
    return [tuple(buf[8 * i:8 * i + 8]) for i in range(n.value)]


def version() -> str:
    return lib().fe_attn_version().decode()


# ---------------------------------------------------------------------------
# Host driver (include/fe_driver.h)
# ---------------------------------------------------------------------------

def graph_buckets(maximum: int):
    """fe::graph_buckets (src/common.cpp:45-51): batch sizes that get a graph."""
    n = _int()
    _check(lib().fe_graph_buckets(maximum, None, 0, ctypes.byref(n)))
    out = (ctypes.c_int64 * max(1, n.value))()
    _check(lib().fe_graph_buckets(maximum, out, n.value, ctypes.byref(n)))
    return list(out[:n.value])


_READY_FN = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p, ctypes.POINTER(ctypes.c_int64), ctypes.c_int64,
                             ctypes.c_int32)
_EVICT_FN = ctypes.CFUNCTYPE(None, ctypes.c_void_p, ctypes.POINTER(ctypes.c_int64), ctypes.c_int64,
                             ctypes.c_int32)


def _tokens(tokens):
    arr = (ctypes.c_int64 * max(1, len(tokens)))(*[int(t) for t in tokens])
    return arr, len(tokens)


class Blocks:
    """FIFO KV page allocator with its prefix cache: fe::BlockManager
    (src/scheduler.cpp:5-36), sequences keyed by an integer id.  `ready(key,
    page)` / `evict(key, page)` (key a tuple of token ids) stand for the
    reference's prefix_page_ready / on_evict_page hooks."""

    def __init__(self, total: int, block_size: int, caching: bool = False):
        handle = _vp()
        _check(lib().fe_blocks_create_ex(total, block_size, int(bool(caching)), ctypes.byref(handle)))
        self._h = handle
        self._hooks = None

    def set_hooks(self, ready=None, evict=None) -> None:
        r = _READY_FN(lambda _u, key, n, page: int(bool(ready(tuple(key[:n]), page)))) if ready else None
        e = _EVICT_FN(lambda _u, key, n, page: evict(tuple(key[:n]), page)) if evict else None
        _check(lib().fe_blocks_set_prefix_hooks(self._h, ctypes.cast(r, _vp) if r else None,
                                                ctypes.cast(e, _vp) if e else None, None))
        self._hooks = (r, e)  # the library holds raw pointers to these

    def probe(self, seq: int, tokens) -> int:
        arr, n = _tokens(tokens)
        cached = ctypes.c_int64()
        _check(lib().fe_blocks_probe(self._h, seq, arr, n, ctypes.byref(cached)))
        return cached.value

    def publish(self, seq: int, tokens, computed: int) -> None:
        arr, n = _tokens(tokens)
        _check(lib().fe_blocks_publish(self._h, seq, arr, n, computed))

    def forget(self, seq: int) -> None:
        _check(lib().fe_blocks_forget(self._h, seq))

    def free_pages(self) -> int:
        return lib().fe_blocks_free_pages(self._h)

    def stats(self) -> dict:
        st = PrefixStats()
        _check(lib().fe_blocks_prefix_stats(self._h, ctypes.byref(st)))
        return {"prefix_requests": st.requests, "prefix_hit_requests": st.hit_requests,
                "prefix_cached_blocks": st.cached_blocks, "prefix_new_blocks": st.new_blocks,
                "prefix_resident_blocks": st.resident_blocks, "prefix_evictions": st.evictions}

    def ensure(self, seq: int, target_tokens: int) -> bool:
        ok = _int()
        _check(lib().fe_blocks_ensure(self._h, seq, target_tokens, ctypes.byref(ok)))
        return bool(ok.value)

    def release(self, seq: int) -> None:
        _check(lib().fe_blocks_release(self._h, seq))

    def table(self, seq: int):
        n = _int()
        _check(lib().fe_blocks_table(self._h, seq, None, 0, ctypes.byref(n)))
        out = (ctypes.c_int32 * max(1, n.value))()
        _check(lib().fe_blocks_table(self._h, seq, out, n.value, ctypes.byref(n)))
        return list(out[:n.value])

    def used(self) -> int:
        return lib().fe_blocks_used(self._h)

    def close(self) -> None:
        if getattr(self, "_h", None) is not None and self._h.value:
            lib().fe_blocks_destroy(self._h)
            self._h = _vp()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def prepare_metadata(starts, rows, tables, page: int, max_model_len: int, count: Optional[int] = None,
                     entry_rows: int = 0, dummy_page: int = 0):
    """CudaModel::prepare (src/cuda_model.cpp:131-142): returns a dict of numpy
    arrays positions, slots (int64) and qo, kv, pages, last (int32)."""
    import numpy as np

    n = len(starts)
    count = n if count is None else count
    off = [0]
    for t in tables:
        off.append(off[-1] + len(t))
    flat = [p for t in tables for p in t]
    c_start = (ctypes.c_int64 * max(1, n))(*starts)
    c_rows = _i32(rows)
    c_off = _i32(off)
    c_tab = _i32(flat)
    nr, npg = _int(), _int()
    args = (n, c_start, c_rows, c_off, c_tab, count, entry_rows, page, max_model_len, dummy_page)
    _check(lib().fe_prepare_metadata(*args, None, None, 0, None, None, None, 0, None, ctypes.byref(nr),
                                     ctypes.byref(npg)))
    positions = np.zeros(max(1, nr.value), np.int64)
    slots = np.zeros(max(1, nr.value), np.int64)
    qo = np.zeros(count + 1, np.int32)
    kv = np.zeros(count + 1, np.int32)
    pages = np.zeros(max(1, npg.value), np.int32)
    last = np.zeros(max(1, count), np.int32)
    p64 = lambda a: a.ctypes.data_as(ctypes.POINTER(ctypes.c_int64))
    p32 = lambda a: a.ctypes.data_as(_i32p)
    _check(lib().fe_prepare_metadata(*args, p64(positions), p64(slots), nr.value, p32(qo), p32(kv), p32(pages),
                                     npg.value, p32(last), ctypes.byref(nr), ctypes.byref(npg)))
    return {"positions": positions[:nr.value], "slots": slots[:nr.value], "qo": qo, "kv": kv,
            "pages": pages[:npg.value], "last": last[:count]}


def rope_table(table, max_len: int, dim: int, theta: float, stream=None) -> None:
    """Fills a device fp32 tensor [max_len, dim] with the cos | sin table
    (src/cuda_model.cpp:44-47)."""
    _check(lib().fe_rope_table(_ptr(table), max_len, dim, float(theta), _stream(stream)))


# ---------------------------------------------------------------------------
# Per-token operators (include/fe_ops.h)
# ---------------------------------------------------------------------------

def norm(x, weight, output, rows: int, width: int, eps: float, bf16: bool, residual=None, new_residual=None,
         stream=None) -> None:
    """fe::cuda::norm (native_cuda.hpp:11): RMSNorm of [rows][width]."""
    _check(lib().fe_norm(_ptr(x), _ptr(residual), _ptr(weight), _ptr(output), _ptr(new_residual), rows, width,
                         float(eps), int(bool(bf16)), _stream(stream)))


def silu_mul(gate_up, output, rows: int, width: int, bf16: bool, stream=None) -> None:
    """fe::cuda::silu_mul (native_cuda.hpp:12)."""
    _check(lib().fe_silu_mul(_ptr(gate_up), _ptr(output), rows, width, int(bool(bf16)), _stream(stream)))


def accept(draft, verify, out, batch: int, k: int, stream=None) -> None:
    """fe::cuda::accept (native_cuda.hpp:15): int64 draft [batch][k], verify
    [batch][k+1] -> out [batch][k+2]."""
    _check(lib().fe_accept(_ptr(draft), _ptr(verify), _ptr(out), batch, k, _stream(stream)))


def norm_rope_append(qkv, row_stride: int, q_weight, k_weight, eps: float, q_out, k_cache, v_cache, pos, slots,
                     cache, rows: int, hq: int, hkv: int, bf16: bool, max_positions: int, cache_slots: int,
                     dim: int = 128, stream=None) -> None:
    """q/k RMSNorm + RoPE + paged append in one pass (src/cuda_model.cpp:91-95)."""
    _check(lib().fe_norm_rope_append(_ptr(qkv), row_stride, _ptr(q_weight), _ptr(k_weight), float(eps),
                                     _ptr(q_out), _ptr(k_cache), _ptr(v_cache), _ptr(pos), _ptr(slots), _ptr(cache),
                                     rows, hq, hkv, dim, int(bool(bf16)), max_positions, cache_slots,
                                     _stream(stream)))
