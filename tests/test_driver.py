"""Host driver (include/fe_driver.h) on the CPU against oracle/step_metadata.py:
graph buckets and the KV page allocator (both also checked against the
reference's own host assertions, tests/host_tests.cpp:13,33), and the
per-step metadata builder (src/cuda_model.cpp:131-142) bit for bit, graph
padding and error cases included."""

import ctypes
import os

import numpy as np
import pytest

import feattn
from feattn import workloads as W
from oracle import step_metadata as S


def test_graph_buckets_reference_assertion():
    # tests/host_tests.cpp:13
    assert feattn.graph_buckets(7) == [1, 2, 4, 7]
    assert S.graph_buckets(7) == [1, 2, 4, 7]


def test_graph_buckets_match_oracle():
    for maximum in range(1, 600):
        assert feattn.graph_buckets(maximum) == S.graph_buckets(maximum), maximum


@pytest.mark.parametrize("maximum", [1, 2, 3, 8, 9, 15, 16, 17, 64, 100, 256, 1000])
def test_graph_buckets_properties(maximum):
    got = feattn.graph_buckets(maximum)
    assert got == sorted(set(got)), "strictly increasing"
    assert got[-1] == maximum and got[0] == 1
    # every request count n <= maximum finds a bucket >= n (lower_bound in
    # src/cuda_model.cpp graph_entry) and the padding it adds is < 16 rows
    # once n > 8
    for n in range(1, maximum + 1):
        b = next(x for x in got if x >= n)
        assert b - n < (16 if n > 8 else n)
    small = [x for x in (1, 2, 4, 8) if x <= maximum]
    assert got[:len(small)] == small
    assert set(range(16, maximum + 1, 16)) <= set(got)
    assert len(got) == len(small) + maximum // 16 + (maximum not in small and maximum % 16 != 0)


def test_graph_buckets_rejects_nonpositive():
    for bad in (0, -3):
        with pytest.raises(RuntimeError, match="maximum"):
            feattn.graph_buckets(bad)


@pytest.mark.parametrize("impl", ["native", "oracle"])
def test_blocks_reference_assertions(impl):
    # tests/host_tests.cpp:33: BlockManager(2,16); a needs 2 pages for 17
    # tokens, b cannot get one, nothing is taken on failure; release frees all
    blocks = feattn.Blocks(2, 16) if impl == "native" else S.Blocks(2, 16)
    table = blocks.table if impl == "native" else (lambda s: blocks.tables.get(s, []))
    a, b = 1, 2
    assert blocks.ensure(a, 17)
    assert not blocks.ensure(b, 1)
    assert table(b) == []
    blocks.release(a)
    assert blocks.used() == 0
    assert blocks.ensure(b, 1)
    blocks.release(b)
    assert blocks.used() == 0


def test_blocks_random_ops_match_oracle():
    rng = np.random.default_rng(5)
    native, ref = feattn.Blocks(97, 16), S.Blocks(97, 16)
    for _ in range(3000):
        seq = int(rng.integers(0, 12))
        if rng.random() < 0.25:
            native.release(seq)
            ref.release(seq)
        else:
            target = int(rng.integers(0, 400))
            assert native.ensure(seq, target) == ref.ensure(seq, target)
        assert native.table(seq) == ref.tables.get(seq, [])
        assert native.used() == ref.used()
    native.close()


def test_blocks_fifo_order_and_growth():
    """Free pages start as 0..total-1; ensure takes from the front, release
    appends to the back (src/scheduler.cpp:5,31,35)."""
    blocks = feattn.Blocks(6, 16)
    assert blocks.ensure(10, 16) and blocks.table(10) == [0]
    assert blocks.ensure(10, 16) and blocks.table(10) == [0]        # already covered
    assert blocks.ensure(10, 17) and blocks.table(10) == [0, 1]      # grows by one page
    assert blocks.ensure(11, 40) and blocks.table(11) == [2, 3, 4]
    assert blocks.ensure(10, 1) and blocks.table(10) == [0, 1]       # never shrinks
    assert blocks.used() == 5
    assert not blocks.ensure(12, 33)                                 # needs 3, 1 free
    assert blocks.table(12) == [] and blocks.used() == 5
    blocks.release(11)                                               # free: 5, 2, 3, 4
    blocks.release(10)                                               # free: 5, 2, 3, 4, 0, 1
    blocks.release(99)                                               # unknown: no-op
    assert blocks.used() == 0
    assert blocks.ensure(12, 80) and blocks.table(12) == [5, 2, 3, 4, 0]
    assert blocks.ensure(13, 0) and blocks.table(13) == []
    assert blocks.ensure(13, 5) and blocks.table(13) == [1]
    assert not blocks.ensure(14, 1)
    blocks.close()


def _blocks(impl, total, size, caching=True):
    if impl == "native":
        b = feattn.Blocks(total, size, caching)
        return b, b.table
    b = S.Blocks(total, size, caching)
    return b, (lambda seq: b.tables.get(seq, []))


@pytest.mark.parametrize("impl", ["native", "oracle"])
def test_blocks_prefix_reference_assertions(impl):
    # tests/host_tests.cpp:35-41: BlockManager(4, 16, caching)
    cache, table = _blocks(impl, 4, 16)
    first = same = [7] * 33
    different = [7] * 33
    different[1] = 9
    assert cache.ensure(101, 33)
    cache.publish(101, first, 32)
    assert cache.probe(102, same) == 32
    assert len(table(102)) == 2 and table(102)[0] == table(101)[0]
    assert cache.ensure(102, 33)
    assert cache.probe(103, different) == 0
    cache.release(101)
    assert cache.used() == 3
    cache.release(102)
    assert cache.used() == 0 and cache.stats()["prefix_resident_blocks"] == 2
    cache.probe(102, same)
    assert cache.stats()["prefix_hit_requests"] == 1       # a request counts once
    cache.release(102)
    assert cache.probe(104, [7] * 32) == 16 and len(table(104)) == 1   # one token left to compute
    cache.release(104)
    assert cache.ensure(103, 64)
    assert cache.stats()["prefix_resident_blocks"] == 0 and cache.stats()["prefix_evictions"] == 2
    cache.release(103)
    assert cache.probe(105, [7] * 33) == 0 and cache.used() == 0        # evicted pages are gone


@pytest.mark.parametrize("impl", ["native", "oracle"])
def test_blocks_prefix_hooks_reference_assertions(impl):
    # tests/host_tests.cpp:43-46: publication and reuse wait for the model's
    # readiness; the model is told of evictions
    guarded, _ = _blocks(impl, 2, 16)
    ready, evicted = [False], []
    if impl == "native":
        guarded.set_hooks(ready=lambda key, page: ready[0], evict=lambda key, page: evicted.append((key, page)))
    else:
        guarded.ready = lambda key, page: ready[0]
        guarded.evict = lambda key, page: evicted.append((key, page))
    assert guarded.ensure(201, 17)
    guarded.publish(201, [7] * 17, 16)
    assert guarded.stats()["prefix_resident_blocks"] == 0
    ready[0] = True
    guarded.publish(201, [7] * 17, 16)
    guarded.release(201)
    ready[0] = False
    assert guarded.probe(202, [7] * 17) == 0
    ready[0] = True
    assert guarded.probe(203, [7] * 17) == 16
    guarded.release(203)
    assert guarded.ensure(204, 32) and evicted == [(tuple([7] * 16), 0)]
    guarded.release(204)


def test_blocks_prefix_off_is_a_no_op():
    # BlockManager(total, size) has caching off: probe / publish do nothing
    blocks = feattn.Blocks(4, 16)
    assert blocks.ensure(1, 33)
    blocks.publish(1, [7] * 33, 32)
    assert blocks.probe(2, [7] * 33) == 0 and blocks.table(2) == []
    assert blocks.stats() == dict.fromkeys(S.Blocks(4, 16).stats(), 0)
    blocks.close()


def test_blocks_prefix_errors():
    native, ref = feattn.Blocks(8, 4, True), S.Blocks(8, 4, True)
    for b in (native, ref):
        assert b.ensure(1, 8)
    for b in (native, ref):
        with pytest.raises((RuntimeError, ValueError), match="allocat"):
            b.probe(1, list(range(12)))        # probe after allocation
    for b in (native, ref):
        with pytest.raises((RuntimeError, ValueError)):
            b.publish(1, list(range(12)), 12)  # the third page is not allocated
    # the pages before the failing one stay published, as in the reference
    assert native.stats() == ref.stats() and native.stats()["prefix_new_blocks"] == 2
    for b in (native, ref):
        assert b.ensure(2, 8)
    for b in (native, ref):
        b.publish(2, list(range(100, 108)), 8)
    for b in (native, ref):
        with pytest.raises((RuntimeError, ValueError), match="immutable|another prefix"):
            b.publish(2, list(range(200, 208)), 8)  # same pages, other tokens
    assert native.stats() == ref.stats()
    native.close()


def _prompt(rng, families):
    """A prompt from one of a few families: a shared stem, then a random tail
    (ids from a small vocabulary, so tails collide now and then)."""
    stem = families[int(rng.integers(0, len(families)))]
    cut = int(rng.integers(0, len(stem) + 1))
    tail = rng.integers(0, 3, size=int(rng.integers(0, 40))).tolist()
    return stem[:cut] + tail


@pytest.mark.parametrize("size,total", [(4, 48), (16, 40), (1, 64)])
def test_blocks_prefix_random_ops_match_oracle(size, total):
    rng = np.random.default_rng(size * 1000 + total)
    families = [rng.integers(0, 5, size=int(rng.integers(4, 90))).tolist() for _ in range(4)]
    native, ref = feattn.Blocks(total, size, True), S.Blocks(total, size, True)
    logs = {"native": [], "oracle": []}
    gate = {"salt": 0}

    def hooks(name):
        def ready(key, page):
            logs[name].append(("ready", key, page))
            return (hash(key) + page + gate["salt"]) % 7 != 0
        return ready, lambda key, page: logs[name].append(("evict", key, page))

    r, e = hooks("native")
    native.set_hooks(ready=r, evict=e)
    ref.ready, ref.evict = hooks("oracle")
    tokens = {}
    for step in range(2500):
        seq = int(rng.integers(0, 10))
        if seq not in tokens:
            tokens[seq] = _prompt(rng, families)
        toks = tokens[seq]
        op = rng.random()
        if op < 0.2:
            call = lambda b: b.probe(seq, toks)
        elif op < 0.4:
            target = int(rng.integers(0, len(toks) + 8))
            call = lambda b: b.ensure(seq, target)
        elif op < 0.6:
            computed = int(rng.integers(0, len(toks) + 4))
            call = lambda b: b.publish(seq, toks, computed)
        elif op < 0.75:  # tokens committed (src/scheduler.cpp:94-99)
            toks.extend(rng.integers(0, 3, size=int(rng.integers(1, 3 * size + 2))).tolist())
            call = lambda b: None
        elif op < 0.88:
            call = lambda b: b.release(seq)
        else:
            call = lambda b: b.forget(seq)
            tokens.pop(seq)
        results = []
        for b in (native, ref):
            try:
                results.append(call(b))
            except (RuntimeError, ValueError):
                results.append("error")
        assert results[0] == results[1], (step, op, results)
        if rng.random() < 0.05:
            gate["salt"] += 1
        assert native.table(seq) == ref.tables.get(seq, []), step
        assert native.used() == ref.used() and native.free_pages() == ref.free_pages(), step
        assert native.stats() == ref.stats(), step
        assert logs["native"] == logs["oracle"], step
        # what the mathematics fixes, independent of the oracle: every page is
        # held by as many tables as list it, and a page two sequences share
        # sits at the same index of both tables, whose tokens agree up to it
        holders = {}
        for other in tokens:
            for i, page in enumerate(native.table(other)):
                holders.setdefault(page, []).append((other, i))
        assert native.used() == len(holders) and native.free_pages() == total - len(holders)
        for page, where in holders.items():
            if len(where) > 1:
                i = where[0][1]
                assert all(j == i for _, j in where), (page, where)
                stems = {tuple(tokens[o][:(i + 1) * size]) for o, _ in where}
                assert len(stems) == 1, (page, where)
    native.close()


def test_blocks_rejects_bad_pool():
    for total, size in ((0, 16), (2**31 - 1, 16), (4, 0), (-1, 16)):
        with pytest.raises(RuntimeError):
            feattn.Blocks(total, size)


def _via_driver(b: W.Batch, **kw):
    return feattn.prepare_metadata(b.starts, b.qlens, b.tables, b.page, max_model_len=1 << 20, **kw)


WORKLOADS = [W.qwen3_06b_decode, W.qwen3_8b_decode, W.qwen3_8b_prefill, W.qwen3_30b_mixed,
             W.dflash_block]


def _same(m, want):
    for key in ("positions", "slots", "qo", "kv", "pages", "last"):
        assert m[key].tolist() == want[key], key


@pytest.mark.parametrize("make", WORKLOADS, ids=lambda f: f.__name__)
def test_prepare_metadata_matches_oracle(make):
    b = make()
    _same(_via_driver(b), S.prepare(b.starts, b.qlens, b.tables, b.page, 1 << 20))
    # the workload builder the attention tests use agrees too
    m = _via_driver(b)
    assert np.array_equal(m["slots"], b.slots) and m["pages"].tolist() == b.pages


@pytest.mark.parametrize("count,entry_rows", [(8, 1), (16, 4), (5, 16)])
def test_prepare_metadata_padding_matches_oracle(count, entry_rows):
    b = W.make_batch(32, 8, starts=[100, 7, 2000, 0, 33], qlens=[1, 4, 4, 16, 1], seed=11)
    m = _via_driver(b, count=count, entry_rows=entry_rows, dummy_page=b.blocks)
    _same(m, S.prepare(b.starts, b.qlens, b.tables, b.page, 1 << 20, count=count, entry_rows=entry_rows,
                       dummy_page=b.blocks))


def test_prepare_metadata_slots_closed_form():
    """slot = table[pos // page] * page + pos % page, so the slot of every row
    names the page that the table assigns to its position."""
    b = W.make_batch(8, 8, starts=[0, 15, 16, 33], qlens=[17, 1, 16, 40], seed=7, extra_pages=5)
    m = _via_driver(b)
    r = 0
    for s, (start, rows) in enumerate(zip(b.starts, b.qlens)):
        for j in range(rows):
            p = start + j
            assert m["positions"][r] == p
            assert m["slots"][r] // 16 == b.tables[s][p // 16] and m["slots"][r] % 16 == p % 16
            r += 1
    assert r == b.rows


def test_prepare_metadata_graph_padding():
    """Entries past the real sequences: entry_rows rows at positions
    0..entry_rows-1, slot -1, the dummy page, last = entry_rows
    (src/cuda_model.cpp:141)."""
    b = W.make_batch(32, 8, starts=[100, 7, 2000], qlens=[4, 4, 4], seed=9)
    count = 8
    m = _via_driver(b, count=count, entry_rows=4, dummy_page=b.blocks)
    real_rows = b.rows
    assert m["positions"][:real_rows].tolist() == b.positions.tolist()
    assert m["positions"][real_rows:].tolist() == [0, 1, 2, 3] * (count - b.batch)
    assert (m["slots"][real_rows:] == -1).all()
    assert m["qo"].tolist() == b.qo + [b.qo[-1] + 4 * i for i in range(1, count - b.batch + 1)]
    assert m["kv"].tolist() == b.kv + [b.kv[-1] + i for i in range(1, count - b.batch + 1)]
    assert m["pages"].tolist() == b.pages + [b.blocks] * (count - b.batch)
    assert m["last"].tolist() == b.last + [4] * (count - b.batch)


def test_prepare_metadata_empty_graph_entry():
    """Capture-time prepare with no sequences (src/cuda_model.cpp:150): all
    entries are padding."""
    m = feattn.prepare_metadata([], [], [], 16, 4096, count=4, entry_rows=1, dummy_page=77)
    assert m["positions"].tolist() == [0] * 4 and m["slots"].tolist() == [-1] * 4
    assert m["qo"].tolist() == [0, 1, 2, 3, 4] and m["kv"].tolist() == [0, 1, 2, 3, 4]
    assert m["pages"].tolist() == [77] * 4 and m["last"].tolist() == [1] * 4


def test_prepare_metadata_errors():
    # context beyond max_model_len (src/cuda_model.cpp:136)
    with pytest.raises(RuntimeError, match="max_model_len"):
        feattn.prepare_metadata([4090], [8], [list(range(256))], 16, 4096)
    assert feattn.prepare_metadata([4088], [8], [list(range(256))], 16, 4096)["slots"][-1] == 4095
    # a write slot outside the page table (:137)
    with pytest.raises(RuntimeError, match="slot"):
        feattn.prepare_metadata([15], [2], [[3]], 16, 4096)
    # a context outside the page table with no rows to write (:138)
    with pytest.raises(RuntimeError, match="context"):
        feattn.prepare_metadata([5], [0], [[]], 16, 4096)
    # outputs too small
    lib = feattn.lib()
    one = (ctypes.c_int64 * 1)(5)
    rows = (ctypes.c_int32 * 1)(3)
    off = (ctypes.c_int32 * 2)(0, 1)
    tab = (ctypes.c_int32 * 1)(0)
    pos, slots = (ctypes.c_int64 * 2)(), (ctypes.c_int64 * 2)()
    qo, kv, pages, last = (ctypes.c_int32 * 2)(), (ctypes.c_int32 * 2)(), (ctypes.c_int32 * 1)(), (
        ctypes.c_int32 * 1)()
    nr, npg = ctypes.c_int(), ctypes.c_int()
    rc = lib.fe_prepare_metadata(1, one, rows, off, tab, 1, 0, 16, 4096, 0, pos, slots, 2, qo, kv, pages, 1,
                                 last, ctypes.byref(nr), ctypes.byref(npg))
    assert rc == feattn.FE_ECAPACITY and nr.value == 3 and npg.value == 1


def test_rope_table_rejects_bad_arguments():
    """Checked before any launch, so this runs without a device."""
    lib = feattn.lib()
    buf = (ctypes.c_float * 4)()
    for max_len, dim, theta in ((0, 128, 1e6), (16, 127, 1e6), (16, 128, 0.0), (16, 128, -1.0),
                                (1 << 30, 1 << 20, 1e6)):
        assert lib.fe_rope_table(buf, max_len, dim, theta, None) == feattn.FE_EINVAL
        assert b"rope table" in lib.fe_attn_last_error()
    assert lib.fe_rope_table(None, 16, 128, 1e6, None) == feattn.FE_EINVAL
    assert b"null" in lib.fe_attn_last_error()


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU; --gpus N > 1 exits with a message before
    touching a device."""
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    res = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", "2"], capture_output=True,
                         text=True, timeout=120)
    assert res.returncode != 0
    assert "one GPU" in (res.stdout + res.stderr)
