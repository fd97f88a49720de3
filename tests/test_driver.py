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
