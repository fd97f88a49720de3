"""ORACLE (test infrastructure only): plain-Python restatement of the
reference's per-step host metadata and of its graph batch buckets and KV page
allocator, integer-exact.

  prepare        src/cuda_model.cpp:131-142 (CudaModel::prepare): sequence i
                 with `start` cached tokens and `rows` new rows gets positions
                 start+j, slots table[pos // page] * page + pos % page, rows
                 appended to the query CSR, ceil(len / page) page ids to the
                 page CSR and last = (len - 1) % page + 1 (len = start + rows);
                 a graph entry's extra entries (i >= number of sequences) get
                 `entry_rows` rows at positions 0.., slot -1, the dummy page
                 and last = entry_rows.  Raises where the reference's
                 require() does: len > max_model_len, a write slot or the
                 context outside the page table.
  graph_buckets  src/common.cpp:45-51: 1, 2, 4, 8 (<= maximum), multiples of
                 16 up to maximum, then maximum.
  Blocks         src/scheduler.cpp:5,31,35 (BlockManager without the prefix
                 cache): FIFO free list 0..total-1, ensure takes ceil(target /
                 size) - held pages from the front (all or nothing), release
                 appends a sequence's pages to the back.

Pinned by tests/test_driver.py: graph_buckets(7) == [1, 2, 4, 7] and the
BlockManager(2, 16) sequence of tests/host_tests.cpp:13,33, and the slot
closed form and padding rules on hand-built cases.
"""

from __future__ import annotations

from collections import deque


def graph_buckets(maximum: int):
    if maximum <= 0:
        raise ValueError("maximum must be positive")
    out = [n for n in (1, 2, 4, 8) if n <= maximum]
    out += list(range(16, maximum + 1, 16))
    if not out or out[-1] != maximum:
        out.append(maximum)
    return out


class Blocks:
    def __init__(self, total: int, size: int):
        if not (0 < total < 2 ** 31 - 1 and size > 0):
            raise ValueError("bad pool")
        self.size = size
        self.free = deque(range(total))
        self.tables = {}

    def ensure(self, seq, target: int) -> bool:
        table = self.tables.setdefault(seq, [])
        need = (target + self.size - 1) // self.size
        if need <= len(table):
            return True
        if need - len(table) > len(self.free):
            return False
        while len(table) < need:
            table.append(self.free.popleft())
        return True

    def release(self, seq) -> None:
        self.free.extend(self.tables.pop(seq, []))

    def used(self) -> int:
        return sum(len(t) for t in self.tables.values())


def prepare(starts, rows, tables, page: int, max_model_len: int, count=None, entry_rows: int = 0,
            dummy_page: int = 0):
    n = len(starts)
    count = n if count is None else count
    positions, slots, qo, kv, pages, last = [], [], [0], [0], [], []
    for i in range(count):
        if i < n:
            start, r, table = starts[i], rows[i], tables[i]
            length = start + r
            if length > max_model_len:
                raise ValueError("context exceeds max_model_len")
            for j in range(r):
                pos = start + j
                if pos // page >= len(table):
                    raise ValueError("page table does not cover the write slot")
                positions.append(pos)
                slots.append(table[pos // page] * page + pos % page)
            qo.append(qo[-1] + r)
            npg = (length + page - 1) // page
            if npg > len(table):
                raise ValueError("page table does not cover the context")
            pages.extend(table[:npg])
            kv.append(len(pages))
            last.append((length - 1) % page + 1)
        else:
            positions.extend(range(entry_rows))
            slots.extend([-1] * entry_rows)
            qo.append(qo[-1] + entry_rows)
            pages.append(dummy_page)
            kv.append(len(pages))
            last.append(entry_rows)
    return {"positions": positions, "slots": slots, "qo": qo, "kv": kv, "pages": pages, "last": last}
