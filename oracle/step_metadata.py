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
  Blocks         src/scheduler.cpp:5-36 (BlockManager): FIFO free list
                 0..total-1, ensure takes ceil(target / size) - held pages
                 from the front (all or nothing), evicting a resident cached
                 page it takes; release drops a sequence's hold and appends
                 pages no sequence holds to the back.  Prefix cache: publish
                 maps each full block's whole token prefix to the page that
                 ends it (a dict keyed by the prefix tuple, as the
                 reference's map); probe walks prefixes block by block,
                 stopping one token short of the prompt, and takes shared
                 pages out of the free list by value.

Pinned by tests/test_driver.py: graph_buckets(7) == [1, 2, 4, 7], the
BlockManager sequences of tests/host_tests.cpp:13,33,35-46 (FIFO, prefix
sharing, exact and stale probes, evictions and the readiness / eviction
hooks), and the slot closed form and padding rules on hand-built cases.
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
    """src/scheduler.cpp:5-36.  Sequences are keys of `tables`; `ready(key,
    page)` / `evict(key, page)` stand for prefix_page_ready / on_evict_page
    (include/fe/model.hpp:24-25)."""

    def __init__(self, total: int, size: int, caching: bool = False):
        if not (0 < total < 2 ** 31 - 1 and size > 0):
            raise ValueError("bad pool")
        self.size = size
        self.caching = caching
        self.free = deque(range(total))
        self.refs = [0] * total
        self.tables = {}
        self.state = {}            # seq -> [cached, probed, counted, hit_counted]
        self.cached_keys = {}      # prefix tuple -> page        (cached_)
        self.keys = {}             # page -> prefix tuple        (keys_)
        self.requests = self.hits = self.hit_blocks = self.new_blocks = self.evictions = 0
        self.ready = None
        self.evict = None

    def _state(self, seq):
        return self.state.setdefault(seq, [0, False, False, False])

    def probe(self, seq, tokens) -> int:
        # src/scheduler.cpp:6-17
        st = self._state(seq)
        if not self.caching or st[1]:
            return st[0]
        if self.tables.get(seq) or st[0]:
            raise ValueError("prefix probe must come before allocation")
        st[1] = True
        if not st[2]:
            self.requests += 1
            st[2] = True
        table = self.tables.setdefault(seq, [])
        end = self.size
        while end < len(tokens):
            key = tuple(tokens[:end])
            page = self.cached_keys.get(key)
            if page is None or (self.ready is not None and not self.ready(key, page)):
                break
            if self.refs[page] == 0:
                self.free.remove(page)
            self.refs[page] += 1
            table.append(page)
            st[0] = end
            self.hit_blocks += 1
            end += self.size
        if st[0] and not st[3]:
            self.hits += 1
            st[3] = True
        return st[0]

    def publish(self, seq, tokens, computed: int) -> None:
        # src/scheduler.cpp:18-29
        if not self.caching:
            return
        computed = min(computed, len(tokens))
        table = self.tables.get(seq, [])
        end = self.size
        while end <= computed:
            index = (end - 1) // self.size
            if index >= len(table):
                raise ValueError("publishing an unallocated KV page")
            page, key = table[index], tuple(tokens[:end])
            end += self.size
            if self.ready is not None and not self.ready(key, page):
                continue
            if key in self.cached_keys:
                continue
            if page in self.keys:
                raise ValueError("published KV pages are immutable")
            self.cached_keys[key] = page
            self.keys[page] = key
            self.new_blocks += 1

    def ensure(self, seq, target: int) -> bool:
        # src/scheduler.cpp:31-34
        table = self.tables.setdefault(seq, [])
        need = (target + self.size - 1) // self.size
        if need <= len(table):
            return True
        if need - len(table) > len(self.free):
            return False
        while len(table) < need:
            page = self.free.popleft()
            key = self.keys.pop(page, None)
            if key is not None:
                if self.evict is not None:
                    self.evict(key, page)
                del self.cached_keys[key]
                self.evictions += 1
            assert self.refs[page] == 0
            self.refs[page] = 1
            table.append(page)
        return True

    def release(self, seq) -> None:
        # src/scheduler.cpp:36
        for page in self.tables.pop(seq, []):
            if self.refs[page] <= 0:
                raise ValueError("KV page released twice")
            self.refs[page] -= 1
            if self.refs[page] == 0:
                self.free.append(page)
        if seq in self.state:
            self.state[seq][0] = 0
            self.state[seq][1] = False

    def forget(self, seq) -> None:
        self.release(seq)
        self.state.pop(seq, None)

    def used(self) -> int:
        return sum(1 for r in self.refs if r > 0)

    def free_pages(self) -> int:
        return len(self.free)

    def stats(self) -> dict:
        # src/scheduler.cpp:30
        return {"prefix_requests": self.requests, "prefix_hit_requests": self.hits,
                "prefix_cached_blocks": self.hit_blocks, "prefix_new_blocks": self.new_blocks,
                "prefix_resident_blocks": len(self.cached_keys), "prefix_evictions": self.evictions}


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
