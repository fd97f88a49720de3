"""Host planner (no device): validation mirrors the reference's checks and
the work lists cover every visible (row, head, token) exactly once."""

import numpy as np
import pytest

import feattn
from feattn import workloads as W


def plan_args(b, max_pages=None, max_batch=None):
    return (b.hq, b.hkv, 128, b.page, max_batch or max(1, b.batch), max_pages or b.max_pages(),
            b.blocks, b.qo, b.kv, b.pages, b.last, b.batch, b.rows)


def coverage(b, causal):
    """Counts, per (row, kv head, token), how often a work item covers it
    where the token is visible to the row."""
    items = feattn.dump(*plan_args(b), causal=causal)
    lens = b.lens
    seq_of_row = np.zeros(b.rows, np.int64)
    for s in range(b.batch):
        seq_of_row[b.qo[s]:b.qo[s + 1]] = s
    maxlen = max(lens)
    cnt = np.zeros((b.rows, b.hkv, maxlen), np.int32)
    for kind, seq, q0, nq, kvh, t0, t1, part in items:
        assert 0 <= t0 < t1 <= lens[seq]
        assert t0 % 16 == 0
        if kind == 1:
            assert t0 % 64 == 0
            assert nq * b.group <= 128
        else:
            assert nq * b.group <= 32  # at most two 16-column MFMA blocks
        for r in range(q0, q0 + nq):
            assert seq_of_row[r] == seq
            i = r - b.qo[seq]
            lim = lens[seq] - b.qlens[seq] + i if causal else lens[seq] - 1
            hi = min(t1, lim + 1)
            if hi > t0:
                cnt[r, kvh, t0:hi] += 1
    for r in range(b.rows):
        s = seq_of_row[r]
        i = r - b.qo[s]
        lim = lens[s] - b.qlens[s] + i if causal else lens[s] - 1
        assert (cnt[r, :, :lim + 1] == 1).all(), (r, causal)
        assert (cnt[r, :, lim + 1:] == 0).all()
    return items


@pytest.mark.parametrize("causal", [True, False])
def test_coverage_mixed_ragged(causal):
    b = W.make_batch(32, 4, starts=[0, 5, 700, 100, 4000, 33], qlens=[1, 3, 1, 200, 1, 70],
                     seed=7, extra_pages=2)
    coverage(b, causal)


@pytest.mark.parametrize("causal", [True, False])
def test_coverage_prefill_and_dflash(causal):
    coverage(W.make_batch(32, 8, starts=[0, 1000, 17], qlens=[300, 64, 129], seed=3), causal)
    coverage(W.make_batch(32, 8, starts=[2048, 3000], qlens=[16, 16], seed=4), causal)


def test_coverage_gqa_variants():
    for hq, hkv in ((8, 8), (16, 8), (40, 8), (64, 4)):
        b = W.make_batch(hq, hkv, starts=[10, 300], qlens=[1, 40], seed=hq)
        coverage(b, True)


def test_tile_stream_cut_balances_block_verify():
    """Sixteen 16-row non-causal blocks over long contexts (DFlash verify):
    the tile list is the equal cut of the tile stream -- workgroup k * hkv + h
    takes share k of kv head h, every kv head is cut alike, and no share
    holds more than ceil(total tiles per kv head / (512 / hkv)) tiles."""
    ctx = np.random.default_rng(11).integers(2000, 8001, size=16).tolist()
    b = W.make_batch(32, 8, starts=ctx, qlens=[16] * 16, seed=11, extra_pages=1)
    items = [it for it in coverage(b, False) if it[0] == 1]
    d, t, m, p = feattn.describe(*plan_args(b))
    assert m == 16 * sum(1 for s in range(16) if len([it for it in items if it[1] == s and it[4] == 0]) > 1)
    # runs of equal kv head in list order: h = 0..7, then the next share
    runs = []
    for it in items:
        if runs and runs[-1][0] == it[4]:
            runs[-1][1].append(it)
        else:
            runs.append((it[4], [it]))
    assert [h for h, _ in runs] == list(range(8)) * (len(runs) // 8)
    strip = lambda r: [(x[1], x[2], x[3], x[5], x[6], x[7]) for x in r]
    loads = []
    for k in range(0, len(runs), 8):
        for h in range(1, 8):
            assert strip(runs[k + h][1]) == strip(runs[k][1])
        loads.append(sum((x[6] - x[5] + 63) // 64 for x in runs[k][1]))
    # kv head 0's pieces, share after share, are the stream in order
    stream = [x for k in range(0, len(runs), 8) for x in runs[k][1]]
    for a, c in zip(stream, stream[1:]):
        assert (c[1], c[5]) == ((a[1], a[6]) if a[6] < b.lens[a[1]] else (a[1] + 1, 0))
    total = sum((l + 16 + 63) // 64 for l in ctx)
    quota = -(-total // 64)
    assert sum(loads) == total
    assert len(loads) <= 64 and max(loads) <= quota


@pytest.mark.parametrize("hq,hkv", [(32, 8), (8, 8), (40, 5), (32, 16)])
@pytest.mark.parametrize("causal", [True, False])
def test_tile_stream_cut_balances_chunks(hq, hkv, causal):
    """Chunks of one and two 16-column blocks per wavefront over long
    prefixes, few enough that the longest-first list splits them: the equal
    cut is used, and no share exceeds its exact part of the stream by more
    than one tile step (cost 2) -- the tile granularity must not pile up on
    the last share."""
    b = W.make_batch(hq, hkv, starts=[6000, 9000, 300], qlens=[200, 64, 40], seed=hq + hkv)
    items = [it for it in coverage(b, causal) if it[0] == 1]
    runs = []
    for it in items:
        if runs and runs[-1][0] == it[4]:
            runs[-1][1].append(it)
        else:
            runs.append((it[4], [it]))
    assert [h for h, _ in runs] == list(range(hkv)) * (len(runs) // hkv)
    cost = lambda x: ((x[6] - x[5] + 63) // 64) * (2 if x[3] * b.group > 64 else 1)
    loads = [sum(cost(x) for x in runs[k][1]) for k in range(0, len(runs), hkv)]
    shares = 512 // hkv
    assert len(loads) <= shares
    assert max(loads) <= -(-sum(loads) // shares) + 1


def test_split_kv_produces_merges():
    b = W.long_decode(batch=4, ctx=32768)
    counts = feattn.describe(*plan_args(b))
    assert counts[0] > 4 * 8          # split
    assert counts[2] == 4             # one merge row per sequence
    items = coverage(b, True)
    assert all(it[7] >= 0 for it in items)


def test_decode_config_layout():
    b = W.qwen3_8b_decode()
    d, t, m, p = feattn.describe(*plan_args(b))
    assert t == 0 and d >= 1024 and m <= b.batch


@pytest.mark.parametrize("mutate,code", [
    ("batch_over", feattn.FE_ECAPACITY),
    ("last_zero", feattn.FE_EINVAL),
    ("last_big", feattn.FE_EINVAL),
    ("page_oob", feattn.FE_EINVAL),
    ("len_lt_qlen", feattn.FE_EINVAL),
    ("len_gt_max_context", feattn.FE_EINVAL),
    ("rows_short", feattn.FE_EINVAL),
])
def test_validation(mutate, code):
    b = W.make_batch(32, 8, starts=[40, 3], qlens=[1, 5], seed=1)
    qo, kv, pages, last = list(b.qo), list(b.kv), list(b.pages), list(b.last)
    max_batch, max_pages, rows = 2, b.max_pages(), b.rows
    if mutate == "batch_over":
        max_batch = 1
    elif mutate == "last_zero":
        last[0] = 0
    elif mutate == "last_big":
        last[1] = 17
    elif mutate == "page_oob":
        pages[0] = b.blocks + 1
    elif mutate == "len_lt_qlen":
        qo[2] = qo[1] + 9  # 9 query rows for an 8-token sequence
        rows = qo[2]
    elif mutate == "len_gt_max_context":
        max_pages = 2  # max_context 16 < 41
    elif mutate == "rows_short":
        rows = b.rows - 1
    with pytest.raises(RuntimeError) as e:
        feattn.describe(32, 8, 128, 16, max_batch, max_pages, b.blocks, qo, kv, pages, last,
                        b.batch, rows)
    assert f"error {code}" in str(e.value)


def test_empty_batch_and_zero_row_sequence():
    assert feattn.describe(32, 8, 128, 16, 4, 4, 10, [0], [0], [], [], 0, 0) == (0, 0, 0, 0)
    b = W.make_batch(32, 8, starts=[20, 7], qlens=[0, 2], seed=2)
    items = coverage(b, True)
    assert all(it[1] == 1 for it in items)


def lpt_reference(costs, slots, fast=-1):
    """Longest processing time, stated directly: items in decreasing cost
    order (ties in input order), each to the least-loaded share (lowest index
    among equals); then grouped share by share in that order.  With
    0 <= fast < shares, a share below `fast` is loaded as if it worked 3/2 as
    fast: its load is compared at 2/3 (as 2 * load against 3 * load)."""
    n = len(costs)
    m = max(1, min(slots, n))
    weighted = 0 <= fast < m
    weight = [(2 if s < fast else 3) if weighted else 1 for s in range(m)]
    order = sorted(range(n), key=lambda i: -costs[i])  # sorted() is stable
    loads, share = [0] * m, {}
    for i in order:
        k = min(range(m), key=lambda s: (loads[s] * weight[s], s))
        share[i] = k
        loads[k] += costs[i]
    grouped = [i for k in range(m) for i in order if share[i] == k]
    off = [0]
    for k in range(m):
        off.append(off[-1] + sum(1 for i in order if share[i] == k))
    return grouped, off, loads


@pytest.mark.parametrize("case", ["random", "tied", "over_65536", "few_items", "empty"])
def test_share_assignment_matches_lpt_rule(case):
    """The planner's tile-share assignment (counting sort for costs <= 65536,
    comparison sort above) against the rule stated in Python."""
    rng = np.random.default_rng(11)
    slots = 512
    if case == "random":
        costs = rng.integers(1, 400, size=3000).tolist()
    elif case == "tied":
        costs = rng.choice([4, 8, 8, 16], size=2000).tolist()
    elif case == "over_65536":
        costs = rng.integers(1, 400, size=1500).tolist() + [70000, 65537, 1 << 20]
        rng.shuffle(costs)
    elif case == "few_items":
        costs, slots = [5, 3, 5, 1], 16
    else:
        costs = []
    order, off = feattn.assign_shares(costs, slots)
    want_order, want_off, loads = lpt_reference(costs, slots)
    assert order == want_order
    assert off == want_off
    # the ranges split the list exactly, one per share, at most `slots` of them
    assert off[0] == 0 and off[-1] == len(costs) and all(a <= b for a, b in zip(off, off[1:]))
    assert len(off) - 1 <= max(1, min(slots, len(costs)))
    assert sorted(order) == list(range(len(costs)))
    # longest first inside each share
    for k in range(len(off) - 1):
        c = [costs[i] for i in order[off[k]:off[k + 1]]]
        assert c == sorted(c, reverse=True)
    if costs and case != "over_65536":
        assert max(loads) <= sum(costs) / min(slots, len(costs)) + max(costs)  # the LPT bound


@pytest.mark.parametrize("fast", [0, 1, 256, 511, 512, 4000])
def test_weighted_share_assignment(fast):
    """Shares below `fast` (the first-dispatched workgroup of each CU's pair)
    take 3/2 of the work of the others; `fast` outside [0, shares) weighs all
    shares alike."""
    rng = np.random.default_rng(5)
    slots = 512
    costs = rng.integers(1, 60, size=6000).tolist()
    order, off = feattn.assign_shares(costs, slots, fast)
    want_order, want_off, loads = lpt_reference(costs, slots, fast)
    assert order == want_order and off == want_off
    if fast >= slots:
        assert (order, off) == feattn.assign_shares(costs, slots)
    elif 0 < fast:
        # weighted loads level out to within one item: 2 * fast load ~ 3 * slow load
        quick = [2 * x for x in loads[:fast]]
        slow = [3 * x for x in loads[fast:]]
        spread = max(quick + slow) - min(quick + slow)
        assert spread <= 3 * max(costs)
        ratio = (sum(loads[:fast]) / fast) / (sum(loads[fast:]) / (slots - fast))
        assert abs(ratio - 1.5) < 0.05
    # a different assignment from the unweighted rule whenever the weights differ
    if 0 < fast < slots:
        assert (order, off) != feattn.assign_shares(costs, slots)
    elif fast == 0:  # every share weighted alike
        assert (order, off) == feattn.assign_shares(costs, slots)


def test_share_assignment_rejects_bad_input():
    with pytest.raises(RuntimeError, match="negative cost"):
        feattn.assign_shares([3, -1], 4)
    with pytest.raises(RuntimeError, match="slots"):
        feattn.assign_shares([3], 0)


def check_partial_slots(b, causal):
    """Split-KV bookkeeping of the tile lists (longest-first or stream cut):
    every (partial slot, kv head) is written by exactly one piece, a row cut
    into n pieces owns slots base + s * nq (s < n, in token order) with the
    same base for every kv head, unsplit rows own none, and the slots in use
    are [decode partials, partial rows) with none left unused.  Returns the
    slots in use."""
    items = feattn.dump(*plan_args(b), causal=causal)
    d, t, m, p = feattn.describe(*plan_args(b))
    tile = [it for it in items if it[0] == 1]
    dec = [it for it in items if it[0] == 0]
    dec_slots = {it[7] + r for it in dec if it[7] >= 0 for r in range(it[3])}
    base = max(dec_slots) + 1 if dec_slots else 0
    owner = {}
    pieces = {}
    for kind, seq, q0, nq, kvh, t0, t1, part in tile:
        for r in range(nq):
            pieces.setdefault((q0 + r, kvh), []).append((t0, part + r if part >= 0 else -1))
            if part >= 0:
                key = (part + r, kvh)
                assert key not in owner, key
                owner[key] = (q0 + r, t0)
    used = set()
    for (row, kvh), ps in pieces.items():
        ps.sort()
        if len(ps) == 1:
            assert ps[0][1] == -1, (row, kvh)
            continue
        slots = [s for _, s in ps]
        assert all(s >= 0 for s in slots)
        stride = slots[1] - slots[0]
        assert stride > 0 and slots == [slots[0] + i * stride for i in range(len(slots))], (row, kvh)
        assert [s for _, s in sorted(pieces[(row, 0)])] == slots  # same for every kv head
        used.update(slots)
    if used:
        assert min(used) == base and len(used) == max(used) - base + 1
        if causal:  # describe() counts the causal lists
            assert max(used) == p - 1
    return used


@pytest.mark.parametrize("shape", ["blocks", "chunks", "rows_128_1", "split_decode"])
@pytest.mark.parametrize("causal", [True, False])
def test_partial_slots_are_laid_out_for_the_merge(shape, causal):
    if shape == "blocks":
        b = W.make_batch(32, 8, starts=[3000, 7000, 11000, 1500, 9000, 5000], qlens=[16] * 6, seed=4)
    elif shape == "chunks":
        b = W.make_batch(32, 8, starts=[6000, 9000, 300], qlens=[200, 64, 40], seed=5)
    elif shape == "rows_128_1":
        b = W.make_batch(128, 1, starts=[9000, 3000], qlens=[40, 20], seed=6)
    else:
        b = W.make_batch(32, 8, starts=[20000, 6000, 300, 12000], qlens=[1, 64, 1, 16], seed=7)
    assert check_partial_slots(b, causal)  # every shape here splits tile rows


HEAD_LAYOUTS = [(32, 8), (16, 2), (40, 5), (64, 4), (8, 8), (128, 1), (24, 6), (32, 16), (48, 8), (96, 32)]


@pytest.mark.parametrize("seed", range(24))
def test_random_batches_cover_and_lay_out_partials(seed):
    """Seeded random ragged batches (head layout, batch size, decode rows,
    short blocks and longer chunks, prefixes up to 6000 tokens): every
    visible (row, kv head, token) is covered exactly once with both masks,
    and the partial slots of split rows are laid out for the merge."""
    rng = np.random.default_rng(1000 + seed)
    hq, hkv = HEAD_LAYOUTS[seed % len(HEAD_LAYOUTS)]
    batch = int(rng.integers(1, 9))
    qlens, starts = [], []
    for _ in range(batch):
        kind = rng.integers(0, 3)
        qlens.append(int(1 if kind == 0 else rng.integers(2, 33) if kind == 1 else rng.integers(33, 161)))
        starts.append(int(rng.integers(0, 6001)))
    b = W.make_batch(hq, hkv, starts=starts, qlens=qlens, seed=seed, extra_pages=int(rng.integers(0, 3)))
    for causal in (True, False):
        coverage(b, causal)
        check_partial_slots(b, causal)


def column_blocks_read_tokens_once(items):
    """The tile items of one (sequence, kv head) all cover the same query
    columns (their token ranges are then disjoint pieces)."""
    q0_of = {}
    for kind, seq, q0, nq, kvh, t0, t1, part in items:
        if kind == 1 and q0_of.setdefault((seq, kvh), (q0, nq)) != (q0, nq):
            return False
    return True


@pytest.mark.parametrize("seed", range(40))
def test_single_column_block_rule(seed):
    """The tile launch streams K/V with the non-temporal hint when no
    sequence with tile work is cut into several column blocks; that is
    decided from the query lengths alone (qlen <= 128 / group rows per
    block), which must agree with the planner's actual lists."""
    rng = np.random.default_rng(5000 + seed)
    hq, hkv = HEAD_LAYOUTS[seed % len(HEAD_LAYOUTS)]
    g = hq // hkv
    batch = int(rng.integers(1, 7))
    qlens = [int(rng.choice([1, 2, 16, 128 // g, 128 // g + 1, int(rng.integers(2, 200))])) for _ in range(batch)]
    starts = [int(rng.integers(0, 3000)) for _ in range(batch)]
    b = W.make_batch(hq, hkv, starts=starts, qlens=qlens, seed=seed)
    rule = all(q * g <= 32 or q <= 128 // g for q in qlens)
    for causal in (True, False):
        assert column_blocks_read_tokens_once(feattn.dump(*plan_args(b), causal=causal)) == rule, (qlens, g)


def test_single_column_block_rule_on_the_workloads():
    """DFlash blocks stream; chunked prefill and the mixed step do not."""
    want = {W.dflash_block: True, W.qwen3_8b_prefill: False, W.qwen3_30b_mixed: False}
    for make, once in want.items():
        b = make()
        items = feattn.dump(*plan_args(b), causal=make is not W.dflash_block)
        assert column_blocks_read_tokens_once(items) == once, make.__name__
