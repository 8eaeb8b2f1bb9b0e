"""Host-side checks that need no GPU: the C-ABI library loads and exports every
symbol include/d2sd.h declares, the work planner's output partitions the work
exactly, and the Python surface validates its arguments."""
import ctypes as C
import re
from pathlib import Path

import numpy as np
import pytest
import torch

import d2sd
from d2sd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "d2sd.h"


def header_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(d2sd_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_header_symbol():
    lib = C.CDLL(str(_lib.LIB_PATH))
    names = header_functions()
    assert len(names) >= 12
    for name in names:
        assert hasattr(lib, name), name
    assert sorted(_lib.EXPORTED_SYMBOLS) == names


def test_version_and_error_strings():
    assert "gfx950" in d2sd.version()
    assert _lib.lib.d2sd_last_error() is not None


def _plan(qo, pl, hq=32, hkv=8, d=128, window=-1, num_cus=256, waves=0, max_splits=0, page_size=16,
          page_indptr=None, tok_indptr=None, dynamic=0, kv_dtype=0, split=None, tok2=None):
    desc = _lib.PlanDesc()
    qo = np.asarray(qo, dtype=np.int32)
    pl = np.asarray(pl, dtype=np.int32)
    if page_size and page_indptr is None:
        page_indptr = np.concatenate([[0], np.cumsum((pl + page_size - 1) // page_size)])
    pi = np.asarray(page_indptr, dtype=np.int32) if page_indptr is not None else None
    ti = np.asarray(tok_indptr, dtype=np.int32) if tok_indptr is not None else None
    desc.num_reqs = len(pl)
    desc.qo_indptr = qo.ctypes.data_as(C.POINTER(C.c_int32))
    desc.prefix_len = pl.ctypes.data_as(C.POINTER(C.c_int32))
    desc.page_indptr = pi.ctypes.data_as(C.POINTER(C.c_int32)) if pi is not None else None
    desc.prefix_tok_indptr = ti.ctypes.data_as(C.POINTER(C.c_int32)) if ti is not None else None
    desc.num_qo_heads, desc.num_kv_heads, desc.head_dim = hq, hkv, d
    desc.window_left = window
    desc.kv_dtype = kv_dtype
    desc.page_size = page_size
    desc.num_cus = num_cus
    desc.max_splits = max_splits
    desc.waves_per_block = waves
    desc.dynamic_prefix = dynamic
    sp = np.asarray(split, dtype=np.int32) if split is not None else None
    t2 = np.asarray(tok2, dtype=np.int32) if tok2 is not None else None
    desc.prefix_split = sp.ctypes.data_as(C.POINTER(C.c_int32)) if sp is not None else None
    desc.prefix2_tok_indptr = t2.ctypes.data_as(C.POINTER(C.c_int32)) if t2 is not None else None
    info = _lib.PlanInfo()
    assert _lib.lib.d2sd_cascade_plan(C.byref(desc), None, 0, C.byref(info)) == 0, _lib.lib.d2sd_last_error()
    host = np.zeros(max(info.plan_ints, 8), dtype=np.int32)
    rc = _lib.lib.d2sd_cascade_plan(C.byref(desc), host.ctypes.data_as(C.POINTER(C.c_int32)), host.size,
                                    C.byref(info))
    assert rc == 0, _lib.lib.d2sd_last_error()
    ni, nm = info.num_items, info.num_merges
    items = host[: 16 * ni].reshape(-1, 16)
    merges = host[16 * ni: 16 * ni + 8 * nm].reshape(-1, 8)
    return info, items, merges


MODE_PARTIAL, MODE_FINAL, MODE_NOOP = 0, 1, 3
SRC_PREFIX, SRC_SUFFIX, SRC_BOTH, SRC_PREFIX2 = 0, 1, 2, 3
# VerifyItem fields
REQ, KVH, QT, SRC, KB, KE, SLOT, MODE, Q0, NQ, BASE, COFF, KV0, PLAN_LEN = range(14)


@pytest.mark.parametrize("qo,pl,window,page,hq,waves", [
    ([0, 128], [4096], -1, 16, 32, 0),
    ([256 * i for i in range(33)], [8192] * 32, -1, 16, 64, 0),   # more groups than CUs
    ([0, 256], [8192], -1, 16, 64, 4),
    ([0, 150], [4096], -1, 16, 32, 0),
    ([0, 41], [1024], -1, 0, 32, 0),
    ([0, 256], [8192], 128, 16, 32, 2),
    ([0, 150], [4096], -1, 16, 32, 8),
    ([0, 64, 100, 164], [8192, 20000, 0], -1, 16, 32, 0),
    ([0, 30], [0], -1, 0, 32, 0),
    ([0, 150, 300], [777, 33], 500, 1, 32, 4),
    ([64 * i for i in range(33)], [8192] * 32, -1, 16, 32, 0),
    ([0, 0, 40], [100, 5000], -1, 16, 32, 0),                       # a request with no queries
])
def test_plan_partitions_work(qo, pl, window, page, hq, waves):
    """Every (request, kv head, q-tile) group: prefix items partition its
    visible prefix on 64-key tile boundaries into consecutive slots (each
    naming the window start and the planned length), one suffix item covers
    its nodes, and the group's slots are merged exactly once, by one merge
    item per 32-row block; a group without prefix keys has a FINAL suffix item
    and no merge.  When no group's prefix is split the plan is fused: one
    FINAL item per group reads its whole visible prefix and its suffix
    (SRC_BOTH), with no slots and no merges."""
    hkv = 8
    g = hq // hkv
    page_indptr = None
    if page:
        page_indptr = np.concatenate([[0], np.cumsum((np.asarray(pl) + page - 1) // page)])
    info, items, merges = _plan(qo, pl, hq, hkv, 128, window, page_size=page, waves=waves,
                                page_indptr=page_indptr)
    assert info.workspace_bytes == info.num_slots * info.rows_per_tile * (128 * 2 + 4)
    assert info.prefix_extent == (page_indptr[-1] if page else max([p for p in pl if p > 0] + [0]))
    rows = info.rows_per_tile
    assert info.waves_per_block in (2, 4, 8)
    assert rows == {2: 128, 4: 128, 8: 256}[info.waves_per_block]
    assert items.shape[0] == 0 or items[-1, MODE] != MODE_NOOP
    live = items[items[:, MODE] != MODE_NOOP]
    assert len(live) <= 256 * (1 if info.waves_per_block == 8 else 2) or len(qo) > 30
    pre, suf = {}, {}
    for it in live.tolist():
        key = (it[REQ], it[KVH], it[QT])
        r = it[REQ]
        assert it[Q0] == qo[r] and it[NQ] == qo[r + 1] - qo[r]
        if it[SRC] == SRC_BOTH:
            assert info.fused == 1 and it[MODE] == MODE_FINAL and it[SLOT] == -1 and key not in suf
            Leff = min(pl[r], window) if window >= 0 else pl[r]
            assert (it[KB], it[KE], it[KV0], it[PLAN_LEN]) == (pl[r] - Leff, pl[r], pl[r] - Leff, pl[r])
            assert it[BASE] == (page_indptr[r] if page else 0)
            suf[key] = (-1, MODE_FINAL)
            pre[key] = [(it[KB], it[KE], -1)]
        elif it[SRC] == SRC_PREFIX:
            assert info.fused == 0 and it[MODE] == MODE_PARTIAL
            assert it[BASE] == (page_indptr[r] if page else 0)
            Leff = min(pl[r], window) if window >= 0 else pl[r]
            assert it[KV0] == pl[r] - Leff and it[PLAN_LEN] == pl[r]
            pre.setdefault(key, []).append((it[KB], it[KE], it[SLOT]))
        else:
            assert it[SRC] == SRC_SUFFIX and key not in suf
            assert (it[KB], it[KE], it[BASE]) == (0, qo[r + 1] - qo[r], qo[r])
            suf[key] = (it[SLOT], it[MODE])
    if info.fused:
        assert info.num_slots == 0 and info.num_merges == 0 and info.workspace_bytes == 0
        assert info.max_splits_used == 1
        # one item per group: SRC_BOTH where the request has prefix keys
        want = {(r, h, qt) for r in range(len(pl)) for h in range(hkv)
                for qt in range(-(-(qo[r + 1] - qo[r]) * g // info.rows_per_tile))}
        assert set(suf) == want
        for (r, h, qt) in want:
            Leff = min(pl[r], window) if window >= 0 else pl[r]
            assert ((r, h, qt) in pre) == (Leff > 0)
        return
    all_slots = [c[2] for v in pre.values() for c in v] + [v[0] for v in suf.values() if v[1] == MODE_PARTIAL]
    assert len(all_slots) == len(set(all_slots)) == info.num_slots
    assert sorted(all_slots) == list(range(info.num_slots))
    mg = {}
    for i, m in enumerate(merges.tolist()):
        if m[4] == 0:          # padding
            continue
        key = (m[0], m[1], m[2])
        assert m[7] not in mg.setdefault(key, {})
        mg[key][m[7]] = (m[3], m[4], m[5], m[6], i % 8)
    # every item of a group runs on one XCD (workgroup index % 8) and so do
    # its merge workgroups, when there are at least 8 (request, kv head) pairs
    xcd_of = {}
    for i, it in enumerate(items.tolist()):
        if it[MODE] != MODE_NOOP:
            xcd_of.setdefault((it[REQ], it[KVH], it[QT]), set()).add(i % 8)
    heads = sum(hkv for r in range(len(pl)) if qo[r + 1] > qo[r])
    if heads >= 8:
        assert all(len(v) == 1 for v in xcd_of.values())
    for r in range(len(pl)):
        n = qo[r + 1] - qo[r]
        L = pl[r]
        Leff = min(L, window) if window >= 0 else L
        for h in range(hkv):
            for qt in range((n * g + rows - 1) // rows):
                key = (r, h, qt)
                assert key in suf
                ch = sorted(pre.get(key, []))
                if Leff == 0:
                    assert ch == [] and suf[key] == (-1, MODE_FINAL) and key not in mg
                    continue
                assert ch[0][0] == L - Leff and ch[-1][1] == L
                for (a, b, _), (c, _, _) in zip(ch[:-1], ch[1:]):
                    assert b == c and (b - ch[0][0]) % 64 == 0
                s0 = ch[0][2]
                assert [c[2] for c in ch] == list(range(s0, s0 + len(ch)))
                assert suf[key] == (s0 + len(ch), MODE_PARTIAL)
                blks = [b for b in range(rows // 32) if qt * rows + b * 32 < n * g]
                assert sorted(mg[key]) == blks
                for b in blks:
                    assert mg[key][b][:4] == (s0, len(ch) + 1, qo[r], n)
                    if heads >= 8:
                        assert {mg[key][b][4]} == xcd_of[key]
                # at most 15 chunks, unless the staged-page bound forces more
                assert len(ch) <= 15 or (page and -(-(Leff + 63) // 64) > 15 * _max_chunk_tiles(page))
                if page:
                    for a, b, _ in ch:
                        assert (b - 1) // page - a // page + 1 <= 1024


@pytest.mark.parametrize("qo,pl,split,window,tok1,tok2", [
    ([0, 80], [4096 + 17], [4096], -1, None, None),                 # DTA draft: cache 4096 | context 17
    ([0, 80], [4000 + 5], [4000], -1, [7], [3]),                    # split inside a tile, token offsets
    ([0, 80], [300], [0], -1, None, None),                          # all keys in the second segment
    ([0, 80], [300], [300], -1, None, None),                        # all keys in the first segment
    ([0, 80], [5000], [4990], 100, None, None),                     # window straddles the split
    ([0, 80], [5000], [4000], 100, None, None),                     # window inside the second segment
    ([0, 40, 120, 150], [1000, 9000, 64], [999, 100, 64], -1, [0, 1000, 9000], [0, 1, 9000]),
    ([0, 256], [8192 + 31], [8192], -1, None, None),
])
def test_plan_two_segment_prefix_partitions_keys(qo, pl, split, window, tok1, tok2):
    """A two-segment prefix: per group, the first segment's items and the
    second's (keys shifted by the split) cover the visible keys of the
    concatenation exactly once, in slot order, no item holds keys of both
    segments, each segment's chunks start on 64-key tiles of its own, items
    name their segment's token offset, and no such plan is fused."""
    hkv, hq = 8, 32
    g = hq // hkv
    info, items, merges = _plan(qo, pl, hq, hkv, 128, window, page_size=0, tok_indptr=tok1, split=split, tok2=tok2)
    R = len(pl)
    t1 = tok1 or [0] * R
    t2 = tok2 or [0] * R
    kv0 = [pl[r] - (min(pl[r], window) if window >= 0 else pl[r]) for r in range(R)]
    sees2 = any(qo[r + 1] > qo[r] and pl[r] > max(split[r], kv0[r]) for r in range(R))
    assert info.two_segment == int(sees2)
    assert info.fused == 0 or not sees2
    assert info.prefix_extent == max([t1[r] + split[r] for r in range(R) if split[r] > 0] + [0])
    assert info.prefix2_extent == max([t2[r] + pl[r] - split[r] for r in range(R) if pl[r] > split[r]] + [0])
    live = items[items[:, MODE] != MODE_NOOP].tolist()
    pre = {}
    for it in live:
        r = it[REQ]
        key = (r, it[KVH], it[QT])
        if it[SRC] in (SRC_PREFIX, SRC_BOTH):
            assert it[BASE] == t1[r] and it[KE] <= split[r] and (it[KB] - kv0[r]) % 64 == 0
            pre.setdefault(key, []).append((it[KB], it[KE], it[SLOT], 1))
        elif it[SRC] == SRC_PREFIX2:
            b0 = max(kv0[r], split[r]) - split[r]
            assert it[BASE] == t2[r] and it[MODE] == MODE_PARTIAL and 0 <= it[KB] < it[KE] <= pl[r] - split[r]
            assert (it[KB] - b0) % 64 == 0
            pre.setdefault(key, []).append((it[KB] + split[r], it[KE] + split[r], it[SLOT], 2))
    for r in range(R):
        n = qo[r + 1] - qo[r]
        for h in range(hkv):
            for qt in range(-(-n * g // info.rows_per_tile)):
                ch = sorted(pre.get((r, h, qt), []))
                if kv0[r] == pl[r]:
                    assert ch == []
                    continue
                assert ch[0][0] == kv0[r] and ch[-1][1] == pl[r]
                assert all(b == c for (_, b, _, _), (c, _, _, _) in zip(ch[:-1], ch[1:]))
                assert all(e <= split[r] for _, e, _, s in ch if s == 1)
                assert all(b >= split[r] for b, _, _, s in ch if s == 2)
                if not info.fused:
                    s0 = ch[0][2]
                    assert [c[2] for c in ch] == list(range(s0, s0 + len(ch)))
    blocks = {}
    for m in merges.tolist():
        if m[4]:
            blocks[(m[0], m[1], m[2])] = m[4]
    for key, ch in pre.items():
        if not info.fused:
            assert blocks[key] == len(ch) + 1   # the chunks of both segments and the suffix


@pytest.mark.parametrize("qo,pl,window", [([0, 150], [4608], -1), ([0, 156], [4096], -1), ([0, 64, 100], [9000, 700], -1),
                                          ([0, 150], [4608], 3000), ([64 * i for i in range(9)], [6000] * 8, -1)])
def test_plan_numbers_chunks_first_round_first(qo, pl, window):
    """Plans number the chunks of each group's whole visible prefix 0..S-1 in
    key order, sized as a dynamic plan's kernels partition a run-time prefix
    (the first nt % S chunks one tile longer), and run a group's first chunks
    in the first resident round of its XCD's CUs: every first-round chunk of a
    group precedes its second-round chunks.  A dynamic plan of the shape is
    the same plan."""
    info, items, _ = _plan(qo, pl, window=window)
    _, ditems, _ = _plan(qo, pl, window=window, dynamic=1)
    assert (items == ditems).all()
    CHUNK = 14
    groups = {}
    for i, it in enumerate(items.tolist()):
        if it[MODE] == MODE_NOOP or it[SRC] == SRC_SUFFIX:
            continue
        assert it[CHUNK] != 0
        c, S = it[CHUNK] & 0xFFFF, it[CHUNK] >> 16
        groups.setdefault((it[REQ], it[KVH], it[QT]), []).append((c, S, it[KB], it[KE], i))
    K = 256 // 8
    for (r, h, qt), v in groups.items():
        v.sort()
        S = v[0][1]
        assert [c for c, *_ in v] == list(range(S)) and {x[1] for x in v} == {S}
        L = pl[r]
        k0 = L - (min(L, window) if window >= 0 else L)
        nt = -(-(L - k0) // 64)
        sizes = [-(-(e - b) // 64) for _, _, b, e, _ in v]
        assert v[0][2] == k0 and v[-1][3] == L
        assert sizes == [nt // S + (c < nt % S) for c in range(S)]
        rounds = [(i // 8) // K for *_, i in v]           # workgroup i runs on XCD i % 8, round (i // 8) // K
        assert rounds == sorted(rounds)


@pytest.mark.parametrize("nodes,L,lone,longest_tiles", [(96, 4096, True, 7), (150, 4096, False, 6),
                                                          (96, 2048, False, 3), (96, 8192, True, 13)])
def test_plan_lone_workgroups_where_chunks_stay_short(nodes, L, lone, longest_tiles):
    """24 or 40 q-tile groups.  Where paired chunks would be at least 4 tiles
    and one workgroup per CU keeps the longest prefix chunk under 1.6x that
    length, the plan leaves each CU one workgroup: 96 nodes at 4096 keys get
    10 chunks of 6-7 tiles per group on 33 items per XCD, whose one CU pair
    holds two suffix items.  Otherwise CUs run two workgroups: 150 nodes get
    12 chunks of 5-6 tiles, 64 items per XCD; 96 nodes at 2048 keys keep 15
    chunks of 2-3 tiles (the per-item fixed cost dominates there)."""
    info, items, _ = _plan([0, nodes], [L])
    its = items.tolist()
    K = 256 // 8
    per_xcd = [0] * 8
    for i, it in enumerate(its):
        if it[MODE] != MODE_NOOP:
            per_xcd[i % 8] += 1
    chunks = [it for it in its if it[MODE] != MODE_NOOP and it[SRC] != SRC_SUFFIX]
    longest = max(-(-(it[KE] - it[KB]) // 64) for it in chunks)
    # workgroup i runs on XCD i % 8; i and i + 8K share a CU
    pairs = [(it[SRC], its[i - 8 * K][SRC]) for i, it in enumerate(its) if i // 8 >= K and it[MODE] != MODE_NOOP]
    assert longest == longest_tiles
    if lone:
        assert per_xcd == [K + 1] * 8 and len(chunks) == 24 * 10
        assert pairs == [(SRC_SUFFIX, SRC_SUFFIX)] * 8
    else:
        assert min(per_xcd) > K + 1
        assert any(a == SRC_PREFIX and b == SRC_PREFIX for a, b in pairs)


def test_plan_rejects_bad_two_segment_prefixes():
    """A second segment needs a contiguous first one and a static plan, and
    each split must lie in [0, prefix_len]."""
    qo = np.asarray([0, 10], dtype=np.int32)
    pl = np.asarray([100], dtype=np.int32)
    for page, dyn, sp, code, msg in ((16, 0, 50, 2, b"contiguous"), (0, 1, 50, 2, b"static"),
                                     (0, 0, 101, 1, b"prefix_split"), (0, 0, -1, 1, b"prefix_split")):
        desc = _lib.PlanDesc()
        desc.num_reqs = 1
        desc.qo_indptr = qo.ctypes.data_as(C.POINTER(C.c_int32))
        desc.prefix_len = pl.ctypes.data_as(C.POINTER(C.c_int32))
        desc.num_qo_heads, desc.num_kv_heads, desc.head_dim = 32, 8, 128
        pi = np.asarray([0, 7], dtype=np.int32)
        desc.page_indptr = pi.ctypes.data_as(C.POINTER(C.c_int32))
        desc.page_size, desc.dynamic_prefix = page, dyn
        s = np.asarray([sp], dtype=np.int32)
        desc.prefix_split = s.ctypes.data_as(C.POINTER(C.c_int32))
        info = _lib.PlanInfo()
        assert _lib.lib.d2sd_cascade_plan(C.byref(desc), None, 0, C.byref(info)) == code
        assert msg in _lib.lib.d2sd_last_error()


@pytest.mark.parametrize("field,value,msg", [("k_prefix2", 0, b"k_prefix2"), ("prefix2_extent", 16, b"fewer tokens"),
                                             ("k_prefix2", 8, b"aligned")])
def test_cascade_run_rejects_a_missing_second_segment_without_launching(field, value, msg):
    """A plan that reads a second prefix segment refuses a null, misaligned
    or short second segment before any launch (pointers never dereferenced)."""
    info, _, _ = _plan([0, 10], [300], page_size=0, split=[280])
    assert info.two_segment == 1 and info.prefix2_extent == 20 and info.prefix_extent == 280
    fake = 1 << 20
    a = _lib.RunArgs()
    a.plan = a.q = a.k_suffix = a.v_suffix = a.out = a.k_prefix = a.v_prefix = fake
    a.k_prefix2 = a.v_prefix2 = fake
    a.workspace, a.workspace_bytes = fake, info.workspace_bytes
    a.q_stride_n, a.q_stride_h = 32 * 128, 128
    a.suffix_stride_n, a.suffix_stride_h = 8 * 128, 128
    a.o_stride_n, a.o_stride_h = 32 * 128, 128
    a.prefix_stride_tok, a.prefix_stride_head = 128, 300 * 128
    a.prefix2_stride_tok, a.prefix2_stride_head, a.prefix2_extent = 128, 20 * 128, 20
    a.prefix_extent, a.sm_scale = 300, 0.088
    setattr(a, field, (fake + value) if (field == "k_prefix2" and value) else value)
    rc = _lib.lib.d2sd_cascade_run(C.byref(info), C.byref(a), None)
    assert rc == 1 and msg in _lib.lib.d2sd_last_error()


def _max_chunk_tiles(page):
    """The longest paged chunk (64-key tiles) the kernel can stage: 64 T + 63
    keys from any start span at most 1024 pages."""
    return max(1, (1023 * page - 62) // 64)


@pytest.mark.parametrize("page", [1, 2, 4, 8, 16])
@pytest.mark.parametrize("L", [1000, 16384, 32768, 131072, 262144])
@pytest.mark.parametrize("d,hq,fp8,waves", [(128, 64, 1, 4), (128, 32, 0, 8), (64, 64, 0, 4), (64, 64, 1, 8)])
@pytest.mark.parametrize("dynamic,window", [(0, -1), (1, -1), (1, 5000)])
def test_plan_keeps_paged_chunks_within_staged_pages(page, L, d, hq, fp8, waves, dynamic, window):
    """Every paged prefix item reads at most 1024 pages, the page ids one
    workgroup stages in LDS, even where that needs more than 15 chunks per
    group (page size 1 at 16K keys, 2 at 32K, 16 at 256K), and even for the
    run-time chunks of a dynamic plan (up to 63 keys longer than planned,
    from any start key); the chunks still cover each group's visible prefix
    once."""
    n = 40
    info, items, merges = _plan([0, n], [L], hq=hq, hkv=8, d=d, window=window, waves=waves, page_size=page,
                                dynamic=dynamic, kv_dtype=fp8)
    live = items[items[:, MODE] != MODE_NOOP]
    pre = live[live[:, SRC] != SRC_SUFFIX]
    assert len(pre) > 0
    for it in pre.tolist():
        keys = it[KE] - it[KB]
        assert (it[KE] - 1) // page - it[KB] // page + 1 <= 1024
        if dynamic:
            assert (keys + 63 + page - 2) // page + 1 <= 1024
    Leff = min(L, window) if window >= 0 else L
    by_group = {}
    for it in pre.tolist():
        by_group.setdefault((it[KVH], it[QT]), []).append((it[KB], it[KE]))
    for ch in by_group.values():
        ch.sort()
        assert ch[0][0] == L - Leff and ch[-1][1] == L
        assert all(b == c for (_, b), (c, _) in zip(ch[:-1], ch[1:]))
    # the merge covers every chunk plus the suffix partial of each group
    nslots = {(m[1], m[2]): m[4] for m in merges.tolist() if m[4] > 0}
    assert all(nslots[k] == len(v) + 1 for k, v in by_group.items())
    need = -(-(-(-Leff // 64)) // _max_chunk_tiles(page))   # chunks the staged-page bound forces
    assert max(len(v) for v in by_group.values()) >= need
    if page == 1 and Leff >= 16384:
        assert need > 15


def test_cascade_run_rejects_a_mask_narrower_than_the_widest_request():
    """A tree mask of fewer 64-bit words per row than the widest request's
    nodes need is refused before any launch (the kernel would read the next
    row's words)."""
    info, _, _ = _plan([0, 10, 140], [300, 300], page_size=0)
    assert info.max_qo_len == 130
    fake = 1 << 20
    a = _lib.RunArgs()
    a.plan = a.q = a.k_suffix = a.v_suffix = a.out = a.k_prefix = a.v_prefix = a.tree_mask = fake
    a.workspace, a.workspace_bytes = fake, info.workspace_bytes
    a.q_stride_n, a.q_stride_h = 32 * 128, 128
    a.suffix_stride_n, a.suffix_stride_h = 8 * 128, 128
    a.o_stride_n, a.o_stride_h = 32 * 128, 128
    a.prefix_stride_tok, a.prefix_stride_head = 128, 1024 * 128
    a.prefix_extent, a.sm_scale = 1024, 0.088
    a.mask_mode, a.mask_words = _lib.D2SD_MASK_TREE, 2
    rc = _lib.lib.d2sd_cascade_run(C.byref(info), C.byref(a), None)
    assert rc == 1 and b"mask_words" in _lib.lib.d2sd_last_error()


def test_plan_chooses_waves():
    """waves_per_block 0: 8-wave (256-row) tiles once the 4-wave plan has a
    q-tile group per workgroup slot and a kv head packs > 128 rows (many
    large requests), else 4 waves."""
    qo = [143 * i for i in range(33)]                    # 32 requests x 143 nodes, 64/8 heads
    info, _, _ = _plan(qo, [8192] * 32, hq=64, hkv=8)
    assert info.waves_per_block == 8 and info.rows_per_tile == 256
    info, _, _ = _plan([0, 150], [4096])                 # one request: the prefix is split, 4 waves
    assert info.waves_per_block == 4
    qo = [30 * i for i in range(33)]                     # many requests, 120 rows per kv head
    info, _, _ = _plan(qo, [8192] * 32, hq=32, hkv=8)
    assert info.waves_per_block == 4
    info, _, _ = _plan([143 * i for i in range(33)], [8192] * 32, hq=64, hkv=8, waves=4)
    assert info.waves_per_block == 4                     # an explicit choice stands


def test_plan_fills_the_device_once():
    info, items, _ = _plan([0, 150], [4096])
    live = (items[:, MODE] != MODE_NOOP).sum()
    assert info.waves_per_block == 4 and 256 < live <= 512
    info, items, _ = _plan([0, 41], [1024], page_size=0)
    assert (items[:, MODE] != MODE_NOOP).sum() <= 512


def test_plan_balances_cu_pairs():
    """One request of 4096 keys, 150 nodes (the Qwen3-8B verify step): every
    XCD gets 64 workgroups (two per CU), and the two that share a CU (k-th of
    the first and k-th of the second round of that XCD) hold at most 11
    64-key tiles together, a suffix item counting as twice its tiles."""
    info, items, _ = _plan([0, 150], [4096])
    assert info.num_items == 512 and info.waves_per_block == 4
    cost = [(w[KE] - w[KB] + 63) // 64 if w[SRC] == SRC_PREFIX else 2 * ((w[NQ] + 63) // 64)
            for w in items.tolist()]
    for x in range(8):
        c = cost[x::8]
        assert len(c) == 64
        pairs = [c[k] + c[k + 32] for k in range(32)]
        assert max(pairs) <= 11, pairs


def test_plan_contiguous_token_offsets():
    _, items, _ = _plan([0, 10, 30], [100, 200], page_size=0, tok_indptr=[0, 100])
    for it in items[items[:, MODE] != MODE_NOOP].tolist():
        if it[SRC] == SRC_PREFIX:
            assert it[BASE] == [0, 100][it[REQ]]


def test_plan_xcd_grouping():
    """Items reading the same keys sit on one XCD (work index % 8): with at
    least 8 (request, kv head) pairs, everything of one pair; otherwise every
    key chunk with all the q-tiles that read it."""
    for qo, pl, hkv, key_fn in (([0, 150, 200], [4096, 3000], 8, lambda w: (w[REQ], w[KVH])),
                                ([0, 150], [4096], 4, lambda w: (w[SRC], w[REQ], w[KVH], w[KB]))):
        info, items, _ = _plan(qo, pl, hq=8 * hkv, hkv=hkv)
        xcd = {}
        for i, w in enumerate(items.tolist()):
            if w[MODE] == MODE_NOOP:
                continue
            xcd.setdefault(key_fn(w), set()).add(i % 8)
        assert all(len(s) == 1 for s in xcd.values())
        assert len({x for s in xcd.values() for x in s}) == 8   # all XCDs used


def test_plan_rejects_bad_input():
    desc = _lib.PlanDesc()
    qo = np.asarray([0, 10], dtype=np.int32)
    pl = np.asarray([100], dtype=np.int32)
    desc.num_reqs = 1
    desc.qo_indptr = qo.ctypes.data_as(C.POINTER(C.c_int32))
    desc.prefix_len = pl.ctypes.data_as(C.POINTER(C.c_int32))
    desc.num_qo_heads, desc.num_kv_heads, desc.head_dim = 32, 8, 96
    info = _lib.PlanInfo()
    assert _lib.lib.d2sd_cascade_plan(C.byref(desc), None, 0, C.byref(info)) == 2
    assert b"head_dim" in _lib.lib.d2sd_last_error()
    desc.head_dim, desc.num_qo_heads = 128, 30
    assert _lib.lib.d2sd_cascade_plan(C.byref(desc), None, 0, C.byref(info)) == 1
    desc.num_qo_heads = 32
    desc.page_size = 16                     # paged without page_indptr
    assert _lib.lib.d2sd_cascade_plan(C.byref(desc), None, 0, C.byref(info)) == 1
    assert b"page_indptr" in _lib.lib.d2sd_last_error()
    pi = np.asarray([0, 3], dtype=np.int32)  # 3 pages < ceil(100 / 16)
    desc.page_indptr = pi.ctypes.data_as(C.POINTER(C.c_int32))
    assert _lib.lib.d2sd_cascade_plan(C.byref(desc), None, 0, C.byref(info)) == 1
    desc.page_size, desc.waves_per_block = 0, 6
    assert _lib.lib.d2sd_cascade_plan(C.byref(desc), None, 0, C.byref(info)) == 1


def test_c_abi_rejects_bad_arguments_without_launching():
    lib = _lib.lib
    # misaligned q pointer -> invalid argument before any launch
    rc = lib.d2sd_single_prefill_with_kv_cache(8, 4096, 128, 16, 16, 1024, 128, 16, 4096, 128, None,
                                               4, 4, 32, 8, 128, 0, -1, 0.1, 0, None, 0, None)
    assert rc == 1 and b"aligned" in lib.d2sd_last_error()
    rc = lib.d2sd_local_attention_merge(16, 0, 0, 0, 16, 16, 0, 0, 0, 16, 0, 0, 0, 16, 0, 0,
                                        2, 8, 32, 8, 80, 1, 0.1, None, 0, None)
    assert rc == 2


@pytest.mark.parametrize("page_size,extent,msg", [(0, 299, b"fewer tokens"), (0, -1, b"fewer tokens"),
                                                  (16, 0, b"page count")])
def test_cascade_run_rejects_a_short_prefix_without_launching(page_size, extent, msg):
    """A contiguous k_prefix shorter than the keys the plan reads (300 tokens
    here), or a paged pool of no pages, is refused before any launch (the
    pointers are never dereferenced)."""
    info, _, _ = _plan([0, 10], [300], page_size=page_size)
    assert info.prefix_extent == (300 if page_size == 0 else info.prefix_extent)
    fake = 1 << 20
    a = _lib.RunArgs()
    a.plan = a.q = a.k_suffix = a.v_suffix = a.out = a.k_prefix = a.v_prefix = a.page_table = fake
    a.workspace, a.workspace_bytes = fake, info.workspace_bytes
    a.q_stride_n, a.q_stride_h = 32 * 128, 128
    a.suffix_stride_n, a.suffix_stride_h = 8 * 128, 128
    a.o_stride_n, a.o_stride_h = 32 * 128, 128
    a.prefix_stride_tok, a.prefix_stride_head, a.prefix_stride_page = 128, 300 * 128, 16 * 8 * 128
    a.page_size, a.prefix_extent, a.sm_scale = page_size, extent, 0.088
    rc = _lib.lib.d2sd_cascade_run(C.byref(info), C.byref(a), None)
    assert rc == 1 and msg in _lib.lib.d2sd_last_error()


def test_python_surface_rejects_cpu_tensors():
    q = torch.zeros(4, 32, 128, dtype=torch.bfloat16)
    k = torch.zeros(16, 8, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="device"):
        d2sd.single_prefill_with_kv_cache(q, k, k, causal=True, return_lse=True)
    with pytest.raises(ValueError, match="device"):
        d2sd.merge_state_in_place(q, torch.zeros(4, 32), q.clone(), torch.zeros(4, 32))


def _kv_args(**kw):
    a = _lib.KvAppendArgs()
    base = dict(num_layers=2, num_kv_heads=8, head_dim=128, page_size=16, prefix_len=100, num_accepted=5,
                num_rows=40, pool_pages=64, page_table_len=8, node_ids=8, page_table=8, k_new=8, v_new=8,
                k_pool=8, v_pool=8, new_stride_n=1024, new_stride_h=128, pool_stride_page=16384,
                pool_stride_head=2048, pool_stride_tok=128)
    base.update(kw)
    for k, v in base.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("bad", [dict(page_size=12), dict(head_dim=100), dict(num_rows=0), dict(k_pool=None),
                                 dict(new_stride_h=100), dict(prefix_len=-1), dict(page_table_len=6),
                                 dict(pool_stride_tok=0), dict(pool_dtype=2), dict(pool_dtype=1),
                                 dict(pool_dtype=1, k_scale=8)])
def test_kv_append_rejects_bad_arguments(bad):
    """Argument checks of d2sd_paged_kv_append happen before any GPU work."""
    rc = _lib.lib.d2sd_paged_kv_append(C.byref(_kv_args(**bad)), None)
    assert rc == 1, _lib.lib.d2sd_last_error()            # D2SD_ERR_INVALID_ARG
    assert _lib.lib.d2sd_last_error().startswith(b"paged_kv_append")


def test_commit_rejects_scales_and_dtypes_on_the_host():
    import d2sd
    pool = torch.zeros(4, 2, 16, 8, dtype=torch.float8_e4m3fn)
    new = torch.zeros(3, 2, 8, dtype=torch.bfloat16)
    with pytest.raises(ValueError):   # fp8 pools need scales
        d2sd.PagedKVCommit([pool], [pool], [new], [new])
    with pytest.raises(ValueError):   # scales of the wrong size
        d2sd.PagedKVCommit([pool], [pool], [new], [new], k_scales=torch.ones(3), v_scales=torch.ones(2))
    with pytest.raises(ValueError):   # scales with bf16 pools
        b = torch.zeros(4, 2, 16, 8, dtype=torch.bfloat16)
        d2sd.PagedKVCommit([b], [b], [new], [new], k_scales=torch.ones(2), v_scales=torch.ones(2))
    with pytest.raises(TypeError):
        f = torch.zeros(4, 2, 16, 8, dtype=torch.float16)
        d2sd.PagedKVCommit([f], [f], [new], [new])


def test_kv_append_with_nothing_to_append_launches_nothing():
    assert _lib.lib.d2sd_paged_kv_append(C.byref(_kv_args(num_accepted=0)), None) == 0
    assert _lib.lib.d2sd_paged_kv_append(C.byref(_kv_args(num_layers=0)), None) == 0


@pytest.mark.parametrize("nodes,vocab", [(150, 151936), (1, 7), (1, 151936), (4000, 32000)])
def test_greedy_accept_workspace_covers_the_chunks(nodes, vocab):
    ws = _lib.lib.d2sd_greedy_accept_workspace_size(nodes, vocab)
    assert ws % (8 * nodes) == 0
    chunks = ws // (8 * nodes)
    assert 1 <= chunks and chunks * 1024 <= max(vocab + 1023, 1024) + 8 * chunks


def test_greedy_accept_rejects_bad_arguments():
    a = _lib.AcceptArgs()
    a.num_rows, a.row_len, a.num_nodes, a.vocab, a.logits_dtype = 5, 32, 150, 1000, 0
    a.logits_stride = 1000
    for f in ("logits", "node_index", "draft_ids", "accept_ids", "accept_nodes", "result", "workspace"):
        setattr(a, f, 8)
    a.workspace_bytes = 1 << 30
    for field, bad in (("num_rows", 65), ("logits_dtype", 7), ("logits_stride", 999), ("workspace", None)):
        old = getattr(a, field)
        setattr(a, field, bad)
        assert _lib.lib.d2sd_greedy_accept(C.byref(a), None) == 1
        assert _lib.lib.d2sd_last_error().startswith(b"greedy_accept")
        setattr(a, field, old)
    a.workspace_bytes = 8
    assert _lib.lib.d2sd_greedy_accept(C.byref(a), None) == 3   # D2SD_ERR_WORKSPACE


def test_sample_accept_rejects_bad_arguments():
    s = _lib.SampleAcceptArgs()
    a = s.walk
    a.num_rows, a.row_len, a.num_nodes, a.vocab, a.logits_dtype = 5, 32, 150, 1000, 0
    a.logits_stride = 1000
    for f in ("logits", "node_index", "draft_ids", "accept_ids", "accept_nodes", "result", "workspace"):
        setattr(a, f, 8)
    a.workspace_bytes = 1 << 30
    for t in (-0.5, float("nan"), float("inf")):
        s.temperature = t
        assert _lib.lib.d2sd_sample_accept(C.byref(s), None) == 1
        assert _lib.lib.d2sd_last_error().startswith(b"sample_accept: temperature")
    s.temperature, s.rng_step = 0.7, None       # sampling needs the step counter
    assert _lib.lib.d2sd_sample_accept(C.byref(s), None) == 1
    assert b"rng_step" in _lib.lib.d2sd_last_error()
    s.rng_step = 8
    a.num_rows = 65                              # the walk's own checks apply
    assert _lib.lib.d2sd_sample_accept(C.byref(s), None) == 1
    assert _lib.lib.d2sd_last_error().startswith(b"greedy_accept: num_rows")


def test_accept_rejects_bad_temperature():
    import d2sd
    for t in (-1.0, float("nan"), float("inf")):
        with pytest.raises(ValueError):
            d2sd.TreeAccept(10, 100, 4, "cpu", temperature=t)


def test_bench_workloads_build_and_plan():
    """Every `bench.py --workload` name builds its problem, whose sizes the
    planner accepts (host work only: the plan is computed, nothing runs)."""
    import importlib.util
    spec = importlib.util.spec_from_file_location("bench", Path(__file__).resolve().parents[1] / "bench.py")
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    from d2sd import workloads as wl
    for name, make in bench.OTHER_WORKLOADS.items():
        prob, pools = make(wl, 0)
        assert pools >= 1 and prob.total_q > 0, name
        qo = np.asarray(prob.qo_indptr)
        page = prob.page_size
        pl = np.asarray(prob.prefix_lens)
        page_indptr = np.concatenate([[0], np.cumsum((pl + page - 1) // page)]) if page else None
        info, items, _ = _plan(qo.tolist(), pl.tolist(), prob.num_qo_heads, prob.num_kv_heads, prob.head_dim,
                               prob.window_left, page_size=page, page_indptr=page_indptr)
        assert info.num_items > 0 and info.waves_per_block in (4, 8), name


def test_torch_ops_registered_with_meta_kernels():
    """torch.ops.d2sd.* (libd2sd_torch.so over the C ABI) is registered at
    import; the meta kernels give the output shapes without a device."""
    for op in ("single_prefill_with_kv_cache", "merge_state_in_place", "local_attention_merge", "cascade_run",
               "cascade_run_no_alloc"):
        assert hasattr(torch.ops.d2sd, op)
    q = torch.empty(10, 32, 128, dtype=torch.bfloat16, device="meta")
    k = torch.empty(8, 100, 128, dtype=torch.bfloat16, device="meta")
    o, lse = torch.ops.d2sd.single_prefill_with_kv_cache(q, k, k, True, "HND", 0.1, False)
    assert o.shape == q.shape and o.dtype == torch.bfloat16 and lse.shape == (10, 32) and lse.dtype == torch.float32
    v = torch.empty(10, 32, 128, dtype=torch.bfloat16, device="meta")
    s = torch.empty(10, 32, dtype=torch.float32, device="meta")
    torch.ops.d2sd.merge_state_in_place(v, s, v, s, False)


def test_torch_ops_reject_cpu_tensors():
    q = torch.zeros(4, 32, 128, dtype=torch.bfloat16)
    k = torch.zeros(16, 8, 128, dtype=torch.bfloat16)
    with pytest.raises((RuntimeError, NotImplementedError)):
        torch.ops.d2sd.single_prefill_with_kv_cache(q, k, k, False, "NHD", None, False)
