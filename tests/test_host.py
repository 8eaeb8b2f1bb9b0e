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


def _plan(qo, pl, hq=32, hkv=8, d=128, window=-1, num_cus=256, waves=0, max_splits=0, page_size=16):
    desc = _lib.PlanDesc()
    qo = np.asarray(qo, dtype=np.int32)
    pl = np.asarray(pl, dtype=np.int32)
    desc.num_reqs = len(pl)
    desc.qo_indptr = qo.ctypes.data_as(C.POINTER(C.c_int32))
    desc.prefix_len = pl.ctypes.data_as(C.POINTER(C.c_int32))
    desc.num_qo_heads, desc.num_kv_heads, desc.head_dim = hq, hkv, d
    desc.window_left = window
    desc.kv_dtype = 0
    desc.page_size = page_size
    desc.num_cus = num_cus
    desc.max_splits = max_splits
    desc.waves_per_block = waves
    info = _lib.PlanInfo()
    assert _lib.lib.d2sd_cascade_plan(C.byref(desc), None, 0, C.byref(info)) == 0
    host = np.zeros(max(info.plan_ints, 8), dtype=np.int32)
    rc = _lib.lib.d2sd_cascade_plan(C.byref(desc), host.ctypes.data_as(C.POINTER(C.c_int32)), host.size,
                                    C.byref(info))
    assert rc == 0, _lib.lib.d2sd_last_error()
    npre, nsuf = info.num_prefix_work, info.num_suffix_work
    pre = host[: 8 * npre].reshape(-1, 8)
    suf = host[8 * npre: 8 * (npre + nsuf)].reshape(-1, 8)
    return info, pre, suf


MODE_PARTIAL, MODE_FINAL, MODE_NOOP, MODE_MERGE = 0, 1, 3, 4


@pytest.mark.parametrize("qo,pl,window,page,hq", [
    ([0, 128], [4096], -1, 16, 32),
    ([256 * i for i in range(33)], [8192] * 32, -1, 16, 64),   # more tile groups than CUs
    ([0, 256], [8192], -1, 16, 64),
    ([0, 150], [4096], -1, 16, 32),
    ([0, 41], [1024], -1, 0, 32),
    ([0, 256], [8192], 128, 16, 32),
    ([0, 64, 100, 164], [8192, 20000, 0], -1, 16, 32),
    ([0, 30], [0], -1, 0, 32),
    ([0, 150, 300], [777, 33], 500, 1, 32),
    ([64 * i for i in range(33)], [8192] * 32, -1, 16, 32),
])
def test_plan_partitions_work(qo, pl, window, page, hq):
    hkv = 8
    g = hq // hkv
    info, pre, suf = _plan(qo, pl, hq, hkv, 128, window, page_size=page)
    rows = info.prefix_rows
    assert info.prefix_waves in (4, 8) and rows == 32 * info.prefix_waves
    srows = 32 * info.suffix_waves
    assert rows % srows == 0
    for lst in (pre, suf):
        assert lst.shape[0] == 0 or lst[-1, 7] != MODE_NOOP
    cover, slots = {}, {}
    for req, kvh, qt, src, kb, ke, slot, mode in pre[pre[:, 7] != MODE_NOOP].tolist():
        assert src == 0 and mode == MODE_PARTIAL
        cover.setdefault((req, kvh, qt), []).append((kb, ke, slot))
    all_slots = [c[2] for v in cover.values() for c in v]
    assert len(all_slots) == len(set(all_slots)) == info.num_slots
    blocks = {}
    for req, kvh, qt, src, kb, ke, slot, mode in suf[suf[:, 7] != MODE_NOOP].tolist():
        assert src == 1
        blocks.setdefault((req, kvh), []).append((qt, kb, ke, slot, mode))
    for r in range(len(pl)):
        n = qo[r + 1] - qo[r]
        L = pl[r]
        Leff = min(L, window) if window >= 0 else L
        for h in range(hkv):
            qtiles = (n * g + rows - 1) // rows
            for qt in range(qtiles):
                ch = sorted(cover.get((r, h, qt), []))
                if Leff == 0:
                    assert ch == []
                    continue
                # chunks partition [L - Leff, L) on 64-key tile boundaries
                assert ch[0][0] == L - Leff and ch[-1][1] == L
                for (a, b, _), (c, _, _) in zip(ch[:-1], ch[1:]):
                    assert b == c and (b - ch[0][0]) % 64 == 0
                # the group's slots are consecutive in key order
                assert [c[2] for c in ch] == list(range(ch[0][2], ch[0][2] + len(ch)))
                if page:
                    for a, b, _ in ch:
                        assert (b - 1) // page - a // page + 1 <= 1024
            nb = (n * g + srows - 1) // srows
            bl = sorted(blocks.get((r, h), []))
            assert [b[0] for b in bl] == list(range(nb))
            for b, kb, ke, slot, mode in bl:
                assert (kb, ke) == (0, n)
                ch = sorted(cover.get((r, h, (b * srows) // rows), []))
                if ch:
                    assert mode & 0xff == MODE_MERGE and mode >> 8 == len(ch) and slot == ch[0][2]
                else:
                    assert mode == MODE_FINAL and slot == -1
    assert info.workspace_bytes == info.num_slots * rows * (128 * 2 + 4)


def test_plan_prefix_fits_one_wave_of_workgroups():
    info, pre, _ = _plan([0, 150], [4096])
    live = (pre[:, 7] != MODE_NOOP).sum()
    assert info.prefix_waves == 8 and live <= 256
    info, pre, _ = _plan([0, 41], [1024])
    assert (pre[:, 7] != MODE_NOOP).sum() <= 256 * (2 if info.prefix_waves == 4 else 1)


def test_plan_xcd_grouping():
    """Items reading the same keys sit on one XCD (work index % 8)."""
    info, pre, suf = _plan([0, 150, 200], [4096, 3000])
    for lst, key in ((pre, lambda w: (w[0], w[1], w[4])), (suf, lambda w: (w[0], w[1]))):
        xcd = {}
        for i, w in enumerate(lst.tolist()):
            if w[7] == MODE_NOOP:
                continue
            xcd.setdefault(key(w), set()).add(i % 8)
        assert all(len(s) == 1 for s in xcd.values())


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


def test_c_abi_rejects_bad_arguments_without_launching():
    lib = _lib.lib
    # misaligned q pointer -> invalid argument before any launch
    rc = lib.d2sd_single_prefill_with_kv_cache(8, 4096, 128, 16, 16, 1024, 128, 16, 4096, 128, None,
                                               4, 4, 32, 8, 128, 0, -1, 0.1, 0, None, 0, None)
    assert rc == 1 and b"aligned" in lib.d2sd_last_error()
    rc = lib.d2sd_local_attention_merge(16, 0, 0, 0, 16, 16, 0, 0, 0, 16, 0, 0, 0, 16, 0, 0,
                                        2, 8, 32, 8, 80, 1, 0.1, None, 0, None)
    assert rc == 2


def test_python_surface_rejects_cpu_tensors():
    q = torch.zeros(4, 32, 128, dtype=torch.bfloat16)
    k = torch.zeros(16, 8, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="device"):
        d2sd.single_prefill_with_kv_cache(q, k, k, causal=True, return_lse=True)
    with pytest.raises(ValueError, match="device"):
        d2sd.merge_state_in_place(q, torch.zeros(4, 32), q.clone(), torch.zeros(4, 32))
