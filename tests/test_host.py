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


def _plan(qo, pl, hq=32, hkv=8, d=128, window=-1, num_cus=256, waves=0, max_splits=0):
    desc = _lib.PlanDesc()
    qo = np.asarray(qo, dtype=np.int32)
    pl = np.asarray(pl, dtype=np.int32)
    desc.num_reqs = len(pl)
    desc.qo_indptr = qo.ctypes.data_as(C.POINTER(C.c_int32))
    desc.prefix_len = pl.ctypes.data_as(C.POINTER(C.c_int32))
    desc.num_qo_heads, desc.num_kv_heads, desc.head_dim = hq, hkv, d
    desc.window_left = window
    desc.kv_dtype = 0
    desc.num_cus = num_cus
    desc.max_splits = max_splits
    desc.waves_per_block = waves
    info = _lib.PlanInfo()
    assert _lib.lib.d2sd_cascade_plan(C.byref(desc), None, 0, C.byref(info)) == 0
    host = np.zeros(max(info.plan_ints, 8), dtype=np.int32)
    rc = _lib.lib.d2sd_cascade_plan(C.byref(desc), host.ctypes.data_as(C.POINTER(C.c_int32)), host.size,
                                    C.byref(info))
    assert rc == 0, _lib.lib.d2sd_last_error()
    work = host[: 8 * info.num_work].reshape(-1, 8)
    merge = host[8 * info.num_work: 8 * (info.num_work + info.num_merge)].reshape(-1, 8)
    return info, work, merge


@pytest.mark.parametrize("qo,pl,window", [
    ([0, 128], [4096], -1),
    ([0, 41], [1024], -1),
    ([0, 256], [8192], 128),
    ([0, 64, 100, 164], [8192, 20000, 0], -1),
    ([0, 30], [0], -1),
    ([0, 150, 300], [777, 33], 500),
])
def test_plan_partitions_work(qo, pl, window):
    hq, hkv = 32, 8
    g = hq // hkv
    info, work, merge = _plan(qo, pl, hq, hkv, 128, window)
    rows = info.rows_per_tile
    assert info.waves_per_block in (4, 8) and rows == 32 * info.waves_per_block
    live = work[work[:, 7] != 3]
    # NOOP padding only between live items, never at the end
    assert work.shape[0] == 0 or work[-1, 7] != 3
    cover = {}
    slots = []
    for req, kvh, qt, src, kb, ke, slot, mode in live.tolist():
        cover.setdefault((req, kvh, qt, src), []).append((kb, ke))
        if mode == 0:
            slots.append(slot)
        else:
            assert mode == 1 and slot == -1
    assert len(slots) == len(set(slots)) == info.num_slots
    for r in range(len(pl)):
        n = qo[r + 1] - qo[r]
        qtiles = (n * g + rows - 1) // rows
        L = pl[r]
        Leff = min(L, window) if window >= 0 else L
        for h in range(hkv):
            for qt in range(qtiles):
                # suffix level: exactly one item over [0, n)
                assert cover.get((r, h, qt, 1)) == [(0, n)]
                # prefix level: chunks partition [L - Leff, L), aligned to 64 from the start
                ch = sorted(cover.get((r, h, qt, 0), []))
                if Leff == 0:
                    assert ch == []
                    continue
                assert ch[0][0] == L - Leff and ch[-1][1] == L
                for (a, b), (c, _) in zip(ch[:-1], ch[1:]):
                    assert b == c and (b - ch[0][0]) % 64 == 0
    # merge items: one per group with > 1 item, slots contiguous and matching
    groups = {}
    for req, kvh, qt, src, kb, ke, slot, mode in live.tolist():
        groups.setdefault((req, kvh, qt), []).append(slot)
    for req, kvh, qt, sb, ns, mode, _, _ in merge.tolist():
        s = sorted(groups[(req, kvh, qt)])
        assert s == list(range(sb, sb + ns)) and ns > 1 and mode == 1
    assert len(merge) == sum(1 for v in groups.values() if len(v) > 1)
    assert info.workspace_bytes == info.num_slots * rows * (128 + 1) * 4


def test_plan_xcd_grouping():
    """All q-tiles of one (request, head, key chunk) sit on the same XCD
    (work index % 8)."""
    info, work, _ = _plan([0, 128], [4096])
    xcd = {}
    for i, (req, kvh, qt, src, kb, ke, slot, mode) in enumerate(work.tolist()):
        if mode == 3:
            continue
        xcd.setdefault((req, kvh, src, kb), set()).add(i % 8)
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
