"""CascadeVerifyAttention — plan()/run() for cascade tree-verification attention.

One run() computes, for every request r, what generation/verification.py:127-176
computes per layer with three FlashInfer calls, a CUDA graph and torch
elementwise ops:

  * prefix fetch + sliding-window truncation (verification.py:127-135),
  * shared-prefix attention of every suffix query (verification.py:145-150),
  * suffix attention under the tree (ancestor) mask — the per-row causal
    local level of verification.py:155-162 over unique tree nodes,
  * log-sum-exp merge (verification.py:163-165) and the GPT-OSS sink rescale
    (verification.py:173-176),

with the queries of request r = its tree nodes q[qo_indptr[r]:qo_indptr[r+1]].
plan() does all host work and device uploads; run() only launches kernels
(two per call: attention over prefix key chunks and suffix trees, writing
partial states, then their merge), allocates nothing when `out`/`lse` are
given, and can be captured into a HipGraph.

Device buffers.  The plan, workspace, tree mask and prefix lengths are
always plan-owned.  A page table, sinks or fp8 scales given as a contiguous
device tensor of the kernel's dtype (int32 / float32) are used in place (the
caller may update them between replays); given any other way they are
copied into a plan-owned buffer.  A re-plan with the same shape (work items,
merges, partial slots, mask width, the same optional inputs) rewrites every
plan-owned buffer in place, so a graph captured earlier replays the new plan;
after a run() has been captured, such a re-plan raises rather than hand a
buffer of another identity to the kernels (a caller tensor other than the
one used in place before, or a changed mask width), since the graph would go
on reading the old one.  A re-plan of another shape allocates new buffers,
and a graph captured earlier keeps (and keeps using) its own.  With
dynamic_prefix=True, prefix_len is each request's largest prefix and the
kernels read the current lengths from `prefix_len_dev` (int32, on the
device), so one captured step replays while the cache grows.
"""
from __future__ import annotations

import ctypes as C
from typing import Optional, Sequence, Tuple, Union

import numpy as np
import torch

from . import _lib
from ._lib import check, lib
from .graph import capturing, keep_alive
from .tree import pack_tree_masks

_MASK_MODES = {"none": _lib.D2SD_MASK_NONE, "causal": _lib.D2SD_MASK_CAUSAL, "tree": _lib.D2SD_MASK_TREE}


def _i32(x) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(x, dtype=np.int32))


def _reuse(old: Optional[torch.Tensor], new: torch.Tensor, same_shape: bool) -> torch.Tensor:
    """`new` copied into `old` when the plan keeps its shape (old buffer large
    enough, same dtype), else `new` itself."""
    if (same_shape and old is not None and old.dtype == new.dtype and old.device == new.device
            and old.numel() >= new.numel()):
        old.view(-1)[:new.numel()].copy_(new.view(-1))
        return old
    return new


class CascadeVerifyAttention:
    def __init__(self, device: Union[str, torch.device, None] = None):
        dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        if dev.type == "cuda" and dev.index is None:  # "cuda" names the current device: compare by index
            dev = torch.device("cuda", torch.cuda.current_device())
        self.device = dev
        self._planned = False
        self._captured = False   # a run() was recorded into a graph
        self._owned = set()      # names of the optional-input buffers the plan owns

    def _in_place(self, t: torch.Tensor, dtype: torch.dtype) -> bool:
        return t.device == self.device and t.dtype == dtype and t.is_contiguous()

    def _keeps(self, name: str, src, dtype: torch.dtype) -> bool:
        """Whether _input_buffer(name, src, ...) of a same-shape re-plan
        returns the buffer the kernels read now."""
        old = getattr(self, name, None)
        if src is None or old is None:
            return src is None and old is None
        t = src if isinstance(src, torch.Tensor) else None
        if t is not None and self._in_place(t, dtype):
            return name not in self._owned and t.data_ptr() == old.data_ptr() and t.numel() == old.numel()
        n = t.numel() if t is not None else int(np.asarray(src).size)
        return name in self._owned and old.numel() == n

    def _input_buffer(self, name: str, src, dtype: torch.dtype, same: bool) -> Optional[torch.Tensor]:
        """Device buffer for an optional input (page table, sinks, scales):
        a contiguous device tensor of `dtype` is used in place; anything else
        goes into a plan-owned buffer, rewritten in place by a same-shape
        re-plan when the sizes agree."""
        old = getattr(self, name, None)
        if src is None:
            self._owned.discard(name)
            return None
        t = src if isinstance(src, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(np.asarray(src)))
        if self._in_place(t, dtype):
            self._owned.discard(name)
            return t
        if same and name in self._owned and old is not None and old.numel() == t.numel():
            old.copy_(t.reshape(-1).to(dtype))
            return old
        self._owned.add(name)
        return t.to(device=self.device, dtype=dtype).reshape(-1).contiguous().clone()

    # ------------------------------------------------------------------ plan
    def plan(
        self,
        qo_indptr: Sequence[int],
        prefix_len: Sequence[int],
        num_qo_heads: int,
        num_kv_heads: int,
        head_dim: int,
        *,
        tree_masks: Optional[Sequence[np.ndarray]] = None,
        mask_mode: str = "tree",
        page_size: int = 0,
        page_indptr: Optional[Sequence[int]] = None,
        page_table: Optional[Union[Sequence[int], torch.Tensor]] = None,
        prefix_tok_indptr: Optional[Sequence[int]] = None,
        kv_layout: str = "HND",
        sm_scale: Optional[float] = None,
        window_left: int = -1,
        sinks: Optional[torch.Tensor] = None,
        kv_dtype: torch.dtype = torch.bfloat16,
        k_scale: Optional[torch.Tensor] = None,
        v_scale: Optional[torch.Tensor] = None,
        lse_base2: bool = False,
        max_splits: int = 0,
        waves_per_block: int = 0,
        num_cus: int = 0,
        dynamic_prefix: bool = False,
        prefix_split: Optional[Sequence[int]] = None,
        prefix2_tok_indptr: Optional[Sequence[int]] = None,
    ) -> "CascadeVerifyAttention":
        """Plan one verify call.

        qo_indptr [R+1]: tree nodes of request r are rows qo_indptr[r]:qo_indptr[r+1]
        of q / k_suffix / v_suffix / out / lse.  prefix_len [R]: shared-prefix keys.
        tree_masks: per request a bool [n_r, n_r] ancestor mask (M[i, j] = node j
        is i or an ancestor of i) when mask_mode == "tree".
        Prefix KV at run(): paged (page_size > 0) pool of shape
        [pages, Hkv, P, D] (kv_layout "HND") or [pages, P, Hkv, D] ("NHD") with
        request r's pages page_table[page_indptr[r]:page_indptr[r+1]]; or
        contiguous [Hkv, L, D] ("HND", the DynamicCache layout) / [L, Hkv, D]
        ("NHD"), request r at token offset prefix_tok_indptr[r] (default 0).
        window_left >= 0 keeps the last window_left prefix keys for all queries
        (verification.py:133-135).  sinks [Hq] fp32 applies O *= sigmoid(lse - sink).
        kv_dtype torch.float8_e4m3fn takes per-kv-head fp32 k_scale / v_scale.
        dynamic_prefix: prefix_len is each request's largest prefix; run() uses
        the current lengths in self.prefix_len_dev (set_prefix_len(), or any
        device write, e.g. PagedKVCommit's advance), each clamped to
        [0, planned length].
        prefix_split [R]: a two-segment contiguous prefix (static plans): keys
        [0, prefix_split[r]) of request r come from the first prefix tensor,
        keys [prefix_split[r], prefix_len[r]) from the second, at token
        prefix2_tok_indptr[r] (default 0) of it; run() then takes
        k_prefix = (k_first, k_second) and v_prefix likewise, both in
        kv_layout.  This is the DTA draft's shared level [draft cache |
        projected target context] (model/dflash.py:103-106) without the
        concatenation.
        """
        qo = _i32(qo_indptr)
        pl = _i32(prefix_len)
        R = int(pl.shape[0])
        if qo.shape[0] != R + 1:
            raise ValueError("qo_indptr must have len(prefix_len) + 1 entries")
        if mask_mode not in _MASK_MODES:
            raise ValueError(f"mask_mode must be one of {sorted(_MASK_MODES)}")
        if kv_layout not in ("HND", "NHD"):
            raise ValueError("kv_layout must be 'HND' or 'NHD'")
        if kv_dtype not in (torch.bfloat16, torch.float8_e4m3fn):
            raise TypeError("kv_dtype must be torch.bfloat16 or torch.float8_e4m3fn")
        fp8 = kv_dtype == torch.float8_e4m3fn
        dev = self.device
        pi = None
        if int(page_size) > 0:
            if page_indptr is None or page_table is None:
                raise ValueError("paged prefix needs page_indptr and page_table")
            pi = _i32(page_indptr)
            if pi.shape[0] != R + 1:
                raise ValueError("page_indptr must have R + 1 entries")
        pti = _i32(prefix_tok_indptr) if (prefix_tok_indptr is not None and int(page_size) == 0) else None
        if pti is not None and pti.shape[0] != R:
            raise ValueError("prefix_tok_indptr must have R entries")
        psplit = _i32(prefix_split) if prefix_split is not None else None
        pti2 = _i32(prefix2_tok_indptr) if (prefix2_tok_indptr is not None and psplit is not None) else None
        if psplit is not None:
            if psplit.shape[0] != R or (pti2 is not None and pti2.shape[0] != R):
                raise ValueError("prefix_split and prefix2_tok_indptr must have R entries")
            if int(page_size) > 0 or dynamic_prefix:
                raise ValueError("a two-segment prefix needs a contiguous prefix and a static plan")
        desc = _lib.PlanDesc()
        desc.num_reqs = R
        desc.qo_indptr = qo.ctypes.data_as(C.POINTER(C.c_int32))
        desc.prefix_len = pl.ctypes.data_as(C.POINTER(C.c_int32))
        desc.page_indptr = pi.ctypes.data_as(C.POINTER(C.c_int32)) if pi is not None else None
        desc.prefix_tok_indptr = pti.ctypes.data_as(C.POINTER(C.c_int32)) if pti is not None else None
        desc.num_qo_heads = num_qo_heads
        desc.num_kv_heads = num_kv_heads
        desc.head_dim = head_dim
        desc.window_left = window_left
        desc.kv_dtype = _lib.D2SD_KV_FP8_E4M3 if fp8 else _lib.D2SD_KV_BF16
        desc.page_size = int(page_size)
        desc.num_cus = num_cus
        desc.max_splits = max_splits
        desc.waves_per_block = waves_per_block
        desc.dynamic_prefix = int(bool(dynamic_prefix))
        desc.prefix_split = psplit.ctypes.data_as(C.POINTER(C.c_int32)) if psplit is not None else None
        desc.prefix2_tok_indptr = pti2.ctypes.data_as(C.POINTER(C.c_int32)) if pti2 is not None else None
        info = _lib.PlanInfo()
        # One planner pass into a host buffer kept across plans (16K entries at
        # first); a plan that needs more is planned again into a larger one.
        buf = getattr(self, "_plan_host_buf", None)
        if buf is None:
            buf = np.zeros(1 << 14, dtype=np.int32)
        rc = lib.d2sd_cascade_plan(C.byref(desc), buf.ctypes.data_as(C.POINTER(C.c_int32)), buf.size,
                                   C.byref(info))
        if rc == _lib.D2SD_ERR_WORKSPACE and info.plan_ints > buf.size:
            buf = np.zeros(info.plan_ints, dtype=np.int32)
            rc = lib.d2sd_cascade_plan(C.byref(desc), buf.ctypes.data_as(C.POINTER(C.c_int32)), buf.size,
                                       C.byref(info))
        check(rc, "cascade_plan")
        self._plan_host_buf = buf
        host = buf[:max(info.plan_ints, 8)].copy()

        # ---- inputs, checked before any buffer is touched ----
        mode = _MASK_MODES[mask_mode]
        packed = None
        if mode == _lib.D2SD_MASK_TREE:
            if tree_masks is None or len(tree_masks) != R:
                raise ValueError("mask_mode 'tree' needs one ancestor mask per request")
            for r, m in enumerate(tree_masks):
                n = int(qo[r + 1] - qo[r])
                if m.shape != (n, n):
                    raise ValueError(f"tree_masks[{r}] must be [{n}, {n}], got {m.shape}")
            packed = pack_tree_masks([np.asarray(m, dtype=bool) for m in tree_masks])
        pt = None
        if int(page_size) > 0:
            pt = (page_table if isinstance(page_table, torch.Tensor) else torch.from_numpy(_i32(page_table))).reshape(-1)
            if pt.numel() < int(pi[-1]):
                raise ValueError("page_table shorter than page_indptr[-1]")
        if sinks is not None and sinks.numel() != num_qo_heads:
            raise ValueError("sinks must have num_qo_heads entries")
        k2_scale = v2_scale = None
        if fp8:
            # the scales dequantise prefix keys / values; a plan without any
            # prefix key needs none (as d2sd_cascade_run).  A two-segment
            # prefix takes one scale pair for both segments or a (first,
            # second) pair of each.
            if isinstance(k_scale, (tuple, list)):
                k_scale, k2_scale = k_scale
            if isinstance(v_scale, (tuple, list)):
                v_scale, v2_scale = v_scale
            if info.two_segment:
                k2_scale = k_scale if k2_scale is None else k2_scale
                v2_scale = v_scale if v2_scale is None else v2_scale
            if any(int(x) > 0 for x in prefix_len) and (k_scale is None or v_scale is None):
                raise ValueError("fp8 KV needs k_scale and v_scale")
        else:
            k_scale = v_scale = None
        if not info.two_segment:
            k2_scale = v2_scale = None

        old = getattr(self, "info", None) if self._planned else None
        same = old is not None and all(
            getattr(old, f) == getattr(info, f) for f in
            ("num_items", "num_merges", "waves_per_block", "rows_per_tile", "num_slots", "num_reqs",
             "num_qo_heads", "num_kv_heads", "head_dim", "kv_dtype", "page_size", "dynamic_prefix", "two_segment",
             "fused"))
        mask_words = int(packed.shape[1]) if packed is not None else 0
        same_mask = same and packed is not None and getattr(self, "tree_mask_dev", None) is not None \
            and self.mask_words == mask_words and self.tree_mask_dev.numel() >= packed.size
        if same and self._captured:
            # a graph captured earlier reads these buffers: refuse a re-plan
            # that would give the kernels others
            changed = [n for n, src, dt in (("page_table_dev", pt, torch.int32), ("sinks", sinks, torch.float32),
                                            ("k_scale", k_scale, torch.float32), ("v_scale", v_scale, torch.float32),
                                            ("k2_scale", k2_scale, torch.float32),
                                            ("v2_scale", v2_scale, torch.float32))
                       if not self._keeps(n, src, dt)]
            if (packed is not None) != (getattr(self, "tree_mask_dev", None) is not None) or \
                    (packed is not None and not same_mask):
                changed.append("tree_mask_dev")
            if changed:
                raise RuntimeError(
                    "CascadeVerifyAttention.plan: a graph captured earlier reads this plan's buffers, and this "
                    f"re-plan would hand other ones to the kernels ({', '.join(changed)}); pass the same device "
                    "tensors (or host data), or plan a new CascadeVerifyAttention and capture again")

        # ---- device buffers ----
        self.info = info
        self.info_bytes = torch.frombuffer(bytearray(bytes(info)), dtype=torch.uint8)
        self.plan_host = host
        self.qo_indptr_host = qo
        self.prefix_len_host = pl
        self.plan_dev = _reuse(getattr(self, "plan_dev", None), torch.from_numpy(host).to(dev), same)
        ws = int(max(int(info.workspace_bytes), 16))
        self.workspace = (self.workspace if same and getattr(self, "workspace", None) is not None
                          and self.workspace.numel() >= ws else torch.empty(ws, dtype=torch.uint8, device=dev))
        self.prefix_len_dev = _reuse(getattr(self, "prefix_len_dev", None), torch.from_numpy(pl.copy()).to(dev), same)
        self.mask_mode = mode
        self.total_q = int(qo[-1])
        self.mask_words = mask_words
        if packed is not None:
            self.tree_mask_dev = _reuse(getattr(self, "tree_mask_dev", None),
                                        torch.from_numpy(packed.view(np.int64)).to(dev), same_mask)
        else:
            self.tree_mask_dev = None
        self.page_size = int(page_size)
        self.page_table_dev = self._input_buffer("page_table_dev", pt, torch.int32, same)
        if pt is not None:
            ids = pt[:int(pi[-1])].to("cpu", torch.int64)
            self._page_id_range = (int(ids.min()), int(ids.max())) if ids.numel() else (0, -1)
        self.kv_layout = kv_layout
        self.num_qo_heads, self.num_kv_heads, self.head_dim = num_qo_heads, num_kv_heads, head_dim
        self.sm_scale = float(sm_scale) if sm_scale is not None else head_dim ** -0.5
        self.window_left = window_left
        self.sinks = self._input_buffer("sinks", sinks, torch.float32, same)
        self.kv_dtype = kv_dtype
        self.k_scale = self._input_buffer("k_scale", k_scale, torch.float32, same)
        self.v_scale = self._input_buffer("v_scale", v_scale, torch.float32, same)
        self.k2_scale = self._input_buffer("k2_scale", k2_scale, torch.float32, same)
        self.v2_scale = self._input_buffer("v2_scale", v2_scale, torch.float32, same)
        self.lse_base2 = bool(lse_base2)
        self._planned = True
        return self

    def set_prefix_len(self, prefix_len: Sequence[int]) -> None:
        """Current prefix lengths of a dynamic_prefix plan (host write into
        prefix_len_dev; each is clamped to the planned length by the kernels)."""
        v = torch.from_numpy(_i32(prefix_len))
        if v.numel() != self.prefix_len_dev.numel():
            raise ValueError("one prefix length per request")
        self.prefix_len_dev.copy_(v)

    # ------------------------------------------------------------------- run
    def _prefix_strides(self, k_prefix: torch.Tensor, second: bool = False) -> Tuple[int, int, int, int]:
        """(stride_tok, stride_head, stride_page, extent) in elements; extent =
        pages of a paged pool or tokens of a contiguous prefix (second: the
        second segment of a two-segment prefix)."""
        if self.page_size > 0 and not second:
            if k_prefix.dim() != 4:
                raise ValueError("paged prefix pool must be 4-D")
            if self.kv_layout == "HND":   # [pages, Hkv, P, D]
                _, hkv, P, D = k_prefix.shape
                st, sh, sp = k_prefix.stride(2), k_prefix.stride(1), k_prefix.stride(0)
            else:                         # [pages, P, Hkv, D]
                _, P, hkv, D = k_prefix.shape
                st, sh, sp = k_prefix.stride(1), k_prefix.stride(2), k_prefix.stride(0)
            if P != self.page_size:
                raise ValueError(f"pool page size {P} != planned {self.page_size}")
            extent = k_prefix.shape[0]
            lo, hi = self._page_id_range
            if lo < 0 or hi >= extent:
                raise ValueError(f"page_table holds page ids outside the pool's {extent} pages")
        else:
            if k_prefix.dim() == 4 and k_prefix.shape[0] == 1:
                k_prefix = k_prefix[0]   # DynamicCache [1, Hkv, L, D]
            if k_prefix.dim() != 3:
                raise ValueError("contiguous prefix must be [Hkv, L, D] (HND) or [L, Hkv, D] (NHD)")
            if self.kv_layout == "HND":
                hkv, extent, D = k_prefix.shape
                st, sh, sp = k_prefix.stride(1), k_prefix.stride(0), 0
            else:
                extent, hkv, D = k_prefix.shape
                st, sh, sp = k_prefix.stride(0), k_prefix.stride(1), 0
            need = int(self.info.prefix2_extent if second else self.info.prefix_extent)
            if extent < need:
                raise ValueError(f"k_prefix{' (second segment)' if second else ''} holds {extent} tokens; "
                                 f"the plan reads {need}")
        if hkv != self.num_kv_heads or D != self.head_dim or k_prefix.stride(-1) != 1:
            raise ValueError("prefix KV head count / head_dim / contiguity mismatch")
        return st, sh, sp, extent

    def run(
        self,
        q: torch.Tensor,
        k_suffix: torch.Tensor,
        v_suffix: torch.Tensor,
        k_prefix: Optional[torch.Tensor] = None,
        v_prefix: Optional[torch.Tensor] = None,
        out: Optional[torch.Tensor] = None,
        lse: Optional[torch.Tensor] = None,
    ) -> Tuple[torch.Tensor, torch.Tensor]:
        """q [total_q, Hq, D], k/v_suffix [total_q, Hkv, D] (bf16); prefix KV as
        planned.  Returns (out [total_q, Hq, D] bf16, lse [total_q, Hq] fp32)."""
        return self._launch("cascade_run", q, k_suffix, v_suffix, k_prefix, v_prefix, out, lse)

    def run_no_alloc(self, q, k_suffix, v_suffix, k_prefix=None, v_prefix=None, out=None, lse=None):
        """run() on the library's own per-GPU workspace
        (d2sd_cascade_run_noalloc; at most d2sd_cascade_scratch_bytes() of
        partial states): for callers that cannot allocate.  Calls on one GPU
        share that workspace, so overlapping calls (other streams) race."""
        return self._launch("cascade_run_no_alloc", q, k_suffix, v_suffix, k_prefix, v_prefix, out, lse,
                            workspace=False)

    def run_attention(self, q, k_suffix, v_suffix, k_prefix=None, v_prefix=None, out=None, lse=None):
        """First half of run(): the attention launch alone (prefix key chunks
        and suffix trees; partial states in the plan's workspace).
        run_merge() with the same arguments finishes the call."""
        return self._launch("d2sd_cascade_attention", q, k_suffix, v_suffix, k_prefix, v_prefix, out, lse)

    def run_merge(self, q, k_suffix, v_suffix, k_prefix=None, v_prefix=None, out=None, lse=None):
        """Second half of run(): merge of the workspace partials + sink into
        out / lse."""
        return self._launch("d2sd_cascade_merge", q, k_suffix, v_suffix, k_prefix, v_prefix, out, lse)

    def _launch(self, fn_name, q, k_suffix, v_suffix, k_prefix, v_prefix, out, lse, workspace=True):
        if not self._planned:
            raise RuntimeError("run() before plan()")
        T, hq, d = self.total_q, self.num_qo_heads, self.head_dim
        for name, t, h in (("q", q, hq), ("k_suffix", k_suffix, self.num_kv_heads),
                           ("v_suffix", v_suffix, self.num_kv_heads)):
            if t.shape != (T, h, d) or t.dtype != torch.bfloat16 or t.stride(-1) != 1 or not t.is_cuda:
                raise ValueError(f"{name} must be a bf16 device tensor [{T}, {h}, {d}] with contiguous head_dim")
        if k_suffix.stride() != v_suffix.stride():
            raise ValueError("k_suffix and v_suffix must share strides")
        if out is None:
            out = torch.empty((T, hq, d), dtype=torch.bfloat16, device=q.device)
        if lse is None:
            lse = torch.empty((T, hq), dtype=torch.float32, device=q.device)
        if out.shape != (T, hq, d) or out.dtype != torch.bfloat16 or out.stride(-1) != 1:
            raise ValueError("out must be bf16 [total_q, Hq, D] with contiguous head_dim")
        if lse.shape != (T, hq) or lse.dtype != torch.float32 or lse.stride(-1) != 1:
            raise ValueError("lse must be float32 [total_q, Hq] with contiguous heads")
        if capturing():
            self._captured = True
        a = _lib.RunArgs()
        a.plan = self.plan_dev.data_ptr()
        a.q = q.data_ptr()
        a.q_stride_n, a.q_stride_h = q.stride(0), q.stride(1)
        a.k_suffix, a.v_suffix = k_suffix.data_ptr(), v_suffix.data_ptr()
        a.suffix_stride_n, a.suffix_stride_h = k_suffix.stride(0), k_suffix.stride(1)
        a.mask_mode = self.mask_mode
        a.mask_words = self.mask_words
        a.tree_mask = self.tree_mask_dev.data_ptr() if self.tree_mask_dev is not None else None
        k_prefix2 = v_prefix2 = None
        prefix2 = []
        if isinstance(k_prefix, (tuple, list)) or isinstance(v_prefix, (tuple, list)):
            if not (isinstance(k_prefix, (tuple, list)) and isinstance(v_prefix, (tuple, list))
                    and len(k_prefix) == 2 and len(v_prefix) == 2):
                raise ValueError("a two-segment prefix takes k_prefix = (first, second) and v_prefix likewise")
            if not self.info.two_segment:
                raise ValueError("this plan has a one-segment prefix (plan(prefix_split=...) makes two)")
            (k_prefix, k_prefix2), (v_prefix, v_prefix2) = k_prefix, v_prefix
            if k_prefix2 is None or v_prefix2 is None:
                raise ValueError("the plan reads the second prefix segment; it is None")
            if v_prefix2.shape != k_prefix2.shape or v_prefix2.stride() != k_prefix2.stride():
                raise ValueError("v_prefix's second segment must match k_prefix's in shape and strides")
            if k_prefix2.dtype != self.kv_dtype or v_prefix2.dtype != self.kv_dtype or not k_prefix2.is_cuda:
                raise TypeError(f"prefix KV must be {self.kv_dtype} device tensors")
            st2, sh2, _, extent2 = self._prefix_strides(k_prefix2, second=True)
            a.k_prefix2, a.v_prefix2 = k_prefix2.data_ptr(), v_prefix2.data_ptr()
            a.prefix2_stride_tok, a.prefix2_stride_head, a.prefix2_extent = st2, sh2, extent2
            a.k2_scale = self.k2_scale.data_ptr() if self.k2_scale is not None else None
            a.v2_scale = self.v2_scale.data_ptr() if self.v2_scale is not None else None
            prefix2 = [st2, sh2, extent2]
        elif self.info.two_segment:
            raise ValueError("the plan has a two-segment prefix: pass k_prefix = (first, second) and v_prefix likewise")
        if k_prefix is not None:
            if v_prefix is None or v_prefix.shape != k_prefix.shape or v_prefix.stride() != k_prefix.stride():
                raise ValueError("v_prefix must match k_prefix in shape and strides")
            if k_prefix.dtype != self.kv_dtype or v_prefix.dtype != self.kv_dtype:
                raise TypeError(f"prefix KV must be {self.kv_dtype}")
            st, sh, sp, extent = self._prefix_strides(k_prefix)
            a.k_prefix, a.v_prefix = k_prefix.data_ptr(), v_prefix.data_ptr()
            a.prefix_stride_tok, a.prefix_stride_head, a.prefix_stride_page = st, sh, sp
            a.prefix_extent = extent
        a.page_size = self.page_size
        a.page_table = self.page_table_dev.data_ptr() if self.page_table_dev is not None else None
        a.prefix_len = self.prefix_len_dev.data_ptr()
        a.k_scale = self.k_scale.data_ptr() if self.k_scale is not None else None
        a.v_scale = self.v_scale.data_ptr() if self.v_scale is not None else None
        a.sinks = self.sinks.data_ptr() if self.sinks is not None else None
        a.out = out.data_ptr()
        a.o_stride_n, a.o_stride_h = out.stride(0), out.stride(1)
        a.lse = lse.data_ptr()
        a.lse_stride_n = lse.stride(0)
        a.sm_scale = self.sm_scale
        a.lse_base2 = int(self.lse_base2)
        a.workspace = self.workspace.data_ptr() if workspace else None
        a.workspace_bytes = self.workspace.numel() if workspace else 0
        if fn_name.startswith("cascade_run"):
            # the whole call: through the torch operator (torch.ops.d2sd.cascade_run*)
            getattr(torch.ops.d2sd, fn_name)(
                self.info_bytes, self.plan_dev, self.workspace, q, k_suffix, v_suffix, k_prefix, v_prefix,
                [a.prefix_stride_tok, a.prefix_stride_head, a.prefix_stride_page, a.prefix_extent],
                self.page_table_dev, self.tree_mask_dev, self.mask_mode, self.mask_words, self.prefix_len_dev,
                self.k_scale, self.v_scale, self.sinks, self.sm_scale, self.lse_base2, out, lse,
                k_prefix2, v_prefix2, prefix2, self.k2_scale, self.v2_scale)
        else:
            fn = getattr(lib, fn_name)
            check(fn(C.byref(self.info), C.byref(a), C.c_void_p(torch.cuda.current_stream().cuda_stream)),
                  fn_name)
        keep_alive(self.plan_dev, self.workspace if workspace else None, self.tree_mask_dev, self.page_table_dev, self.prefix_len_dev,
                   self.sinks, self.k_scale, self.v_scale, self.k2_scale, self.v2_scale, q, k_suffix, v_suffix,
                   k_prefix, v_prefix, k_prefix2, v_prefix2, out, lse)
        return out, lse
