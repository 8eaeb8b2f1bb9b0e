"""Accepted-branch KV commit into the paged prefix cache (libd2sd.so).

Replaces the cache growth of generation/d3_generator.py:227-232, which per
layer and step does

    k_win = new_kv[layer][0][valid_block:valid_block + 1, :, :acceptance_length, :]
    layer.keys = torch.cat([layer.keys, k_win], dim=2)      (values alike)

i.e. copies the whole cache.  Here the accepted branch's tokens (their tree
node rows of each layer's suffix K/V, in order) are written in place into the
pages that follow the prefix, for all layers in one launch; the prefix stays
put, so page tables and hipGraphs stay valid across steps.

Pools may also hold fp8 (torch.float8_e4m3fn) with per-layer, per-kv-head
fp32 scales (the cascade kernels' fp8 format, value / scale): the new bf16
rows are quantised on the way in, as clamp(x / scale, -448, 448) cast to
e4m3fn with round-to-nearest-even.
"""
from __future__ import annotations

import ctypes as C
from typing import Sequence

import torch

from . import _lib
from ._lib import check, lib
from .graph import keep_alive


def _layout_strides(pool: torch.Tensor, kv_layout: str):
    # [pages, Hkv, P, D] ("HND") or [pages, P, Hkv, D] ("NHD"), head_dim contiguous
    if kv_layout == "HND":
        return pool.stride(0), pool.stride(1), pool.stride(2), pool.shape[2], pool.shape[1]
    if kv_layout == "NHD":
        return pool.stride(0), pool.stride(2), pool.stride(1), pool.shape[1], pool.shape[2]
    raise ValueError("kv_layout must be 'HND' or 'NHD'")


class PagedKVCommit:
    """Commits accepted tree nodes of every layer into paged K/V pools.

    k_pools / v_pools: per layer a bf16 or float8_e4m3fn page pool
    ([pages, Hkv, P, D] for kv_layout "HND", [pages, P, Hkv, D] for "NHD");
    k_new / v_new: per layer the step's suffix K/V, bf16 [rows, Hkv, D] (the
    tree nodes, as passed to CascadeVerifyAttention.run).  fp8 pools need
    k_scales / v_scales: per layer fp32 [Hkv] (or one tensor for every layer).
    All layers share shapes and strides.  The
    per-layer addresses are kept in device arrays built here once, so that
    commit() allocates nothing and may be captured into a hipGraph (the
    tensors must stay alive and in place).
    """

    def __init__(self, k_pools: Sequence[torch.Tensor], v_pools: Sequence[torch.Tensor],
                 k_new: Sequence[torch.Tensor], v_new: Sequence[torch.Tensor], kv_layout: str = "HND",
                 k_scales=None, v_scales=None):
        n = len(k_pools)
        if not (n == len(v_pools) == len(k_new) == len(v_new)) or n == 0:
            raise ValueError("one k/v pool and one k/v new tensor per layer are required")
        ref_pool, ref_new = k_pools[0], k_new[0]
        if ref_pool.dtype not in (torch.bfloat16, torch.float8_e4m3fn):
            raise TypeError("pools must be bf16 or float8_e4m3fn")
        for t in list(k_pools) + list(v_pools):
            if t.dtype != ref_pool.dtype or t.shape != ref_pool.shape or t.stride() != ref_pool.stride():
                raise ValueError("pools must share one dtype, shape and stride for all layers")
            if t.stride(-1) != 1 or t.device != ref_pool.device:
                raise ValueError("pools must have a contiguous head_dim on one device")
        for t in list(k_new) + list(v_new):
            if t.dtype != torch.bfloat16 or t.shape != ref_new.shape or t.stride() != ref_new.stride():
                raise ValueError("k_new / v_new must be bf16 with one shape and stride for all layers")
            if t.dim() != 3 or t.stride(-1) != 1 or t.device != ref_pool.device:
                raise ValueError("k_new / v_new must be [rows, Hkv, D] with a contiguous head_dim")
        sp, sh, st, page_size, hkv = _layout_strides(ref_pool, kv_layout)
        if ref_new.shape[1] != hkv or ref_new.shape[2] != ref_pool.shape[-1]:
            raise ValueError("k_new / v_new heads and head_dim must match the pools")
        dev = ref_pool.device
        as_addr = lambda ts: torch.tensor([t.data_ptr() for t in ts], dtype=torch.int64, device=dev)
        self._addr = [as_addr(k_new), as_addr(v_new), as_addr(k_pools), as_addr(v_pools)]
        self._keep = (list(k_pools), list(v_pools), list(k_new), list(v_new))
        fp8 = ref_pool.dtype == torch.float8_e4m3fn
        if fp8:
            if k_scales is None or v_scales is None:
                raise ValueError("float8_e4m3fn pools need k_scales and v_scales")

            def per_layer(s):
                ts = [s] * n if isinstance(s, torch.Tensor) else list(s)
                if len(ts) != n:
                    raise ValueError("one scale tensor per layer (or one for all layers)")
                for x in ts:
                    if x.dtype != torch.float32 or x.numel() != hkv or not x.is_contiguous() or x.device != dev:
                        raise ValueError("scales must be contiguous fp32 [Hkv] tensors on the pools' device")
                return ts
            ks, vs = per_layer(k_scales), per_layer(v_scales)
            self._addr += [as_addr(ks), as_addr(vs)]
            self._keep += (ks, vs)
        elif k_scales is not None or v_scales is not None:
            raise ValueError("scales apply to float8_e4m3fn pools only")
        a = _lib.KvAppendArgs()
        a.num_layers = n
        a.num_kv_heads = hkv
        a.head_dim = ref_pool.shape[-1]
        a.page_size = page_size
        a.num_rows = ref_new.shape[0]
        a.pool_pages = ref_pool.shape[0]
        a.k_new, a.v_new, a.k_pool, a.v_pool = (t.data_ptr() for t in self._addr[:4])
        a.new_stride_n, a.new_stride_h = ref_new.stride(0), ref_new.stride(1)
        a.pool_stride_page, a.pool_stride_head, a.pool_stride_tok = sp, sh, st
        if fp8:
            a.pool_dtype = _lib.D2SD_KV_FP8_E4M3
            a.k_scale, a.v_scale = self._addr[4].data_ptr(), self._addr[5].data_ptr()
        self._args = a
        self.page_size = page_size

    def commit(self, page_table: torch.Tensor, prefix_len, node_ids: torch.Tensor,
               num_accepted: int | None = None, num_accepted_dev: torch.Tensor | None = None,
               advance: bool = False) -> None:
        """Writes rows node_ids[:num_accepted] of every layer's k_new / v_new to
        cache positions prefix_len .. prefix_len + num_accepted - 1 of the
        request whose pages are page_table (device int32, covering them).
        num_accepted_dev (device int32, e.g. GreedyAccept's result) makes the
        kernel read the count from the device, capped at num_accepted.
        prefix_len may be a device int32 tensor of one element (e.g. a slice
        of CascadeVerifyAttention.prefix_len_dev): the kernel then reads the
        length there, and advance=True adds the accepted count to it after the
        commit, so that a captured step replays as the cache grows."""
        if page_table.dtype != torch.int32 or node_ids.dtype != torch.int32:
            raise TypeError("page_table and node_ids must be int32")
        if not (page_table.is_contiguous() and node_ids.is_contiguous()):
            raise ValueError("page_table and node_ids must be contiguous")
        n = int(node_ids.numel() if num_accepted is None else num_accepted)
        if n < 0 or n > node_ids.numel():
            raise ValueError("num_accepted out of range")
        dev_len = isinstance(prefix_len, torch.Tensor)
        if dev_len:
            if (prefix_len.dtype != torch.int32 or prefix_len.numel() != 1 or not prefix_len.is_cuda
                    or not prefix_len.is_contiguous()):
                raise TypeError("a device prefix_len must be one contiguous int32 element")
        else:
            if advance:
                raise ValueError("advance needs a device prefix_len")
            if (int(prefix_len) + n + self.page_size - 1) // self.page_size > page_table.numel():
                raise ValueError("page_table does not cover prefix_len + num_accepted tokens")
        a = self._args
        a.prefix_len = 0 if dev_len else int(prefix_len)
        a.prefix_len_dev = prefix_len.data_ptr() if dev_len else None
        a.advance_prefix = int(bool(advance))
        a.num_accepted = n
        a.node_ids = node_ids.data_ptr()
        a.page_table = page_table.data_ptr()
        a.page_table_len = page_table.numel()
        if num_accepted_dev is not None:
            if num_accepted_dev.dtype != torch.int32 or num_accepted_dev.device != page_table.device:
                raise TypeError("num_accepted_dev must be a device int32 tensor")
            a.num_accepted_dev = num_accepted_dev.data_ptr()
        else:
            a.num_accepted_dev = None
        check(lib.d2sd_paged_kv_append(C.byref(a), C.c_void_p(torch.cuda.current_stream().cuda_stream)),
              "paged_kv_append")
        keep_alive(page_table, node_ids, num_accepted_dev, prefix_len if dev_len else None, *self._addr)
