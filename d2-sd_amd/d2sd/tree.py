"""Candidate-token trees for cascade verification.

The reference verifies `bsz` candidate rows of `Lb` tokens, row j sharing its
first s_j tokens with row 0 (generation/d3_generator.py:127-180), by per-row
causal attention (generation/verification.py:155-162).  Those rows are the
root-to-leaf paths of a token tree; here the tree is stored once, as unique
nodes, with
  * parents[i]  : parent node of node i (-1 for a root), parents[i] < i,
  * node_index  : [bsz, Lb] node of (row, position) — the gather/scatter map
                  between the reference's row layout and the node layout,
  * an ancestor mask M[i, j] = (j is i or an ancestor of i), packed as
    little-endian uint64 words per row for the kernels.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import List, Optional, Sequence

import numpy as np
import torch


@dataclass
class TokenTree:
    parents: np.ndarray      # int32 [n]
    node_index: np.ndarray   # int32 [bsz, Lb]
    shared: List[int]        # tokens row j shares with row 0 (row 0: Lb)

    @property
    def num_nodes(self) -> int:
        return int(self.parents.shape[0])

    @property
    def num_rows(self) -> int:
        return int(self.node_index.shape[0])

    @property
    def row_len(self) -> int:
        return int(self.node_index.shape[1])

    def ancestor_mask(self) -> np.ndarray:
        return ancestor_mask(self.parents)


def tree_from_shared_prefixes(row_len: int, shared: Sequence[int]) -> TokenTree:
    """Rows of `row_len` tokens; row j shares its first shared[j] tokens with
    row 0 (shared[0] is ignored).  Unshared tokens are new nodes, numbered in
    row-major order of first appearance, so parents[i] < i."""
    bsz = len(shared)
    node_index = np.zeros((bsz, row_len), dtype=np.int32)
    parents: List[int] = []
    for p in range(row_len):
        node_index[0, p] = p
        parents.append(p - 1)
    shared_out = [row_len]
    for j in range(1, bsz):
        s = int(shared[j])
        if not 0 <= s <= row_len:
            raise ValueError(f"shared[{j}]={s} outside [0, {row_len}]")
        shared_out.append(s)
        for p in range(row_len):
            if p < s:
                node_index[j, p] = node_index[0, p]
            else:
                node_index[j, p] = len(parents)
                parents.append(int(node_index[j, p - 1]) if p > 0 else -1)
    return TokenTree(np.asarray(parents, dtype=np.int32), node_index, shared_out)


def ancestor_mask(parents: np.ndarray) -> np.ndarray:
    """bool [n, n]: M[i, j] = j is i or an ancestor of i."""
    n = int(len(parents))
    m = np.zeros((n, n), dtype=bool)
    for i in range(n):
        par = int(parents[i])
        if par >= i:
            raise ValueError("parents must satisfy parents[i] < i")
        if par >= 0:
            m[i] = m[par]
        m[i, i] = True
    return m


def pack_mask_rows(mask: np.ndarray, words: Optional[int] = None) -> np.ndarray:
    """bool [rows, n] -> uint64 [rows, words]; bit j % 64 of word j // 64."""
    rows, n = mask.shape
    words = words if words is not None else max(1, (n + 63) // 64)
    if words * 64 < n:
        raise ValueError("too few words for the mask width")
    padded = np.zeros((rows, words * 64), dtype=np.uint8)
    padded[:, :n] = mask
    bits = np.packbits(padded.reshape(rows, words, 64), axis=-1, bitorder="little")  # [rows, words, 8]
    return bits.view("<u8").reshape(rows, words).astype(np.uint64)


def pack_tree_masks(masks: Sequence[np.ndarray]) -> np.ndarray:
    """Per-request ancestor masks -> one uint64 [sum n_r, words] array whose
    rows follow the requests' query order (words = max over requests)."""
    words = max([max(1, (m.shape[0] + 63) // 64) for m in masks] + [1])
    return np.concatenate([pack_mask_rows(m, words) for m in masks], axis=0) if masks else \
        np.zeros((0, words), dtype=np.uint64)


def _round_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest bfloat16 (ties to even), returned as float32."""
    a = np.asarray(x, dtype=np.float32)
    u = a.reshape(-1).copy().view(np.uint32)
    u = (u + (np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1)))) & np.uint32(0xFFFF0000)
    return u.view(np.float32).reshape(a.shape)


def d3_rejection_rates(conf: np.ndarray, dtype: str = "bfloat16") -> np.ndarray:
    """rates[0] = 1 - c0; rates[k] = prod(c_<k) * (1 - c_k)
    (generation/d3_generator.py:116-121), with torch's arithmetic for the
    dtype of `conf` there (the draft's softmax probabilities: bfloat16 for a
    bf16 model), as its GPU kernels do it:
      * bfloat16: conf rounded to bf16; the cumulative product runs
        sequentially, each product computed in float32 and rounded to bf16
        (torch.cumprod on a bf16 device tensor); 1 - c and the products
        likewise; stored into float32 rates;
      * float32: the same in float32 throughout.
    (torch's CPU cumprod would instead keep a float32 running product for
    bf16 input.)  Returns float32 [len(conf)]."""
    if dtype not in ("bfloat16", "float32"):
        raise ValueError("dtype must be 'bfloat16' or 'float32'")
    rnd = _round_bf16 if dtype == "bfloat16" else (lambda x: np.asarray(x, dtype=np.float32))
    c = rnd(np.asarray(conf, dtype=np.float32))
    n = c.shape[0]
    cum = np.empty(n, dtype=np.float32)
    acc = np.float32(1.0)
    for i in range(n):
        acc = rnd(np.float32(acc * c[i]))
        cum[i] = acc
    one_minus = rnd(np.float32(1.0) - c)
    rates = np.empty(n, dtype=np.float32)
    rates[0] = one_minus[0]
    if n > 1:
        rates[1:] = rnd(cum[:-1] * one_minus[1:])
    return rates


def d3_select_boundaries(rates: np.ndarray, topk: int) -> List[int]:
    """sorted(torch.topk(rates, topk).indices) (d3_generator.py:123-125), with
    equal rates taken in index order (torch.topk leaves the order of ties
    unspecified)."""
    order = sorted(range(len(rates)), key=lambda i: (-float(rates[i]), i))
    return sorted(order[:topk])


def d3_verify_tree(conf: np.ndarray, block_size: int = 16, block_size_2: int = 32, topk: int = 4,
                   dtype: str = "bfloat16") -> TokenTree:
    """Verify tree of one D2SD step (generation/d3_generator.py:116-180).

    conf: the block_size-1 per-position draft confidences (dtype: their torch
    dtype, see d3_rejection_rates).  The top-k rejection boundaries pl become
    rows that keep the first pl+1 tokens of the DFlash block and continue with
    a DTA re-draft; with block_size_2 > block_size, row 0 is the DFlash block
    plus its own DTA continuation.  With block_size_2 == block_size the DFlash
    block itself is the last row.
    """
    rates = d3_rejection_rates(conf, dtype)
    k = min(topk, block_size - 1)
    sel = d3_select_boundaries(rates, k)
    shared_pl = [pl + 1 for pl in sel if pl + 1 < block_size_2]
    if block_size_2 > block_size:
        shared = [block_size_2] + shared_pl
        return tree_from_shared_prefixes(block_size_2, shared)
    # block_size_2 == block_size: rows = [DTA rows..., DFlash row]; use the
    # DFlash row as the tree's row 0 and map back.
    base = tree_from_shared_prefixes(block_size_2, [block_size_2] + shared_pl)
    order = list(range(1, len(shared_pl) + 1)) + [0]
    return TokenTree(base.parents, base.node_index[order], [base.shared[i] for i in order])


class D3TreeBuilder:
    """The verify tree of one D2SD step built on the device (d2sd_d3_tree_build,
    generation/d3_generator.py:116-180 without the host top-k): rates, top-k
    boundaries, rows, and the node tree the cascade kernels read, into
    fixed-capacity device buffers made here once (allocation-free and
    capturable afterwards).

    After build(conf): num_nodes / num_rows [1], parents [capacity],
    node_index [rows_cap, block_size_2], tree_mask int64 [capacity,
    mask_words], shared [rows_cap], rates [block_size - 1] (all int32 but the
    mask and the float32 rates).  Nodes past num_nodes are roots seeing only
    themselves and rows past num_rows repeat the DFlash row, so a cascade plan
    for `capacity` nodes and a GreedyAccept over `rows_cap` rows serve every
    step unchanged.
    """

    def __init__(self, block_size: int = 16, block_size_2: int = 32, topk: int = 4, device=None,
                 capacity: Optional[int] = None):
        from . import _lib  # noqa: F401  (loads libd2sd.so)
        dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        k = min(topk, block_size - 1)
        self.block_size, self.block_size_2, self.topk = int(block_size), int(block_size_2), int(topk)
        self.capacity = int(capacity) if capacity is not None else block_size_2 + k * (block_size_2 - 1)
        self.rows_cap = k + 1
        self.mask_words = (self.capacity + 63) // 64
        i32 = dict(dtype=torch.int32, device=dev)
        self.num_nodes = torch.zeros(1, **i32)
        self.num_rows = torch.zeros(1, **i32)
        self.parents = torch.zeros(self.capacity, **i32)
        self.node_index = torch.zeros(self.rows_cap, self.block_size_2, **i32)
        self.tree_mask = torch.zeros(self.capacity, self.mask_words, dtype=torch.int64, device=dev)
        self.shared = torch.zeros(self.rows_cap, **i32)
        self.rates = torch.zeros(self.block_size - 1, dtype=torch.float32, device=dev)

    def build(self, conf: torch.Tensor, tree_mask: Optional[torch.Tensor] = None) -> "D3TreeBuilder":
        """conf: device [block_size - 1] bf16 or float32 (the draft's
        probabilities of its tokens).  tree_mask: optional device int64
        [capacity, mask_words] written instead of self.tree_mask (e.g. a
        cascade plan's mask buffer)."""
        import ctypes as C
        from . import _lib
        from .graph import keep_alive
        if conf.dtype not in (torch.bfloat16, torch.float32) or conf.numel() != self.block_size - 1:
            raise ValueError(f"conf must be bf16 or float32 with {self.block_size - 1} entries")
        if not conf.is_cuda or not conf.is_contiguous():
            raise ValueError("conf must be a contiguous device tensor")
        mask = self.tree_mask if tree_mask is None else tree_mask
        if (mask.dtype != torch.int64 or mask.shape != (self.capacity, self.mask_words) or not mask.is_contiguous()
                or mask.device != self.parents.device):
            raise ValueError(f"tree_mask must be a contiguous int64 [{self.capacity}, {self.mask_words}] device tensor")
        a = _lib.TreeArgs()
        a.conf = conf.data_ptr()
        a.conf_dtype = _lib.D2SD_DTYPE_BF16 if conf.dtype == torch.bfloat16 else _lib.D2SD_DTYPE_F32
        a.block_size, a.block_size_2, a.topk = self.block_size, self.block_size_2, self.topk
        a.capacity, a.rows_cap, a.mask_words = self.capacity, self.rows_cap, self.mask_words
        a.num_nodes, a.num_rows = self.num_nodes.data_ptr(), self.num_rows.data_ptr()
        a.parents, a.node_index = self.parents.data_ptr(), self.node_index.data_ptr()
        a.tree_mask, a.shared, a.rates = mask.data_ptr(), self.shared.data_ptr(), self.rates.data_ptr()
        _lib.check(_lib.lib.d2sd_d3_tree_build(C.byref(a), C.c_void_p(torch.cuda.current_stream().cuda_stream)),
                   "d3_tree_build")
        keep_alive(conf, mask, self.num_nodes, self.num_rows, self.parents, self.node_index, self.shared, self.rates)
        return self

    def host_tree(self) -> TokenTree:
        """The built tree as a TokenTree (reads the device buffers; synchronises)."""
        n, rows = int(self.num_nodes[0]), int(self.num_rows[0])
        return TokenTree(self.parents[:n].cpu().numpy().astype(np.int32),
                         self.node_index[:rows].cpu().numpy().astype(np.int32),
                         [int(s) for s in self.shared[:rows].cpu().tolist()])


def padded_ancestor_mask(tree: TokenTree, capacity: int) -> np.ndarray:
    """bool [capacity, capacity]: the tree's ancestor mask, nodes past its size
    seeing only themselves (the layout D3TreeBuilder writes)."""
    m = np.eye(capacity, dtype=bool)
    n = tree.num_nodes
    m[:n, :n] = ancestor_mask(tree.parents)
    return m


def to_device_mask(tree_masks: Sequence[np.ndarray], device) -> torch.Tensor:
    packed = pack_tree_masks(tree_masks)
    return torch.from_numpy(packed.view(np.int64)).to(device)


__all__ = ["TokenTree", "tree_from_shared_prefixes", "ancestor_mask", "pack_mask_rows", "pack_tree_masks",
           "d3_rejection_rates", "d3_select_boundaries", "d3_verify_tree", "D3TreeBuilder", "padded_ancestor_mask",
           "to_device_mask"]
