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


def d3_rejection_rates(conf: np.ndarray) -> np.ndarray:
    """rates[0] = 1 - c0; rates[k] = prod(c_<k) * (1 - c_k)
    (generation/d3_generator.py:117-121)."""
    conf = np.asarray(conf, dtype=np.float64)
    cum = np.cumprod(conf)
    rates = np.empty_like(conf)
    rates[0] = 1.0 - conf[0]
    rates[1:] = cum[:-1] * (1.0 - conf[1:])
    return rates


def d3_verify_tree(conf: np.ndarray, block_size: int = 16, block_size_2: int = 32, topk: int = 4) -> TokenTree:
    """Verify tree of one D2SD step (generation/d3_generator.py:116-180).

    conf: the block_size-1 per-position draft confidences.  The top-k
    rejection boundaries pl become rows that keep the first pl+1 tokens of the
    DFlash block and continue with a DTA re-draft; with block_size_2 >
    block_size, row 0 is the DFlash block plus its own DTA continuation.  With
    block_size_2 == block_size the DFlash block itself is the last row.
    """
    rates = d3_rejection_rates(conf)
    k = min(topk, block_size - 1)
    # torch.topk order does not matter: the reference sorts (d3_generator.py:125)
    sel = sorted(np.argsort(-rates, kind="stable")[:k].tolist())
    shared_pl = [pl + 1 for pl in sel if pl + 1 < block_size_2]
    if block_size_2 > block_size:
        shared = [block_size_2] + shared_pl
        return tree_from_shared_prefixes(block_size_2, shared)
    # block_size_2 == block_size: rows = [DTA rows..., DFlash row]; use the
    # DFlash row as the tree's row 0 and map back.
    base = tree_from_shared_prefixes(block_size_2, [block_size_2] + shared_pl)
    order = list(range(1, len(shared_pl) + 1)) + [0]
    return TokenTree(base.parents, base.node_index[order], [base.shared[i] for i in order])


def to_device_mask(tree_masks: Sequence[np.ndarray], device) -> torch.Tensor:
    packed = pack_tree_masks(tree_masks)
    return torch.from_numpy(packed.view(np.int64)).to(device)


__all__ = ["TokenTree", "tree_from_shared_prefixes", "ancestor_mask", "pack_mask_rows", "pack_tree_masks",
           "d3_rejection_rates", "d3_verify_tree", "to_device_mask"]
