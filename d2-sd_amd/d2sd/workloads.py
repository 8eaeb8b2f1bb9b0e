"""Seeded synthetic verify-attention problems (Q/K/V ~ N(0,1), rounded to bf16).

Shapes follow the verify step of generation/verification.py:127-176 at the
model shapes the reference runs (Qwen3-8B: 32 query / 8 kv heads, head_dim
128; GPT-OSS-20B: 64 / 8, head_dim 64; Qwen3-32B: 64 / 8, head_dim 128).
Tree geometry follows generation/d3_generator.py:116-180 (d3_verify_tree) or
random shared-prefix branches.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional, Sequence

import numpy as np
import torch

from .tree import TokenTree, ancestor_mask, d3_verify_tree


def tree_from_branches(row_len: int, parent_row: Sequence[int], shared: Sequence[int]) -> TokenTree:
    """Row r (r >= 1) shares its first shared[r] tokens with row parent_row[r] < r."""
    bsz = len(shared)
    node_index = np.zeros((bsz, row_len), dtype=np.int32)
    parents: List[int] = []
    for p in range(row_len):
        node_index[0, p] = p
        parents.append(p - 1)
    for r in range(1, bsz):
        pr, s = int(parent_row[r]), int(shared[r])
        if not 0 <= pr < r or not 0 <= s <= row_len:
            raise ValueError("bad branch spec")
        for p in range(row_len):
            if p < s:
                node_index[r, p] = node_index[pr, p]
            else:
                node_index[r, p] = len(parents)
                parents.append(int(node_index[r, p - 1]) if p > 0 else -1)
    return TokenTree(np.asarray(parents, dtype=np.int32), node_index, [row_len] + list(shared[1:]))


def random_branch_tree(rng: np.random.Generator, branches: int, row_len: int, chain_to_row0: bool = True) -> TokenTree:
    """`branches` rows of `row_len`; row r shares p_r ~ U{0..row_len-1} tokens
    with row 0 (chain_to_row0) or with a uniformly chosen earlier row."""
    shared = [row_len] + [int(rng.integers(0, row_len)) for _ in range(branches - 1)]
    parent_row = [0] + [0 if chain_to_row0 else int(rng.integers(0, r)) for r in range(1, branches)]
    return tree_from_branches(row_len, parent_row, shared)


@dataclass
class Request:
    tree: TokenTree
    prefix_len: int

    @property
    def n(self) -> int:
        return self.tree.num_nodes


@dataclass
class VerifyProblem:
    name: str
    num_qo_heads: int
    num_kv_heads: int
    head_dim: int
    requests: List[Request]
    page_size: int = 0            # 0: contiguous prefix
    kv_dtype: torch.dtype = torch.bfloat16
    window_left: int = -1
    with_sinks: bool = False
    layers: int = 1
    seed: int = 0
    meta: dict = field(default_factory=dict)

    @property
    def qo_indptr(self) -> List[int]:
        out = [0]
        for r in self.requests:
            out.append(out[-1] + r.n)
        return out

    @property
    def total_q(self) -> int:
        return self.qo_indptr[-1]

    @property
    def prefix_lens(self) -> List[int]:
        return [r.prefix_len for r in self.requests]

    def tree_masks(self) -> List[np.ndarray]:
        return [ancestor_mask(r.tree.parents) for r in self.requests]

    def visible_prefix(self, r: int) -> int:
        L = self.requests[r].prefix_len
        return min(L, self.window_left) if self.window_left >= 0 else L


def config1(seed: int = 0) -> VerifyProblem:
    """Single layer, Qwen3-8B shape, contiguous prefix 1024 ([Hkv, L, D]
    DynamicCache layout), 4 branches x 16, branch i shares p_i ~ U{0..15}
    tokens with branch 0."""
    rng = np.random.default_rng(seed)
    tree = random_branch_tree(rng, 4, 16)
    return VerifyProblem("cfg1_qwen3_8b_L1024_tree4x16", 32, 8, 128, [Request(tree, 1024)], page_size=0, seed=seed)


def config2(seed: int = 0, layers: int = 36) -> VerifyProblem:
    """All 36 layers of one D2SD verify step at Qwen3-8B shape: paged prefix
    4096 (page 16, random page permutation), DFlash block 16 + top-4 DTA
    branches of block 32 (d3_verify_tree with conf ~ U(0,1)^15)."""
    rng = np.random.default_rng(seed)
    conf = rng.uniform(0.0, 1.0, size=15)
    tree = d3_verify_tree(conf, block_size=16, block_size_2=32, topk=4)
    return VerifyProblem("cfg2_qwen3_8b_L4096_paged16_d3tree_36layers", 32, 8, 128, [Request(tree, 4096)],
                         page_size=16, layers=layers, seed=seed, meta={"conf": conf.tolist()})


def northstar(seed: int = 0, layers: int = 36) -> VerifyProblem:
    """The north-star shape: Qwen3-8B heads (32/8, head_dim 128), paged prefix
    4096 (page 16, random page permutation) and the "4 x 16 + 32" tree of the
    d3 geometry (generation/d3_generator.py:123-147): a 32-token main row
    (the DFlash block of 16 and its DTA continuation to block_size_2 = 32) and
    four branches that each share the main row's first 16 tokens and add 16
    of their own, N = 32 + 4 x 16 = 96 nodes."""
    tree = tree_from_branches(32, [0, 0, 0, 0, 0], [32, 16, 16, 16, 16])
    return VerifyProblem("northstar_qwen3_8b_L4096_paged16_tree4x16+32", 32, 8, 128, [Request(tree, 4096)],
                         page_size=16, layers=layers, seed=seed)


def config3(seed: int = 0, num_reqs: int = 8) -> VerifyProblem:
    """8 requests, prefix ~ U{8192..32768}, paged 16, 4 x 16 trees."""
    rng = np.random.default_rng(seed)
    reqs = [Request(random_branch_tree(rng, 4, 16), int(rng.integers(8192, 32769))) for _ in range(num_reqs)]
    return VerifyProblem("cfg3_qwen3_8b_batch8_L8k-32k_paged16", 32, 8, 128, reqs, page_size=16, seed=seed)


def config4(seed: int = 0, sliding: bool = False) -> VerifyProblem:
    """GPT-OSS-20B shape (64/8 heads, head_dim 64), prefix 8192 paged 16,
    8 x 32 random ancestor tree, per-head sinks; sliding layers keep the last
    128 prefix keys."""
    rng = np.random.default_rng(seed)
    tree = random_branch_tree(rng, 8, 32, chain_to_row0=False)
    return VerifyProblem("cfg4_gpt_oss_20b_L8192_tree8x32" + ("_sliding128" if sliding else "_full"), 64, 8, 64,
                         [Request(tree, 8192)], page_size=16, window_left=128 if sliding else -1,
                         with_sinks=True, seed=seed)


def config5(seed: int = 0, num_reqs: int = 32) -> VerifyProblem:
    """Qwen3-32B shape (64/8 heads, head_dim 128), 32 requests x prefix 8192
    paged 16, fp8 e4m3fn KV with per-kv-head scales, 8 x 32 random trees."""
    rng = np.random.default_rng(seed)
    reqs = [Request(random_branch_tree(rng, 8, 32, chain_to_row0=False), 8192) for _ in range(num_reqs)]
    return VerifyProblem("cfg5_qwen3_32b_batch32_L8192_fp8kv", 64, 8, 128, reqs, page_size=16,
                         kv_dtype=torch.float8_e4m3fn, seed=seed)


@dataclass
class LayerTensors:
    q: torch.Tensor
    k_suffix: torch.Tensor
    v_suffix: torch.Tensor
    k_prefix: Optional[torch.Tensor]   # pool [pages, Hkv, P, D] or [Hkv, L_total, D]
    v_prefix: Optional[torch.Tensor]


@dataclass
class MaterializedProblem:
    problem: VerifyProblem
    layers: List[LayerTensors]
    page_table: Optional[torch.Tensor]    # int32 [total pages]
    page_indptr: Optional[List[int]]
    prefix_tok_indptr: Optional[List[int]]
    sinks: Optional[torch.Tensor]
    k_scale: Optional[torch.Tensor]
    v_scale: Optional[torch.Tensor]


def _randn_bf16(shape, gen: torch.Generator, device) -> torch.Tensor:
    return torch.randn(shape, generator=gen, device=device, dtype=torch.float32).to(torch.bfloat16)


def materialize(prob: VerifyProblem, device, layers: Optional[int] = None) -> MaterializedProblem:
    """Allocate and fill the problem's tensors on `device` (deterministic in
    prob.seed).  Paged pools are HND [pages, Hkv, P, D] with one randomly
    permuted page table over all requests; a contiguous prefix is the
    DynamicCache layout [Hkv, sum L, D]."""
    device = torch.device(device)
    gen = torch.Generator(device=device)
    gen.manual_seed(prob.seed + 1)
    rng = np.random.default_rng(prob.seed + 2)
    hq, hkv, d = prob.num_qo_heads, prob.num_kv_heads, prob.head_dim
    T = prob.total_q
    nl = prob.layers if layers is None else layers
    page_table = page_indptr = tok_indptr = None
    if prob.page_size > 0:
        P = prob.page_size
        pages = [(r.prefix_len + P - 1) // P for r in prob.requests]
        page_indptr = [0]
        for c in pages:
            page_indptr.append(page_indptr[-1] + c)
        total_pages = page_indptr[-1]
        page_table = torch.from_numpy(rng.permutation(total_pages).astype(np.int32)).to(device)
        pool_shape = (max(total_pages, 1), hkv, P, d)
    else:
        tok_indptr = [0]
        for r in prob.requests:
            tok_indptr.append(tok_indptr[-1] + r.prefix_len)
        pool_shape = (hkv, max(tok_indptr[-1], 1), d)
    k_scale = v_scale = None
    if prob.kv_dtype == torch.float8_e4m3fn:
        # per-kv-head scale = absmax / 448 of the N(0,1) data (fixed below
        # after generation per layer 0; same scale for all layers)
        pass
    out_layers = []
    for _ in range(nl):
        q = _randn_bf16((T, hq, d), gen, device)
        ks = _randn_bf16((T, hkv, d), gen, device)
        vs = _randn_bf16((T, hkv, d), gen, device)
        has_prefix = any(r.prefix_len > 0 for r in prob.requests)
        kp = vp = None
        if has_prefix:
            kf = torch.randn(pool_shape, generator=gen, device=device, dtype=torch.float32)
            vf = torch.randn(pool_shape, generator=gen, device=device, dtype=torch.float32)
            if prob.kv_dtype == torch.float8_e4m3fn:
                head_axis = 1 if prob.page_size > 0 else 0
                red = [a for a in range(4 if prob.page_size > 0 else 3) if a != head_axis]
                if k_scale is None:
                    k_scale = (kf.abs().amax(dim=red) / 448.0).float()
                    v_scale = (vf.abs().amax(dim=red) / 448.0).float()
                shape = [1] * kf.dim()
                shape[head_axis] = hkv
                kp = (kf / k_scale.view(shape)).to(torch.float8_e4m3fn)
                vp = (vf / v_scale.view(shape)).to(torch.float8_e4m3fn)
            else:
                kp, vp = kf.to(torch.bfloat16), vf.to(torch.bfloat16)
            del kf, vf
        out_layers.append(LayerTensors(q, ks, vs, kp, vp))
    sinks = torch.randn((hq,), generator=gen, device=device, dtype=torch.float32) if prob.with_sinks else None
    return MaterializedProblem(prob, out_layers, page_table, page_indptr,
                               tok_indptr[:-1] if tok_indptr is not None else None, sinks, k_scale, v_scale)


def plan_for(attn, mp: MaterializedProblem, **kw):
    """Call CascadeVerifyAttention.plan for a materialized problem."""
    prob = mp.problem
    return attn.plan(prob.qo_indptr, prob.prefix_lens, prob.num_qo_heads, prob.num_kv_heads, prob.head_dim,
                     tree_masks=prob.tree_masks(), mask_mode="tree", page_size=prob.page_size,
                     page_indptr=mp.page_indptr, page_table=mp.page_table, prefix_tok_indptr=mp.prefix_tok_indptr,
                     kv_layout="HND", window_left=prob.window_left, sinks=mp.sinks, kv_dtype=prob.kv_dtype,
                     k_scale=mp.k_scale, v_scale=mp.v_scale, **kw)


def prefix_bytes_flops(prob: VerifyProblem) -> tuple:
    """Algorithmic bytes and flops of the prefix level (per layer):
    bytes = sum_r [2 L_eff Hkv D b_kv + N Hq D 2 (Q) + N Hq D 2 (O) + N Hq 4 (LSE)
                   + 4 ceil(L/P) (page table)] (+ 2 Hkv 4 fp8 scales),
    flops = sum_r 4 N Hq L_eff D."""
    b_kv = 1 if prob.kv_dtype == torch.float8_e4m3fn else 2
    hq, hkv, d = prob.num_qo_heads, prob.num_kv_heads, prob.head_dim
    nbytes = 0
    flops = 0
    for i, r in enumerate(prob.requests):
        Leff = prob.visible_prefix(i)
        n = r.n
        nbytes += 2 * Leff * hkv * d * b_kv + n * hq * d * 2 * 2 + n * hq * 4
        if prob.page_size > 0:
            nbytes += 4 * ((r.prefix_len + prob.page_size - 1) // prob.page_size)
        flops += 4 * n * hq * Leff * d
    if b_kv == 1:
        nbytes += 2 * hkv * 4
    return nbytes, flops


def verify_bytes_flops(prob: VerifyProblem) -> tuple:
    """Whole verify attention (prefix + suffix tree): adds suffix KV
    2 N Hkv D 2, the tree mask N ceil(N/64) 8 and masked suffix flops
    4 Hq D sum_i |anc(i)|."""
    nbytes, flops = prefix_bytes_flops(prob)
    hq, hkv, d = prob.num_qo_heads, prob.num_kv_heads, prob.head_dim
    for r in prob.requests:
        n = r.n
        anc = int(ancestor_mask(r.tree.parents).sum())
        nbytes += 2 * n * hkv * d * 2 + n * ((n + 63) // 64) * 8
        flops += 4 * hq * d * anc
    return nbytes, flops


def attention_launch_bytes_flops(prob: VerifyProblem) -> tuple:
    """Algorithmic bytes and flops of the attention launch of run() (per
    layer): both levels' K/V once (prefix at the cache dtype, suffix bf16),
    Q once, the page table and the tree mask; flops over visible (query,
    key) pairs only.  O / LSE are written by the merge launch and partial
    states are implementation traffic, so neither is counted here."""
    hq, hkv, d = prob.num_qo_heads, prob.num_kv_heads, prob.head_dim
    b_kv = 1 if prob.kv_dtype == torch.float8_e4m3fn else 2
    nbytes = 0
    flops = 0
    for i, r in enumerate(prob.requests):
        Leff = prob.visible_prefix(i)
        n = r.n
        anc = int(ancestor_mask(r.tree.parents).sum())
        nbytes += 2 * Leff * hkv * d * b_kv + 2 * n * hkv * d * 2 + n * hq * d * 2 + n * ((n + 63) // 64) * 8
        if prob.page_size > 0:
            nbytes += 4 * ((r.prefix_len + prob.page_size - 1) // prob.page_size)
        flops += 4 * hq * d * (n * Leff + anc)
    if b_kv == 1:
        nbytes += 2 * hkv * 4
    return nbytes, flops
