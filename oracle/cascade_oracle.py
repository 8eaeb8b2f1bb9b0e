"""CPU oracle for cascade tree-verification attention.

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and bench.py's
CPU-baseline leg may import this module, and only as the checker / the timed
CPU baseline — never as a product path.

It restates the reference's verify-attention algorithm on the CPU in float64
(or float32 for the timed baseline):

  reference path                                   function here
  generation/verification.py:127-135 prefix+window  window_prefix_ref
  verification.py:145-150 (flashinfer single prefill, shared level, non-causal)
  verification.py:159-162 (local level, causal)    single_prefill_ref / attention_ref
  verification.py:163-165, cascade_graph.py:58-60 (flashinfer merge_state_in_place)
                                                   merge_state_ref
  verification.py:173-176 (GPT-OSS sink)           sink_rescale_ref
  verification.py:127-176 as a whole (row layout)  cascade_verify_rows_ref
  the same over unique tree nodes, single pass     cascade_tree_ref
  d3_generator.py:227-232 (accepted-branch commit) commit_accepted_ref
  the same into an fp8 e4m3fn pool                  quantize_e4m3fn_ref
  d3_generator.py:204-225 (greedy acceptance walk) greedy_accept_ref
  d3_generator.py:204-225 at temperature > 0 (model/utils.py:34-37,
  torch.multinomial's exponential race)            sample_scores_ref, sampled_accept_ref
  Philox4x32-10 (the counter-based generator the sampled walk draws from)
                                                   philox4x32_10
  verification.py:113-123 (QK RMSNorm + RoPE)       qk_norm_rope_ref
  model/dflash.py:103-108 (DTA shared level, [draft cache | context])
                                                   dta_shared_prefix_ref

FlashInfer itself (flashinfer-python>=0.2.0, requirements.txt:13) is not
vendored in the reference and not installed here.  Its published algorithm for
the two calls the reference makes is restated from its documentation:
softmax attention with scale sm_scale, query head h reading kv head
h // (Hq // Hkv), causal alignment to the bottom-right corner
(key j visible to query i iff j <= i + kv_len - qo_len), and merge_state
  s = log(e^{s_a} + e^{s_b}),  v = (v_a e^{s_a} + v_b e^{s_b}) / e^{s}.
The LSE here is the natural log; FlashInfer's own LSE base (its kernels work
in the exp2 domain) is parity unpinned, as are its bf16 rounding of P before
P.V and its accumulation order (bit-level parity).

How each function is pinned (tests/test_oracle.py): against pure-Python
float64 loops in tests/golden/make_golden.py (written independently of this
module) and the committed fixtures they produce; against invariants (split
prefix merged == unsplit; merge commutative / associative; empty prefix ->
pure tree attention; chain tree == causal; constant V -> that V; page-table
permutation invariance); against the reference's three-step row-layout
algorithm vs. the single-pass tree form; and, for the sink, against the
installed transformers GPT-OSS eager attention (a library routine).
dta_shared_prefix_ref is pinned token by token to the reference's cat order
and by the split-KV identity (its attention == the merge of the two
segments' attentions).
philox4x32_10 is pinned to the published known-answer vectors of Random123
(the generator's authors' reference release); sample_scores_ref to the
mathematics it restates: sampled frequencies follow softmax(x) (chi-square),
and its choice equals torch.multinomial's argmax(p / E) on the same E.
"""
from __future__ import annotations

import math
from typing import List, Optional, Tuple

import numpy as np
import torch
import torch.nn.functional as F

Tensor = torch.Tensor


def _expand_kv(k: Tensor, hq: int) -> Tensor:
    """[L, Hkv, D] -> [L, Hq, D] with query head h reading kv head h // g."""
    hkv = k.shape[1]
    if hq % hkv:
        raise ValueError("Hq must be a multiple of Hkv")
    return k.repeat_interleave(hq // hkv, dim=1)


def attention_ref(q: Tensor, k: Tensor, v: Tensor, mask: Optional[Tensor], sm_scale: float,
                  dtype: torch.dtype = torch.float64) -> Tuple[Tensor, Tensor]:
    """Masked GQA softmax attention.  q [n, Hq, D], k/v [L, Hkv, D],
    mask bool [n, L] (True = visible) or None.  Returns (o [n, Hq, D],
    lse [n, Hq]) in `dtype`; rows with no visible key give o = 0, lse = -inf."""
    n, hq, d = q.shape
    L = k.shape[0]
    qd, kd, vd = q.to(dtype), _expand_kv(k.to(dtype), hq), _expand_kv(v.to(dtype), hq)
    if L == 0:
        return torch.zeros(n, hq, d, dtype=dtype), torch.full((n, hq), -math.inf, dtype=dtype)
    scores = torch.einsum("nhd,lhd->hnl", qd, kd) * sm_scale          # [Hq, n, L]
    if mask is not None:
        scores = scores.masked_fill(~mask.bool()[None], -math.inf)
    lse = torch.logsumexp(scores, dim=-1)                              # [Hq, n]
    empty = torch.isinf(lse) & (lse < 0)
    p = torch.exp(scores - torch.where(empty, torch.zeros_like(lse), lse)[..., None])
    p = torch.where(empty[..., None], torch.zeros_like(p), p)
    o = torch.einsum("hnl,lhd->nhd", p, vd)
    return o, lse.transpose(0, 1).contiguous()


def attention_sdpa_ref(q: Tensor, k: Tensor, v: Tensor, mask: Optional[Tensor], sm_scale: float,
                       dtype: torch.dtype = torch.float32) -> Tuple[Tensor, Tensor]:
    """Same contract via torch.nn.functional.scaled_dot_product_attention
    (enable_gqa) for O and torch.logsumexp for LSE — the formulation the CPU
    baseline times.  Every row must have at least one visible key."""
    n, hq, d = q.shape
    qd = q.to(dtype).transpose(0, 1)[None]                             # [1, Hq, n, D]
    kd = k.to(dtype).transpose(0, 1)[None]                             # [1, Hkv, L, D]
    vd = v.to(dtype).transpose(0, 1)[None]
    m = mask.bool()[None, None] if mask is not None else None
    o = F.scaled_dot_product_attention(qd, kd, vd, attn_mask=m, scale=sm_scale, enable_gqa=True)
    scores = torch.matmul(qd, _expand_kv(k.to(dtype), hq).transpose(0, 1)[None].transpose(-1, -2)) * sm_scale
    if m is not None:
        scores = scores.masked_fill(~m, -math.inf)
    lse = torch.logsumexp(scores, dim=-1)[0].transpose(0, 1)
    return o[0].transpose(0, 1).contiguous(), lse.contiguous()


def causal_mask(qo_len: int, kv_len: int) -> Tensor:
    """FlashInfer causal rule: key j visible to query i iff j <= i + kv_len - qo_len."""
    i = torch.arange(qo_len)[:, None]
    j = torch.arange(kv_len)[None, :]
    return j <= i + (kv_len - qo_len)


def single_prefill_ref(q: Tensor, k: Tensor, v: Tensor, causal: bool, sm_scale: float,
                       dtype: torch.dtype = torch.float64) -> Tuple[Tensor, Tensor]:
    """flashinfer.single_prefill_with_kv_cache(q, k, v, causal, return_lse=True,
    sm_scale) as called at generation/verification.py:145-148 and 159-162."""
    mask = causal_mask(q.shape[0], k.shape[0]) if causal else None
    return attention_ref(q, k, v, mask, sm_scale, dtype)


def merge_state_ref(v: Tensor, s: Tensor, v_other: Tensor, s_other: Tensor) -> Tuple[Tensor, Tensor]:
    """flashinfer.merge_state_in_place semantics (generation/verification.py:163-165;
    model/cascade_graph.py:58-60), out of place, in float64.  An operand with
    s = -inf contributes nothing; both -inf leaves (v, -inf)."""
    v, s, v_other, s_other = (x.to(torch.float64) for x in (v, s, v_other, s_other))
    m = torch.maximum(s, s_other)
    both_empty = torch.isinf(m) & (m < 0)
    m_safe = torch.where(both_empty, torch.zeros_like(m), m)
    ea, eb = torch.exp(s - m_safe), torch.exp(s_other - m_safe)
    tot = ea + eb
    tot_safe = torch.where(both_empty, torch.ones_like(tot), tot)
    out = (v * ea[..., None] + v_other * eb[..., None]) / tot_safe[..., None]
    out = torch.where(both_empty[..., None], v, out)
    lse = torch.where(both_empty, s, m_safe + torch.log(tot_safe))
    return out, lse


def sink_rescale_ref(o: Tensor, lse: Tensor, sinks: Tensor) -> Tensor:
    """GPT-OSS sink (generation/verification.py:173-176): O * sigmoid(lse - sink_h),
    lse = the merged natural-log LSE [..., Hq], sinks [Hq]."""
    return o * torch.sigmoid(lse.to(torch.float64) - sinks.to(torch.float64))[..., None]


def window_prefix_ref(k: Tensor, v: Tensor, window: int) -> Tuple[Tensor, Tensor]:
    """Sliding-window prefix rule (generation/verification.py:132-135): if the
    prefix [L, Hkv, D] is longer than `window`, keep its last `window` keys for
    every query; -1 / None keeps all."""
    if window is not None and window >= 0 and k.shape[0] > window:
        return k[k.shape[0] - window:], v[v.shape[0] - window:]
    return k, v


def cascade_verify_rows_ref(q_rows: Tensor, k_rows: Tensor, v_rows: Tensor, k_prefix: Tensor,
                            v_prefix: Tensor, sm_scale: float, window: int = -1,
                            sinks: Optional[Tensor] = None, causal: bool = True) -> Tuple[Tensor, Tensor]:
    """The reference's per-layer attention block, step by step
    (generation/verification.py:127-176), on bsz candidate rows:
      q_rows [bsz, Lb, Hq, D]; k_rows / v_rows [bsz, Lb, Hkv, D] (the rows' new
      KV); k_prefix / v_prefix [L, Hkv, D] (NHD).
    1. window truncation of the prefix (132-135)
    2. shared level: all bsz*Lb queries vs the prefix, non-causal (142-150)
    3. per row i: local causal attention over the row's own Lb keys (158-162)
    4. merge_state_in_place of the local into the shared state (163-165)
    5. GPT-OSS sink rescale with the merged LSE (173-176)
    Returns (out [bsz, Lb, Hq, D], lse [bsz, Lb, Hq]) in float64."""
    bsz, lb, hq, d = q_rows.shape
    kp, vp = window_prefix_ref(k_prefix, v_prefix, window)
    q_all = q_rows.reshape(bsz * lb, hq, d)
    o_sh, lse_sh = single_prefill_ref(q_all, kp, vp, causal=False, sm_scale=sm_scale)
    o_sh = o_sh.view(bsz, lb, hq, d)
    lse_sh = lse_sh.view(bsz, lb, hq)
    outs, lses = [], []
    for i in range(bsz):
        o_l, lse_l = single_prefill_ref(q_rows[i], k_rows[i], v_rows[i], causal=causal, sm_scale=sm_scale)
        o_m, lse_m = merge_state_ref(o_sh[i], lse_sh[i], o_l, lse_l)
        outs.append(o_m)
        lses.append(lse_m)
    out = torch.stack(outs)
    lse = torch.stack(lses)
    if sinks is not None:
        out = sink_rescale_ref(out, lse, sinks)
    return out, lse


def cascade_tree_ref(q: Tensor, k_suffix: Tensor, v_suffix: Tensor, k_prefix: Optional[Tensor],
                     v_prefix: Optional[Tensor], anc_mask: Tensor, sm_scale: float, window: int = -1,
                     sinks: Optional[Tensor] = None, dtype: torch.dtype = torch.float64,
                     use_sdpa: bool = False) -> Tuple[Tensor, Tensor]:
    """Single-pass form over unique tree nodes: one masked softmax over
    [prefix || suffix] keys with mask [ones(N, L_eff) || M], M[i, j] = node j is
    i or an ancestor of i.  q [N, Hq, D], k/v_suffix [N, Hkv, D],
    k/v_prefix [L, Hkv, D] or None."""
    n = q.shape[0]
    if k_prefix is not None and k_prefix.shape[0] > 0:
        kp, vp = window_prefix_ref(k_prefix, v_prefix, window)
        # concatenate in the computation dtype: a dequantised (fp32) prefix
        # must not be rounded to the suffix's bf16
        k_all = torch.cat([kp.to(dtype), k_suffix.to(dtype)], 0)
        v_all = torch.cat([vp.to(dtype), v_suffix.to(dtype)], 0)
        mask = torch.cat([torch.ones(n, kp.shape[0], dtype=torch.bool), anc_mask.bool()], 1)
    else:
        k_all, v_all, mask = k_suffix, v_suffix, anc_mask.bool()
    fn = attention_sdpa_ref if use_sdpa else attention_ref
    o, lse = fn(q, k_all, v_all, mask, sm_scale, dtype)
    if sinks is not None:
        o = o * torch.sigmoid(lse.to(dtype) - sinks.to(dtype))[..., None]
    return o, lse


def dta_shared_prefix_ref(k_cache: Tensor, v_cache: Tensor, k_ctx: Tensor, v_ctx: Tensor) -> Tuple[Tensor, Tensor]:
    """The DTA draft's shared level (model/dflash.py:103-108): the draft
    cache [Hkv, Lc, D] and the projected target context [Hkv, C, D] joined
    along tokens (torch.cat(..., dim=1)), then made NHD [Lc + C, Hkv, D]
    (transpose(0, 1).contiguous()), the layout single_prefill reads."""
    k = torch.cat([k_cache, k_ctx], dim=1).transpose(0, 1).contiguous()
    v = torch.cat([v_cache, v_ctx], dim=1).transpose(0, 1).contiguous()
    return k, v


def ancestor_mask_from_rows(node_index: np.ndarray, num_nodes: int) -> np.ndarray:
    """Ancestor mask rebuilt from the row layout alone: node j is visible to
    node i iff some row holds i at position p and j at a position <= p (the
    reference's per-row causal rule, verification.py:161)."""
    m = np.zeros((num_nodes, num_nodes), dtype=bool)
    for row in np.asarray(node_index):
        for p, i in enumerate(row):
            m[int(i), [int(x) for x in row[:p + 1]]] = True
    return m


def fp8_dequant_ref(x: Tensor, scale: Tensor) -> Tensor:
    """fp8 e4m3fn [.., Hkv, D] (or [pages, Hkv, P, D]) times a per-kv-head scale,
    in float32.  `head_dim_axis` of the scale is the Hkv axis given by the caller
    via broadcasting."""
    return x.to(torch.float32) * scale.to(torch.float32)


def gather_paged(pool: Tensor, page_table: List[int], length: int, layout: str = "HND") -> Tensor:
    """Paged pool [pages, Hkv, P, D] (HND) or [pages, P, Hkv, D] (NHD) ->
    contiguous [length, Hkv, D] in page_table order."""
    if layout == "HND":
        pages = pool[torch.as_tensor(list(page_table), dtype=torch.long)].permute(0, 2, 1, 3)
    else:
        pages = pool[torch.as_tensor(list(page_table), dtype=torch.long)]
    flat = pages.reshape(-1, pages.shape[2], pages.shape[3])
    return flat[:length]


def quantize_e4m3fn_ref(x: Tensor, scale: Tensor) -> Tensor:
    """bf16 values [.., Hkv, D] into an fp8 pool's format: x / scale[head] in
    fp32, clamped to the largest finite e4m3fn (448), then torch's
    float -> float8_e4m3fn cast (round to nearest even)."""
    q = x.float() / scale.float()[:, None]
    return q.clamp(-448.0, 448.0).to(torch.float8_e4m3fn)


def commit_accepted_ref(pool: Tensor, page_table: List[int], prefix_len: int, new: Tensor,
                        node_ids: List[int], layout: str = "HND", scale: Optional[Tensor] = None) -> Tensor:
    """Accepted-branch commit (generation/d3_generator.py:227-232): the cache
    grows by the accepted row's tokens, here the tree nodes node_ids of `new`
    ([rows, Hkv, D]) in order, at positions prefix_len .. prefix_len + n - 1 of
    the paged pool.  Returns a new pool; nodes outside [0, rows) are skipped
    (nothing written), as by the kernel.  An fp8 pool stores
    quantize_e4m3fn_ref(row, scale) (scale: fp32 [Hkv])."""
    if pool.dtype == torch.float8_e4m3fn:
        new = quantize_e4m3fn_ref(new, scale)
    out = pool.clone()
    P = pool.shape[2] if layout == "HND" else pool.shape[1]
    for i, node in enumerate(node_ids):
        if not 0 <= node < new.shape[0]:
            continue
        t = prefix_len + i
        page, slot = page_table[t // P], t % P
        if layout == "HND":
            out[page, :, slot, :] = new[node]
        else:
            out[page, slot, :, :] = new[node]
    return out


def qk_norm_rope_ref(x: Tensor, weight: Optional[Tensor], cos: Optional[Tensor], sin: Optional[Tensor],
                     eps: float = 1e-6) -> Tensor:
    """generation/verification.py:113-123 on x [tokens, heads, D] (bf16): the
    per-head RMSNorm of transformers' Qwen3RMSNorm (fp32 statistics, result
    cast to bf16, times the bf16 weight) when weight is given, then the
    rotate_half RoPE of _apply_rotary_pos_emb_qwen3 (cos / sin [tokens, D]) or
    the split-half form of _apply_rotary_pos_emb_gpt_oss (cos / sin
    [tokens, D/2]), as bf16 tensor ops."""
    y = x
    if weight is not None:
        h = x.to(torch.float32)
        var = h.pow(2).mean(-1, keepdim=True)
        h = h * torch.rsqrt(var + eps)
        y = weight * h.to(x.dtype)
    if cos is None:
        return y
    c, s_ = cos.unsqueeze(1), sin.unsqueeze(1)
    if cos.shape[-1] == x.shape[-1]:
        half = x.shape[-1] // 2
        rot = torch.cat((-y[..., half:], y[..., :half]), dim=-1)
        return (y * c) + (rot * s_)
    first, second = torch.chunk(y, 2, dim=-1)
    return torch.cat([first * c - second * s_, second * c + first * s_], dim=-1)


def greedy_accept_ref(node_logits: Tensor, node_index, draft_ids) -> Tuple[List[int], List[int], int, int]:
    """The acceptance loop of generation/d3_generator.py:204-225 at temperature
    0 (sample() is torch.argmax, model/utils.py:28-33), literally, on the rows'
    logits output_logits[row, pos] = node_logits[node_index[row][pos]] and the
    rows' draft tokens block_output_ids = draft_ids.  Returns (accept_ids,
    accepted nodes, acceptance_length, valid_block)."""
    node_index = torch.as_tensor(node_index, dtype=torch.long)
    block_output_ids = torch.as_tensor(draft_ids, dtype=torch.long)
    bsz, block_size_2 = node_index.shape
    output_logits = node_logits[node_index]                  # [bsz, Lb, V]
    valid_blocks = torch.ones(bsz)
    acceptance_length = 0
    accept_ids: List[int] = []
    nodes: List[int] = []
    while True:
        valid_block = int((valid_blocks > 0).nonzero(as_tuple=True)[0][0])
        logit = output_logits[valid_block, acceptance_length, :]
        sampled_token = int(torch.argmax(logit))
        nodes.append(int(node_index[valid_block, acceptance_length]))
        acceptance_length += 1
        accept_ids.append(sampled_token)
        if acceptance_length == block_size_2:
            break
        next_tokens = block_output_ids[:, acceptance_length]
        valid_mask = next_tokens == sampled_token
        valid_blocks = torch.where(valid_mask, valid_blocks, torch.zeros_like(valid_blocks))
        if valid_blocks.sum() == 0.:
            break
    return accept_ids, nodes, acceptance_length, valid_block


PHILOX_M = (0xD2511F53, 0xCD9E8D57)
PHILOX_W = (0x9E3779B9, 0xBB67AE85)


def philox4x32_10(ctr: np.ndarray, key: Tuple[int, int]) -> np.ndarray:
    """Philox4x32-10 (Salmon, Moraes, Dror and Shaw, "Parallel random numbers:
    as easy as 1, 2, 3", SC 2011), vectorised: ctr [..., 4] uint32 words
    (c0..c3), key (k0, k1) -> [..., 4] uint32.  Ten rounds of
    (c0, c1, c2, c3) <- (hi(M1 c2) ^ c1 ^ k0, lo(M1 c2), hi(M0 c0) ^ c3 ^ k1, lo(M0 c0))
    with the key bumped by the Weyl constants (W0, W1) between rounds."""
    m32 = np.uint64(0xFFFFFFFF)
    c = [np.asarray(ctr, dtype=np.uint64)[..., i] for i in range(4)]
    k0, k1 = np.uint64(key[0] & 0xFFFFFFFF), np.uint64(key[1] & 0xFFFFFFFF)
    for _ in range(10):
        p0 = c[0] * np.uint64(PHILOX_M[0])
        p1 = c[2] * np.uint64(PHILOX_M[1])
        c = [(p1 >> np.uint64(32)) ^ c[1] ^ k0, p1 & m32, (p0 >> np.uint64(32)) ^ c[3] ^ k1, p0 & m32]
        k0 = (k0 + np.uint64(PHILOX_W[0])) & m32
        k1 = (k1 + np.uint64(PHILOX_W[1])) & m32
    return np.stack(c, -1).astype(np.uint32)


def sample_uniforms_ref(num_nodes: int, vocab: int, seed: int, offset: int) -> np.ndarray:
    """The uniform variate of (node n, token v) at step counter `offset`: word
    v % 4 of Philox4x32-10 with counter (v // 4, n, offset low, offset high)
    and key (seed low, seed high), as u = (2 (w >> 9) + 1) 2^-24, in (0, 1)
    and exact in fp32.  float64 [num_nodes, vocab]."""
    q = np.arange((vocab + 3) // 4, dtype=np.uint64)
    n = np.arange(num_nodes, dtype=np.uint64)
    ctr = np.zeros((num_nodes, q.size, 4), dtype=np.uint64)
    ctr[..., 0] = q[None, :]
    ctr[..., 1] = n[:, None]
    ctr[..., 2] = offset & 0xFFFFFFFF
    ctr[..., 3] = (offset >> 32) & 0xFFFFFFFF
    w = philox4x32_10(ctr, (seed & 0xFFFFFFFF, (seed >> 32) & 0xFFFFFFFF)).reshape(num_nodes, -1)[:, :vocab]
    return ((w >> np.uint32(9)).astype(np.float64) * 2.0 + 1.0) * 2.0 ** -24


def scaled_logits_ref(node_logits: Tensor, temperature: float) -> np.ndarray:
    """`logits / temperature` as torch computes it on the GPU for a Python
    scalar (model/utils.py:34): logits times the fp32 reciprocal of the
    temperature in fp32, rounded to the logits dtype.  float64 array."""
    inv = np.float32(1.0) / np.float32(temperature)
    x = node_logits.float() * torch.tensor(inv, dtype=torch.float32)
    return x.to(node_logits.dtype).double().numpy()


def sample_scores_ref(node_logits: Tensor, temperature: float, seed: int, offset: int) -> np.ndarray:
    """Per (node, token) score whose argmax is the token sampled from
    softmax(x) (model/utils.py:34-37), x = scaled_logits_ref: torch.multinomial
    of one sample is argmax(p / E) with E ~ Exp(1) (the exponential race), and
    log2(p / E) = x log2(e) - log2(E) - log2(sum) ranks the same.  E = -ln(u)
    of sample_uniforms_ref.  float64 [num_nodes, vocab]."""
    x = scaled_logits_ref(node_logits, temperature)
    u = sample_uniforms_ref(x.shape[0], x.shape[1], seed, offset)
    e = -np.log1p(-(1.0 - u))
    return x * (1.0 / math.log(2.0)) - np.log2(e)


def sampled_accept_ref(node_logits: Tensor, node_index, draft_ids, temperature: float, seed: int,
                       offset: int) -> Tuple[List[int], List[int], int, int]:
    """The acceptance loop of d3_generator.py:204-225 at temperature > 0:
    sample() draws each accepted token from softmax(logits / T) of the first
    valid row's node.  Each node is visited at most once per walk, so drawing
    every node's token up front (sample_scores_ref at this step counter) and
    walking greedily over those scores is the same process."""
    scores = torch.from_numpy(sample_scores_ref(node_logits, temperature, seed, offset))
    return greedy_accept_ref(scores, node_index, draft_ids)


__all__ = [
    "attention_ref", "attention_sdpa_ref", "causal_mask", "single_prefill_ref", "merge_state_ref",
    "sink_rescale_ref", "window_prefix_ref", "cascade_verify_rows_ref", "cascade_tree_ref",
    "ancestor_mask_from_rows", "fp8_dequant_ref", "gather_paged", "commit_accepted_ref", "quantize_e4m3fn_ref",
    "greedy_accept_ref", "qk_norm_rope_ref", "philox4x32_10", "sample_uniforms_ref", "scaled_logits_ref",
    "sample_scores_ref", "sampled_accept_ref",
]
