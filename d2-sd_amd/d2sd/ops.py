"""FlashInfer-compatible entry points used by the reference's verify path.

    single_prefill_with_kv_cache  <- flashinfer.single_prefill_with_kv_cache
                                     (generation/verification.py:145, 159;
                                      model/cascade_graph.py:54; model/dflash.py:112, 127)
    merge_state_in_place          <- flashinfer.merge_state_in_place
                                     (generation/verification.py:163;
                                      model/cascade_graph.py:58; model/dflash.py:131)
    merge_state                   <- flashinfer.merge_state (out-of-place form)

Same names, argument meaning and return convention as the FlashInfer calls the
reference makes; every call goes through the torch operators torch.ops.d2sd.*
(libd2sd_torch.so) to the gfx950 kernels of libd2sd.so on the current HIP
stream.  The returned LSE is the natural logarithm of the softmax
denominator (pass lse_base2=True for base 2).
"""
from __future__ import annotations

import ctypes as C
from typing import Optional, Tuple, Union

import torch

from . import _lib
from ._lib import check, lib


def _stream() -> C.c_void_p:
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def _need_device(*ts: torch.Tensor) -> None:
    for t in ts:
        if not t.is_cuda:
            raise ValueError("d2sd kernels need ROCm device tensors (got a CPU tensor)")


def _need_bf16(*ts: torch.Tensor) -> None:
    for t in ts:
        if t.dtype != torch.bfloat16:
            raise TypeError(f"d2sd kernels take bfloat16 q/k/v/o (got {t.dtype})")


def _need_rows(name: str, t: torch.Tensor) -> None:
    if t.dim() != 3 or t.stride(-1) != 1:
        raise ValueError(f"{name} must be 3-D with a contiguous last dimension, got shape "
                         f"{tuple(t.shape)} strides {t.stride()}")


def single_prefill_with_kv_cache(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    custom_mask: Optional[torch.Tensor] = None,
    packed_custom_mask: Optional[torch.Tensor] = None,
    causal: bool = False,
    kv_layout: str = "NHD",
    pos_encoding_mode: str = "NONE",
    use_fp16_qk_reduction: bool = False,
    sm_scale: Optional[float] = None,
    window_left: int = -1,
    logits_soft_cap: Optional[float] = None,
    rope_scale: Optional[float] = None,
    rope_theta: Optional[float] = None,
    return_lse: bool = False,
    lse_base2: bool = False,
) -> Union[torch.Tensor, Tuple[torch.Tensor, torch.Tensor]]:
    """Attention of q [qo_len, Hq, D] over k, v [kv_len, Hkv, D] (kv_layout
    "NHD") or [Hkv, kv_len, D] ("HND"), GQA head map h -> h // (Hq // Hkv).

    causal=True keeps key j for query i iff j <= i + kv_len - qo_len.
    Returns out (q's shape, bf16) or (out, lse [qo_len, Hq] fp32).
    """
    if custom_mask is not None or packed_custom_mask is not None:
        raise NotImplementedError("custom masks: use CascadeVerifyAttention (tree mask)")
    if pos_encoding_mode != "NONE" or logits_soft_cap not in (None, 0.0) or rope_scale or rope_theta:
        raise NotImplementedError("only pos_encoding_mode='NONE' without soft-cap is supported")
    if window_left != -1:
        raise NotImplementedError("window_left: use CascadeVerifyAttention(window_left=...)")
    if use_fp16_qk_reduction:
        raise NotImplementedError("use_fp16_qk_reduction")
    _need_device(q, k, v)
    _need_bf16(q, k, v)
    _need_rows("q", q)
    _need_rows("k", k)
    _need_rows("v", v)
    if k.stride() != v.stride() or k.shape != v.shape:
        raise ValueError("k and v must have the same shape and strides")
    qo_len, hq, d = q.shape
    if kv_layout == "NHD":
        kv_len, hkv, dk = k.shape
        s_n, s_h = k.stride(0), k.stride(1)
    elif kv_layout == "HND":
        hkv, kv_len, dk = k.shape
        s_n, s_h = k.stride(1), k.stride(0)
    else:
        raise ValueError(f"kv_layout must be 'NHD' or 'HND', got {kv_layout!r}")
    if dk != d:
        raise ValueError("q and k head_dim differ")
    if sm_scale is None:
        sm_scale = d ** -0.5
    out, lse = torch.ops.d2sd.single_prefill_with_kv_cache(q, k, v, bool(causal), kv_layout, float(sm_scale),
                                                           bool(lse_base2))
    return (out, lse) if return_lse else out


def merge_state_in_place(v: torch.Tensor, s: torch.Tensor, v_other: torch.Tensor, s_other: torch.Tensor,
                         mask: Optional[torch.Tensor] = None, lse_base2: bool = False) -> None:
    """v [n, H, D] bf16 and s [n, H] fp32 become the merge of (v, s) and
    (v_other, s_other): s' = logaddexp(s, s_other),
    v' = v*exp(s - s') + v_other*exp(s_other - s')."""
    if mask is not None:
        raise NotImplementedError("merge_state_in_place(mask=...)")
    _need_device(v, s, v_other, s_other)
    _need_bf16(v, v_other)
    _need_rows("v", v)
    _need_rows("v_other", v_other)
    if v.shape != v_other.shape or s.shape != v.shape[:2] or s_other.shape != v.shape[:2]:
        raise ValueError("merge_state_in_place: shape mismatch")
    if s.dtype != torch.float32 or s_other.dtype != torch.float32:
        raise TypeError("merge_state_in_place: s and s_other must be float32")
    if s.stride(1) != 1 or s_other.stride(1) != 1:
        raise ValueError("merge_state_in_place: s / s_other need a contiguous head dimension")
    torch.ops.d2sd.merge_state_in_place(v, s, v_other, s_other, bool(lse_base2))


def merge_state(v_a: torch.Tensor, s_a: torch.Tensor, v_b: torch.Tensor, s_b: torch.Tensor,
                lse_base2: bool = False) -> Tuple[torch.Tensor, torch.Tensor]:
    """Out-of-place merge of two attention states; returns (v, s)."""
    v = v_a.clone()
    s = s_a.clone()
    merge_state_in_place(v, s, v_b, s_b, lse_base2=lse_base2)
    return v, s


def local_attention_merge(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, out: torch.Tensor,
                          lse: torch.Tensor, causal: bool, sm_scale: float,
                          sinks: Optional[torch.Tensor] = None, lse_base2: bool = False) -> None:
    """One launch of the per-row local attention + in-place merge loop of
    model/cascade_graph.py:52-60: q/out [bsz, Lb, Hq, D], k/v [bsz, Lb, Hkv, D],
    lse [bsz, Lb, Hq]; out/lse are updated in place."""
    _need_device(q, k, v, out, lse)
    _need_bf16(q, k, v, out)
    if q.dim() != 4 or k.dim() != 4 or out.shape != q.shape or k.shape != v.shape:
        raise ValueError("local_attention_merge: q/out [bsz, Lb, Hq, D], k/v [bsz, Lb, Hkv, D]")
    if k.stride() != v.stride() or q.stride(-1) != 1 or k.stride(-1) != 1 or out.stride(-1) != 1:
        raise ValueError("local_attention_merge: contiguous head_dim and equal k/v strides required")
    if lse.dtype != torch.float32 or lse.shape != q.shape[:3] or lse.stride(-1) != 1:
        raise ValueError("local_attention_merge: lse must be float32 [bsz, Lb, Hq] with contiguous heads")
    bsz, lb, hq, d = q.shape
    hkv = k.shape[2]
    if k.shape[0] != bsz or k.shape[1] != lb or k.shape[3] != d:
        raise ValueError("local_attention_merge: k/v shape mismatch")
    if sinks is not None:
        if sinks.dtype != torch.float32 or sinks.numel() != hq or not sinks.is_contiguous():
            raise ValueError("sinks must be a contiguous float32 [Hq] tensor")
    torch.ops.d2sd.local_attention_merge(q, k, v, out, lse, bool(causal), float(sm_scale), sinks,
                                         bool(lse_base2))


__all__ = ["single_prefill_with_kv_cache", "merge_state_in_place", "merge_state", "local_attention_merge"]
_ = _lib


def qk_norm_rope(q: torch.Tensor, k: torch.Tensor, q_norm: Optional[torch.Tensor] = None,
                 k_norm: Optional[torch.Tensor] = None, cos: Optional[torch.Tensor] = None,
                 sin: Optional[torch.Tensor] = None, eps: float = 1e-6) -> Tuple[torch.Tensor, torch.Tensor]:
    """Per-head RMSNorm (weights q_norm / k_norm, bf16 [D]) then rotary
    embedding (cos / sin bf16 [tokens, D], or [tokens, D/2] for the GPT-OSS
    form), in place on q [tokens, Hq, D] and k [tokens, Hkv, D] (bf16).
    Replaces generation/verification.py:113-123 (q_norm / k_norm, transposes,
    _apply_rotary_pos_emb_qwen3 / _gpt_oss) with the same bf16 rounding
    steps; returns (q, k)."""
    if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16:
        raise TypeError("q and k must be bf16")
    if q.dim() != 3 or k.dim() != 3 or q.shape[0] != k.shape[0] or q.shape[2] != k.shape[2]:
        raise ValueError("q [tokens, Hq, D] and k [tokens, Hkv, D] with one token count and head_dim")
    if q.stride(2) != 1 or k.stride(2) != 1:
        raise ValueError("head_dim must be contiguous")
    d = q.shape[2]
    a = _lib.QkRopeArgs()
    a.q, a.k = q.data_ptr(), k.data_ptr()
    a.q_stride_n, a.q_stride_h = q.stride(0), q.stride(1)
    a.k_stride_n, a.k_stride_h = k.stride(0), k.stride(1)
    for name, w in (("q_norm", q_norm), ("k_norm", k_norm)):
        if w is not None:
            if w.dtype != torch.bfloat16 or w.numel() != d or not w.is_contiguous():
                raise ValueError(f"{name} must be a contiguous bf16 [head_dim] weight")
            setattr(a, name, w.data_ptr())
    if (cos is None) != (sin is None):
        raise ValueError("cos and sin go together")
    if cos is not None:
        if cos.dtype != torch.bfloat16 or sin.dtype != torch.bfloat16 or cos.shape != sin.shape:
            raise ValueError("cos / sin must be bf16 of one shape")
        if cos.dim() != 2 or cos.shape[0] != q.shape[0] or cos.shape[1] not in (d, d // 2):
            raise ValueError("cos / sin must be [tokens, head_dim] or [tokens, head_dim / 2]")
        if cos.stride(1) != 1 or sin.stride() != cos.stride():
            raise ValueError("cos / sin rows must be contiguous with one stride")
        a.cos, a.sin, a.cs_stride = cos.data_ptr(), sin.data_ptr(), cos.stride(0)
        a.half_cos = 1 if cos.shape[1] == d // 2 else 0
    a.eps = float(eps)
    a.num_tokens, a.num_qo_heads, a.num_kv_heads, a.head_dim = q.shape[0], q.shape[1], k.shape[1], d
    check(lib.d2sd_qk_norm_rope(C.byref(a), _stream()), "qk_norm_rope")
    return q, k
