"""GPU parity of the fused QK RMSNorm + RoPE (d2sd.qk_norm_rope, qk_rope.hip)
against the oracle (qk_norm_rope_ref, generation/verification.py:113-123).

Tolerance.  The only freedom is the fp32 summation order of the RMS
statistic (and the last bit of its reciprocal square root), which can move
the bf16 rounding of x / rms by one ulp; times the weight (< 2) and rounded
again, y = bf16(w * bf16(x / rms)) then moves by at most two ulps of y.  So:
after the norm, every element within two ulps of the oracle's; after the
rotation out_i = bf16(bf16(y_i c_i) + bf16(y_j s_i)) (j the rotation
partner, |c|, |s| <= 1), every element within four ulps of
max(|y_i|, |y_j|), the inputs' scale (each product moves by at most two ulps
of that scale plus its own rounding, and the sum can cancel); and in both
cases at least 99% of all elements bit-identical.
"""
import pytest
import torch

from oracle import cascade_oracle as orc
import d2sd

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _ulp(x):
    return torch.exp2(torch.floor(torch.log2(x.abs().clamp_min(1e-30))) - 7)


def _close(got, ref, scale, ulps, tag):
    """|got - ref| <= ulps * ulp(scale) elementwise, >= 99% identical."""
    got, ref = got.float().cpu(), ref.float()
    diff = (got - ref).abs()
    assert torch.isfinite(got).all(), tag
    bound = ulps * _ulp(scale.float())
    assert (diff <= bound + 1e-30).all(), f"{tag}: max diff / bound {(diff / bound).max().item():.2f}"
    same = (diff == 0).float().mean().item()
    assert same >= 0.99, f"{tag}: only {same:.4f} identical"


def _rope_scale(y):
    """max(|y_i|, |y_partner(i)|) with the partner i +- D/2."""
    half = y.shape[-1] // 2
    partner = torch.cat([y[..., half:], y[..., :half]], -1)
    return torch.maximum(y.float().abs(), partner.float().abs())


def _rope_table(T, D, half, g, base=1e6, offset=4000):
    pos = torch.arange(T) + offset + torch.randint(0, 50, (T,), generator=g)
    inv = 1.0 / (base ** (torch.arange(0, D, 2).float() / D))
    ang = pos[:, None].float() * inv[None]
    emb = ang if half else torch.cat([ang, ang], -1)
    return emb.cos().to(torch.bfloat16), emb.sin().to(torch.bfloat16)


@pytest.mark.parametrize("hq,hkv,d,norm,half", [(32, 8, 128, True, False),    # Qwen3-8B
                                                 (64, 8, 64, False, True),    # GPT-OSS-20B
                                                 (64, 8, 128, True, False),   # Qwen3-32B
                                                 (16, 4, 256, True, False),
                                                 (8, 2, 128, True, None)])    # norm only
def test_qk_norm_rope_matches_oracle(hq, hkv, d, norm, half):
    g = torch.Generator().manual_seed(hq + d)
    T = 150
    # q / k as strided views of one fused projection output [T, Hq + 2 Hkv, D]
    qkv = (torch.randn(T, hq + 2 * hkv, d, generator=g) * 2).to(torch.bfloat16)
    q, k = qkv[:, :hq], qkv[:, hq:hq + hkv]
    wq = (torch.rand(d, generator=g) + 0.5).to(torch.bfloat16) if norm else None
    wk = (torch.rand(d, generator=g) + 0.5).to(torch.bfloat16) if norm else None
    cos = sin = None
    if half is not None:
        cos, sin = _rope_table(T, d, half, g)
    dev = lambda t: None if t is None else t.to(DEV)
    y_q = orc.qk_norm_rope_ref(q, wq, None, None, 1e-6)
    y_k = orc.qk_norm_rope_ref(k, wk, None, None, 1e-6)
    if norm:
        # the norm alone
        q1, k1 = q.clone().to(DEV), k.clone().to(DEV)
        d2sd.qk_norm_rope(q1, k1, dev(wq), dev(wk), None, None, 1e-6)
        torch.cuda.synchronize()
        _close(q1, y_q, y_q, 2, "q norm")
        _close(k1, y_k, y_k, 2, "k norm")
    ref_q = orc.qk_norm_rope_ref(q, wq, cos, sin, 1e-6)
    ref_k = orc.qk_norm_rope_ref(k, wk, cos, sin, 1e-6)
    qkv_d = qkv.to(DEV)
    qd, kd = qkv_d[:, :hq], qkv_d[:, hq:hq + hkv]
    d2sd.qk_norm_rope(qd, kd, dev(wq), dev(wk), dev(cos), dev(sin), 1e-6)
    torch.cuda.synchronize()
    rope = half is not None
    _close(qd, ref_q, _rope_scale(y_q) if rope else y_q, 4 if rope else 2, "q")
    _close(kd, ref_k, _rope_scale(y_k) if rope else y_k, 4 if rope else 2, "k")
    # V (the rest of the fused buffer) is untouched
    assert torch.equal(qkv_d[:, hq + hkv:].cpu(), qkv[:, hq + hkv:])
