"""GPU parity of the device-side candidate-tree build (d2sd.tree.D3TreeBuilder,
tree_build.hip) against the host restatement d2sd.tree.d3_verify_tree
(generation/d3_generator.py:116-180): integer outputs and the ancestor mask,
bit-exact, over 240 seeded confidence vectors (half of them drawn from a
coarse set, so that equal rates occur), bf16 and fp32 confidences, and both
row layouts (block_size_2 > block_size and ==).  Also pins the restated rates
against the reference's own torch lines run on the GPU, and the top-k choice
against torch.topk where no tie sits at the boundary."""
import numpy as np
import pytest
import torch

import d2sd
from d2sd import tree as dtree

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _confs(n, count, seed):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        out.append(rng.uniform(size=n) if i % 2 else rng.choice([0.0, 0.25, 0.5, 0.75, 1.0, 0.9, 0.1], size=n))
    return out


def _torch_rates(conf):
    """generation/d3_generator.py:117-121 on the device."""
    cum_prod = torch.cumprod(conf, dim=0)
    rates = torch.empty(conf.shape[0], device=conf.device)
    rates[0] = 1.0 - conf[0]
    rates[1:] = cum_prod[:-1] * (1.0 - conf[1:])
    return rates


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("bs,bs2,k", [(16, 32, 4), (16, 16, 4), (8, 12, 3), (16, 32, 15)])
def test_device_tree_equals_host_tree(dtype, bs, bs2, k):
    builder = dtree.D3TreeBuilder(bs, bs2, k, DEV)
    tie_rows = 0
    for i, c in enumerate(_confs(bs - 1, 240, seed=bs * 100 + bs2 + k)):
        conf = torch.tensor(c, dtype=torch.float32).to(dtype).to(DEV)
        builder.build(conf)
        torch.cuda.synchronize()
        name = "bfloat16" if dtype == torch.bfloat16 else "float32"
        host = dtree.d3_verify_tree(conf.float().cpu().numpy(), bs, bs2, k, dtype=name)
        rates = dtree.d3_rejection_rates(conf.float().cpu().numpy(), name)
        assert np.array_equal(builder.rates.cpu().numpy().view(np.uint32), rates.view(np.uint32)), i
        dev = builder.host_tree()
        assert dev.num_nodes == host.num_nodes, i
        assert np.array_equal(dev.parents, host.parents), i
        assert np.array_equal(dev.node_index, host.node_index), i
        assert dev.shared == list(host.shared), i
        want = dtree.pack_mask_rows(dtree.padded_ancestor_mask(host, builder.capacity), builder.mask_words)
        assert np.array_equal(builder.tree_mask.cpu().numpy().view(np.uint64), want), i
        # padding rows repeat the DFlash row
        nr = host.num_rows
        dflash = host.node_index[nr - 1 if bs2 == bs else 0]
        for r in range(nr, builder.rows_cap):
            assert np.array_equal(builder.node_index[r].cpu().numpy(), dflash)
        srt = np.sort(rates)[::-1]
        tie_rows += int(len(srt) > k and srt[k - 1] == srt[k])
    assert tie_rows > 0 or k >= bs - 1   # ties at the top-k boundary were exercised


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_restated_rates_match_the_reference_lines_on_the_gpu(dtype):
    """d3_rejection_rates == the reference's torch lines executed on the GPU,
    bit for bit; the top-k set == sorted(torch.topk) when no tie sits at the
    4th / 5th rate."""
    name = "bfloat16" if dtype == torch.bfloat16 else "float32"
    checked = 0
    for i, c in enumerate(_confs(15, 300, seed=5)):
        conf = torch.tensor(c, dtype=torch.float32).to(dtype).to(DEV)
        ref = _torch_rates(conf).cpu().numpy()
        got = dtree.d3_rejection_rates(conf.float().cpu().numpy(), name)
        assert np.array_equal(ref.view(np.uint32), got.view(np.uint32)), (i, ref, got)
        srt = np.sort(ref)[::-1]
        if srt[3] != srt[4]:
            sel = sorted(torch.topk(torch.from_numpy(ref).to(DEV), 4).indices.tolist())
            assert sel == dtree.d3_select_boundaries(got, 4)
            checked += 1
    assert checked > 100


def test_device_tree_feeds_the_cascade_plan():
    """The builder writes the mask straight into a cascade plan made for its
    capacity; the attention then matches a plan made from the host tree on
    the rows of the real nodes."""
    from d2sd import workloads as wl
    from test_gpu_parity import check_close
    builder = dtree.D3TreeBuilder(16, 32, 4, DEV)
    cap = builder.capacity
    conf = torch.tensor(np.random.default_rng(1).uniform(size=15), dtype=torch.float32).to(torch.bfloat16).to(DEV)
    gen = torch.Generator(device=DEV).manual_seed(3)
    hq, hkv, d, L = 32, 8, 128, 700
    q = torch.randn(cap, hq, d, generator=gen, device=DEV).to(torch.bfloat16)
    ks = torch.randn(cap, hkv, d, generator=gen, device=DEV).to(torch.bfloat16)
    vs = torch.randn(cap, hkv, d, generator=gen, device=DEV).to(torch.bfloat16)
    kp = torch.randn(hkv, L, d, generator=gen, device=DEV).to(torch.bfloat16)
    vp = torch.randn(hkv, L, d, generator=gen, device=DEV).to(torch.bfloat16)
    attn = d2sd.CascadeVerifyAttention(DEV).plan([0, cap], [L], hq, hkv, d, tree_masks=[np.eye(cap, dtype=bool)],
                                                 kv_layout="HND")
    builder.build(conf, tree_mask=attn.tree_mask_dev)
    o, lse = attn.run(q, ks, vs, kp, vp)
    host = dtree.d3_verify_tree(conf.float().cpu().numpy())
    n = host.num_nodes
    ref = d2sd.CascadeVerifyAttention(DEV).plan([0, n], [L], hq, hkv, d, tree_masks=[host.ancestor_mask()],
                                                kv_layout="HND")
    o2, l2 = ref.run(q[:n].contiguous(), ks[:n].contiguous(), vs[:n].contiguous(), kp, vp)
    torch.cuda.synchronize()
    check_close(o[:n], o2.float().cpu(), lse[:n], l2.cpu(), "device tree vs host tree plan")
