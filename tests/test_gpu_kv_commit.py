"""GPU parity of the accepted-branch KV commit (d2sd.PagedKVCommit, kv_append.hip)
against the oracle (commit_accepted_ref, generation/d3_generator.py:227-232).

A byte copy: the kernel's pools must equal the oracle's bit for bit.
"""
import numpy as np
import pytest
import torch

from oracle import cascade_oracle as orc
import d2sd
from d2sd import tree as dtree

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _setup(layers, pool_pages, P, hkv, d, rows, layout, seed):
    g = torch.Generator().manual_seed(seed)
    shape = (pool_pages, hkv, P, d) if layout == "HND" else (pool_pages, P, hkv, d)
    kp = [torch.randn(shape, generator=g).to(torch.bfloat16) for _ in range(layers)]
    vp = [torch.randn(shape, generator=g).to(torch.bfloat16) for _ in range(layers)]
    kn = [torch.randn(rows, hkv, d, generator=g).to(torch.bfloat16) for _ in range(layers)]
    vn = [torch.randn(rows, hkv, d, generator=g).to(torch.bfloat16) for _ in range(layers)]
    return g, kp, vp, kn, vn


@pytest.mark.parametrize("layout", ["HND", "NHD"])
@pytest.mark.parametrize("L,n,P,hkv,d", [(0, 1, 16, 8, 128), (4095, 32, 16, 8, 128), (100, 17, 16, 8, 64),
                                          (5, 31, 4, 2, 128), (64, 0, 16, 8, 128), (7, 3, 1, 1, 8)])
def test_commit_matches_oracle(layout, L, n, P, hkv, d):
    layers, rows = 3, 40
    pages_needed = max(1, (L + n + P - 1) // P)
    pool_pages = pages_needed + 5
    g, kp, vp, kn, vn = _setup(layers, pool_pages, P, hkv, d, rows, layout, seed=L + 7 * n)
    table = torch.randperm(pool_pages, generator=g)[:pages_needed].to(torch.int32)
    nodes = torch.randint(0, rows, (max(n, 1),), generator=g, dtype=torch.int32)
    if n > 2:
        nodes[1] = -1      # skipped: writes nothing
        nodes[2] = rows    # skipped
    exp_k = [orc.commit_accepted_ref(kp[l], table.tolist(), L, kn[l], nodes[:n].tolist(), layout) for l in range(layers)]
    exp_v = [orc.commit_accepted_ref(vp[l], table.tolist(), L, vn[l], nodes[:n].tolist(), layout) for l in range(layers)]
    kpd = [t.to(DEV) for t in kp]
    vpd = [t.to(DEV) for t in vp]
    knd = [t.to(DEV) for t in kn]
    vnd = [t.to(DEV) for t in vn]
    c = d2sd.PagedKVCommit(kpd, vpd, knd, vnd, kv_layout=layout)
    c.commit(table.to(DEV), L, nodes.to(DEV), num_accepted=n)
    torch.cuda.synchronize()
    for l in range(layers):
        assert torch.equal(kpd[l].cpu(), exp_k[l]), f"layer {l} K"
        assert torch.equal(vpd[l].cpu(), exp_v[l]), f"layer {l} V"


def test_commit_of_a_d3_branch_at_full_size_equals_cat():
    """Qwen3-8B shape, 36 layers, L = 4096 paged at 16: committing an accepted
    branch of a d3 verify tree (its first acceptance_length node rows) is the
    reference's torch.cat of that row's new K/V (d3_generator.py:228-231)."""
    layers, P, hkv, d, L = 36, 16, 8, 128, 4096
    tr = dtree.d3_verify_tree(np.random.default_rng(0).uniform(size=15))
    rows = tr.num_nodes
    valid_block, acc = 1, 20
    nodes = torch.as_tensor(tr.node_index[valid_block][:acc], dtype=torch.int32)
    pages_needed = (L + acc + P - 1) // P
    pool_pages = pages_needed + 8
    g = torch.Generator().manual_seed(3)
    kpd = [torch.randn(pool_pages, hkv, P, d, generator=g).to(torch.bfloat16).to(DEV) for _ in range(layers)]
    vpd = [torch.randn(pool_pages, hkv, P, d, generator=g).to(torch.bfloat16).to(DEV) for _ in range(layers)]
    knd = [torch.randn(rows, hkv, d, generator=g).to(torch.bfloat16).to(DEV) for _ in range(layers)]
    vnd = [torch.randn(rows, hkv, d, generator=g).to(torch.bfloat16).to(DEV) for _ in range(layers)]
    table = torch.randperm(pool_pages, generator=g)[:pages_needed].to(torch.int32)
    before_k = [orc.gather_paged(t.cpu(), table.tolist(), L) for t in kpd[:3] + kpd[-1:]]
    c = d2sd.PagedKVCommit(kpd, vpd, knd, vnd)
    c.commit(table.to(DEV), L, nodes.to(DEV))
    torch.cuda.synchronize()
    for j, l in enumerate([0, 1, 2, layers - 1]):
        after = orc.gather_paged(kpd[l].cpu(), table.tolist(), L + acc)
        assert torch.equal(after, torch.cat([before_k[j], knd[l].cpu()[nodes.long()]], 0)), f"layer {l}"


def test_commit_replays_in_a_graph():
    """Captured once, replayed with new node ids in the same device buffer."""
    layers, P, hkv, d, L, n, rows = 2, 16, 8, 128, 30, 8, 16
    g, kp, vp, kn, vn = _setup(layers, 8, P, hkv, d, rows, "HND", seed=11)
    kpd = [t.to(DEV) for t in kp]
    vpd = [t.to(DEV) for t in vp]
    knd = [t.to(DEV) for t in kn]
    vnd = [t.to(DEV) for t in vn]
    table = torch.arange(4, dtype=torch.int32, device=DEV)
    nodes = torch.zeros(n, dtype=torch.int32, device=DEV)
    c = d2sd.PagedKVCommit(kpd, vpd, knd, vnd)
    graph = d2sd.HipGraph()
    with graph.capture():
        c.commit(table, L, nodes)
    for rep in range(3):
        ids = torch.randperm(rows, generator=g)[:n].to(torch.int32)
        nodes.copy_(ids.to(DEV))
        torch.cuda.synchronize()
        ref = [orc.commit_accepted_ref(kpd[l].cpu(), table.tolist(), L, kn[l], ids.tolist()) for l in range(layers)]
        graph.replay()
        torch.cuda.synchronize()
        for l in range(layers):
            assert torch.equal(kpd[l].cpu(), ref[l]), f"replay {rep} layer {l}"


# ---- fp8 e4m3fn pools (the cascade kernels' fp8 format, value / scale) ----

def _every_bf16(rows, hkv, d):
    bits = torch.arange(65536, dtype=torch.int32).to(torch.int16)
    return bits.view(torch.bfloat16).view(rows, hkv, d)


def test_fp8_commit_quantises_every_bf16_value_like_the_oracle():
    """All 65536 bf16 bit patterns (infinities and NaNs of both signs
    included) committed into an fp8 pool, kv head 0 at scale 1 (the cast
    alone) and head 1 at 0.37 (the fp32 quotient first): every byte equals the
    oracle's (a NaN stays the NaN byte 0x7F with its sign, an infinity
    saturates at +-448)."""
    hkv, d, P = 2, 128, 16
    rows = 65536 // (hkv * d)
    new = _every_bf16(rows, hkv, d)
    assert torch.isnan(new).any() and torch.isinf(new).any()
    pages = rows // P
    g = torch.Generator().manual_seed(3)
    pool = (torch.randn(pages + 2, hkv, P, d, generator=g)).to(torch.float8_e4m3fn)
    scale = torch.tensor([1.0, 0.37], dtype=torch.float32)
    table = torch.randperm(pages + 2, generator=g)[:pages].to(torch.int32)
    nodes = torch.arange(rows, dtype=torch.int32)
    exp = orc.commit_accepted_ref(pool, table.tolist(), 0, new, nodes.tolist(), "HND", scale)
    kpd, vpd = pool.to(DEV), pool.clone().to(DEV)
    c = d2sd.PagedKVCommit([kpd], [vpd], [new.to(DEV)], [new.to(DEV)], k_scales=scale.to(DEV),
                           v_scales=scale.to(DEV))
    c.commit(table.to(DEV), 0, nodes.to(DEV))
    torch.cuda.synchronize()
    for name, got in (("K", kpd), ("V", vpd)):
        diff = (got.cpu().view(torch.uint8) != exp.view(torch.uint8))
        assert not diff.any(), f"{name}: {int(diff.sum())} bytes differ"


@pytest.mark.parametrize("layout", ["HND", "NHD"])
def test_fp8_commit_matches_oracle_with_per_layer_scales(layout):
    layers, P, hkv, d, L, n, rows = 3, 16, 8, 128, 37, 21, 40
    pages_needed = (L + n + P - 1) // P
    pool_pages = pages_needed + 4
    g, kp, vp, kn, vn = _setup(layers, pool_pages, P, hkv, d, rows, layout, seed=5)
    kp = [t.to(torch.float8_e4m3fn) for t in kp]
    vp = [t.to(torch.float8_e4m3fn) for t in vp]
    ks = [torch.rand(hkv, generator=g) * 0.02 + 0.001 for _ in range(layers)]   # large quotients saturate
    vs = [torch.rand(hkv, generator=g) * 0.5 + 0.01 for _ in range(layers)]
    table = torch.randperm(pool_pages, generator=g)[:pages_needed].to(torch.int32)
    nodes = torch.randint(0, rows, (n,), generator=g, dtype=torch.int32)
    exp_k = [orc.commit_accepted_ref(kp[l], table.tolist(), L, kn[l], nodes.tolist(), layout, ks[l]) for l in range(layers)]
    exp_v = [orc.commit_accepted_ref(vp[l], table.tolist(), L, vn[l], nodes.tolist(), layout, vs[l]) for l in range(layers)]
    kpd = [t.to(DEV) for t in kp]
    vpd = [t.to(DEV) for t in vp]
    c = d2sd.PagedKVCommit(kpd, vpd, [t.to(DEV) for t in kn], [t.to(DEV) for t in vn], kv_layout=layout,
                           k_scales=[s.to(DEV) for s in ks], v_scales=[s.to(DEV) for s in vs])
    c.commit(table.to(DEV), L, nodes.to(DEV))
    torch.cuda.synchronize()
    for l in range(layers):
        assert torch.equal(kpd[l].cpu().view(torch.uint8), exp_k[l].view(torch.uint8)), f"layer {l} K"
        assert torch.equal(vpd[l].cpu().view(torch.uint8), exp_v[l].view(torch.uint8)), f"layer {l} V"


def test_fp8_commit_then_cascade_reads_it_back():
    """Qwen3-32B heads (64/8, D 128) over an fp8 paged prefix with per-kv-head
    scales: commit an accepted branch of a d3 tree into the fp8 pool, then run
    the next step's cascade attention over the grown prefix; the result
    matches the oracle on the dequantised pool (the commit writes the format
    the attention reads)."""
    hq, hkv, d, P, L0 = 64, 8, 128, 16, 300
    tr = dtree.d3_verify_tree(np.random.default_rng(2).uniform(size=15))
    N = tr.num_nodes
    n = 20
    pages = (L0 + n + P - 1) // P
    g = torch.Generator().manual_seed(11)
    kf = torch.randn(pages + 3, hkv, P, d, generator=g)
    vf = torch.randn(pages + 3, hkv, P, d, generator=g)
    ks = (kf.abs().amax(dim=(0, 2, 3)) / 448.0).float()
    vs = (vf.abs().amax(dim=(0, 2, 3)) / 448.0).float()
    kpool = (kf / ks[None, :, None, None]).to(torch.float8_e4m3fn).to(DEV)
    vpool = (vf / vs[None, :, None, None]).to(torch.float8_e4m3fn).to(DEV)
    table = torch.randperm(pages + 3, generator=g)[:pages].to(torch.int32).to(DEV)
    kn = torch.randn(N, hkv, d, generator=g).to(torch.bfloat16).to(DEV)
    vn = torch.randn(N, hkv, d, generator=g).to(torch.bfloat16).to(DEV)
    nodes = torch.as_tensor(tr.node_index[1, :n], dtype=torch.int32, device=DEV)
    c = d2sd.PagedKVCommit([kpool], [vpool], [kn], [vn], k_scales=ks.to(DEV), v_scales=vs.to(DEV))
    c.commit(table, L0, nodes)
    L = L0 + n
    q = torch.randn(N, hq, d, generator=g).to(torch.bfloat16).to(DEV)
    ks2 = torch.randn(N, hkv, d, generator=g).to(torch.bfloat16).to(DEV)
    vs2 = torch.randn(N, hkv, d, generator=g).to(torch.bfloat16).to(DEV)
    attn = d2sd.CascadeVerifyAttention(DEV).plan(
        [0, N], [L], hq, hkv, d, tree_masks=[tr.ancestor_mask()], page_size=P, page_indptr=[0, pages],
        page_table=table, kv_layout="HND", kv_dtype=torch.float8_e4m3fn, k_scale=ks.to(DEV), v_scale=vs.to(DEV))
    o, lse = attn.run(q, ks2, vs2, kpool, vpool)
    torch.cuda.synchronize()
    pl = table.cpu().tolist()
    kp = orc.gather_paged(kpool.cpu(), pl, L).float() * ks[None, :, None]
    vp = orc.gather_paged(vpool.cpu(), pl, L).float() * vs[None, :, None]
    # the committed rows read back as the quantised new rows
    assert torch.equal(kp[L0:], orc.quantize_e4m3fn_ref(kn.cpu()[nodes.cpu().long()], ks).float() * ks[None, :, None])
    o_ref, lse_ref = orc.cascade_tree_ref(q.cpu(), ks2.cpu(), vs2.cpu(), kp, vp, torch.as_tensor(tr.ancestor_mask()),
                                          d ** -0.5)
    from test_gpu_parity import check_close
    check_close(o, o_ref, lse, lse_ref, "fp8 commit then cascade")
