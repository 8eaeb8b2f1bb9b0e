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
