"""One captured verify step replayed while the cache grows.

The step is what generation/d3_generator.py:196-232 runs per decoding step
after the drafts: the cascade verify attention of every layer
(verification.py:127-176), the greedy acceptance walk (d3_generator.py:204-225
at temperature 0) and the commit of the accepted branch into the cache
(d3_generator.py:227-232).  Here all three are captured once into a HipGraph:
the attention plan is a dynamic-prefix plan for the largest prefix of the next
steps, the commit reads the cache length from the plan's device array and
advances it by the accepted count, so every replay sees the cache the previous
one left.  Each replay is checked against the oracle at that step's length.
"""
import numpy as np
import pytest
import torch

from oracle import cascade_oracle as orc
import d2sd
from d2sd import tree as dtree

from test_gpu_parity import check_close
from test_gpu_accept import _drafts_following

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _rand(shape, gen):
    return torch.randn(shape, generator=gen, device=DEV).to(torch.bfloat16)


def test_step_graph_replays_as_prefix_grows():
    hq, hkv, d, P, layers, vocab = 32, 8, 128, 16, 2, 1000
    L0, steps = 1000, 4
    tr = dtree.d3_verify_tree(np.random.default_rng(3).uniform(size=15))
    N, rows, lb = tr.num_nodes, tr.num_rows, tr.row_len
    Lmax = L0 + steps * lb
    npages = (Lmax + P - 1) // P
    pool_pages = npages + 5
    gen = torch.Generator(device=DEV).manual_seed(7)
    kp = [_rand((pool_pages, hkv, P, d), gen) for _ in range(layers)]
    vp = [_rand((pool_pages, hkv, P, d), gen) for _ in range(layers)]
    table = torch.randperm(pool_pages, generator=gen, device=DEV)[:npages].to(torch.int32)
    q = [torch.empty(N, hq, d, dtype=torch.bfloat16, device=DEV) for _ in range(layers)]
    ks = [torch.empty(N, hkv, d, dtype=torch.bfloat16, device=DEV) for _ in range(layers)]
    vs = [torch.empty(N, hkv, d, dtype=torch.bfloat16, device=DEV) for _ in range(layers)]
    out = [torch.empty(N, hq, d, dtype=torch.bfloat16, device=DEV) for _ in range(layers)]
    lse = [torch.empty(N, hq, dtype=torch.float32, device=DEV) for _ in range(layers)]
    logits = torch.empty(N, vocab, dtype=torch.bfloat16, device=DEV)
    drafts = torch.empty(rows, lb, dtype=torch.int64, device=DEV)
    node_index = torch.as_tensor(tr.node_index, dtype=torch.int32, device=DEV)

    attn = d2sd.CascadeVerifyAttention(DEV).plan(
        [0, N], [Lmax], hq, hkv, d, tree_masks=[tr.ancestor_mask()], page_size=P, page_indptr=[0, npages],
        page_table=table, kv_layout="HND", dynamic_prefix=True)
    attn.set_prefix_len([L0])
    acc = d2sd.GreedyAccept(N, vocab, lb, DEV)
    commit = d2sd.PagedKVCommit(kp, vp, ks, vs)

    graph = d2sd.HipGraph()
    with graph.capture():
        for l in range(layers):
            attn.run(q[l], ks[l], vs[l], kp[l], vp[l], out=out[l], lse=lse[l])
        _, nodes, res = acc(logits, node_index, drafts)
        commit.commit(table, attn.prefix_len_dev[0:1], nodes, num_accepted=lb, num_accepted_dev=res, advance=True)

    hgen = torch.Generator().manual_seed(11)
    mask = torch.as_tensor(tr.ancestor_mask())
    pages = table.cpu().tolist()
    seen = set()
    for s, keep in enumerate(([4, 9, 0, 20, 2], [32, 1, 1, 1, 1], [0, 0, 0, 0, 0], [2, 30, 5, 5, 12])):
        for l in range(layers):
            q[l].copy_(_rand(q[l].shape, gen))
            ks[l].copy_(_rand(ks[l].shape, gen))
            vs[l].copy_(_rand(vs[l].shape, gen))
        lg = torch.randn(N, vocab, generator=hgen).to(torch.bfloat16)
        dr = _drafts_following(lg, node_index.cpu().long(), keep, hgen)
        logits.copy_(lg)
        drafts.copy_(dr)
        L = int(attn.prefix_len_dev[0])
        pool_before = [kp[0].clone(), vp[0].clone()]
        graph.replay()
        torch.cuda.synchronize()
        # attention at this step's prefix length
        for l in range(layers):
            kpre = orc.gather_paged(kp[l].cpu(), pages, L)
            vpre = orc.gather_paged(vp[l].cpu(), pages, L)
            o_ref, lse_ref = orc.cascade_tree_ref(q[l].cpu(), ks[l].cpu(), vs[l].cpu(), kpre, vpre, mask,
                                                  d ** -0.5)
            check_close(out[l], o_ref, lse[l], lse_ref, f"step {s} layer {l} (prefix {L})")
        # acceptance and the commit of its branch
        ids, acc_nodes, n, vb = orc.greedy_accept_ref(lg.float(), node_index.cpu(), dr)
        assert res.cpu().tolist() == [n, vb]
        assert int(attn.prefix_len_dev[0]) == L + n
        seen.add(n)
        for l in range(layers):
            for pool, new in ((kp[l], ks[l]), (vp[l], vs[l])):
                got = orc.gather_paged(pool.cpu(), pages, L + n)[L:]
                assert torch.equal(got, new.cpu()[acc_nodes]), f"step {s} layer {l}: committed rows differ"
        # nothing else of the pool changed
        for pool, before in zip((kp[0], vp[0]), pool_before):
            changed = (pool != before).flatten(1).any(1).nonzero().flatten().tolist()
            allowed = {pages[t // P] for t in range(L, L + n)}
            assert set(changed) <= allowed
    assert len(seen) >= 3  # the steps accepted different lengths


def test_step_graph_with_device_tree_build():
    """The whole verify step without a host round trip: the candidate tree of
    the step's draft confidences is built on the device (D3TreeBuilder, the
    host top-k of d3_generator.py:116-125 included) into the mask buffer of a
    cascade plan made for the largest tree, then attention, acceptance and
    commit as above, all in one graph replayed over steps with new
    confidences (new trees).  Every step is checked against the oracle on the
    host tree of the same confidences."""
    hq, hkv, d, P, layers, vocab = 32, 8, 128, 16, 2, 1000
    L0, steps = 900, 4
    builder = dtree.D3TreeBuilder(16, 32, 4, DEV)
    cap, rows, lb = builder.capacity, builder.rows_cap, builder.block_size_2
    Lmax = L0 + steps * lb
    npages = (Lmax + P - 1) // P
    pool_pages = npages + 3
    gen = torch.Generator(device=DEV).manual_seed(17)
    kp = [_rand((pool_pages, hkv, P, d), gen) for _ in range(layers)]
    vp = [_rand((pool_pages, hkv, P, d), gen) for _ in range(layers)]
    table = torch.randperm(pool_pages, generator=gen, device=DEV)[:npages].to(torch.int32)
    q = [torch.empty(cap, hq, d, dtype=torch.bfloat16, device=DEV) for _ in range(layers)]
    ks = [torch.empty(cap, hkv, d, dtype=torch.bfloat16, device=DEV) for _ in range(layers)]
    vs = [torch.empty(cap, hkv, d, dtype=torch.bfloat16, device=DEV) for _ in range(layers)]
    out = [torch.empty(cap, hq, d, dtype=torch.bfloat16, device=DEV) for _ in range(layers)]
    lse = [torch.empty(cap, hq, dtype=torch.float32, device=DEV) for _ in range(layers)]
    logits = torch.empty(cap, vocab, dtype=torch.bfloat16, device=DEV)
    drafts = torch.empty(rows, lb, dtype=torch.int64, device=DEV)
    conf = torch.empty(15, dtype=torch.bfloat16, device=DEV)

    attn = d2sd.CascadeVerifyAttention(DEV).plan(
        [0, cap], [Lmax], hq, hkv, d, tree_masks=[np.eye(cap, dtype=bool)], page_size=P,
        page_indptr=[0, npages], page_table=table, kv_layout="HND", dynamic_prefix=True)
    attn.set_prefix_len([L0])
    acc = d2sd.GreedyAccept(cap, vocab, lb, DEV)
    commit = d2sd.PagedKVCommit(kp, vp, ks, vs)
    graph = d2sd.HipGraph()
    with graph.capture():
        builder.build(conf, tree_mask=attn.tree_mask_dev)
        for l in range(layers):
            attn.run(q[l], ks[l], vs[l], kp[l], vp[l], out=out[l], lse=lse[l])
        _, nodes, res = acc(logits, builder.node_index, drafts)
        commit.commit(table, attn.prefix_len_dev[0:1], nodes, num_accepted=lb, num_accepted_dev=res, advance=True)

    hgen = torch.Generator().manual_seed(19)
    rng = np.random.default_rng(23)
    pages = table.cpu().tolist()
    seen_nodes = set()
    for s, keep in enumerate(([5, 9, 0, 20, 2], [32, 1, 1, 1, 1], [0, 0, 0, 0, 0], [2, 30, 5, 5, 12])):
        c = torch.tensor(rng.uniform(size=15), dtype=torch.float32).to(torch.bfloat16)
        host = dtree.d3_verify_tree(c.float().numpy())
        seen_nodes.add(host.num_nodes)
        ni = np.concatenate([host.node_index] + [host.node_index[:1]] * (rows - host.num_rows))  # padded rows
        for l in range(layers):
            q[l].copy_(_rand(q[l].shape, gen))
            ks[l].copy_(_rand(ks[l].shape, gen))
            vs[l].copy_(_rand(vs[l].shape, gen))
        lg = torch.randn(cap, vocab, generator=hgen).to(torch.bfloat16)
        dr = _drafts_following(lg, torch.as_tensor(ni, dtype=torch.long), keep, hgen)
        dr[host.num_rows:] = dr[0]          # padded rows repeat the DFlash row's drafts
        conf.copy_(c)
        logits.copy_(lg)
        drafts.copy_(dr)
        L = int(attn.prefix_len_dev[0])
        graph.replay()
        torch.cuda.synchronize()
        assert int(builder.num_nodes[0]) == host.num_nodes
        assert np.array_equal(builder.node_index.cpu().numpy(), ni)
        n_nodes = host.num_nodes
        mask = torch.as_tensor(host.ancestor_mask())
        for l in range(layers):
            kpre = orc.gather_paged(kp[l].cpu(), pages, L)
            vpre = orc.gather_paged(vp[l].cpu(), pages, L)
            o_ref, lse_ref = orc.cascade_tree_ref(q[l].cpu()[:n_nodes], ks[l].cpu()[:n_nodes], vs[l].cpu()[:n_nodes],
                                                  kpre, vpre, mask, d ** -0.5)
            check_close(out[l][:n_nodes], o_ref, lse[l][:n_nodes], lse_ref, f"step {s} layer {l} (prefix {L})")
        ids, acc_nodes, n, vb = orc.greedy_accept_ref(lg.float(), ni, dr)
        assert res.cpu().tolist() == [n, vb]
        assert int(attn.prefix_len_dev[0]) == L + n
        for l in range(layers):
            got = orc.gather_paged(kp[l].cpu(), pages, L + n)[L:]
            assert torch.equal(got, ks[l].cpu()[acc_nodes])
    assert len(seen_nodes) >= 2   # the steps built different trees
