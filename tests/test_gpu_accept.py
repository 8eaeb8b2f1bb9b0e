"""GPU parity of the greedy acceptance walk (d2sd.GreedyAccept, accept.hip)
against the oracle (greedy_accept_ref, generation/d3_generator.py:204-225 at
temperature 0).  Integer outputs: exact equality."""
import numpy as np
import pytest
import torch

from oracle import cascade_oracle as orc
import d2sd
from d2sd import tree as dtree

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _drafts_following(node_logits, node_index, keep, gen):
    """Draft tokens per (row, position): row r repeats the target's argmax
    chain for its first keep[r] positions, then random tokens."""
    am = node_logits.float().argmax(-1)
    rows, lb = node_index.shape
    d = torch.randint(0, node_logits.shape[1], (rows, lb), generator=gen)
    for r in range(rows):
        for p in range(1, min(keep[r], lb)):
            d[r, p] = am[node_index[r, p - 1]]
    return d


def _check(node_logits, node_index, drafts):
    ids, nodes, n, vb = orc.greedy_accept_ref(node_logits.float(), node_index, drafts)
    acc = d2sd.GreedyAccept(node_logits.shape[0], node_logits.shape[1], node_index.shape[1], DEV)
    g_ids, g_nodes, g_res = acc(node_logits.to(DEV), torch.as_tensor(node_index, dtype=torch.int32).to(DEV),
                                torch.as_tensor(drafts, dtype=torch.int64).to(DEV))
    torch.cuda.synchronize()
    res = g_res.cpu().tolist()
    assert res == [n, vb], (res, n, vb)
    assert g_ids.cpu()[:n].tolist() == ids and g_nodes.cpu()[:n].tolist() == nodes
    return n, vb


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("vocab", [151936, 32000, 1001, 7])
def test_accept_matches_oracle_on_d3_trees(dtype, vocab):
    gen = torch.Generator().manual_seed(vocab)
    tr = dtree.d3_verify_tree(np.random.default_rng(vocab).uniform(size=15))
    node_index = torch.as_tensor(tr.node_index, dtype=torch.long)
    logits = torch.randn(tr.num_nodes, vocab, generator=gen).to(dtype)
    lengths = set()
    for keep in ([32, 32, 32, 32, 32], [3, 9, 0, 20, 1], [0, 0, 0, 0, 0], [1, 17, 17, 5, 30]):
        drafts = _drafts_following(logits, node_index, keep, gen)
        n, _ = _check(logits, node_index, drafts)
        lengths.add(n)
    assert len(lengths) >= 3  # the cases reach different acceptance lengths


def test_accept_ties_take_the_first_index():
    gen = torch.Generator().manual_seed(5)
    node_index = torch.tensor([[0, 1, 2, 3]])
    logits = torch.randn(4, 5000, generator=gen).to(torch.bfloat16)
    for j, (a, b) in enumerate([(10, 4000), (2500, 2501), (0, 4999), (777, 3333)]):
        logits[j, a] = logits[j, b] = 50.0       # exact bf16 ties, far above the rest
    am = [10, 2500, 0, 777]
    drafts = torch.tensor([[0, am[0], am[1], am[2]]])
    n, _ = _check(logits, node_index, drafts)
    assert n == 4


def test_accept_then_commit_in_one_graph():
    """The walk's outputs feed the KV commit on the device (no host sync):
    captured once, replayed; the pools equal the oracle commit of the
    oracle's accepted nodes."""
    gen = torch.Generator().manual_seed(9)
    tr = dtree.d3_verify_tree(np.random.default_rng(9).uniform(size=15))
    node_index = torch.as_tensor(tr.node_index, dtype=torch.long)
    N, lb, V = tr.num_nodes, tr.node_index.shape[1], 4096
    logits = torch.randn(N, V, generator=gen).to(torch.bfloat16)
    drafts = _drafts_following(logits, node_index, [2, 12, 5, 0, 7], gen)
    ids, nodes, n, vb = orc.greedy_accept_ref(logits.float(), node_index, drafts)
    layers, P, hkv, d, L = 2, 16, 8, 128, 100
    pages = (L + lb + P - 1) // P
    kp = [torch.randn(pages + 2, hkv, P, d, generator=gen).to(torch.bfloat16) for _ in range(layers)]
    kn = [torch.randn(N, hkv, d, generator=gen).to(torch.bfloat16) for _ in range(layers)]
    table = torch.randperm(pages + 2, generator=gen)[:pages].to(torch.int32)
    exp = [orc.commit_accepted_ref(kp[l], table.tolist(), L, kn[l], nodes) for l in range(layers)]
    kpd = [t.to(DEV) for t in kp]
    vpd = [t.clone().to(DEV) for t in kp]
    knd = [t.to(DEV) for t in kn]
    acc = d2sd.GreedyAccept(N, V, lb, DEV)
    commit = d2sd.PagedKVCommit(kpd, vpd, knd, [t.clone() for t in knd])
    lg, ni, dr, tb = (logits.to(DEV), node_index.to(torch.int32).to(DEV), drafts.to(DEV), table.to(DEV))
    graph = d2sd.HipGraph()
    with graph.capture():
        _, acc_nodes, res = acc(lg, ni, dr)
        commit.commit(tb, L, acc_nodes, num_accepted=lb, num_accepted_dev=res[:1])
    graph.replay()
    torch.cuda.synchronize()
    assert res.cpu().tolist() == [n, vb]
    for l in range(layers):
        assert torch.equal(kpd[l].cpu(), exp[l]), f"layer {l}"
