"""GPU parity of the acceptance walk (d2sd.GreedyAccept / TreeAccept,
accept.hip) against the oracle: greedy_accept_ref (generation/
d3_generator.py:204-225 at temperature 0) and sampled_accept_ref (the same walk
at temperature > 0, model/utils.py:34-37, drawing from the Philox stream of
seed and step).  Integer outputs: exact equality; the sampled draws also
against softmax(logits / T) by a chi-square test."""
import numpy as np
import pytest
import torch

from oracle import cascade_oracle as orc
import d2sd
from d2sd import tree as dtree

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_scaled_logits_ref_is_torch_gpu_division(dtype):
    """The oracle's logits / T (what the sampled walk draws from,
    model/utils.py:34) equals torch's own division of a device tensor by a
    Python scalar, bit for bit, over 8 x 32000 logits of widely spread
    magnitudes (subnormal to 1e4) at several temperatures."""
    gen = torch.Generator().manual_seed(34)
    lg = torch.randn(8, 32000, generator=gen) * torch.exp2(torch.randint(-140, 14, (8, 32000), generator=gen).float())
    lg = lg.to(dtype)
    lg_dev = lg.to(DEV)
    for t in (1e-4, 0.3, 0.7, 1.0, 1.3, 2.5, 7.0):
        got = (lg_dev / t).cpu().double().numpy()
        want = orc.scaled_logits_ref(lg, t)
        diff = got != want
        assert not diff.any(), f"T={t}: {int(diff.sum())} of {diff.size} values differ"


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


# ---- sampled walk (temperature > 0, model/utils.py:34-37) ----

# Every node's token is the argmax of its float64 oracle scores; the device
# computes the same scores in fp32 (error below 1e-5 for |logits / T| < 64),
# so a top-2 gap above 1e-4 decides every node, and the seeds below are
# chosen so that all gaps clear it (checked in each test).
_MARGIN = 1e-4


def _top2_gap(scores):
    top2 = np.sort(scores, axis=-1)[:, -2:]
    return float((top2[:, 1] - top2[:, 0]).min())


def _sampled_cases():
    return [(151936, 1.0, torch.bfloat16), (32000, 0.7, torch.bfloat16), (32000, 0.7, torch.float32),
            (1001, 1.5, torch.bfloat16), (1001, 1.5, torch.float32), (7, 1.0, torch.float32)]


def _sampled_setup(vocab, temp, dtype):
    gen = torch.Generator().manual_seed(vocab + 3)
    tr = dtree.d3_verify_tree(np.random.default_rng(vocab).uniform(size=15))
    node_index = torch.as_tensor(tr.node_index, dtype=torch.long)
    logits = (torch.randn(tr.num_nodes, vocab, generator=gen) * 2.0).to(dtype)
    return gen, node_index, logits


SAMPLE_SEED = {151936: 21, 32000: 21, 1001: 21, 7: 21}
SAMPLE_KEEPS = ([32, 32, 32, 32, 32], [3, 9, 0, 20, 1], [0, 0, 0, 0, 0])


@pytest.mark.parametrize("vocab,temp,dtype", _sampled_cases())
def test_sampled_walk_matches_oracle(vocab, temp, dtype):
    """Tokens, nodes, length and valid row equal the oracle's sampled walk
    (sampled_accept_ref) on the same seed and step, and every node's draw
    equals the oracle's; consecutive calls advance the device step counter."""
    gen, node_index, logits = _sampled_setup(vocab, temp, dtype)
    seed = SAMPLE_SEED[vocab]
    acc = d2sd.TreeAccept(logits.shape[0], vocab, node_index.shape[1], DEV, temperature=temp, seed=seed)
    lg_dev = logits.to(DEV)
    ni_dev = node_index.to(torch.int32).to(DEV)
    lengths = set()
    for step, keep in enumerate(SAMPLE_KEEPS):
        scores = orc.sample_scores_ref(logits, temp, seed, step)
        assert _top2_gap(scores) > _MARGIN, f"seed {seed} step {step} leaves a node undecided"
        drafts = _drafts_following(torch.from_numpy(scores), node_index, keep, gen)
        ids, nodes, n, vb = orc.sampled_accept_ref(logits, node_index, drafts, temp, seed, step)
        g_ids, g_nodes, g_res = acc(lg_dev, ni_dev, drafts.to(DEV))
        torch.cuda.synchronize()
        assert g_res.cpu().tolist() == [n, vb], (step, g_res.cpu().tolist(), n, vb)
        assert g_ids.cpu()[:n].tolist() == ids and g_nodes.cpu()[:n].tolist() == nodes
        assert torch.equal(acc.node_tokens.cpu(), torch.from_numpy(scores.argmax(-1)))
        lengths.add(n)
    assert int(acc.rng_step[0]) == len(SAMPLE_KEEPS)
    assert len(lengths) >= 2


def test_sampled_tokens_follow_softmax_on_device():
    """4096 nodes with the same logits, eight calls: the 32768 device draws
    follow softmax(logits / T) (chi-square), with T applied as torch does."""
    gen = torch.Generator().manual_seed(31)
    V, N, temp = 48, 4096, 0.8
    row = (torch.randn(1, V, generator=gen) * 2.0).to(torch.bfloat16)
    acc = d2sd.TreeAccept(N, V, 1, DEV, temperature=temp, seed=99)
    lg = row.expand(N, -1).contiguous().to(DEV)
    ni = torch.zeros(1, 1, dtype=torch.int32, device=DEV)
    dr = torch.zeros(1, 1, dtype=torch.int64, device=DEV)
    counts = torch.zeros(V, dtype=torch.int64)
    draws = []
    for _ in range(8):
        acc(lg, ni, dr)
        tok = acc.node_tokens.cpu()
        draws.append(tok)
        counts += torch.bincount(tok, minlength=V)
    assert int(acc.rng_step[0]) == 8
    assert not torch.equal(draws[0], draws[1])
    from scipy import stats
    probs = torch.softmax(torch.from_numpy(orc.scaled_logits_ref(row, temp))[0], -1).numpy()
    exp = probs * counts.sum().item()
    keep = exp >= 5
    obs = np.append(counts.numpy()[keep], counts.numpy()[~keep].sum())
    ex = np.append(exp[keep], exp[~keep].sum())
    assert stats.chisquare(obs, ex).pvalue > 1e-4


def test_sampled_walk_replays_draw_anew():
    """Captured once, replayed: each replay advances the step counter and
    draws the oracle's tokens of that step."""
    gen, node_index, logits = _sampled_setup(1001, 0.9, torch.bfloat16)
    seed = 5
    acc = d2sd.TreeAccept(logits.shape[0], 1001, node_index.shape[1], DEV, temperature=0.9, seed=seed)
    lg, ni = logits.to(DEV), node_index.to(torch.int32).to(DEV)
    dr = torch.zeros(node_index.shape, dtype=torch.int64, device=DEV)
    graph = d2sd.HipGraph()
    with graph.capture():
        acc(lg, ni, dr)
    start = int(acc.rng_step[0])  # capture launches nothing
    seen = []
    for k in range(3):
        graph.replay()
        torch.cuda.synchronize()
        scores = orc.sample_scores_ref(logits, 0.9, seed, start + k)
        assert _top2_gap(scores) > _MARGIN
        assert torch.equal(acc.node_tokens.cpu(), torch.from_numpy(scores.argmax(-1))), f"replay {k}"
        seen.append(acc.node_tokens.cpu())
    assert int(acc.rng_step[0]) == start + 3
    assert not torch.equal(seen[0], seen[1])


def test_zero_temperature_is_the_greedy_walk():
    gen, node_index, logits = _sampled_setup(1001, 1.0, torch.bfloat16)
    drafts = _drafts_following(logits, node_index, [4, 9, 0, 20, 2], gen)
    acc = d2sd.TreeAccept(logits.shape[0], 1001, node_index.shape[1], DEV, temperature=0.0)
    g_ids, g_nodes, g_res = acc(logits.to(DEV), node_index.to(torch.int32).to(DEV), drafts.to(DEV))
    torch.cuda.synchronize()
    ids, nodes, n, vb = orc.greedy_accept_ref(logits.float(), node_index, drafts)
    assert g_res.cpu().tolist() == [n, vb] and g_ids.cpu()[:n].tolist() == ids
    assert torch.equal(acc.node_tokens.cpu(), logits.float().argmax(-1))
    assert int(acc.rng_step[0]) == 0
