"""Pins the CPU oracle (oracle/cascade_oracle.py) — CPU only.

Each oracle function is checked against something other than its own formula:
the loop-computed fixtures of tests/golden/make_golden.py, invariants of the
mathematics, the reference's three-step row-layout algorithm vs the single-pass
tree form, and the installed transformers GPT-OSS eager attention for the sink.
A few tests plant a mistake in the oracle and require the pins to catch it.
"""
import math

import numpy as np
import pytest
import torch

from oracle import cascade_oracle as orc
from d2sd import tree as dtree
from d2sd import workloads as wl

T = torch.from_numpy


def _close(a, b, tol=1e-9):
    a = torch.as_tensor(a, dtype=torch.float64)
    b = torch.as_tensor(b, dtype=torch.float64)
    fin = torch.isfinite(b)
    assert torch.equal(torch.isfinite(a), fin)
    assert torch.all(a[~fin] == b[~fin])
    if fin.any():
        err = (a[fin] - b[fin]).abs().max().item()
        assert err <= tol, err


# --------------------------------------------------------------- fixtures
def test_golden_gqa_nomask(golden):
    c = golden["gqa_nomask"]
    o, lse = orc.single_prefill_ref(T(c["q"]), T(c["k"]), T(c["v"]), causal=False, sm_scale=float(c["sm_scale"]))
    _close(o, c["o"])
    _close(lse, c["lse"])


def test_golden_causal(golden):
    c = golden["causal"]
    o, lse = orc.single_prefill_ref(T(c["q"]), T(c["k"]), T(c["v"]), causal=True, sm_scale=float(c["sm_scale"]))
    _close(o, c["o"])
    _close(lse, c["lse"])


@pytest.mark.parametrize("case", ["tree_small", "tree_d64", "tree_d128"])
def test_golden_tree_single_pass(golden, case):
    c = golden[case]
    m = dtree.ancestor_mask(c["parents"])
    sinks = T(c["sinks"]) if "sinks" in c else None
    o, lse = orc.cascade_tree_ref(T(c["q"]), T(c["k_suffix"]), T(c["v_suffix"]), T(c["k_prefix"]),
                                  T(c["v_prefix"]), T(m), float(c["sm_scale"]), int(c["window"]), sinks)
    _close(o, c["o"])
    _close(lse, c["lse"])


@pytest.mark.parametrize("case", ["tree_small", "tree_d64", "tree_d128"])
def test_golden_tree_row_layout(golden, case):
    """The reference's own 3-step algorithm (shared prefill over all rows,
    per-row causal local prefill, merge_state, sink) reproduces the fixture
    after gathering node values into rows."""
    c = golden[case]
    idx = torch.as_tensor(c["node_index"], dtype=torch.long)
    q, ks, vs = T(c["q"]), T(c["k_suffix"]), T(c["v_suffix"])
    sinks = T(c["sinks"]) if "sinks" in c else None
    o, lse = orc.cascade_verify_rows_ref(q[idx], ks[idx], vs[idx], T(c["k_prefix"]), T(c["v_prefix"]),
                                         float(c["sm_scale"]), int(c["window"]), sinks)
    _close(o, T(c["o"])[idx])
    _close(lse, T(c["lse"])[idx])


def test_golden_merge(golden):
    c = golden["merge"]
    v, s = orc.merge_state_ref(T(c["va"]), T(c["sa"]), T(c["vb"]), T(c["sb"]))
    _close(v, c["v"], 1e-12)
    _close(s, c["s"], 1e-12)


# ------------------------------------------------------------- invariants
def _rand(gen, *shape):
    return torch.randn(*shape, generator=gen, dtype=torch.float64)


def test_sdpa_form_matches_explicit_form():
    gen = torch.Generator().manual_seed(1)
    q, k, v = _rand(gen, 7, 8, 32), _rand(gen, 19, 2, 32), _rand(gen, 19, 2, 32)
    mask = torch.rand(7, 19, generator=gen) < 0.7
    mask[:, 0] = True
    o1, l1 = orc.attention_ref(q, k, v, mask, 0.2)
    o2, l2 = orc.attention_sdpa_ref(q, k, v, mask, 0.2, dtype=torch.float64)
    _close(o1, o2, 1e-10)
    _close(l1, l2, 1e-10)


@pytest.mark.parametrize("splits", [[5, 11], [1, 2, 3, 30], [17]])
def test_split_prefix_merge_equals_unsplit(splits):
    gen = torch.Generator().manual_seed(2)
    q, k, v = _rand(gen, 6, 4, 16), _rand(gen, 40, 2, 16), _rand(gen, 40, 2, 16)
    o_ref, l_ref = orc.single_prefill_ref(q, k, v, False, 0.25)
    bounds = [0] + splits + [40]
    o_acc = torch.zeros_like(o_ref)
    l_acc = torch.full_like(l_ref, -math.inf)
    for a, b in zip(bounds[:-1], bounds[1:]):
        o_p, l_p = orc.single_prefill_ref(q, k[a:b], v[a:b], False, 0.25)
        o_acc, l_acc = orc.merge_state_ref(o_acc, l_acc, o_p, l_p)
    _close(o_acc, o_ref, 1e-12)
    _close(l_acc, l_ref, 1e-12)


def test_dta_shared_prefix_is_cache_then_context():
    """dflash.py:103-108: key t of the DTA shared level is draft-cache token t
    for t < Lc and context token t - Lc after it, keys and values alike; and
    the shared level's attention equals the merge of the two segments'
    attentions (the split-KV identity a two-segment plan relies on)."""
    gen = torch.Generator().manual_seed(5)
    hkv, lc, c, d = 2, 13, 5, 16
    kc, vc, kx, vx = (_rand(gen, hkv, n, d) for n in (lc, lc, c, c))
    k, v = orc.dta_shared_prefix_ref(kc, vc, kx, vx)
    assert k.shape == v.shape == (lc + c, hkv, d) and k.is_contiguous()
    for t in range(lc + c):
        for h in range(hkv):
            src_k, src_v = (kc[h, t], vc[h, t]) if t < lc else (kx[h, t - lc], vx[h, t - lc])
            assert torch.equal(k[t, h], src_k) and torch.equal(v[t, h], src_v)
    q = _rand(gen, 7, 4, d)
    o_ref, l_ref = orc.single_prefill_ref(q, k, v, False, 0.25)
    o_a, l_a = orc.single_prefill_ref(q, kc.transpose(0, 1), vc.transpose(0, 1), False, 0.25)
    o_b, l_b = orc.single_prefill_ref(q, kx.transpose(0, 1), vx.transpose(0, 1), False, 0.25)
    o_m, l_m = orc.merge_state_ref(o_a, l_a, o_b, l_b)
    _close(o_m, o_ref, 1e-12)
    _close(l_m, l_ref, 1e-12)


def test_merge_commutative_associative():
    gen = torch.Generator().manual_seed(3)
    st = [(_rand(gen, 3, 2, 8), _rand(gen, 3, 2) * 3) for _ in range(3)]
    ab = orc.merge_state_ref(*st[0], *st[1])
    ba = orc.merge_state_ref(*st[1], *st[0])
    _close(ab[0], ba[0], 1e-12)
    _close(ab[1], ba[1], 1e-12)
    left = orc.merge_state_ref(*ab, *st[2])
    bc = orc.merge_state_ref(*st[1], *st[2])
    right = orc.merge_state_ref(*st[0], *bc)
    _close(left[0], right[0], 1e-12)
    _close(left[1], right[1], 1e-12)


def test_empty_prefix_is_pure_tree_attention():
    gen = torch.Generator().manual_seed(4)
    t = dtree.tree_from_shared_prefixes(6, [6, 2, 4])
    m = torch.as_tensor(t.ancestor_mask())
    n = t.num_nodes
    q, ks, vs = _rand(gen, n, 4, 16), _rand(gen, n, 2, 16), _rand(gen, n, 2, 16)
    o1, l1 = orc.cascade_tree_ref(q, ks, vs, None, None, m, 0.3)
    o2, l2 = orc.attention_ref(q, ks, vs, m, 0.3)
    _close(o1, o2, 1e-12)
    _close(l1, l2, 1e-12)


def test_chain_tree_equals_causal_prefill():
    gen = torch.Generator().manual_seed(5)
    n, L = 9, 23
    t = dtree.tree_from_shared_prefixes(n, [n])
    q, ks, vs = _rand(gen, n, 4, 16), _rand(gen, n, 1, 16), _rand(gen, n, 1, 16)
    kp, vp = _rand(gen, L, 1, 16), _rand(gen, L, 1, 16)
    o1, l1 = orc.cascade_tree_ref(q, ks, vs, kp, vp, torch.as_tensor(t.ancestor_mask()), 0.25)
    o2, l2 = orc.single_prefill_ref(q, torch.cat([kp, ks]), torch.cat([vp, vs]), True, 0.25)
    _close(o1, o2, 1e-12)
    _close(l1, l2, 1e-12)


def test_constant_v_gives_v():
    gen = torch.Generator().manual_seed(6)
    q, k = _rand(gen, 5, 4, 8), _rand(gen, 12, 2, 8)
    v = torch.ones(12, 2, 8, dtype=torch.float64) * torch.tensor([1.5, -2.0], dtype=torch.float64)[None, :, None]
    o, _ = orc.single_prefill_ref(q, k, v, True, 0.5)
    expect = torch.tensor([1.5] * 2 + [-2.0] * 2, dtype=torch.float64)[None, :, None].expand_as(o)
    _close(o, expect, 1e-12)


def test_page_permutation_invariance():
    gen = torch.Generator().manual_seed(7)
    P, pages, hkv, d, L = 4, 6, 2, 8, 21
    pool = _rand(gen, pages, hkv, P, d)
    table = [3, 0, 5, 1, 4, 2]
    k1 = orc.gather_paged(pool, table, L)
    perm = [2, 4, 0, 5, 1, 3]                      # pool2[perm[i]] = pool[i]
    pool2 = torch.empty_like(pool)
    for i, pi in enumerate(perm):
        pool2[pi] = pool[i]
    k2 = orc.gather_paged(pool2, [perm[t] for t in table], L)
    assert torch.equal(k1, k2)
    assert torch.equal(k1[:4], pool[3].permute(1, 0, 2))


def test_window_keeps_last_keys():
    gen = torch.Generator().manual_seed(8)
    k, v = _rand(gen, 30, 2, 8), _rand(gen, 30, 2, 8)
    kw, vw = orc.window_prefix_ref(k, v, 7)
    assert torch.equal(kw, k[23:]) and torch.equal(vw, v[23:])
    assert orc.window_prefix_ref(k, v, 64)[0] is k
    assert orc.window_prefix_ref(k, v, -1)[0] is k


def test_sink_matches_transformers_gpt_oss_eager():
    from types import SimpleNamespace
    from transformers.models.gpt_oss.modeling_gpt_oss import eager_attention_forward
    gen = torch.Generator().manual_seed(9)
    t = dtree.tree_from_shared_prefixes(5, [5, 1, 3])
    m = torch.as_tensor(t.ancestor_mask())
    n, L, hq, hkv, d = t.num_nodes, 13, 8, 2, 16
    q, ks, vs = _rand(gen, n, hq, d), _rand(gen, n, hkv, d), _rand(gen, n, hkv, d)
    kp, vp = _rand(gen, L, hkv, d), _rand(gen, L, hkv, d)
    sinks = _rand(gen, hq)
    o, _ = orc.cascade_tree_ref(q, ks, vs, kp, vp, m, d ** -0.5, sinks=sinks)
    full = torch.cat([torch.ones(n, L, dtype=torch.bool), m], 1)
    add = torch.zeros(n, L + n, dtype=torch.float64).masked_fill(~full, -math.inf)[None, None]
    mod = SimpleNamespace(num_key_value_groups=hq // hkv, sinks=sinks, training=False)
    k_all = torch.cat([kp, ks]).transpose(0, 1)[None]
    v_all = torch.cat([vp, vs]).transpose(0, 1)[None]
    ref, _ = eager_attention_forward(mod, q.transpose(0, 1)[None], k_all, v_all, add, d ** -0.5)
    _close(o, ref[0], 1e-12)


@pytest.mark.parametrize("seed", [0, 1, 2, 3])
def test_row_layout_equals_tree_layout_d3(seed):
    rng = np.random.default_rng(seed)
    t = dtree.d3_verify_tree(rng.uniform(size=7), block_size=8, block_size_2=12, topk=3)
    idx = torch.as_tensor(t.node_index, dtype=torch.long)
    gen = torch.Generator().manual_seed(seed)
    n = t.num_nodes
    q, ks, vs = _rand(gen, n, 4, 16), _rand(gen, n, 2, 16), _rand(gen, n, 2, 16)
    kp, vp = _rand(gen, 20, 2, 16), _rand(gen, 20, 2, 16)
    sinks = _rand(gen, 4)
    o_t, l_t = orc.cascade_tree_ref(q, ks, vs, kp, vp, torch.as_tensor(t.ancestor_mask()), 0.25, 9, sinks)
    o_r, l_r = orc.cascade_verify_rows_ref(q[idx], ks[idx], vs[idx], kp, vp, 0.25, 9, sinks)
    _close(o_r, o_t[idx], 1e-12)
    _close(l_r, l_t[idx], 1e-12)


def test_tree_ref_keeps_prefix_precision():
    """A float prefix (e.g. fp8 dequantised with an fp32 scale) is used at full
    precision next to a bf16 suffix."""
    gen = torch.Generator().manual_seed(10)
    t = dtree.tree_from_shared_prefixes(4, [4, 2])
    m = torch.as_tensor(t.ancestor_mask())
    n = t.num_nodes
    q = _rand(gen, n, 4, 16).to(torch.bfloat16)
    ks, vs = _rand(gen, n, 2, 16).to(torch.bfloat16), _rand(gen, n, 2, 16).to(torch.bfloat16)
    kp, vp = _rand(gen, 9, 2, 16) * 1.0009765, _rand(gen, 9, 2, 16) * 1.0009765
    o1, l1 = orc.cascade_tree_ref(q, ks, vs, kp, vp, m, 0.25)
    full = torch.cat([torch.ones(n, 9, dtype=torch.bool), m], 1)
    o2, l2 = orc.attention_ref(q.double(), torch.cat([kp, ks.double()]), torch.cat([vp, vs.double()]), full, 0.25)
    _close(o1, o2, 1e-12)
    _close(l1, l2, 1e-12)


def test_fp8_dequant_exact():
    x = torch.tensor([0.0, 1.0, -1.5, 448.0, 2.0 ** -9, -(2.0 ** -6) * 0.875], dtype=torch.float32)
    f8 = x.to(torch.float8_e4m3fn)
    assert torch.equal(orc.fp8_dequant_ref(f8, torch.tensor(1.0)), x)


# ------------------------------------------------- planted-mistake checks
def test_planted_wrong_gqa_map_is_caught(golden, monkeypatch):
    c = golden["gqa_nomask"]
    monkeypatch.setattr(orc, "_expand_kv", lambda k, hq: k.repeat(1, hq // k.shape[1], 1))
    o, _ = orc.single_prefill_ref(T(c["q"]), T(c["k"]), T(c["v"]), causal=False, sm_scale=float(c["sm_scale"]))
    assert (o - T(c["o"])).abs().max() > 1e-3


def test_planted_top_left_causal_is_caught(golden, monkeypatch):
    c = golden["causal"]
    monkeypatch.setattr(orc, "causal_mask", lambda n, L: torch.arange(L)[None, :] <= torch.arange(n)[:, None])
    o, _ = orc.single_prefill_ref(T(c["q"]), T(c["k"]), T(c["v"]), causal=True, sm_scale=float(c["sm_scale"]))
    assert (o - T(c["o"])).abs().max() > 1e-3


def test_planted_missing_window_is_caught(golden, monkeypatch):
    c = golden["tree_small"]
    monkeypatch.setattr(orc, "window_prefix_ref", lambda k, v, w: (k, v))
    o, _ = orc.cascade_tree_ref(T(c["q"]), T(c["k_suffix"]), T(c["v_suffix"]), T(c["k_prefix"]),
                                T(c["v_prefix"]), T(dtree.ancestor_mask(c["parents"])), float(c["sm_scale"]),
                                int(c["window"]), T(c["sinks"]))
    assert (o - T(c["o"])).abs().max() > 1e-3


def test_planted_base2_lse_is_caught(golden):
    c = golden["gqa_nomask"]
    _, lse = orc.single_prefill_ref(T(c["q"]), T(c["k"]), T(c["v"]), causal=False, sm_scale=float(c["sm_scale"]))
    assert (lse / math.log(2) - T(c["lse"])).abs().max() > 1e-2


# ------------------------------------------------ tree geometry (host code)
@pytest.mark.parametrize("seed", range(6))
def test_tree_mask_two_constructions_agree(seed):
    rng = np.random.default_rng(seed)
    trees = [dtree.d3_verify_tree(rng.uniform(size=15)),
             dtree.d3_verify_tree(rng.uniform(size=15), 16, 16, 4),
             wl.random_branch_tree(rng, 8, 32, chain_to_row0=False),
             wl.random_branch_tree(rng, 4, 16)]
    for t in trees:
        m1 = dtree.ancestor_mask(t.parents)
        m2 = orc.ancestor_mask_from_rows(t.node_index, t.num_nodes)
        assert np.array_equal(m1, m2)


def test_d3_tree_sizes_match_reference_geometry():
    sizes = []
    for seed in range(200):
        rng = np.random.default_rng(seed)
        t = dtree.d3_verify_tree(rng.uniform(size=15), 16, 32, 4)
        assert t.num_rows == 5 and t.row_len == 32
        # row j shares pl_j + 1 tokens with row 0, pl_j distinct in [0, 14]
        assert all(1 <= s <= 15 for s in t.shared[1:]) and len(set(t.shared[1:])) == 4
        assert t.num_nodes == 32 + sum(32 - s for s in t.shared[1:])
        sizes.append(t.num_nodes)
    assert 106 <= min(sizes) and max(sizes) <= 150


def test_d3_rates_formula():
    conf = np.array([0.9, 0.5, 0.8, 0.3])
    r = dtree.d3_rejection_rates(conf, "float32")
    assert np.allclose(r, [0.1, 0.9 * 0.5, 0.9 * 0.5 * 0.2, 0.9 * 0.5 * 0.8 * 0.7])


def _reference_rates_torch(conf: torch.Tensor) -> torch.Tensor:
    """generation/d3_generator.py:117-121, executed with torch on conf's
    dtype; the cumulative product as a sequential loop of torch bf16 products,
    which is what torch.cumprod computes on a device tensor (pinned in
    tests/test_gpu_tree_build.py; its CPU kernel keeps a float32 running
    product instead)."""
    cum_prod = conf.clone()
    for i in range(1, conf.shape[0]):
        cum_prod[i] = cum_prod[i - 1] * conf[i]
    rates = torch.empty(conf.shape[0])
    rates[0] = 1.0 - conf[0]
    rates[1:] = cum_prod[:-1] * (1.0 - conf[1:])
    return rates


@pytest.mark.parametrize("dtype", ["bfloat16"])
def test_d3_rates_match_torch_arithmetic(dtype):
    """The restatement equals the reference's own torch lines, bit for bit,
    on random and on coarse (tie-rich) confidences (bf16, the draft
    probabilities' dtype; fp32 is pinned on the GPU, where torch's cumprod
    runs as the reference ran it)."""
    rng = np.random.default_rng(17)
    tdt = getattr(torch, dtype)
    for i in range(300):
        conf = rng.uniform(size=15) if i % 2 else rng.choice([0.0, 0.25, 0.5, 0.75, 1.0, 0.9, 0.1], size=15)
        c = torch.tensor(conf, dtype=torch.float32).to(tdt)
        ref = _reference_rates_torch(c).numpy()
        got = dtree.d3_rejection_rates(c.float().numpy(), dtype)
        assert np.array_equal(ref.view(np.uint32), got.view(np.uint32)), (i, ref, got)


def test_d3_selection_matches_torch_topk_without_boundary_ties():
    """sorted(torch.topk(rates, 4)) == the restatement whenever the 4th and
    5th largest rates differ (ties there are ordered by index here; torch.topk
    leaves their order unspecified)."""
    rng = np.random.default_rng(23)
    checked = 0
    for _ in range(400):
        c = torch.tensor(rng.uniform(size=15), dtype=torch.float32).to(torch.bfloat16)
        rates = _reference_rates_torch(c)
        srt = torch.sort(rates, descending=True).values
        if srt[3] == srt[4]:
            continue
        ref = sorted(torch.topk(rates, 4).indices.tolist())
        assert ref == dtree.d3_select_boundaries(dtree.d3_rejection_rates(c.float().numpy()), 4)
        checked += 1
    assert checked > 300


def test_pack_mask_bits():
    m = np.zeros((2, 70), dtype=bool)
    m[0, [0, 5, 63]] = True
    m[1, [64, 69]] = True
    p = dtree.pack_mask_rows(m)
    assert p.shape == (2, 2)
    assert int(p[0, 0]) == (1 | (1 << 5) | (1 << 63)) and int(p[0, 1]) == 0
    assert int(p[1, 0]) == 0 and int(p[1, 1]) == (1 | (1 << 5))


# ---- accepted-branch commit (generation/d3_generator.py:227-232) ----

def _cat_form(pool, table, L, new, nodes, layout):
    """The reference's own operation: cache = torch.cat([cache, k_win], dim=2)
    on the contiguous view."""
    return torch.cat([orc.gather_paged(pool, table, L, layout), new[torch.as_tensor(nodes, dtype=torch.long)]], 0)


@pytest.mark.parametrize("layout", ["HND", "NHD"])
@pytest.mark.parametrize("L,n,P", [(0, 5, 4), (3, 2, 2), (7, 9, 4), (16, 16, 16), (31, 1, 16)])
def test_commit_equals_cat_and_touches_only_new_slots(layout, L, n, P):
    g = torch.Generator().manual_seed(L * 131 + n)
    hkv, d, rows = 2, 8, 12
    pages_needed = (L + n + P - 1) // P
    pool_pages = pages_needed + 3
    shape = (pool_pages, hkv, P, d) if layout == "HND" else (pool_pages, P, hkv, d)
    pool = torch.randn(shape, generator=g)
    table = torch.randperm(pool_pages, generator=g)[:pages_needed].tolist()
    new = torch.randn(rows, hkv, d, generator=g)
    nodes = torch.randint(0, rows, (n,), generator=g).tolist()
    out = orc.commit_accepted_ref(pool, table, L, new, nodes, layout)
    assert torch.equal(orc.gather_paged(out, table, L + n, layout), _cat_form(pool, table, L, new, nodes, layout))
    # nothing else changed: the old prefix, other pages, slots past the end
    written = torch.zeros(shape[:3] if layout == "HND" else shape[:2], dtype=torch.bool)
    for i in range(n):
        t = L + i
        if layout == "HND":
            written[table[t // P], :, t % P] = True
        else:
            written[table[t // P], t % P] = True
    keep = ~written
    assert torch.equal(out[keep], pool[keep])


def test_commit_known_answer_and_skipped_nodes():
    # P = 2, prefix of 3 tokens: new tokens go to page table[1] slot 1, then table[2] slot 0
    pool = torch.zeros(4, 1, 2, 1)                       # HND, Hkv 1, D 1
    new = torch.tensor([[[10.]], [[20.]], [[30.]]])
    out = orc.commit_accepted_ref(pool, [3, 1, 0], 3, new, [2, 0], "HND")
    assert out[1, 0, 1, 0] == 30. and out[0, 0, 0, 0] == 10.
    assert out.sum() == 40.
    # a node id outside [0, rows) writes nothing (positions still advance)
    out = orc.commit_accepted_ref(pool, [3, 1, 0], 3, new, [-1, 1], "HND")
    assert out[1, 0, 1, 0] == 0. and out[0, 0, 0, 0] == 20. and out.sum() == 20.


def test_fp8_quantiser_is_round_to_nearest_even_with_clamp():
    """quantize_e4m3fn_ref against brute force over every finite bf16 value:
    the nearest of the 253 finite e4m3fn values to clamp(x, +-448), ties to
    the even mantissa; and each e4m3fn value maps to itself."""
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    vals = codes.view(torch.float8_e4m3fn).float()
    fin = torch.isfinite(vals)
    grid = vals[fin].double().numpy()
    grid_codes = codes[fin].numpy()
    # each finite e4m3fn value maps to itself
    back = orc.quantize_e4m3fn_ref(vals[fin].view(1, -1, 1), torch.ones(1)).view(torch.uint8).flatten()
    assert torch.equal(back.float(), vals[fin].to(torch.float8_e4m3fn).view(torch.uint8).float())
    bits = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    x = bits[torch.isfinite(bits)]
    got = orc.quantize_e4m3fn_ref(x.view(1, -1, 1), torch.ones(1)).view(-1).float().double().numpy()
    xc = np.clip(x.double().numpy(), -448.0, 448.0)
    dist = np.abs(xc[:, None] - grid[None, :])
    best = dist.min(1)
    cand = dist <= best[:, None]
    # among equidistant candidates the even mantissa (code & 1 == 0), +0 for zero
    pick = np.where(cand & ((grid_codes[None, :] & 1) == 0), 1, 0) * 2 + cand
    want = grid[pick.argmax(1)]
    zero = xc == 0
    assert np.array_equal(got[~zero], want[~zero])
    assert np.all(got[zero] == 0)


# ---- greedy acceptance walk (generation/d3_generator.py:204-225) ----

def _chain_logits(tokens_per_node, vocab=11):
    """Logits whose argmax at node j is tokens_per_node[j]."""
    lg = torch.zeros(len(tokens_per_node), vocab)
    for j, t in enumerate(tokens_per_node):
        lg[j, t] = 1.0
    return lg


def test_accept_full_agreement_accepts_every_position():
    # one chain of 4 nodes; the draft row follows the target's argmax
    lg = _chain_logits([5, 6, 7, 8])
    ids, nodes, n, vb = orc.greedy_accept_ref(lg, [[0, 1, 2, 3]], [[9, 5, 6, 7]])
    assert (ids, nodes, n, vb) == ([5, 6, 7, 8], [0, 1, 2, 3], 4, 0)


def test_accept_switches_to_the_first_matching_row():
    # rows share node 0; row 0 drafts token 3 at position 1 (rejected), row 1
    # drafts 4 (accepted: argmax of node 0); then row 1's node 2 gives 2, and
    # its draft at position 2 is 7 (rejected) -> length 2, valid_block 1
    lg = _chain_logits([4, 9, 2])
    ids, nodes, n, vb = orc.greedy_accept_ref(lg, [[0, 1, 1], [0, 2, 2]], [[0, 3, 0], [0, 4, 7]])
    assert (ids, nodes, n, vb) == ([4, 2], [0, 2], 2, 1)


def test_accept_first_position_always_accepted():
    lg = _chain_logits([1, 2])
    ids, nodes, n, vb = orc.greedy_accept_ref(lg, [[0, 1]], [[0, 5]])
    assert (ids, n, vb) == ([1], 1, 0)


def test_accept_argmax_ties_take_the_first_index():
    lg = torch.zeros(1, 8)
    lg[0, 3] = lg[0, 6] = 2.0
    ids, _, n, _ = orc.greedy_accept_ref(lg, [[0]], [[0]])
    assert ids == [3] and n == 1


# ---- sampled acceptance (d3_generator.py:204-225 at temperature > 0) ----

def test_philox_known_answer_vectors():
    """Philox4x32-10 against the known-answer vectors published with
    Random123 (counter, key -> output)."""
    kat = [
        ([0, 0, 0, 0], (0, 0), [0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8]),
        ([0xffffffff] * 4, (0xffffffff, 0xffffffff), [0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd]),
        ([0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344], (0xa4093822, 0x299f31d0),
         [0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1]),
    ]
    ctr = np.array([c for c, _, _ in kat], dtype=np.uint64)
    for i, (c, k, want) in enumerate(kat):
        assert orc.philox4x32_10(ctr[i], k).tolist() == want
    # vectorised form == one counter at a time
    out = orc.philox4x32_10(ctr, (0xa4093822, 0x299f31d0))
    assert out[2].tolist() == kat[2][2]


def test_sample_uniforms_range_and_independence():
    u = orc.sample_uniforms_ref(64, 1001, seed=5, offset=3)
    assert u.shape == (64, 1001) and u.min() > 0.0 and u.max() < 1.0
    assert abs(u.mean() - 0.5) < 0.01 and abs(u.var() - 1 / 12) < 0.005
    # exactly representable in fp32
    assert np.array_equal(u.astype(np.float32).astype(np.float64), u)
    # another step, seed or node gives another stream
    assert not np.array_equal(u, orc.sample_uniforms_ref(64, 1001, seed=5, offset=4))
    assert not np.array_equal(u, orc.sample_uniforms_ref(64, 1001, seed=6, offset=3))
    assert not np.array_equal(u[0], u[1])
    # token v uses word v % 4 of counter (v // 4, node, step): truncating the
    # vocabulary does not change the variates of the tokens kept
    assert np.array_equal(orc.sample_uniforms_ref(64, 13, seed=5, offset=3), u[:, :13])


def _sample_counts(logits_row, temperature, nodes, seed, scores_fn=orc.sample_scores_ref):
    lg = logits_row.expand(nodes, -1).contiguous()
    choice = scores_fn(lg, temperature, seed, 0).argmax(-1)
    return np.bincount(choice, minlength=lg.shape[1])


def _chi2_pvalue(counts, probs):
    from scipy import stats
    exp = probs * counts.sum()
    keep = exp >= 5  # pool the rare tokens into one cell
    obs = np.append(counts[keep], counts[~keep].sum())
    ex = np.append(exp[keep], exp[~keep].sum())
    if ex[-1] == 0:
        obs, ex = obs[:-1], ex[:-1]
    return stats.chisquare(obs, ex).pvalue


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_sampled_tokens_follow_softmax(dtype):
    """The draws are multinomial samples of softmax(x), x = the scaled logits
    (model/utils.py:34-37), and a plausible mistake in the scores is caught."""
    gen = torch.Generator().manual_seed(1)
    row = (torch.randn(1, 24, generator=gen) * 2.0).to(dtype)
    temp = 0.8
    x = torch.from_numpy(orc.scaled_logits_ref(row, temp))[0]
    probs = torch.softmax(x, -1).numpy()
    counts = _sample_counts(row, temp, 40000, seed=11)
    assert _chi2_pvalue(counts, probs) > 1e-4

    def wrong_temperature(lg, t, seed, off):   # planted: T applied twice
        return orc.sample_scores_ref(lg, t * t, seed, off)

    def wrong_sign(lg, t, seed, off):          # planted: + log2(E) instead of - log2(E)
        xs = orc.scaled_logits_ref(lg, t)
        e = -np.log(orc.sample_uniforms_ref(xs.shape[0], xs.shape[1], seed, off))
        return xs / math.log(2.0) + np.log2(e)

    for planted in (wrong_temperature, wrong_sign):
        assert _chi2_pvalue(_sample_counts(row, temp, 40000, 11, planted), probs) < 1e-6


def test_sampled_choice_equals_torch_multinomial_race():
    """torch.multinomial(p, 1) is argmax(p / E) with E ~ Exp(1)
    (aten/src/ATen/native/Distributions.cpp); on the same E the log-space
    scores choose the same token."""
    gen = torch.Generator().manual_seed(2)
    lg = torch.randn(200, 1000, generator=gen).to(torch.bfloat16)
    temp = 0.7
    scores = orc.sample_scores_ref(lg, temp, seed=9, offset=4)
    x = torch.from_numpy(orc.scaled_logits_ref(lg, temp))
    e = torch.from_numpy(-np.log(orc.sample_uniforms_ref(200, 1000, 9, 4)))
    race = (torch.softmax(x, -1) / e).argmax(-1)
    assert torch.equal(race, torch.from_numpy(scores.argmax(-1)))


def test_sampled_walk_at_tiny_temperature_is_greedy():
    gen = torch.Generator().manual_seed(4)
    tr = dtree.d3_verify_tree(np.random.default_rng(4).uniform(size=15))
    lg = torch.randn(tr.num_nodes, 500, generator=gen)
    am = lg.argmax(-1)
    drafts = torch.randint(0, 500, tr.node_index.shape, generator=gen)
    drafts[0, 1:] = am[torch.as_tensor(tr.node_index[0, :-1], dtype=torch.long)]
    greedy = orc.greedy_accept_ref(lg, tr.node_index, drafts)
    assert orc.sampled_accept_ref(lg, tr.node_index, drafts, 1e-4, seed=1, offset=0) == greedy
    assert greedy[2] == tr.node_index.shape[1]


def test_scaled_logits_follow_torch_gpu_division():
    """torch divides a GPU tensor by a Python scalar as a multiplication by
    the fp32 reciprocal; on bf16 logits the product is rounded to bf16."""
    lg = torch.tensor([[1.0, 3.0, -7.5, 0.1]]).to(torch.bfloat16)
    x = orc.scaled_logits_ref(lg, 0.3)
    inv = np.float32(1) / np.float32(0.3)
    want = (lg.float() * torch.tensor(inv)).to(torch.bfloat16).double().numpy()
    assert np.array_equal(x, want)
    assert np.array_equal(x, x.astype(np.float32).astype(np.float64))


# ---- QK RMSNorm + RoPE (generation/verification.py:113-123) ----

def test_qk_norm_rope_ref_matches_transformers_qwen3():
    """The restatement equals the installed transformers Qwen3 routines (the
    library the reference calls: Qwen3RMSNorm, rotate_half RoPE)."""
    from transformers.models.qwen3 import modeling_qwen3 as mq
    g = torch.Generator().manual_seed(0)
    T, H, D = 7, 4, 128
    x = (torch.randn(T, H, D, generator=g) * 3).to(torch.bfloat16)
    norm = mq.Qwen3RMSNorm(D, eps=1e-6).to(torch.bfloat16)
    with torch.no_grad():
        norm.weight.copy_((torch.rand(D, generator=g) + 0.5).to(torch.bfloat16))
    pos = torch.arange(T) + 4000
    inv = 1.0 / (1e6 ** (torch.arange(0, D, 2).float() / D))
    ang = pos[:, None].float() * inv[None]
    emb = torch.cat([ang, ang], -1)
    cos, sin = emb.cos().to(torch.bfloat16), emb.sin().to(torch.bfloat16)
    with torch.no_grad():
        y = norm(x)                                                   # [T, H, D]
        q_hf, _ = mq.apply_rotary_pos_emb(y.transpose(0, 1)[None], y.transpose(0, 1)[None], cos[None], sin[None])
    ref = orc.qk_norm_rope_ref(x, norm.weight.detach(), cos, sin, 1e-6)
    assert torch.equal(ref, q_hf[0].transpose(0, 1))


def test_qk_norm_rope_ref_gpt_oss_form_equals_rotate_half_form():
    """The GPT-OSS split-half RoPE with D/2 columns equals the rotate_half
    form with the halves duplicated (both restated from verification.py:21-42)."""
    g = torch.Generator().manual_seed(1)
    x = torch.randn(5, 3, 64, generator=g).to(torch.bfloat16)
    c = torch.randn(5, 32, generator=g).to(torch.bfloat16)
    s = torch.randn(5, 32, generator=g).to(torch.bfloat16)
    a = orc.qk_norm_rope_ref(x, None, c, s)
    b = orc.qk_norm_rope_ref(x, None, torch.cat([c, c], -1), torch.cat([s, s], -1))
    assert torch.equal(a, b)
