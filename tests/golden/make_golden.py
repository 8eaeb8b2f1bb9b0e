"""Writes tests/golden/cascade_golden.npz: known-answer vectors for cascade
verify attention, computed with pure-Python float64 loops that share no code
with oracle/ or the d2sd package.

The reference (catnanami/D2-SD) ships no tests, fixtures or golden vectors
for this path, and FlashInfer — which holds its arithmetic — is not vendored
or installed, so these vectors come from the definitions the reference's call
sites fix (generation/verification.py:127-176):
  * softmax attention, logits q.k * sm_scale, query head h -> kv head h // g;
  * causal alignment: key j visible to query i iff j <= i + kv_len - qo_len;
  * cascade = one softmax over [window-truncated prefix || the node's
    ancestors-or-self in the candidate tree];
  * GPT-OSS sink (HF definition): an extra logit per head in the softmax
    denominator with no value, i.e. O = sum_j e^{s_j} v_j / (sum_j e^{s_j} + e^{sink});
  * merge: s = log(e^a + e^b), v = (v_a e^a + v_b e^b) / e^s.
Inputs are rounded to bfloat16-representable values so that GPU tests can feed
the same numbers.  Run:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import math
from pathlib import Path

import numpy as np

OUT = Path(__file__).resolve().parent / "cascade_golden.npz"


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round float64 -> nearest bfloat16 (ties to even), returned as float32."""
    f = np.asarray(x, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    u = (u + 0x7FFF + lsb) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def randn(rng: np.random.Generator, *shape) -> np.ndarray:
    return bf16_round(rng.standard_normal(shape))


def loop_attention(q, k, v, visible, scale, sinks=None):
    """q [n, Hq, D], k/v [L, Hkv, D]; visible(i, j) -> bool.  Returns (o, lse)
    with lse = log sum_j e^{s_j} over visible keys (sink excluded)."""
    n, hq, d = q.shape
    L, hkv, _ = k.shape
    g = hq // hkv
    o = np.zeros((n, hq, d))
    lse = np.full((n, hq), -np.inf)
    for i in range(n):
        for h in range(hq):
            kh = h // g
            logits = []
            for j in range(L):
                if visible(i, j):
                    s = 0.0
                    for t in range(d):
                        s += float(q[i, h, t]) * float(k[j, kh, t])
                    logits.append((j, s * scale))
            if not logits:
                continue
            m = max(s for _, s in logits)
            z = sum(math.exp(s - m) for _, s in logits)
            lse[i, h] = m + math.log(z)
            denom = z + (math.exp(float(sinks[h]) - m) if sinks is not None else 0.0)
            for t in range(d):
                acc = 0.0
                for j, s in logits:
                    acc += math.exp(s - m) * float(v[j, kh, t])
                o[i, h, t] = acc / denom
    return o, lse


def shared_prefix_tree(row_len, shared):
    """node_index [rows, row_len], parents [n]: row r shares its first
    shared[r] tokens with row 0; new nodes numbered in row-major order."""
    node_index = [[p for p in range(row_len)]]
    parents = [p - 1 for p in range(row_len)]
    for r in range(1, len(shared)):
        row = []
        for p in range(row_len):
            if p < shared[r]:
                row.append(node_index[0][p])
            else:
                parents.append(row[p - 1] if p > 0 else -1)
                row.append(len(parents) - 1)
        node_index.append(row)
    return np.array(node_index, dtype=np.int32), np.array(parents, dtype=np.int32)


def is_ancestor_or_self(parents, i, j):
    while i >= 0:
        if i == j:
            return True
        i = int(parents[i])
    return False


def cascade_case(rng, hq, hkv, d, row_len, shared, L, window, with_sinks):
    node_index, parents = shared_prefix_tree(row_len, shared)
    n = len(parents)
    q = randn(rng, n, hq, d)
    ks, vs = randn(rng, n, hkv, d), randn(rng, n, hkv, d)
    kp, vp = randn(rng, L, hkv, d), randn(rng, L, hkv, d)
    sinks = randn(rng, hq) if with_sinks else None
    Leff = min(L, window) if window >= 0 else L
    k_all = np.concatenate([kp[L - Leff:], ks], 0)
    v_all = np.concatenate([vp[L - Leff:], vs], 0)

    def vis(i, j):
        return True if j < Leff else is_ancestor_or_self(parents, i, j - Leff)

    o, lse = loop_attention(q, k_all, v_all, vis, d ** -0.5, sinks)
    case = dict(q=q, k_suffix=ks, v_suffix=vs, k_prefix=kp, v_prefix=vp, node_index=node_index,
                parents=parents, window=np.int32(window), o=o, lse=lse, sm_scale=np.float64(d ** -0.5))
    if with_sinks:
        case["sinks"] = sinks
    return case


def main() -> None:
    rng = np.random.default_rng(20260101)
    data = {}

    def put(prefix, case):
        for k, v in case.items():
            data[f"{prefix}/{k}"] = np.asarray(v)

    # A: non-causal GQA single prefill (verification.py:145 shape class)
    q, k, v = randn(rng, 5, 4, 16), randn(rng, 11, 2, 16), randn(rng, 11, 2, 16)
    o, lse = loop_attention(q, k, v, lambda i, j: True, 16 ** -0.5)
    put("gqa_nomask", dict(q=q, k=k, v=v, o=o, lse=lse, sm_scale=np.float64(16 ** -0.5)))

    # B: causal, qo_len < kv_len (bottom-right alignment; verification.py:159-162)
    q, k, v = randn(rng, 6, 4, 8), randn(rng, 9, 1, 8), randn(rng, 9, 1, 8)
    o, lse = loop_attention(q, k, v, lambda i, j: j <= i + (9 - 6), 8 ** -0.5)
    put("causal", dict(q=q, k=k, v=v, o=o, lse=lse, sm_scale=np.float64(8 ** -0.5)))

    # C: tree cascade with window and sinks (tiny, CPU)
    put("tree_small", cascade_case(rng, 4, 2, 16, 5, [5, 2, 0, 3], 13, 8, True))

    # D: merge_state with empty operands
    va, vb = randn(rng, 3, 2, 8), randn(rng, 3, 2, 8)
    sa = np.array([[0.5, -np.inf], [1.25, -np.inf], [-2.0, 3.0]])
    sb = np.array([[-0.75, 0.1], [-np.inf, -np.inf], [4.0, 3.0]])
    vm = np.zeros_like(va, dtype=np.float64)
    sm = np.zeros_like(sa)
    for i in range(3):
        for h in range(2):
            a, b = sa[i, h], sb[i, h]
            if a == -np.inf and b == -np.inf:
                vm[i, h] = va[i, h]
                sm[i, h] = -np.inf
                continue
            m = max(a, b)
            ea = 0.0 if a == -np.inf else math.exp(a - m)
            eb = 0.0 if b == -np.inf else math.exp(b - m)
            vm[i, h] = (va[i, h].astype(np.float64) * ea + vb[i, h].astype(np.float64) * eb) / (ea + eb)
            sm[i, h] = m + math.log(ea + eb)
    put("merge", dict(va=va, sa=sa, vb=vb, sb=sb, v=vm, s=sm))

    # E/F: GPU-shaped cascade cases (head_dim 64 and 128, prefix tails)
    put("tree_d64", cascade_case(rng, 8, 2, 64, 8, [8, 3, 1], 70, -1, False))
    put("tree_d128", cascade_case(rng, 4, 1, 128, 6, [6, 2], 40, 32, True))

    np.savez_compressed(OUT, **data)
    print(f"wrote {OUT} ({len(data)} arrays)")


if __name__ == "__main__":
    main()
