"""The allocation-free cascade entry point (d2sd_cascade_run_noalloc, through
the C ABI) against d2sd_cascade_run with a caller workspace: bit-identical O
and LSE, on two calls in a row (Qwen3-8B verify step, then a smaller
problem), with no caller workspace passed; a plan too large for the
library's workspace is rejected before any launch."""
import pytest
import torch

import d2sd
from d2sd import _lib
from d2sd import workloads as wl

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _both(prob):
    mp = wl.materialize(prob, DEV, layers=1)
    attn = d2sd.CascadeVerifyAttention(DEV)
    wl.plan_for(attn, mp)
    lt = mp.layers[0]
    assert 0 < attn.info.workspace_bytes <= _lib.lib.d2sd_cascade_scratch_bytes()
    o_ref, l_ref = attn.run(lt.q, lt.k_suffix, lt.v_suffix, lt.k_prefix, lt.v_prefix)
    o, l = attn.run_no_alloc(lt.q, lt.k_suffix, lt.v_suffix, lt.k_prefix, lt.v_prefix)
    torch.cuda.synchronize()
    assert torch.equal(o, o_ref) and torch.equal(l, l_ref)
    return attn.info.workspace_bytes


def test_no_alloc_matches_workspace_run_on_two_calls():
    big = _both(wl.config2(0, layers=1))
    small = _both(wl.config1(0))
    assert small < big


def test_no_alloc_rejects_plans_beyond_its_workspace():
    prob = wl.config3(0)
    attn = d2sd.CascadeVerifyAttention(DEV)
    mp = wl.materialize(prob, DEV, layers=1)
    # 8 long requests split for 4x the CUs: ~57 MiB of partial states
    wl.plan_for(attn, mp, num_cus=1024)
    assert attn.info.workspace_bytes > _lib.lib.d2sd_cascade_scratch_bytes()
    lt = mp.layers[0]
    with pytest.raises(RuntimeError, match="workspace"):
        attn.run_no_alloc(lt.q, lt.k_suffix, lt.v_suffix, lt.k_prefix, lt.v_prefix)
