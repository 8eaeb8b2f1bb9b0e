"""d2sd — MI355X (gfx950) cascade tree-verification attention for D2SD.

Drop-in surface of the reference's verify path:
  single_prefill_with_kv_cache, merge_state_in_place   (flashinfer names)
  CascadeGraphRunner                                    (model/cascade_graph.py)
and the tree-level API
  CascadeVerifyAttention.plan() / .run()
  PagedKVCommit.commit()        (accepted-branch KV append, d3_generator.py:227-232)
  GreedyAccept() / TreeAccept() (acceptance walk, greedy or sampled, d3_generator.py:204-225)
All device work runs hand-written HIP kernels in libd2sd.so (C ABI:
include/d2sd.h); importing raises if the library has not been built.
"""
from ._lib import LIB_PATH, version
from .ops import (local_attention_merge, merge_state, merge_state_in_place, qk_norm_rope,
                  single_prefill_with_kv_cache)
from .graph import HipGraph
from .cascade_graph import CascadeGraphRunner
from .cascade import CascadeVerifyAttention
from .kv_commit import PagedKVCommit
from .accept import GreedyAccept, TreeAccept
from . import tree

__all__ = [
    "LIB_PATH", "version", "single_prefill_with_kv_cache", "merge_state_in_place", "merge_state",
    "local_attention_merge", "qk_norm_rope", "HipGraph", "CascadeGraphRunner", "CascadeVerifyAttention", "PagedKVCommit", "GreedyAccept", "TreeAccept",
    "tree",
]
