"""Acceptance walk of the verify tree on the device (libd2sd.so).

Replaces generation/d3_generator.py:204-225, which walks the candidate rows on
the host with a nonzero(), a sum() and a Python list per accepted token.  Here
every node's token and the walk run in two launches with no host
synchronisation; the accepted nodes and their count feed
PagedKVCommit.commit(..., num_accepted_dev=...) directly.

temperature 0 (below 1e-5, the reference's threshold) is greedy: torch.argmax,
model/utils.py:28-33.  A positive temperature draws every accepted token from
softmax(logits / T) as torch.multinomial does (model/utils.py:34-37): the
exponential race argmax(p / E), here with E from an in-kernel Philox4x32-10
stream keyed by `seed` and a device step counter that each call advances, so
replays of a captured step draw independently.  The stream is not torch's:
sampled walks match the reference in distribution.
"""
from __future__ import annotations

import ctypes as C

import torch

from . import _lib
from ._lib import check, lib
from .graph import keep_alive


class GreedyAccept:
    """Preallocated outputs and workspace for one tree shape.

    __call__(logits [num_nodes, vocab] bf16/fp32, node_index [rows, row_len]
    int32, draft_ids [rows, row_len] int64), all on the device, returns device
    tensors (accept_ids [row_len] int64, accept_nodes [row_len] int32,
    result [2] int32 = (acceptance_length, valid_block)); only the first
    acceptance_length entries of the first two are written.  `node_tokens`
    [num_nodes] int64 holds every node's token of the last call.
    Allocation-free and capturable after construction.

    temperature > 0 samples (see the module docstring); `rng_step` is the
    device step counter (int64 [1]), advanced by one per sampling call.
    """

    def __init__(self, num_nodes: int, vocab: int, row_len: int, device, temperature: float = 0.0,
                 seed: int = 0):
        self.num_nodes, self.vocab, self.row_len = int(num_nodes), int(vocab), int(row_len)
        temperature = float(temperature)
        if not (temperature >= 0.0 and temperature < float("inf")):
            raise ValueError("temperature must be finite and >= 0")
        self.temperature, self.seed = temperature, int(seed) & 0xFFFFFFFFFFFFFFFF
        ws = lib.d2sd_greedy_accept_workspace_size(self.num_nodes, self.vocab)
        self.workspace = torch.empty(max(int(ws), 8), dtype=torch.uint8, device=device)
        self.accept_ids = torch.zeros(self.row_len, dtype=torch.int64, device=device)
        self.accept_nodes = torch.zeros(self.row_len, dtype=torch.int32, device=device)
        self.result = torch.zeros(2, dtype=torch.int32, device=device)
        self.node_tokens = torch.zeros(self.num_nodes, dtype=torch.int64, device=device)
        self.rng_step = torch.zeros(1, dtype=torch.int64, device=device)

    def __call__(self, logits: torch.Tensor, node_index: torch.Tensor, draft_ids: torch.Tensor):
        if logits.dim() != 2 or logits.shape != (self.num_nodes, self.vocab) or logits.stride(1) != 1:
            raise ValueError("logits must be [num_nodes, vocab] with a contiguous vocabulary")
        if logits.dtype not in (torch.bfloat16, torch.float32):
            raise TypeError("logits must be bf16 or fp32")
        if node_index.dtype != torch.int32 or draft_ids.dtype != torch.int64:
            raise TypeError("node_index must be int32 and draft_ids int64")
        if node_index.shape != draft_ids.shape or node_index.shape[1] != self.row_len:
            raise ValueError("node_index and draft_ids must both be [rows, row_len]")
        if not (node_index.is_contiguous() and draft_ids.is_contiguous()):
            raise ValueError("node_index and draft_ids must be contiguous")
        a = _lib.AcceptArgs()
        a.num_rows = node_index.shape[0]
        a.row_len = self.row_len
        a.num_nodes = self.num_nodes
        a.vocab = self.vocab
        a.logits_dtype = _lib.D2SD_DTYPE_BF16 if logits.dtype == torch.bfloat16 else _lib.D2SD_DTYPE_F32
        a.logits = logits.data_ptr()
        a.logits_stride = logits.stride(0)
        a.node_index = node_index.data_ptr()
        a.draft_ids = draft_ids.data_ptr()
        a.accept_ids = self.accept_ids.data_ptr()
        a.accept_nodes = self.accept_nodes.data_ptr()
        a.result = self.result.data_ptr()
        a.workspace = self.workspace.data_ptr()
        a.workspace_bytes = self.workspace.numel()
        s = _lib.SampleAcceptArgs()
        s.walk = a
        s.temperature = self.temperature
        s.seed = self.seed
        s.rng_step = self.rng_step.data_ptr()
        s.node_tokens = self.node_tokens.data_ptr()
        check(lib.d2sd_sample_accept(C.byref(s), C.c_void_p(torch.cuda.current_stream().cuda_stream)),
              "sample_accept")
        keep_alive(logits, node_index, draft_ids, self.workspace, self.accept_ids, self.accept_nodes, self.result,
                   self.node_tokens, self.rng_step)
        return self.accept_ids, self.accept_nodes, self.result


TreeAccept = GreedyAccept
