"""HIP-graph replay of the DeepSeekMoE forward for decode-sized batches.

At a few tokens per call (workload C3, M = 1 .. 128) the forward is bound by
host time: its four or five entry points, their argument checks and output
allocations take longer than the kernels.  ``DecodeGraph`` captures one forward of a
fixed input shape into a HIP graph (torch.cuda.CUDAGraph, which is a HIP
graph on ROCm) and replays it: the caller writes the tokens into the
captured input buffer (``__call__`` copies them) and reads the captured
output.  The captured kernels are the same launches as the eager forward, so
a replay returns the eager result bit for bit; the module's
``_last_indices`` and counts are the graph's buffers, updated by every
replay, and ``_last_weights`` is formed from the graph's fp32 weights buffer
when it is read.  No captured kernel uses hipMemsetAsync.

Inference only (no autograd); the module's parameters must not be
reallocated after capture (in-place updates are seen by later replays).
Capture and replay run under the autocast state active at construction.
"""
from __future__ import annotations

import torch

from .moe import DeepSeekMoE


class DecodeGraph:
    """Forward of ``module`` on inputs shaped like ``example``, replayed from a
    HIP graph.  ``graph(x)`` copies ``x`` into the captured input and returns
    the captured output tensor (overwritten by the next replay; clone it to
    keep it)."""

    def __init__(self, module: DeepSeekMoE, example: torch.Tensor, warmup: int = 2):
        if not example.is_cuda:
            raise RuntimeError("DecodeGraph needs a ROCm tensor")
        self.module = module
        self.x = example.detach().clone()
        # Eager warm-up on a side stream, as torch requires before capture
        # (the library and its kernels load, the allocator sees the sizes).
        side = torch.cuda.Stream(device=self.x.device)
        side.wait_stream(torch.cuda.current_stream(self.x.device))
        with torch.cuda.stream(side), torch.no_grad():
            for _ in range(warmup):
                module(self.x)
        torch.cuda.current_stream(self.x.device).wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.no_grad(), torch.cuda.graph(self.graph):
            self.y = module(self.x)
        self.last_indices = module._last_indices
        self.route_weights = module._route_weights  # the graph's fp32 weights buffer
        self.score_dtype = module._score_dtype
        self.last_counts = module._last_counts

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        if x.shape != self.x.shape or x.dtype != self.x.dtype:
            raise ValueError(f"captured for {tuple(self.x.shape)} {self.x.dtype}, got {tuple(x.shape)} {x.dtype}")
        self.x.copy_(x)
        return self.replay()

    def replay(self) -> torch.Tensor:
        """Replay on the current contents of ``self.x`` (for callers that
        write the tokens into the captured input in place, which saves the
        copy of ``__call__``)."""
        self.graph.replay()
        m = self.module
        m.__dict__.update(_last_indices=self.last_indices, _route_weights=self.route_weights,
                          _score_dtype=self.score_dtype, _lw=None, _last_counts=self.last_counts,
                          _counts_of=self.last_indices)
        return self.y
