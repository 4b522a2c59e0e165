"""Captured decode-step graphs of the MoE block per token bucket.

The reference engine captures one HIP graph per decode bucket and replays the smallest
bucket that holds a step's rows (engine/fast/model.py:1947-2093, buckets
``DECODE_BUCKETS`` model.py:67-68, ``ENGINE_DECODE_BUCKETS``). ``MoeGraphs`` does the same
for one MoE block call: per bucket it keeps static input and output buffers, warms the
call up on its capture stream (so the library's workspace for that stream exists before
capture and stays the graph's static workspace) and captures it; ``run`` copies the rows
in, replays and returns a view of the first B output rows.

Padding rows repeat the step's last row: they route to experts the step already uses, so
they add no expert weight traffic (a zero row would route to experts of its own), and a
row's output does not depend on the other rows of its call, so the real rows' bits are
those of an eager call on the padded batch.
"""

from __future__ import annotations

import os

import torch

from . import _lib, block

# engine/fast/model.py:67-68
DECODE_BUCKETS = tuple(sorted({int(b) for b in os.environ.get(
    "ENGINE_DECODE_BUCKETS", "1,2,3,4,5,6,8,16,32").split(",") if b.strip()}))


class MoeGraphs:
    """Graphs of ``block.moe(x, mlp, top_k, decode=True, residual=r)`` per bucket, or with
    ``norm=(weight, eps)`` of ``block.add_rms_moe(x, h, weight, eps, mlp, top_k,
    decode=True)``; ``run(x, second)`` takes r (respectively h) as its second input."""

    def __init__(self, mlp, top_k: int, hidden: int, device, buckets=DECODE_BUCKETS,
                 norm=None):
        self.mlp, self.top_k, self.hidden = mlp, top_k, hidden
        self.device = torch.device(device)
        self.buckets = tuple(sorted(buckets))
        self.norm = norm
        self.stream = torch.cuda.Stream(self.device)
        self.pool = torch.cuda.graph_pool_handle()
        self.graphs: dict[int, tuple] = {}

    def bucket(self, rows: int) -> int:
        for b in self.buckets:
            if b >= rows:
                return b
        raise ValueError(f"{rows} rows exceed the largest bucket {self.buckets[-1]}")

    def _call(self, x, y):
        if self.norm is None:
            return block.moe(x, self.mlp, self.top_k, decode=True, residual=y)
        w, eps = self.norm
        return block.add_rms_moe(x, y, w, eps, self.mlp, self.top_k, decode=True)

    def capture(self, size: int) -> None:
        """Capture bucket ``size`` (done on first use by ``run``)."""
        x = torch.zeros(size, self.hidden, dtype=torch.bfloat16, device=self.device)
        y = torch.zeros_like(x)
        self.stream.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(self.stream):
            self._call(x, y)  # workspace and router pack outside the capture
            # the graph keeps this workspace: a larger bucket's warm-up may replace the
            # stream's workspace, and the graphs captured before still address this one
            ws = _lib.workspace(self.device, 0)
        torch.cuda.current_stream(self.device).wait_stream(self.stream)
        torch.cuda.synchronize(self.device)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, pool=self.pool, stream=self.stream):
            out = self._call(x, y)
        torch.cuda.synchronize(self.device)
        self.graphs[size] = (graph, x, y, out, ws)

    def run(self, x: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
        """The block's output for the rows of ``x`` [B, H] (and ``y``), replayed from the
        smallest bucket >= B on the current stream. The result is a view of the bucket's
        static output: copy it before the next ``run`` of the same bucket."""
        rows = x.shape[0]
        if rows == 0:
            return torch.empty(0, self.hidden, dtype=torch.bfloat16, device=self.device)
        size = self.bucket(rows)
        if size not in self.graphs:
            self.capture(size)
        graph, xs, ys, out, _ = self.graphs[size]
        xs[:rows].copy_(x)
        ys[:rows].copy_(y)
        if rows < size:
            xs[rows:].copy_(x[rows - 1 : rows].expand(size - rows, -1))
            ys[rows:].copy_(y[rows - 1 : rows].expand(size - rows, -1))
        graph.replay()
        return out[:rows]
