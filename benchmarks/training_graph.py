"""A complete training step of the model, captured in one HIP graph.

The graph holds the whole step: the gradients cleared in place, the compiled
model and cross entropy under BF16 autocast, the backward of every
microbatch, and a fused, capturable AdamW update.  Replays run it with no
host work; new batches are copied into the static inputs outside the timed
region (``copy_inputs``), then ``replay()``.

The contract and its interface follow the reference's
``benchmarks/training_graph.py`` (``capture_training_step(model, optimizer,
tokens, targets, accumulation=...)``, ``copy_inputs``, ``replay``); the
capture follows PyTorch's rules for ``torch.cuda.graph``: every warm-up
allocation and the static inputs are made on the capture stream, the
gradients are cleared with ``zero_`` (``set_to_none=False``, so replays clear
the same buffers), and the warm-up steps are undone before and after the
capture so that the first replay is the caller's first step.
"""

from __future__ import annotations

import torch
from torch import Tensor
from torch.nn import functional as F


def _loss(logits: Tensor, targets: Tensor) -> Tensor:
    return F.cross_entropy(logits.float().flatten(0, 1), targets.flatten())


def _step(model, loss_fn, optimizer: torch.optim.Optimizer, tokens: Tensor, targets: Tensor,
          accumulation: int) -> Tensor:
    """One optimizer step over ``accumulation`` equal microbatches; returns the
    last microbatch's loss."""
    optimizer.zero_grad(set_to_none=False)
    loss = None
    with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
        for micro_tokens, micro_targets in zip(tokens.chunk(accumulation), targets.chunk(accumulation)):
            loss = loss_fn(model(micro_tokens), micro_targets)
            (loss / accumulation).backward()
    optimizer.step()
    return loss


class _StateSnapshot:
    """Model parameters/buffers and optimizer state, restored in place (the
    graph keeps the tensors' addresses).  Optimizer state that did not exist
    when the snapshot was taken is reset to AdamW's initial values."""

    def __init__(self, model: torch.nn.Module, optimizer: torch.optim.Optimizer) -> None:
        self.model = {name: t.detach().clone() for name, t in model.state_dict().items()}
        self.optimizer = {id(p): {k: (v.detach().clone() if torch.is_tensor(v) else v) for k, v in state.items()}
                          for p, state in optimizer.state.items()}

    @torch.no_grad()
    def restore(self, model: torch.nn.Module, optimizer: torch.optim.Optimizer) -> None:
        current = model.state_dict()
        for name, value in self.model.items():
            current[name].copy_(value)
        for p, state in optimizer.state.items():
            saved = self.optimizer.get(id(p), {})
            for key, value in state.items():
                if torch.is_tensor(value):
                    value.copy_(saved[key]) if key in saved else value.zero_()


class CapturedTrainingStep:
    """A fixed-shape HIP graph of one complete optimizer step."""

    def __init__(self, model: torch.nn.Module, optimizer: torch.optim.Optimizer, tokens: Tensor, targets: Tensor,
                 accumulation: int = 1, warmup: int = 2) -> None:
        if not isinstance(accumulation, int) or isinstance(accumulation, bool) or accumulation < 1:
            raise ValueError("accumulation must be a positive integer")
        if tokens.device.type != "cuda" or targets.device != tokens.device:
            raise ValueError("tokens and targets must be on the same GPU")
        if tokens.ndim != 2 or targets.shape != tokens.shape or tokens.shape[0] % accumulation:
            raise ValueError("tokens and targets: matching [batch, sequence], batch divisible by accumulation")
        for group in optimizer.param_groups:
            if not (group.get("fused") and group.get("capturable")):
                raise ValueError("the optimizer must be built with fused=True and capturable=True")
        self.model, self.optimizer, self.accumulation = model, optimizer, accumulation
        self.compiled_model = torch.compile(model, fullgraph=True, dynamic=False)
        self.compiled_loss = torch.compile(_loss, fullgraph=True, dynamic=False)
        snapshot = _StateSnapshot(model, optimizer)
        self.stream = torch.cuda.Stream(device=tokens.device)
        self.stream.wait_stream(torch.cuda.current_stream(tokens.device))
        with torch.cuda.stream(self.stream):
            self.tokens = tokens.detach().clone()
            self.targets = targets.detach().clone()
            for _ in range(warmup):
                self._run()
            snapshot.restore(model, optimizer)
        self.stream.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=self.stream):
            self.loss = self._run()
        with torch.cuda.stream(self.stream):  # the capture ran one real step: undo it
            snapshot.restore(model, optimizer)
        self.stream.synchronize()
        self.loss = self.loss.detach()

    def _run(self) -> Tensor:
        return _step(self.compiled_model, self.compiled_loss, self.optimizer, self.tokens, self.targets,
                     self.accumulation)

    def copy_inputs(self, tokens: Tensor, targets: Tensor) -> None:
        """Copy a new batch into the graph's inputs (outside any timed region)."""
        if tokens.shape != self.tokens.shape or targets.shape != self.targets.shape:
            raise ValueError("a replay's batch must have the captured shape")
        self.tokens.copy_(tokens)
        self.targets.copy_(targets)

    def replay(self) -> Tensor:
        """Run the captured step; returns its (last microbatch's) loss tensor."""
        self.graph.replay()
        return self.loss


def capture_training_step(model: torch.nn.Module, optimizer: torch.optim.Optimizer, tokens: Tensor,
                          targets: Tensor, *, accumulation: int = 1) -> CapturedTrainingStep:
    """Compile and capture one complete training step for a fixed batch shape.
    The optimizer must be AdamW (or another optimizer) with ``fused=True`` and
    ``capturable=True``; two warm-up steps initialise the compiler and the
    optimizer state and are undone."""
    return CapturedTrainingStep(model, optimizer, tokens, targets, accumulation)


__all__ = ["CapturedTrainingStep", "capture_training_step"]
