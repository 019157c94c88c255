"""The caller of the hot path: a compact causal language model whose residual
stream is a sequence of AttnRes reads.

Mirrors the interface of the reference's `benchmarks/model.py`
(`TrainingConfig` :56-117, `CausalAttnResLM` :180-355, `make_model` :358-367,
`training_step` :504-530): every sublayer output (attention, then MLP) becomes
a depth source, and the input of every later sublayer and of the LM head is a
read ``attnres(sources, query_i)`` with one learned query per read.

* Full schedule: a read sees the embedding and every earlier sublayer output
  (S = 1 .. 2L+1 sources).
* Block schedule: sublayer outputs are summed into blocks (``block_count``
  evenly sized blocks of source events); a read sees the completed blocks and
  the running partial sum of the current block.

The surrounding Transformer is ordinary PyTorch in the model's dtype; reads
cast their sources to BF16 and their output back (reference `_read`,
model.py:279-291).  Under ``torch.autocast`` the embedding is cast to the
autocast dtype (reference model.py:243-244), so with BF16 autocast the whole
residual stream is BF16 and those casts are no-ops.  ``backend`` is ``"kernel"`` (the HIP operator) or any
callable with the ``attnres`` signature, e.g. the CPU oracle for parity tests.

``source_bank=True`` (HIP backend; no reference counterpart) keeps the
residual stream in an ``attnres.SourceBank``: each source is cast to BF16
once, reads take slots of one packed buffer, and the reads' backward sums
every source's gradient in FP32 inside the kernels, instead of the per-read
casts, stacks and autograd additions of the plain path.  In the Block
schedule, completed blocks sit in slots 0..k and each running partial in a
slot of its own; ``push_sum`` forms the partial and its BF16 copy in one
kernel (the caller step of reference model.py:333 fused with the next read's
cast), and the block's last partial is written straight into the next
completed slot.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Callable, Sequence

import torch
from torch import Tensor, nn
from torch.nn import functional as F

Backend = str | Callable[..., Tensor]


@dataclass
class TrainingConfig:
    """Shape and schedule of :class:`CausalAttnResLM` (reference model.py:56-117).

    ``rank`` defaults to ``width`` (standard AttnRes); ``variant="sliced"``
    allows ``rank < width`` (keys are the last ``rank`` coordinates).
    ``source_layout`` chooses how a read passes its sources: one packed
    ``[S, B, T, D]`` tensor (a stack) or an ordered tuple (no copy).
    """

    layers: int = 2
    width: int = 128
    heads: int = 4
    ffn: int = 384
    batch: int = 2
    sequence: int = 64
    vocab: int = 512
    block_count: int = 2
    variant: str = "standard"
    mode: str = "full"
    rank: int | None = None
    source_layout: str = "packed"

    def __post_init__(self) -> None:
        for name in ("layers", "width", "heads", "ffn", "batch", "sequence", "vocab", "block_count"):
            value = getattr(self, name)
            if isinstance(value, bool) or not isinstance(value, int) or value < 1:
                raise ValueError(f"{name} must be a positive integer")
        if self.width % self.heads:
            raise ValueError("width must be divisible by heads")
        self.variant, self.mode, self.source_layout = (
            str(self.variant).lower(), str(self.mode).lower(), str(self.source_layout).lower())
        if self.variant not in ("standard", "sliced"):
            raise ValueError("variant must be 'standard' or 'sliced'")
        if self.mode not in ("full", "block"):
            raise ValueError("mode must be 'full' or 'block'")
        if self.source_layout not in ("packed", "list"):
            raise ValueError("source_layout must be 'packed' or 'list'")
        if self.rank is None:
            self.rank = self.width
        if isinstance(self.rank, bool) or not isinstance(self.rank, int) or not 1 <= self.rank <= self.width:
            raise ValueError("rank must be an integer with 1 <= rank <= width")
        if self.variant == "standard" and self.rank != self.width:
            raise ValueError("standard AttnRes requires rank == width")


def block_ends(events: int, blocks: int) -> tuple[int, ...]:
    """One-based event indices that close each of ``min(events, blocks)``
    evenly sized blocks of source events (reference model.py:120-125)."""
    count = min(events, blocks)
    return tuple(math.ceil(events * i / count) for i in range(1, count + 1))


class TransformerLayer(nn.Module):
    """Pre-norm causal self-attention and a SwiGLU MLP, as two sublayers."""

    def __init__(self, config: TrainingConfig) -> None:
        super().__init__()
        d = config.width
        self.heads = config.heads
        self.attn_norm = nn.LayerNorm(d)
        self.qkv = nn.Linear(d, 3 * d, bias=False)
        self.attn_out = nn.Linear(d, d, bias=False)
        self.mlp_norm = nn.LayerNorm(d)
        self.gate_up = nn.Linear(d, 2 * config.ffn, bias=False)
        self.down = nn.Linear(config.ffn, d, bias=False)

    def attention(self, x: Tensor) -> Tensor:
        b, t, d = x.shape
        q, k, v = self.qkv(self.attn_norm(x)).view(b, t, 3, self.heads, d // self.heads).unbind(2)
        y = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2),
                                           is_causal=True)
        return self.attn_out(y.transpose(1, 2).reshape(b, t, d))

    def mlp(self, x: Tensor) -> Tensor:
        gate, up = self.gate_up(self.mlp_norm(x)).chunk(2, dim=-1)
        return self.down(F.silu(gate) * up)


class CausalAttnResLM(nn.Module):
    """Small causal Transformer with Full or Block AttnRes residual reads."""

    def __init__(self, config: TrainingConfig, backend: Backend = "kernel", *, source_bank: bool = False,
                 bank_gradients: str = "gather", compile_layers: bool = False) -> None:
        super().__init__()
        if source_bank and backend != "kernel":
            raise ValueError("source_bank needs the HIP backend")
        if bank_gradients not in ("gather", "accumulate"):
            raise ValueError("bank_gradients must be 'gather' or 'accumulate'")
        self.config = config
        self.backend = backend
        self.source_bank = bool(source_bank)
        self.bank_gradients = bank_gradients
        self.token_embedding = nn.Embedding(config.vocab, config.width)
        self.position_embedding = nn.Parameter(torch.empty(config.sequence, config.width))
        self.layers = nn.ModuleList(TransformerLayer(config) for _ in range(config.layers))
        self.lm_head = nn.Linear(config.width, config.vocab, bias=False)
        # one query per read: before sublayers 2 .. 2L and before the LM head
        self.queries = nn.ParameterList(nn.Parameter(torch.empty(config.rank)) for _ in range(2 * config.layers))
        self.reset_parameters()
        if compile_layers:
            # regional compilation: each sublayer fused by inductor, while the residual stream
            # (reads, source bank) between them stays eager
            for layer in self.layers:
                layer.attention = torch.compile(layer.attention, fullgraph=True)
                layer.mlp = torch.compile(layer.mlp, fullgraph=True)

    def reset_parameters(self) -> None:
        for module in self.modules():
            if isinstance(module, (nn.Linear, nn.Embedding)):
                nn.init.normal_(module.weight, std=0.02)
            elif isinstance(module, nn.LayerNorm):
                nn.init.ones_(module.weight)
                nn.init.zeros_(module.bias)
        nn.init.normal_(self.position_embedding, std=0.02)
        for query in self.queries:  # non-zero: the first reads are not uniform averages
            nn.init.normal_(query, std=0.02)

    def _operator(self) -> Callable[..., Tensor]:
        if self.backend == "kernel":
            from attnres import attnres

            return attnres
        if callable(self.backend):
            return self.backend
        raise ValueError("backend must be 'kernel' or a callable")

    def read(self, sources: Sequence[Tensor], query: Tensor) -> Tensor:
        """One residual read: BF16 sources and query, output in the model dtype."""
        dtype = sources[0].dtype
        bf16 = tuple(source.to(torch.bfloat16) for source in sources)
        values = bf16 if self.config.source_layout == "list" else torch.stack(bf16, dim=0)
        return self._operator()(values, query.to(torch.bfloat16)).to(dtype)

    def _sublayer(self, event: int, x: Tensor) -> Tensor:
        layer = self.layers[event // 2]
        return layer.attention(x) if event % 2 == 0 else layer.mlp(x)

    def _forward_full_bank(self, embedded: Tensor) -> Tensor:
        from attnres import SourceBank

        bank = SourceBank(2 * self.config.layers + 1, gradients=self.bank_gradients)
        bank.push(embedded)
        for event in range(2 * self.config.layers):
            x = embedded if event == 0 else bank.read(self.queries[event - 1].to(torch.bfloat16)).to(embedded.dtype)
            bank.push(self._sublayer(event, x))
        return bank.read(self.queries[-1].to(torch.bfloat16)).to(embedded.dtype)

    def _forward_full(self, embedded: Tensor) -> Tensor:
        if self.source_bank:
            return self._forward_full_bank(embedded)
        sources = [embedded]
        for event in range(2 * self.config.layers):
            x = embedded if event == 0 else self.read(sources, self.queries[event - 1])
            sources.append(self._sublayer(event, x))
        return self.read(sources, self.queries[-1])

    def _forward_block_bank(self, embedded: Tensor) -> Tensor:
        from attnres import SourceBank

        events = 2 * self.config.layers
        ends = block_ends(events, self.config.block_count)
        # slots 0..len(ends): the embedding and the completed blocks; then one per mid-block partial
        bank = SourceBank(len(ends) + 1 + events - len(ends), gradients=self.bank_gradients)
        bank.push(embedded, slot=0)
        completed, scratch, event = 1, len(ends) + 1, 0
        for end in ends:
            partial: Tensor | None = None
            tail: int | None = None
            while event < end:
                if event == 0:
                    x = embedded
                else:
                    query = self.queries[event - 1].to(torch.bfloat16)
                    x = bank.read(query, count=completed, tail=tail).to(embedded.dtype)
                emitted = self._sublayer(event, x)
                event += 1
                slot = completed if event == end else scratch  # the block's last partial is its completed slot
                if slot == scratch:
                    scratch += 1
                if partial is None:
                    partial = emitted
                    bank.push(emitted, slot=slot)
                else:
                    partial = bank.push_sum(partial, emitted, slot=slot)
                tail = slot
            completed += 1
        return bank.read(self.queries[-1].to(torch.bfloat16), count=completed).to(embedded.dtype)

    def _forward_block(self, embedded: Tensor) -> Tensor:
        if self.source_bank:
            return self._forward_block_bank(embedded)
        events = 2 * self.config.layers
        completed = [embedded]
        partial: Tensor | None = None
        event = 0
        for end in block_ends(events, self.config.block_count):
            while event < end:
                if event == 0:
                    x = embedded
                else:
                    x = self.read(completed if partial is None else [*completed, partial], self.queries[event - 1])
                emitted = self._sublayer(event, x)
                partial = emitted if partial is None else partial + emitted
                event += 1
            completed.append(partial)
            partial = None
        return self.read(completed, self.queries[-1])

    def forward(self, tokens: Tensor) -> Tensor:
        if tokens.ndim != 2:
            raise ValueError("tokens must have shape [batch, sequence]")
        if tokens.dtype.is_floating_point or tokens.dtype == torch.bool:
            raise TypeError("tokens must contain integer token ids")
        if tokens.shape[1] > self.config.sequence:
            raise ValueError("token sequence exceeds configured sequence length")
        embedded = self.token_embedding(tokens) + self.position_embedding[: tokens.shape[1]]
        if torch.is_autocast_enabled(embedded.device.type):  # the stream in the autocast dtype (model.py:243-244)
            embedded = embedded.to(torch.get_autocast_dtype(embedded.device.type))
        hidden = self._forward_full(embedded) if self.config.mode == "full" else self._forward_block(embedded)
        return self.lm_head(hidden)


def make_model(config: TrainingConfig, backend: Backend = "kernel", *, source_bank: bool = False,
               bank_gradients: str = "gather", compile_layers: bool = False) -> CausalAttnResLM:
    """Construct a model with the given residual-read backend (``bank_gradients``:
    the source bank's gradient path, see ``attnres.SourceBank``; ``compile_layers``:
    each attention and MLP sublayer under ``torch.compile(fullgraph=True)``)."""
    if not isinstance(config, TrainingConfig):
        raise TypeError("config must be a TrainingConfig")
    if not (backend == "kernel" or callable(backend)):
        raise ValueError("backend must be 'kernel' or a callable")
    return CausalAttnResLM(config, backend, source_bank=source_bank, bank_gradients=bank_gradients,
                           compile_layers=compile_layers)


def training_step(model: nn.Module, optimizer: torch.optim.Optimizer, tokens: Tensor, targets: Tensor,
                  *, accumulation: int = 1) -> Tensor:
    """One optimizer step over ``accumulation`` micro-batches (split along the
    batch axis, or given as a leading axis); returns the detached mean loss
    (reference model.py:504-530)."""
    if isinstance(accumulation, bool) or not isinstance(accumulation, int) or accumulation < 1:
        raise ValueError("accumulation must be a positive integer")
    if tokens.shape != targets.shape:
        raise ValueError("tokens and targets must have matching shapes")
    if tokens.ndim == 3:
        if tokens.shape[0] != accumulation:
            raise ValueError("3D token input must have leading dimension equal to accumulation")
        batches = list(zip(tokens.unbind(0), targets.unbind(0)))
    elif tokens.ndim == 2:
        if tokens.shape[0] < accumulation:
            raise ValueError("batch dimension must be at least accumulation")
        batches = list(zip(tokens.tensor_split(accumulation), targets.tensor_split(accumulation)))
    else:
        raise ValueError("tokens and targets must have shape [batch, sequence]")
    optimizer.zero_grad(set_to_none=True)
    losses = []
    for micro_tokens, micro_targets in batches:
        logits = model(micro_tokens)
        loss = F.cross_entropy(logits.reshape(-1, logits.shape[-1]).float(), micro_targets.reshape(-1))
        losses.append(loss.detach())
        (loss / len(batches)).backward()
    optimizer.step()
    return torch.stack(losses).mean()


__all__ = ["TrainingConfig", "CausalAttnResLM", "TransformerLayer", "block_ends", "make_model", "training_step"]
