"""The model caller on the GPU: the HIP read inside the residual stream.

The model (FP32 outside the reads, as in the reference's default) is run with
the HIP operator on the GPU and with the CPU oracle on the same weights; the
logits and every parameter gradient must agree within a BF16-read tolerance
(each read rounds its output to BF16 once, as the oracle does, so the models
differ only by the reads' last-ulp differences carried through the layers).
The reference qualifies its model path the same way, by loss and gradient
parity against the oracle-backed model (`tests/test_pre_timing_gate.py:70-113`).
"""

from __future__ import annotations

import copy

import pytest
import torch

from benchmarks.model import TrainingConfig, make_model, training_step
from oracle.oracle import oracle

pytestmark = pytest.mark.gpu


def _config(mode, layout, variant):
    return TrainingConfig(layers=3, width=64, heads=4, ffn=128, batch=2, sequence=32, vocab=97,
                          block_count=2, mode=mode, source_layout=layout, variant=variant,
                          rank=64 if variant == "standard" else 16)


def _relative_error(a, b):
    return float((a - b).abs().max() / b.abs().max().clamp_min(1e-12))


@pytest.mark.parametrize("variant", ["standard", "sliced"])
@pytest.mark.parametrize("layout", ["packed", "list"])
@pytest.mark.parametrize("mode", ["full", "block"])
def test_model_matches_oracle_model(mode, layout, variant):
    config = _config(mode, layout, variant)
    print(f"model parity mode={mode} layout={layout} variant={variant}", flush=True)
    torch.manual_seed(11)
    reference = make_model(config, backend=oracle)
    candidate = make_model(config, backend="kernel")
    candidate.load_state_dict(reference.state_dict())
    candidate.cuda()
    tokens = torch.randint(config.vocab, (config.batch, config.sequence))
    expected = reference(tokens)
    actual = candidate(tokens.cuda())
    assert _relative_error(actual.cpu(), expected) < 2e-2
    weight = torch.randn(expected.shape)
    (expected * weight).sum().backward()
    (actual * weight.cuda()).sum().backward()
    for (name, p), q in zip(candidate.named_parameters(), reference.parameters()):
        assert p.grad is not None, name
        assert _relative_error(p.grad.cpu(), q.grad) < 5e-2, name


@pytest.mark.parametrize("mode", ["full", "block"])
def test_compiled_model_step_matches_eager(mode):
    config = _config(mode, "packed", "standard")
    print(f"compiled model mode={mode}", flush=True)
    torch.manual_seed(23)
    eager = make_model(config, backend="kernel").cuda()
    compiled_model = copy.deepcopy(eager)
    tokens = torch.randint(config.vocab, (config.batch, config.sequence), device="cuda")
    compiled = torch.compile(compiled_model, fullgraph=True, backend="aot_eager")
    a = eager(tokens)
    b = compiled(tokens)
    torch.testing.assert_close(b, a, rtol=1e-4, atol=1e-5)
    a.float().square().mean().backward()
    b.float().square().mean().backward()
    for (name, p), q in zip(eager.named_parameters(), compiled_model.parameters()):
        torch.testing.assert_close(q.grad, p.grad, rtol=1e-3, atol=1e-6, msg=name)


def test_training_steps_reduce_the_loss():
    config = _config("block", "list", "standard")
    torch.manual_seed(29)
    model = make_model(config, backend="kernel").cuda()
    optimizer = torch.optim.AdamW(model.parameters(), lr=3e-3)
    tokens = torch.randint(config.vocab, (config.batch, config.sequence), device="cuda")
    targets = torch.roll(tokens, -1, dims=1)
    losses = [float(training_step(model, optimizer, tokens, targets)) for _ in range(12)]
    assert all(torch.isfinite(torch.tensor(losses)))
    assert losses[-1] < losses[0]


def test_source_bank_model_matches_the_plain_model():
    config = _config("full", "packed", "standard")
    torch.manual_seed(37)
    plain = make_model(config, backend="kernel").cuda()
    banked = make_model(config, backend="kernel", source_bank=True).cuda()
    banked.load_state_dict(plain.state_dict())
    tokens = torch.randint(config.vocab, (config.batch, config.sequence), device="cuda")
    a, b = plain(tokens), banked(tokens)
    assert torch.equal(a, b)
    weight = torch.randn_like(a)
    (a * weight).sum().backward()
    (b * weight).sum().backward()
    for (name, p), q in zip(plain.named_parameters(), banked.parameters()):
        assert _relative_error(q.grad, p.grad) < 2e-2, name


@pytest.mark.parametrize("blocks", [2, 3])
def test_block_source_bank_model_matches_the_plain_model(blocks):
    config = TrainingConfig(layers=3, width=64, heads=4, ffn=128, batch=2, sequence=32, vocab=97,
                            block_count=blocks, mode="block", source_layout="packed", variant="standard")
    torch.manual_seed(53)
    plain = make_model(config, backend="kernel").cuda()
    banked = make_model(config, backend="kernel", source_bank=True).cuda()
    banked.load_state_dict(plain.state_dict())
    tokens = torch.randint(config.vocab, (config.batch, config.sequence), device="cuda")
    print(f"block bank model blocks={blocks}", flush=True)
    a, b = plain(tokens), banked(tokens)
    assert torch.equal(a, b)
    weight = torch.randn_like(a)
    (a * weight).sum().backward()
    (b * weight).sum().backward()
    for (name, p), q in zip(plain.named_parameters(), banked.parameters()):
        assert _relative_error(q.grad, p.grad) < 2e-2, name


@pytest.mark.parametrize("mode", ["full", "block"])
def test_inductor_compiled_model_step_matches_eager(mode):
    """The default torch.compile backend (inductor) around the whole model,
    fullgraph: the reads stay opaque custom ops between inductor's fused
    kernels; logits and parameter gradients match the eager model."""
    config = _config(mode, "packed", "standard")
    print(f"inductor model mode={mode}", flush=True)
    torch.manual_seed(61)
    eager = make_model(config, backend="kernel").cuda()
    compiled_model = copy.deepcopy(eager)
    tokens = torch.randint(config.vocab, (config.batch, config.sequence), device="cuda")
    torch._dynamo.reset()
    compiled = torch.compile(compiled_model, fullgraph=True)
    a = eager(tokens)
    b = compiled(tokens)
    torch.testing.assert_close(b, a, rtol=1e-4, atol=1e-5)
    a.float().square().mean().backward()
    b.float().square().mean().backward()
    for (name, p), q in zip(eager.named_parameters(), compiled_model.parameters()):
        assert _relative_error(q.grad, p.grad) < 1e-2, name


@pytest.mark.parametrize("mode", ["full", "block"])
def test_bank_model_with_compiled_sublayers_matches_eager(mode):
    """Regional compilation (each sublayer under inductor) around the eager
    source bank: the same logits and gradients as the eager bank model, to FP32
    reordering."""
    config = _config(mode, "packed", "standard")
    print(f"compiled sublayers + bank mode={mode}", flush=True)
    torch.manual_seed(71)
    eager = make_model(config, backend="kernel", source_bank=True).cuda()
    torch._dynamo.reset()
    compiled = make_model(config, backend="kernel", source_bank=True, compile_layers=True).cuda()
    compiled.load_state_dict(eager.state_dict())
    tokens = torch.randint(config.vocab, (config.batch, config.sequence), device="cuda")
    a, b = eager(tokens), compiled(tokens)
    torch.testing.assert_close(b, a, rtol=1e-3, atol=1e-4)
    a.float().square().mean().backward()
    b.float().square().mean().backward()
    for (name, p), q in zip(eager.named_parameters(), compiled.parameters()):
        assert _relative_error(q.grad, p.grad) < 2e-2, name


@pytest.mark.parametrize("mode", ["full", "block"])
def test_bf16_autocast_model_with_and_without_the_bank(mode):
    """Under BF16 autocast the residual stream is BF16 (the embedding is cast,
    reference model.py:243-244): the plain and the source-bank model give the
    same logits, close gradients, and a few training steps reduce the loss."""
    config = _config(mode, "packed", "standard")
    print(f"bf16 autocast model mode={mode}", flush=True)
    torch.manual_seed(73)
    plain = make_model(config, backend="kernel").cuda()
    banked = make_model(config, backend="kernel", source_bank=True).cuda()
    banked.load_state_dict(plain.state_dict())
    tokens = torch.randint(config.vocab, (config.batch, config.sequence), device="cuda")
    with torch.autocast("cuda", dtype=torch.bfloat16):
        a, b = plain(tokens), banked(tokens)
        assert a.dtype == torch.bfloat16
        assert torch.equal(a, b)
        weight = torch.randn_like(a, dtype=torch.float32)
        (a.float() * weight).sum().backward()
        (b.float() * weight).sum().backward()
    for (name, p), q in zip(plain.named_parameters(), banked.parameters()):
        assert _relative_error(q.grad, p.grad) < 3e-2, name
    optimizer = torch.optim.AdamW(banked.parameters(), lr=3e-3)
    targets = torch.roll(tokens, -1, dims=1)
    losses = []
    for _ in range(8):
        # one autocast context per step: a context kept across steps reuses its BF16 weight casts
        with torch.autocast("cuda", dtype=torch.bfloat16):
            losses.append(float(training_step(banked, optimizer, tokens, targets)))
    assert losses[-1] < losses[0]


@pytest.mark.parametrize("layout", ["packed", "list"])
@pytest.mark.parametrize("mode", ["full", "block"])
def test_checkpointed_compiled_model_matches_oracle_model(mode, layout):
    """Activation checkpointing through the reads (reference
    validation/training_checks.py:35-37, 79-88): the model under
    torch.utils.checkpoint(..., use_reentrant=False) inside
    torch.compile(fullgraph=True) against the oracle-backed model on the same
    weights, and against the same HIP model without checkpointing.  With 3
    layers the Full schedule reads 1..7 sources, so both the recompute reads
    (S <= 6) and a saving read (S = 7) run their forward twice (once more in
    the backward's recomputation)."""
    from torch.utils.checkpoint import checkpoint

    config = _config(mode, layout, "standard")
    print(f"checkpointed compiled model mode={mode} layout={layout}", flush=True)
    torch.manual_seed(31)
    reference = make_model(config, backend=oracle)
    candidate = make_model(config, backend="kernel")
    candidate.load_state_dict(reference.state_dict())
    candidate.cuda()
    plain = copy.deepcopy(candidate)
    tokens = torch.randint(config.vocab, (config.batch, config.sequence))
    weight = torch.randn(config.batch, config.sequence, config.vocab)
    torch._dynamo.reset()
    checked = torch.compile(lambda x: checkpoint(candidate, x, use_reentrant=False), fullgraph=True, dynamic=False)
    actual = checked(tokens.cuda())
    expected = reference(tokens)
    baseline = plain(tokens.cuda())
    assert _relative_error(actual.cpu(), expected) < 2e-2
    # inductor reorders the FP32 work around the reads, which can move a read's BF16 rounding
    assert _relative_error(actual, baseline) < 1e-2
    (expected * weight).sum().backward()
    (actual * weight.cuda()).sum().backward()
    (baseline * weight.cuda()).sum().backward()
    for (name, p), q, b in zip(candidate.named_parameters(), reference.parameters(), plain.parameters()):
        assert p.grad is not None, name
        assert _relative_error(p.grad.cpu(), q.grad) < 5e-2, name
        assert _relative_error(p.grad, b.grad) < 2e-2, name


@pytest.mark.parametrize("gradients", ["gather", "accumulate"])
@pytest.mark.parametrize("mode", ["full", "block"])
def test_checkpointed_bank_model_matches_the_bank_model(mode, gradients):
    """The source-bank model (eager) under torch.utils.checkpoint(...,
    use_reentrant=False): the backward re-runs the forward, building a second
    bank whose reads give the same bits; gradients equal the bank model's
    without checkpointing."""
    from torch.utils.checkpoint import checkpoint

    config = _config(mode, "packed", "standard")
    print(f"checkpointed bank model mode={mode} gradients={gradients}", flush=True)
    torch.manual_seed(37)
    model = make_model(config, backend="kernel", source_bank=True, bank_gradients=gradients).cuda()
    other = copy.deepcopy(model)
    tokens = torch.randint(config.vocab, (config.batch, config.sequence), device="cuda")
    weight = torch.randn(config.batch, config.sequence, config.vocab, device="cuda")
    a = checkpoint(model, tokens, use_reentrant=False)
    b = other(tokens)
    assert torch.equal(a, b)
    (a * weight).sum().backward()
    (b * weight).sum().backward()
    for (name, p), q in zip(model.named_parameters(), other.parameters()):
        assert p.grad is not None, name
        torch.testing.assert_close(p.grad, q.grad, rtol=1e-5, atol=1e-7, msg=name)


@pytest.mark.parametrize("mode", ["full", "block"])
def test_captured_training_step_matches_compiled_steps(mode):
    """A whole training step in one HIP graph (benchmarks/training_graph.py:
    compiled model and loss under BF16 autocast, two accumulated microbatches,
    fused capturable AdamW): three replays on changed batches give the losses
    and parameters of three compiled steps run eagerly from the same start."""
    from benchmarks.training_graph import _loss, _step, capture_training_step

    config = _config(mode, "packed", "standard")
    print(f"captured training step mode={mode}", flush=True)
    torch.manual_seed(41)
    model = make_model(config, backend="kernel").cuda()
    twin = copy.deepcopy(model)
    optimizer = torch.optim.AdamW(model.parameters(), lr=1e-3, fused=True, capturable=True)
    twin_optimizer = torch.optim.AdamW(twin.parameters(), lr=1e-3, fused=True, capturable=True)
    batches = [(torch.randint(config.vocab, (2 * config.batch, config.sequence), device="cuda"),
                torch.randint(config.vocab, (2 * config.batch, config.sequence), device="cuda")) for _ in range(3)]
    torch._dynamo.reset()
    captured = capture_training_step(model, optimizer, *batches[0], accumulation=2)
    twin_model = torch.compile(twin, fullgraph=True, dynamic=False)
    twin_loss = torch.compile(_loss, fullgraph=True, dynamic=False)
    for index, (tokens, targets) in enumerate(batches):
        captured.copy_inputs(tokens, targets)
        loss = captured.replay().clone()
        expected = _step(twin_model, twin_loss, twin_optimizer, tokens, targets, 2)
        torch.cuda.synchronize()
        torch.testing.assert_close(loss, expected.detach(), rtol=1e-4, atol=1e-5, msg=f"step {index}")
    for (name, p), q in zip(model.named_parameters(), twin.parameters()):
        torch.testing.assert_close(p, q, rtol=1e-4, atol=1e-6, msg=name)
