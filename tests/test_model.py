"""The model caller (`benchmarks/model.py`) on the CPU with the oracle as its
read: schedules, gradients to every parameter, layouts, training steps.

Follows the properties the reference checks for its caller
(`tests/test_training.py:50-170`, `tests/test_model_routes.py`): the Full
schedule reads 2, 3, ... sources and the Block schedule the completed blocks
plus the running partial; every parameter (all queries included) receives a
gradient; packed and list layouts give identical results; a training step
with accumulation moves the weights.
"""

from __future__ import annotations

import pytest
import torch

from benchmarks.model import TrainingConfig, block_ends, make_model, training_step
from oracle.oracle import oracle


def _tiny(**kwargs) -> TrainingConfig:
    base = dict(layers=2, width=16, heads=4, ffn=32, batch=2, sequence=5, vocab=31, block_count=2)
    base.update(kwargs)
    return TrainingConfig(**base)


def _recording_oracle(seen):
    def read(values, query):
        seen.append(len(values) if isinstance(values, tuple) else values.shape[0])
        return oracle(values, query)
    return read


def test_config_rules():
    with pytest.raises(ValueError, match="rank == width"):
        TrainingConfig(width=16, heads=4, rank=4, variant="standard")
    assert TrainingConfig(width=16, heads=4).rank == 16
    assert TrainingConfig(width=16, heads=4, variant="sliced", rank=4).rank == 4
    for bad in (dict(layers=0), dict(width=15, heads=4), dict(mode="other"), dict(source_layout="x"),
                dict(layers=True), dict(variant="sliced", rank=17, width=16)):
        with pytest.raises(ValueError):
            TrainingConfig(**{**dict(width=16, heads=4), **bad})
    with pytest.raises(TypeError):
        make_model(dict(width=16))
    with pytest.raises(ValueError):
        make_model(_tiny(), backend="other")
    with pytest.raises(ValueError, match="source_bank"):
        make_model(_tiny(), backend=oracle, source_bank=True)
    with pytest.raises(ValueError, match="source_bank"):
        make_model(_tiny(mode="block"), backend=oracle, source_bank=True)


def test_block_ends():
    assert block_ends(4, 2) == (2, 4)
    assert block_ends(5, 2) == (3, 5)
    assert block_ends(3, 8) == (1, 2, 3)
    assert block_ends(48, 8)[-1] == 48 and len(block_ends(48, 8)) == 8


@pytest.mark.parametrize("mode,expected", [("full", [2, 3, 4, 5]), ("block", [2, 2, 3, 3])])
@pytest.mark.parametrize("variant", ["standard", "sliced"])
def test_schedule_and_every_parameter_gets_a_gradient(mode, expected, variant):
    seen = []
    torch.manual_seed(13)
    model = make_model(_tiny(mode=mode, variant=variant, rank=16 if variant == "standard" else 4),
                       backend=_recording_oracle(seen))
    tokens = torch.randint(31, (2, 5))
    logits = model(tokens)
    assert logits.shape == (2, 5, 31)
    assert seen == expected
    logits.float().square().mean().backward()
    for name, parameter in model.named_parameters():
        assert parameter.grad is not None and torch.count_nonzero(parameter.grad) > 0, name
    assert all(torch.count_nonzero(q).item() for q in model.queries)


@pytest.mark.parametrize("mode", ["full", "block"])
def test_list_and_packed_layouts_agree_exactly(mode):
    torch.manual_seed(17)
    packed = make_model(_tiny(mode=mode), backend=oracle)
    listed = make_model(_tiny(mode=mode, source_layout="list"), backend=oracle)
    listed.load_state_dict(packed.state_dict())
    tokens = torch.randint(31, (2, 5))
    a, b = packed(tokens), listed(tokens)
    torch.testing.assert_close(a, b, rtol=0, atol=0)
    a.sum().backward()
    b.sum().backward()
    for (name, p), q in zip(packed.named_parameters(), listed.parameters()):
        torch.testing.assert_close(p.grad, q.grad, rtol=0, atol=0, msg=name)


def test_state_topology_is_stable():
    first, second = make_model(_tiny(), backend=oracle), make_model(_tiny(), backend=oracle)
    assert [(k, tuple(v.shape), v.dtype) for k, v in first.state_dict().items()] == \
           [(k, tuple(v.shape), v.dtype) for k, v in second.state_dict().items()]
    assert len(first.queries) == 2 * first.config.layers


def test_training_step_with_accumulation_moves_weights():
    config = _tiny(layers=1, block_count=1, variant="sliced", rank=3)
    torch.manual_seed(3)
    model = make_model(config, backend=oracle)
    optimizer = torch.optim.AdamW(model.parameters(), lr=1e-2)
    tokens = torch.randint(config.vocab, (2, config.batch, config.sequence))
    targets = torch.randint(config.vocab, (2, config.batch, config.sequence))
    before = {n: p.detach().clone() for n, p in model.named_parameters()}
    loss = training_step(model, optimizer, tokens, targets, accumulation=2)
    assert loss.ndim == 0 and torch.isfinite(loss)
    assert all(not torch.equal(before[n], p) for n, p in model.named_parameters())
    with pytest.raises(ValueError):
        training_step(model, optimizer, tokens, targets, accumulation=3)
    with pytest.raises(ValueError):
        training_step(model, optimizer, tokens[0], targets[0], accumulation=0)


def test_forward_rejects_bad_tokens():
    model = make_model(_tiny(), backend=oracle)
    with pytest.raises(ValueError):
        model(torch.zeros(5, dtype=torch.long))
    with pytest.raises(TypeError):
        model(torch.zeros(2, 5))
    with pytest.raises(ValueError):
        model(torch.zeros(2, 6, dtype=torch.long))
