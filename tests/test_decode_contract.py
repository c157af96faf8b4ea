"""Contract errors of the decode-loop mirror, raised before any GPU work
(CBT/core.py:42-46, :71-74, :207-224): the same exception types as the reference."""

from types import SimpleNamespace

import pytest
import torch

from interattn_amd import decode


def _method(**kw):
    base = dict(condition_delta_mode="range_bound", condition_block_size=64, condition_eps=0.1,
                full_attention_layers=0, max_new_tokens=4)
    base.update(kw)
    return SimpleNamespace(**base)


def _call(ids, method, fn=decode.generate_condition_block_cached):
    return fn(model=None, tokenizer=None, input_ids=ids, attention_mask=torch.ones_like(ids), method=method,
              **({"device": "cpu"} if fn is decode.generate_condition_block_cached else {}))


def test_delta_mode_must_be_range_bound():
    with pytest.raises(ValueError, match="range_bound"):
        _call(torch.zeros((1, 4), dtype=torch.long), _method(condition_delta_mode="ball"))


def test_batch_must_be_one():
    with pytest.raises(ValueError, match="batch_size=1"):
        _call(torch.zeros((2, 4), dtype=torch.long), _method())


def test_graph_loop_requires_skip_stats(monkeypatch):
    monkeypatch.delenv("CONDITION_BLOCK_SKIP_STATS", raising=False)
    with pytest.raises(ValueError, match="SKIP_STATS"):
        _call(torch.zeros((1, 4), dtype=torch.long), _method(), fn=decode._generate_condition_block_cuda_graph)


def test_graph_loop_requires_no_dense_layers(monkeypatch):
    monkeypatch.setenv("CONDITION_BLOCK_SKIP_STATS", "1")
    with pytest.raises(ValueError, match="full_attention_layers=0"):
        _call(torch.zeros((1, 4), dtype=torch.long), _method(full_attention_layers=2),
              fn=decode._generate_condition_block_cuda_graph)


def test_prefill_only_entry_is_removed():
    with pytest.raises(RuntimeError):
        decode.run_prefill_only_condition_block()


def test_stats_helpers(monkeypatch):
    monkeypatch.delenv("CONDITION_BLOCK_SKIP_STATS", raising=False)
    s = decode.full_attention_stats_for_heads(32, [9, 19])
    assert s["rows"] == 64 and s["total_available"] == (10 + 20) * 32 == s["hybrid_tokens"]
    agg, by = {}, {}
    decode._merge_stats_lazy(agg, s)
    decode._merge_stats_lazy(agg, s)
    assert agg["rows"] == 128
    summ = decode.summarize_condition_block_step_metadata([decode._summarize_stats_lazy(agg, by)])
    assert summ["condition_block_equiv_budget"] == 1.0


def test_mask_is_prefix_decision():
    import torch

    from interattn_amd.condition_block import _MASK_PREFIX_HINT, mask_is_prefix, mask_prefix_hint

    assert mask_is_prefix(torch.ones((1, 7), dtype=torch.long))
    assert mask_is_prefix(torch.tensor([[1, 1, 1, 0, 0], [1, 0, 0, 0, 0]]))
    assert not mask_is_prefix(torch.tensor([[0, 0, 1, 1, 1]]))      # left padding
    assert not mask_is_prefix(torch.tensor([[1, 0, 1, 1, 1]]))      # a hole
    assert _MASK_PREFIX_HINT.get() is None
    with mask_prefix_hint(False):
        assert _MASK_PREFIX_HINT.get() is False
        with mask_prefix_hint(True):
            assert _MASK_PREFIX_HINT.get() is True
        assert _MASK_PREFIX_HINT.get() is False
    assert _MASK_PREFIX_HINT.get() is None
