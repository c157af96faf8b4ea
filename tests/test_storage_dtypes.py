"""Summary storage dtypes follow the reference's switches and errors
(``_summary_storage_dtypes``, CBT/core.py:411-446)."""

import pytest
import torch

from interattn_amd.condition_block import _summary_storage_dtypes


@pytest.fixture(autouse=True)
def _clean(monkeypatch):
    for name in ("CONDITION_BLOCK_SUMMARY_DTYPE", "CONDITION_BLOCK_MIXED_SUMMARIES", "CONDITION_BLOCK_K_BAR_DTYPE"):
        monkeypatch.delenv(name, raising=False)


def test_default_is_float32():
    assert _summary_storage_dtypes(torch.bfloat16) == (torch.float32,) * 3


def test_mixed_layout(monkeypatch):
    monkeypatch.setenv("CONDITION_BLOCK_MIXED_SUMMARIES", "1")
    assert _summary_storage_dtypes(torch.bfloat16) == (torch.float32, torch.bfloat16, torch.bfloat16)
    monkeypatch.setenv("CONDITION_BLOCK_K_BAR_DTYPE", "bfloat16")
    assert _summary_storage_dtypes(torch.bfloat16) == (torch.bfloat16, torch.bfloat16, torch.bfloat16)
    assert _summary_storage_dtypes(torch.float32) == (torch.bfloat16, torch.bfloat16, torch.float32)


def test_uniform_bf16(monkeypatch):
    monkeypatch.setenv("CONDITION_BLOCK_SUMMARY_DTYPE", "bfloat16")
    assert _summary_storage_dtypes(torch.bfloat16) == (torch.bfloat16,) * 3


@pytest.mark.parametrize("env", [
    {"CONDITION_BLOCK_K_BAR_DTYPE": "float16"},
    {"CONDITION_BLOCK_K_BAR_DTYPE": "bfloat16"},                                   # needs mixed
    {"CONDITION_BLOCK_MIXED_SUMMARIES": "1", "CONDITION_BLOCK_SUMMARY_DTYPE": "bfloat16"},
])
def test_rejected_combinations(monkeypatch, env):
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    with pytest.raises(ValueError):
        _summary_storage_dtypes(torch.bfloat16)


def test_keywords_override_environment(monkeypatch):
    monkeypatch.setenv("CONDITION_BLOCK_MIXED_SUMMARIES", "1")
    assert _summary_storage_dtypes(torch.bfloat16, mixed=False) == (torch.float32,) * 3
