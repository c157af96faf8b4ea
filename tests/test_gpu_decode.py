"""End-to-end decode through the reference's HF hook on a small random-weight Llama
(no checkpoint is available offline): the condition-block runner, the cached
generation loop and the graph-replayed loop of ``interattn_amd.decode``.

With eps = 0 every block with a positive condition is selected, so the hybrid
attention equals exact attention: per-step logits must match the dense model's
(float32, 1e-3 abs) and greedy tokens must be identical.  The graph loop must emit
the eager loop's tokens.  With eps = 1e9 no block is selected (representatives +
suffix only): the logits stay finite and the routing statistics count zero
selected blocks.
"""

import os
from types import SimpleNamespace

import pytest
import torch

from tests._util import announce

pytestmark = pytest.mark.gpu

transformers = pytest.importorskip("transformers")


def _model(device, dtype=torch.float32, layers=2, head_dim=64):
    from transformers import LlamaConfig, LlamaForCausalLM

    torch.manual_seed(0)
    cfg = LlamaConfig(vocab_size=256, hidden_size=8 * head_dim, intermediate_size=1024, num_hidden_layers=layers,
                      num_attention_heads=8, num_key_value_heads=2, max_position_embeddings=2048,
                      attn_implementation="eager")
    return LlamaForCausalLM(cfg).to(device=device, dtype=dtype).eval()


def _method(eps, n_new, block=32, full_layers=0):
    return SimpleNamespace(condition_delta_mode="range_bound", condition_block_size=block, condition_eps=eps,
                           full_attention_layers=full_layers, max_new_tokens=n_new)


def _dense_greedy(model, ids, n_new):
    """Reference: the same model with torch SDPA attention, greedy, DynamicCache."""
    from interattn_amd.decode import model_attention_implementation

    toks, logits_all = [], []
    with model_attention_implementation(model, "sdpa"), torch.no_grad():
        out = model(input_ids=ids, use_cache=True, logits_to_keep=1)
        pkv = out.past_key_values
        nxt = out.logits[:, -1].float().argmax(-1, keepdim=True)
        toks.append(nxt)
        logits_all.append(out.logits[:, -1].float())
        for _ in range(n_new - 1):
            out = model(input_ids=nxt, past_key_values=pkv, use_cache=True, logits_to_keep=1)
            pkv = out.past_key_values
            logits_all.append(out.logits[:, -1].float())
            nxt = out.logits[:, -1].float().argmax(-1, keepdim=True)
            toks.append(nxt)
    return torch.cat(toks, 1), logits_all


def _runner_logits(model, ids, n_new, eps, block, full_layers, forced_tokens):
    """Drive the runner step by step feeding ``forced_tokens`` (teacher forcing), so
    the logits of every step can be compared with the dense model's."""
    from interattn_amd.decode import ConditionBlockDecodeRunner, condition_block_decode_context, \
        model_attention_implementation

    p = int(ids.shape[1])
    with model_attention_implementation(model, "sdpa"), torch.no_grad():
        out = model(input_ids=ids, use_cache=True, logits_to_keep=1)
    pkv = out.past_key_values
    logits_all = [out.logits[:, -1].float()]
    runner = ConditionBlockDecodeRunner(model=model, model_config=model.config,
                                        layer_idx_list=list(range(model.config.num_hidden_layers)),
                                        full_attention_layers=full_layers, block_size=block, eps=eps,
                                        prompt_len=p, pos=p, prompt_prefix_cache={})
    stats = []
    with condition_block_decode_context(runner), torch.no_grad():
        for step in range(1, n_new):
            runner.reset_step(p + step - 1)
            out = model(input_ids=forced_tokens[:, step - 1:step], past_key_values=pkv, use_cache=True,
                        logits_to_keep=1)
            pkv = out.past_key_values
            logits_all.append(out.logits[:, -1].float())
            stats.append(runner.summarize())
    return logits_all, stats


@pytest.mark.parametrize("full_layers", [0, 1])
def test_runner_eps0_equals_dense(device, full_layers):
    announce(f"decode runner eps=0 full_layers={full_layers}")
    model = _model(device)
    g = torch.Generator().manual_seed(1)
    ids = torch.randint(0, 256, (1, 203), generator=g).to(device)
    n_new = 6
    ref_tok, ref_logits = _dense_greedy(model, ids, n_new)
    got_logits, stats = _runner_logits(model, ids, n_new, 0.0, 32, full_layers, ref_tok)
    for i, (a, b) in enumerate(zip(got_logits, ref_logits)):
        err = (a - b).abs().max().item()
        assert err < 1e-3, f"step {i}: max |logit diff| {err}"
    # every existing prompt block of the compressed layers is selected
    agg = stats[-1]["aggregate"]
    assert int(agg["selected_clusters"]) == int(agg["clusters"])


def test_generate_cached_matches_dense_tokens(device, monkeypatch):
    from interattn_amd.decode import generate_condition_block_cached

    announce("generate_condition_block_cached eps=0")
    monkeypatch.delenv("CONDITION_BLOCK_CUDA_GRAPH", raising=False)
    monkeypatch.delenv("CONDITION_BLOCK_SKIP_STATS", raising=False)
    model = _model(device)
    ids = torch.randint(0, 256, (1, 150), generator=torch.Generator().manual_seed(2)).to(device)
    mask = torch.ones_like(ids)
    ref_tok, _ = _dense_greedy(model, ids, 8)
    out, meta = generate_condition_block_cached(model=model, tokenizer=None, input_ids=ids, attention_mask=mask,
                                                method=_method(0.0, 8), device=device)
    assert torch.equal(out, ref_tok)
    assert meta["condition_block_equiv_budget"] > 0.99


def test_graph_loop_matches_eager_loop(device, monkeypatch):
    from interattn_amd.decode import generate_condition_block_cached

    announce("graph decode loop vs eager loop, eps=0.05")
    model = _model(device)
    ids = torch.randint(0, 256, (1, 260), generator=torch.Generator().manual_seed(3)).to(device)
    mask = torch.ones_like(ids)
    monkeypatch.setenv("CONDITION_BLOCK_SKIP_STATS", "1")
    monkeypatch.setenv("CONDITION_BLOCK_POST_PREFILL_STATIC_CACHE", "1")
    monkeypatch.delenv("CONDITION_BLOCK_CUDA_GRAPH", raising=False)
    eager, meta_e = generate_condition_block_cached(model=model, tokenizer=None, input_ids=ids, attention_mask=mask,
                                                    method=_method(0.05, 10), device=device)
    monkeypatch.delenv("CONDITION_BLOCK_POST_PREFILL_STATIC_CACHE", raising=False)
    monkeypatch.setenv("CONDITION_BLOCK_CUDA_GRAPH", "1")
    graphed, meta_g = generate_condition_block_cached(model=model, tokenizer=None, input_ids=ids,
                                                      attention_mask=mask, method=_method(0.05, 10), device=device)
    assert meta_g.get("cuda_graph_decode") is True
    assert torch.equal(eager, graphed), (eager, graphed)


@pytest.mark.parametrize("graph", [False, True])
def test_static_cache_loops_match_dense_tokens(device, monkeypatch, graph):
    """eps = 0 (every block selected: exact attention) through the static-cache loops:
    the prompt K/V moved into a StaticCache and the decode steps written after it, so
    the greedy tokens equal the dense model's."""
    from interattn_amd.decode import generate_condition_block_cached

    announce(f"static-cache decode loop, graph={graph}, eps=0 vs dense")
    model = _model(device)
    ids = torch.randint(0, 256, (1, 190), generator=torch.Generator().manual_seed(5)).to(device)
    ref_tok, _ = _dense_greedy(model, ids, 9)
    monkeypatch.setenv("CONDITION_BLOCK_SKIP_STATS", "1")
    if graph:
        monkeypatch.setenv("CONDITION_BLOCK_CUDA_GRAPH", "1")
        monkeypatch.delenv("CONDITION_BLOCK_POST_PREFILL_STATIC_CACHE", raising=False)
    else:
        monkeypatch.delenv("CONDITION_BLOCK_CUDA_GRAPH", raising=False)
        monkeypatch.setenv("CONDITION_BLOCK_POST_PREFILL_STATIC_CACHE", "1")
    out, _ = generate_condition_block_cached(model=model, tokenizer=None, input_ids=ids,
                                             attention_mask=torch.ones_like(ids), method=_method(0.0, 9),
                                             device=device)
    assert torch.equal(out, ref_tok), (out, ref_tok)


def test_runner_no_blocks_selected(device):
    announce("decode runner eps=1e9")
    model = _model(device, dtype=torch.bfloat16, head_dim=128)
    ids = torch.randint(0, 256, (1, 333), generator=torch.Generator().manual_seed(4)).to(device)
    ref_tok, ref_logits = _dense_greedy(model, ids, 4)
    got_logits, stats = _runner_logits(model, ids, 4, 1e9, 64, 0, ref_tok)
    assert all(torch.isfinite(x).all() for x in got_logits)
    agg = stats[-1]["aggregate"]
    assert int(agg["selected_clusters"]) == 0 and int(agg["clusters"]) > 0


def _dense_batch_greedy(model, ids, n_new):
    """Batched dense reference (equal-length prompts, no padding)."""
    from interattn_amd.decode import model_attention_implementation

    toks, logits_all = [], []
    with model_attention_implementation(model, "sdpa"), torch.no_grad():
        out = model(input_ids=ids, use_cache=True, logits_to_keep=1)
        pkv = out.past_key_values
        for _ in range(n_new):
            logits_all.append(out.logits[:, -1].float())
            nxt = out.logits[:, -1].float().argmax(-1, keepdim=True)
            toks.append(nxt)
            out = model(input_ids=nxt, past_key_values=pkv, use_cache=True, logits_to_keep=1)
            pkv = out.past_key_values
    return torch.cat(toks, 1), logits_all


def _paged_runner_logits(model, ids, forced_tokens, **runner_kw):
    """Teacher-forced decode through ``PagedTopkDecodeRunner`` (prefill included)."""
    from interattn_amd.decode import PagedTopkDecodeRunner, condition_block_decode_context

    runner = PagedTopkDecodeRunner(model=model, batch_size=int(ids.shape[0]), **runner_kw)
    logits_all = []
    with condition_block_decode_context(runner), torch.no_grad():
        out = model(input_ids=ids, use_cache=True, logits_to_keep=1)
        pkv = out.past_key_values
        for step in range(forced_tokens.shape[1]):
            logits_all.append(out.logits[:, -1].float())
            out = model(input_ids=forced_tokens[:, step:step + 1], past_key_values=pkv, use_cache=True,
                        logits_to_keep=1)
            pkv = out.past_key_values
    return logits_all, runner


@pytest.mark.parametrize("full_layers", [0, 1])
def test_paged_runner_all_blocks_equals_dense(device, full_layers):
    """Paged pool + top-k with k >= every block: exact attention, so the logits of a
    batch-2 teacher-forced decode equal the dense model's; the pool lengths advance
    by one per step."""
    announce(f"paged top-k runner, all blocks, full_layers={full_layers}")
    model = _model(device)
    ids = torch.randint(0, 256, (2, 150), generator=torch.Generator().manual_seed(6)).to(device)
    n_new = 6
    ref_tok, ref_logits = _dense_batch_greedy(model, ids, n_new)
    got, runner = _paged_runner_logits(model, ids, ref_tok, max_seq_len=256, block_size=32, k=8,
                                       full_attention_layers=full_layers)
    for i, (a, b) in enumerate(zip(got, ref_logits)):
        err = (a - b).abs().max().item()
        assert err < 1e-3, f"step {i}: max |logit diff| {err}"
    for seq in runner.seq_lens:
        assert seq.cpu().tolist() == [150 + n_new] * 2


def test_paged_runner_sparse_bf16(device):
    """bf16 model, top-4 + first + last block of 64 (sparse attention, no closed-form
    logits): the decode runs end to end with finite logits and every layer's pool
    length advanced by one per step."""
    announce("paged top-k runner, sparse, bf16")
    model = _model(device, dtype=torch.bfloat16, head_dim=128)
    ids = torch.randint(0, 256, (2, 333), generator=torch.Generator().manual_seed(7)).to(device)
    ref_tok, _ = _dense_batch_greedy(model, ids, 4)
    got, runner = _paged_runner_logits(model, ids, ref_tok, max_seq_len=512, block_size=64, k=4, forced_first=1,
                                       forced_last=1)
    assert all(torch.isfinite(x).all() for x in got)
    for seq in runner.seq_lens:
        assert seq.cpu().tolist() == [337, 337]
