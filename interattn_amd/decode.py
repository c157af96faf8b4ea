"""Decode-loop integration: the reference's HF attention hook, its runner and its
generation loops (eager, and one graph replay per token) over the HIP kernels.

Mirrors, with the same names, arguments, environment switches and ``ValueError``
contract, ``llama/script/analysis/condition_block_gen/methods/condition_block_triton_impl/core.py``
(``CBT/core.py``): ``generate_condition_block_cached`` (:60-186),
``_generate_condition_block_cuda_graph`` (:189-314), ``_static_cache_from_prefill``
(:317-328), ``ConditionBlockDecodeRunner`` (:1203-1355), the attention contexts
(:1358-1400), ``_sdpa_prefill_attention_forward`` (:1180-1200) and the lazy step
statistics (:1403-1530, ``CBG/methods/patching.py:69-95``).  Single-token decode of
every compressed layer runs the fused condition path of
``interattn_amd.condition_block``; uncompressed layers run the HIP dense decode;
prompt prefill stays on torch SDPA exactly as in the reference.  On ROCm
``torch.cuda.CUDAGraph`` records a HIP graph.
"""

import contextlib
import os
from types import SimpleNamespace

import torch
import torch.nn.functional as F

from .condition_block import _build_prompt_blocks, _condition_block_decode_output, _sdpa_full_attention_forward

__all__ = [
    "ConditionBlockDecodeRunner",
    "PagedTopkDecodeRunner",
    "condition_block_decode_context",
    "full_attention_sdpa_context",
    "model_attention_implementation",
    "generate_condition_block_cached",
    "full_attention_stats_for_heads",
    "summarize_condition_block_step_metadata",
]


def _modeling_llama():
    from transformers.models.llama import modeling_llama

    return modeling_llama


# ------------------------------------------------------------------ step statistics

def merge_stats(total, add):
    """``CBG/methods/patching.py:69-71``."""
    for key, value in add.items():
        total[key] = int(total.get(key, 0)) + int(value)


def summarize_stats(aggregate_stats, stats_by_layer):
    """``CBG/methods/patching.py:74-95``."""
    total_available = max(int(aggregate_stats.get("total_available", 0)), 1)
    rows = max(int(aggregate_stats.get("rows", 0)), 1)
    hybrid_tokens = int(aggregate_stats.get("hybrid_tokens", 0))
    aggregate = {
        **aggregate_stats,
        "mean_hybrid_tokens": float(hybrid_tokens / rows),
        "mean_budget_causal": float(hybrid_tokens / total_available),
        "mean_budget_visible": float(hybrid_tokens / total_available),
    }
    by_layer = {}
    for layer_idx, stats in stats_by_layer.items():
        layer_total = max(int(stats.get("total_available", 0)), 1)
        layer_rows = max(int(stats.get("rows", 0)), 1)
        layer_hybrid = int(stats.get("hybrid_tokens", 0))
        by_layer[layer_idx] = {
            **stats,
            "mean_hybrid_tokens": float(layer_hybrid / layer_rows),
            "mean_budget_causal": float(layer_hybrid / layer_total),
            "mean_budget_visible": float(layer_hybrid / layer_total),
        }
    return {"aggregate": aggregate, "by_layer": by_layer}


def full_attention_stats_for_heads(n_heads, pos_list):
    """Routing statistics of a dense layer (CBT/core.py:1463-1472)."""
    total_available = sum(int(pos) + 1 for pos in pos_list) * int(n_heads)
    return {
        "rows": int(n_heads) * len(pos_list),
        "clusters": 0,
        "selected_clusters": 0,
        "selected_tokens": total_available,
        "hybrid_tokens": total_available,
        "total_available": total_available,
    }


def _merge_stats_lazy(total, add):
    for key, value in add.items():
        total[key] = total[key] + value if key in total else value


def _to_python_number(value):
    if torch.is_tensor(value):
        value = value.detach().cpu()
        if value.numel() != 1:
            raise ValueError("Expected scalar tensor in condition-block stats.")
        return int(value.item())
    return int(value)


def _stats_ratio(numerator, denominator):
    return float(_to_python_number(numerator) / max(_to_python_number(denominator), 1))


def _materialize_stats(stats):
    return {key: _to_python_number(value) for key, value in stats.items()}


def _summarize_stats_lazy(aggregate_stats, stats_by_layer):
    """Synchronisation-free per-step summary (CBT/core.py:1439-1447)."""
    return {"aggregate": dict(aggregate_stats),
            "by_layer": {int(i): dict(s) for i, s in stats_by_layer.items()}}


def _full_generation_step_metadata(model, pos_list):
    aggregate, by_layer = {}, {}
    n_heads = int(model.config.num_attention_heads)
    for layer_idx in range(int(model.config.num_hidden_layers)):
        stats = full_attention_stats_for_heads(n_heads, pos_list)
        by_layer[layer_idx] = stats
        merge_stats(aggregate, stats)
    return summarize_stats(aggregate, by_layer)


def summarize_condition_block_step_metadata(step_metadata):
    """Materialise the per-step statistics after generation (CBT/core.py:1486-1530)."""
    if os.environ.get("CONDITION_BLOCK_SKIP_STATS") == "1":
        return {"condition_block_stats_disabled": True}
    aggregate = {}
    by_step = []
    for step_idx, metadata in enumerate(step_metadata):
        if not metadata:
            continue
        step_aggregate = metadata.get("aggregate", {})
        by_step.append({"step": step_idx,
                        "equiv_budget": _stats_ratio(step_aggregate.get("hybrid_tokens", 0),
                                                     step_aggregate.get("total_available", 0))})
        for key, value in step_aggregate.items():
            if not key.startswith("mean_"):
                _merge_stats_lazy(aggregate, {key: value})
    materialized = _materialize_stats(aggregate)
    total_available = max(int(materialized.get("total_available", 0)), 1)
    rows = max(int(materialized.get("rows", 0)), 1)
    hybrid_tokens = int(materialized.get("hybrid_tokens", 0))
    equiv_budget = float(hybrid_tokens / total_available)
    return {
        "condition_block_equiv_budget": equiv_budget,
        "condition_block_budget": {**materialized, "mean_hybrid_tokens": float(hybrid_tokens / rows),
                                   "mean_budget_causal": equiv_budget, "mean_budget_visible": equiv_budget,
                                   "by_step": by_step},
    }


# ------------------------------------------------------------------ attention functions

def _sdpa_prefill_attention_forward(module, query, key, value, attention_mask, scaling, dropout=0.0, **_kwargs):
    """Causal prompt prefill on torch SDPA (CBT/core.py:1180-1200)."""
    attn_output = F.scaled_dot_product_attention(
        query, key, value, attn_mask=None, dropout_p=float(dropout) if module.training else 0.0, is_causal=True,
        scale=scaling, enable_gqa=query.shape[1] != key.shape[1])
    return attn_output.transpose(1, 2).contiguous(), None


class ConditionBlockDecodeRunner:
    """The HF attention hook of the condition-block decode (CBT/core.py:1203-1355):
    builds each layer's prompt summaries on its first decode step, then routes every
    single-token decode of a compressed layer through the fused HIP path."""

    def __init__(self, *, model, model_config, layer_idx_list, full_attention_layers, block_size, eps, prompt_len,
                 pos, prompt_prefix_cache, term1_mass_exp=False):
        self.model_config = model_config
        self.module_to_layer_idx = {id(layer.self_attn): int(i) for i, layer in enumerate(model.model.layers)}
        self.layer_idx_set = {int(i) for i in layer_idx_list}
        self.full_attention_layers = int(full_attention_layers)
        self.block_size = int(block_size)
        self.eps = float(eps)
        self.prompt_len = int(prompt_len)
        self.pos = int(pos)
        self.prompt_prefix_cache = prompt_prefix_cache
        self.term1_mass_exp = bool(term1_mass_exp)
        self.workspace_by_layer = {}
        self.stats_by_layer = {}
        self.aggregate_stats = {}
        self.skip_stats = os.environ.get("CONDITION_BLOCK_SKIP_STATS") == "1"
        # suffix length read by the fused decode on the device: refreshed by
        # reset_step() in the eager loop, advanced inside the graph otherwise
        self.suffix_len_dev = torch.zeros((), dtype=torch.int32, device=next(model.parameters()).device)
        # full static-cache views + suffix_len_dev keep every shape step-invariant
        self.static_suffix = False

    def should_compress(self, layer_idx):
        return int(layer_idx) in self.layer_idx_set and int(layer_idx) >= self.full_attention_layers

    def summarize(self):
        return _summarize_stats_lazy(self.aggregate_stats, self.stats_by_layer)

    def reset_step(self, pos):
        self.pos = int(pos)
        self.suffix_len_dev.fill_(max(self.pos + 1 - self.prompt_len, 0))
        self.stats_by_layer.clear()
        self.aggregate_stats.clear()

    def hybrid_attention_forward(self, module, query, key, value, attention_mask, scaling, dropout=0.0, **kwargs):
        layer_idx = getattr(module, "layer_idx", None)
        if layer_idx is None:
            layer_idx = self.module_to_layer_idx.get(id(module))
        if query.shape[2] != 1:
            return _sdpa_prefill_attention_forward(module, query, key, value, attention_mask, scaling=scaling,
                                                   dropout=dropout, **kwargs)
        if layer_idx is None or not self.should_compress(layer_idx):
            if layer_idx in self.layer_idx_set and not self.skip_stats:
                stats = full_attention_stats_for_heads(query.shape[1], [self.pos])
                self.stats_by_layer[int(layer_idx)] = stats
                _merge_stats_lazy(self.aggregate_stats, stats)
            return _sdpa_full_attention_forward(module, query, key, value, attention_mask, scaling=scaling,
                                                dropout=dropout, **kwargs)
        if query.shape[0] != 1 or query.shape[2] != 1:
            raise ValueError("condition_block fast path expects batch_size=1 and q_len=1.")
        if self.pos < self.prompt_len:
            raise ValueError("condition_block fast path expects generated-token decode positions.")
        _batch, n_heads, q_len, head_dim = query.shape
        n_kv_heads = int(key.shape[1])
        if n_heads % n_kv_heads != 0:
            raise ValueError("condition_block fast path expects grouped query attention.")
        q_grouped = query[0].reshape(n_kv_heads, n_heads // n_kv_heads, q_len, head_dim)
        if self.static_suffix:
            k_all, v_all = key[0], value[0]
        else:
            k_all = key[0, :, :self.pos + 1]
            v_all = value[0, :, :self.pos + 1]
        cache_key = (int(layer_idx), self.prompt_len, self.block_size)
        prompt_prefix = self.prompt_prefix_cache.get(cache_key)
        if prompt_prefix is None:
            prompt_prefix = _build_prompt_blocks(k_all[:, :self.prompt_len], v_all[:, :self.prompt_len],
                                                 self.block_size)
            self.prompt_prefix_cache[cache_key] = prompt_prefix
        output, stats = _condition_block_decode_output(
            q_grouped=q_grouped, prompt_prefix=prompt_prefix, k_suffix=k_all[:, self.prompt_len:],
            v_suffix=v_all[:, self.prompt_len:], suffix_len_dev=self.suffix_len_dev, block_size=self.block_size,
            eps=self.eps, prompt_len=self.prompt_len, attention_dtype=query.dtype,
            workspace=self.workspace_by_layer.setdefault(int(layer_idx), {}), term1_mass_exp=self.term1_mass_exp,
            collect_stats=not self.skip_stats)
        output = output.reshape(n_heads, q_len, head_dim).permute(1, 0, 2).unsqueeze(0)
        if stats is not None:
            self.stats_by_layer[int(layer_idx)] = stats
            _merge_stats_lazy(self.aggregate_stats, stats)
        return output.to(query.dtype), None


class PagedTopkDecodeRunner:
    """HF attention hook serving decode from a paged KV pool with the top-k rule (the
    outer hook of ``ConditionBlockDecodeRunner``, CBT/core.py:1203-1355, with the
    paged pool as its KV store; no reference counterpart).

    Each layer owns a pool ``[n_pages, Hkv, page_size, D]`` in the model's dtype;
    all layers share one block table ``[batch, ceil(max_seq_len / page_size)]`` (a
    seeded permutation of the pages).  Prompt prefill runs torch SDPA and copies the
    prompt's K/V into the pool, then builds the block summaries.  Every single-token
    decode appends the new K/V row on the device (``append_kv``), refreshes the
    summaries the new token touched (``update_block_summaries``) and runs the fused
    top-k layer call (``sparse_topk_decode``); layers below ``full_attention_layers``
    run the HIP paged dense decode.  Prompts of one batch share a length (no
    padding).  Install with ``condition_block_decode_context(runner)``."""

    def __init__(self, *, model, batch_size, max_seq_len, block_size, k, forced_first=0, forced_last=0,
                 page_size=16, full_attention_layers=0, k_bar_dtype=None, seed=0):
        from . import ops

        self._ops = ops
        cfg = model.config
        param = next(model.parameters())
        self.device, self.dtype = param.device, param.dtype
        if self.dtype not in (torch.bfloat16, torch.float32):
            raise ValueError("the paged runner serves bf16 or fp32 models")
        self.n_layers = int(cfg.num_hidden_layers)
        self.n_kv_heads = int(cfg.num_key_value_heads)
        self.head_dim = int(getattr(cfg, "head_dim", None) or cfg.hidden_size // cfg.num_attention_heads)
        self.batch_size, self.max_seq_len = int(batch_size), int(max_seq_len)
        self.block_size, self.k = int(block_size), int(k)
        self.forced_first, self.forced_last = int(forced_first), int(forced_last)
        self.page_size = int(page_size)
        self.full_attention_layers = int(full_attention_layers)
        self.k_bar_dtype = k_bar_dtype or self.dtype
        if self.block_size % 16 or self.page_size % 16:
            raise ValueError("block_size and page_size must be multiples of 16")
        self.nb_max = -(-self.max_seq_len // self.block_size)
        pages_per_seq = -(-self.max_seq_len // self.page_size)
        gen = torch.Generator(device="cpu").manual_seed(int(seed))
        perm = torch.randperm(self.batch_size * pages_per_seq, generator=gen).to(torch.int32)
        self.block_table = perm.view(self.batch_size, pages_per_seq).to(self.device)
        shape = (self.batch_size * pages_per_seq, self.n_kv_heads, self.page_size, self.head_dim)
        self.pools = [(torch.zeros(shape, device=self.device, dtype=self.dtype),
                       torch.zeros(shape, device=self.device, dtype=self.dtype)) for _ in range(self.n_layers)]
        # each layer advances its own lengths (append_kv moves them on the device)
        self.seq_lens = [torch.zeros(self.batch_size, device=self.device, dtype=torch.int32)
                         for _ in range(self.n_layers)]
        self.old_seq_lens = [torch.zeros_like(t) for t in self.seq_lens]
        self.summaries = [None] * self.n_layers
        self.workspace_by_layer = [{} for _ in range(self.n_layers)]
        self.module_to_layer_idx = {id(layer.self_attn): int(i) for i, layer in enumerate(model.model.layers)}

    def _layer(self, module):
        idx = getattr(module, "layer_idx", None)
        return int(self.module_to_layer_idx[id(module)] if idx is None else idx)

    def _fill(self, layer, key, value):
        """Copy the prompt's K/V [B, Hkv, T, D] into the layer's pool, build summaries."""
        b, hkv, t, d = key.shape
        if b != self.batch_size or hkv != self.n_kv_heads or d != self.head_dim:
            raise ValueError("prompt K/V do not match the runner's batch / heads / head_dim")
        if t > self.max_seq_len:
            raise ValueError("prompt longer than max_seq_len")
        pk, pv = self.pools[layer]
        n_pg = -(-t // self.page_size)
        pages = self.block_table[:, :n_pg].reshape(-1).long()
        for src, pool in ((key, pk), (value, pv)):
            x = F.pad(src, (0, 0, 0, n_pg * self.page_size - t))
            x = x.view(b, hkv, n_pg, self.page_size, d).permute(0, 2, 1, 3, 4)
            pool[pages] = x.reshape(b * n_pg, hkv, self.page_size, d).to(pool.dtype)
        self.seq_lens[layer].fill_(t)
        if layer >= self.full_attention_layers:
            self.summaries[layer] = self._ops.build_block_summaries(
                pk, pv, self.block_table, self.seq_lens[layer], self.block_size, nb_max=self.nb_max,
                k_bar_dtype=self.k_bar_dtype)

    def hybrid_attention_forward(self, module, query, key, value, attention_mask, scaling, dropout=0.0, **kwargs):
        layer = self._layer(module)
        if query.shape[2] != 1:
            self._fill(layer, key, value)
            return _sdpa_prefill_attention_forward(module, query, key, value, attention_mask, scaling=scaling,
                                                   dropout=dropout, **kwargs)
        if self.summaries[layer] is None and layer >= self.full_attention_layers:
            raise ValueError("paged runner: decode before the prompt was prefilled")
        ops = self._ops
        pk, pv = self.pools[layer]
        seq, old = self.seq_lens[layer], self.old_seq_lens[layer]
        old.copy_(seq)
        ops.append_kv(pk, pv, self.block_table, seq, key[:, :, -1].to(pk.dtype), value[:, :, -1].to(pv.dtype))
        q = query[:, :, 0].contiguous()
        ws = self.workspace_by_layer[layer]
        if layer < self.full_attention_layers:
            out = ops.paged_decode(q, pk, pv, self.block_table, seq, max_seq_len=self.max_seq_len, scale=scaling,
                                   out_dtype=query.dtype, workspace=ws)
        else:
            summ = self.summaries[layer]
            ops.update_block_summaries(summ, pk, pv, self.block_table, old, seq, self.block_size, max_new_tokens=1)
            out = ops.sparse_topk_decode(q, pk, pv, self.block_table, seq, summ["k_bar"], self.k,
                                         block_size=self.block_size, forced_first=self.forced_first,
                                         forced_last=self.forced_last, scale=scaling, out_dtype=query.dtype,
                                         workspace=ws)
        return out.unsqueeze(1), None


# ------------------------------------------------------------------ contexts

@contextlib.contextmanager
def _no_causal_mask_context():
    """Skip HF causal-mask construction in the graphed step (CBT/core.py:1358-1370)."""
    ml = _modeling_llama()
    original = ml.create_causal_mask
    ml.create_causal_mask = lambda *args, **kwargs: None
    try:
        yield
    finally:
        ml.create_causal_mask = original


@contextlib.contextmanager
def condition_block_decode_context(runner):
    """Install ``runner.hybrid_attention_forward`` as HF's eager attention (CBT/core.py:1373-1380)."""
    ml = _modeling_llama()
    original = ml.eager_attention_forward
    ml.eager_attention_forward = runner.hybrid_attention_forward
    try:
        yield runner
    finally:
        ml.eager_attention_forward = original


@contextlib.contextmanager
def full_attention_sdpa_context():
    """Every decode on the HIP dense path (CBT/core.py:1383-1390)."""
    ml = _modeling_llama()
    original = ml.eager_attention_forward
    ml.eager_attention_forward = _sdpa_full_attention_forward
    try:
        yield
    finally:
        ml.eager_attention_forward = original


@contextlib.contextmanager
def model_attention_implementation(model, implementation):
    original = model.config._attn_implementation
    model.config._attn_implementation = implementation
    try:
        yield
    finally:
        model.config._attn_implementation = original


# ------------------------------------------------------------------ generation loops

def run_prefill_only_condition_block(**_kwargs):
    raise RuntimeError("condition_block now uses the cached generate path only. "
                       "Call generate_condition_block_cached through generate_with_method().")


def build_condition_args(method, prompt_len):
    return SimpleNamespace(seq_len=int(prompt_len), block_size=method.condition_block_size,
                           full_attention_layers=int(method.full_attention_layers),
                           delta_mode=method.condition_delta_mode)


def _stop_token_ids(tokenizer, dataset):
    ids = []
    if tokenizer is not None and tokenizer.eos_token_id is not None:
        ids.append(int(tokenizer.eos_token_id))
    if tokenizer is not None and dataset == "samsum":
        newline_ids = tokenizer.encode("\n", add_special_tokens=False)
        if newline_ids:
            ids.append(int(newline_ids[-1]))
    return ids


def _should_stop(next_id, stop_ids_tensor):
    if stop_ids_tensor is None:
        return False
    return bool(torch.isin(next_id, stop_ids_tensor).all().item())


def _static_cache_from_prefill(config, prefill_cache, max_cache_len):
    """Move the prefill KV into a StaticCache of ``max_cache_len`` (CBT/core.py:317-328)."""
    from transformers import StaticCache

    static_cache = StaticCache(config=config, max_cache_len=int(max_cache_len))
    for layer_idx, source_layer in enumerate(prefill_cache.layers):
        key_states, value_states = source_layer.keys, source_layer.values
        target = static_cache.layers[layer_idx]
        target.lazy_initialization(key_states[:, :, :1], value_states[:, :, :1])
        seq_len = int(key_states.shape[2])
        target.keys[:, :, :seq_len].copy_(key_states)
        target.values[:, :, :seq_len].copy_(value_states)
    return static_cache


def generate_condition_block_cached(*, model, tokenizer, input_ids, attention_mask, method, device, dataset=None,
                                    term1_mass_exp=False):
    """Greedy generation with SDPA prefill and condition-block decode (CBT/core.py:60-186).
    ``method`` carries ``condition_delta_mode, condition_block_size, condition_eps,
    full_attention_layers, max_new_tokens``.  Returns ``(output_ids [1, n], metadata)``."""
    if method.condition_delta_mode != "range_bound":
        raise ValueError("condition_block only supports delta_mode='range_bound'.")
    if int(input_ids.shape[0]) != 1:
        raise ValueError("condition_block generate currently expects batch_size=1.")
    if os.environ.get("CONDITION_BLOCK_CUDA_GRAPH") == "1":
        return _generate_condition_block_cuda_graph(model=model, tokenizer=tokenizer, input_ids=input_ids,
                                                    attention_mask=attention_mask, method=method, dataset=dataset,
                                                    term1_mass_exp=term1_mass_exp)
    from transformers import StaticCache

    prompt_len = int(input_ids.shape[1])
    max_new_tokens = int(method.max_new_tokens)
    if max_new_tokens <= 0:
        return (torch.empty((1, 0), device=input_ids.device, dtype=input_ids.dtype),
                summarize_condition_block_step_metadata([]))
    stop_token_ids = _stop_token_ids(tokenizer, dataset)
    stop_ids_tensor = (torch.tensor(stop_token_ids, device=input_ids.device, dtype=input_ids.dtype)
                       if stop_token_ids else None)
    layer_idx_list = list(range(int(model.config.num_hidden_layers)))
    prompt_prefix_cache = {}
    generated, step_metadata = [], []
    collect_stats = os.environ.get("CONDITION_BLOCK_SKIP_STATS") != "1"
    cur_mask = attention_mask
    total_len = prompt_len
    past_key_values = None
    if os.environ.get("CONDITION_BLOCK_STATIC_CACHE") == "1":
        past_key_values = StaticCache(config=model.config, max_cache_len=prompt_len + max_new_tokens)
    with model_attention_implementation(model, "sdpa"), torch.no_grad():
        outputs = model(input_ids=input_ids, attention_mask=cur_mask, past_key_values=past_key_values,
                        use_cache=True, logits_to_keep=1)
    logits = outputs.logits.float()
    past_key_values = outputs.past_key_values
    if os.environ.get("CONDITION_BLOCK_POST_PREFILL_STATIC_CACHE") == "1":
        past_key_values = _static_cache_from_prefill(model.config, past_key_values,
                                                     max_cache_len=prompt_len + max_new_tokens)
    if collect_stats:
        step_metadata.append(_full_generation_step_metadata(model, [total_len - 1]))
    next_id = torch.argmax(logits[:, -1, :], dim=-1, keepdim=True)
    generated.append(next_id)
    if _should_stop(next_id, stop_ids_tensor):
        return torch.cat(generated, dim=1), summarize_condition_block_step_metadata(step_metadata)
    cur_mask = torch.cat([cur_mask, torch.ones_like(next_id)], dim=1)
    step_input_ids = next_id
    total_len += 1
    runner = ConditionBlockDecodeRunner(model=model, model_config=model.config, layer_idx_list=layer_idx_list,
                                        full_attention_layers=method.full_attention_layers,
                                        block_size=method.condition_block_size, eps=method.condition_eps,
                                        prompt_len=prompt_len, pos=total_len - 1,
                                        prompt_prefix_cache=prompt_prefix_cache, term1_mass_exp=term1_mass_exp)
    with condition_block_decode_context(runner):
        for _step in range(1, max_new_tokens):
            runner.reset_step(total_len - 1)
            with torch.no_grad():
                cache_position = None
                if os.environ.get("CONDITION_BLOCK_POST_PREFILL_STATIC_CACHE") == "1":
                    cache_position = torch.tensor([total_len - 1], device=input_ids.device, dtype=torch.long)
                outputs = model(input_ids=step_input_ids, attention_mask=cur_mask, past_key_values=past_key_values,
                                use_cache=True, logits_to_keep=1, cache_position=cache_position)
            logits = outputs.logits.float()
            past_key_values = outputs.past_key_values
            if collect_stats:
                step_metadata.append(runner.summarize())
            next_id = torch.argmax(logits[:, -1, :], dim=-1, keepdim=True)
            generated.append(next_id)
            if _should_stop(next_id, stop_ids_tensor):
                break
            cur_mask = torch.cat([cur_mask, torch.ones_like(next_id)], dim=1)
            step_input_ids = next_id
            total_len += 1
    return torch.cat(generated, dim=1), summarize_condition_block_step_metadata(step_metadata)


def _generate_condition_block_cuda_graph(*, model, tokenizer, input_ids, attention_mask, method, dataset=None,
                                         term1_mass_exp=False):
    """One graph replay per generated token (CBT/core.py:189-314): SDPA prefill, the
    prompt KV moved into a StaticCache, three eager warm-up steps (summaries and
    workspaces), then the whole decode step (forward, argmax, state advance) captured
    once and replayed.  Requires CONDITION_BLOCK_SKIP_STATS=1 and
    full_attention_layers=0; stop tokens are applied by truncation afterwards."""
    if os.environ.get("CONDITION_BLOCK_SKIP_STATS") != "1":
        raise ValueError("CONDITION_BLOCK_CUDA_GRAPH=1 requires CONDITION_BLOCK_SKIP_STATS=1.")
    if int(method.full_attention_layers) != 0:
        raise ValueError("CUDA-graph decode supports full_attention_layers=0 only.")
    if int(method.condition_block_size) <= 0 or int(method.condition_block_size) % 16:
        raise ValueError("CUDA-graph decode requires a block size that is a positive multiple of 16.")
    prompt_len = int(input_ids.shape[1])
    max_new_tokens = int(method.max_new_tokens)
    if max_new_tokens <= 0:
        return (torch.empty((1, 0), device=input_ids.device, dtype=input_ids.dtype),
                summarize_condition_block_step_metadata([]))
    with model_attention_implementation(model, "sdpa"), torch.no_grad():
        outputs = model(input_ids=input_ids, attention_mask=attention_mask, use_cache=True, logits_to_keep=1)
    past_key_values = _static_cache_from_prefill(model.config, outputs.past_key_values,
                                                 max_cache_len=prompt_len + max_new_tokens)
    dev = input_ids.device
    out_tokens = torch.zeros(max_new_tokens, dtype=input_ids.dtype, device=dev)
    next_id = torch.argmax(outputs.logits.float()[:, -1, :], dim=-1)
    out_tokens[0] = next_id[0]
    del outputs
    input_ids_buf = next_id.view(1, 1).clone()
    cache_pos_buf = torch.tensor([prompt_len], device=dev, dtype=torch.long)
    step_idx_buf = torch.ones(1, device=dev, dtype=torch.long)
    runner = ConditionBlockDecodeRunner(model=model, model_config=model.config,
                                        layer_idx_list=list(range(int(model.config.num_hidden_layers))),
                                        full_attention_layers=method.full_attention_layers,
                                        block_size=method.condition_block_size, eps=method.condition_eps,
                                        prompt_len=prompt_len, pos=prompt_len, prompt_prefix_cache={},
                                        term1_mass_exp=term1_mass_exp)
    runner.static_suffix = True
    runner.suffix_len_dev.fill_(1)

    def _decode_step():
        step_outputs = model(input_ids=input_ids_buf, attention_mask=None, past_key_values=past_key_values,
                             use_cache=True, logits_to_keep=1, cache_position=cache_pos_buf)
        step_next = torch.argmax(step_outputs.logits.float()[0, -1], dim=-1)
        out_tokens.index_copy_(0, step_idx_buf, step_next.view(1))
        input_ids_buf.copy_(step_next.view(1, 1))
        cache_pos_buf.add_(1)
        step_idx_buf.add_(1)
        runner.suffix_len_dev.add_(1)

    warmup_steps = min(3, max_new_tokens - 1)
    with condition_block_decode_context(runner), _no_causal_mask_context(), torch.no_grad():
        side_stream = torch.cuda.Stream()
        side_stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side_stream):
            for _ in range(warmup_steps):
                _decode_step()
        torch.cuda.current_stream().wait_stream(side_stream)
        remaining = max_new_tokens - 1 - warmup_steps
        if remaining > 0:
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                _decode_step()
            for _ in range(remaining):
                graph.replay()
    torch.cuda.synchronize()
    tokens = out_tokens.tolist()
    stop_token_ids = set(_stop_token_ids(tokenizer, dataset))
    n_keep = len(tokens)
    for idx, token in enumerate(tokens):
        if token in stop_token_ids:
            n_keep = idx + 1
            break
    output_ids = out_tokens[:n_keep].view(1, -1).to(dtype=input_ids.dtype)
    return output_ids, {"condition_block_stats_disabled": True, "cuda_graph_decode": True}
