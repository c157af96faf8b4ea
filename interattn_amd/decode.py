"""Decode-loop integration: the HF attention hook of the condition-block decode and
greedy generation over it (eager, and one graph replay per token).

The public names, their arguments, the environment switches
(``CONDITION_BLOCK_SKIP_STATS``, ``CONDITION_BLOCK_CUDA_GRAPH``,
``CONDITION_BLOCK_STATIC_CACHE``, ``CONDITION_BLOCK_POST_PREFILL_STATIC_CACHE``) and
the ``ValueError`` texts are the reference's interface
(``llama/script/analysis/condition_block_gen/methods/condition_block_triton_impl/core.py``,
``CBT/core.py`` below: the loops :60-330, the runner :1203-1355, the contexts
:1358-1400, the statistics helpers :1403-1530 and ``CBG/methods/patching.py:69-95``),
so the reference's decode driver can call this module in its place.

How it is built here:

* one ``_GreedyStep`` object owns the per-token device state (next input id,
  cache position, output slot, the runner's suffix length) and runs one decode
  step; the eager loop calls it token by token, the graph loop captures it once and
  replays it;
* the prompt K/V reach a ``StaticCache`` through the cache's own ``update`` (so its
  length counter is right for the decode steps that follow);
* routing statistics stay on the device during generation (the runner takes them
  from the fused call's selection output) and are read back in one transfer when
  generation ends;
* the four attention contexts share one attribute-swapping context manager.

Single-token decode of a compressed layer runs ``condition_block``'s fused HIP
path; other decode layers run the HIP dense decode; prompt prefill stays on torch
SDPA as in the reference.  On ROCm ``torch.cuda.CUDAGraph`` records a HIP graph.
"""

import contextlib
import os
from types import SimpleNamespace

import torch
import torch.nn.functional as F

from .condition_block import (_build_prompt_blocks, _condition_block_decode_output, _sdpa_full_attention_forward,
                              mask_is_prefix, mask_prefix_hint)

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

_SKIP_STATS = "CONDITION_BLOCK_SKIP_STATS"


def _env_on(name):
    return os.environ.get(name) == "1"


def _modeling_llama():
    from transformers.models.llama import modeling_llama

    return modeling_llama


# ------------------------------------------------------------------ routing statistics

def _with_means(stats):
    """``stats`` plus its derived ratios: hybrid tokens per query row, and per visible
    token (the causal and visible budgets coincide for a decode step)."""
    hybrid = float(int(stats.get("hybrid_tokens", 0)))
    budget = hybrid / max(int(stats.get("total_available", 0)), 1)
    return {**stats, "mean_hybrid_tokens": hybrid / max(int(stats.get("rows", 0)), 1),
            "mean_budget_causal": budget, "mean_budget_visible": budget}


def merge_stats(total, add):
    """Add ``add``'s counts into ``total`` as Python ints (CBG/methods/patching.py:69)."""
    total.update({key: int(total.get(key, 0)) + int(val) for key, val in add.items()})


def summarize_stats(aggregate_stats, stats_by_layer):
    """Aggregate and per-layer statistics with their ratios (CBG/methods/patching.py:74)."""
    return {"aggregate": _with_means(aggregate_stats),
            "by_layer": {layer: _with_means(s) for layer, s in stats_by_layer.items()}}


def full_attention_stats_for_heads(n_heads, pos_list):
    """Statistics of a dense layer (CBT/core.py:1463): every visible token is attended
    by every query head."""
    visible = int(n_heads) * sum(int(pos) + 1 for pos in pos_list)
    return dict(rows=int(n_heads) * len(pos_list), clusters=0, selected_clusters=0, selected_tokens=visible,
                hybrid_tokens=visible, total_available=visible)


def _merge_stats_lazy(total, add):
    """Add ``add`` into ``total`` without a host synchronisation (values may be device
    tensors)."""
    for key, val in add.items():
        total[key] = val if key not in total else total[key] + val


def _summarize_stats_lazy(aggregate_stats, stats_by_layer):
    """Per-step snapshot of the runner's statistics (kept lazy: no device read)."""
    return {"aggregate": dict(aggregate_stats), "by_layer": {int(k): dict(v) for k, v in stats_by_layer.items()}}


def _full_generation_step_metadata(model, pos_list):
    n_layers, n_heads = int(model.config.num_hidden_layers), int(model.config.num_attention_heads)
    by_layer = {i: full_attention_stats_for_heads(n_heads, pos_list) for i in range(n_layers)}
    aggregate = {}
    for s in by_layer.values():
        merge_stats(aggregate, s)
    return summarize_stats(aggregate, by_layer)


def _read_back(values):
    """Python ints of a list of ints / one-element device tensors, with one transfer."""
    tensors = [v for v in values if torch.is_tensor(v)]
    if any(t.numel() != 1 for t in tensors):
        raise ValueError("Expected scalar tensor in condition-block stats.")
    host = iter(torch.stack([t.detach().reshape(()).to(torch.int64) for t in tensors]).tolist()) if tensors else None
    return [int(next(host)) if torch.is_tensor(v) else int(v) for v in values]


def summarize_condition_block_step_metadata(step_metadata):
    """Budget summary of a generation (CBT/core.py:1486): per-step equivalent budget
    and the totals, read back from the device once."""
    if _env_on(_SKIP_STATS):
        return {"condition_block_stats_disabled": True}
    steps = [(i, m.get("aggregate", {})) for i, m in enumerate(step_metadata) if m]
    totals = {}
    for _, agg in steps:
        _merge_stats_lazy(totals, {k: v for k, v in agg.items() if not k.startswith("mean_")})
    # one transfer for every step's (hybrid, available) pair and every total
    flat = [agg.get(k, 0) for _, agg in steps for k in ("hybrid_tokens", "total_available")]
    keys = list(totals)
    host = _read_back(flat + [totals[k] for k in keys])
    pairs, tot = host[:len(flat)], dict(zip(keys, host[len(flat):]))
    by_step = [{"step": i, "equiv_budget": float(pairs[2 * n] / max(pairs[2 * n + 1], 1))}
               for n, (i, _) in enumerate(steps)]
    summary = _with_means(tot)
    return {"condition_block_equiv_budget": summary["mean_budget_causal"],
            "condition_block_budget": {**summary, "by_step": by_step}}


# ------------------------------------------------------------------ attention functions

def _sdpa_prefill_attention_forward(module, query, key, value, attention_mask, scaling, dropout=0.0, **_kwargs):
    """Causal prompt prefill on torch SDPA (CBT/core.py:1180): ``[B, Hq, L, D]`` in,
    ``([B, L, Hq, D], None)`` out; grouped-query heads are expanded by SDPA."""
    p_drop = float(dropout) if module.training else 0.0
    out = F.scaled_dot_product_attention(query, key, value, dropout_p=p_drop, is_causal=True, scale=scaling,
                                         enable_gqa=query.shape[1] != key.shape[1])
    return out.transpose(1, 2).contiguous(), None


class ConditionBlockDecodeRunner:
    """The HF attention hook of the condition-block decode (CBT/core.py:1203-1355).

    Per call: prompt prefill (``q_len > 1``) goes to SDPA; a decode step of a layer
    outside ``layer_idx_list`` or below ``full_attention_layers`` goes to the HIP
    dense decode; any other decode step builds (once per layer) the layer's prompt
    summaries and runs the fused HIP condition path over the prompt blocks plus the
    exact suffix of generated tokens.  The suffix length is read by the kernels from
    ``suffix_len_dev``: ``reset_step`` writes it in the eager loop, the graph loop
    advances it on the device.  With ``static_suffix`` the hook passes the whole
    static-cache rows, so every shape is the same at every step."""

    def __init__(self, *, model, model_config, layer_idx_list, full_attention_layers, block_size, eps, prompt_len,
                 pos, prompt_prefix_cache, term1_mass_exp=False):
        self.model_config = model_config
        self.module_to_layer_idx = {id(layer.self_attn): i for i, layer in enumerate(model.model.layers)}
        self.layer_idx_set = set(map(int, layer_idx_list))
        self.full_attention_layers = int(full_attention_layers)
        self.block_size, self.eps = int(block_size), float(eps)
        self.prompt_len, self.pos = int(prompt_len), int(pos)
        self.prompt_prefix_cache = prompt_prefix_cache
        self.term1_mass_exp = bool(term1_mass_exp)
        self.workspace_by_layer = {}
        self.stats_by_layer, self.aggregate_stats = {}, {}
        self.skip_stats = _env_on(_SKIP_STATS)
        self.suffix_len_dev = torch.zeros((), dtype=torch.int32, device=next(model.parameters()).device)
        self.static_suffix = False

    def should_compress(self, layer_idx):
        return int(layer_idx) >= self.full_attention_layers and int(layer_idx) in self.layer_idx_set

    def summarize(self):
        return _summarize_stats_lazy(self.aggregate_stats, self.stats_by_layer)

    def reset_step(self, pos):
        """Start decode position ``pos``: the suffix holds the generated tokens up to it."""
        self.pos = int(pos)
        self.suffix_len_dev.fill_(max(0, self.pos + 1 - self.prompt_len))
        self.stats_by_layer.clear()
        self.aggregate_stats.clear()

    def _record(self, layer_idx, stats):
        self.stats_by_layer[int(layer_idx)] = stats
        _merge_stats_lazy(self.aggregate_stats, stats)

    def _prefix(self, layer_idx, k_rows, v_rows):
        """Prompt summaries of one layer, built on its first decode step and kept."""
        key = (int(layer_idx), self.prompt_len, self.block_size)
        if key not in self.prompt_prefix_cache:
            p = self.prompt_len
            self.prompt_prefix_cache[key] = _build_prompt_blocks(k_rows[:, :p], v_rows[:, :p], self.block_size)
        return self.prompt_prefix_cache[key]

    def hybrid_attention_forward(self, module, query, key, value, attention_mask, scaling, dropout=0.0, **kwargs):
        layer_idx = getattr(module, "layer_idx", None)
        if layer_idx is None:
            layer_idx = self.module_to_layer_idx.get(id(module))
        if query.shape[2] != 1:
            return _sdpa_prefill_attention_forward(module, query, key, value, attention_mask, scaling=scaling,
                                                   dropout=dropout, **kwargs)
        if layer_idx is None or not self.should_compress(layer_idx):
            if not self.skip_stats and layer_idx in self.layer_idx_set:
                self._record(layer_idx, full_attention_stats_for_heads(query.shape[1], [self.pos]))
            return _sdpa_full_attention_forward(module, query, key, value, attention_mask, scaling=scaling,
                                                dropout=dropout, **kwargs)
        return self._sparse_decode(int(layer_idx), query, key, value)

    def _sparse_decode(self, layer_idx, query, key, value):
        batch, n_heads, q_len, head_dim = query.shape
        if batch != 1 or q_len != 1:
            raise ValueError("condition_block fast path expects batch_size=1 and q_len=1.")
        if self.pos < self.prompt_len:
            raise ValueError("condition_block fast path expects generated-token decode positions.")
        n_kv_heads = int(key.shape[1])
        if n_heads % n_kv_heads:
            raise ValueError("condition_block fast path expects grouped query attention.")
        # rows of the cache this step may read: the whole static cache (validity from
        # suffix_len_dev), else the visible prefix
        visible = key.shape[2] if self.static_suffix else self.pos + 1
        k_rows, v_rows = key[0, :, :visible], value[0, :, :visible]
        prefix = self._prefix(layer_idx, k_rows, v_rows)
        out, stats = _condition_block_decode_output(
            q_grouped=query[0].view(n_kv_heads, n_heads // n_kv_heads, 1, head_dim), prompt_prefix=prefix,
            k_suffix=k_rows[:, self.prompt_len:], v_suffix=v_rows[:, self.prompt_len:],
            suffix_len_dev=self.suffix_len_dev, block_size=self.block_size, eps=self.eps,
            prompt_len=self.prompt_len, attention_dtype=query.dtype,
            workspace=self.workspace_by_layer.setdefault(layer_idx, {}), term1_mass_exp=self.term1_mass_exp,
            collect_stats=not self.skip_stats)
        if stats is not None:
            self._record(layer_idx, stats)
        # [Hkv, G, 1, D] -> the HF layout [1, q_len, Hq, D]
        return out.reshape(1, 1, n_heads, head_dim).to(query.dtype), None


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
def _swapped(owner, name, value):
    """Temporarily replace ``owner.name`` with ``value``."""
    saved = getattr(owner, name)
    setattr(owner, name, value)
    try:
        yield
    finally:
        setattr(owner, name, saved)


def _no_causal_mask_context():
    """No HF causal-mask construction during the graphed step (CBT/core.py:1358): the
    sparse layers ignore the mask, and building it copies a host scalar to the device,
    which graph capture forbids."""
    return _swapped(_modeling_llama(), "create_causal_mask", lambda *args, **kwargs: None)


@contextlib.contextmanager
def condition_block_decode_context(runner):
    """Route HF's eager attention through ``runner`` (CBT/core.py:1373)."""
    with _swapped(_modeling_llama(), "eager_attention_forward", runner.hybrid_attention_forward):
        yield runner


def full_attention_sdpa_context():
    """Every decode on the HIP dense path (CBT/core.py:1383)."""
    return _swapped(_modeling_llama(), "eager_attention_forward", _sdpa_full_attention_forward)


def model_attention_implementation(model, implementation):
    """Run the model under another HF attention implementation (CBT/core.py:1393)."""
    return _swapped(model.config, "_attn_implementation", implementation)


# ------------------------------------------------------------------ generation

def run_prefill_only_condition_block(**_kwargs):
    raise RuntimeError("condition_block now uses the cached generate path only. "
                       "Call generate_condition_block_cached through generate_with_method().")


def build_condition_args(method, prompt_len):
    return SimpleNamespace(seq_len=int(prompt_len), block_size=method.condition_block_size,
                           full_attention_layers=int(method.full_attention_layers),
                           delta_mode=method.condition_delta_mode)


def _stop_token_ids(tokenizer, dataset):
    """EOS, plus the newline token for samsum (its answers are one line)."""
    if tokenizer is None:
        return []
    ids = [] if tokenizer.eos_token_id is None else [int(tokenizer.eos_token_id)]
    if dataset == "samsum":
        ids += [int(t) for t in tokenizer.encode("\n", add_special_tokens=False)[-1:]]
    return ids


def _static_cache_from_prefill(config, prefill_cache, max_cache_len):
    """A ``StaticCache`` of ``max_cache_len`` holding the prefill's K/V (CBT/core.py:317):
    written through the cache's ``update`` so that its length counter points past the
    prompt and the first decode step writes right after it."""
    from transformers import StaticCache

    static = StaticCache(config=config, max_cache_len=int(max_cache_len))
    for i, layer in enumerate(prefill_cache.layers):
        static.update(layer.keys, layer.values, i)
    return static


def _prefill(model, input_ids, attention_mask, past_key_values=None):
    """Prompt forward on torch SDPA; returns (first greedy token [1, 1], KV cache)."""
    with model_attention_implementation(model, "sdpa"), torch.no_grad():
        out = model(input_ids=input_ids, attention_mask=attention_mask, past_key_values=past_key_values,
                    use_cache=True, logits_to_keep=1)
    return out.logits[:, -1].float().argmax(-1, keepdim=True), out.past_key_values


class _GreedyStep:
    """Device state of greedy decoding and one decode step over it.

    ``tokens[i]`` receives generated token ``i``; the step feeds ``step_ids`` at
    ``cache_pos``, writes the argmax at ``tokens[slot]`` and advances the input, the
    position, the slot and (graph mode) the runner's suffix length, all on the
    device, so one step can be captured and replayed.  The eager loop runs the same
    step and additionally grows the attention mask on the host."""

    def __init__(self, model, runner, cache, first, prompt_len, n_new, *, mask=None, advance_suffix=False):
        dev = first.device
        self.model, self.runner, self.cache = model, runner, cache
        self.tokens = torch.zeros(n_new, dtype=first.dtype, device=dev)
        self.tokens[:1] = first.view(1)
        self.step_ids = first.view(1, 1).clone()
        self.cache_pos = torch.full((1,), int(prompt_len), dtype=torch.long, device=dev)
        self.slot = torch.ones(1, dtype=torch.long, device=dev)
        self.mask = mask
        self.advance_suffix = advance_suffix

    def __call__(self):
        out = self.model(input_ids=self.step_ids, attention_mask=self.mask, past_key_values=self.cache,
                         use_cache=True, logits_to_keep=1, cache_position=self.cache_pos)
        nxt = out.logits[0, -1].float().argmax(-1).view(1)
        self.tokens.index_copy_(0, self.slot, nxt)
        self.step_ids.copy_(nxt.view(1, 1))
        self.cache_pos.add_(1)
        self.slot.add_(1)
        if self.advance_suffix:
            self.runner.suffix_len_dev.add_(1)
        self.cache = out.past_key_values
        return nxt


def _runner_for(model, method, prompt_len, pos, term1_mass_exp):
    return ConditionBlockDecodeRunner(
        model=model, model_config=model.config, layer_idx_list=range(int(model.config.num_hidden_layers)),
        full_attention_layers=method.full_attention_layers, block_size=method.condition_block_size,
        eps=method.condition_eps, prompt_len=prompt_len, pos=pos, prompt_prefix_cache={},
        term1_mass_exp=term1_mass_exp)


def generate_condition_block_cached(*, model, tokenizer, input_ids, attention_mask, method, device, dataset=None,
                                    term1_mass_exp=False):
    """Greedy generation: SDPA prefill, then condition-block decode one token at a
    time (CBT/core.py:60-186), stopping at a stop token.  ``method`` carries
    ``condition_delta_mode, condition_block_size, condition_eps,
    full_attention_layers, max_new_tokens``.  Returns ``(output_ids [1, n], metadata)``;
    with ``CONDITION_BLOCK_CUDA_GRAPH=1`` the graph-replay loop runs instead."""
    if method.condition_delta_mode != "range_bound":
        raise ValueError("condition_block only supports delta_mode='range_bound'.")
    if int(input_ids.shape[0]) != 1:
        raise ValueError("condition_block generate currently expects batch_size=1.")
    if _env_on("CONDITION_BLOCK_CUDA_GRAPH"):
        return _generate_condition_block_cuda_graph(model=model, tokenizer=tokenizer, input_ids=input_ids,
                                                    attention_mask=attention_mask, method=method, dataset=dataset,
                                                    term1_mass_exp=term1_mass_exp)
    prompt_len, n_new = int(input_ids.shape[1]), int(method.max_new_tokens)
    if n_new <= 0:
        return input_ids.new_empty((1, 0)), summarize_condition_block_step_metadata([])
    stop_ids = torch.tensor(_stop_token_ids(tokenizer, dataset), device=input_ids.device, dtype=input_ids.dtype)
    cache = None
    if _env_on("CONDITION_BLOCK_STATIC_CACHE"):
        from transformers import StaticCache

        cache = StaticCache(config=model.config, max_cache_len=prompt_len + n_new)
    first, cache = _prefill(model, input_ids, attention_mask, cache)
    if _env_on("CONDITION_BLOCK_POST_PREFILL_STATIC_CACHE"):
        cache = _static_cache_from_prefill(model.config, cache, prompt_len + n_new)
    collect = not _env_on(_SKIP_STATS)
    metadata = [_full_generation_step_metadata(model, [prompt_len - 1])] if collect else []
    runner = _runner_for(model, method, prompt_len, prompt_len, term1_mass_exp)
    step = _GreedyStep(model, runner, cache, first.view(1), prompt_len, n_new,
                       mask=torch.cat([attention_mask, torch.ones_like(first)], dim=1))
    n_done = 1
    with condition_block_decode_context(runner), mask_prefix_hint(mask_is_prefix(step.mask)), torch.no_grad():
        while n_done < n_new and not bool(torch.isin(step.tokens[n_done - 1], stop_ids)):
            runner.reset_step(prompt_len + n_done - 1)
            step()
            if collect:
                metadata.append(runner.summarize())
            n_done += 1
            step.mask = torch.cat([step.mask, step.mask.new_ones((1, 1))], dim=1)
    return step.tokens[:n_done].view(1, -1).to(input_ids.dtype), summarize_condition_block_step_metadata(metadata)


def _generate_condition_block_cuda_graph(*, model, tokenizer, input_ids, attention_mask, method, dataset=None,
                                         term1_mass_exp=False):
    """One graph replay per generated token (CBT/core.py:189-314): SDPA prefill, the
    prompt K/V moved into a ``StaticCache``, a few eager steps on a side stream
    (summaries and workspaces are allocated there), then the decode step captured
    once and replayed; stop tokens truncate the output afterwards.  Requires
    ``CONDITION_BLOCK_SKIP_STATS=1``, ``full_attention_layers=0`` and a block size
    that is a positive multiple of 16 (every such size runs the fused HIP path)."""
    if not _env_on(_SKIP_STATS):
        raise ValueError("CONDITION_BLOCK_CUDA_GRAPH=1 requires CONDITION_BLOCK_SKIP_STATS=1.")
    if int(method.full_attention_layers) != 0:
        raise ValueError("CUDA-graph decode supports full_attention_layers=0 only.")
    block = int(method.condition_block_size)
    if block <= 0 or block % 16:
        raise ValueError("CUDA-graph decode requires a block size that is a positive multiple of 16.")
    prompt_len, n_new = int(input_ids.shape[1]), int(method.max_new_tokens)
    if n_new <= 0:
        return input_ids.new_empty((1, 0)), summarize_condition_block_step_metadata([])
    first, cache = _prefill(model, input_ids, attention_mask)
    cache = _static_cache_from_prefill(model.config, cache, prompt_len + n_new)
    runner = _runner_for(model, method, prompt_len, prompt_len, term1_mass_exp)
    runner.static_suffix = True
    runner.suffix_len_dev.fill_(1)
    step = _GreedyStep(model, runner, cache, first.view(1), prompt_len, n_new, advance_suffix=True)
    eager_steps = min(3, n_new - 1)
    with condition_block_decode_context(runner), _no_causal_mask_context(), torch.no_grad():
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(eager_steps):
                step()
        torch.cuda.current_stream().wait_stream(side)
        if n_new - 1 > eager_steps:
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                step()
            for _ in range(n_new - 1 - eager_steps):
                graph.replay()
    torch.cuda.synchronize()
    stops = set(_stop_token_ids(tokenizer, dataset))
    tokens = step.tokens.tolist()
    n_keep = next((i + 1 for i, t in enumerate(tokens) if t in stops), len(tokens))
    out = step.tokens[:n_keep].view(1, -1).to(input_ids.dtype)
    return out, {"condition_block_stats_disabled": True, "cuda_graph_decode": True}
