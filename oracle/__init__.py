"""CPU oracle for the condition-block sparse decode-attention path.

TEST INFRASTRUCTURE ONLY.  Nothing in ``interattn_amd`` imports this package:
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` use it, and only as the checker.  The product path is the HIP
library and fails loudly when that library is missing.

Every function restates the reference's algorithm in numpy (float64 unless a
rounding point of the reference is being emulated) and cites the reference
file:line it follows.  Paths are relative to the reference repository root;
``CBT`` abbreviates
``llama/script/analysis/condition_block_gen/methods/condition_block_triton_impl``
and ``CBG`` abbreviates ``llama/script/analysis/condition_block_gen``.

How each function is pinned (checked by ``tests/test_oracle.py``):

=====================================  =========================================
function                               pinned by
=====================================  =========================================
numerics.bf16_round / fp8 codec        torch's own bf16 / float8_e4m3fn casts
paged.paged_gather / scatter           brute-force loop + permutation invariance
summaries.build_block_summaries        per-block brute-force loops, invariants,
                                       golden fixtures from the reference
select.topk_block_scores/select_topk   brute-force sort, forced-block rules
select.quest_block_scores              upper bound of every token's score,
                                       one-token blocks, all-positive /
                                       all-negative query closed forms
torch_path.topk_layer_call             the numpy oracle above (selection
                                       exact, outputs to float32 rounding)
select.select_condition_eager          golden fixtures from the reference,
                                       eps=0 / eps=1e9 closed forms
select.selection_stats_chunked         chunked LSE == global LSE, golden s/delta
attention.dense_decode                 torch SDPA (float64) with GQA
attention.sparse_decode                all-blocks == dense, brute-force mask
attention.hybrid_decode_dense          golden fixtures from the reference,
                                       all-selected == SDPA, none-selected ==
                                       closed-form representative softmax
attention.splitk_merge                 n_chunks=1 identity, chunking invariance
=====================================  =========================================
"""

from . import numerics, paged, summaries, select, attention  # noqa: F401

# torch_path (the timed CPU baseline) is imported on demand: it needs torch
