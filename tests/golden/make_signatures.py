"""Extract the call signatures of the reference's entry points on this path by
parsing its source text (ast; nothing is imported or executed) and write them to
``reference_signatures.json`` beside this script.  Run in the build container only:

    python tests/golden/make_signatures.py /root/reference

For each function: positional parameter names, keyword-only parameter names, which
of them have defaults, and whether ``*args`` / ``**kwargs`` are accepted.  Methods are
keyed ``Class.method``.
"""

import ast
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CBT = "llama/script/analysis/condition_block_gen/methods/condition_block_triton_impl/core.py"
FIXED = "llama/script/analysis/condition_block_gen/real_attention_benchmark/fixed_mask.py"

WANTED = {
    CBT: [
        "_summary_storage_dtypes", "_build_prompt_blocks", "_run_condition_block_selection_stats",
        "_select_prompt_blocks_triton", "_condition_block_decode_output", "_condition_block_decode_output_fused_triton",
        "_sdpa_full_attention_forward", "_sdpa_prefill_attention_forward", "_condition_stats",
        "generate_condition_block_cached", "_generate_condition_block_cuda_graph", "_static_cache_from_prefill",
        "condition_block_decode_context", "full_attention_sdpa_context", "model_attention_implementation",
        "full_attention_stats_for_heads", "summarize_condition_block_step_metadata", "build_condition_args",
        "run_prefill_only_condition_block",
        "ConditionBlockDecodeRunner.__init__", "ConditionBlockDecodeRunner.hybrid_attention_forward",
        "ConditionBlockDecodeRunner.reset_step", "ConditionBlockDecodeRunner.should_compress",
        "ConditionBlockDecodeRunner.summarize",
    ],
    FIXED: ["fixed_mask_hybrid_attention"],
}


def describe(fn):
    a = fn.args
    pos = [x.arg for x in a.posonlyargs + a.args]
    n_def = len(a.defaults)
    pos_def = pos[len(pos) - n_def:] if n_def else []
    kw = [x.arg for x in a.kwonlyargs]
    kw_def = [x.arg for x, d in zip(a.kwonlyargs, a.kw_defaults) if d is not None]
    return {"positional": pos, "positional_with_default": pos_def, "keyword_only": kw,
            "keyword_only_with_default": kw_def, "varargs": a.vararg is not None, "varkw": a.kwarg is not None}


def main(root):
    out = {}
    for rel, names in WANTED.items():
        tree = ast.parse(open(os.path.join(root, rel)).read())
        found = {}
        for node in tree.body:
            if isinstance(node, ast.FunctionDef):
                found[node.name] = node
            elif isinstance(node, ast.ClassDef):
                for sub in node.body:
                    if isinstance(sub, ast.FunctionDef):
                        found[f"{node.name}.{sub.name}"] = sub
        for name in names:
            out[name] = {"source": f"{rel}:{found[name].lineno}", **describe(found[name])}
    with open(os.path.join(HERE, "reference_signatures.json"), "w") as f:
        json.dump(out, f, indent=1, sort_keys=True)
    print(f"wrote {len(out)} signatures")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
