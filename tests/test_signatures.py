"""The reference-API mirror keeps the reference's call signatures: the golden file
``tests/golden/reference_signatures.json`` holds the signatures of the reference's
entry points, extracted from its source text by ``tests/golden/make_signatures.py``
(ast, nothing imported).  Every reference call must bind to ours: the same
positional parameters in the same order, every keyword-only parameter present,
defaults wherever the reference has one, extra parameters only with defaults."""

import inspect
import json
import os

import pytest

from interattn_amd import condition_block, decode

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
REF = json.load(open(os.path.join(HERE, "reference_signatures.json")))


def _resolve(name):
    obj = None
    for mod in (condition_block, decode):
        head, _, tail = name.partition(".")
        if hasattr(mod, head):
            obj = getattr(mod, head)
            if tail:
                obj = getattr(obj, tail)
            return obj
    raise AssertionError(f"{name} is not provided")


@pytest.mark.parametrize("name", sorted(REF))
def test_signature_matches_reference(name):
    ref = REF[name]
    sig = inspect.signature(_resolve(name))
    params = list(sig.parameters.values())
    pos = [p for p in params if p.kind in (p.POSITIONAL_ONLY, p.POSITIONAL_OR_KEYWORD)]
    kw = {p.name: p for p in params if p.kind == p.KEYWORD_ONLY}
    has_varkw = any(p.kind == p.VAR_KEYWORD for p in params)
    has_varargs = any(p.kind == p.VAR_POSITIONAL for p in params)
    assert [p.name for p in pos[:len(ref["positional"])]] == ref["positional"], ref["source"]
    for extra in pos[len(ref["positional"]):]:
        assert extra.default is not extra.empty, f"extra positional {extra.name} needs a default"
    by_name = {p.name: p for p in params}
    for nm in ref["positional_with_default"] + ref["keyword_only_with_default"]:
        assert by_name[nm].default is not inspect.Parameter.empty, f"{nm} must keep a default"
    for nm in ref["keyword_only"]:
        assert nm in kw or nm in by_name, f"keyword {nm} missing"
    for nm, p in kw.items():
        if nm not in ref["keyword_only"]:
            assert p.default is not p.empty, f"extra keyword {nm} needs a default"
    if ref["varkw"]:
        assert has_varkw, "the reference accepts **kwargs"
    if ref["varargs"]:
        assert has_varargs, "the reference accepts *args"
