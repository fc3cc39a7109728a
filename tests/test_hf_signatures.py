"""The drop-in wrappers keep the signatures of HF's replaceable delta-rule functions (transformers 5.15.0
models/qwen3_5/modeling_qwen3_5.py: torch_chunk_gated_delta_rule at HF:249, torch_recurrent_gated_delta_rule at
HF:331, plugged in by name through use_kernel_func_from_hub_with_fallback at HF:248 / HF:330): the same parameter
names in the same order, the same defaults where HF has one, extra parameters only after them with defaults, and
**kwargs. HF's source is read as text (ast); nothing of it is imported or run. CPU only."""
import ast
import importlib.util
import inspect
import os

import pytest

import q35hip

HF_FUNCS = {"torch_chunk_gated_delta_rule": "chunk_gated_delta_rule",
            "torch_recurrent_gated_delta_rule": "recurrent_gated_delta_rule"}


def _hf_defs():
    spec = importlib.util.find_spec("transformers")
    if spec is None or not spec.submodule_search_locations:
        pytest.skip("transformers is not installed: nothing to compare against")
    path = os.path.join(list(spec.submodule_search_locations)[0], "models", "qwen3_5", "modeling_qwen3_5.py")
    if not os.path.exists(path):
        pytest.skip("this transformers has no qwen3_5 model")
    with open(path) as f:
        tree = ast.parse(f.read())
    return {n.name: n for n in tree.body if isinstance(n, ast.FunctionDef) and n.name in HF_FUNCS}


@pytest.mark.parametrize("hf_name", sorted(HF_FUNCS))
def test_wrapper_signature_matches_hf(hf_name):
    fn = _hf_defs()[hf_name]
    hf_args = [a.arg for a in fn.args.args]
    hf_defaults = dict(zip(hf_args[len(hf_args) - len(fn.args.defaults):],
                           [ast.literal_eval(d) for d in fn.args.defaults]))
    assert fn.args.kwarg is not None
    ours = inspect.signature(getattr(q35hip, HF_FUNCS[hf_name])).parameters
    names = [n for n, p in ours.items() if p.kind == p.POSITIONAL_OR_KEYWORD]
    assert names[:len(hf_args)] == hf_args, (names, hf_args)
    for n, d in hf_defaults.items():
        assert ours[n].default == d, (n, ours[n].default, d)
    for n in names[len(hf_args):]:
        assert ours[n].default is not inspect.Parameter.empty, f"extra parameter {n} needs a default"
    assert any(p.kind == p.VAR_KEYWORD for p in ours.values())
