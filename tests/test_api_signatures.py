"""The kernel-level mirrors keep the reference's Python signatures.

kernels/flash_attn.py:130-137 defines
    flash_attention(q, k, v, causal=True, sm_scale=None, use_triton=True)
and kernels/rope.py:99-105
    apply_rope(q, k, cos, sin, use_triton=True).
The expected parameter lists are written out below; when the reference tree is
present (this container, not the GPU box) its source is also parsed as text
with ``ast`` (never imported) and compared, so a drift on either side fails.
"""

import ast
import inspect
import os

import pytest

from nano_qwen_amd import ops
import nano_qwen_amd as nq

REF = "/root/reference"
EXPECTED = {
    ("kernels/flash_attn.py", "flash_attention"): [
        ("q", inspect.Parameter.empty), ("k", inspect.Parameter.empty), ("v", inspect.Parameter.empty),
        ("causal", True), ("sm_scale", None), ("use_triton", True)],
    ("kernels/rope.py", "apply_rope"): [
        ("q", inspect.Parameter.empty), ("k", inspect.Parameter.empty), ("cos", inspect.Parameter.empty),
        ("sin", inspect.Parameter.empty), ("use_triton", True)],
}


def _mirror_params(fn):
    return [(p.name, p.default) for p in inspect.signature(fn).parameters.values()]


@pytest.mark.parametrize("key", list(EXPECTED))
def test_mirror_signature_matches_reference(key):
    _, name = key
    fn = getattr(ops, name)
    assert _mirror_params(fn) == EXPECTED[key]
    assert getattr(nq, name) is fn  # the package re-exports the mirror


def _ref_params(path, name):
    tree = ast.parse(open(path).read())
    for node in tree.body:
        if isinstance(node, ast.FunctionDef) and node.name == name:
            a = node.args
            names = [x.arg for x in a.args]
            defaults = [ast.literal_eval(d) for d in a.defaults]
            pad = [inspect.Parameter.empty] * (len(names) - len(defaults))
            return list(zip(names, pad + defaults))
    raise AssertionError(f"{name} not found in {path}")


@pytest.mark.skipif(not os.path.isdir(REF), reason="reference tree not present")
@pytest.mark.parametrize("key", list(EXPECTED))
def test_expected_signature_is_the_reference_source(key):
    rel, name = key
    assert _ref_params(os.path.join(REF, rel), name) == EXPECTED[key]
