"""INTEGRATION.md's replacement block for ``FastBSRoformer.forward`` (fast.py:377-387) reads only names that
exist at that point of the reference's ``forward``, or that the block defines itself, and every ``self.``
attribute it reads exists on the reference's ``FastBSRoformer`` or is one the ``_configure`` snippet sets
on ``self.net``; the op-by-op ``_transformer_cpp`` snippet reads only ``self.`` attributes the reference
class has.  The reference's fast.py is parsed as text (ast), never imported; skipped where it is absent.
"""

from __future__ import annotations

import ast
import builtins
import re
import textwrap
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
DOC = ROOT / "INTEGRATION.md"
REF_FAST = Path("/root/reference/src/turbo_roformer/fast.py")

pytestmark = pytest.mark.skipif(not REF_FAST.exists(), reason="the reference checkout is not present")


def _code_blocks(text: str) -> list[str]:
    return [m.group(1) for m in re.finditer(r"```python\n(.*?)```", text, re.S)]


def _block_with(marker: str) -> ast.Module:
    blocks = [b for b in _code_blocks(DOC.read_text()) if marker in b]
    assert len(blocks) == 1, f"exactly one INTEGRATION.md block contains {marker!r}"
    return ast.parse(textwrap.dedent(blocks[0]))


def _reference_class() -> ast.ClassDef:
    tree = ast.parse(REF_FAST.read_text())
    return next(n for n in tree.body if isinstance(n, ast.ClassDef) and n.name == "FastBSRoformer")


def _module_names() -> set[str]:
    tree = ast.parse(REF_FAST.read_text())
    names = set()
    for n in tree.body:
        if isinstance(n, (ast.Import, ast.ImportFrom)):
            names |= {(a.asname or a.name).split(".")[0] for a in n.names}
        elif isinstance(n, (ast.FunctionDef, ast.ClassDef)):
            names.add(n.name)
        elif isinstance(n, (ast.Assign, ast.AnnAssign)):
            for t in n.targets if isinstance(n, ast.Assign) else [n.target]:
                names |= {x.id for x in ast.walk(t) if isinstance(x, ast.Name)}
    return names


def _stored(nodes) -> set[str]:
    return {x.id for n in nodes for x in ast.walk(n) if isinstance(x, ast.Name) and isinstance(x.ctx, ast.Store)}


def _loaded(tree) -> set[str]:
    return {x.id for x in ast.walk(tree) if isinstance(x, ast.Name) and isinstance(x.ctx, ast.Load)}


def _self_attrs_read(tree) -> set[str]:
    return {x.attr for x in ast.walk(tree)
            if isinstance(x, ast.Attribute) and isinstance(x.value, ast.Name) and x.value.id == "self"
            and isinstance(x.ctx, ast.Load)}


def _class_attrs(cls: ast.ClassDef) -> set[str]:
    attrs = {n.name for n in cls.body if isinstance(n, (ast.FunctionDef, ast.AsyncFunctionDef))}
    for x in ast.walk(cls):
        if isinstance(x, ast.Attribute) and isinstance(x.value, ast.Name) and x.value.id == "self" \
                and isinstance(x.ctx, ast.Store):
            attrs.add(x.attr)
    return attrs


def _configure_sets() -> set[str]:
    tree = _block_with("resolve_backend(backend)")
    out = set()
    for x in ast.walk(tree):
        if isinstance(x, ast.Attribute) and isinstance(x.ctx, ast.Store) and isinstance(x.value, ast.Attribute) \
                and isinstance(x.value.value, ast.Name) and x.value.value.id == "self" and x.value.attr == "net":
            out.add(x.attr)
    return out


def _forward_before_band_split() -> tuple[ast.FunctionDef, set[str]]:
    fwd = next(n for n in _reference_class().body if isinstance(n, ast.FunctionDef) and n.name == "forward")
    cut = next(i for i, st in enumerate(fwd.body)
               if isinstance(st, ast.With) and "band_split" in ast.unparse(st.items[0].context_expr))
    defined = {a.arg for a in fwd.args.args} | _stored(fwd.body[:cut])
    return fwd, defined


def test_forward_block_reads_only_names_in_scope():
    snippet = _block_with('with tm("band_split")')
    _, before = _forward_before_band_split()
    allowed = before | _stored(snippet.body) | _module_names() | set(dir(builtins))
    missing = _loaded(snippet) - allowed
    assert not missing, f"names read by the block but not defined in forward's scope: {sorted(missing)}"
    # the lines after the block (complex multiply, iSTFT) read mask; the block sets it on both branches
    assert "mask" in _stored(snippet.body)


def test_forward_block_reads_only_existing_attributes():
    snippet = _block_with('with tm("band_split")')
    hip_attrs = _configure_sets()
    assert {"stack", "hip_band_split", "mask_head"} <= hip_attrs
    unknown = _self_attrs_read(snippet) - _class_attrs(_reference_class()) - hip_attrs
    assert not unknown, f"self attributes neither on FastBSRoformer nor set by _configure: {sorted(unknown)}"


def test_op_by_op_loop_reads_only_existing_attributes():
    snippet = _block_with("hip_ops.gemm_res_norm(O")
    unknown = _self_attrs_read(snippet) - _class_attrs(_reference_class())
    assert not unknown, f"self attributes not on FastBSRoformer: {sorted(unknown)}"
