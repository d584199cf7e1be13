"""Kernel-body fingerprints: the guard that keeps signature dispatch honest.

A decorated kernel is matched to a native kernel by its name and parameter names
(pyasc_amd.registry).  Two bodies with the same signature can compute different
things, so a body is also compared, by a fingerprint of its syntax tree, with the
bodies the registered native kernel stands for (the reference's kernels of that
signature, recorded in kernel_fingerprints.json by make_fingerprints.py).

Normalisation, so that a fingerprint depends only on what the body computes:
  - comments, blank lines and formatting are not in the tree;
  - a leading docstring is dropped;
  - local names (anything the body assigns or binds: assignment and loop targets,
    ``with ... as``, comprehension variables) are renamed _v0, _v1, ... in order
    of first appearance, so renaming a local variable keeps the fingerprint;
  - a temporary that is assigned once (``t = expr``) and read once, in the
    statement right after, is replaced by its expression there, so
    ``t = x + y; store(t, ...)`` and ``store(x + y, ...)`` agree;
  - the loop hints of ``range`` / ``asc2.range`` (``unroll_factor``, ``parallel``)
    are dropped: they set attributes of the loop (python/asc/language/tile/range.py:
    16-36), not what it computes;
  - parameter names, attribute names, module names and constants are kept.
The tree is serialised with ``ast.dump`` (field names, no line numbers) and hashed
with SHA-256; the first 16 hex digits are the fingerprint.

A body made only of a docstring, ``pass`` and ``...`` is a *declaration*: it
states the signature and computes nothing itself, so it binds to the registered
native kernel by signature alone (the form the build-defined kernels, which have
no reference body, are declared in).
"""
from __future__ import annotations

import ast
import copy
import hashlib
import inspect
import json
import os
import textwrap
from typing import Callable, Dict, FrozenSet, List, Optional, Tuple

DECLARATION = "declaration"
FINGERPRINTS_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "kernel_fingerprints.json")


def _strip_docstring(body: List[ast.stmt]) -> List[ast.stmt]:
    if body and isinstance(body[0], ast.Expr) and isinstance(body[0].value, ast.Constant) \
            and isinstance(body[0].value.value, str):
        return body[1:]
    return body


def is_declaration(body: List[ast.stmt]) -> bool:
    """True for a body of only a docstring, ``pass`` and ``...``."""
    for stmt in _strip_docstring(body):
        if isinstance(stmt, ast.Pass):
            continue
        if isinstance(stmt, ast.Expr) and isinstance(stmt.value, ast.Constant) and stmt.value.value is Ellipsis:
            continue
        return False
    return True


LOOP_HINTS = frozenset({"unroll_factor", "parallel"})


def _is_range(func: ast.expr) -> bool:
    return (isinstance(func, ast.Name) and func.id == "range") or \
        (isinstance(func, ast.Attribute) and func.attr == "range")


class _LocalRenamer(ast.NodeTransformer):
    """Renames the names a body binds to _v0, _v1, ... in order of first binding and
    drops the loop hints of range calls."""

    def __init__(self, bound: List[str]):
        self.mapping = {name: f"_v{i}" for i, name in enumerate(bound)}

    def visit_Call(self, node: ast.Call) -> ast.Call:
        self.generic_visit(node)
        if _is_range(node.func):
            node.keywords = [k for k in node.keywords if k.arg not in LOOP_HINTS]
        return node

    def visit_Name(self, node: ast.Name) -> ast.Name:
        new = self.mapping.get(node.id)
        if new is not None:
            return ast.copy_location(ast.Name(id=new, ctx=node.ctx), node)
        return node


def _bound_names(body: List[ast.stmt], params: Tuple[str, ...]) -> List[str]:
    """Names the body binds (Store context), in order of first appearance, parameters excluded."""
    order: List[str] = []
    seen = set(params)
    for stmt in body:
        for node in ast.walk(stmt):
            if isinstance(node, ast.Name) and isinstance(node.ctx, (ast.Store, ast.Del)) and node.id not in seen:
                seen.add(node.id)
                order.append(node.id)
    return order


def _name_counts(nodes) -> Tuple[Dict[str, int], Dict[str, int]]:
    loads: Dict[str, int] = {}
    stores: Dict[str, int] = {}
    for root in nodes:
        for node in ast.walk(root):
            if isinstance(node, ast.Name):
                d = loads if isinstance(node.ctx, ast.Load) else stores
                d[node.id] = d.get(node.id, 0) + 1
    return loads, stores


class _Substitute(ast.NodeTransformer):
    def __init__(self, name: str, expr: ast.expr):
        self.name, self.expr = name, expr

    def visit_Name(self, node: ast.Name) -> ast.expr:
        if node.id == self.name and isinstance(node.ctx, ast.Load):
            return copy.deepcopy(self.expr)
        return node


def _inline_temporaries(body: List[ast.stmt], loads: Dict[str, int], stores: Dict[str, int]) -> List[ast.stmt]:
    """Substitutes single-use temporaries into the next statement, in every block."""
    out: List[ast.stmt] = []
    for stmt in body:
        for field in ("body", "orelse", "finalbody"):
            block = getattr(stmt, field, None)
            if isinstance(block, list) and block and isinstance(block[0], ast.stmt):
                setattr(stmt, field, _inline_temporaries(block, loads, stores))
        prev = out[-1] if out else None
        if (isinstance(prev, ast.Assign) and len(prev.targets) == 1 and isinstance(prev.targets[0], ast.Name)):
            name = prev.targets[0].id
            used_here = sum(1 for n in ast.walk(stmt) if isinstance(n, ast.Name) and n.id == name)
            if stores.get(name) == 1 and loads.get(name) == 1 and used_here == 1:
                out.pop()
                stmt = _Substitute(name, prev.value).visit(stmt)
        out.append(stmt)
    return out


def body_fingerprint(func: ast.FunctionDef) -> str:
    """Fingerprint of a parsed function's body ("declaration" for an empty body)."""
    params = tuple(a.arg for a in func.args.args)
    body = _strip_docstring(list(func.body))
    if is_declaration(body):
        return DECLARATION
    body = [_clone(stmt) for stmt in body]
    loads, stores = _name_counts(body)
    body = _inline_temporaries(body, loads, stores)
    renamer = _LocalRenamer(_bound_names(body, params))
    text = "\n".join(ast.dump(renamer.visit(stmt), annotate_fields=True, include_attributes=False)
                     for stmt in body)
    return hashlib.sha256(text.encode()).hexdigest()[:16]


def _clone(node: ast.AST) -> ast.AST:
    return copy.deepcopy(node)


def function_node(fn: Callable) -> Optional[ast.FunctionDef]:
    """The parsed definition of ``fn`` (None when its source is not available)."""
    try:
        src = textwrap.dedent(inspect.getsource(fn))
    except (OSError, TypeError):
        return None
    tree = ast.parse(src)
    for node in tree.body:
        if isinstance(node, (ast.FunctionDef, ast.AsyncFunctionDef)) and node.name == fn.__name__:
            return node
    return None


def fingerprint_of(fn: Callable) -> Optional[str]:
    node = function_node(fn)
    return None if node is None else body_fingerprint(node)


def signature_key(name: str, params: Tuple[str, ...]) -> str:
    return f"{name}({', '.join(params)})"


_table: Optional[Dict[str, FrozenSet[str]]] = None


def known_fingerprints() -> Dict[str, FrozenSet[str]]:
    """signature key -> fingerprints of the reference bodies of that signature."""
    global _table
    if _table is None:
        with open(FINGERPRINTS_FILE) as f:
            data = json.load(f)
        _table = {key: frozenset(item["fingerprint"] for item in items) for key, items in data["kernels"].items()}
    return _table
