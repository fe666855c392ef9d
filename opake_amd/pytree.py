"""Minimal pytree utilities with the reference's leaf order.

The reference flattens with optree 0.20.0, which visits ``dict`` keys in
sorted order (``packages/opake-engine/src/opake/api/engine/pytree.py:90-164``).
Leaf order matters on this path: the reference-stream Gaussian noise is drawn
leaf by leaf from one generator in flatten order.  Supported containers are
``dict`` (sorted keys), ``list``, ``tuple`` and namedtuples; ``None`` is an
empty subtree, as in optree.  Everything else is a leaf.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Callable

import torch

from opake_amd.exceptions import InputTypeError

ParamPath = tuple  # tuple[str | int, ...]; the reference's ``ParamPath`` alias


@dataclass(frozen=True)
class TreeDef:
    """Structure of a flattened tree: node kind, aux data and children."""

    kind: str  # "leaf" | "none" | "dict" | "list" | "tuple" | "namedtuple"
    aux: Any
    children: tuple

    @property
    def num_leaves(self) -> int:
        if self.kind == "leaf":
            return 1
        return sum(c.num_leaves for c in self.children)


_LEAF = TreeDef("leaf", None, ())
_NONE = TreeDef("none", None, ())


def _is_namedtuple(x: Any) -> bool:
    return isinstance(x, tuple) and hasattr(x, "_fields")


def _flatten(tree: Any, path: tuple, paths: list, leaves: list) -> TreeDef:
    if tree is None:
        return _NONE
    if isinstance(tree, dict):
        keys = sorted(tree.keys())
        children = tuple(_flatten(tree[k], path + (k,), paths, leaves) for k in keys)
        return TreeDef("dict", (tuple(keys), type(tree)), children)
    if _is_namedtuple(tree):
        children = tuple(
            _flatten(v, path + (f,), paths, leaves) for f, v in zip(tree._fields, tree)
        )
        return TreeDef("namedtuple", type(tree), children)
    if isinstance(tree, (list, tuple)):
        children = tuple(_flatten(v, path + (i,), paths, leaves) for i, v in enumerate(tree))
        return TreeDef("list" if isinstance(tree, list) else "tuple", None, children)
    paths.append(path)
    leaves.append(tree)
    return _LEAF


def tree_flatten_with_paths(tree: Any) -> tuple[list[ParamPath], list[Any], TreeDef]:
    """Flatten to ``(paths, leaves, treedef)``; a root leaf has path ``()``."""
    paths: list = []
    leaves: list = []
    treedef = _flatten(tree, (), paths, leaves)
    return paths, leaves, treedef


def tree_flatten(tree: Any) -> tuple[list[Any], TreeDef]:
    _, leaves, treedef = tree_flatten_with_paths(tree)
    return leaves, treedef


def _unflatten(treedef: TreeDef, it) -> Any:
    if treedef.kind == "leaf":
        return next(it)
    if treedef.kind == "none":
        return None
    if treedef.kind == "dict":
        keys, cls = treedef.aux
        values = [_unflatten(c, it) for c in treedef.children]
        out = dict(zip(keys, values))
        return out if cls is dict else cls(out)
    values = [_unflatten(c, it) for c in treedef.children]
    if treedef.kind == "list":
        return values
    if treedef.kind == "namedtuple":
        return treedef.aux(*values)
    return tuple(values)


def tree_unflatten(treedef: TreeDef, leaves: list[Any]) -> Any:
    it = iter(leaves)
    out = _unflatten(treedef, it)
    return out


def tree_leaves(tree: Any) -> list[torch.Tensor]:
    """Tensor leaves of ``tree``; rejects DP wrappers like the reference."""
    flat, _ = tree_flatten(tree)
    from opake_amd.types import ClippedPytree

    if any(isinstance(leaf, ClippedPytree) for leaf in flat):
        raise InputTypeError(
            "Expected raw tensor pytrees; got a ClippedPytree leaf. "
            "Pass `.pytree` instead."
        )
    return [leaf for leaf in flat if isinstance(leaf, torch.Tensor)]


def tree_map(fn: Callable[..., Any], *trees: Any) -> Any:
    leaves0, treedef = tree_flatten(trees[0])
    others = [tree_flatten(t)[0] for t in trees[1:]]
    for o in others:
        if len(o) != len(leaves0):
            raise InputTypeError("tree_map: trees have different structures")
    return tree_unflatten(treedef, [fn(*xs) for xs in zip(leaves0, *others)])


def param_path(path: Any) -> ParamPath:
    """Normalize a path or a flat string key to a tuple path (reference
    ``pytree.py:51-69``)."""
    if isinstance(path, str):
        return (path,)
    out = []
    for part in path:
        if isinstance(part, (str, int)):
            out.append(part)
        else:
            key = getattr(part, "key", getattr(part, "idx", getattr(part, "name", None)))
            if key is None:
                raise InputTypeError(f"unsupported path entry {part!r}")
            out.append(key)
    return tuple(out)


def param_path_display(path: ParamPath) -> str:
    return ".".join(str(p) for p in path)


__all__ = [
    "ParamPath",
    "TreeDef",
    "param_path",
    "param_path_display",
    "tree_flatten",
    "tree_flatten_with_paths",
    "tree_leaves",
    "tree_map",
    "tree_unflatten",
]
