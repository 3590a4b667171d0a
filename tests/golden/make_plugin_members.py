"""Writes tests/golden/plugin_members.json: the members the reference's three
attention-plugin classes define, each with the line that defines it.

It reads vllm_gr/v1/attention/backends/beam_attn.py as text with ``ast``
(nothing of the reference is imported or run) and lists, for
``BeamAttentionBackend``, ``BeamAttentionImpl`` and
``BeamAttentionMetadataBuilder``:

* class attributes and methods whose names do not start with ``_``, plus
  ``_cudagraph_support`` (vLLM reads it from the builder class);
* attributes ``__init__`` assigns on ``self`` (instance members), public only.

    python tests/golden/make_plugin_members.py [/root/reference]
"""

from __future__ import annotations

import ast
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REL = "vllm_gr/v1/attention/backends/beam_attn.py"
CLASSES = ("BeamAttentionBackend", "BeamAttentionImpl", "BeamAttentionMetadataBuilder")
KEEP_PRIVATE = {"_cudagraph_support"}


def _public(name: str) -> bool:
    return not name.startswith("_") or name in KEEP_PRIVATE


def members(src: str) -> dict:
    tree = ast.parse(src)
    out = {}
    for node in tree.body:
        if not isinstance(node, ast.ClassDef) or node.name not in CLASSES:
            continue
        cls, inst = {}, {}
        for item in node.body:
            if isinstance(item, (ast.FunctionDef, ast.AsyncFunctionDef)):
                if _public(item.name):
                    cls[item.name] = item.lineno
                if item.name == "__init__":
                    for sub in ast.walk(item):
                        targets = sub.targets if isinstance(sub, ast.Assign) else (
                            [sub.target] if isinstance(sub, ast.AnnAssign) else [])
                        for t in targets:
                            if (isinstance(t, ast.Attribute) and isinstance(t.value, ast.Name)
                                    and t.value.id == "self" and _public(t.attr)):
                                inst.setdefault(t.attr, sub.lineno)
            elif isinstance(item, ast.Assign):
                for t in item.targets:
                    if isinstance(t, ast.Name) and _public(t.id):
                        cls[t.id] = item.lineno
            elif isinstance(item, ast.AnnAssign) and isinstance(item.target, ast.Name):
                if _public(item.target.id):
                    cls[item.target.id] = item.lineno
        out[node.name] = {"class": dict(sorted(cls.items())), "instance": dict(sorted(inst.items()))}
    return out


def main() -> None:
    ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    with open(os.path.join(ref, REL)) as f:
        data = {"source": REL, "classes": members(f.read())}
    with open(os.path.join(HERE, "plugin_members.json"), "w") as f:
        json.dump(data, f, indent=1, sort_keys=True)
        f.write("\n")


if __name__ == "__main__":
    main()
