"""Writes superl8_names.json: every name the reference's paged-KV path looks
up on the external ``superl8`` package, with the file:line of each use.

    python tests/golden/make_superl8_names.py

Run in the container that holds the reference checkout (default
/root/reference, or the path given as the first argument).  The reference's
files are parsed as text (``ast``), never imported or executed.  A use is an
attribute chain rooted at the name ``superl8`` (``superl8.quantize_i8_rowwise``,
``superl8.quant.rotation.rotate_last``), a name imported ``from superl8...``,
or a ``getattr(superl8, "name", ...)`` probe.
"""

from __future__ import annotations

import ast
import json
import sys
from pathlib import Path

OUT = Path(__file__).resolve().parent / "superl8_names.json"

# The reference files on the quantized paged-KV path (the cache, the
# attention layers that call it, the graph capture, the pipeline's rotation
# patch) and the reference's own tests of that path.
FILES = (
    "superl8serve/engine/kv_cache.py",
    "superl8serve/layers/gqa_attention.py",
    "superl8serve/layers/gated_gqa_attention.py",
    "superl8serve/engine/cuda_graph.py",
    "superl8serve/dist/pipeline.py",
    "tests/test_k8v3_cache.py",
    "tests/test_kv_eviction.py",
    "tests/test_paged_engine.py",
    "tests/test_prefix_cache.py",
    "tests/test_decode_staging.py",
)


def _chain(node: ast.AST) -> list[str] | None:
    parts = []
    while isinstance(node, ast.Attribute):
        parts.append(node.attr)
        node = node.value
    if isinstance(node, ast.Name) and node.id == "superl8":
        return ["superl8", *reversed(parts)]
    return None


def collect(root: Path) -> dict[str, list[str]]:
    uses: dict[str, set[str]] = {}

    def add(name: str, where: str) -> None:
        uses.setdefault(name, set()).add(where)

    for rel in FILES:
        tree = ast.parse((root / rel).read_text(), filename=rel)
        short = rel.split("/", 1)[1]
        # attribute chains: record only maximal chains (superl8.a.b, not also superl8.a)
        inner: set[int] = set()
        for node in ast.walk(tree):
            if isinstance(node, ast.Attribute) and isinstance(node.value, ast.Attribute):
                inner.add(id(node.value))
        for node in ast.walk(tree):
            if isinstance(node, ast.Attribute) and id(node) not in inner:
                ch = _chain(node)
                if ch:
                    add(".".join(ch), f"{short}:{node.lineno}")
            elif isinstance(node, ast.ImportFrom) and node.module and node.module.split(".")[0] == "superl8":
                for alias in node.names:
                    add(f"{node.module}.{alias.name}", f"{short}:{node.lineno}")
            elif (isinstance(node, ast.Call) and isinstance(node.func, ast.Name) and node.func.id == "getattr"
                  and len(node.args) >= 2 and isinstance(node.args[0], ast.Name) and node.args[0].id == "superl8"
                  and isinstance(node.args[1], ast.Constant) and isinstance(node.args[1].value, str)):
                add(f"superl8.{node.args[1].value}", f"{short}:{node.lineno}")
    return {k: sorted(v, key=lambda s: (s.split(":")[0], int(s.split(":")[1]))) for k, v in sorted(uses.items())}


def main() -> None:
    root = Path(sys.argv[1]) if len(sys.argv) > 1 else Path("/root/reference")
    names = collect(root)
    OUT.write_text(json.dumps({"files": list(FILES), "names": names}, indent=1) + "\n")
    print(f"wrote {OUT} ({len(names)} names)")


if __name__ == "__main__":
    main()
