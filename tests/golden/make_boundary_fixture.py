"""Write the call sites of the reference's EasyFHE boundary as data.

Runs in the build container only (it reads the reference tree at
/root/reference as text; nothing is imported or run from it).  Every
``.py`` file under llama3fhe/ is parsed; each import of ``easyfhe`` (``import
easyfhe``, ``import easyfhe as torch``, ``import easyfhe.bs.openfhe as bs``,
``from easyfhe import fhe``) binds an alias to a module path, and every call
``alias.name(...)`` or ``alias.sub.name(...)`` is recorded with its module,
name, positional-argument count, keyword names and whether it passes
``*args`` / ``**kwargs``; so is every call through an object's ``fhe``
attribute (``crypto_context.fhe.homo_rotate(...)``: the backend's handle on
``easyfhe.fhe``, llama3fhe/backend.py:177-313), as a call of
``easyfhe.fhe``.  Attribute reads that are not calls (``fhe.Cipher``
in annotations, ``torch.float64``) are recorded as names that must exist.

The output ``boundary_calls.json`` is the fixture of
tests/test_boundary_conformance.py.

    python tests/golden/make_boundary_fixture.py
"""

from __future__ import annotations

import ast
import json
from pathlib import Path

REF = Path("/root/reference/llama3fhe")
OUT = Path(__file__).resolve().parent / "boundary_calls.json"


def _aliases(tree: ast.Module) -> dict[str, str]:
    out: dict[str, str] = {}
    for node in ast.walk(tree):
        if isinstance(node, ast.Import):
            for a in node.names:
                if a.name == "easyfhe" or a.name.startswith("easyfhe."):
                    if a.asname:
                        out[a.asname] = a.name
                    else:
                        out["easyfhe"] = "easyfhe"
        elif isinstance(node, ast.ImportFrom) and node.module and (
                node.module == "easyfhe" or node.module.startswith("easyfhe.")):
            for a in node.names:
                out[a.asname or a.name] = f"{node.module}.{a.name}"
    return out


def _chain(node: ast.AST) -> list[str] | None:
    parts = []
    while isinstance(node, ast.Attribute):
        parts.append(node.attr)
        node = node.value
    if isinstance(node, ast.Name):
        parts.append(node.id)
        return parts[::-1]
    return None


def main() -> None:
    calls: dict[tuple, dict] = {}
    names: dict[str, list[str]] = {}
    for path in sorted(REF.rglob("*.py")):
        rel = str(path.relative_to(REF.parent))
        tree = ast.parse(path.read_text(encoding="utf-8"))
        al = _aliases(tree)
        call_funcs = set()
        for node in ast.walk(tree):
            if not isinstance(node, ast.Call):
                continue
            ch = _chain(node.func)
            if not ch or len(ch) < 2:
                continue
            if ch[0] in al:
                target = al[ch[0]].split(".") + ch[1:]
            elif ch[-2] == "fhe":
                target = ["easyfhe", "fhe", ch[-1]]
            else:
                continue
            call_funcs.add(id(node.func))
            module, name = ".".join(target[:-1]), target[-1]
            star = any(isinstance(a, ast.Starred) for a in node.args) or any(
                k.arg is None for k in node.keywords)
            npos = sum(1 for a in node.args if not isinstance(a, ast.Starred))
            kw = tuple(sorted(k.arg for k in node.keywords if k.arg is not None))
            key = (module, name, npos, kw, star)
            rec = calls.setdefault(key, {"module": module, "name": name, "positional": npos,
                                         "keywords": list(kw), "star": star, "sites": []})
            rec["sites"].append(f"{rel}:{node.lineno}")
        for node in ast.walk(tree):
            if isinstance(node, ast.Attribute) and id(node) not in call_funcs:
                ch = _chain(node)
                if ch and len(ch) >= 2 and ch[0] in al:
                    target = al[ch[0]].split(".") + ch[1:]
                    names.setdefault(".".join(target), []).append(f"{rel}:{node.lineno}")
    data = {
        "calls": sorted(calls.values(), key=lambda r: (r["module"], r["name"], r["positional"],
                                                       r["keywords"])),
        "names": {k: sorted(set(v))[:4] for k, v in sorted(names.items())},
    }
    OUT.write_text(json.dumps(data, indent=1) + "\n", encoding="utf-8")
    print(f"wrote {OUT}: {len(data['calls'])} call shapes, {len(data['names'])} attribute names")


if __name__ == "__main__":
    main()
