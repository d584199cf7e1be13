"""Writes kernel_fingerprints.json: for every registered kernel signature, the body
fingerprints (pyasc_amd.fingerprint) of the reference's kernels with that signature.

    python -m pyasc_amd.make_fingerprints [/root/reference]

The reference's test and tutorial files are read as text and parsed with ``ast``;
nothing of them is imported or executed, and only the fingerprints (hashes) and the
file:line of each kernel are written.  A signature the reference does not define (a
build-defined kernel) gets an empty list: it accepts declaration bodies only.
"""
from __future__ import annotations

import ast
import json
import os
import sys

from . import registry
from .fingerprint import FINGERPRINTS_FILE, body_fingerprint, signature_key

SEARCH_DIRS = ("python/test", "python/tutorials")
DECORATORS = ("asc.jit", "asc2.jit")


def scan(reference_root: str):
    """(signature key, fingerprint, 'file:line') of every jit kernel under SEARCH_DIRS."""
    for sub in SEARCH_DIRS:
        for dirpath, _, files in os.walk(os.path.join(reference_root, sub)):
            for fname in sorted(files):
                if not fname.endswith(".py"):
                    continue
                path = os.path.join(dirpath, fname)
                with open(path, encoding="utf-8") as f:
                    tree = ast.parse(f.read())
                for node in ast.walk(tree):
                    if not isinstance(node, ast.FunctionDef):
                        continue
                    if not any(ast.unparse(d).startswith(DECORATORS) for d in node.decorator_list):
                        continue
                    params = tuple(a.arg for a in node.args.args)
                    yield (signature_key(node.name, params), body_fingerprint(node),
                           f"{os.path.relpath(path, reference_root)}:{node.lineno}")


def main(argv) -> int:
    root = argv[1] if len(argv) > 1 else "/root/reference"
    wanted = {signature_key(n, p) for n, p in registry.entries()}
    table = {key: [] for key in sorted(wanted)}
    for key, fp, where in scan(root):
        if key in table and all(item["fingerprint"] != fp for item in table[key]):
            table[key].append({"fingerprint": fp, "source": where})
    out = {"format": "sha256 of the normalised body AST, first 16 hex digits (pyasc_amd/fingerprint.py)",
           "python": f"{sys.version_info.major}.{sys.version_info.minor}",
           "kernels": table}
    with open(FINGERPRINTS_FILE, "w") as f:
        json.dump(out, f, indent=1, sort_keys=True)
        f.write("\n")
    missing = [k for k, v in table.items() if not v]
    print(f"wrote {FINGERPRINTS_FILE}: {len(table)} signatures, {len(missing)} build-defined (declaration only)")
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv))
