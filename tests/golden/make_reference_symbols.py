"""Write reference_symbols.json: every function, macro, structure function,
condition, variable and CFFI Lisp name llambda's sources define, read from
the reference checkout (default /root/reference, or the first argument).

tests/test_integration_lisp.py checks the Lisp that INTEGRATION.md asks a
maintainer to add against this list: each name the adapter calls must be
defined there or by the reference.  Run it again when the reference moves:

    python tests/golden/make_reference_symbols.py [/path/to/llambda]
"""
import glob
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))

from lisp_forms import defined_names, read_all  # noqa: E402

# the files the llambda system loads, in its order (llambda.asd:8-22)
SOURCES = ["package.lisp", "accelerator.lisp", "architecture.lisp", "llambda.lisp",
           "accelerators/*.lisp", "architectures/*.lisp"]


def main() -> None:
    root = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    files, names = [], set()
    for pattern in SOURCES:
        for path in sorted(glob.glob(os.path.join(root, pattern))):
            with open(path, encoding="utf-8") as f:
                names |= defined_names(read_all(f.read()))
            files.append(os.path.relpath(path, root))
    out = {"sources": files, "names": sorted(names)}
    with open(os.path.join(HERE, "reference_symbols.json"), "w") as f:
        json.dump(out, f, indent=0)
        f.write("\n")
    print(f"{len(names)} names from {len(files)} files")


if __name__ == "__main__":
    main()
