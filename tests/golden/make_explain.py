"""Writes tests/golden/explain/*.txt: the kernel texts the reference's
`presk explain` documents print (section 9, "The kernels and the host"),
from its own snapshot files
crates/presk-explain/tests/snapshots/documents__{layernorm,mlp,tutorial,
tutorial-typed,tutorial-opt,minigpt}.snap -- data: the reference's lowering
of those programs under their plans, each kernel with its `// kN:` header
(sites and launch counts).  Run in the build container only (it reads
/root/reference).

    python tests/golden/make_explain.py
"""
import os
import re

REF = os.environ.get("PRESK_REF", "/root/reference")
SNAPS = os.path.join(REF, "crates", "presk-explain", "tests", "snapshots")
HERE = os.path.dirname(os.path.abspath(__file__))
DOCS = ["layernorm", "mlp", "tutorial", "tutorial-typed", "tutorial-opt", "minigpt"]


def kernel_blocks(text):
    """The `// kN` headers and kernel texts inside the document's text blocks."""
    out, cur, inb = [], None, False
    for line in text.split("\n"):
        if line.startswith("```"):
            inb = line == "```text"
            continue
        if not inb:
            continue
        if re.match(r"^// k\d+:", line):
            cur = [line]
        elif cur is not None:
            cur.append(line)
            if line == "}":
                out.append("\n".join(cur))
                cur = None
    return out


def main():
    os.makedirs(os.path.join(HERE, "explain"), exist_ok=True)
    for d in DOCS:
        with open(os.path.join(SNAPS, f"documents__{d}.snap")) as f:
            blocks = kernel_blocks(f.read())
        with open(os.path.join(HERE, "explain", f"{d}.txt"), "w") as f:
            f.write("\n".join(blocks) + "\n")
        print(d, len(blocks))


if __name__ == "__main__":
    main()
