"""Write reference_lines.json: the line count of every text file of the reference that the sources
here cite as <path>:<line>.  Paths are relative to h2-own-inference-engine/ (the engine's folder);
files outside it carry a leading "./" (relative to the reference's root), as the citations do.

Run in a container that has the reference at /root/reference:
    python tests/golden/make_reference_lines.py
The JSON is the fixture tests/test_citations.py reads (the reference itself is not needed there)."""
import json
import os

ROOT = "/root/reference"
ENGINE = os.path.join(ROOT, "h2-own-inference-engine")
EXTS = (".js", ".c", ".py", ".md", ".html", ".json", ".txt")


def main():
    out = {}
    for base, dirs, files in os.walk(ROOT):
        dirs[:] = sorted(d for d in dirs if not d.startswith("."))
        for f in sorted(files):
            if not f.endswith(EXTS):
                continue
            p = os.path.join(base, f)
            with open(p, "rb") as fh:
                data = fh.read()
            n = data.count(b"\n") + (0 if data.endswith(b"\n") or not data else 1)
            rel = os.path.relpath(p, ENGINE) if p.startswith(ENGINE + os.sep) else "./" + os.path.relpath(p, ROOT)
            out[rel] = n
    dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), "reference_lines.json")
    with open(dst, "w") as fh:
        json.dump(out, fh, indent=1, sort_keys=True)
        fh.write("\n")
    print(dst, len(out), "files")


if __name__ == "__main__":
    main()
