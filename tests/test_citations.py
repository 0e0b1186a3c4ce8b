"""Every citation of a reference file as <path>:<line>[-<line>][, <line>...] in the boundary and
kernel sources and in the design documents points inside the cited file.

Line counts come from tests/golden/reference_lines.json (written by make_reference_lines.py next to
it), so this runs without the reference.  Paths are relative to the engine's folder
(h2-own-inference-engine/) or start with "./" for the reference's root, as the citations are
written; a bare file name (kernels.c) is resolved when exactly one reference file has that name."""
import json
import os
import re

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LINES = json.load(open(os.path.join(REPO, "tests", "golden", "reference_lines.json")))
PKG = "e2e-browser-voice-agent_amd"
SOURCES = ["include", f"{PKG}/engine", f"{PKG}/node", f"{PKG}/csrc", f"{PKG}/py", "oracle", "tests",
           "bench.py", "__graft_entry__.py", "DESIGN.md", "INTEGRATION.md"]
SKIP_DIRS = {"golden", "__pycache__", "lib"}

CITE = re.compile(r"(?<![\w/.-])((?:\./)?(?:[\w.-]+/)*[\w.-]+\.(?:js|c|py|md|html|json)):"
                  r"(\d+(?:-\d+)?(?:,\s?\d+(?:-\d+)?)*)")


def _files():
    for s in SOURCES:
        p = os.path.join(REPO, s)
        if os.path.isfile(p):
            yield p
            continue
        for base, dirs, files in os.walk(p):
            dirs[:] = [d for d in dirs if d not in SKIP_DIRS]
            for f in files:
                if f.endswith((".h", ".hip", ".c", ".js", ".py", ".md")) and f != os.path.basename(__file__):
                    yield os.path.join(base, f)


def _resolve(path):
    """The reference file a cited path names, or None when it names none (a file of this repo)."""
    if path.startswith("h2-own-inference-engine/"):
        path = path[len("h2-own-inference-engine/"):]
    if path in LINES:
        return path
    hits = [k for k in LINES if k.endswith("/" + path)]
    return hits[0] if len(hits) == 1 else None


def citations():
    out = []
    for f in _files():
        text = open(f, encoding="utf-8", errors="replace").read()
        for m in CITE.finditer(text):
            ref = _resolve(m.group(1))
            if ref is None:
                continue
            line = text.count("\n", 0, m.start()) + 1
            for part in re.split(r",\s?", m.group(2)):
                a, _, b = part.partition("-")
                out.append((os.path.relpath(f, REPO), line, m.group(0), ref, int(a), int(b or a)))
    return out


def test_fixture_has_the_engine_files():
    for f in ["engine/kernels.c", "engine/cpu.js", "engine/cpu-worker.js", "engine/llm.js", "engine/gguf.js"]:
        assert LINES[f] > 50


def test_citations_found():
    assert len(citations()) > 40


def test_every_citation_lies_inside_its_file():
    bad = [f"{src}:{line}: {text} (file has {LINES[ref]} lines)"
           for src, line, text, ref, a, b in citations() if not (1 <= a <= b <= LINES[ref])]
    assert not bad, "\n".join(bad)


@pytest.mark.parametrize("text,ok", [("engine/cpu.js:17-69", True), ("engine/cpu.js:199-250", False),
                                     ("kernels.c:496", True), ("kernels.c:497", False),
                                     ("engine/llm.js:23-29, 140", False)])
def test_checker_flags_lines_past_the_end(text, ok):
    m = CITE.search(text)
    ref = _resolve(m.group(1))
    parts = [p.partition("-") for p in re.split(r",\s?", m.group(2))]
    assert all(1 <= int(a) <= int(b or a) <= LINES[ref] for a, _, b in parts) == ok
