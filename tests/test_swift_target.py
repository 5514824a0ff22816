"""The Swift C target (swift/): its module map exposes the C ABI header and links the
library, and the Linux operator layer calls only entry points the header declares, each with
the header's number of arguments.  This image has no Swift toolchain, so these are text
checks; `swift build` in swift/ compile-checks the same files where Swift is installed."""
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mingtts_hip.h")
SWIFT = os.path.join(ROOT, "swift", "Sources", "MingTTSHIP", "KernelsHIP.swift")
MODULEMAP = os.path.join(ROOT, "swift", "Sources", "CMingHIP", "module.modulemap")
SHIM = os.path.join(ROOT, "swift", "Sources", "CMingHIP", "shim.h")

# The reference's Encoder methods on the path and their argument labels (Kernels.swift:132-283);
# "_" is an unlabelled argument.
ENCODER_METHODS = {
    "linear": ["_", "rows", "_", "_", "flags", "gate"],
    "rmsnorm": ["_", "rows", "width", "weight", "_", "eps"],
    "ropeCache": ["_", "rows", "heads", "kvHeads", "pos0", "cache", "invFreq"],
    "attention": ["_", "rows", "heads", "kvHeads", "pos0", "window", "cache", "_"],
    "ditAttention": ["_", "batch", "seq", "heads", "invFreq", "_"],
    "flowAssemble": ["y", "history", "cemb", "condBias", "temb", "xEmbedder", "_"],
    "flowEuler": ["y", "pred", "predRow", "nullRow", "latentDim", "cfg", "dt", "capture"],
    "upsample4": ["prev", "cur", "next", "hidden", "_"],
    "istftFrames": ["spec", "count", "nfft", "cosTable", "window", "frames", "frame0", "ring"],
    "istftEmit": ["frames", "window", "nfft", "hop", "s0", "count", "lastFrame", "ring", "_"],
}


def _split_top(args: str) -> list[str]:
    out, depth, cur = [], 0, ""
    for ch in args:
        if ch in "([{":
            depth += 1
        elif ch in ")]}":
            depth -= 1
        if ch == "," and depth == 0:
            out.append(cur.strip())
            cur = ""
        else:
            cur += ch
    if cur.strip():
        out.append(cur.strip())
    return out


def _balanced(text: str, start: int) -> str:
    """The text inside the parentheses opening at text[start]."""
    depth = 0
    for i in range(start, len(text)):
        if text[i] == "(":
            depth += 1
        elif text[i] == ")":
            depth -= 1
            if depth == 0:
                return text[start + 1:i]
    raise AssertionError("unbalanced parentheses")


def header_arity() -> dict[str, int]:
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    out = {}
    for m in re.finditer(r"\b(mt_\w+)\s*\(", text):
        before = text[:m.start()].rstrip()
        if not re.search(r"(int|void|uint64_t|char)\s*\**$", before):
            continue  # a call or a macro, not a declaration
        params = _balanced(text, m.end() - 1)
        n = 0 if params.strip() in ("", "void") else len(_split_top(params))
        out[m.group(1)] = n
    return out


def swift_calls() -> list[tuple[str, int]]:
    text = open(SWIFT).read()
    calls = []
    for m in re.finditer(r"\b(mt_\w+)\(", text):
        if m.group(1) == "mt_gemv_params":
            continue
        calls.append((m.group(1), len(_split_top(_balanced(text, m.end() - 1)))))
    return calls


def test_module_map_exposes_the_header_and_links_the_library():
    mm = open(MODULEMAP).read()
    assert re.search(r'module\s+CMingHIP\s+\[system\]', mm)
    assert 'header "shim.h"' in mm and 'link "mingtts_hip"' in mm
    assert "#include <mingtts_hip.h>" in open(SHIM).read()


def test_swift_calls_match_the_header():
    decl = header_arity()
    assert "mt_linear" in decl and decl["mt_linear"] == 9
    calls = swift_calls()
    assert len(calls) >= 12
    for name, n in calls:
        assert name in decl, f"{name} is not declared in include/mingtts_hip.h"
        assert n == decl[name], f"{name}: {n} arguments in the Swift call, {decl[name]} in the header"


@pytest.mark.parametrize("method", sorted(ENCODER_METHODS))
def test_swift_encoder_keeps_the_reference_labels(method):
    text = open(SWIFT).read()
    m = re.search(r"func " + method + r"\(", text)
    assert m, f"Encoder.{method} missing"
    params = _split_top(_balanced(text, m.end() - 1))
    labels = [p.split(":")[0].split()[0] for p in params]
    assert labels == ENCODER_METHODS[method]
