"""CPU check of the Swift wrapper (swift/Sources/FlashVSRLCSA/FlashVSRLCSA.swift) against the C ABI it binds.

No Swift toolchain is in this image, so the wrapper is never compiled here. What can be checked without one: every
C function the wrapper calls is declared in include/fvsr_lcsa.h and listed in the Python binding's signature table,
and every call passes as many arguments as the prototype has parameters.
"""
import os
import re

from fvsr_lcsa import _abi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "fvsr_lcsa.h")
SWIFT = os.path.join(ROOT, "swift", "Sources", "FlashVSRLCSA", "FlashVSRLCSA.swift")


def _split_args(text: str) -> list:
    """Top-level comma split of an argument list (parentheses, brackets and braces balanced)."""
    out, depth, cur = [], 0, ""
    for ch in text:
        if ch in "([{":
            depth += 1
        elif ch in ")]}":
            depth -= 1
        if ch == "," and depth == 0:
            out.append(cur)
            cur = ""
        else:
            cur += ch
    if cur.strip():
        out.append(cur)
    return [a.strip() for a in out]


def _balanced(text: str, start: int) -> str:
    """The text between the parenthesis at `start` and its match."""
    depth = 0
    for i in range(start, len(text)):
        if text[i] == "(":
            depth += 1
        elif text[i] == ")":
            depth -= 1
            if depth == 0:
                return text[start + 1:i]
    raise ValueError("unbalanced parentheses")


def header_prototypes() -> dict:
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    protos = {}
    for m in re.finditer(r"^\s*(?:const\s+)?\w+\*?\s+\*?(fvsr_\w+)\(", text, flags=re.M):
        args = _balanced(text, m.end() - 1)
        params = [] if args.strip() in ("", "void") else _split_args(args)
        protos[m.group(1)] = len(params)
    return protos


def header_types() -> set:
    """Type names the header declares (enums and structs the wrapper constructs, e.g. fvsr_attn_mode(rawValue:))."""
    text = open(HEADER).read()
    return (set(re.findall(r"typedef\s+(?:enum|struct)\s+(fvsr_\w+)", text)) |
            set(re.findall(r"}\s*(fvsr_\w+)\s*;", text)))


def swift_calls() -> list:
    """(C function, argument count) of every call of a C function in the wrapper (constructions of the header's
    types left out)."""
    text = open(SWIFT).read()
    text = "\n".join(line.split("//")[0] for line in text.splitlines())   # drop comments
    types = header_types()
    calls = []
    for m in re.finditer(r"\b(fvsr_\w+)\(", text):
        if m.group(1) not in types:
            calls.append((m.group(1), len(_split_args(_balanced(text, m.end() - 1)))))
    return calls


def test_every_wrapper_call_is_declared_and_bound():
    protos = header_prototypes()
    calls = swift_calls()
    assert len(calls) >= 20
    for name, _ in calls:
        assert name in protos, f"{name} is called by the Swift wrapper but not declared in include/fvsr_lcsa.h"
        assert name in _abi.SIGNATURES, f"{name} is not in the binding's signature table"


def test_every_wrapper_call_passes_the_prototype_arity():
    protos = header_prototypes()
    for name, n in swift_calls():
        assert n == protos[name], f"{name}: the Swift wrapper passes {n} arguments, the prototype has {protos[name]}"


def test_signature_table_matches_prototype_arity():
    protos = header_prototypes()
    for name, n in protos.items():
        argtypes = _abi.SIGNATURES[name][1]
        assert len(argtypes) == n, f"{name}: signature table has {len(argtypes)} arguments, the prototype {n}"


def test_every_constant_the_wrapper_names_is_declared():
    """The enumerators the wrapper passes (FVSR_DTYPE_*, FVSR_ATTN_*, FVSR_LAYOUT_*) exist in the header, so the
    imported Clang module provides them."""
    header = open(HEADER).read()
    declared = set(re.findall(r"\b(FVSR_[A-Z0-9_]+)\s*=", header)) | set(re.findall(r"#define\s+(FVSR_[A-Z0-9_]+)", header))
    text = "\n".join(line.split("//")[0] for line in open(SWIFT).read().splitlines())
    used = set(re.findall(r"\b(FVSR_[A-Z0-9_]+)\b", text))
    assert used, "the wrapper names no FVSR_ constant"
    assert used <= declared, f"not declared in include/fvsr_lcsa.h: {sorted(used - declared)}"

