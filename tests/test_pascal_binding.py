"""CPU checks of pascal/nnhip.pas, the Free Pascal side of the drop-in.

No Free Pascal compiler is installed in this image or on the GPU boxes, so
the unit is checked structurally: every C entry point of
include/tensorium_hip.h has exactly one `external` declaration with the same
parameter count and matching types; every call the unit makes passes that
many arguments; and TNNHip<T> declares every public method of the
reference's TNNCuda<T> (nncuda.pas:100-157) with the same signature."""
import json
import os
import re
import sys

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
from pascal_sig import parse_methods  # noqa: E402

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "tensorium_hip.h")
UNIT = os.path.join(ROOT, "pascal", "nnhip.pas")

# public method signatures of TNNCuda<T>, nncuda.pas:100-157, recorded by
# tests/golden/make_tnncuda_signatures.py
SIGNATURES = os.path.join(ROOT, "tests", "golden", "tnncuda_signatures.json")


def tnncuda_methods():
    return json.load(open(SIGNATURES))["methods"]


C_TO_PAS = {
    "int32_t": "LongInt", "int64_t": "Int64", "float": "Single", "float*": "PSingle", "int64_t*": "PInt64",
    "int32_t*": "PLongInt", "void*": "Pointer", "void**": "PPointer", "float**": "PPSingle",
}


def strip_c_comments(text):
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.sub(r"//[^\n]*", "", text)


def header_decls():
    text = strip_c_comments(open(HEADER).read())
    out = {}
    for m in re.finditer(r"\b(?:int32_t|const\s+char\s*\*)\s*(tnh_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", text):
        name, params = m.group(1), m.group(2).strip()
        types = []
        if params and params != "void":
            for p in params.split(","):
                p = re.sub(r"\bconst\b", "", p)
                p = re.sub(r"[A-Za-z_][A-Za-z0-9_]*\s*$", "", p.strip())  # drop the parameter name
                p = re.sub(r"\s+", "", p)
                types.append(p)
        out[name] = types
    return out


def unit_text():
    text = open(UNIT).read()
    text = re.sub(r"\{[^}]*\}", "", text)  # { } comments
    return re.sub(r"//[^\n]*", "", text)


def pascal_externals():
    text = unit_text()
    out = {}
    pat = r"function\s+(tnh_[a-z0-9_]+)\s*(?:\(([^)]*)\))?\s*:\s*(\w+)\s*;\s*cdecl\s*;\s*external\s+libtnh\s*;"
    for m in re.finditer(pat, text):
        name, params, ret = m.group(1), m.group(2) or "", m.group(3)
        assert name not in out, "declared twice: " + name
        types, names = [], []
        for group in filter(None, (g.strip() for g in params.split(";"))):
            idents, typ = group.rsplit(":", 1)
            for ident in idents.split(","):
                names.append(ident.strip())
                types.append(typ.strip())
        lowered = [n.lower() for n in names]
        assert len(set(lowered)) == len(lowered), "duplicate parameter (Pascal is case-insensitive): " + name
        out[name] = (types, ret)
    return out


def test_every_header_entry_point_has_one_matching_external():
    decls = header_decls()
    ext = pascal_externals()
    assert len(decls) >= 70
    assert sorted(decls) == sorted(ext)
    for name, ctypes_ in decls.items():
        types, ret = ext[name]
        assert ret == ("PAnsiChar" if name == "tnh_last_error" else "LongInt"), name
        assert len(types) == len(ctypes_), name
        for i, (c, p) in enumerate(zip(ctypes_, types)):
            assert C_TO_PAS[c] == p, (name, i, c, p)


def split_args(s):
    depth, cur, out = 0, "", []
    for ch in s:
        if ch == "(":
            depth += 1
        elif ch == ")":
            depth -= 1
        if ch == "," and depth == 0:
            out.append(cur)
            cur = ""
        else:
            cur += ch
    if cur.strip():
        out.append(cur)
    return out


def test_every_call_passes_the_declared_number_of_arguments():
    text = unit_text()
    impl = text[text.index("implementation"):]
    ext = pascal_externals()
    calls = 0
    for m in re.finditer(r"\b(tnh_[a-z0-9_]+)\(", impl):
        start = m.end()
        depth, i = 1, start
        while depth:
            depth += {"(": 1, ")": -1}.get(impl[i], 0)
            i += 1
        args = split_args(impl[start:i - 1])
        assert len(args) == len(ext[m.group(1)][0]), (m.group(1), len(args))
        calls += 1
    assert calls >= 50


def tnnhip_methods():
    text = unit_text()
    return parse_methods(text[text.index("TNNHip<T> = class"):text.index("implementation")])


def test_tnnhip_declares_every_tnncuda_method_with_its_signature():
    """Every public method of TNNCuda<T> is declared in TNNHip<T> with the
    same kind, parameter names, modifiers (const / var), types, defaults and
    order, and the same result type, so `cuda.` -> `hip.` compiles at every
    call site; each is implemented."""
    mine = {m["name"]: m for m in tnnhip_methods()}
    ref = tnncuda_methods()
    assert len(ref) == 53
    for r in ref:
        assert r["name"] in mine, "not declared: " + r["name"]
        m = mine[r["name"]]
        assert m["kind"] == r["kind"], (r["name"], m["kind"], r["kind"])
        assert m["result"] == r["result"], (r["name"], m["result"], r["result"])
        assert len(m["params"]) == len(r["params"]), (r["name"], m["params"], r["params"])
        for i, (a, b) in enumerate(zip(m["params"], r["params"])):
            assert a == b, (r["name"], i, a, b)
    text = unit_text()
    impl = text[text.index("implementation"):]
    for name in mine:
        assert re.search(r"TNNHip<T>\.%s\b" % name, impl), "no implementation: " + name


def test_signature_parser_catches_a_changed_parameter():
    """The comparison above sees a parameter added, renamed or retyped."""
    base = "procedure backwardMaxPool(const aBatch, outC: SizeInt; output: TCUMem; const indexes: TCUMem);"
    ref = parse_methods(base)[0]
    for variant in (base.replace("const indexes", "indexes"),
                    base.replace("outC", "outChannels"),
                    base.replace("output: TCUMem", "output: PSingle"),
                    base.replace(");", "; const h: SizeInt);")):
        assert parse_methods(variant)[0]["params"] != ref["params"], variant
    assert ref["params"][0] == ["const", "abatch", "sizeint", ""]


def test_unit_is_complete_text():
    raw = open(UNIT).read()
    assert "…" not in raw and "..." not in raw
    assert raw.rstrip().endswith("end.")


PLAN_UNIT = os.path.join(ROOT, "pascal", "nnhipnet.pas")


def test_plan_unit_calls_tnnhip_methods_with_their_arity():
    """pascal/nnhipnet.pas (the channels-last TNNet forward) calls only
    methods TNNHip<T> declares, each with at least its parameters without a
    default and at most all of them."""
    mine = {}
    for m in tnnhip_methods():
        mine.setdefault(m["name"].lower(), []).append(m)
    text = strip_comments_pas(open(PLAN_UNIT).read())
    impl = text[text.index("implementation"):]
    calls = 0
    for m in re.finditer(r"\bhip\.(\w+)\s*\(", impl):
        start = m.end()
        depth, i = 1, start
        while depth:
            depth += {"(": 1, ")": -1}.get(impl[i], 0)
            i += 1
        n = len(split_args(impl[start:i - 1]))
        decls = mine.get(m.group(1).lower())
        assert decls, "TNNHip has no method " + m.group(1)
        assert any(sum(1 for p in d["params"] if not p[3]) <= n <= len(d["params"]) for d in decls), \
            (m.group(1), n)
        calls += 1
    assert calls >= 12
    for name in ("createDeviceBuffer", "freeDeviceBuffer"):
        assert re.search(r"\bhip\.%s\b" % name, impl), name
    assert text.rstrip().endswith("end.")


def strip_comments_pas(text):
    text = re.sub(r"\{[^}]*\}", "", text)
    return re.sub(r"//[^\n]*", "", text)
