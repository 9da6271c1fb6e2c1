"""Parser of Free Pascal method declarations, shared by the signature test of
pascal/nnhip.pas and the script that records TNNCuda's signatures.

parse_methods(text) returns, in order, one entry per procedure / function /
constructor / destructor declaration:
  {"kind": "procedure" | "function" | "class function" | "constructor" |
           "destructor",
   "name": str,
   "params": [[modifier, name, type, default], ...]   (lowercased, spaces
            removed; modifier "" | "const" | "var" | "out" | "constref"),
   "result": type or ""}
Comments ({ }, (* *), //) are removed first."""
import re

_DECL = re.compile(r"\b(class\s+function|class\s+procedure|procedure|function|constructor|destructor)\s+(\w+)\s*",
                   re.I)


def strip_comments(text):
    text = re.sub(r"\{[^}]*\}", "", text)
    text = re.sub(r"\(\*.*?\*\)", "", text, flags=re.S)
    return re.sub(r"//[^\n]*", "", text)


def _norm(s):
    return re.sub(r"\s+", "", s).lower()


def _params(body):
    out = []
    depth, cur, groups = 0, "", []
    for ch in body:  # split on ';' outside brackets (TArray<...> has none, defaults may)
        if ch in "(<[":
            depth += 1
        elif ch in ")>]":
            depth -= 1
        if ch == ";" and depth == 0:
            groups.append(cur)
            cur = ""
        else:
            cur += ch
    if cur.strip():
        groups.append(cur)
    for g in groups:
        g = g.strip()
        mod = ""
        m = re.match(r"(const|var|out|constref)\s+", g, re.I)
        if m:
            mod, g = m.group(1).lower(), g[m.end():]
        names, rest = g.split(":", 1)
        typ, default = (rest.split("=", 1) + [""])[:2]
        for n in names.split(","):
            out.append([mod, _norm(n).lstrip("&"), _norm(typ), _norm(default)])
    return out


def parse_methods(text):
    text = strip_comments(text)
    out = []
    for m in _DECL.finditer(text):
        kind = re.sub(r"\s+", " ", m.group(1).lower())
        name = m.group(2)
        i = m.end()
        params = []
        if i < len(text) and text[i] == "(":
            depth, j = 1, i + 1
            while depth:
                depth += {"(": 1, ")": -1}.get(text[j], 0)
                j += 1
            params = _params(text[i + 1:j - 1])
            i = j
        rest = text[i:text.index(";", i)]
        result = _norm(rest.split(":", 1)[1]) if ":" in rest else ""
        out.append({"kind": kind, "name": name, "params": params, "result": result})
    return out
