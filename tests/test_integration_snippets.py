"""The code that INTEGRATION.md shows a maintainer, checked against include/vsmp.h (CPU only):
- every ```c block compiles as C11 against the header (gcc -Werror), so a call with a wrong
  argument count or type fails here;
- every ctypes signature the ```python blocks set (`lib.fn.argtypes = [...]`, `.restype`) names a
  declared entry point and has its parameter count and kinds (pointer, int, long long, unsigned long
  long, float, double).
The CMake blocks are tested by tests/test_swap_build.py."""
import ast
import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
DOC = ROOT / "INTEGRATION.md"
HEADER = ROOT / "include" / "vsmp.h"


def blocks(lang):
    return re.findall(r"```" + lang + r"\n(.*?)```", DOC.read_text(), re.S)


def c_kind(decl):
    """Kind of one C parameter or return type: ptr, int, longlong, ulonglong, float, double, void."""
    d = re.sub(r"/\*.*?\*/", "", decl).strip()
    if "*" in d:
        return "ptr"
    words = [w for w in re.findall(r"[A-Za-z_]\w*", d) if w not in ("const", "VSMP_API")]
    if not words:
        return "void"
    # drop the parameter's name (the last word, when more than the type's words are left)
    types = {"void", "int", "long", "unsigned", "float", "double", "char", "size_t"}
    if len(words) > 1 and words[-1] not in types:
        words = words[:-1]
    t = " ".join(words)
    return {"void": "void", "int": "int", "long long": "longlong", "unsigned long long": "ulonglong", "float": "float",
            "double": "double", "size_t": "size_t"}[t]


def declarations():
    """name -> (return kind, [parameter kinds]) of every VSMP_API function in the header."""
    src = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    out = {}
    for ret, name, params in re.findall(r"VSMP_API\s+([\w\s\*]+?)\s*\b(vsmp_\w+)\s*\(([^)]*)\)\s*;", src, re.S):
        ps = [p for p in (x.strip() for x in params.split(",")) if p]
        kinds = [] if ps == ["void"] else [c_kind(p) for p in ps]
        out[name] = (c_kind(ret), kinds)
    return out


CTYPES_KIND = {"c_void_p": "ptr", "c_char_p": "ptr", "c_int": "int", "c_longlong": "longlong",
               "c_ulonglong": "ulonglong", "c_float": "float", "c_double": "double"}


def py_kind(node, aliases):
    """Kind of one ctypes type expression of a snippet (`_P`, `ctypes.c_int`, `ctypes.POINTER(X)`)."""
    if isinstance(node, ast.Constant) and node.value is None:
        return "void"
    if isinstance(node, ast.Name):
        if node.id in aliases:
            return aliases[node.id]
        return "ptr" if node.id.endswith("Structure") else CTYPES_KIND[node.id]
    if isinstance(node, ast.Attribute):
        return CTYPES_KIND[node.attr]
    if isinstance(node, ast.Call) and isinstance(node.func, ast.Attribute) and node.func.attr == "POINTER":
        return "ptr"
    raise AssertionError(f"unexpected ctypes expression {ast.dump(node)}")


def ctypes_signatures():
    """(function, 'argtypes'|'restype', kinds) for every assignment the python blocks make."""
    found = []
    for code in blocks("python"):
        tree = ast.parse(code)
        aliases = {}
        for st in ast.walk(tree):
            if not isinstance(st, ast.Assign):
                continue
            targets = st.targets[0].elts if isinstance(st.targets[0], ast.Tuple) else [st.targets[0]]
            values = st.value.elts if isinstance(st.value, ast.Tuple) and len(targets) > 1 else [st.value]
            for t, v in zip(targets, values):
                if isinstance(t, ast.Name) and isinstance(v, ast.Attribute) and v.attr in CTYPES_KIND:
                    aliases[t.id] = CTYPES_KIND[v.attr]
                if isinstance(t, ast.Attribute) and t.attr in ("argtypes", "restype") and isinstance(t.value, ast.Attribute):
                    fn = t.value.attr
                    if not fn.startswith("vsmp_"):
                        continue
                    kinds = [py_kind(e, aliases) for e in v.elts] if t.attr == "argtypes" else py_kind(v, aliases)
                    found.append((fn, t.attr, kinds))
    return found


def test_header_parse_sees_every_entry_point():
    d = declarations()
    assert len(d) == len(re.findall(r"^VSMP_API\s", re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S), re.M))
    assert d["vsmp_pick_batch"][1] == ["ptr", "ptr", "int", "int", "longlong", "ptr", "int", "ptr", "ptr", "int", "ptr",
                                       "ptr", "ulonglong", "ptr", "ptr", "ptr"]


def test_ctypes_signatures_match_the_header():
    decl = declarations()
    sigs = ctypes_signatures()
    assert any(fn == "vsmp_pick_batch" and what == "argtypes" for fn, what, _ in sigs), "no pick_batch signature shown"
    for fn, what, kinds in sigs:
        assert fn in decl, f"{fn} is not declared in include/vsmp.h"
        ret, params = decl[fn]
        if what == "argtypes":
            assert kinds == params, (fn, kinds, params)
        else:
            # ctypes returns pointers as c_void_p / c_char_p and an int as c_int
            assert kinds == ret, (fn, kinds, ret)


# The free variables of the snippets, with the types the prose around them gives.
FREE = {
    "d_logits": "const float* d_logits", "B": "int B", "V": "int V", "ld": "long long ld", "d_hist": "const int* d_hist",
    "d_off": "const int* d_off", "step": "unsigned long long step", "d_out": "int* d_out", "stream": "void* stream",
    "cfg": "vsmp_params cfg", "prompt": "const int* prompt", "n_prompt": "int n_prompt", "vocab": "int vocab",
    "d_tok": "int* d_tok", "N": "int N", "row": "int row", "prompt_ids": "const int* prompt_ids", "n": "int n",
    "d_ids": "int* d_ids", "d_active": "const int* d_active", "ctx": "vsmp_ctx* ctx", "d_hidden": "const void* d_hidden",
    "ldh": "long long ldh", "d_head": "const void* d_head", "ldw": "long long ldw", "D": "int D",
    "d_hist_off": "const int* d_hist_off", "d_rng": "unsigned long long* d_rng", "slot": "int slot",
    "d_slots": "const int* d_slots", "n_live": "int n_live", "req": "vsmp_params req",
}


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc absent")
@pytest.mark.parametrize("i", range(len(blocks("c"))))
def test_c_snippet_compiles_against_the_header(i, tmp_path):
    code = blocks("c")[i]
    body = "\n".join(line for line in code.splitlines() if not line.startswith("#include"))
    names = set(re.findall(r"\b[A-Za-z_]\w*\b", re.sub(r"/\*.*?\*/", "", body, flags=re.S)))
    declared_here = set(re.findall(r"\b(?:vsmp_\w+\*?|int|vsmp_params)\s*\*?\s*([A-Za-z_]\w*)\s*=", body))
    decls = [FREE[n] for n in sorted(names - declared_here) if n in FREE]
    # `params` is a host array of per-sequence parameters where it is passed as is, one struct where its address is taken
    if re.search(r"\bparams\b", body) and "params" not in declared_here:
        decls.append("vsmp_params params" if "&params" in body else "const vsmp_params* params")
    src = ("#include <stdio.h>\n#include <stddef.h>\n#include \"vsmp.h\"\n"
           f"void snippet(void);\nvoid snippet(void) {{\n" + "".join(f"  {d} = 0;\n" if "*" in d or d.split()[0] in
                                                                        ("int", "long", "unsigned") else f"  {d} = {{0}};\n"
                                                                        for d in decls) + body + "\n}\n")
    f = tmp_path / f"snippet{i}.c"
    f.write_text(src)
    r = subprocess.run(["gcc", "-std=c11", "-Wall", "-Wextra", "-Werror", "-Wno-unused-variable",
                        "-Wno-unused-but-set-variable", "-Wno-missing-field-initializers", "-I", str(ROOT / "include"),
                        "-c", str(f), "-o", str(tmp_path / f"snippet{i}.o")], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr + "\n" + src
