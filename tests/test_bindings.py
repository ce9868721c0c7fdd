"""C-ABI contract of the C# binding source (smallmind_amd/bindings/csharp/Smx.cs): every
function include/smx.h declares is bound, with the same parameter count and a compatible type
per parameter (the binding cannot be compiled here: no .NET toolchain)."""
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

# C parameter type -> C# spellings that marshal to it
SCALARS = {"int": {"int"}, "int32_t": {"int"}, "int64_t": {"long"}, "uint64_t": {"ulong"}, "float": {"float"},
           "double": {"double"}, "size_t": {"nuint"}}


def _c_decls():
    t = re.sub(r"/\*.*?\*/", "", open(os.path.join(ROOT, "include", "smx.h")).read(), flags=re.S)
    out = {}
    for m in re.finditer(r"SMX_API\s+([^;(]*?)\b(smx_\w+)\s*\(([^)]*)\)\s*;", t, re.S):
        ps = [" ".join(p.split()) for p in m.group(3).split(",")]
        out[m.group(2)] = (m.group(1).strip(), [] if ps == ["void"] else ps)
    return out


def _cs_decls():
    t = open(os.path.join(ROOT, "smallmind_amd", "bindings", "csharp", "Smx.cs")).read()
    t = re.sub(r"\[MarshalAs\([^\]]*\)\]\s*", "", t)
    out = {}
    for m in re.finditer(r"\[DllImport\(Lib\)\]\s*public static extern\s+(\w+\*?)\s+(smx_\w+)\s*\(([^)]*)\)\s*;", t, re.S):
        ps = [" ".join(p.split()) for p in m.group(3).split(",")]
        out[m.group(2)] = (m.group(1), [p for p in ps if p])
    return out


def _compatible(c, cs):
    c = c.replace("const ", "").strip()
    ctype = re.sub(r"\s*\b\w+$", "", c) if not c.endswith("*") else c   # drop the parameter name
    cs_type = cs.rsplit(" ", 1)[0]
    base = ctype.replace("*", "").strip()
    stars = ctype.count("*")
    if stars == 0:
        return cs_type in SCALARS.get(base, set())
    if base == "char":
        return cs_type == "string"
    if base.startswith("smx_") and base not in ("smx_model_config", "smx_gen_stats", "smx_sampling"):
        # handles: IntPtr by value, out IntPtr for T **, IntPtr* for arrays of handles
        return cs_type in ({"IntPtr"} if stars == 1 else {"out IntPtr", "IntPtr*"})
    if base in ("smx_model_config", "smx_gen_stats", "smx_sampling"):
        names = {"smx_model_config": "ModelConfig", "smx_gen_stats": "GenStats", "smx_sampling": "Sampling"}
        n = names[base]
        return cs_type in {f"in {n}", f"out {n}", f"{n}*"}
    if base == "void":
        return cs_type in {"void*", "IntPtr"}
    mapped = {"int": "int", "int32_t": "int", "int64_t": "long", "float": "float"}.get(base)
    return mapped is not None and cs_type in {f"{mapped}*", f"out {mapped}"}


def test_every_c_function_is_bound_with_compatible_parameters():
    c, cs = _c_decls(), _cs_decls()
    assert len(c) >= 38
    assert sorted(cs) == sorted(c), set(c) ^ set(cs)
    for name, (cret, cps) in c.items():
        csret, csps = cs[name]
        assert len(cps) == len(csps), (name, cps, csps)
        want_ret = {"int": "int", "int64_t": "long", "const char *": "IntPtr"}[cret]
        assert csret == want_ret, (name, cret, csret)
        for cp, csp in zip(cps, csps):
            assert _compatible(cp, csp), (name, cp, csp)


def test_status_codes_and_type_ids_match_the_header():
    h = open(os.path.join(ROOT, "include", "smx.h")).read()
    cs = open(os.path.join(ROOT, "smallmind_amd", "bindings", "csharp", "Smx.cs")).read()
    for name, val in re.findall(r"SMX_(E\w+|OK)\s*=\s*(-?\d+)", h):
        assert re.search(rf"\b{name}\s*=\s*{val}\b", cs), name
    for name, val in re.findall(r"SMX_TYPE_(\w+)\s*=\s*(\d+)", h):
        assert re.search(rf"\b{name}\s*=\s*{val}\b", cs), name
