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


def _c_struct_fields(name):
    """(type, field) pairs of `typedef struct name {...}` in include/smx.h, arrays expanded."""
    h = open(os.path.join(ROOT, "include", "smx.h")).read()
    body = re.search(r"typedef struct %s \{(.*?)\} %s;" % (name, name), h, re.S).group(1)
    body = re.sub(r"/\*.*?\*/", "", body, flags=re.S)
    out = []
    for decl in body.split(";"):
        decl = decl.strip()
        if not decl:
            continue
        m = re.match(r"(\w+)\s+(\w+)(?:\[(\d+)\])?$", decl)
        assert m, decl
        out += [(m.group(1), m.group(2))] * int(m.group(3) or 1)
    return out


def _cs_struct_types(name):
    cs = open(os.path.join(ROOT, "smallmind_amd", "bindings", "csharp", "Smx.cs")).read()
    one_line = re.search(r"public struct %s \{([^}\n]*)\}" % name, cs)
    body = one_line.group(1) if one_line else re.search(r"public struct %s\b[^{]*\{(.*?)\n\s*\}" % name, cs,
                                                         re.S).group(1)
    body = re.sub(r"//[^\n]*", "", body)
    types = []
    for decl in body.split(";"):
        m = re.match(r"\s*public\s+(?:fixed\s+)?(\w+)\s+(.*)", decl.strip(), re.S)
        if not m:
            continue
        t, names = m.group(1), m.group(2)
        for nm in names.split(","):
            arr = re.search(r"\[(\d+)\]", nm)
            types += [t] * (int(arr.group(1)) if arr else 1)
    return types


def test_struct_layouts_match_the_header():
    """smx_sampling, smx_model_config and smx_gen_stats: the ctypes structures the Python host
    passes and the C# structs declare the header's field types in the header's order."""
    import ctypes

    from smallmind_amd import _lib as L
    c_to_ctypes = {"float": ctypes.c_float, "double": ctypes.c_double, "int32_t": ctypes.c_int32}
    c_to_cs = {"float": "float", "double": "double", "int32_t": "int"}
    for cname, py, csname in (("smx_sampling", L.SamplingC, "Sampling"), ("smx_model_config", L.ModelConfigC,
                                                                          "ModelConfig"),
                              ("smx_gen_stats", L.GenStatsC, "GenStats")):
        fields = _c_struct_fields(cname)
        flat = []
        for fname, ftype in py._fields_:
            n = getattr(ftype, "_length_", 1)
            base = getattr(ftype, "_type_", ftype) if n > 1 else ftype
            flat += [base] * n
        assert [c_to_ctypes[t] for t, _ in fields] == flat, cname
        assert [c_to_cs[t] for t, _ in fields] == _cs_struct_types(csname), cname
