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


def _class_body(cs: str, name: str) -> tuple:
    """(declaration line, body text) of `class name` in C# source."""
    m = re.search(r"(internal|public)[^\n]*\bclass %s\b([^\n{]*)" % name, cs)
    assert m, name
    start = cs.index("{", m.end())
    depth, i = 0, start
    while True:
        depth += {"{": 1, "}": -1}.get(cs[i], 0)
        if depth == 0:
            return m.group(0), cs[start:i]
        i += 1


def _sig(text: str) -> str:
    return " ".join(re.sub(r"\s*([(),])\s*", r"\1", text).split())


# The reference's interface members, as declared (text copied with file:line so a drift in
# either side fails here).
IWEIGHT_MEMBERS = {   # src/SmallMind.Quantization/Abstractions/IWeightTensor.cs
    "int Rows": 12, "int Cols": 17, "QuantScheme Scheme": 22,
    "void MatMul(ReadOnlySpan<float> activations,Span<float> output,int m,int k,int n)": 33,
    "float[] ToFloat32()": 41,
}
IRUNTIME_MEMBERS = {  # src/SmallMind.Runtime/Execution/IRuntimeExecutor.cs
    "PrefillResult Prefill(ReadOnlySpan<int> promptTokens,ExecutionContext context)": 17,
    "DecodeResult Decode(int nextToken,ExecutionContext context)": 26,
}


def _public_members(body: str) -> set:
    out = set()
    for m in re.finditer(r"public\s+([\w<>\[\],. ]+?\s+\w+)\s*(\([^)]*\)|=>|\{)", body):
        head = _sig(m.group(1))
        out.add(head + (_sig(m.group(2)) if m.group(2).startswith("(") else ""))
    return out


def test_csharp_backend_classes_implement_the_reference_interfaces():
    """GpuWeightTensor declares every IWeightTensor member and GpuRuntimeExecutor every
    IRuntimeExecutor member with the interface's exact signature, and each class names the
    interface in its base list."""
    cs = open(os.path.join(ROOT, "smallmind_amd", "bindings", "csharp", "Smx.cs")).read()
    for cls, iface, members in (("GpuWeightTensor", "IWeightTensor", IWEIGHT_MEMBERS),
                                ("GpuRuntimeExecutor", "IRuntimeExecutor", IRUNTIME_MEMBERS)):
        decl, body = _class_body(cs, cls)
        assert re.search(r":\s*[^{]*\b%s\b" % iface, decl), decl
        have = _public_members(body)
        for sig, line in members.items():
            assert _sig(sig) in have, (cls, sig, f"{iface}.cs:{line}", sorted(have))


def test_weight_tensor_orientation_is_the_one_linear_injects():
    """Linear.SetQuantizedWeight accepts a weight only when Rows == outFeatures and
    Cols == inFeatures (NeuralNet.cs:89), and ForwardQuantized calls MatMul with
    k = inFeatures, n = outFeatures (NeuralNet.cs:168-173): Rows/Cols report out/in and MatMul
    checks k against Cols and n against Rows."""
    cs = open(os.path.join(ROOT, "smallmind_amd", "bindings", "csharp", "Smx.cs")).read()
    _, body = _class_body(cs, "GpuWeightTensor")
    assert re.search(r"public int Rows => _out;", body)
    assert re.search(r"public int Cols => _in;", body)
    assert re.search(r"if \(k != Cols\) throw new ArgumentException", body)
    assert re.search(r"if \(n != Rows\) throw new ArgumentException", body)
    assert re.search(r"new float\[_out \* _in\]", body)


def _integration_csharp_blocks():
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    return re.findall(r"```csharp\n(.*?)```", text, re.S)


def test_integration_excerpts_match_the_header():
    """Every C# struct and DllImport excerpt in INTEGRATION.md declares the header's field types
    in order and a parameter list compatible with include/smx.h, so a maintainer copying an
    excerpt gets the binding Smx.cs has (a float where the header has a double would shift every
    later field)."""
    c = _c_decls()
    c_to_cs = {"float": "float", "double": "double", "int32_t": "int"}
    names = {"Sampling": "smx_sampling", "ModelConfig": "smx_model_config", "GenStats": "smx_gen_stats"}
    seen_structs, seen_funcs = set(), set()
    for block in _integration_csharp_blocks():
        for sm in re.finditer(r"public struct (\w+)\b[^{]*\{(.*?)\}", block, re.S):
            cname = names[sm.group(1)]
            body = re.sub(r"//[^\n]*", "", sm.group(2))
            types = []
            for decl in body.split(";"):
                m = re.match(r"\s*public\s+(?:fixed\s+)?(\w+)\s+(.*)", decl.strip(), re.S)
                if not m:
                    continue
                for nm in m.group(2).split(","):
                    arr = re.search(r"\[(\d+)\]", nm)
                    types += [m.group(1)] * (int(arr.group(1)) if arr else 1)
            assert types == [c_to_cs[t] for t, _ in _c_struct_fields(cname)], (sm.group(1), types)
            seen_structs.add(sm.group(1))
        block = re.sub(r"\[MarshalAs\([^\]]*\)\]\s*", "", block)
        for fm in re.finditer(r"\[DllImport\(Lib\)\]\s*public static extern\s+(\w+\*?)\s+(smx_\w+)\s*\(([^)]*)\)\s*;",
                              block, re.S):
            name = fm.group(2)
            assert name in c, name
            ps = [p for p in (" ".join(x.split()) for x in fm.group(3).split(",")) if p]
            assert len(ps) == len(c[name][1]), (name, ps)
            for cp, csp in zip(c[name][1], ps):
                assert _compatible(cp, csp), (name, cp, csp)
            seen_funcs.add(name)
    assert seen_structs == {"Sampling", "ModelConfig", "GenStats"}, seen_structs
    assert {"smx_session_cancel", "smx_session_set_max_time", "smx_session_generate"} <= seen_funcs
