"""The Swift glue (swift/Sources) against the C ABI it binds.

No Swift toolchain exists here, so the glue is checked structurally: every
tbh_* function it calls is declared in include/tinybrain_hip.h with the same
number of parameters, every struct it builds uses the C struct's fields in
declaration order (Swift's memberwise initialisers of imported C structs take
all fields, in order), every TBH_* constant it names exists, and the module
map's shim header reaches the ABI header.
"""
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "tinybrain_hip.h")
SWIFT = os.path.join(ROOT, "swift", "Sources", "TinyBrainHIP", "HIPBackend.swift")
MODMAP_DIR = os.path.join(ROOT, "swift", "Sources", "CTinyBrainHIP")


def _strip_c_comments(s):
    return re.sub(r"/\*.*?\*/", "", s, flags=re.S)


def _split_top(args):
    """Top-level comma split of an argument list (ignores nested (), [], {})."""
    out, depth, cur = [], 0, []
    for ch in args:
        if ch in "([{":
            depth += 1
        elif ch in ")]}":
            depth -= 1
        if ch == "," and depth == 0:
            out.append("".join(cur).strip())
            cur = []
        else:
            cur.append(ch)
    tail = "".join(cur).strip()
    if tail:
        out.append(tail)
    return out


def _header_functions():
    text = _strip_c_comments(open(HEADER).read())
    funcs = {}
    for m in re.finditer(r"\b(?:tbh_status|int32_t|const char \*)\s*(tbh_\w+)\s*\(([^;]*?)\)\s*;", text, re.S):
        params = m.group(2).strip()
        funcs[m.group(1)] = 0 if params in ("", "void") else len(_split_top(params))
    return funcs


def _header_struct_fields(name):
    text = _strip_c_comments(open(HEADER).read())
    m = re.search(r"typedef struct %s \{(.*?)\} %s;" % (name, name), text, re.S)
    assert m, name
    fields = []
    for decl in m.group(1).split(";"):
        decl = decl.strip()
        if decl:
            fields.append(re.findall(r"(\w+)\s*(?:\[\w*\])?$", decl)[0])
    return fields


def _calls(src, name_re):
    """(name, [args]) of every call matching name_re, with balanced parens."""
    out = []
    for m in re.finditer(r"\b(%s)\s*\(" % name_re, src):
        i, depth = m.end(), 1
        while depth:
            depth += {"(": 1, ")": -1}.get(src[i], 0)
            i += 1
        out.append((m.group(1), _split_top(src[m.end():i - 1])))
    return out


def _swift_source():
    src = open(SWIFT).read()
    return re.sub(r"//[^\n]*", "", src)   # comments cite reference calls in prose


def test_every_abi_call_matches_the_header():
    funcs = _header_functions()
    calls = [(n, a) for n, a in _calls(_swift_source(), r"tbh_\w+")
             if n not in ("tbh_qtensor_desc", "tbh_attention_shape")]
    assert calls, "no ABI calls found"
    called = set()
    for name, args in calls:
        assert name in funcs, f"{name} is not declared in tinybrain_hip.h"
        assert len(args) == funcs[name], f"{name}: {len(args)} arguments, header declares {funcs[name]}"
        called.add(name)
    # the protocol entry points the glue must bind
    for need in ("tbh_device_open", "tbh_device_close", "tbh_weight_create", "tbh_weight_destroy",
                 "tbh_matmul", "tbh_dequantize", "tbh_softmax", "tbh_rmsnorm", "tbh_silu", "tbh_gelu",
                 "tbh_attention", "tbh_last_error"):
        assert need in called, need


def test_struct_initialisers_use_every_field_in_order():
    src = _swift_source()
    for struct in ("tbh_qtensor_desc", "tbh_attention_shape"):
        fields = _header_struct_fields(struct)
        inits = _calls(src, struct)
        assert inits, struct
        for _, args in inits:
            labels = [a.split(":", 1)[0].strip() for a in args]
            assert labels == fields, (struct, labels, fields)


def test_constants_exist():
    header = open(HEADER).read()
    for const in set(re.findall(r"\bTBH_[A-Z0-9_]+\b", _swift_source())):
        assert re.search(r"\b%s\b" % const, header), const


def test_module_map_reaches_the_header():
    modmap = open(os.path.join(MODMAP_DIR, "module.modulemap")).read()
    assert re.search(r'link\s+"tinybrain_hip"', modmap)
    shim = re.search(r'header\s+"([^"]+)"', modmap).group(1)
    inc = re.search(r'#include\s+"([^"]+)"', open(os.path.join(MODMAP_DIR, shim)).read()).group(1)
    assert os.path.samefile(os.path.join(MODMAP_DIR, inc), HEADER)


def test_backend_conforms_to_the_reference_protocols():
    # the five protocols of Backend.swift:173-228 and their method signatures
    src = _swift_source()
    decl = re.search(r"class HIPBackend:([^{]*)\{", src).group(1)
    for proto in ("QuantizedMatMulBackend", "SoftmaxBackend", "RMSNormBackend", "ActivationBackend",
                  "AttentionBackend"):
        assert proto in decl, proto
    for sig in (r"func matmulQuantized\(_ input: Tensor<Float>, _ quantized: QuantizedTensor\) throws -> Tensor<Float>",
                r"func softmax\(_ input: Tensor<Float>\) throws -> Tensor<Float>",
                r"func rmsnorm\(_ input: Tensor<Float>, weight: Tensor<Float>, eps: Float\) throws -> Tensor<Float>",
                r"func silu\(_ input: Tensor<Float>\) throws -> Tensor<Float>",
                r"func gelu\(_ input: Tensor<Float>\) throws -> Tensor<Float>",
                r"func attention\(query: Tensor<Float>, keys: Tensor<Float>, values: Tensor<Float>,\s*"
                r"mask: Tensor<Float>\?, headDim: Int, numHeads: Int, numKVHeads: Int\) throws -> Tensor<Float>"):
        assert re.search(sig, src), sig
