"""Write tests/golden/reference_capi_signatures.json: the ctypes signatures the reference's
binding declares (snowllm/_capi.py:201-831, the `_SIGS` tuples) for the snowllm_* entry points
that this build's header (include/snowverify.h) declares.

The reference file is read as text and parsed with `ast`; nothing of it is imported or
executed. Each `("snowllm_name", restype, [argtypes])` tuple is folded by a small evaluator
that knows only list literals, `+`, `*` by an integer and the type names the file uses, and
the result is written as type-name strings ("P" = c_void_p, "S" = the stream, passed as
c_void_p). Run it in a container that holds the reference:

    python tests/golden/make_reference_capi_signatures.py /root/reference/snowllm/_capi.py
"""
import ast
import json
import pathlib
import re
import sys

NAMES = {"P": "P", "c_void_p": "P", "S": "S", "c_int": "c_int", "c_int64": "c_int64",
         "c_float": "c_float", "c_char_p": "c_char_p", "c_int32": "c_int32", "None": "None",
         "c_double": "c_double", "c_uint64": "c_uint64", "c_size_t": "c_size_t"}


def fold(node):
    """A type expression -> a type name, or a list of them."""
    if isinstance(node, ast.Constant) and node.value is None:
        return "None"
    if isinstance(node, ast.Constant) and isinstance(node.value, int):
        return node.value
    if isinstance(node, ast.Name):
        if node.id not in NAMES:
            raise ValueError(f"unknown type name {node.id}")
        return NAMES[node.id]
    if isinstance(node, ast.Attribute):          # ctypes.c_int64 and the like
        return NAMES[node.attr]
    if isinstance(node, ast.Call) and isinstance(node.func, ast.Name) and node.func.id == "POINTER":
        return "P"
    if isinstance(node, ast.List):
        out = []
        for e in node.elts:
            v = fold(e)
            out.extend(v if isinstance(v, list) else [v])
        return out
    if isinstance(node, ast.BinOp) and isinstance(node.op, ast.Add):
        return fold(node.left) + fold(node.right)
    if isinstance(node, ast.BinOp) and isinstance(node.op, ast.Mult):
        a, b = fold(node.left), fold(node.right)
        return a * b if isinstance(b, int) else b * a
    raise ValueError(f"unsupported expression {ast.dump(node)[:80]}")


def signatures(source: str) -> dict:
    sigs = {}
    for node in ast.walk(ast.parse(source)):
        if not (isinstance(node, ast.Tuple) and len(node.elts) == 3):
            continue
        name = node.elts[0]
        if not (isinstance(name, ast.Constant) and isinstance(name.value, str)
                and name.value.startswith("snowllm_")):
            continue
        try:
            res, args = fold(node.elts[1]), fold(node.elts[2])
        except (ValueError, KeyError):
            continue
        if isinstance(args, list):
            sigs[name.value] = {"restype": res, "argtypes": args}
    return sigs


def declared(header: pathlib.Path) -> set:
    return set(re.findall(r"\b(snowllm_[a-z0-9_]+)\s*\(", header.read_text()))


def main():
    src = pathlib.Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/snowllm/_capi.py")
    header = pathlib.Path(__file__).resolve().parents[2] / "include" / "snowverify.h"
    names = declared(header)
    sigs = {n: v for n, v in signatures(src.read_text()).items() if n in names}
    out = pathlib.Path(__file__).with_name("reference_capi_signatures.json")
    out.write_text(json.dumps({"source": "snowllm/_capi.py (SnowLLM 0.3.x)", "count": len(sigs),
                               "signatures": dict(sorted(sigs.items()))}, indent=0) + "\n")
    print(f"{len(sigs)} signatures -> {out}")


if __name__ == "__main__":
    main()
