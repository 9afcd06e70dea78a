"""Writes ref_bindings_signatures.json: the ctypes signature of every C entry
point the reference's Python seam declares (ref scripts/kcmm/bindings.py,
the loader vLLM's patches use), read from that file's text with `ast` --
nothing of the reference is imported or run.  Each type is reduced to an
ABI kind (ptr, u32, u64, i32, f32, size, void) so the fixture is data.

Run from the repository root where /root/reference exists:
    python tests/golden/make_ref_bindings.py
"""
import ast
import json
from pathlib import Path

SRC = Path("/root/reference/scripts/kcmm/bindings.py")
OUT = Path(__file__).with_name("ref_bindings_signatures.json")

KINDS = {"c_uint32": "u32", "c_uint64": "u64", "c_size_t": "size", "c_int": "i32",
         "c_int32": "i32", "c_float": "f32", "c_char_p": "ptr", "c_void_p": "ptr",
         "c_int64": "i64", "c_uint8": "u8", "c_uint16": "u16"}


def kind(node, pointer_names):
    if isinstance(node, ast.Constant) and node.value is None:
        return "void"
    if isinstance(node, ast.Call) and getattr(node.func, "attr", "") == "POINTER":
        return "ptr"
    if isinstance(node, ast.Attribute):
        return KINDS.get(node.attr, node.attr)
    if isinstance(node, ast.Name):
        return "ptr" if node.id in pointer_names else node.id
    return ast.unparse(node)


def main():
    tree = ast.parse(SRC.read_text())
    # names bound to pointer types (e.g. `pool = ctypes.c_void_p`)
    pointer_names = set()
    for n in ast.walk(tree):
        if isinstance(n, ast.Assign) and len(n.targets) == 1 and isinstance(n.targets[0], ast.Name):
            v = n.value
            if (isinstance(v, ast.Attribute) and v.attr in ("c_void_p", "c_char_p")) or \
               (isinstance(v, ast.Call) and getattr(v.func, "attr", "") == "POINTER"):
                pointer_names.add(n.targets[0].id)
    sigs = {}
    for n in ast.walk(tree):
        if not (isinstance(n, ast.Assign) and len(n.targets) == 1):
            continue
        t = n.targets[0]
        if not (isinstance(t, ast.Attribute) and t.attr in ("argtypes", "restype")):
            continue
        fn = t.value.attr if isinstance(t.value, ast.Attribute) else None
        if not fn or not fn.startswith("kcmm_"):
            continue
        entry = sigs.setdefault(fn, {})
        if t.attr == "argtypes":
            entry["args"] = [kind(e, pointer_names) for e in n.value.elts]
        else:
            entry["ret"] = kind(n.value, pointer_names)
    OUT.write_text(json.dumps({"source": "scripts/kcmm/bindings.py", "functions": sigs},
                              indent=1, sort_keys=True) + "\n")
    print(f"{len(sigs)} functions -> {OUT}")


if __name__ == "__main__":
    main()
