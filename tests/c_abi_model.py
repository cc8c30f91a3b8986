"""The C declarations of include/*.h as bindgen would turn them into Rust,
for checking them against how the reference's Rust code uses its bindings.

The headers are parsed by clang (-ast-dump=json); integer macros are read
from the header text. Rust types follow bindgen's rules for the reference's
build (build.rs:132-158: default enum style, no macro-type callback): a
non-negative integer #define is u32 and a negative one i32; a C enum becomes
constants of its underlying type, `unsigned int` (u32) when no enumerator is
negative, else `int` (i32); int32_t/uint32_t/uint64_t/float/double map to
i32/u32/u64/f32/f64; a pointer is *const or *mut of its pointee."""
from __future__ import annotations

import glob
import json
import os
import re
import shutil
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(ROOT, "include")


def clang():
    for cand in ("/opt/rocm/llvm/bin/clang", shutil.which("clang") or ""):
        if cand and os.path.exists(cand):
            return cand
    return None


_PRIM = {"int": "i32", "unsigned int": "u32", "long": "i64", "unsigned long": "u64", "long long": "i64",
         "unsigned long long": "u64", "short": "i16", "unsigned short": "u16", "signed char": "i8",
         "char": "i8", "unsigned char": "u8", "float": "f32", "double": "f64", "void": "()"}


class Headers:
    def __init__(self):
        self.records = {}    # struct name -> {field: C type (desugared)}
        self.typedefs = {}   # typedef name -> desugared C type
        self.enums = {}      # enum name -> {"unsigned": bool, "values": {name: value}}
        self.functions = {}  # name -> (return C type, [param C types])
        self.macros = {}     # name -> int value
        self._parse()

    def _parse(self):
        headers = sorted(glob.glob(os.path.join(INCLUDE, "*.h")))
        src = "".join(f'#include "{os.path.basename(h)}"\n' for h in headers)
        out = subprocess.run([clang(), "-x", "c", "-std=c11", "-fsyntax-only", "-Xclang", "-ast-dump=json",
                              "-I", INCLUDE, "-"], input=src, capture_output=True, text=True, check=True).stdout
        ast = json.loads(out)
        for node in ast.get("inner", []):
            kind, name = node.get("kind"), node.get("name", "")
            if not (name.startswith("rk_npu_") or kind == "EnumDecl"):
                continue
            if kind == "RecordDecl" and node.get("completeDefinition"):
                self.records[name] = {f["name"]: self._type(f["type"]) for f in node.get("inner", [])
                                      if f.get("kind") == "FieldDecl"}
            elif kind == "RecordDecl":
                self.records.setdefault(name, None)  # opaque
            elif kind == "TypedefDecl":
                self.typedefs[name] = self._type(node["type"])
            elif kind == "EnumDecl":
                values = {}
                for c in node.get("inner", []):
                    if c.get("kind") == "EnumConstantDecl":
                        values[c["name"]] = self._enum_value(c, values)
                self.enums[name] = {"unsigned": all(v >= 0 for v in values.values()), "values": values}
            elif kind == "FunctionDecl":
                params = [self._type(p["type"]) for p in node.get("inner", []) if p.get("kind") == "ParmVarDecl"]
                ret = node["type"]["qualType"].split("(")[0].strip()
                self.functions[name] = (ret, params)
        for h in headers:
            text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
            for m in re.finditer(r"^\s*#define\s+(RK_NPU_\w+)\s+\(?\s*(-?\s*(?:0x[0-9a-fA-F]+|\d+))[uUlL]*\s*\)?"
                                 r"(?:\s*<<\s*(\d+))?\)?\s*$", text, flags=re.M):
                v = int(m.group(2).replace(" ", ""), 0)
                if m.group(3):
                    v <<= int(m.group(3))
                self.macros[m.group(1)] = v

    @staticmethod
    def _type(t):
        return t.get("desugaredQualType", t["qualType"])

    @staticmethod
    def _enum_value(node, previous):
        for inner in node.get("inner", []):
            if "value" in inner:
                return int(inner["value"])
            for sub in inner.get("inner", []):
                if "value" in sub:
                    return int(sub["value"])
        return (max(previous.values()) + 1) if previous else 0

    # ---- names -------------------------------------------------------------
    def declared_names(self):
        names = set(self.records) | set(self.typedefs) | set(self.functions) | set(self.macros)
        for e in self.enums.values():
            names |= set(e["values"])
        return names

    # ---- Rust types --------------------------------------------------------
    def rust_type(self, ctype: str) -> str:
        c = ctype.strip()
        c = re.sub(r"\bconst\s+", "", c) if not c.endswith("*") else c
        if c.endswith("*"):
            pointee = c[:-1].strip()
            const = pointee.startswith("const ") or pointee.endswith(" const")
            pointee = pointee.replace("const ", "").replace(" const", "").strip()
            return ("*const " if const else "*mut ") + self.rust_type(pointee)
        if c.startswith("enum "):
            e = self.enums.get(c[5:].strip())
            return "u32" if (e is None or e["unsigned"]) else "i32"
        if c.startswith("struct "):
            return c[7:].strip()
        if c in self.typedefs and self.typedefs[c] != c:
            return self.rust_type(self.typedefs[c])
        return _PRIM.get(c, c)

    def constant_type(self, name: str):
        if name in self.macros:
            return "u32" if self.macros[name] >= 0 else "i32"
        for e in self.enums.values():
            if name in e["values"]:
                return "u32" if e["unsigned"] else "i32"
        return None

    def record_of(self, tname: str):
        """Fields of a struct named directly or through a typedef."""
        if tname in self.records and self.records[tname] is not None:
            return self.records[tname]
        t = self.typedefs.get(tname, "")
        if t.startswith("struct "):
            return self.records.get(t[7:].strip())
        return None

    def field_type(self, tname: str, path: str):
        """C type at the end of a dotted field path, or None if a step is missing."""
        ctype = None
        for part in path.split("."):
            rec = self.record_of(tname)
            if rec is None or part not in rec:
                return None
            ctype = rec[part]
            tname = ctype[7:].strip() if ctype.startswith("struct ") else ctype
        return ctype
