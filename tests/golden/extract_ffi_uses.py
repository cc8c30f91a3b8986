"""Extracts, from the reference's Rust sources, what its bindgen-generated FFI
declarations must provide: every rk_npu_* / RK_NPU_* identifier the Rust code
uses from the bindings, the fields it reads or writes on each binding struct,
the constants it assigns to or compares with those fields, and the argument
count of every call into the library. Writes tests/golden/reference_ffi_uses.json,
which tests/test_abi.py checks this repository's headers against.

Run in a container that holds the reference checkout:
    python3 tests/golden/extract_ffi_uses.py /root/reference
"""
from __future__ import annotations

import json
import os
import re
import sys

# rk_npu_* / RK_NPU_* words that are not binding identifiers: environment
# variables, CMake definitions, library and header base names (build.rs,
# src/npu.rs:467-481, src/model/workspace.rs:82, src/model/trace.rs:54).
NOT_BINDINGS = {
    "RK_NPU_ENABLE_TRACE", "RK_NPU_I8_NPU_REDUCE", "RK_NPU_MATMUL_ROOT", "RK_NPU_PERFETTO_ROOT",
    "RK_NPU_PREFILL_CACHE_DOMAIN_MIB", "RK_NPU_TRACE_ROOT", "RK_NPU_W4A8_K_TILE_MULTIPLIER",
    "RK_NPU_W8A8_NPU_DEQUANT", "rk_npu_matmul", "rk_npu_matmul_static", "rk_npu_trace",
    "rk_npu_gdn", "rk_npu_mla_f16", "rk_npu_mm_gelu", "rk_npu_mm_tune",
}
IDENT = re.compile(r"\b(?:rk_npu|RK_NPU)_[A-Za-z0-9_]+\b")


def rust_files(root):
    for d, _, files in os.walk(os.path.join(root, "src")):
        for f in sorted(files):
            if f.endswith(".rs"):
                yield os.path.join(d, f)


def strip_comments(text):
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.sub(r"//[^\n]*", "", text)


def split_args(text, start):
    """Top-level arguments (stripped text) of the call whose '(' is at text[start]."""
    depth, i, cur, out = 0, start, [], []
    while i < len(text):
        c = text[i]
        if c in "([{":
            depth += 1
            if depth == 1:
                i += 1
                continue
        elif c in ")]}":
            depth -= 1
            if depth == 0:
                if "".join(cur).strip():
                    out.append("".join(cur).strip())
                return out
        elif c == "," and depth == 1:
            out.append("".join(cur).strip())
            cur = []
            i += 1
            continue
        cur.append(c)
        i += 1
    return None


def call_args(text, start):
    """Top-level argument count of the call whose '(' is at text[start]."""
    depth, args, i, nonempty = 0, 1, start, False
    while i < len(text):
        c = text[i]
        if c in "([{":
            depth += 1
        elif c in ")]}":
            depth -= 1
            if depth == 0:
                return args if nonempty else 0
        elif c == "," and depth == 1:
            # a trailing comma before ')' does not start an argument
            rest = text[i + 1:].lstrip()
            if not rest.startswith(")"):
                args += 1
        elif depth == 1 and not c.isspace():
            nonempty = True
        i += 1
    return None


def fn_bodies(text):
    """Each `fn`'s text from its name to its closing brace (nested functions
    and closures stay inside their enclosing function's text)."""
    out = []
    for m in re.finditer(r"\bfn\s+\w+", text):
        i = text.find("{", m.end())
        semi = text.find(";", m.end())
        if i < 0 or (0 <= semi < i):
            continue  # a declaration without a body
        depth, j = 0, i
        while j < len(text):
            if text[j] == "{":
                depth += 1
            elif text[j] == "}":
                depth -= 1
                if depth == 0:
                    break
            j += 1
        out.append(text[m.start():j + 1])
    return out


def scan_fields(body, rel, fields, consts, returns):
    """Field accesses on local variables and parameters of binding struct
    types within one function body: (type, field path up to three levels).
    A variable's type at a use is that of its latest `let` before the use
    (shadowing), or of the parameter of that name; a `let` initialised from
    rk_npu_T::default() or from a crate function returning rk_npu_T types it."""
    lets = {}  # var -> [(position, type or None)]
    for m in re.finditer(r"\blet\s+(?:mut\s+)?(\w+)\s*(?::\s*([\w:<>&]+)\s*)?=\s*([^;]*)", body):
        var, annot, init = m.group(1), m.group(2), m.group(3)
        ty = None
        if annot and annot.startswith("rk_npu_"):
            ty = annot
        else:
            d = re.match(r"\s*(rk_npu_\w+)::default\(\)", init)
            f = re.match(r"\s*(\w+)\s*\(", init)
            if d:
                ty = d.group(1)
            elif f and f.group(1) in returns:
                ty = returns[f.group(1)]
        lets.setdefault(var, []).append((m.start(), ty))
    params = {}
    header = body[:body.find("{")]
    for m in re.finditer(r"\b(\w+)\s*:\s*&?(?:mut\s+)?(rk_npu_\w+)\b(?!\s*[>(])", header):
        params[m.group(1)] = m.group(2)
    names = set(params) | {v for v, ds in lets.items() if any(t for _, t in ds)}
    for var in names:
        for m in re.finditer(r"(?<![\w.])" + re.escape(var) + r"((?:\.[A-Za-z_]\w*)+)", body):
            ty = params.get(var)
            for pos, t in lets.get(var, []):
                if pos < m.start():
                    ty = t
            if not ty:
                continue
            chain = m.group(1).split(".")[1:]
            if body[m.end():m.end() + 1] in ("(", ":"):
                chain = chain[:-1]  # a method call (or a path), not a field
            if not chain or chain[0] == "raw":
                continue
            field = ".".join(chain[:3])
            fields.add((ty, field, rel))
            c = re.match(r"\s*(==|=)\s*(RK_NPU_\w+)(?!\s+as\b)", body[m.end():m.end() + 80])
            if c and not re.match(r"\w", body[m.end() + c.end():m.end() + c.end() + 1]):
                consts.add((ty, field, c.group(2), "assign" if c.group(1) == "=" else "compare"))


def main(root):
    ids, calls, fields, consts, const_args = set(), {}, set(), set(), set()
    # crate functions returning a binding struct by value
    returns = {}
    for path in rust_files(root):
        text = strip_comments(open(path, encoding="utf-8").read())
        for m in re.finditer(r"\bfn\s+(\w+)\s*\([^{;]*?\)\s*->\s*(rk_npu_\w+)\s*\{", text, flags=re.S):
            returns[m.group(1)] = m.group(2)
    # any `.field = RK_NPU_X` / `.field == RK_NPU_X`, whatever the receiver
    named = set()
    for path in rust_files(root):
        text = strip_comments(open(path, encoding="utf-8").read())
        rel = os.path.relpath(path, root)
        for m in IDENT.finditer(text):
            name = m.group(0)
            if name in NOT_BINDINGS:
                continue
            # inside a string literal (error messages, env names): skip
            line = text[text.rfind("\n", 0, m.start()) + 1:text.find("\n", m.end())]
            before = line[:m.start() - (text.rfind("\n", 0, m.start()) + 1)]
            if before.count('"') % 2 == 1:
                continue
            ids.add(name)
            after = text[m.end():m.end() + 1]
            if name.startswith("rk_npu_") and after == "(":
                n = call_args(text, m.end())
                if n is not None:
                    calls.setdefault(name, set()).add(n)
                    for i, a in enumerate(split_args(text, m.end()) or []):
                        if re.fullmatch(r"RK_NPU_\w+", a):
                            const_args.add((name, i, a))
        for body in fn_bodies(text):
            scan_fields(body, rel, fields, consts, returns)
        for m in re.finditer(r"\.([A-Za-z_]\w*)\s*(==|=)\s*(RK_NPU_\w+)\b(?!\s+as\b)", text):
            named.add((m.group(1), m.group(3), "assign" if m.group(2) == "=" else "compare"))
    out = {
        "source": "reference src/**/*.rs (comments removed)",
        "identifiers": sorted(ids),
        "call_arity": {k: sorted(v) for k, v in sorted(calls.items())},
        "fields": sorted({(t, f) for t, f, _ in fields}),
        "field_constants": sorted(consts),
        "named_field_constants": sorted(named),
        "constant_arguments": sorted(const_args),
    }
    dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), "reference_ffi_uses.json")
    with open(dst, "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")
    print(f"{len(ids)} identifiers, {len(calls)} called functions, {len(out['fields'])} fields -> {dst}")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
