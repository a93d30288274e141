"""ABI qualification of libomega_gpu against the reference's Omega ABI manifest.

The reference qualifies an Omega archive before linking it (aien-abi-conformance
src/build.rs:166-239 `qualify_built`, src/probe.rs:40-140 `check_c`): the manifest's structs must
be declared with the same fields in the same order, every function must have a prototype of the
manifest's signature, a C probe compiled against the headers must print the manifest's layout and
constant facts (sizeof / _Alignof of each struct; offset, width, element kind and count of each
field; each constant's value), and the archive must define every function. This module runs the
same three checks against include/omega_gpu.h and the built libomega_gpu.a / .so, so a maintainer
can qualify this library the way the reference qualifies Omega's (the prebuilt-override link of
`qualify_prebuilt`, build.rs:255-300, checks only the symbols).

Manifest format (aien-abi-conformance src/manifest.rs:21-80): one fact per line,
  struct <name> <size> <align>
  field <struct> <name> <offset> <size> <kind> <count>
  const <name> <value>
  fn <name> fn(<arg kinds>) -> <ret>
with kinds in Rust spelling (u32, *const u16, *mut *mut OmegaGpuTensor, c_char, ...).

Usage: python -m omega_amd.qualify [manifest] [--header include/omega_gpu.h] [--lib libomega_gpu.a]
"""
from __future__ import annotations

import os
import re
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
REPO = os.path.dirname(PKG)
HEADER = os.path.join(REPO, "include", "omega_gpu.h")
ARCHIVE = os.path.join(PKG, "_build", "libomega_gpu.a")
SHARED = os.path.join(PKG, "_build", "libomega_gpu.so")

# C scalar types and their manifest kinds
C_KINDS = {
    "uint8_t": "u8", "int8_t": "i8", "uint16_t": "u16", "int16_t": "i16", "uint32_t": "u32",
    "int32_t": "i32", "uint64_t": "u64", "int64_t": "i64", "int": "i32", "unsigned": "u32",
    "unsigned int": "u32", "size_t": "usize", "float": "f32", "double": "f64", "bool": "bool",
    "_Bool": "bool", "char": "c_char", "void": "c_void",
}


class Manifest:
    def __init__(self, text: str):
        self.structs: list[tuple[str, int, int]] = []
        self.fields: list[tuple[str, str, int, int, str, int]] = []
        self.consts: list[tuple[str, int]] = []
        self.fns: list[tuple[str, str]] = []
        for no, raw in enumerate(text.splitlines(), 1):
            line = raw.split("#", 1)[0].strip()
            if not line:
                continue
            w = line.split()
            if w[0] in ("abi", "header"):
                continue
            if w[0] == "struct" and len(w) == 4:
                self.structs.append((w[1], int(w[2]), int(w[3])))
            elif w[0] == "field" and len(w) == 7:
                self.fields.append((w[1], w[2], int(w[3]), int(w[4]), w[5], int(w[6])))
            elif w[0] == "const" and len(w) == 3:
                self.consts.append((w[1], int(w[2])))
            elif w[0] == "fn" and len(w) >= 3:
                self.fns.append((w[1], " ".join(w[2:])))
            else:
                raise ValueError(f"manifest line {no}: cannot parse {raw!r}")

    def field_names(self, struct: str) -> list[str]:
        return [f[1] for f in self.fields if f[0] == struct]

    def layout_lines(self) -> list[str]:
        out = [f"struct {n} {s} {a}" for n, s, a in self.structs]
        out += [f"field {s} {n} {o} {z} {k} {c}" for s, n, o, z, k, c in self.fields]
        out += [f"const {n} {v}" for n, v in self.consts]
        return out


# ---------------------------------------------------------------- header parsing
def _strip_comments(src: str) -> str:
    src = re.sub(r"/\*.*?\*/", " ", src, flags=re.S)
    return re.sub(r"//[^\n]*", " ", src)


def header_structs(src: str) -> dict[str, list[str]]:
    """typedef struct Name { ... } Name; -> ordered field names (comma declarators split)."""
    out = {}
    for m in re.finditer(r"typedef\s+struct\s+(\w+)\s*\{(.*?)\}\s*(\w+)\s*;", src, flags=re.S):
        names = []
        for decl in m.group(2).split(";"):
            decl = " ".join(decl.split())
            if not decl:
                continue
            parts = decl.split(",")
            first = parts[0]
            tail = [first.split()[-1]] + [p.strip() for p in parts[1:]]
            for d in tail:
                d = re.sub(r"\[.*?\]", "", d).replace("*", "").strip()
                names.append(d)
        out[m.group(3)] = names
    return out


def _c_type_to_kind(t: str) -> str:
    """One C parameter / return type (no name) in manifest spelling."""
    t = " ".join(t.replace("*", " * ").split())
    stars = t.count("*")
    words = [w for w in t.split() if w != "*"]
    # `const` binds to the pointee for `const T *`; a `T *const` is not used by this ABI
    const = "const" in words and words.index("const") == 0
    base_words = [w for w in words if w not in ("const", "struct", "enum")]
    base = " ".join(base_words)
    kind = C_KINDS.get(base, base)
    if stars == 0:
        return "()" if kind == "c_void" else kind
    inner = ("*const " if const else "*mut ") + kind
    for _ in range(stars - 1):
        inner = "*mut " + inner
    return inner


def header_fns(src: str) -> dict[str, str]:
    """Prototypes `ret name(params);` -> manifest signature `fn(kinds) -> ret`."""
    out = {}
    flat = " ".join(re.sub(r"^\s*#[^\n]*", " ", src, flags=re.M).split())
    for stmt in re.split(r"[;{}]", flat):
        m = re.fullmatch(r"\s*([A-Za-z_][\w\s\*]*?)\b(omega_gpu_\w+)\s*\(([^()]*)\)\s*", stmt)
        if not m:
            continue
        ret, name, params = m.group(1).strip(), m.group(2), m.group(3).strip()
        if ret.startswith("typedef"):
            continue
        args = []
        if params and params != "void":
            for p in params.split(","):
                words = " ".join(p.replace("*", " * ").split()).split()
                # the parameter name is the last word when a type word precedes it
                if len(words) > 1 and re.fullmatch(r"[A-Za-z_]\w*", words[-1]) and \
                        any(w not in ("const", "struct", "enum") for w in words[:-1]):
                    words = words[:-1]
                args.append(_c_type_to_kind(" ".join(words)))
        out[name] = f"fn({', '.join(args)}) -> {_c_type_to_kind(ret)}"
    return out


# ---------------------------------------------------------------- probe
def probe_source(m: Manifest, header: str) -> str:
    lines = ["#include <stddef.h>", "#include <stdbool.h>", "#include <stdint.h>", "#include <stdio.h>",
             f'#include "{header}"',
             '_Static_assert(sizeof(long) == 8 && sizeof(void *) == 8, "LP64 only");',
             "#define K(x) _Generic((x), uint8_t: \"u8\", int8_t: \"i8\", uint16_t: \"u16\", "
             "int16_t: \"i16\", uint32_t: \"u32\", int32_t: \"i32\", unsigned long: \"u64\", "
             "long: \"i64\", unsigned long long: \"u64\", long long: \"i64\", float: \"f32\", "
             "double: \"f64\", bool: \"bool\", char: \"c_char\", default: \"?\")",
             "int main(void) {"]
    for n, _, _ in m.structs:
        lines.append(f'    printf("struct {n} %zu %zu\\n", sizeof({n}), _Alignof({n}));')
    for s, f, _, _, _, count in m.fields:
        el = f"((({s} *)0)->{f}[0])" if count > 1 else f"((({s} *)0)->{f})"
        lines.append(f'    printf("field {s} {f} %zu %zu %s %zu\\n", offsetof({s}, {f}), '
                     f"sizeof((({s} *)0)->{f}), K({el}), sizeof((({s} *)0)->{f}) / sizeof({el}));")
    for n, _ in m.consts:
        lines.append(f'    printf("const {n} %lld\\n", (long long)({n}));')
    lines += ["    return 0;", "}"]
    return "\n".join(lines) + "\n"


def run_probe(m: Manifest, header: str, cc: str = "gcc") -> list[str]:
    with tempfile.TemporaryDirectory() as d:
        src = os.path.join(d, "probe.c")
        exe = os.path.join(d, "probe")
        with open(src, "w") as f:
            f.write(probe_source(m, os.path.abspath(header)))
        r = subprocess.run([cc, "-std=c11", "-Wall", "-o", exe, src], capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"probe does not compile:\n{r.stderr}")
        r = subprocess.run([exe], capture_output=True, text=True, check=True)
        return r.stdout.splitlines()


def defined_symbols(lib: str) -> set[str]:
    dyn = ["-D"] if lib.endswith(".so") else []
    r = subprocess.run(["nm", "-g", "--defined-only", *dyn, lib], capture_output=True, text=True, check=True)
    syms = set()
    for line in r.stdout.splitlines():
        w = line.split()
        if len(w) >= 3 and w[1] in ("T", "D", "B", "R", "W"):
            syms.add(w[2])
    return syms


def check(manifest_text: str, header: str = HEADER, libs=(ARCHIVE, SHARED)) -> tuple[str, list[str]]:
    """(report, errors): the three checks of check_c; no errors means the library qualifies."""
    m = Manifest(manifest_text)
    errs: list[str] = []
    src = _strip_comments(open(header).read())
    structs, fns = header_structs(src), header_fns(src)
    for s, _, _ in m.structs:
        want = m.field_names(s)
        got = structs.get(s)
        if got is None:
            errs.append(f"struct {s}: not declared in the header")
        elif got != want:
            errs.append(f"struct {s}: C fields {got} != manifest fields {want}")
    for n, sig in m.fns:
        got = fns.get(n)
        if got is None:
            errs.append(f"fn {n}: no prototype in the header")
        elif got != sig:
            errs.append(f"fn {n}: C signature `{got}` != manifest `{sig}`")
    try:
        lines = run_probe(m, header)
    except RuntimeError as e:
        errs.append(str(e))
        lines = []
    for want in m.layout_lines():
        if want not in lines:
            key = " ".join(want.split()[: 3 if want.startswith("field ") else 2]) + " "
            got = next((x for x in lines if x.startswith(key)), "(absent)")
            errs.append(f"layout: C `{got}` != manifest `{want}`")
    for lib in libs:
        syms = defined_symbols(lib)
        for n, _ in m.fns:
            if n not in syms:
                errs.append(f"symbol {n}: not defined in {os.path.basename(lib)}")
    report = (f"headers: {len(m.structs)} structs, {len(m.fns)} functions; "
              f"probe: {len(m.layout_lines())} layout/constant facts; "
              f"symbols: {len(m.fns)} functions in {', '.join(os.path.basename(x) for x in libs)}")
    return report, errs


def main(argv=None) -> int:
    import argparse

    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("manifest", nargs="?", default=os.path.join(REPO, "tests", "golden", "omega_gpu.manifest"))
    ap.add_argument("--header", default=HEADER)
    ap.add_argument("--lib", action="append")
    a = ap.parse_args(argv)
    report, errs = check(open(a.manifest).read(), a.header, tuple(a.lib or (ARCHIVE, SHARED)))
    print(report)
    for e in errs:
        print("  -", e)
    print("qualified" if not errs else f"{len(errs)} problem(s): not qualified")
    return 0 if not errs else 1


if __name__ == "__main__":
    sys.exit(main())
