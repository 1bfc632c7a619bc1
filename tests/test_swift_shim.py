"""The SwiftPM system-library target: its module map builds the CBSAttn
module from the C header with ROCm's clang (-fmodules), a C translation unit
that imports it sees every entry point with the declared types, and the
Swift sources call only functions the header declares, with as many
arguments as each takes."""
from __future__ import annotations

import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SWIFT = os.path.join(ROOT, "swift")
HEADER = os.path.join(ROOT, "include", "bsattn.h")


def _clang():
    for c in ("/opt/rocm/llvm/bin/clang", shutil.which("clang")):
        if c and os.path.exists(c):
            return c
    pytest.skip("no clang")


def _declarations():
    """name -> argument count of every function the header declares."""
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    out = {}
    for m in re.finditer(r"\b(bsattn_\w+)\s*\(([^;{]*?)\)\s*;", text):
        args = m.group(2).strip()
        out[m.group(1)] = 0 if args in ("", "void") else args.count(",") + 1
    return out


def test_module_map_builds_and_exports_every_entry_point(tmp_path):
    decls = _declarations()
    assert len(decls) >= 28
    uses = "\n".join(f"    (void)&{n};" for n in sorted(decls))
    src = tmp_path / "use.c"
    src.write_text(
        "#pragma clang module import CBSAttn\n"
        "int main(void) {\n"
        "    bsattn_desc d = {0};\n"
        "    bsattn_cache* c = 0;\n"
        "    d.max_seqs = 1; d.dtype = BSATTN_BF16;\n"
        "    int rc = bsattn_cache_create(&d, &c);\n"
        "    rc |= bsattn_decode(c, 0, 0, 1, 0.125f, 0, 0, 0);\n"
        "    rc |= (BSATTN_ERR_NOMEM != -5);\n"
        f"{uses}\n"
        "    return rc;\n"
        "}\n")
    cmd = [_clang(), "-fmodules", "-fsyntax-only", "-Werror",
           f"-fmodule-map-file={os.path.join(SWIFT, 'Sources', 'CBSAttn', 'module.modulemap')}",
           f"-fmodules-cache-path={tmp_path / 'mc'}", str(src)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    # a misspelt entry point must fail through the module too
    bad = tmp_path / "bad.c"
    bad.write_text("#pragma clang module import CBSAttn\nint main(void) { return bsattn_no_such_call(); }\n")
    r = subprocess.run(cmd[:-1] + [str(bad)], capture_output=True, text=True)
    assert r.returncode != 0


def test_package_declares_the_system_library():
    pkg = open(os.path.join(SWIFT, "Package.swift")).read()
    assert '.systemLibrary(name: "CBSAttn", path: "Sources/CBSAttn")' in pkg
    assert '"CBSAttn"' in pkg and '"MLXLMCommon"' in pkg
    mm = open(os.path.join(SWIFT, "Sources", "CBSAttn", "module.modulemap")).read()
    assert 'link "bsattn"' in mm


def _swift_calls():
    calls = []
    d = os.path.join(SWIFT, "Sources", "MLXLMBlockSparse")
    for f in sorted(os.listdir(d)):
        text = open(os.path.join(d, f)).read()
        for m in re.finditer(r"\b(bsattn_\w+)\(", text):
            # count top-level commas up to the matching parenthesis
            i, depth, commas, empty = m.end(), 1, 0, True
            while depth:
                ch = text[i]
                if ch in "([":
                    depth += 1
                elif ch in ")]":
                    depth -= 1
                elif ch == "," and depth == 1:
                    commas += 1
                if depth and not ch.isspace():
                    empty = False
                i += 1
            calls.append((f, m.group(1), 0 if empty else commas + 1))
    return calls


def test_swift_calls_match_the_header():
    decls = _declarations()
    calls = _swift_calls()
    assert len(calls) >= 15
    for f, name, n in calls:
        if name == "bsattn_desc" or name == "bsattn_info":
            continue  # struct initializers
        assert name in decls, f"{f}: {name} is not declared in bsattn.h"
        assert n == decls[name], f"{f}: {name} called with {n} arguments, declared with {decls[name]}"


def test_swift_cache_implements_the_kvcache_protocol():
    """Every requirement of KVCache (KVCache.swift:38-77) and of
    QuantizedKVCacheProtocol (:94-118) has an implementation."""
    text = open(os.path.join(SWIFT, "Sources", "MLXLMBlockSparse", "BlockSparseKVCache.swift")).read()
    for req in ("public var offset: Int", "public var maxSize: Int?",
                "public func update(keys: MLXArray, values: MLXArray) -> (MLXArray, MLXArray)",
                "public var state: [MLXArray]", "public var metaState: [String]",
                "public var isTrimmable: Bool", "public func trim(_ n: Int) -> Int",
                "public func makeMask(n: Int, windowSize: Int?, returnArray: Bool)",
                "public func copy() -> any KVCache", "public func innerState() -> [MLXArray]",
                "public var groupSize: Int", "public var bits: Int", "public var mode: QuantizationMode",
                "public func updateQuantized(keys: MLXArray, values: MLXArray)",
                "public func getQuantizedState()"):
        assert req in text, req
