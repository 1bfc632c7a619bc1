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


# ---------------------------------------------------------------------------
# Argument labels.  No Swift compiler is here, so calls between the Swift
# files are checked by their labels: a call must name the parameters of one
# declaration of that name in order, omitting only defaulted ones, and pass
# positional arguments only where the declaration's external name is `_`.

HOOK = os.path.join(SWIFT, "MLXLMCommonHook", "CacheHooks.swift")
SOURCES = os.path.join(SWIFT, "Sources", "MLXLMBlockSparse")


def _balanced(text, i):
    """Index just past the parenthesis that closes the one before text[i]."""
    depth = 1
    while depth:
        ch = text[i]
        if ch in "([{":
            depth += 1
        elif ch in ")]}":
            depth -= 1
        elif ch == '"':  # skip string literals (interpolations nest parentheses)
            j = i + 1
            while text[j] != '"':
                if text[j] == "\\" and text[j + 1] == "(":
                    j = _balanced(text, j + 2) - 1
                j += 1
            i = j
        i += 1
    return i


def _split_top(args):
    parts, depth, cur = [], 0, ""
    for ch in args:
        if ch in "([{":
            depth += 1
        elif ch in ")]}":
            depth -= 1
        if ch == "," and depth == 0:
            parts.append(cur)
            cur = ""
        else:
            cur += ch
    if cur.strip():
        parts.append(cur)
    return [p.strip() for p in parts]


def _declared(text, name):
    """Parameter lists [(external label, has default)] of every `init(` (name
    "init") or `func name(` declared in text."""
    pat = r"\binit\s*\(" if name == "init" else r"\bfunc\s+" + re.escape(name) + r"\s*\("
    out = []
    for m in re.finditer(pat, text):
        end = _balanced(text, m.end())
        params = []
        for p in _split_top(text[m.end():end - 1]):
            head = p.split(":", 1)[0].split()
            assert head, f"unparsed parameter {p!r} of {name}"
            params.append((head[0], "=" in p.split(":", 1)[1]))
        out.append(params)
    return out


def _calls(text, callee):
    """Argument labels (None for positional) of every call `callee(` in text."""
    out = []
    for m in re.finditer(r"(?<![\w.])" + re.escape(callee) + r"\s*\(", text):
        if re.search(r"\b(func|init)\s*$", text[:m.start()]):
            continue
        end = _balanced(text, m.end())
        labels = []
        for a in _split_top(text[m.end():end - 1]):
            lm = re.match(r"(\w+)\s*:(?!:)", a)
            labels.append(lm.group(1) if lm else None)
        out.append(labels)
    return out


def _fits(labels, params):
    i = 0
    for lab in labels:
        while i < len(params):
            ext, has_default = params[i]
            if (lab is None and ext == "_") or lab == ext:
                break
            if not has_default:
                return False
            i += 1
        else:
            return False
        i += 1
    return all(d for _, d in params[i:])


def _check_calls(text, callee, decls, min_calls=1):
    calls = _calls(text, callee)
    assert len(calls) >= min_calls, f"expected calls of {callee}"
    for labels in calls:
        assert any(_fits(labels, p) for p in decls), \
            f"{callee}({', '.join(str(l) for l in labels)}) fits no declaration {decls}"


def _insertions():
    """The two insertions the hook file's header comment gives."""
    head = open(HOOK).read().split("public protocol", 1)[0]
    blocks, cur = [], []
    for line in head.splitlines():
        body = line[2:] if line.startswith("//") else None
        if body is not None and body.startswith("        "):
            cur.append(body[8:])
        elif cur:
            blocks.append("\n".join(cur))
            cur = []
    return blocks


def test_hook_insertions_name_what_the_hook_and_cache_declare():
    hook = open(HOOK).read()
    cache_src = {f: open(os.path.join(SOURCES, f)).read() for f in os.listdir(SOURCES)}
    attention = cache_src["Attention.swift"]
    ins = _insertions()
    assert len(ins) == 2, ins
    branch, default_case = ins
    # the branch: the protocol's one requirement, called with its labels
    assert "public protocol AttendingKVCache: KVCache" in hook
    assert "cache as? AttendingKVCache" in branch
    proto = _declared(hook, "updateAndAttend")
    assert len(proto) == 1 and [p for p, _ in proto[0]] == ["queries", "keys", "values", "scale", "mask"]
    _check_calls(branch, "attending.updateAndAttend", proto)
    # the block-sparse cache conforms and implements it with the same labels
    assert re.search(r"extension BlockSparseKVCache\s*:\s*AttendingKVCache", attention)
    impl = _declared(attention, "updateAndAttend")
    assert len(impl) == 1 and [p for p, _ in impl[0]] == [p for p, _ in proto[0]]
    # the loader's default case: PromptCacheClasses.make with its labels
    _check_calls(default_case, "PromptCacheClasses.make", _declared(hook, "make"))
    assert "default:" in default_case and "Unknown cache class" in default_case
    # INTEGRATION.md shows the same two insertions
    doc = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    squash = lambda s: re.sub(r"\s+", " ", s).strip()
    for block in ins:
        assert squash(block) in squash(doc), f"INTEGRATION.md lacks the insertion:\n{block}"


def test_swift_calls_use_declared_labels():
    """Initializer and method calls between the Swift files name declared
    parameters in declaration order."""
    cache = open(os.path.join(SOURCES, "BlockSparseKVCache.swift")).read()
    plain_cls, quant_cls = cache.split("public final class QuantizedBlockSparseKVCache", 1)
    plain_inits = [p for p in _declared(plain_cls, "init") if p and p[0][0] != "adopting"]
    quant_inits = _declared(quant_cls, "init")
    assert plain_inits and quant_inits
    everything = "\n".join(open(os.path.join(SOURCES, f)).read() for f in sorted(os.listdir(SOURCES)))
    _check_calls(everything, "BlockSparseKVCache", plain_inits, min_calls=2)
    _check_calls(everything, "QuantizedBlockSparseKVCache", quant_inits, min_calls=2)
    for method in ("appendDecode", "decodeMulti", "prefill", "append", "appendQuantized",
                   "exportQuantized", "export"):
        decls = _declared(cache, method)
        assert decls, method
        calls = _calls(everything, method) + _calls(everything, "bs." + method)
        for labels in calls:
            assert any(_fits(labels, p) for p in decls), f"{method}{labels} fits no declaration"


def test_prompt_cache_maker_reads_the_metastate_the_cache_writes():
    """The maker registered for loadPromptCache reads metaState in the order
    the cache's getter writes it, and builds the quantized class for kvBits."""
    cache = open(os.path.join(SOURCES, "BlockSparseKVCache.swift")).read()
    pc = open(os.path.join(SOURCES, "PromptCache.swift")).read()
    getter = re.search(r"public var metaState: \[String\] \{\s*get \{\s*\[(.*?)\]", cache, re.S).group(1)
    fields = [f.strip() for f in getter.split(",")]
    assert fields == ["desc.block_size", "desc.top_k", "desc.sink_blocks", "desc.recent_blocks",
                      "Int32(offset)", "desc.kv_bits", "desc.group_size"], fields
    m = re.search(r"let \(blockSize, topK, sinkBlocks, recentBlocks, kvBits, groupSize\) =\s*"
                  r"\(v\[0\], v\[1\], v\[2\], v\[3\], v\[5\], v\[6\]\)", pc)
    assert m, "maker reads metaState out of order"
    assert 'PromptCacheClasses.register(promptCacheClassName)' in pc
    assert 'promptCacheClassName = "BlockSparseKVCache"' in pc
    # the Python writer uses the same class name
    from bsattn import prompt_cache
    assert prompt_cache.CLASS_NAME == "BlockSparseKVCache"
