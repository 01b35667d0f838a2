"""Find the `match` expressions over lloom-tensor's device enums in Rust
source, and add the `Hip` arms a `hip` feature build needs.

The `hip` feature adds a `Hip` variant to `Device`, `DeviceLocation`,
`Storage` and `QStorage` (lloom-tensor/src/device.rs:29-47,
storage.rs:38-42, quantized/mod.rs:129-133).  Every `match` on those enums
that names the `Metal` variant and has no catch-all arm then needs a `Hip`
arm, or the feature does not compile.  This module is a small Rust lexer
and `match`/arm parser (no Rust toolchain exists here): `scan` lists the
matches, `add_hip_arms` inserts one `#[cfg(feature = "hip")]` arm per
match that lacks one, after its last `Metal` arm:

* the functions listed in `SERVE` (accessors, constructors, host copies,
  f32 <-> f16 casts, the GGUF load seam): the `Cuda` arm's own body with
  `Cuda` replaced by `Hip`, which the Hip backend types provide;
* every other function: `crate::bail!` naming the function and the enum
  (a refusal by name, as the reference's CUDA/Metal stand-ins do).

`check` reports the matches that still lack a `Hip` arm; the CPU test runs
it on a copy of lloom-tensor with the patch applied.
"""
import os
import re
import sys

ENUMS = ("Device", "DeviceLocation", "Storage", "QStorage")


# ------------------------------------------------------------------ lexer --

def lex(src):
    """Tokens (kind, text, start, end); comments and whitespace dropped."""
    toks = []
    i, n = 0, len(src)
    while i < n:
        c = src[i]
        if c.isspace():
            i += 1
            continue
        if src.startswith("//", i):
            j = src.find("\n", i)
            i = n if j < 0 else j
            continue
        if src.startswith("/*", i):
            depth, j = 1, i + 2
            while j < n and depth:
                if src.startswith("/*", j):
                    depth, j = depth + 1, j + 2
                elif src.startswith("*/", j):
                    depth, j = depth - 1, j + 2
                else:
                    j += 1
            i = j
            continue
        m = re.match(r'(?:b|c)?r(#*)"', src[i:])
        if m:  # raw string
            hashes = m.group(1)
            end = src.find('"' + hashes, i + m.end())
            j = n if end < 0 else end + 1 + len(hashes)
            toks.append(("str", src[i:j], i, j))
            i = j
            continue
        if c == '"' or (c in "bc" and src.startswith('"', i + 1)):
            j = i + (1 if c == '"' else 2)
            while j < n and src[j] != '"':
                j += 2 if src[j] == "\\" else 1
            toks.append(("str", src[i:j + 1], i, j + 1))
            i = j + 1
            continue
        if c == "'" or (c == "b" and src.startswith("'", i + 1)):
            k = i + (1 if c == "'" else 2)
            m = re.match(r"(?:\\(?:x[0-9a-fA-F]{2}|u\{[0-9a-fA-F]+\}|.)|[^\\'])'", src[k:])
            if m:  # char literal
                toks.append(("char", src[i:k + m.end()], i, k + m.end()))
                i = k + m.end()
                continue
            m = re.match(r"[A-Za-z_][A-Za-z0-9_]*", src[k:])  # lifetime
            j = k + (m.end() if m else 0)
            toks.append(("life", src[i:j], i, j))
            i = j
            continue
        m = re.match(r"[A-Za-z_][A-Za-z0-9_]*", src[i:])
        if m:
            if m.group(0) in ("r", "br") and src.startswith("#", i + m.end()):
                pass
            toks.append(("id", m.group(0), i, i + m.end()))
            i += m.end()
            continue
        m = re.match(r"[0-9][0-9A-Za-z_.]*", src[i:])
        if m:
            txt = m.group(0).rstrip(".")
            toks.append(("num", txt, i, i + len(txt)))
            i += len(txt)
            continue
        for p in ("::", "=>", "->", "..=", "...", "..", "==", "!=", "<=", ">=", "&&", "||", "+=", "-=", "*=", "/="):
            if src.startswith(p, i):
                toks.append(("p", p, i, i + len(p)))
                i += len(p)
                break
        else:
            toks.append(("p", c, i, i + 1))
            i += 1
    return toks


OPEN = {"(": ")", "[": "]", "{": "}"}


def match_close(toks, k):
    """Index of the token closing the bracket at k."""
    want, depth = OPEN[toks[k][1]], 0
    for j in range(k, len(toks)):
        t = toks[j][1] if toks[j][0] == "p" else None
        if t in OPEN:
            depth += 1
        elif t in (")", "]", "}"):
            depth -= 1
            if depth == 0:
                return j
    raise ValueError("unbalanced brackets")


# ------------------------------------------------------------ the parser --

class Arm:
    def __init__(self, pat, body, start, end, attrs):
        self.pat = pat      # token list of the pattern (guard included)
        self.body = body    # token index range of the body (lo, hi) inclusive
        self.start = start  # token index of the arm's first token (attributes included)
        self.end = end      # token index of the arm's last token (its comma included)
        self.attrs = attrs  # attribute token lists


class Match:
    def __init__(self, kw, open_, close, arms):
        self.kw, self.open, self.close, self.arms = kw, open_, close, arms


def parse_arms(toks, open_, close):
    arms, k = [], open_ + 1
    while k < close:
        start, attrs = k, []
        while toks[k][1] == "#" and toks[k + 1][1] == "[":
            e = match_close(toks, k + 1)
            attrs.append(toks[k:e + 1])
            k = e + 1
        p0 = k
        while not (toks[k][0] == "p" and toks[k][1] == "=>"):
            if toks[k][0] == "p" and toks[k][1] in OPEN:
                k = match_close(toks, k)
            k += 1
        pat = toks[p0:k]
        k += 1
        b0 = k
        if toks[k][0] == "p" and toks[k][1] == "{":
            k = match_close(toks, k)
            b1 = k
            if k + 1 < close and toks[k + 1][1] == ",":
                k += 1
        else:
            while k < close and not (toks[k][0] == "p" and toks[k][1] == ","):
                if toks[k][0] == "p" and toks[k][1] in OPEN:
                    k = match_close(toks, k)
                k += 1
            b1 = k - 1
            if k >= close:
                k = close - 1
        arms.append(Arm(pat, (b0, b1), start, k, attrs))
        k += 1
    return arms


def find_matches(toks):
    out = []
    for i, t in enumerate(toks):
        if t[0] != "id" or t[1] != "match":
            continue
        if i > 0 and toks[i - 1][1] in ("::", "."):  # a path or method named `match`
            continue
        j, depth = i + 1, 0
        while j < len(toks):
            s = toks[j][1] if toks[j][0] == "p" else None
            if s in ("(", "["):
                j = match_close(toks, j) + 1
                continue
            if s == "{":
                break
            if s in (";",):
                j = -1
                break
            j += 1
        if j < 0 or j >= len(toks):
            continue
        close = match_close(toks, j)
        try:
            arms = parse_arms(toks, j, close)
        except (ValueError, IndexError):
            continue
        out.append(Match(i, j, close, arms))
    return out


def impl_type_at(toks, k):
    """The `Self` type of the impl block around token k (None outside one)."""
    depth, j = 0, k
    while j >= 0:
        s = toks[j][1] if toks[j][0] == "p" else None
        if s == "}":
            depth += 1
        elif s == "{":
            if depth == 0:
                # is this brace the body of an `impl ...`?
                h = j - 1
                while h >= 0 and not (toks[h][0] == "p" and toks[h][1] in (";", "}", "{")):
                    if toks[h][0] == "id" and toks[h][1] == "impl":
                        head = [t[1] for t in toks[h:j]]
                        if "for" in head:
                            head = head[head.index("for") + 1:]
                        names = [x for x in head if re.match(r"[A-Za-z_]\w*$", x) and x not in ("impl", "crate", "where")]
                        return names[0] if names else None
                    h -= 1
            else:
                depth -= 1
        j -= 1
    return None


def fn_at(toks, k):
    """(name, returns_result) of the fn whose body holds token k."""
    depth, j = 0, k
    while j >= 0:
        s = toks[j][1] if toks[j][0] == "p" else None
        if s == "}":
            depth += 1
        elif s == "{":
            if depth == 0:
                h = j - 1
                while h >= 0 and not (toks[h][0] == "p" and toks[h][1] in (";", "}", "{")):
                    if toks[h][0] == "id" and toks[h][1] == "fn":
                        name = toks[h + 1][1]
                        sig = [t[1] for t in toks[h:j]]
                        ret = sig[sig.index("->") + 1:] if "->" in sig else []
                        return name, any("Result" in x for x in ret)
                    h -= 1
            else:
                depth -= 1
        j -= 1
    return None, False


def variant_refs(pat, toks, at, variant):
    """(enum, path text) of each `<path>::<variant>` in a pattern whose enum is one of ENUMS."""
    refs = []
    for q in range(len(pat)):
        if pat[q][0] == "id" and pat[q][1] == variant and q >= 2 and pat[q - 1][1] == "::":
            enum = pat[q - 2][1]
            if enum == "Self":
                enum = impl_type_at(toks, at)
            if enum in ENUMS:
                # the whole path: walk back over `a::b::`
                s = q - 2
                while s >= 2 and pat[s - 1][1] == "::" and pat[s - 2][0] == "id":
                    s -= 2
                refs.append((enum, "".join(t[1] for t in pat[s:q - 1])))
    return refs


def is_catch_all(arm):
    pat = [t[1] for t in arm.pat]
    if "if" in pat:
        return False
    if pat == ["_"] or (len(pat) == 1 and re.match(r"[a-z_]\w*$", pat[0])):
        return True
    if len(pat) == 2 and pat[0] in ("ref", "mut") and re.match(r"[a-z_]\w*$", pat[1]):
        return True
    if pat and pat[0] == "(" and pat[-1] == ")":  # a tuple of bindings / wildcards
        inner = [x for x in pat[1:-1] if x != ","]
        return all(x == "_" or re.match(r"[a-z_]\w*$", x) for x in inner) and len(inner) > 0
    return False


def scan(src):
    """The matches over ENUMS that name Metal: (match, metal arms, has hip, has catch-all)."""
    toks = lex(src)
    found = []
    for m in find_matches(toks):
        metal = [a for a in m.arms if variant_refs(a.pat, toks, m.kw, "Metal")]
        if not metal:
            continue
        hip = any(variant_refs(a.pat, toks, m.kw, "Hip") for a in m.arms)
        catch = any(is_catch_all(a) for a in m.arms)
        found.append((m, metal, hip, catch))
    return toks, found


def hip_pattern(pat_toks, toks, at):
    """The Metal arm's pattern with every listed enum's Metal variant as Hip
    (bindings kept) and every other alternative of an or-pattern dropped."""
    text = "".join(t[1] + (" " if t[0] == "id" else "") for t in pat_toks)
    # split top-level or-alternatives
    alts, depth, cur = [], 0, []
    for t in pat_toks:
        s = t[1] if t[0] == "p" else None
        if s in OPEN:
            depth += 1
        elif s in (")", "]", "}"):
            depth -= 1
        if s == "|" and depth == 0:
            alts.append(cur)
            cur = []
        else:
            cur.append(t)
    alts.append(cur)
    keep = [a for a in alts if variant_refs(a, toks, at, "Metal")]
    out = []
    for a in keep:
        s = ""
        for q, t in enumerate(a):
            word = t[1]
            if t[0] == "id" and word == "Metal" and q >= 2 and a[q - 1][1] == "::":
                enum = a[q - 2][1]
                if enum == "Self":
                    enum = impl_type_at(toks, at)
                if enum in ENUMS:
                    word = "Hip"
            if t[0] in ("id", "num") and s and (s[-1].isalnum() or s[-1] == "_"):
                s += " "
            s += word
        out.append(s)
    del text
    return " | ".join(out)


def body_text(src, toks, arm):
    b0, b1 = arm.body
    return src[toks[b0][2]:toks[b1][3]]


# Functions whose Hip arm serves the op: the Cuda arm's body with Cuda
# replaced by Hip (the Hip backend types provide the same-named methods:
# constructors and host copies for f32 / f16 / u32 / u8, location, the
# compute-dtype and pass hooks, f32 <-> f16 casts, the GGUF load seam).
# Every other function's Hip arm refuses by name.
SERVE = {
    "src/device.rs": {"location", "supports_bf16", "zeros", "alloc_uninit", "storage_from_slice", "storage",
                      "storage_owned", "synchronize", "begin_pass", "finish_pass", "abort_pass",
                      "admit_compute_dtype", "as_metal_device"},
    "src/display.rs": {"fmt_dt", "fmt"},
    "src/storage.rs": {"device", "dtype", "to_dtype"},
    "src/tensor.rs": {"to_scalar", "to_vec1", "to_vec2", "to_vec3"},
    "src/quantized/ggml_file.rs": {"from_raw_data"},
    "benches/benchmarks/mod.rs": {"sync", "bench_name"},
}

CUDA_TO_HIP = [("QCudaStorage", "QHipStorage"), ("CudaStorage", "HipStorage"), ("CudaDevice", "HipDevice"),
               ("cuda_backend", "hip_backend"), ("Cuda", "Hip"), ("cuda", "hip")]


def to_hip(text):
    for a, b in CUDA_TO_HIP:
        text = re.sub(r"\b" + a + r"\b", b, text)
    return re.sub(r"\bcuda_", "hip_", text)


def hip_arm(src, toks, m, metal_arm, rel):
    """(pattern, body) of the Hip arm for match m."""
    name, _ = fn_at(toks, m.kw)
    enums = sorted({e for e, _ in variant_refs(metal_arm.pat, toks, m.kw, "Metal")})
    if name in SERVE.get(rel, ()):
        cuda = [a for a in m.arms if variant_refs(a.pat, toks, m.kw, "Cuda")]
        if cuda:
            arm = cuda[-1]
            pat = src[arm.pat[0][2]:arm.pat[-1][3]]
            return to_hip(pat), to_hip(body_text(src, toks, arm))
    pat = hip_pattern(metal_arm.pat, toks, m.kw)
    # a refusal binds nothing
    pat = re.sub(r"::Hip\(\s*(?:ref\s+|mut\s+)?[a-z_]\w*\s*\)", "::Hip(_)", pat)
    pat = re.sub(r"::Hip\s*\{[^}]*\}", "::Hip { .. }", pat)
    mac = "crate::bail!" if rel.startswith("src/") else "lloom_tensor::bail!"
    return pat, '{}("{} is not supported on a hip {}")'.format(mac, name or "this op", "/".join(enums))


def add_hip_arms(src, rel=""):
    """src with a cfg'd Hip arm in every match over ENUMS that names Metal and
    has neither a Hip arm nor a catch-all (after its last Metal arm)."""
    toks, found = scan(src)
    edits = []
    for m, metal, hip, catch in found:
        if hip or catch:
            continue
        last = metal[-1]
        pat, body = hip_arm(src, toks, m, last, rel)
        line0 = src.rfind("\n", 0, toks[last.start][2]) + 1
        indent = re.match(r"[ \t]*", src[line0:]).group(0)
        end = toks[last.end][3]
        sep = "" if toks[last.end][1] == "," or src[toks[last.body[1]][2]] == "}" else ","
        arm = "{}\n{}#[cfg(feature = \"hip\")]\n{}{} => {}{}".format(
            sep, indent, indent, pat, body, "" if body.rstrip().endswith("}") else ",")
        edits.append((end, arm))
    for pos, text in sorted(edits, reverse=True):
        src = src[:pos] + text + src[pos:]
    return src, len(edits)


def check(src):
    """Descriptions of the matches over ENUMS naming Metal with no Hip arm and no catch-all."""
    toks, found = scan(src)
    bad = []
    for m, metal, hip, catch in found:
        if not hip and not catch:
            line = src.count("\n", 0, toks[m.kw][2]) + 1
            name, _ = fn_at(toks, m.kw)
            bad.append("line {} (fn {})".format(line, name))
    return bad


def rust_files(root):
    for d, _, fs in os.walk(root):
        for f in fs:
            if f.endswith(".rs"):
                yield os.path.join(d, f)


if __name__ == "__main__":
    mode, root = sys.argv[1], sys.argv[2]
    total = 0
    for path in sorted(rust_files(root)):
        src = open(path, encoding="utf-8").read()
        if "Metal" not in src:
            continue
        if mode == "add":
            new, n = add_hip_arms(src, os.path.relpath(path, root).replace(os.sep, "/"))
            if n:
                open(path, "w", encoding="utf-8").write(new)
                print("{}: {} arms".format(os.path.relpath(path, root), n))
                total += n
        else:
            for b in check(src):
                print("{}: {}".format(os.path.relpath(path, root), b))
                total += 1
    print("total", total)
