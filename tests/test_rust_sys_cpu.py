"""The Rust binding crate (rust/lloom-hip-sys) against the C header.

No Rust toolchain is needed: both files are parsed and every declaration is
compared.  The header is the source of truth: each function it declares
must appear in the crate's extern block with the same name, the same
parameter names in the same order, and the Rust type that has the C type's
ABI; each enum constant must appear as a `pub const` with the same value;
and the crate must declare nothing the header does not.
"""
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "lloom_hip.h")
CRATE = os.path.join(ROOT, "rust", "lloom-hip-sys")

# C spelling (whitespace-normalised) -> Rust spelling, for the types the ABI uses.
C_TO_RUST = {
    "int": "c_int", "int64_t": "i64", "uint64_t": "u64", "size_t": "usize", "float": "f32",
    "void*": "*mut c_void", "const void*": "*const c_void",
    "float*": "*mut f32", "const float*": "*const f32",
    "const uint32_t*": "*const u32", "size_t*": "*mut usize",
    "const char*": "*const c_char",
    "void**": "*mut *mut c_void",
    "lloom_hip_ctx*": "*mut lloom_hip_ctx", "lloom_hip_ctx**": "*mut *mut lloom_hip_ctx",
}


def _strip_c_comments(text):
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    return re.sub(r"//[^\n]*", " ", text)


def _c_type(decl):
    """'const float* x_dev' -> ('const float*', 'x_dev')."""
    decl = re.sub(r"\s*\*\s*", "* ", decl.strip())
    decl = re.sub(r"\*\s+\*", "**", decl)
    *ty, name = decl.split()
    return " ".join(ty).replace("* ", "*").replace(" *", "*"), name


def header_functions():
    text = _strip_c_comments(open(HEADER).read())
    out = {}
    for ret, name, params in re.findall(r"([A-Za-z_][\w ]*\**)\s*\b(lloom_hip_\w+)\s*\(([^)]*)\)\s*;", text):
        ret = re.sub(r"\s+", " ", ret.strip())
        ret = re.sub(r"\s*\*", "*", ret)
        plist = [] if params.strip() in ("", "void") else [_c_type(p) for p in params.split(",")]
        out[name] = (ret, plist)
    return out


def header_constants():
    text = _strip_c_comments(open(HEADER).read())
    consts = {}
    for body in re.findall(r"enum\s*\{([^}]*)\}", text):
        for name, value in re.findall(r"(LLOOM_HIP_\w+)\s*=\s*(-?\d+)", body):
            consts[name] = int(value)
    return consts


def crate_functions():
    src = open(os.path.join(CRATE, "src", "lib.rs")).read()
    src = re.sub(r"//[^\n]*", " ", src)
    block = re.search(r'extern\s+"C"\s*\{(.*)\n\}', src, flags=re.S).group(1)
    out = {}
    for name, params, ret in re.findall(r"pub fn (\w+)\s*\(([^)]*)\)\s*(?:->\s*([^;]+))?;", block, flags=re.S):
        plist = []
        for p in params.split(","):
            p = " ".join(p.split())
            if not p:
                continue
            pname, ty = p.split(":", 1)
            plist.append((ty.strip(), pname.strip()))
        out[name] = ((ret or "").strip(), plist)
    return out


def crate_constants():
    src = open(os.path.join(CRATE, "src", "lib.rs")).read()
    return {n: int(v) for n, v in re.findall(r"pub const (LLOOM_HIP_\w+)\s*:\s*c_int\s*=\s*(-?\d+)\s*;", src)}


def test_header_parses_completely():
    fns = header_functions()
    assert len(fns) >= 28 and "lloom_hip_qmatmul" in fns and "lloom_hip_qmatmul_noalloc" in fns
    for name, (ret, params) in fns.items():
        assert ret in C_TO_RUST or ret in ("const char*", "void*"), (name, ret)
        for ty, _ in params:
            assert ty in C_TO_RUST, (name, ty)


def test_every_header_function_is_bound_with_the_same_signature():
    hdr, crate = header_functions(), crate_functions()
    assert sorted(hdr) == sorted(crate), (set(hdr) ^ set(crate))
    for name, (ret, params) in hdr.items():
        cret, cparams = crate[name]
        assert cret == C_TO_RUST[ret], (name, ret, cret)
        assert len(cparams) == len(params), (name, len(params), len(cparams))
        for (cty, cname), (rty, rname) in zip(params, cparams):
            assert rname == cname, (name, cname, rname)
            assert rty == C_TO_RUST[cty], (name, cname, cty, rty)


def test_every_constant_matches():
    hdr, crate = header_constants(), crate_constants()
    assert len(hdr) >= 19
    assert hdr == crate, {k: (hdr.get(k), crate.get(k)) for k in set(hdr) | set(crate) if hdr.get(k) != crate.get(k)}


def test_extern_block_order_follows_the_header():
    text = _strip_c_comments(open(HEADER).read())
    hdr_order = re.findall(r"\b(lloom_hip_\w+)\s*\(", text)
    src = open(os.path.join(CRATE, "src", "lib.rs")).read()
    crate_order = re.findall(r"pub fn (lloom_hip_\w+)", src)
    assert crate_order == [n for n in hdr_order if n in set(crate_order)]


def test_manifest_and_build_script_link_the_library():
    cargo = open(os.path.join(CRATE, "Cargo.toml")).read()
    assert re.search(r'^name = "lloom-hip-sys"$', cargo, flags=re.M)
    assert re.search(r'^links = "lloom_hip"$', cargo, flags=re.M)
    build = open(os.path.join(CRATE, "build.rs")).read()
    assert "cargo:rustc-link-lib=dylib=lloom_hip" in build
    assert "LLOOM_HIP_LIB_DIR" in build and "liblloom_hip.so" in build
    src = open(os.path.join(CRATE, "src", "lib.rs")).read()
    assert '#[link(name = "lloom_hip")]' in src


def _call_args(text, start):
    """Top-level comma-separated arguments of the call whose '(' is at `start`."""
    depth, args, cur = 0, [], ""
    for ch in text[start:]:
        if ch in "([{":
            depth += 1
            if depth == 1:
                continue
        elif ch in ")]}":
            depth -= 1
            if depth == 0:
                if cur.strip():
                    args.append(cur.strip())
                return args
        if depth == 1 and ch == ",":
            args.append(cur.strip())
            cur = ""
        else:
            cur += ch
    raise AssertionError("unbalanced call")


def test_patch_calls_match_the_binding():
    """Every `sys::lloom_hip_*` call the lloom-tensor patch adds names a bound
    function and passes as many arguments as it takes."""
    patch = open(os.path.join(ROOT, "rust", "patches", "lloom-tensor-hip.patch")).read()
    added = "\n".join(line[1:] for line in patch.splitlines() if line.startswith("+") and not line.startswith("+++"))
    crate = crate_functions()
    calls = list(re.finditer(r"sys::(lloom_hip_\w+)\s*\(", added))
    assert len(calls) >= 15
    seen = set()
    for c in calls:
        name = c.group(1)
        assert name in crate, name
        args = _call_args(added, c.end() - 1)
        assert len(args) == len(crate[name][1]), (name, args)
        seen.add(name)
    for must in ("lloom_hip_qmatmul_store", "lloom_hip_moe_matmul", "lloom_hip_moe_matmul_pair",
                 "lloom_hip_moe_matmul_glu", "lloom_hip_embedding", "lloom_hip_dequantize", "lloom_hip_quantize"):
        assert must in seen, must
    for const in re.findall(r"sys::(LLOOM_HIP_\w+)", added):
        assert const in crate_constants(), const


# ------------------------------------------------ the lloom-tensor patch ---

REFERENCE_TENSOR = "/root/reference/lloom-tensor"
PATCH = os.path.join(ROOT, "rust", "patches", "lloom-tensor-hip.patch")


def _rust_arms():
    import importlib.util

    spec = importlib.util.spec_from_file_location("rust_arms", os.path.join(ROOT, "rust", "patches", "rust_arms.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_rust_arms_parser_on_known_matches():
    """The match scanner on small Rust snippets: a match over Storage with a
    Metal arm and no catch-all is reported until it has a Hip arm; a
    catch-all, an unrelated enum or a `matches!` needs none; a refusal arm
    binds nothing and names the function."""
    R = _rust_arms()
    src = '''
impl Storage {
    pub fn dtype(&self) -> DType {
        match self {
            Self::Cpu(s) => s.dtype(),
            Self::Cuda(s) => s.dtype(),
            Self::Metal(s) => s.dtype(),
        }
    }
    pub fn affine(&self, layout: &Layout, mul: f64) -> Result<Self> {
        match self {
            Self::Cpu(s) => Ok(Self::Cpu(s.affine(layout, mul)?)),
            Self::Cuda(s) => { let s = s.affine(layout, mul)?; Ok(Self::Cuda(s)) }
            Self::Metal(s) => { let s = s.affine(layout, mul)?; Ok(Self::Metal(s)) }
        }
    }
    fn pair(&self, rhs: &Self) -> bool {
        match (self, rhs) {
            (Self::Metal(a), Self::Metal(b)) => a.same(b),
            (lhs, rhs) => false,
        }
    }
}
fn other(b: Backend) -> u32 { match b { Backend::Metal => 1, Backend::Cuda => 2 } }
fn is_metal(d: &Device) -> bool { matches!(d, Device::Metal(_)) }
'''
    bad = R.check(src)
    assert len(bad) == 2 and all("fn dtype" in b or "fn affine" in b for b in bad), bad
    out, n = R.add_hip_arms(src, "src/storage.rs")
    assert n == 2 and R.check(out) == []
    assert 'Self::Hip(_) => crate::bail!("affine is not supported on a hip Storage")' in out
    assert "Self::Hip(s) => s.dtype()" in out  # served: dtype is an accessor
    assert out.count('#[cfg(feature = "hip")]') == 2


def test_patch_gives_every_device_match_a_hip_arm(tmp_path):
    """The lloom-tensor patch applied to a copy of the reference crate: the
    Hip variants exist and every match over Device, DeviceLocation, Storage
    or QStorage that names Metal has a Hip arm or a catch-all (what the
    `hip` feature needs to compile past them)."""
    import shutil
    import subprocess

    import pytest

    if not os.path.isdir(REFERENCE_TENSOR):
        pytest.skip("the reference checkout is not present")
    dst = tmp_path / "lloom-tensor"
    shutil.copytree(REFERENCE_TENSOR, dst, ignore=shutil.ignore_patterns("target"))
    r = subprocess.run(["patch", "-p1", "-s", "-i", PATCH], cwd=tmp_path, capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    src = dst / "src"
    dev = (src / "device.rs").read_text()
    assert re.search(r'#\[cfg\(feature = "hip"\)\]\s*Hip\(crate::HipDevice\)', dev)
    assert re.search(r'#\[cfg\(feature = "hip"\)\]\s*Hip \{ gpu_id: usize \}', dev)
    assert re.search(r'#\[cfg\(feature = "hip"\)\]\s*Hip\(', (src / "storage.rs").read_text())
    assert re.search(r'#\[cfg\(feature = "hip"\)\]\s*Hip\(', (src / "quantized" / "mod.rs").read_text())
    R = _rust_arms()
    missing = []
    for path in R.rust_files(str(dst)):
        text = open(path, encoding="utf-8").read()
        if "Metal" in text:
            missing += ["{}: {}".format(os.path.relpath(path, dst), b) for b in R.check(text)]
    assert not missing, "matches without a Hip arm:\n" + "\n".join(missing)
