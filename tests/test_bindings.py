"""The two non-Python callers of the C ABI, without a GPU:

* tests/c/host_checks.c, a C program built against include/llmk_sampler.h
  (-std=c99 -pedantic -Werror) and linked to libllmk_sampler.so, runs the
  argument checks of every entry point;
* rust/llm-kernel/src/hip_sampler.rs, the Rust binding (no Rust toolchain
  here): its `extern "C"` block declares the header's functions with the
  header's parameter counts, its `#[repr(C)]` args struct has the header's
  fields in order with the same widths, and its constants equal the
  header's;
* rust/apply.sh applies the binding and the sampling-parameter plumbing
  (types.rs:176-196, llm-cli/src/lib.rs:22-31 and :144-150,
  llm-ffi/src/lib.rs) to a copy of llm-rs, when the reference tree is
  present in this container (skipped elsewhere)."""
import os
import re
import shutil
import subprocess

import pytest

from llmk import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HDR = os.path.join(ROOT, "include", "llmk_sampler.h")
RS = os.path.join(ROOT, "rust", "llm-kernel", "src", "hip_sampler.rs")
REFERENCE = "/root/reference"


def _strip_c_comments(s):
    return re.sub(r"/\*.*?\*/", "", s, flags=re.S)


def test_c_program_host_checks(tmp_path):
    assert os.path.exists(_lib.LIB_PATH), "build first: python -c 'import __graft_entry__ as g; g.build()'"
    libdir = os.path.dirname(_lib.LIB_PATH)
    exe = tmp_path / "host_checks"
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Wextra", "-Werror", "-pedantic",
                    "-I", os.path.join(ROOT, "include"), os.path.join(ROOT, "tests", "c", "host_checks.c"),
                    "-L", libdir, "-lllmk_sampler", f"-Wl,-rpath,{libdir}", "-o", str(exe)], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.startswith("ok "), r.stdout


def test_header_compiles_as_cpp(tmp_path):
    src = tmp_path / "h.cpp"
    src.write_text('#include "llmk_sampler.h"\nint main() { return sizeof(llmk_sample_batch_args) == 192 ? 0 : 1; }\n')
    subprocess.run(["g++", "-std=c++11", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"),
                    str(src), "-o", str(tmp_path / "h")], check=True)
    assert subprocess.run([str(tmp_path / "h")]).returncode == 0


def _c_functions():
    src = _strip_c_comments(open(HDR).read())
    out = {}
    for m in re.finditer(r"\b(?:int|void|const char\*)\s+(llmk_[a-z_]+)\s*\(([^)]*)\)\s*;", src):
        params = [p for p in m.group(2).split(",") if p.strip() and p.strip() != "void"]
        out[m.group(1)] = len(params)
    return out


def _rust_functions():
    src = open(RS).read()
    block = re.search(r'extern "C" \{(.*?)\n\}', src, flags=re.S).group(1)
    out = {}
    for m in re.finditer(r"pub fn (llmk_[a-z_]+)\((.*?)\)", block, flags=re.S):
        params = [p for p in m.group(2).split(",") if p.strip()]
        out[m.group(1)] = len(params)
    return out


def test_rust_extern_block_matches_the_header():
    c, r = _c_functions(), _rust_functions()
    assert sorted(c) == sorted(_lib.EXPORTED_SYMBOLS)
    assert c == r


# C type -> (Rust types accepted, bytes)
C2RS = {"const void*": ("*const c_void",), "int32_t": ("i32",), "uint32_t": ("u32",),
        "uint64_t": ("u64",), "float": ("f32",), "const float*": ("*const f32",),
        "const int32_t*": ("*const i32",), "const uint32_t*": ("*const u32",),
        "uint32_t*": ("*mut u32",), "float*": ("*mut f32",)}


def test_rust_args_struct_matches_the_header():
    src = _strip_c_comments(open(HDR).read())
    body = re.search(r"typedef struct \{(.*?)\} llmk_sample_batch_args;", src, flags=re.S).group(1)
    cf = []
    for decl in body.split(";"):
        decl = " ".join(decl.split())
        if not decl:
            continue
        m = re.match(r"(.*?)\s*\b([a-z_]+)$", decl)
        ty = m.group(1).replace(" *", "*").strip()
        cf.append((m.group(2), ty))
    rs = open(RS).read()
    rbody = re.search(r"pub struct LlmkSampleBatchArgs \{(.*?)\n\}", rs, flags=re.S).group(1)
    rf = re.findall(r"pub ([a-z_]+): ([^,]+),", rbody)
    assert [n for n, _ in cf] == [n for n, _ in rf]
    for (n, cty), (_, rty) in zip(cf, rf):
        assert rty.strip() in C2RS[cty], (n, cty, rty)
    # and the ctypes mirror the Python binding uses
    assert [n for n, _ in cf] == [f for f, _ in _lib.SampleBatchArgs._fields_]


def test_rust_constants_match_the_header():
    hdr = open(HDR).read()
    rs = open(RS).read()
    names = re.findall(r"#define (LLMK_[A-Z0-9_]+) ", hdr)
    assert len(names) >= 13
    for name in names:
        hv = int(re.search(rf"#define {name} \(?(-?(?:0x)?[0-9a-f]+)u?\)?", hdr).group(1), 0)
        m = re.search(rf"pub const {name}: [iu]32 = (-?(?:0x)?[0-9a-f_]+);", rs)
        assert m, name
        assert int(m.group(1).replace("_", ""), 0) == hv, name
    for name, v in (("LLMK_F32", 0), ("LLMK_BF16", 1), ("LLMK_F16", 2)):
        assert re.search(rf"pub const {name}: i32 = {v};", rs)


@pytest.mark.skipif(not os.path.isdir(os.path.join(REFERENCE, "llm-core")),
                    reason="the llm-rs tree is not in this container")
def test_rust_patches_apply_to_llm_rs(tmp_path):
    dst = tmp_path / "llm-rs"
    os.makedirs(dst)
    for crate in ("llm-core", "llm-cli", "llm-ffi", "llm-kernel", "llm-scheduler", "llm-tests"):
        shutil.copytree(os.path.join(REFERENCE, crate), dst / crate,
                        ignore=shutil.ignore_patterns("target", "*.gguf", "*.safetensors", "*.bin"))
    r = subprocess.run([os.path.join(ROOT, "rust", "apply.sh"), str(dst)], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    types = (dst / "llm-core" / "src" / "types.rs").read_text()
    for f in ("presence_penalty", "frequency_penalty", "min_p", "seed", "logit_bias"):
        assert f"pub {f}:" in types
    cli = (dst / "llm-cli" / "src" / "lib.rs").read_text()
    assert "top_k: req.top_k.unwrap_or(40)" in cli and "pub logit_bias: Option<" in cli
    ffi = (dst / "llm-ffi" / "src" / "lib.rs").read_text()
    assert "pub mod request_v2;" in ffi and "pub mod sampler;" in ffi
    assert (dst / "llm-kernel" / "src" / "hip_sampler.rs").exists()
    # every struct literal of the extended types now fills the new fields
    for dp, _, fs in os.walk(dst):
        for f in fs:
            if not f.endswith(".rs"):
                continue
            txt = open(os.path.join(dp, f)).read()
            for m in re.finditer(r"(?:SampleParams|ChatCompletionRequest) \{\n", txt):
                depth, i = 1, m.end()
                while depth:  # to the matching brace
                    depth += {"{": 1, "}": -1}.get(txt[i], 0)
                    i += 1
                lit = txt[m.end():i]
                if "pub " in lit or "fn " in lit:
                    continue  # a definition or impl, not a literal
                assert "..Default::default()" in lit or "logit_bias" in lit, (f, lit[:200])
    # a second run refuses (the new files exist already) and changes nothing
    r2 = subprocess.run([os.path.join(ROOT, "rust", "apply.sh"), str(dst)], capture_output=True, text=True)
    assert r2.returncode != 0
    assert (dst / "llm-core" / "src" / "types.rs").read_text() == types
