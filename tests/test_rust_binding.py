"""The Rust binding (rust/qe-sys, source only: no Rust toolchain in the build image) against the C
header it binds: every `fn qe_*` of its extern block is declared in include/qe.h with the same
argument count and vice versa, its QE_* constants have the header's values, and its #[repr(C)]
structs list the header's fields in the header's order."""
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "qe.h")
CRATE = os.path.join(ROOT, "rust", "qe-sys")


def strip_c(text):
    return re.sub(r"/\*.*?\*/", "", text, flags=re.S)


def strip_rust(text):
    return re.sub(r"//[^\n]*", "", text)


def split_args(args):
    """top-level comma split (the Rust side may hold fn types in parentheses)"""
    out, depth, cur = [], 0, ""
    for ch in args:
        if ch in "(<":
            depth += 1
        elif ch in ")>":
            depth -= 1
        if ch == "," and depth == 0:
            out.append(cur)
            cur = ""
        else:
            cur += ch
    out.append(cur)
    return [a.strip() for a in out if a.strip()]


def c_functions():
    text = strip_c(open(HEADER).read())
    text = re.sub(r"typedef[^;]*;", "", text)
    fns = {}
    for name, args in re.findall(r"\b(qe_[a-z0-9_]+)\s*\(([^;{]*?)\)\s*;", text, flags=re.S):
        a = split_args(args)
        fns[name] = 0 if a == ["void"] else len(a)
    return fns


def rust_extern_block():
    text = strip_rust(open(os.path.join(CRATE, "src", "lib.rs")).read())
    m = re.search(r'extern "C"\s*\{(.*)\n\}', text, flags=re.S)
    assert m, "no extern block in lib.rs"
    return m.group(1)


def rust_functions():
    fns = {}
    for name, args in re.findall(r"pub fn (qe_[a-z0-9_]+)\s*\((.*?)\)\s*(?:->[^;]*)?;", rust_extern_block(),
                                 flags=re.S):
        fns[name] = len(split_args(args))
    return fns


def test_crate_files_exist():
    for f in ("Cargo.toml", "build.rs", "src/lib.rs", "src/hip_inference.rs"):
        assert os.path.isfile(os.path.join(CRATE, f)), f
    toml = open(os.path.join(CRATE, "Cargo.toml")).read()
    assert re.search(r'^name = "qe-sys"', toml, flags=re.M)
    assert 'pub mod hip_inference;' in open(os.path.join(CRATE, "src", "lib.rs")).read()


def test_every_header_function_is_bound_with_its_argument_count():
    c, r = c_functions(), rust_functions()
    assert len(c) >= 29
    assert sorted(c) == sorted(r), (sorted(set(c) - set(r)), sorted(set(r) - set(c)))
    wrong = {n: (c[n], r[n]) for n in c if c[n] != r[n]}
    assert not wrong, wrong


def test_constants_match_the_header():
    hdr = dict(re.findall(r"#define (QE_[A-Z0-9_]+) (0x[0-9A-Fa-f]+|\d+)u?", open(HEADER).read()))
    rs = dict(re.findall(r"pub const (QE_[A-Z0-9_]+): \w+ = (0x[0-9A-Fa-f_]+|\d+);",
                         open(os.path.join(CRATE, "src", "lib.rs")).read()))
    assert sorted(hdr) == sorted(rs), (sorted(set(hdr) - set(rs)), sorted(set(rs) - set(hdr)))
    for k in hdr:
        assert int(hdr[k], 0) == int(rs[k].replace("_", ""), 0), k


def c_struct_fields(name):
    text = strip_c(open(HEADER).read())
    m = re.search(r"typedef struct(?: \w+)? \{([^{}]*)\} " + name + ";", text)
    assert m, name
    return re.findall(r"\b(\w+);", m.group(1))


def rust_struct_fields(name):
    text = strip_rust(open(os.path.join(CRATE, "src", "lib.rs")).read())
    m = re.search(r"#\[repr\(C\)\][^{]*?pub struct " + name + r" \{(.*?)\}", text, flags=re.S)
    assert m, name
    return re.findall(r"pub (\w+):", m.group(1))


def test_structs_match_the_header():
    for s in ("qe_config", "qe_lookup_stats"):
        assert c_struct_fields(s) == rust_struct_fields(s), s
    # field types of the config: u64 x 7, f32, f32, u32, as uint64_t x 7, float, float, uint32_t
    text = strip_rust(open(os.path.join(CRATE, "src", "lib.rs")).read())
    body = re.search(r"pub struct qe_config \{(.*?)\}", text, flags=re.S).group(1)
    assert re.findall(r":\s*(\w+),", body) == ["u64"] * 7 + ["f32", "f32", "u32"]


def test_the_parser_sees_a_wrong_argument_count():
    """the check above fails on a binding with one argument dropped"""
    block = rust_extern_block()
    bad = block.replace("kv: *mut qe_kv, logits_out: *mut f32) -> c_int;", "kv: *mut qe_kv) -> c_int;", 1)
    assert bad != block
    fns = {n: len(split_args(a)) for n, a in re.findall(r"pub fn (qe_[a-z0-9_]+)\s*\((.*?)\)\s*(?:->[^;]*)?;", bad,
                                                         flags=re.S)}
    assert fns["qe_forward"] == c_functions()["qe_forward"] - 1
