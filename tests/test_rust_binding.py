"""The Rust FFI crate (rust/huncho-rocm-sys) against include/huncho_rocm.h, without cargo (the
image has none): every prototype is declared in the crate's extern "C" block with the same
parameter and return types under the C -> Rust mapping (int -> c_int, long -> c_long, size_t
-> usize, const T* -> *const T, ...), every #define constant has the same value, and every
typedef'd struct has the same fields in the same order with the same types (its repr(C) layout)."""
import re

import pytest

from cdecl import (HEADER, RUST_LIB, c_to_rust, header_defines, header_prototypes, header_structs, rust_consts,
                   rust_externs, rust_structs)


def test_mapping_examples():
    assert c_to_rust("const int32_t*") == "*const i32"
    assert c_to_rust("hk_ctx**") == "*mut *mut hk_ctx"
    assert c_to_rust("const void*") == "*const c_void"
    assert c_to_rust("long") == "c_long" and c_to_rust("size_t") == "usize" and c_to_rust("double") == "f64"


def test_every_prototype_is_declared_with_the_same_types():
    want, got = header_prototypes(), rust_externs()
    assert len(want) >= 60
    assert set(want) == set(got), (set(want) ^ set(got))
    for name, (ret, params) in want.items():
        gret, gparams = got[name]
        assert gret == (ret if ret != "()" else "()"), (name, ret, gret)
        assert gparams == params, (name, params, gparams)


def test_constants_match():
    want, got = header_defines(), rust_consts()
    assert want == got


def test_structs_match():
    want, got = header_structs(), rust_structs()
    for name, fields in want.items():
        assert name in got, name
        assert got[name] == fields, (name, fields, got[name])


def test_crate_files_present():
    root = RUST_LIB.parents[1]
    cargo = (root / "Cargo.toml").read_text()
    assert 'name = "huncho-rocm-sys"' in cargo and 'links = "huncho_rocm"' in cargo
    assert "rustc-link-lib=dylib=huncho_rocm" in (root / "build.rs").read_text()
    assert HEADER.exists()
