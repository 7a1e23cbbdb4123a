"""The C-ABI library loads and exports every function include/awq.h declares
(no compute calls: these run without a GPU)."""
import os
import re
import subprocess

import cube_awq
from cube_awq import _lib
from conftest import REPO


def _declared_functions():
    names = set()
    for fn in os.listdir(os.path.join(REPO, "include")):
        if fn.endswith(".h"):
            text = open(os.path.join(REPO, "include", fn)).read()
            text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
            names |= set(re.findall(r"\b(awq_[a-z0-9_]+)\s*\(", text))
    return names


def test_header_declares_what_the_binding_wraps():
    assert _declared_functions() == set(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = cube_awq.lib()
    for name in _declared_functions():
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r" T (awq_[a-z0-9_]+)$", out, flags=re.M))
    assert _declared_functions() <= exported


def test_library_is_gfx950_only():
    out = subprocess.run(["/opt/rocm/llvm/bin/clang-offload-bundler", "--list", "--type=o",
                          f"--input={_lib.LIB_PATH}"], capture_output=True, text=True)
    if out.returncode == 0 and out.stdout.strip():
        targets = [t for t in out.stdout.split() if "amdgcn" in t]
        assert targets and all("gfx950" in t for t in targets), targets


def test_version_and_constants():
    lib = cube_awq.lib()
    assert lib.awq_version() >= 100
    s = lib.awq_shape_config_new(1, 32, 64, 8, 32, 64)
    assert (s.m, s.n, s.k, s.tile_m, s.tile_n, s.inner_k, s.line_size, s.m_valid) == \
        (1, 32, 64, 8, 32, 64, 4, 1)
    s = lib.awq_shape_config_new_with_valid_m(32, 32, 32, 32, 32, 32, 33)
    assert s.m_valid == 33
