"""The C-ABI library loads on the CPU and exports every declared entry point."""

import ctypes
import os

import pytest

from kadllm_amd import _lib


def test_library_is_built():
    assert os.path.exists(_lib.LIB_PATH), "run python -m kadllm_amd.csrc.build"


def test_exports_every_declared_symbol():
    lib = _lib.load()
    declared = _lib.header_symbols()
    assert "kad_gdn_suffix_replay" in declared
    missing = [s for s in declared if not hasattr(lib, s)]
    assert not missing, f"declared in include/kadllm_hip.h but not exported: {missing}"


def test_signature_table_covers_header():
    declared = set(_lib.header_symbols()) - {"kad_last_error", "kad_abi_version"}
    assert declared == set(_lib.SIGNATURES), declared ^ set(_lib.SIGNATURES)


def _letter(param):
    p = " ".join(param.split())
    if p.startswith("kad_stream_t"):
        return "s"
    if "*" in p:
        return "p"
    if p.startswith("int64_t"):
        return "l"
    if p.startswith("int "):
        return "i"
    if p.startswith("float"):
        return "f"
    raise AssertionError(f"unclassified parameter {param!r}")


def test_signature_types_match_header():
    import re
    text = open(_lib.HEADER_PATH).read()
    for name, sig in _lib.SIGNATURES.items():
        m = re.search(r"int\s+" + name + r"\s*\(([^;]*)\);", text, re.S)
        assert m, name
        params = [p for p in m.group(1).split(",") if p.strip() and p.strip() != "void"]
        letters = "".join(_letter(p) for p in params)
        assert letters == sig, (name, letters, sig)


def test_abi_version_and_error_string():
    lib = _lib.load()
    assert lib.kad_abi_version() >= 1
    # argument validation runs on the host, before any device work
    rc = lib.kad_selftest_mfma16(None, None, None, None)
    assert rc == -1
    assert b"null" in lib.kad_last_error()
