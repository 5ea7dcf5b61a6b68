"""CPU checks of the C ABI: the library loads, exports every symbol the header
declares, and reports errors through status codes. No compute calls: there is
no GPU in the build container."""
import ctypes
import os
import re

import numpy as np
import pytest

import midman_hip as mh


def header_functions():
    src = open(mh.HEADER_PATH).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(mmh_[a-z0-9_]+)\s*\(", src)))


def test_header_and_binding_agree():
    names = header_functions()
    assert len(names) >= 30
    assert set(names) == set(mh._SIGNATURES), set(names) ^ set(mh._SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = mh.lib()
    missing = [n for n in header_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_abi_version_and_empty_error():
    assert mh.abi_version() == 1
    assert mh.last_error() == ""


def test_invalid_handles_are_argument_errors_not_crashes():
    lib = mh.lib()
    assert lib.mmh_context_destroy(12345) == mh.ERR_ARGUMENT
    assert "invalid context handle" in mh.last_error()
    assert lib.mmh_model_destroy(777) == mh.ERR_ARGUMENT
    assert lib.mmh_synchronize(0) == mh.ERR_ARGUMENT
    assert lib.mmh_gemm_nn(99, None, None, None, 1, 1, 1, 0) == mh.ERR_ARGUMENT
    n = ctypes.c_int64()
    assert lib.mmh_model_param_count(5, ctypes.byref(n)) == mh.ERR_ARGUMENT
    with pytest.raises(mh.ArgumentError):
        mh.check(lib.mmh_timer_start(-3))


def test_context_create_rejects_null_output_pointer():
    assert mh.lib().mmh_context_create(0, None) == mh.ERR_ARGUMENT


def test_status_code_values_match_the_reference_abi():
    # crates/midman-api/src/ffi.rs:44-61
    assert (mh.OK, mh.STOPPED, mh.ERR_ARGUMENT, mh.ERR_CONFIG, mh.ERR_SHAPE, mh.ERR_INDEX,
            mh.ERR_OTHER, mh.ERR_PANIC) == (0, 1, -1, -2, -3, -4, -5, -99)
    src = open(mh.HEADER_PATH).read()
    for name, val in [("MMH_OK", "0"), ("MMH_ERR_ARGUMENT", "(-1)"), ("MMH_ERR_INDEX", "(-4)"),
                      ("MMH_ERR_PANIC", "(-99)")]:
        assert re.search(rf"#define {name} {re.escape(val)}", src), name


def test_presets_match_the_oracle_config():
    import mm_oracle as O
    for name, cfg in mh.PRESETS.items():
        c = O.preset(name)
        assert c.as_list()[:7] == cfg[:7], name
        assert O.param_count(c) > 0
