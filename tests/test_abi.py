"""The C ABI library: it loads, exports every function include/ftx.h
declares, and reports errors as status codes (no GPU needed)."""
import ctypes as C
import os
import subprocess

import pytest

from xwfes_amd import ftx
import pyoracle as P


def test_library_exports_every_declared_function():
    lib = ftx.load()
    names = ftx.header_functions()
    assert len(names) >= 25
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_exports_match_nm():
    out = subprocess.run(["nm", "-D", "--defined-only", ftx.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l and "ftx_" in l}
    assert set(ftx.header_functions()) <= exported


@pytest.mark.parametrize("dt", sorted(P.BLOCK))
def test_row_bytes_match_oracle(dt):
    lib = ftx.load()
    for n in (0, 1, 31, 32, 33, 256, 4096, 4097, 14336):
        assert lib.ftx_row_bytes(dt, n) == P.row_bytes(dt, n)
    assert lib.ftx_row_bytes(99, 32) == 0


def test_null_and_bad_arguments_are_status_codes():
    lib = ftx.load()
    assert lib.ftx_create(0, None) == -1
    assert lib.ftx_destroy(None) == 0
    assert lib.ftx_sync(None) == -1
    assert lib.ftx_matmul(None, None, 1, 1, None, None) == -1
    assert lib.ftx_verify_step(None, None, None, None) == -1
    assert lib.ftx_accept(None, None) == -1
    assert lib.ftx_last_error(None) == b"no context"


def test_dtype_ids_match_reference_and_oracle():
    assert (ftx.F32, ftx.F16, ftx.Q4_0, ftx.Q4_1, ftx.Q8_0, ftx.BF16) == (0, 1, 2, 3, 8, 30)
    assert (ftx.Q4_K, ftx.Q6_K) == (P.Q4_K, P.Q6_K)
    assert ftx.BLOCK == P.BLOCK
