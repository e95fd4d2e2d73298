"""The C ABI library: it loads without a GPU, exports every symbol include/qwenny_hip.h declares, and its error paths
report through status codes and qh_last_error (no compute calls without a GPU)."""

import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

from qwenny_amd import Wt, pack_quant, packed_sizes
from qwenny_amd._lib import LIB_PATH, SIGNATURES, QhError, check, lib
from tests.helpers import make_quant

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "qwenny_hip.h")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(qh_[a-z0-9_]+)\s*\(", text)))


def test_header_symbols_exported():
    names = declared()
    assert len(names) >= 20
    out = subprocess.run(["nm", "-D", "--defined-only", LIB_PATH], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\bT (qh_[a-z0-9_]+)", out))
    assert set(names) <= exported, set(names) - exported
    assert set(names) == set(SIGNATURES), set(names) ^ set(SIGNATURES)
    for n in names:
        assert getattr(lib(), n) is not None


def test_header_compiles_as_c():
    src = '#include "qwenny_hip.h"\nint main(void) { return QH_OK + QH_WT_I4 + QH_EPI_SILU - 3; }\n'
    r = subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-I", os.path.dirname(HEADER), "-x", "c", "-", "-o",
                        "/dev/null"], input=src, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_errors_report():
    with pytest.raises(QhError) as e:
        packed_sizes(Wt.I4, 17, 128)
    assert "multiple of 16" in str(e.value) and e.value.code == -1
    assert "multiple of 16" in lib().qh_last_error().decode()
    with pytest.raises(QhError):
        packed_sizes(7, 16, 128)
    with pytest.raises(QhError) as e:  # codes past 32-bit offsets: 2^31 16-bit weights
        packed_sizes(Wt.BF16, 1 << 17, 1 << 14)
    assert "4 GiB" in str(e.value)
    assert packed_sizes(Wt.I4, 248320, 5120)[0] == 248320 * 5120 // 2
    q = make_quant(1, "i4", 32, 256)
    with pytest.raises(QhError):  # 8-bit storage for a 4-bit matrix
        pack_quant(q, np.arange(32), Wt.I8)
    with pytest.raises(QhError):  # rows not in whole tiles
        pack_quant(q, np.arange(24), Wt.I4)
    with pytest.raises(QhError):  # a row beyond the matrix
        pack_quant(q, np.arange(16) + 20, Wt.I4)
    with pytest.raises(QhError):  # zero points needed
        pack_quant(q, np.arange(32), Wt.I4Z)
    check(0)


def test_sizes():
    # codes: 1 KiB (int4) / 2 KiB (int8) per 16 rows x 128 columns; scales and zero points by quads of 4 groups
    assert packed_sizes(Wt.I4, 32, 256) == (2 * 2 * 1024, 2 * 1 * 16 * 4 * 2, 0)
    assert packed_sizes(Wt.I4Z, 32, 256) == (4096, 256, 2 * 16 * 2)
    assert packed_sizes(Wt.I4Z_S32, 32, 1024) == (2 * 8 * 1024, 2 * 2 * 16 * 4 * 4, 2 * 2 * 16 * 2)
    assert packed_sizes(Wt.I8, 16, 128) == (2048, 16 * 4 * 4, 0)


def test_gemm_rejects_null_without_gpu():
    r = lib().qh_gemm(None, None, None, None, 0, 1, None, 0, None, 0, None, 0)
    assert r < 0 and "null" in lib().qh_last_error().decode()
    assert lib().qh_part_len(None, None, 0, 16) == 0
