"""The C ABI on the host: libnq_hip.so loads, exports every entry point that
include/nq.h declares with the binding's signature table, and rejects bad
arguments before anything is enqueued (no GPU needed for any of this)."""
import ctypes
import os
import re

import numpy as np
import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "nq.h")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(nq_[a-z0-9_]+)\s*\(", text))


@pytest.fixture(scope="module")
def lib():
    from nanoinfer_amd import _lib
    return _lib.load()


def test_every_declared_symbol_is_exported_and_bound(lib):
    from nanoinfer_amd import _lib
    names = declared()
    assert len(names) >= 14
    for n in names:
        assert hasattr(lib, n), n
    assert names == set(_lib.SIGNATURES), names ^ set(_lib.SIGNATURES)


def test_no_reference_or_oracle_linkage():
    so = open(os.path.join(ROOT, "nanoinfer_amd", "libnq_hip.so"), "rb").read()
    assert b"nqo_" not in so and b"nqr_" not in so and b"liboracle" not in so


def test_version_and_status_names(lib):
    assert b"gfx950" in lib.nq_version()
    assert lib.nq_status_name(0) == b"NQ_OK"
    assert lib.nq_status_name(1) == b"NQ_BAD_SHAPE"
    assert lib.nq_status_name(99) == b"NQ_UNKNOWN"


def test_validation_before_launch(lib):
    from nanoinfer_amd import _lib as L
    fake = ctypes.c_void_p(0x1000)
    # negative shapes (reference: std::invalid_argument)
    assert lib.nq_linear_q8(fake, 0, fake, fake, None, fake, 0, -1, 4, 4, None) == L.NQ_BAD_SHAPE
    assert b"negative" in lib.nq_last_error()
    # group must be positive (quant.cpp:297)
    assert lib.nq_quantize_q4g(fake, 2, 8, 0, fake, fake, 0, None) == L.NQ_BAD_SHAPE
    assert b"group must be positive" in lib.nq_last_error()
    assert lib.nq_linear_q4g(fake, 0, fake, fake, 0, 0, None, fake, 0, 1, 1, 32, None) == L.NQ_BAD_SHAPE
    # unknown dtype / path
    assert lib.nq_linear_q8(fake, 7, fake, fake, None, fake, 0, 1, 4, 16, None) == L.NQ_BAD_ARG
    assert lib.nq_w8a8_acc_i32(fake, fake, fake, 1, 1, 16, None, 0, 9, None) == L.NQ_BAD_ARG
    # int32 overflow bound of the W8A8 core
    assert lib.nq_w8a8_acc_i32(fake, fake, fake, 1, 1, 200000, None, 0, 0, None) == L.NQ_BAD_SHAPE
    # misaligned fp32 pointer
    odd = ctypes.c_void_p(0x1001)
    assert lib.nq_linear_q8(odd, 0, fake, fake, None, fake, 0, 1, 4, 16, None) == L.NQ_BAD_ALIGN
    # null pointers
    assert lib.nq_linear_q8(None, 0, fake, fake, None, fake, 0, 1, 4, 16, None) == L.NQ_BAD_ARG
    # empty problems are no-ops
    assert lib.nq_linear_q8(None, 0, None, None, None, None, 0, 0, 4, 16, None) == L.NQ_OK


def test_w8a8_workspace_too_small(lib):
    from nanoinfer_amd import _lib as L
    fake = ctypes.c_void_p(0x1000)
    need = lib.nq_linear_w8a8_workspace_size(16, 1536, 1536)
    assert need >= 16 * 1536 + 16 * 4
    assert lib.nq_linear_w8a8(fake, 0, fake, fake, None, fake, 1, 16, 1536, 1536, fake, need - 1, 0,
                              None) == L.NQ_BAD_ARG
    assert b"workspace" in lib.nq_last_error()
    assert lib.nq_linear_w8a8_workspace_size(0, 5, 5) == 0


def test_weight_only_split_workspace_rules(lib):
    """The split-K linears need the planes nq_linear_wq_workspace_size gives
    (checked before any launch); shapes that do not split take none."""
    from nanoinfer_amd import _lib as L
    fake = ctypes.c_void_p(0x1000)
    need = lib.nq_linear_wq_workspace_size(64, 1536, 8960)
    assert need >= 2 * 64 * 1536 * 4 and need % 256 == 0
    assert lib.nq_linear_q8_ws(fake, 1, fake, fake, None, fake, 1, 64, 1536, 8960, fake, need - 256,
                               None) == L.NQ_BAD_ARG
    assert b"workspace" in lib.nq_last_error()
    assert lib.nq_linear_q4g_ws(fake, 1, fake, fake, 1, 32, None, fake, 1, 64, 1536, 8960, None, 0,
                                None) == L.NQ_BAD_ARG
    odd = ctypes.c_void_p(0x1010)
    assert lib.nq_linear_q8_ws(fake, 1, fake, fake, None, fake, 1, 64, 1536, 8960, odd, need,
                               None) == L.NQ_BAD_ALIGN
    # decode-sized m and short K with a full grid: no planes
    assert lib.nq_linear_wq_workspace_size(1, 1536, 8960) == 0
    assert lib.nq_linear_wq_workspace_size(8, 1536, 8960) == 0
    assert lib.nq_linear_wq_workspace_size(12, 1536, 8960) > 0     # m = 9..15: split wide tiles
    assert lib.nq_linear_wq_workspace_size(12, 896, 4864) == 0     # small weight: GEMV slices
    assert lib.nq_linear_wq_workspace_size(64, 1536, 1536) == 0
    assert lib.nq_linear_wq_workspace_size(0, 1536, 8960) == 0
    assert lib.nq_linear_q8_ws(fake, 1, fake, fake, None, fake, 1, 0, 1536, 8960, None, 0, None) == L.NQ_OK


def test_embedding_rejects_out_of_range_id(lib):
    from nanoinfer_amd import _lib as L
    fake = ctypes.c_void_p(0x1000)
    ids = np.array([0, 3], np.int64)                                     # test_quant.cpp:403-411
    st = lib.nq_embedding_q8(fake, fake, 3, 4, ids.ctypes.data_as(ctypes.c_void_p), 2, fake, 0, None)
    assert st == L.NQ_BAD_ARG and b"out of range" in lib.nq_last_error()


def test_check_maps_to_value_error():
    from nanoinfer_amd import _lib as L
    L.load().nq_linear_q8(None, 0, None, None, None, None, 0, -1, 1, 1, None)
    with pytest.raises(ValueError):
        L.check(L.NQ_BAD_SHAPE)
    with pytest.raises(RuntimeError):
        L.check(L.NQ_HIP_ERROR)


def test_workspace_sizes_all_shapes():
    """Workspace queries are defined for every shape, including K shorter than
    one MFMA slab (a division by zero once hid there) and m on either side of
    the skinny / prefill boundary."""
    from nanoinfer_amd import _lib
    lib = _lib.load()
    for m in (1, 3, 8, 64, 65, 130, 512, 2048):
        for n in (1, 65, 256, 8960):
            for k in (0, 1, 16, 48, 64, 1536, 8960):
                g = lib.nq_gemm_w8a8_workspace_size(m, n, k)
                lw = lib.nq_linear_w8a8_workspace_size(m, n, k)
                assert g % 256 == 0 and lw >= g


def test_weight_only_path_validation(lib):
    """nq_linear_q8_ex / nq_linear_q4g_ex: an unknown path, and a forced MFMA
    path whose operand contract fails (k % 32 != 0, a Q4G group that is not
    32 * 2^j, x not 16-byte aligned), are refused before any launch."""
    from nanoinfer_amd import _lib as L
    fake = ctypes.c_void_p(0x1000)
    assert lib.nq_linear_q8_ex(fake, 1, fake, fake, None, fake, 1, 1, 64, 64, None, 0, 7, None) == L.NQ_BAD_ARG
    assert b"unknown path" in lib.nq_last_error()
    assert lib.nq_linear_q8_ex(fake, 1, fake, fake, None, fake, 1, 1, 64, 48, None, 0, L.NQ_PATH_MFMA,
                               None) == L.NQ_BAD_ARG
    assert b"MFMA path" in lib.nq_last_error()
    x16 = ctypes.c_void_p(0x1008)                     # fp16-aligned, not 16-byte aligned
    assert lib.nq_linear_q8_ex(x16, 1, fake, fake, None, fake, 1, 1, 64, 64, None, 0, L.NQ_PATH_MFMA,
                               None) == L.NQ_BAD_ARG
    assert lib.nq_linear_q4g_ex(fake, 1, fake, fake, 1, 96, None, fake, 1, 1, 64, 192, None, 0, L.NQ_PATH_MFMA,
                                None) == L.NQ_BAD_ARG
    assert lib.nq_linear_q4g_ex(fake, 1, fake, fake, 1, 32, None, fake, 1, 1, 64, 64, None, 0, -1,
                                None) == L.NQ_BAD_ARG
    # the split-K workspace rule holds on every path
    need = lib.nq_linear_wq_workspace_size(64, 1536, 8960)
    assert lib.nq_linear_q8_ex(fake, 1, fake, fake, None, fake, 1, 64, 1536, 8960, fake, need - 256,
                               L.NQ_PATH_GEMV, None) == L.NQ_BAD_ARG
