"""NIT0 / NIT1 weight files on the host: nq_nit_info accepts the reference's
formats and rejects exactly load_bin's malformed cases (cpp/tests/test_io.cpp:51-112)."""
import os

import numpy as np
import pytest

from nit_util import write_nit0, write_nit1


def test_info_nit0_nit1(nq, tmp_path):
    p0, p1, p2 = str(tmp_path / "a.bin"), str(tmp_path / "b.bin"), str(tmp_path / "c.bin")
    write_nit0(p0, np.arange(6, dtype=np.float32).reshape(2, 3))
    write_nit1(p1, np.array([1.0, -2.5, 0.0], np.float32), 1)       # test_io.cpp:68-84
    write_nit1(p2, np.zeros((4, 5, 6), np.float32), 0)
    assert nq.nit_info(p0) == (0, (2, 3))
    assert nq.nit_info(p1) == (1, (3,))
    assert nq.nit_info(p2) == (0, (4, 5, 6))
    with open(p1, "rb") as f:                                         # payload bits 0x3F80, 0xC020, 0x0000
        assert f.read()[-6:] == bytes([0x80, 0x3F, 0x20, 0xC0, 0x00, 0x00])


def _raw(path, *parts):
    with open(path, "wb") as f:
        for p in parts:
            f.write(p if isinstance(p, bytes) else np.asarray(p).tobytes())


def test_info_rejects_malformed(nq, tmp_path):
    from nanoinfer_amd._lib import NQ_IO_ERROR, NqError
    cases = {
        "trailing": (b"NIT0", np.int32([2, 2, 3]), np.zeros(6, np.float32), b"\0"),     # test_io.cpp:58-66
        "dtype": (b"NIT1", np.int32([7, 1, 1]), np.float32([1.0])),                      # :86-98
        "short_bf16": (b"NIT1", np.int32([1, 1, 4]), np.uint16([0x3F80, 0x3F80])),       # :100-112
        "magic": (b"NIT2", np.int32([1, 1]), np.float32([0.0])),
        "neg_ndim": (b"NIT0", np.int32([-1])),
        "neg_dim": (b"NIT0", np.int32([2, 3, -1])),
        "short_header": (b"NIT0", np.int32([3, 2])),
        "short_fp32": (b"NIT0", np.int32([1, 3]), np.float32([1.0, 2.0])),
    }
    for name, parts in cases.items():
        p = str(tmp_path / f"{name}.bin")
        _raw(p, *parts)
        with pytest.raises(NqError) as e:
            nq.nit_info(p)
        assert e.value.status == NQ_IO_ERROR, name
    with pytest.raises(NqError) as e:
        nq.nit_info(str(tmp_path / "missing.bin"))
    assert e.value.status == NQ_IO_ERROR
    assert not os.path.exists(str(tmp_path / "missing.bin"))
