"""Quantize-on-load from NIT0 / NIT1 files: codes and scales equal the oracle's
quantize of load_bin's fp32 tensor bit for bit (fp32 and bf16 payloads, several
upload chunks, odd in-features), and the fp32 loader inflates bf16 exactly
(cpp/tests/test_io.cpp:68-84)."""
import numpy as np
import pytest
import torch

from gpu_util import host, to_dev
from nit_util import bf16_exact, write_nit0, write_nit1

pytestmark = pytest.mark.gpu


def test_load_f32_exact(dev, nq, tmp_path):
    p = str(tmp_path / "b.bin")
    write_nit1(p, np.array([1.0, -2.5, 0.0], np.float32), 1)
    assert host(nq.load_nit(p)).tolist() == [1.0, -2.5, 0.0]
    a = np.random.default_rng(1).normal(0, 1, (33, 7)).astype(np.float32)
    write_nit0(p, a)
    assert np.array_equal(host(nq.load_nit(p)), a)
    write_nit1(p, a, 1)
    assert np.array_equal(host(nq.load_nit(p)), bf16_exact(a))


@pytest.mark.parametrize("fmt", ["nit0", "nit1_f32", "nit1_bf16"])
def test_load_q8_matches_oracle(dev, nq, orc, tmp_path, fmt):
    w = np.random.default_rng(5).normal(0, 0.02, (300, 896)).astype(np.float32)
    w[7] = 0.0                                        # all-zero row -> scale 0
    p = str(tmp_path / "w.bin")
    if fmt == "nit0":
        write_nit0(p, w)
    else:
        write_nit1(p, w, 1 if fmt == "nit1_bf16" else 0)
        if fmt == "nit1_bf16":
            w = bf16_exact(w)
    t = nq.load_nit_q8(p)
    q, s = orc.quantize_q8(w)
    assert np.array_equal(host(t.q), q) and np.array_equal(host(t.scale), s)


@pytest.mark.parametrize("k,group,sdt", [(1536, 32, torch.float16), (1001, 64, torch.float32)])
def test_load_q4g_matches_oracle(dev, nq, orc, tmp_path, k, group, sdt):
    w = bf16_exact(np.random.default_rng(k).normal(0, 0.02, (130, k)).astype(np.float32))
    p = str(tmp_path / "w.bin")
    write_nit1(p, w, 1)
    t = nq.load_nit_q4g(p, group, scale_dtype=sdt)
    ref = nq.quantize_q4g(to_dev(w, dev), group, scale_dtype=sdt)   # device quantizer, oracle-pinned elsewhere
    assert torch.equal(t.q, ref.q) and torch.equal(t.scale, ref.scale)
    q, s = orc.quantize_q4g(w, group)
    assert np.array_equal(host(t.q), q)


@pytest.mark.parametrize("dtype", [0, 1])
def test_load_q8_several_chunks(dev, nq, tmp_path, dtype):
    """> 64 MiB of payload: two upload chunks through both pinned buffers."""
    rows, k = 9000, 2048 if dtype == 0 else 4096
    g = torch.Generator(device=dev).manual_seed(11)
    wd = torch.randn((rows, k), generator=g, device=dev) * 0.02
    w = host(wd)
    if dtype == 1:
        w = bf16_exact(w)
    p = str(tmp_path / "big.bin")
    write_nit1(p, w, dtype)
    t = nq.load_nit_q8(p)
    ref = nq.quantize_q8(to_dev(w, dev))
    assert torch.equal(t.q, ref.q) and torch.equal(t.scale, ref.scale)


def test_shape_and_file_errors(dev, nq, tmp_path):
    from nanoinfer_amd._lib import NqError
    p = str(tmp_path / "v.bin")
    write_nit0(p, np.zeros(5, np.float32))
    with pytest.raises(ValueError):
        nq.load_nit_q8(p)                              # 1-D: not a [out, in] weight
    with pytest.raises(NqError):
        nq.load_nit(str(tmp_path / "missing.bin"))
