"""GPU: the C++ host layer (its own C++ test executable) and the nicpp module
against the oracle."""
import os
import subprocess

import numpy as np
import pytest

from conftest import ROOT
from gpu_util import assert_close_rms

pytestmark = pytest.mark.gpu


def test_cpp_host_test_binary(dev):
    exe = os.path.join(ROOT, "tests", "cpp", "test_host.bin")
    assert os.path.exists(exe), "build() compiles tests/cpp/test_host.bin"
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0 and "test_host: ok" in r.stdout, r.stdout + r.stderr


@pytest.mark.parametrize("mode", ["q8", "w8a8", "q4g", "q4"])
def test_nicpp_weights_vs_oracle(dev, orc, mode):
    from nanoinfer_amd import nicpp
    be = nicpp.make_backend("hip")
    rng = np.random.default_rng(3)
    w = rng.normal(0, 0.02, (96, 256)).astype(np.float32)
    x = rng.normal(0, 1, (4, 256)).astype(np.float32)
    b = rng.normal(0, 1, 96).astype(np.float32)
    wt = be.make_quant_weight(w, nicpp.quant_mode(mode))
    y = wt.linear(x, b)
    if mode in ("q8", "w8a8"):
        q, s = orc.quantize_q8(w)
        ref = orc.linear_q8(x, q, s, b) if mode == "q8" else orc.linear_w8a8(x, q, s, b)
    elif mode == "q4g":
        q, s = orc.quantize_q4g(w, 32)
        ref = orc.linear_q4g(x, q, s, 32, b)
    else:
        q, s = orc.quantize_q4(w)
        ref = orc.linear_q4(x, q, s, b)
    assert_close_rms(y, ref, f"nicpp {mode}")
    assert nicpp.format_name(wt.format()) == mode
    assert wt.fp32_bytes() == 96 * 256 * 4 and wt.bytes() < wt.fp32_bytes()


def test_nicpp_embed_and_errors(dev, orc):
    from nanoinfer_amd import nicpp
    be = nicpp.make_backend("hip")
    rng = np.random.default_rng(4)
    table = rng.normal(0, 1, (50, 64)).astype(np.float32)
    emb = be.make_embed_weight(table)
    q, s = orc.quantize_q8(table)
    assert np.array_equal(emb.gather([0, 49, 7]), orc.embedding_q8(q, s, [0, 49, 7]))
    with pytest.raises(ValueError):
        emb.gather([50])                                            # quant.cpp:127
    wt = be.make_quant_weight(table, nicpp.QuantMode.Q8)
    with pytest.raises(RuntimeError):
        wt.gather([0])                                              # quant.cpp:473-475
    with pytest.raises(ValueError):
        wt.linear(np.zeros((2, 63), np.float32))                    # x cols must match
    assert be.make_quant_weight(table, nicpp.QuantMode.NONE) is None


@pytest.mark.parametrize("mode", ["w8a8", "q4g"])
def test_nicpp_load_quant_weight(dev, tmp_path, mode):
    """A weight loaded from a NIT1 bf16 file equals make_quant_weight of the
    same values (quantize-on-load, serialize.cpp:11-72)."""
    from nanoinfer_amd import nicpp
    from nit_util import bf16_exact, write_nit1
    be = nicpp.make_backend("hip")
    rng = np.random.default_rng(9)
    w = bf16_exact(rng.normal(0, 0.02, (96, 256)).astype(np.float32))
    x = rng.normal(0, 1, (3, 256)).astype(np.float32)
    p = str(tmp_path / "w.bin")
    write_nit1(p, w, 1)
    a = be.load_quant_weight(p, nicpp.quant_mode(mode))
    b = be.make_quant_weight(w, nicpp.quant_mode(mode))
    assert nicpp.format_name(a.format()) == mode
    assert np.array_equal(a.linear(x), b.linear(x))
    with pytest.raises(RuntimeError):
        be.load_quant_weight(str(tmp_path / "missing.bin"), nicpp.quant_mode(mode))
