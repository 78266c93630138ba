"""The nicpp seam on the host: module imports, QuantMode / quant_mode / Format
surface of the reference binding (cpp/bindings/nicpp.cpp:51-76), backend device
validation. No device work."""
import pytest


@pytest.fixture(scope="module")
def nicpp():
    from nanoinfer_amd import nicpp
    return nicpp


def test_quant_mode_surface(nicpp):
    assert nicpp.quant_mode("w8a8") == nicpp.QuantMode.W8A8
    assert nicpp.quant_mode("q4g") == nicpp.QuantMode.Q4G
    assert nicpp.quant_mode("fp32") == nicpp.QuantMode.NONE
    assert set(nicpp.QuantMode.__members__) == {"NONE", "Q8", "Q4", "Q4G", "W8A8"}
    with pytest.raises(ValueError):
        nicpp.quant_mode("int3")


def test_format_names(nicpp):
    F = nicpp.Format
    assert [nicpp.format_name(f) for f in (F.F32, F.F16, F.Q8, F.Q4, F.Q4G, F.W8A8)] == \
        ["f32", "f16", "q8", "q4", "q4g", "w8a8"]


def test_backend_device_validation(nicpp):
    assert nicpp.make_backend("hip").device == "hip"
    with pytest.raises(ValueError):
        nicpp.make_backend("cuda")


def test_python_mirror_surface():
    """nanoinfer_amd.quant mirrors the reference's enums and factory names."""
    from nanoinfer_amd import quant as nq
    assert nq.quant_mode("w8a8") == nq.QuantMode.W8A8
    assert nq.format_name(nq.Format.Q4G) == "q4g"
    for name in ("quantize_q8", "quantize_q4g", "quantize_q4", "linear_q8", "linear_w8a8", "linear_q4g",
                 "linear_q4", "embedding_q8", "make_quantized", "make_q8_embed", "act_quant"):
        assert callable(getattr(nq, name))
