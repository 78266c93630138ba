"""The CPU reference decoder used for greedy-token parity: the oracle's quant
path and the reference's own quant.cpp build give the same tokens."""
import pytest

from model_ref import RefModel

PROMPT = [3, 17, 42, 7, 99, 5, 250, 11]


@pytest.mark.parametrize("mode", ["w8a8", "q8", "q4g"])
def test_ref_model_oracle_matches_reference_build(orc, mode):
    import oracle
    from nanoinfer_amd.model import Config, random_weights
    ref = oracle.reference()
    if ref is None:
        pytest.skip("reference build (oracle/_ref) not present")
    cfg = Config(hidden=256, heads=4, kv_heads=2, head_dim=64, intermediate=512, layers=2, vocab=1024,
                 max_pos=64, tie_embeddings=False)
    w = random_weights(cfg, 0)
    a = RefModel(orc, cfg, w, mode)
    b = RefModel(ref, cfg, w, mode)
    assert a.generate(PROMPT, 8) == b.generate(PROMPT, 8)
