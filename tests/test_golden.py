"""The oracle and the synthetic generator reproduce the committed golden
fixtures (tests/golden/encoder_golden.npz, written by make_golden.py after a
cross-check against transformers.BertModel)."""
import os

import numpy as np
import pytest

import oracle
from edgebert_amd import synth

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "encoder_golden.npz")


@pytest.fixture(scope="module")
def g():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def test_generator_matches_golden(g, weights_for):
    assert synth.weights_sha256(weights_for(synth.MINILM_L6)) == g["minilm_weights_sha256"].tobytes().hex()
    assert synth.weights_sha256(weights_for(synth.TINY)) == g["tiny_weights_sha256"].tobytes().hex()
    ids, mask, _ = synth.make_inputs(synth.CONFIGS["c1"])
    np.testing.assert_array_equal(ids, g["c1_ids"])
    np.testing.assert_array_equal(mask, g["c1_mask"])
    ids, mask, _ = synth.make_inputs(synth.CONFIGS["c2"])
    np.testing.assert_array_equal(ids[:8], g["c2_ids"])
    np.testing.assert_array_equal(mask[:8], g["c2_mask"])


def test_oracle_matches_golden(g, weights_for):
    om = oracle.OracleModel(synth.MINILM_L6, weights_for(synth.MINILM_L6))
    np.testing.assert_allclose(om.encode(g["c1_ids"], g["c1_mask"]), g["c1_out"], rtol=0, atol=1e-6)
    np.testing.assert_allclose(om.forward(g["c1_ids"], g["c1_mask"]), g["c1_pooled"], rtol=0, atol=1e-6)
    np.testing.assert_allclose(om.encode(g["c2_ids"], g["c2_mask"]), g["c2_out"], rtol=0, atol=1e-6)
    omt = oracle.OracleModel(synth.TINY, weights_for(synth.TINY))
    pooled, trace = omt.forward_trace(g["tiny_ids"].astype(np.float32), g["tiny_mask"].astype(np.float32))
    np.testing.assert_allclose(pooled, g["tiny_pooled"], rtol=0, atol=1e-6)
    np.testing.assert_allclose(trace, g["tiny_trace"], rtol=0, atol=1e-6)


def test_planted_mistake_is_caught(g, weights_for):
    """A plausible oracle mistake (LayerNorm gamma and beta swapped in one
    layer) moves the output far outside the tolerance the fixtures are checked at."""
    w = dict(weights_for(synth.MINILM_L6))
    p = "encoder.layer.3.attention.output.LayerNorm."
    w[p + "weight"], w[p + "bias"] = w[p + "bias"], w[p + "weight"]
    out = oracle.OracleModel(synth.MINILM_L6, w).encode(g["c1_ids"], g["c1_mask"])
    assert np.abs(out - g["c1_out"]).max() > 1e-3
