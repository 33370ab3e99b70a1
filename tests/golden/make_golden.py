"""Writes the golden fixtures of the encoder path into tests/golden/.

The reference publishes no numeric vectors that can be used offline (its
README values need the real all-MiniLM-L6-v2 checkpoint and tokenizer), so
the fixtures are made here from the deterministic synthetic models and
inputs, by the CPU oracle, and each is cross-checked before it is written
against an independent implementation of the same encoder
(``transformers.BertModel``, tanh GELU, eager attention) to 1e-5.

Run from the repo root:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(HERE))

import oracle  # noqa: E402
from edgebert_amd import synth  # noqa: E402
from test_oracle import hf_encode  # noqa: E402


def check(name, got, want, atol=1e-5):
    err = float(np.abs(got - want).max())
    print(f"{name}: max |oracle - transformers| = {err:.3e}")
    if not err <= atol:
        raise SystemExit(f"{name}: oracle and transformers disagree ({err})")


def main():
    out = {}
    # c1: MiniLM-L6 shape, batch 2 x 8 tokens.
    spec = synth.CONFIGS["c1"]
    w = synth.make_weights(spec.model)
    ids, mask, _ = synth.make_inputs(spec)
    om = oracle.OracleModel(spec.model, w)
    c1 = om.encode(ids, mask, normalize=True)
    check("c1", c1, hf_encode(spec.model, w, ids, mask))
    out.update(c1_ids=ids, c1_mask=mask, c1_out=c1, c1_pooled=om.forward(ids, mask))
    out["minilm_weights_sha256"] = np.frombuffer(bytes.fromhex(synth.weights_sha256(w)), np.uint8)

    # c2 first 8 sequences: padded, key-padding mask.
    spec = synth.CONFIGS["c2"]
    ids, mask, _ = synth.make_inputs(spec)
    ids, mask = ids[:8], mask[:8]
    c2 = om.encode(ids, mask, normalize=True)
    check("c2[:8]", c2, hf_encode(spec.model, w, ids, mask))
    out.update(c2_ids=ids, c2_mask=mask, c2_out=c2)

    # tiny shape: hidden state after every layer of a padded batch.
    cfg = synth.TINY
    wt = synth.make_weights(cfg)
    spec = synth.InputSpec("tiny", cfg, 4, 16, 1, 16, 7)
    ids, mask, _ = synth.make_inputs(spec)
    omt = oracle.OracleModel(cfg, wt)
    pooled, trace = omt.forward_trace(ids.astype(np.float32), mask.astype(np.float32))
    want, hs = hf_encode(cfg, wt, ids, mask, normalize=False, hidden_states=True)
    check("tiny pooled", pooled, want)
    for i, h in enumerate(hs):
        check(f"tiny hidden {i}", trace[i], h, atol=5e-5)
    out.update(tiny_ids=ids, tiny_mask=mask, tiny_pooled=pooled, tiny_trace=trace)
    out["tiny_weights_sha256"] = np.frombuffer(bytes.fromhex(synth.weights_sha256(wt)), np.uint8)

    path = os.path.join(HERE, "encoder_golden.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
