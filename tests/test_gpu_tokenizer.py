"""Texts -> vectors / scores through the native tokenizer and the GPU forward
(ebh_encode_texts, ebh_score_texts): the same results as the ids the HF
``tokenizers`` library (the reference's tokenizer) produces, run through the
id entry points."""
import numpy as np
import pytest

from test_tokenizer import build, sentences

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def eb():
    import torch
    import edgebert_amd
    assert torch.cuda.is_available(), "gpu tests need a GPU"
    return edgebert_amd


def test_encode_texts_gives_the_workload_ids_and_vectors(eb, weights_for):
    """c2 spelled as words of the synthetic vocabulary: the texts tokenise back
    to the workload's ids, and ebh_encode_texts equals ebh_encode on them."""
    from edgebert_amd import synth
    spec = eb.CONFIGS["c2"]
    ids, mask, lengths = eb.make_inputs(spec)
    tok = eb.Tokenizer.from_str(synth.tokenizer_json(spec.model))
    texts = synth.make_texts(ids, lengths)
    t_ids, t_mask = tok.encode_batch_ids(texts)
    S = t_ids.shape[1]
    assert np.array_equal(t_ids, ids[:, :S]) and np.array_equal(t_mask, mask[:, :S])
    m = eb.Model.from_weights(weights_for(spec.model), spec.model, "fp32", tokenizer=tok)
    got = m.encode_texts(texts, True)
    want = m.encode_ids(ids, mask, normalize=True)
    assert np.array_equal(got, want)
    assert np.array_equal(m.encode_texts(texts, True, nthreads=1), got)


def test_native_and_hf_tokenizers_give_the_same_vectors(eb, weights_for, tmp_path):
    """Mixed-script text (accents, CJK, punctuation, control characters, a
    literal [SEP]) through Model.encode with either tokenizer."""
    from edgebert_amd.tokenizer import Tokenizer, hf_tokenizer
    path = build(tmp_path)
    texts = sentences(64, seed=5)
    w = weights_for(eb.MINILM_L6)
    native = eb.Model.from_weights(w, eb.MINILM_L6, "fp32", tokenizer=Tokenizer.from_file(path))
    hf = eb.Model.from_weights(w, eb.MINILM_L6, "fp32", tokenizer=hf_tokenizer(path))
    a = np.array(native.encode(texts, True))
    b = np.array(hf.encode(texts, True))
    assert np.array_equal(a, b)


def test_score_texts_matches_hf_tokenised_pairs(eb, weights_for, tmp_path):
    """Cross-encoder scoring from text pairs ("q [SEP] d", src/lib.rs:331)."""
    from edgebert_amd.tokenizer import Tokenizer, hf_encode_batch_ids, hf_tokenizer
    path = build(tmp_path)
    w = dict(weights_for(eb.MINILM_L6))
    rng = np.random.default_rng(0)
    w["classifier.weight"] = (0.05 * rng.standard_normal((1, 384))).astype(np.float32)
    w["classifier.bias"] = np.array([0.1], np.float32)
    qs, ds = sentences(24, seed=8), sentences(24, seed=9)
    m = eb.Model.from_weights(w, eb.MINILM_L6, "fp32", tokenizer=Tokenizer.from_file(path))
    got = np.array(m.score_batch(list(zip(qs, ds))), np.float32)
    ids, mask = hf_encode_batch_ids(hf_tokenizer(path), [f"{q} [SEP] {d}" for q, d in zip(qs, ds)])
    want = m.score_ids(ids.astype(np.uint32), mask.astype(np.uint32))
    assert np.array_equal(got, want)
    assert m.score_pair(qs[3], ds[3]) == pytest.approx(float(got[3]), abs=2e-6)


def test_encode_batch_runs_sub_batches_concurrently_with_the_same_results(eb, weights_for):
    """encode_batch (src/lib.rs:438-450) over sub-batches on two host threads:
    every vector equal to its sub-batch encoded alone."""
    from edgebert_amd import synth
    spec = eb.CONFIGS["c2"]
    ids, mask, lengths = eb.make_inputs(spec)
    tok = eb.Tokenizer.from_str(synth.tokenizer_json(spec.model))
    texts = synth.make_texts(ids, lengths)
    subs = [texts[0:10], texts[10:11], texts[11:32]]
    m = eb.Model.from_weights(weights_for(spec.model), spec.model, "fp32", tokenizer=tok)
    alone = [m.encode_texts(b, True) for b in subs]
    many = m.encode_texts_many(subs, True, workers=2)
    for a, b in zip(alone, many):
        assert np.array_equal(a, b)
    lists = m.encode_batch(subs, True, workers=2)
    for a, b in zip(alone, lists):
        assert np.array_equal(a, np.array(b, np.float32))
