"""Cross-encoder scoring (Model::score_pair / score_batch, src/lib.rs:327-399)
through the C ABI (ebh_score, ebh_score_device) against the CPU oracle's
restatement: the pooled forward row dotted with classifier.weight plus
classifier.bias, each pair run alone and unpadded on the CPU."""
import json

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

# Scores are dot products of pooled rows (|x| ~ 1) with a N(0, 0.02) weight:
# fp32 embedding parity (<= 1e-4 per element) bounds them well inside this.
SCORE_MAX_ABS = 1e-4


@pytest.fixture(scope="module")
def eb():
    import edgebert_amd
    edgebert_amd.lib()
    return edgebert_amd


def _head(H, seed=11):
    rng = np.random.default_rng(seed)
    return {"classifier.weight": (0.02 * rng.standard_normal((1, H))).astype(np.float32),
            "classifier.bias": np.array([0.125], np.float32)}


def _pair_inputs(eb, cfg, B, seed):
    """[CLS] query [SEP] document [SEP] encodings of random lengths, zero-padded."""
    spec = eb.synth.InputSpec("pairs", cfg, B, 96, 6, 96, seed)
    ids, mask, _ = eb.make_inputs(spec)
    return ids, mask


@pytest.fixture(scope="module")
def minilm(eb, weights_for):
    cfg = eb.CONFIGS["c2"].model
    w = {**weights_for(cfg), **_head(cfg.hidden_size)}
    m = eb.Model.from_weights(w, cfg)
    yield cfg, w, m
    m.close()


def test_scores_match_oracle_per_pair(eb, minilm):
    import oracle
    cfg, w, m = minilm
    ids, mask = _pair_inputs(eb, cfg, 16, 5)
    got = m.score_ids(ids, mask)
    om = oracle.OracleModel(cfg, w)
    want = np.array([om.score(ids[b][mask[b] != 0][None, :], mask[b][mask[b] != 0][None, :])[0]
                     for b in range(ids.shape[0])], np.float32)
    err = float(np.abs(got - want).max())
    print(f"cross-encoder scores vs oracle: max_abs={err:.3e} (|score| max {np.abs(want).max():.3f})")
    assert err <= SCORE_MAX_ABS


def test_batch_equals_each_pair_alone(eb, minilm):
    """score_batch runs every pair in one padded batch; the reference scores them
    one by one (src/lib.rs:381-383).  Each pair's score must not depend on the
    others."""
    cfg, w, m = minilm
    ids, mask = _pair_inputs(eb, cfg, 12, 9)
    batched = m.score_ids(ids, mask)
    alone = np.array([m.score_ids(ids[b][mask[b] != 0][None, :], mask[b][mask[b] != 0][None, :])[0]
                      for b in range(ids.shape[0])], np.float32)
    np.testing.assert_allclose(batched, alone, rtol=0, atol=1e-5)


def test_device_entry_point(eb, minilm):
    import torch
    cfg, w, m = minilm
    ids, mask = _pair_inputs(eb, cfg, 8, 3)
    want = m.score_ids(ids, mask)
    d_ids = torch.from_numpy(ids.astype(np.int32)).cuda()
    d_mask = torch.from_numpy(mask.astype(np.int32)).cuda()
    d_out = torch.full((ids.shape[0],), float("nan"), device="cuda")
    torch.cuda.synchronize()
    m.score_device(d_ids.data_ptr(), d_mask.data_ptr(), ids.shape[0], ids.shape[1], d_out.data_ptr())
    m.synchronize()
    np.testing.assert_allclose(d_out.cpu().numpy(), want, rtol=0, atol=1e-6)


def test_head_errors(eb, weights_for):
    from edgebert_amd import _native as N
    cfg = eb.synth.TINY
    w = weights_for(cfg)
    H = cfg.hidden_size
    plain = eb.Model.from_weights(w, cfg)
    ids = np.array([[101, 1000, 102]], np.uint32)
    with pytest.raises(N.EbhError) as e:
        plain.score_ids(ids, np.ones_like(ids))
    assert e.value.code == N.EBH_ERR_STATE and "not a cross-encoder" in str(e.value)
    plain.close()
    for name, arr, code in [("classifier.weight", np.zeros((2, H), np.float32), N.EBH_ERR_SHAPE),
                            ("classifier.weight", np.zeros(H + 1, np.float32), N.EBH_ERR_SHAPE),
                            ("classifier.bias", np.zeros(2, np.float32), N.EBH_ERR_SHAPE)]:
        with pytest.raises(N.EbhError) as e:
            eb.Model.from_weights({**w, **_head(H), name: arr}, cfg)
        assert e.value.code == code
    with pytest.raises(N.EbhError) as e:       # the pair is required together
        eb.Model.from_weights({**w, "classifier.weight": np.zeros(H, np.float32)}, cfg)
    assert e.value.code == N.EBH_ERR_NOT_FOUND and "classifier.bias" in str(e.value)
    # [H] (the reference's get_array1) and [1, H] (checkpoint layout) score alike
    m1 = eb.Model.from_weights({**w, **_head(H)}, cfg)
    h = _head(H)
    m2 = eb.Model.from_weights({**w, "classifier.weight": h["classifier.weight"].reshape(H),
                                "classifier.bias": h["classifier.bias"]}, cfg)
    np.testing.assert_array_equal(m1.score_ids(ids, np.ones_like(ids)), m2.score_ids(ids, np.ones_like(ids)))
    m1.close()
    m2.close()


def test_safetensors_cross_encoder(eb, tmp_path, weights_for):
    """model.safetensors with a classifier head loads it; scores equal those of
    the same tensors handed over one by one."""
    from safetensors.numpy import save_file
    cfg = eb.synth.TINY
    w = {**weights_for(cfg), **_head(cfg.hidden_size, seed=4)}
    save_file({k: np.ascontiguousarray(v) for k, v in w.items()}, str(tmp_path / "model.safetensors"))
    with open(tmp_path / "config.json", "w") as f:
        json.dump({"hidden_size": cfg.hidden_size, "num_attention_heads": cfg.num_attention_heads,
                   "num_hidden_layers": cfg.num_hidden_layers, "intermediate_size": cfg.intermediate_size,
                   "vocab_size": cfg.vocab_size, "max_position_embeddings": cfg.max_position_embeddings,
                   "layer_norm_eps": cfg.layer_norm_eps, "hidden_act": "gelu", "model_type": "bert"}, f)
    m1 = eb.Model.from_pretrained_path(str(tmp_path))
    m2 = eb.Model.from_weights(w, cfg)
    ids, mask, _ = eb.make_inputs(eb.synth.InputSpec("t", cfg, 5, 20, 3, 20, 4))
    np.testing.assert_array_equal(m1.score_ids(ids, mask), m2.score_ids(ids, mask))
    m1.close()
    m2.close()
