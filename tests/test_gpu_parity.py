"""Parity of the HIP path (through the C ABI) with the CPU oracle.

Bars: token ids bit-exact; fp32 max-abs embedding
difference <= 1e-4 and cosine >= 0.99999 per sequence against the oracle's
run of that sequence alone, unpadded; bf16 GEMMs cosine >= 0.999.
"""
import numpy as np
import pytest

from conftest import cosine_rows

pytestmark = pytest.mark.gpu

FP32_MAX_ABS = 1e-4
FP32_MIN_COS = 0.99999
BF16_MIN_COS = 0.999


@pytest.fixture(scope="module")
def eb():
    import edgebert_amd
    edgebert_amd.lib()
    return edgebert_amd


@pytest.fixture(scope="module")
def oracle_mod():
    import oracle
    return oracle


_MODELS = {}


def gpu_model(eb, cfg, weights, dtype="fp32"):
    key = (cfg, dtype)
    if key not in _MODELS:
        _MODELS[key] = eb.Model.from_weights(weights, cfg, dtype)
    return _MODELS[key]


def _report(name, got, want):
    err = float(np.abs(got - want).max())
    cos = float(cosine_rows(got, want).min())
    print(f"{name}: max_abs={err:.3e} min_cos={cos:.9f}", flush=True)
    return err, cos


@pytest.mark.parametrize("cname", ["c1", "c2", "c4"])
def test_encode_matches_unpadded_oracle(eb, oracle_mod, weights_for, cname):
    spec = eb.CONFIGS[cname]
    w = weights_for(spec.model)
    ids, mask, lengths = eb.make_inputs(spec)
    m = gpu_model(eb, spec.model, w)
    got = m.encode_ids(ids, mask, normalize=True)
    want = oracle_mod.OracleModel(spec.model, w).encode_unpadded(ids, mask, normalize=True)
    err, cos = _report(f"{cname} encode vs unpadded oracle", got, want)
    assert err <= FP32_MAX_ABS and cos >= FP32_MIN_COS
    tok, pos, cu = m.last_tokens(spec.batch)
    assert np.array_equal(tok, ids[mask != 0]), "token ids reaching the GPU differ"
    assert np.array_equal(pos, np.nonzero(mask)[1].astype(np.int32))
    assert np.array_equal(cu, np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32))


@pytest.mark.parametrize("cname", ["c2", "c3", "c4"])
def test_split_product_gemms_match_unpadded_oracle(eb, oracle_mod, weights_for, cname):
    """An EBH_DTYPE_F32_BF16X6 model (fp32 GEMM products from six bf16 MFMA
    products) holds the fp32 bars against the oracle's unpadded run (c3: a
    16-sequence subsample of the full batch)."""
    spec = eb.CONFIGS[cname]
    w = weights_for(spec.model)
    ids, mask, lengths = eb.make_inputs(spec)
    m = gpu_model(eb, spec.model, w, "fp32-bf16x6")
    got = m.encode_ids(ids, mask, normalize=True)
    sel = np.arange(spec.batch) if cname != "c3" else np.arange(5, spec.batch, spec.batch // 16)[:16]
    want = oracle_mod.OracleModel(spec.model, w).encode_unpadded(ids[sel], mask[sel], normalize=True)
    err, cos = _report(f"{cname} fp32-bf16x6 vs unpadded oracle", got[sel], want)
    assert err <= FP32_MAX_ABS and cos >= FP32_MIN_COS


@pytest.mark.parametrize("cname", ["c1", "c2"])
def test_forward_matches_padded_oracle(eb, oracle_mod, weights_for, cname):
    """Model::forward on the reference's f32 arrays vs the oracle's padded run."""
    spec = eb.CONFIGS[cname]
    w = weights_for(spec.model)
    ids, mask, _ = eb.make_inputs(spec)
    m = gpu_model(eb, spec.model, w)
    got = m.forward(ids.astype(np.float32), mask.astype(np.float32))
    want = oracle_mod.OracleModel(spec.model, w).forward(ids.astype(np.float32),
                                                         mask.astype(np.float32))
    err, cos = _report(f"{cname} forward vs padded oracle", got, want)
    assert err <= FP32_MAX_ABS and cos >= FP32_MIN_COS


def test_c3_every_sequence_and_properties(eb, oracle_mod, weights_for):
    """Headline shape (256 x 128): every sequence against the oracle, and
    size-independent properties over the whole batch."""
    spec = eb.CONFIGS["c3"]
    w = weights_for(spec.model)
    ids, mask, _ = eb.make_inputs(spec)
    m = gpu_model(eb, spec.model, w)
    got = m.encode_ids(ids, mask, normalize=True)
    assert np.isfinite(got).all()
    np.testing.assert_allclose(np.linalg.norm(got.astype(np.float64), axis=1), 1.0, atol=1e-5)
    want = oracle_mod.OracleModel(spec.model, w).encode(ids, mask, normalize=True)
    err, cos = _report("c3 all 256 sequences", got, want)
    assert err <= FP32_MAX_ABS and cos >= FP32_MIN_COS
    # batch-permutation equivariance: each row is computed independently of its slot
    perm = np.random.default_rng(0).permutation(spec.batch)
    got_p = m.encode_ids(ids[perm], mask[perm], normalize=True)
    assert np.array_equal(got_p, got[perm])
    # duplicated sentences give identical vectors (self-cosine 1, src/lib.rs:1255-1258)
    dup = np.repeat(ids[:4], 2, axis=0)
    got_d = m.encode_ids(dup, np.ones_like(dup), normalize=True)
    assert np.array_equal(got_d[0::2], got_d[1::2])


def test_large_ragged_batch_takes_the_fused_paths(eb, oracle_mod, weights_for):
    """512 sequences of 64..128 tokens: the grid is sized for 512 x 128 rows but
    only the packed tokens exist, so the wide-tile GEMMs and the fused
    GEMM + LayerNorm run with fewer real rows than their tiles cover (ragged
    last row block, descriptors ending at the packed count).  24 sequences
    against the oracle, all rows finite and unit-norm."""
    from edgebert_amd.synth import InputSpec, MINILM_L6, make_inputs
    spec = InputSpec("ragged512", MINILM_L6, 512, 128, 64, 128, 11)
    w = weights_for(spec.model)
    ids, mask, lengths = make_inputs(spec)
    assert 512 * 64 < int(mask.sum()) < 512 * 128
    m = gpu_model(eb, spec.model, w)
    got = m.encode_ids(ids, mask, normalize=True)
    assert np.isfinite(got).all()
    np.testing.assert_allclose(np.linalg.norm(got.astype(np.float64), axis=1), 1.0, atol=1e-5)
    sel = np.arange(0, spec.batch, spec.batch // 24)[:24]
    want = oracle_mod.OracleModel(spec.model, w).encode_unpadded(ids[sel], mask[sel], normalize=True)
    err, cos = _report("ragged 512 subsample", got[sel], want)
    assert err <= FP32_MAX_ABS and cos >= FP32_MIN_COS


def test_many_ragged_sequences_any_batch_order(eb, oracle_mod, weights_for):
    """1,500 sequences of 1..40 tokens: more sequences than the packing scan's
    workgroup has threads, so its length sort (the order the attention grid
    takes the sequences in) walks the batch in strides, with many equal
    lengths.  Every row unit-norm, 25 sequences against the oracle, and a
    permuted batch gives the permuted rows bit for bit (each sequence's vector
    depends on that sequence only, whichever workgroup computes it)."""
    from edgebert_amd.synth import InputSpec, MINILM_L6, make_inputs
    spec = InputSpec("ragged1500", MINILM_L6, 1500, 40, 1, 40, 5)
    w = weights_for(spec.model)
    ids, mask, lengths = make_inputs(spec)
    m = gpu_model(eb, spec.model, w)
    got = m.encode_ids(ids, mask, normalize=True)
    np.testing.assert_allclose(np.linalg.norm(got.astype(np.float64), axis=1), 1.0, atol=1e-5)
    sel = np.arange(0, spec.batch, spec.batch // 25)[:25]
    want = oracle_mod.OracleModel(spec.model, w).encode_unpadded(ids[sel], mask[sel], normalize=True)
    err, cos = _report("ragged 1500 subsample", got[sel], want)
    assert err <= FP32_MAX_ABS and cos >= FP32_MIN_COS
    perm = np.random.default_rng(3).permutation(spec.batch)
    got_p = m.encode_ids(np.ascontiguousarray(ids[perm]), np.ascontiguousarray(mask[perm]), normalize=True)
    assert np.array_equal(got_p, got[perm])


def test_bert_base_fp32_few_tokens_split_k(eb, oracle_mod, weights_for):
    """BERT-base in fp32 with 3 short sentences: the bias-free projections are
    split over K (6 splits at K = 768, 8 at K = 3072) into partial products
    that the LayerNorm sums in order."""
    from edgebert_amd.synth import InputSpec, BERT_BASE, make_inputs
    spec = InputSpec("bert_few", BERT_BASE, 3, 24, 5, 24, 12)
    w = weights_for(spec.model)
    ids, mask, _ = make_inputs(spec)
    got = gpu_model(eb, spec.model, w).encode_ids(ids, mask, normalize=True)
    want = oracle_mod.OracleModel(spec.model, w).encode_unpadded(ids, mask, normalize=True)
    err, cos = _report("BERT-base fp32 few tokens", got, want)
    assert err <= FP32_MAX_ABS and cos >= FP32_MIN_COS


def test_bf16_bert_base(eb, oracle_mod, weights_for):
    """c5 shape (BERT-base, head_dim 64) with bf16 GEMMs on a 24-sequence sample."""
    spec = eb.CONFIGS["c5"]
    w = weights_for(spec.model)
    ids, mask, _ = eb.make_inputs(spec)
    ids, mask = ids[:24], mask[:24]
    want = oracle_mod.OracleModel(spec.model, w).encode(ids, mask, normalize=True)
    m16 = gpu_model(eb, spec.model, w, "bf16")
    got16 = m16.encode_ids(ids, mask, normalize=True)
    _, cos16 = _report("c5 bf16 vs fp32 oracle", got16, want)
    assert cos16 >= BF16_MIN_COS
    m32 = gpu_model(eb, spec.model, w, "fp32")
    got32 = m32.encode_ids(ids, mask, normalize=True)
    err, cos = _report("c5-shape fp32 vs oracle", got32, want)
    assert err <= FP32_MAX_ABS and cos >= FP32_MIN_COS


def test_c5_full_batch_bf16(eb, oracle_mod, weights_for):
    """c5 at its configured size: BERT-base, 1024 x 128 tokens, bf16 GEMMs and
    attention with fp32 accumulation.  Every row finite and unit-norm; a batch
    permutation gives bit-identical rows; 64 sequences spread over the batch
    against the fp32 oracle (cosine >= 0.999 each)."""
    spec = eb.CONFIGS["c5"]
    assert (spec.batch, spec.seq_len) == (1024, 128)
    w = weights_for(spec.model)
    ids, mask, _ = eb.make_inputs(spec)
    m16 = gpu_model(eb, spec.model, w, "bf16")
    got = m16.encode_ids(ids, mask, normalize=True)
    assert got.shape == (1024, 768) and np.isfinite(got).all()
    np.testing.assert_allclose(np.linalg.norm(got.astype(np.float64), axis=1), 1.0, atol=1e-5)
    perm = np.random.default_rng(5).permutation(spec.batch)
    got_p = m16.encode_ids(ids[perm], mask[perm], normalize=True)
    assert np.array_equal(got_p, got[perm])
    sel = np.arange(3, spec.batch, spec.batch // 64)[:64]
    want = oracle_mod.OracleModel(spec.model, w).encode(ids[sel], mask[sel], normalize=True)
    _, cos = _report("c5 full batch bf16, 64 sequences vs fp32 oracle", got[sel], want)
    assert cos >= BF16_MIN_COS


@pytest.mark.parametrize("model_name,B,S,lo,hi", [
    ("minilm", 1, 1, 1, 1), ("minilm", 5, 12, 3, 12), ("minilm", 4, 16, 16, 16),
    ("minilm", 8, 8, 2, 8), ("minilm", 2, 8, 8, 8), ("minilm", 64, 1, 1, 1), ("minilm", 3, 21, 1, 21),
    ("bert", 2, 24, 9, 24)])
def test_few_token_forwards(eb, oracle_mod, weights_for, model_name, B, S, lo, hi):
    """At most 64 padded tokens: every projection takes the few-token GEMM
    kernel (16-row blocks, the bias-free ones split over K), over 1 to 4 row
    blocks with ragged last blocks; for MiniLM (heads of 32) attention and the
    output projection run as one launch writing a partial per head, summed by
    the one-row-per-workgroup LayerNorm (64 sequences of one token, a
    sequence of 21 beside ones of a single token).  Repeated calls (the later
    ones replayed as a HIP graph) give bit-identical vectors; each sequence
    matches the oracle's unpadded run."""
    from edgebert_amd.synth import InputSpec, MINILM_L6, BERT_BASE, make_inputs
    cfg = MINILM_L6 if model_name == "minilm" else BERT_BASE
    spec = InputSpec(f"few_{model_name}_{B}x{S}", cfg, B, S, lo, hi, 20 + B * S)
    w = weights_for(cfg)
    ids, mask, _ = make_inputs(spec)
    m = gpu_model(eb, cfg, w)
    got = m.encode_ids(ids, mask, normalize=True)
    for _ in range(3):
        assert np.array_equal(m.encode_ids(ids, mask, normalize=True), got)
    want = oracle_mod.OracleModel(cfg, w).encode_unpadded(ids, mask, normalize=True)
    err, cos = _report(f"few tokens {model_name} {B}x{S}", got, want)
    assert err <= FP32_MAX_ABS and cos >= FP32_MIN_COS


def test_bf16_minilm_padded(eb, oracle_mod, weights_for):
    """MiniLM shape (head_dim 32) with bf16 GEMMs and a bf16 residual stream, on
    the padded c2 batch: each sequence against the fp32 oracle's unpadded run."""
    spec = eb.CONFIGS["c2"]
    w = weights_for(spec.model)
    ids, mask, _ = eb.make_inputs(spec)
    got = gpu_model(eb, spec.model, w, "bf16").encode_ids(ids, mask, normalize=True)
    want = oracle_mod.OracleModel(spec.model, w).encode_unpadded(ids, mask, normalize=True)
    _, cos = _report("c2 MiniLM bf16 vs fp32 oracle", got, want)
    assert cos >= BF16_MIN_COS


@pytest.mark.parametrize("B,S,lo,hi", [(1, 1, 1, 1), (2, 8, 8, 8), (5, 12, 3, 12)])
def test_bf16_minilm_few_tokens(eb, oracle_mod, weights_for, B, S, lo, hi):
    """bf16 MiniLM at a handful of tokens: bf16 GEMM tiles far larger than the
    packed rows, a single ragged row block, and the bf16 pool's half-used
    second chunk (H = 384).  Each sequence against the fp32 oracle's unpadded
    run; repeated calls (graph replays) give bit-identical vectors."""
    from edgebert_amd.synth import InputSpec, MINILM_L6, make_inputs
    spec = InputSpec(f"few16_{B}x{S}", MINILM_L6, B, S, lo, hi, 40 + B * S)
    w = weights_for(MINILM_L6)
    ids, mask, _ = make_inputs(spec)
    m = gpu_model(eb, MINILM_L6, w, "bf16")
    got = m.encode_ids(ids, mask, normalize=True)
    for _ in range(2):
        assert np.array_equal(m.encode_ids(ids, mask, normalize=True), got)
    want = oracle_mod.OracleModel(MINILM_L6, w).encode_unpadded(ids, mask, normalize=True)
    _, cos = _report(f"bf16 MiniLM few tokens {B}x{S}", got, want)
    assert cos >= BF16_MIN_COS


@pytest.mark.parametrize("B,lo", [(64, 128), (96, 128), (128, 8)])
def test_mid_size_batches_match_oracle(eb, oracle_mod, weights_for, B, lo):
    """MiniLM batches of 8k-16k padded positions, dense or ragged, through the
    host-buffer entry point (too few 128-row blocks for the fused GEMM +
    LayerNorm, so the kernels are the device path's): FFN up (and at 96 x 128
    the QKV projection) on 128 x
    96 tiles in place of the wide ones; the attention-output and FFN-down
    products split on 128 x 96 tiles (64 x 128), or on 128 x 128 tiles (96 x
    128, 128 x 128); fewer sequences than CUs, so the pool sums 32-row chunks;
    packing in one workgroup (64 x 128) or in three kernels.  16 sequences
    against the oracle's unpadded run; every row unit-norm."""
    from edgebert_amd.synth import InputSpec, MINILM_L6, make_inputs
    spec = InputSpec(f"mid{B}", MINILM_L6, B, 128, lo, 128, 90 + B)
    w = weights_for(MINILM_L6)
    ids, mask, _ = make_inputs(spec)
    got = gpu_model(eb, MINILM_L6, w).encode_ids(ids, mask, normalize=True)
    np.testing.assert_allclose(np.linalg.norm(got.astype(np.float64), axis=1), 1.0, atol=1e-5)
    sel = np.arange(1, B, B // 16)[:16]
    want = oracle_mod.OracleModel(MINILM_L6, w).encode_unpadded(ids[sel], mask[sel], normalize=True)
    err, cos = _report(f"MiniLM {B}x128 (lengths {lo}-128)", got[sel], want)
    assert err <= FP32_MAX_ABS and cos >= FP32_MIN_COS


def test_ragged_large_batch_host_path(eb, oracle_mod, weights_for):
    """256 sentences of 8..128 tokens padded to 128 through the host-buffer
    entry point: the host counts the packed rows (about half of B*S), too few
    128-row blocks for the fused GEMM + LayerNorm, so the attention-output and
    FFN-down products take the split path sized for the real rows.  16
    sequences against the oracle's unpadded run; every row unit-norm."""
    from edgebert_amd.synth import InputSpec, MINILM_L6, make_inputs
    spec = InputSpec("ragged256", MINILM_L6, 256, 128, 8, 128, 77)
    w = weights_for(MINILM_L6)
    ids, mask, _ = make_inputs(spec)
    assert int(mask.sum()) < 256 * 128 // 2 + 4096
    got = gpu_model(eb, MINILM_L6, w).encode_ids(ids, mask, normalize=True)
    np.testing.assert_allclose(np.linalg.norm(got.astype(np.float64), axis=1), 1.0, atol=1e-5)
    sel = np.arange(0, 256, 16)
    want = oracle_mod.OracleModel(MINILM_L6, w).encode_unpadded(ids[sel], mask[sel], normalize=True)
    err, cos = _report("ragged 256 host path", got[sel], want)
    assert err <= FP32_MAX_ABS and cos >= FP32_MIN_COS
