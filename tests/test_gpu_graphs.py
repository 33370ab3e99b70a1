"""Graph replay of whole forwards (ebh_set_graph_replay): the second call with
a shape and set of buffers records the forward as a HIP graph, later calls
replay it.  Every replay must equal the direct launches bit for bit, with the
inputs rewritten in place, other GPU work and synchronisations between
replays, through workspace growth, a bad id, and the host, device and scoring
entry points."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def env():
    import torch
    import edgebert_amd
    assert torch.cuda.is_available(), "gpu tests need a GPU"
    edgebert_amd.lib()
    return torch, edgebert_amd


def _inputs(eb, cfg, B, S, lo, seed):
    ids, mask, _ = eb.make_inputs(eb.synth.InputSpec("g", cfg, B, S, lo, S, seed))
    return ids.astype(np.int32), mask.astype(np.int32)


def _pair(eb, weights, cfg, dtype):
    on = eb.Model.from_weights(weights, cfg, dtype)
    off = eb.Model.from_weights(weights, cfg, dtype)
    off.set_graph_replay(False)
    return on, off


def _other_work(torch):
    """Unrelated eager GPU work between replays."""
    a = torch.randn(512, 512, device="cuda")
    (a @ a).sum().item()


@pytest.mark.parametrize("cname,B,S,lo,dtype", [("c1", 2, 8, 8, "fp32"), ("c2", 32, 128, 8, "fp32"),
                                                 ("c2", 8, 64, 4, "bf16")])
def test_device_replays_equal_direct_launches(env, weights_for, cname, B, S, lo, dtype):
    torch, eb = env
    cfg = eb.CONFIGS[cname].model
    on, off = _pair(eb, weights_for(cfg), cfg, dtype)
    H = cfg.hidden_size
    d_ids = torch.zeros((B, S), dtype=torch.int32, device="cuda")
    d_mask = torch.zeros((B, S), dtype=torch.int32, device="cuda")
    out_on = torch.full((B, H), float("nan"), device="cuda")
    out_off = torch.full((B, H), float("nan"), device="cuda")
    for k in range(6):        # call 1 direct, call 2 records, calls 3.. replay
        ids, mask = _inputs(eb, cfg, B, S, lo, seed=100 + k)
        d_ids.copy_(torch.from_numpy(ids))
        d_mask.copy_(torch.from_numpy(mask))
        torch.cuda.synchronize()
        on.encode_device(d_ids.data_ptr(), d_mask.data_ptr(), B, S, out_on.data_ptr(), normalize=k % 2 == 0)
        on.synchronize()
        off.encode_device(d_ids.data_ptr(), d_mask.data_ptr(), B, S, out_off.data_ptr(), normalize=k % 2 == 0)
        off.synchronize()
        _other_work(torch)
        assert torch.equal(out_on, out_off), f"call {k}"
        # the replayed result is that input's, not a stale one
        want = on.encode_ids(ids.astype(np.uint32), mask.astype(np.uint32), normalize=k % 2 == 0)
        assert np.array_equal(out_on.cpu().numpy(), want), f"call {k}"
    on.close()
    off.close()


def test_host_path_replays_through_workspace_growth(env, weights_for):
    """ebh_encode (pinned staging): the same small shape before and after a
    larger batch grows the workspace (which drops the recordings)."""
    torch, eb = env
    cfg = eb.MINILM_L6
    on, off = _pair(eb, weights_for(cfg), cfg, "fp32")
    shapes = [(4, 16), (4, 16), (4, 16), (64, 128), (4, 16), (4, 16), (4, 16), (64, 128), (64, 128)]
    for k, (B, S) in enumerate(shapes):
        ids, mask = _inputs(eb, cfg, B, S, max(2, S // 4), seed=200 + k)
        a = on.encode_ids(ids.astype(np.uint32), mask.astype(np.uint32), normalize=True)
        b = off.encode_ids(ids.astype(np.uint32), mask.astype(np.uint32), normalize=True)
        _other_work(torch)
        assert np.array_equal(a, b), f"call {k} shape {(B, S)}"
    on.close()
    off.close()


def test_bad_id_is_reported_under_replay(env, weights_for):
    """The device-side id check still fires on a replayed forward, and the
    next good replay clears it."""
    torch, eb = env
    cfg = eb.MINILM_L6
    on = eb.Model.from_weights(weights_for(cfg), cfg, "fp32")
    B, S = 2, 8
    d_ids = torch.zeros((B, S), dtype=torch.int32, device="cuda")
    d_mask = torch.ones((B, S), dtype=torch.int32, device="cuda")
    out = torch.empty((B, cfg.hidden_size), device="cuda")
    ids, _ = _inputs(eb, cfg, B, S, S, seed=7)
    for _ in range(3):
        d_ids.copy_(torch.from_numpy(ids))
        on.encode_device(d_ids.data_ptr(), d_mask.data_ptr(), B, S, out.data_ptr())
        on.synchronize()
    bad = ids.copy()
    bad[1, 3] = cfg.vocab_size
    d_ids.copy_(torch.from_numpy(bad))
    on.encode_device(d_ids.data_ptr(), d_mask.data_ptr(), B, S, out.data_ptr())
    with pytest.raises(eb.EbhError):
        on.synchronize()
    d_ids.copy_(torch.from_numpy(ids))
    on.encode_device(d_ids.data_ptr(), d_mask.data_ptr(), B, S, out.data_ptr())
    on.synchronize()
    on.close()


def test_scores_replay(env, weights_for):
    """Cross-encoder scoring, host and device entry points, replayed."""
    torch, eb = env
    cfg = eb.MINILM_L6
    w = dict(weights_for(cfg))
    rng = np.random.default_rng(3)
    w["classifier.weight"] = (0.05 * rng.standard_normal((1, cfg.hidden_size))).astype(np.float32)
    w["classifier.bias"] = np.array([0.1], np.float32)
    on, off = _pair(eb, w, cfg, "fp32")
    B, S = 6, 40
    d_ids = torch.zeros((B, S), dtype=torch.int32, device="cuda")
    d_mask = torch.zeros((B, S), dtype=torch.int32, device="cuda")
    s_on = torch.empty(B, device="cuda")
    s_off = torch.empty(B, device="cuda")
    for k in range(5):
        ids, mask = _inputs(eb, cfg, B, S, 5, seed=300 + k)
        a = on.score_ids(ids.astype(np.uint32), mask.astype(np.uint32))
        b = off.score_ids(ids.astype(np.uint32), mask.astype(np.uint32))
        assert np.array_equal(a, b), f"host call {k}"
        d_ids.copy_(torch.from_numpy(ids))
        d_mask.copy_(torch.from_numpy(mask))
        on.score_device(d_ids.data_ptr(), d_mask.data_ptr(), B, S, s_on.data_ptr())
        off.score_device(d_ids.data_ptr(), d_mask.data_ptr(), B, S, s_off.data_ptr())
        on.synchronize()
        off.synchronize()
        _other_work(torch)
        assert torch.equal(s_on, s_off), f"device call {k}"
        assert np.array_equal(s_on.cpu().numpy(), a), f"device call {k}"
    on.close()
    off.close()


def test_replay_toggles_and_profiling_runs_direct(env, weights_for):
    """Turning replay off and on, and profiling a kernel family (which runs the
    launches directly), keep results equal."""
    torch, eb = env
    cfg = eb.MINILM_L6
    m = eb.Model.from_weights(weights_for(cfg), cfg, "fp32")
    ids, mask = _inputs(eb, cfg, 3, 24, 6, seed=9)
    ref = m.encode_ids(ids.astype(np.uint32), mask.astype(np.uint32))
    for k in range(3):
        assert np.array_equal(m.encode_ids(ids.astype(np.uint32), mask.astype(np.uint32)), ref)
    m.set_graph_replay(False)
    assert np.array_equal(m.encode_ids(ids.astype(np.uint32), mask.astype(np.uint32)), ref)
    m.set_graph_replay(True)
    m.profile_enable("gemm_ffn_up")
    for k in range(3):
        assert np.array_equal(m.encode_ids(ids.astype(np.uint32), mask.astype(np.uint32)), ref)
    launches, _ = m.profile_read()
    assert launches == 3 * cfg.num_hidden_layers
    m.profile_enable("none")
    for k in range(3):
        assert np.array_equal(m.encode_ids(ids.astype(np.uint32), mask.astype(np.uint32)), ref)
    m.close()
