"""The no-allocation entry point (ebh_encode_device_noalloc) through the C ABI,
against the allocating ebh_encode_device on the same inputs: two calls in a
row, the second smaller, bit-identical results (the same kernels with the same
arguments, only the workspace differs); sizes beyond the static scratch are
rejected; no device memory is taken; the id-range flag is reported by
ebh_synchronize of the model that raised it, and of no other.  Passes alone in
a fresh process and after the other tests."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def env(weights_for):
    import torch
    import edgebert_amd as eb
    from edgebert_amd import _native as N, synth
    assert torch.cuda.is_available(), "gpu tests need a GPU"
    w = weights_for(synth.MINILM_L6)
    return torch, eb, N, synth, w


def _dev_inputs(torch, synth, spec):
    ids, mask, _ = synth.make_inputs(spec)
    return (torch.from_numpy(ids.astype(np.int32)).cuda(), torch.from_numpy(mask.astype(np.int32)).cuda())


def _noalloc(N, m, ids, mask, B, S, out, stream, normalize=1):
    return N.lib().ebh_encode_device_noalloc(m._h, ctypes.c_void_p(ids.data_ptr()), ctypes.c_void_p(mask.data_ptr()),
                                             B, S, normalize, ctypes.c_void_p(out.data_ptr()),
                                             ctypes.c_void_p(stream))


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
def test_noalloc_matches_encode_device_two_calls(env, dtype):
    torch, eb, N, synth, w = env
    cfg = synth.MINILM_L6
    m = eb.Model.from_weights(w, cfg, dtype)
    s = torch.cuda.current_stream().cuda_stream
    try:
        specs = [synth.CONFIGS["c2"], synth.InputSpec("small", cfg, 5, 24, 3, 24, 31)]
        for spec in specs:                     # the second call is smaller than the first
            B, S = spec.batch, spec.seq_len
            ids, mask = _dev_inputs(torch, synth, spec)
            want = torch.full((B, cfg.hidden_size), float("nan"), device="cuda")
            got = torch.full((B, cfg.hidden_size), float("nan"), device="cuda")
            m.set_graph_replay(False)
            m.encode_device(ids.data_ptr(), mask.data_ptr(), B, S, want.data_ptr(), True, s)
            N.check(_noalloc(N, m, ids, mask, B, S, got, s))
            m.synchronize()
            assert torch.isfinite(got).all()
            assert torch.equal(got, want), f"{spec.name}: max diff {(got - want).abs().max().item()}"
    finally:
        m.close()


def test_noalloc_takes_no_device_memory_and_rejects_large_batches(env):
    torch, eb, N, synth, w = env
    cfg = synth.MINILM_L6
    s = torch.cuda.current_stream().cuda_stream
    spec = synth.CONFIGS["c2"]
    B, S = spec.batch, spec.seq_len
    ids, mask = _dev_inputs(torch, synth, spec)
    out = torch.empty((B, cfg.hidden_size), device="cuda")
    warm = eb.Model.from_weights(w, cfg, "fp32")   # every kernel launched once before measuring
    warm.encode_device(ids.data_ptr(), mask.data_ptr(), B, S, out.data_ptr(), True, s)
    warm.synchronize()
    m = eb.Model.from_weights(w, cfg, "fp32")      # has never run a forward: no workspace yet
    try:
        torch.cuda.synchronize()
        free0, _ = torch.cuda.mem_get_info()
        for _ in range(3):
            N.check(_noalloc(N, m, ids, mask, B, S, out, s))
        m.synchronize()
        free1, _ = torch.cuda.mem_get_info()
        # the allocating entry point would take its 66 MB workspace here
        assert free0 - free1 < 8 << 20, (free0, free1)
        big = synth.CONFIGS["c3"]
        bids, bmask = _dev_inputs(torch, synth, big)
        bout = torch.empty((big.batch, cfg.hidden_size), device="cuda")
        rc = _noalloc(N, m, bids, bmask, big.batch, big.seq_len, bout, s)
        assert rc == N.EBH_ERR_RANGE
        assert "static scratch" in N.last_error()
    finally:
        m.close()
        warm.close()


def test_noalloc_reports_bad_ids_on_synchronize(env):
    torch, eb, N, synth, w = env
    cfg = synth.MINILM_L6
    s = torch.cuda.current_stream().cuda_stream
    m = eb.Model.from_weights(w, cfg, "fp32")
    try:
        ids = torch.full((3, 40), 101, dtype=torch.int32, device="cuda")
        mask = torch.ones_like(ids)
        out = torch.empty((3, cfg.hidden_size), device="cuda")
        bad = ids.clone()
        bad[2, 5] = cfg.vocab_size + 7
        N.check(_noalloc(N, m, bad, mask, 3, 40, out, s))
        N.check(_noalloc(N, m, ids, mask, 3, 40, out, s))    # a clean call after it: still reported
        with pytest.raises(eb.EbhError, match="out of range"):
            m.synchronize()
        N.check(_noalloc(N, m, ids, mask, 3, 40, out, s))
        m.synchronize()
        assert torch.isfinite(out).all()
    finally:
        m.close()


def test_noalloc_bad_id_is_reported_by_its_own_model_only(env):
    """Two models: a bad id in model a's no-allocation forward is reported by
    a's ebh_synchronize, not by b's (b's own forwards are clean), and b's
    results are those of a clean run.  The two forwards share the device's
    scratch array, so they must not overlap: each model runs on its own
    stream here, and the device is synchronised between them."""
    torch, eb, N, synth, w = env
    cfg = synth.MINILM_L6
    s = torch.cuda.current_stream().cuda_stream
    a = eb.Model.from_weights(w, cfg, "fp32")
    b = eb.Model.from_weights(w, cfg, "fp32")
    try:
        ids = torch.full((2, 24), 101, dtype=torch.int32, device="cuda")
        mask = torch.ones_like(ids)
        bad = ids.clone()
        bad[1, 3] = cfg.vocab_size + 11
        out_a = torch.empty((2, cfg.hidden_size), device="cuda")
        out_b = torch.empty((2, cfg.hidden_size), device="cuda")
        want = torch.empty((2, cfg.hidden_size), device="cuda")
        b.set_graph_replay(False)
        b.encode_device(ids.data_ptr(), mask.data_ptr(), 2, 24, want.data_ptr(), True, s)
        b.synchronize()
        N.check(_noalloc(N, a, bad, mask, 2, 24, out_a, s))
        torch.cuda.synchronize()                             # a's forward done, its flag raised
        N.check(_noalloc(N, b, ids, mask, 2, 24, out_b, s))
        b.synchronize()                                      # clean: a's flag is not b's
        assert torch.equal(out_b, want)
        with pytest.raises(eb.EbhError, match="out of range"):
            a.synchronize()
        a.synchronize()                                      # reported once, then cleared
    finally:
        a.close()
        b.close()
