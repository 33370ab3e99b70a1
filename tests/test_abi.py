"""The C ABI of libedgebert_hip.so without a GPU: the library loads, exports
every function include/*.h declares, and validates on the host (config,
tensor names and shapes, safetensors parsing, arguments) before any HIP call.

Error behaviour follows the reference: a missing tensor is "Tensor <name> not
found" (src/weights.rs:51), a 2-D tensor where a 1-D one is expected is
"Expected 1D tensor" (src/weights.rs:53-57), a shape mismatch is a shape
error (src/weights.rs:67-68).
"""
import ctypes
import json
import struct
import threading

import numpy as np
import pytest

import edgebert_amd as eb
from edgebert_amd import _native as N
from edgebert_amd import synth
from edgebert_amd.model import _cfg_struct


def _gpu_visible() -> bool:
    import torch
    return torch.cuda.device_count() > 0


@pytest.fixture(scope="module")
def L():
    return eb.lib()


def _create(L, cfg=synth.TINY):
    h = ctypes.c_void_p()
    cs = _cfg_struct(cfg)
    rc = L.ebh_create(ctypes.byref(cs), ctypes.byref(h))
    return rc, h


def _set(L, h, name, arr):
    a = np.ascontiguousarray(arr, np.float32)
    shape = (ctypes.c_int64 * max(a.ndim, 1))(*a.shape)
    return L.ebh_set_tensor(h, name.encode(), ctypes.c_void_p(a.ctypes.data), shape, a.ndim)


def test_exports_every_header_symbol(L):
    names = eb.header_symbols()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing


def test_header_symbols_have_bindings():
    assert set(eb.header_symbols()) == set(N._SIGS)


@pytest.mark.parametrize("field,value,msg", [
    ("hidden_size", 100, "multiple of num_attention_heads"),
    ("num_attention_heads", 8, "head_dim 48"),
    ("hidden_size", 0, "positive"),
    ("vocab_size", -1, "positive"),
    ("hidden_size", 4096, "above the supported"),
    ("intermediate_size", 1001, "multiples of 8"),
])
def test_create_rejects_bad_config(L, field, value, msg):
    import dataclasses
    cfg = dataclasses.replace(synth.MINILM_L6, **{field: value})
    if field == "hidden_size" and value == 4096:
        cfg = dataclasses.replace(cfg, num_attention_heads=64)
    rc, h = _create(L, cfg)
    assert rc == N.EBH_ERR_INVALID_ARG
    assert msg in N.last_error()
    assert not h.value


def test_set_tensor_validation(L):
    rc, h = _create(L)
    assert rc == N.EBH_OK
    try:
        H = synth.TINY.hidden_size
        assert _set(L, h, "embeddings.nonsense", np.zeros(H)) == N.EBH_ERR_NOT_FOUND
        assert "unknown tensor" in N.last_error()
        rc = _set(L, h, "encoder.layer.0.attention.self.query.bias", np.zeros((1, H)))
        assert rc == N.EBH_ERR_SHAPE and "Expected 1D tensor" in N.last_error()
        rc = _set(L, h, "encoder.layer.0.intermediate.dense.weight", np.zeros((H, 256)))
        assert rc == N.EBH_ERR_SHAPE and "expected [256, 64]" in N.last_error()
        assert _set(L, h, "encoder.layer.0.intermediate.dense.weight", np.zeros((256, H))) == N.EBH_OK
        assert L.ebh_set_tensor(h, None, None, None, 0) == N.EBH_ERR_INVALID_ARG
    finally:
        L.ebh_destroy(h)


def test_finalize_reports_missing_tensor(L, weights_for):
    rc, h = _create(L)
    try:
        for name, arr in weights_for(synth.TINY).items():
            if name != "encoder.layer.1.output.LayerNorm.bias":
                assert _set(L, h, name, arr) == N.EBH_OK
        assert L.ebh_finalize(h, N.EBH_DTYPE_F32) == N.EBH_ERR_NOT_FOUND
        assert N.last_error() == "Tensor encoder.layer.1.output.LayerNorm.bias not found"
        assert L.ebh_finalize(h, 7) == N.EBH_ERR_INVALID_ARG
    finally:
        L.ebh_destroy(h)


def test_calls_before_finalize_fail(L):
    rc, h = _create(L)
    try:
        ids = np.zeros((1, 4), np.float32)
        out = np.zeros((1, synth.TINY.hidden_size), np.float32)
        p = lambda a: ctypes.c_void_p(a.ctypes.data)
        assert L.ebh_forward(h, p(ids), p(ids), 1, 4, p(out)) == N.EBH_ERR_STATE
        assert "not finalized" in N.last_error()
        assert L.ebh_encode(h, p(ids), p(ids), 1, 4, 1, p(out)) == N.EBH_ERR_STATE
        assert L.ebh_synchronize(h) == N.EBH_ERR_STATE
        assert L.ebh_forward(None, p(ids), p(ids), 1, 4, p(out)) == N.EBH_ERR_INVALID_ARG
    finally:
        L.ebh_destroy(h)
    L.ebh_destroy(None)  # no-op


def test_last_error_is_thread_local(L):
    msgs = {}

    def worker(tag, field):
        import dataclasses
        cfg = dataclasses.replace(synth.TINY, **{field: 0})
        _create(L, cfg)
        msgs[tag] = N.last_error()

    t = threading.Thread(target=worker, args=("t", "vocab_size"))
    t.start()
    t.join()
    rc, h = _create(L)
    L.ebh_destroy(h)
    assert msgs["t"] and "positive" in msgs["t"]


def test_op_entry_points_validate_before_launch(L):
    nul = None
    assert L.ebh_op_gemm(nul, 4, nul, 4, 0, nul, nul, 0, nul, 4, 1, 1, 4, 0, nul) == N.EBH_ERR_INVALID_ARG
    buf = np.zeros(64, np.float32)
    p = ctypes.c_void_p(buf.ctypes.data)
    # K not a multiple of 4, unknown epilogue, residual epilogue without a residual
    assert L.ebh_op_gemm(p, 6, p, 6, 0, p, nul, 0, p, 4, 1, 4, 6, 0, nul) == N.EBH_ERR_INVALID_ARG
    assert L.ebh_op_gemm(p, 4, p, 4, 0, p, nul, 0, p, 4, 1, 4, 4, 9, nul) == N.EBH_ERR_INVALID_ARG
    assert L.ebh_op_gemm(p, 4, p, 4, 0, p, nul, 0, p, 4, 1, 4, 4, 2, nul) == N.EBH_ERR_INVALID_ARG
    assert L.ebh_op_attention(p, p, 1, 8, 96, 2, p, nul) == N.EBH_ERR_INVALID_ARG  # head_dim 48
    assert L.ebh_op_layer_norm(p, p, p, 1, 4096, 1e-12, p, nul) == N.EBH_ERR_INVALID_ARG
    assert L.ebh_op_add_layer_norm(p, nul, p, p, p, 1, 64, 1e-12, nul) == N.EBH_ERR_INVALID_ARG
    assert L.ebh_op_gemm(p, 4, p, 4, 0, nul, nul, 0, p, 4, 1, 4, 4, 0, nul) == N.EBH_ERR_INVALID_ARG  # bias needed
    assert L.ebh_op_pool(p, p, -1, 64, 4, 1, p, p, nul) == N.EBH_ERR_INVALID_ARG
    if buf.ctypes.data % 16 == 0:   # S > 32: the chunk sums need a partials buffer
        assert L.ebh_op_pool(p, p, 1, 64, 64, 1, nul, p, nul) == N.EBH_ERR_INVALID_ARG
    assert L.ebh_op_pack(p, p, -1, 4, p, p, p, p, p, p, nul) == N.EBH_ERR_INVALID_ARG
    assert L.ebh_op_f32_to_bf16(p, p, -1, nul) == N.EBH_ERR_INVALID_ARG


def test_gemm_ops_reject_strides_past_32bit_lane_offsets(L):
    """The persistent GEMM kernels address a k-tile load as a per-tile base plus
    a 32-bit lane offset of up to 384 rows of a stride: the bf16 op and the
    fused LayerNorm op refuse strides whose offsets would wrap, naming them,
    before any launch (fp32 ebh_op_gemm runs such strides on its guarded
    64-bit kernel instead)."""
    buf = np.zeros(256, np.float32)
    base = buf.ctypes.data
    p = ctypes.c_void_p(base + (-base) % 16)
    nul = None
    max16, max32 = 5_592_405, 2_796_202
    assert (max16 + 1) * 384 * 2 + 64 * 2 > 2 ** 32 >= max16 * 384 * 2 + 64 * 2
    assert (max32 + 1) * 384 * 4 + 64 * 4 > 2 ** 32 >= max32 * 384 * 4 + 64 * 4
    big16 = max16 + 3          # the next multiple of 8
    rc = L.ebh_op_gemm_bf16(p, big16, p, 64, p, p, 256, 1, 1, 256, 64, 0, nul)
    assert rc == N.EBH_ERR_INVALID_ARG and "too large" in N.last_error()
    rc = L.ebh_op_gemm_bf16(p, 64, p, big16, p, p, 256, 1, 1, 256, 64, 0, nul)
    assert rc == N.EBH_ERR_INVALID_ARG and "too large" in N.last_error()
    big32 = max32 + 2          # the next multiple of 4
    rc = L.ebh_op_gemm_add_layer_norm(p, big32, p, 32, p, p, p, p, 1, 384, 32, 1e-12, nul)
    assert rc == N.EBH_ERR_INVALID_ARG and "too large" in N.last_error()
    rc = L.ebh_op_gemm_add_layer_norm(p, 32, p, big32, p, p, p, p, 1, 384, 32, 1e-12, nul)
    assert rc == N.EBH_ERR_INVALID_ARG and "too large" in N.last_error()


# ---------------------------------------------------------------------------
# safetensors (ModelWeights::load, src/weights.rs:15-45)
# ---------------------------------------------------------------------------
def _write_safetensors(path, tensors, dtype_override=None, raw_header=None):
    """Minimal writer: 8-byte LE header length, JSON header, raw data."""
    header, blobs, off = {"__metadata__": {"format": "pt"}}, [], 0
    for name, (dt, arr) in tensors.items():
        data = arr.tobytes()
        header[name] = {"dtype": dt, "shape": list(arr.shape), "data_offsets": [off, off + len(data)]}
        blobs.append(data)
        off += len(data)
    h = raw_header if raw_header is not None else json.dumps(header).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)


def _load(L, path):
    rc, h = _create(L)
    assert rc == N.EBH_OK
    rc = L.ebh_load_safetensors(h, str(path).encode())
    return rc, h


def test_safetensors_loads_every_tensor(L, tmp_path, weights_for):
    w = weights_for(synth.TINY)
    t = {k: ("F32", v) for k, v in w.items()}
    t["pooler.dense.weight"] = ("F32", np.zeros((4, 4), np.float32))            # skipped
    t["embeddings.position_ids"] = ("I64", np.arange(64, dtype=np.int64)[None])  # skipped
    # half-precision tensors are widened exactly
    t["embeddings.LayerNorm.weight"] = ("F16", w["embeddings.LayerNorm.weight"].astype(np.float16))
    bf = (w["encoder.layer.0.output.dense.bias"].view(np.uint32) >> 16).astype(np.uint16)
    t["encoder.layer.0.output.dense.bias"] = ("BF16", bf)
    p = tmp_path / "model.safetensors"
    _write_safetensors(p, t)
    rc, h = _load(L, p)
    try:
        assert rc == N.EBH_OK, N.last_error()
        if _gpu_visible():
            pytest.skip("finalize would allocate on the GPU; covered by the gpu tests")
        # every tensor arrived: finalize gets past the completeness check to its first HIP call
        rc = L.ebh_finalize(h, N.EBH_DTYPE_F32)
        assert rc == N.EBH_ERR_HIP, (rc, N.last_error())
    finally:
        L.ebh_destroy(h)


@pytest.mark.parametrize("case,code,msg", [
    ("missing_file", N.EBH_ERR_NOT_FOUND, "cannot open"),
    ("bad_json", N.EBH_ERR_SHAPE, "bad header JSON"),
    ("bad_dtype", N.EBH_ERR_SHAPE, "unsupported dtype I32"),
    ("bad_offsets", N.EBH_ERR_SHAPE, "bad data_offsets"),
    ("neg_shape", N.EBH_ERR_SHAPE, "bad shape"),
    ("wrong_shape", N.EBH_ERR_SHAPE, "Shape error"),
    ("truncated", N.EBH_ERR_SHAPE, "truncated"),
])
def test_safetensors_errors(L, tmp_path, case, code, msg):
    p = tmp_path / "m.safetensors"
    H = synth.TINY.hidden_size
    name = "embeddings.LayerNorm.bias"
    if case == "bad_json":
        _write_safetensors(p, {}, raw_header=b"{not json")
    elif case == "bad_dtype":
        _write_safetensors(p, {name: ("I32", np.zeros(H, np.int32))})
    elif case == "bad_offsets":
        hdr = json.dumps({name: {"dtype": "F32", "shape": [H], "data_offsets": [0, 4 * H + 8]}}).encode()
        with open(p, "wb") as f:
            f.write(struct.pack("<Q", len(hdr)) + hdr + b"\0" * (4 * H))
    elif case == "neg_shape":
        hdr = json.dumps({name: {"dtype": "F32", "shape": [-H], "data_offsets": [0, 4 * H]}}).encode()
        with open(p, "wb") as f:
            f.write(struct.pack("<Q", len(hdr)) + hdr + b"\0" * (4 * H))
    elif case == "wrong_shape":
        _write_safetensors(p, {"encoder.layer.0.output.dense.weight": ("F32", np.zeros((H, H), np.float32))})
    elif case == "truncated":
        with open(p, "wb") as f:
            f.write(struct.pack("<Q", 1000) + b"{}")
    if case == "missing_file":
        p = tmp_path / "absent.safetensors"
    rc, h = _load(L, p)
    L.ebh_destroy(h)
    assert rc == code, (rc, N.last_error())
    assert msg in N.last_error()


# ---------------------------------------------------------------------------
# host-side mirror of the reference API (no GPU calls)
# ---------------------------------------------------------------------------
def test_cosine_similarity_mirror():
    a = np.arange(1, 10, dtype=np.float32)
    assert abs(eb.cosine_similarity(a, a) - 1.0) < 1e-6
    b = a[::-1].copy()
    assert abs(eb.cosine_similarity(a, b) - eb.cosine_similarity(b, a)) < 1e-7


def test_synthetic_generator_is_deterministic():
    w1 = synth.make_weights(synth.TINY)
    w2 = synth.make_weights(synth.TINY)
    assert synth.weights_sha256(w1) == synth.weights_sha256(w2)
    x = w1["encoder.layer.0.intermediate.dense.weight"].astype(np.float64)
    assert abs(x.mean()) < 1e-3 and abs(x.std() - 0.02) < 1e-3
    assert (w1["embeddings.LayerNorm.weight"] == 1).all() and (w1["embeddings.LayerNorm.bias"] == 0).all()
    # splitmix64 known answers: seed 0 gives 0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4
    r = synth.splitmix64(0, np.arange(2, dtype=np.uint64))
    assert [int(v) for v in r] == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4]
    # FNV-1a 64 known answer: "a" -> 0xaf63dc4c8601ec8c
    assert synth.fnv1a64("a") == 0xAF63DC4C8601EC8C


@pytest.mark.parametrize("cname", list(synth.CONFIGS))
def test_input_layout(cname):
    """[CLS] ids... [SEP] then pad 0 / mask 0 (src/lib.rs:588-601)."""
    spec = synth.CONFIGS[cname]
    ids, mask, lengths = synth.make_inputs(spec)
    B, S = ids.shape
    assert (B, S) == (spec.batch, spec.seq_len)
    assert ((lengths >= spec.len_lo) & (lengths <= spec.len_hi)).all()
    assert (ids[:, 0] == synth.CLS_ID).all()
    assert (ids[np.arange(B), lengths - 1] == synth.SEP_ID).all()
    for b in range(B):
        body = ids[b, 1:lengths[b] - 1]
        assert ((body >= 1000) & (body <= 30521)).all()
        assert (ids[b, lengths[b]:] == 0).all() and (mask[b, lengths[b]:] == 0).all()
        assert (mask[b, :lengths[b]] == 1).all()
