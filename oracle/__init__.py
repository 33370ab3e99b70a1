"""ctypes wrapper around ``liboracle.so``, the CPU restatement of EdgeBERT's
encoder forward (``oracle.c``).

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg import this package, and only as the
checker (or the timed CPU baseline); the HIP product path in ``edgebert_amd``
never routes through it.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None

_f32p = ctypes.POINTER(ctypes.c_float)
_i64p = ctypes.POINTER(ctypes.c_int64)


def lib():
    global _LIB
    if _LIB is None:
        # EDGEBERT_ORACLE_LIB selects another build (the sanitizer build of
        # `make -C oracle sanitize`).
        path = os.environ.get("EDGEBERT_ORACLE_LIB") or os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is missing: build it with `make -C oracle` "
                               "(or __graft_entry__.build())")
        L = ctypes.CDLL(path)
        L.orc_last_error.restype = ctypes.c_char_p
        L.orc_model_new.restype = ctypes.c_void_p
        L.orc_model_new.argtypes = [ctypes.c_int] * 7 + [ctypes.c_float]
        L.orc_set_tensor.argtypes = [ctypes.c_void_p, ctypes.c_char_p, _f32p, _i64p, ctypes.c_int]
        L.orc_model_build.argtypes = [ctypes.c_void_p]
        L.orc_model_free.argtypes = [ctypes.c_void_p]
        L.orc_forward.argtypes = [ctypes.c_void_p, _f32p, _f32p, ctypes.c_int, ctypes.c_int, _f32p]
        L.orc_forward_trace.argtypes = [ctypes.c_void_p, _f32p, _f32p, ctypes.c_int,
                                        ctypes.c_int, _f32p, _f32p]
        L.orc_sgemm.argtypes = [ctypes.c_int] * 3 + [_f32p, ctypes.c_int, _f32p, ctypes.c_int,
                                                     _f32p, ctypes.c_int]
        L.orc_matmul_3d_2d.argtypes = [_f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, _f32p,
                                       ctypes.c_int, _f32p]
        L.orc_matmul_4d.argtypes = [_f32p, _f32p] + [ctypes.c_int] * 5 + [_f32p]
        L.orc_softmax.argtypes = [_f32p, ctypes.c_int64, ctypes.c_int]
        L.orc_apply_attention_mask.argtypes = [_f32p, _f32p] + [ctypes.c_int] * 4
        L.orc_gelu.argtypes = [_f32p, ctypes.c_int64]
        L.orc_layer_norm.argtypes = [_f32p, ctypes.c_int64, ctypes.c_int, _f32p, _f32p,
                                     ctypes.c_float, _f32p]
        L.orc_mean_pool.argtypes = [_f32p, _f32p] + [ctypes.c_int] * 3 + [_f32p]
        L.orc_normalize.argtypes = [_f32p, ctypes.c_int, ctypes.c_int]
        L.orc_cosine_similarity.restype = ctypes.c_float
        L.orc_cosine_similarity.argtypes = [_f32p, _f32p, ctypes.c_int]
        L.orc_dot.restype = ctypes.c_float
        L.orc_dot.argtypes = [_f32p, _f32p, ctypes.c_int]
        L.orc_set_blas_sgemm.argtypes = [ctypes.c_void_p]
        L.orc_set_num_threads.argtypes = [ctypes.c_int]
        L.orc_get_num_threads.restype = ctypes.c_int
        _LIB = L
    return _LIB


def _p(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(_f32p)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


class OracleError(RuntimeError):
    pass


def _check(rc: int):
    if rc != 0:
        raise OracleError(lib().orc_last_error().decode())


_BLAS = None


def openblas_sgemm():
    """(path, address of cblas_sgemm, set_num_threads) of the OpenBLAS that
    numpy links (ILP64, symbol suffix ``64_``), or None when there is none."""
    global _BLAS
    if _BLAS is None:
        import glob
        libs = os.path.join(os.path.dirname(os.path.dirname(np.__file__)), "numpy.libs")
        found = ()
        for path in sorted(glob.glob(os.path.join(libs, "libscipy_openblas64_*.so"))):
            L = ctypes.CDLL(path)
            try:
                fn = ctypes.cast(L.scipy_cblas_sgemm64_, ctypes.c_void_p).value
                nt = L.scipy_openblas_set_num_threads64_
            except AttributeError:
                continue
            nt.argtypes = [ctypes.c_int]
            found = (path, fn, nt)
            break
        _BLAS = found
    return _BLAS or None


def use_openblas(enabled: bool) -> str | None:
    """Route every product of the oracle through OpenBLAS's cblas_sgemm (the
    reference built with ``--features openblas``), or back to the built-in
    sgemm.  OpenBLAS runs one thread per call; the batch slices spread over the
    oracle's OpenMP threads.  Returns the library's path (None when disabled)."""
    if not enabled:
        lib().orc_set_blas_sgemm(None)
        return None
    b = openblas_sgemm()
    if b is None:
        raise OracleError("numpy's OpenBLAS (libscipy_openblas64_) was not found")
    path, fn, nt = b
    nt(1)
    lib().orc_set_blas_sgemm(fn)
    return path


def set_num_threads(n: int):
    lib().orc_set_num_threads(int(n))


def get_num_threads() -> int:
    return lib().orc_get_num_threads()


class OracleModel:
    """``Model::from_weights`` + ``forward`` (src/lib.rs:155-260, 621-666) on the CPU."""

    def __init__(self, cfg, weights: dict):
        L = lib()
        self.cfg = cfg
        # Cross-encoder head (from_cross_encoder_weights, src/lib.rs:385-399):
        # kept here; the C model holds the encoder.
        self.classifier = None
        if "classifier.weight" in weights:
            w = _f32(weights["classifier.weight"]).reshape(-1)
            b = _f32(weights["classifier.bias"]).reshape(-1)
            if w.size != cfg.hidden_size or b.size != 1:
                raise OracleError("classifier.weight must hold hidden_size values and classifier.bias one")
            self.classifier = (np.ascontiguousarray(w), np.float32(b[0]))
        weights = {k: v for k, v in weights.items() if not k.startswith("classifier.")}
        self._h = L.orc_model_new(cfg.hidden_size, cfg.num_attention_heads, cfg.num_hidden_layers,
                                  cfg.intermediate_size, cfg.vocab_size,
                                  cfg.max_position_embeddings, cfg.type_vocab_size,
                                  cfg.layer_norm_eps)
        if not self._h:
            raise OracleError(L.orc_last_error().decode())
        for name, arr in weights.items():
            a = _f32(arr)
            shape = (ctypes.c_int64 * a.ndim)(*a.shape)
            _check(L.orc_set_tensor(self._h, name.encode(), _p(a), shape, a.ndim))
        _check(L.orc_model_build(self._h))

    def __del__(self):
        if getattr(self, "_h", None):
            lib().orc_model_free(self._h)
            self._h = None

    def forward(self, input_ids, attention_mask) -> np.ndarray:
        """ids / mask as the reference's f32 ``[B,S]`` arrays -> pooled ``[B,H]``."""
        ids, mask = _f32(input_ids), _f32(attention_mask)
        B, S = ids.shape
        out = np.zeros((B, self.cfg.hidden_size), np.float32)
        _check(lib().orc_forward(self._h, _p(ids), _p(mask), B, S, _p(out)))
        return out

    def forward_trace(self, input_ids, attention_mask):
        ids, mask = _f32(input_ids), _f32(attention_mask)
        B, S = ids.shape
        H, L = self.cfg.hidden_size, self.cfg.num_hidden_layers
        out = np.zeros((B, H), np.float32)
        trace = np.zeros((L + 1, B, S, H), np.float32)
        _check(lib().orc_forward_trace(self._h, _p(ids), _p(mask), B, S, _p(out), _p(trace)))
        return out, trace

    def encode(self, input_ids, attention_mask, normalize: bool = True) -> np.ndarray:
        """``encode_uncached`` after tokenisation (src/lib.rs:588-612)."""
        out = self.forward(input_ids, attention_mask)
        if normalize:
            normalize_rows(out)
        return out

    def score(self, input_ids, attention_mask) -> np.ndarray:
        """``score_pair`` per row (src/lib.rs:327-376): pooled ``forward`` row
        ``.dot(classifier.weight) + classifier.bias``, in fp32."""
        if self.classifier is None:
            raise OracleError("Model is not a cross-encoder")
        w, b = self.classifier
        pooled = self.forward(input_ids, attention_mask)
        return np.array([np.float32(lib().orc_dot(_p(np.ascontiguousarray(r)), _p(w), w.size)) + b
                         for r in pooled], np.float32)

    def encode_unpadded(self, ids, mask, normalize: bool = True) -> np.ndarray:
        """Each sequence run alone at its own length (the padding-free CPU run)."""
        ids, mask = np.asarray(ids), np.asarray(mask)
        rows = []
        for b in range(ids.shape[0]):
            keep = mask[b] != 0
            rows.append(self.encode(ids[b][keep][None, :], mask[b][keep][None, :], normalize)[0])
        return np.stack(rows) if rows else np.zeros((0, self.cfg.hidden_size), np.float32)


# ---- individual ops ---------------------------------------------------------

def sgemm(a, b) -> np.ndarray:
    a, b = _f32(a), _f32(b)
    m, k = a.shape
    n = b.shape[1]
    c = np.zeros((m, n), np.float32)
    lib().orc_sgemm(m, n, k, _p(a), k, _p(b), n, _p(c), n)
    return c


def matmul_3d_2d(a, b) -> np.ndarray:
    a, b = _f32(a), _f32(b)
    batch, m, k = a.shape
    n = b.shape[1]
    c = np.zeros((batch, m, n), np.float32)
    lib().orc_matmul_3d_2d(_p(a), batch, m, k, _p(b), n, _p(c))
    return c


def matmul_4d(a, b) -> np.ndarray:
    a, b = _f32(a), _f32(b)
    B, h, s1, d = a.shape
    s2 = b.shape[3]
    c = np.zeros((B, h, s1, s2), np.float32)
    lib().orc_matmul_4d(_p(a), _p(b), B, h, s1, d, s2, _p(c))
    return c


def softmax(x) -> np.ndarray:
    y = _f32(x).copy()
    lib().orc_softmax(_p(y), y.size // y.shape[-1] if y.size else 0, y.shape[-1])
    return y


def apply_attention_mask(scores, mask) -> np.ndarray:
    s = _f32(scores).copy()
    m = _f32(mask)
    B, nh, S1, S2 = s.shape
    lib().orc_apply_attention_mask(_p(s), _p(m), B, nh, S1, S2)
    return s


def gelu(x) -> np.ndarray:
    y = _f32(x).copy()
    lib().orc_gelu(_p(y), y.size)
    return y


def layer_norm(x, weight, bias, eps) -> np.ndarray:
    x = _f32(x)
    H = x.shape[-1]
    y = np.empty_like(x)
    lib().orc_layer_norm(_p(x), x.size // H, H, _p(_f32(weight)), _p(_f32(bias)), eps, _p(y))
    return y


def mean_pool(hidden, mask) -> np.ndarray:
    h, m = _f32(hidden), _f32(mask)
    B, S, H = h.shape
    out = np.zeros((B, H), np.float32)
    lib().orc_mean_pool(_p(h), _p(m), B, S, H, _p(out))
    return out


def normalize_rows(x: np.ndarray) -> np.ndarray:
    """In place, as ``encode_uncached`` does (src/lib.rs:605-612)."""
    assert x.dtype == np.float32 and x.flags["C_CONTIGUOUS"]
    B, H = x.shape
    lib().orc_normalize(_p(x), B, H)
    return x


def cosine_similarity(a, b) -> float:
    a, b = _f32(a), _f32(b)
    return float(lib().orc_cosine_similarity(_p(a), _p(b), min(a.size, b.size)))
