"""Host-side mirror of the reference ``Model`` (src/lib.rs:40-60, 155-666) over
the gfx950 C ABI.

Same entry points and meaning as the Rust API for this path:

* ``Model.from_weights(weights, config)``   <- ``Model::from_weights`` (src/lib.rs:155)
* ``Model.from_pretrained_path(dir)``       <- ``Model::from_pretrained_path`` (src/lib.rs:307)
* ``Model.forward(input_ids, attention_mask)`` <- ``Model::forward`` (src/lib.rs:621):
  f32 ``[B, S]`` ids / mask in, mean-pooled ``[B, H]`` out (not normalised)
* ``Model.encode_ids(ids, mask, normalize)`` <- ``encode_uncached`` after
  tokenisation (src/lib.rs:588-612)
* ``Model.encode(texts, normalize)``          <- ``Model::encode`` (src/lib.rs:479-520),
  including its 1000-entry LRU cache keyed ``"{text}||{normalize}"``; needs
  a tokenizer (``tokenizer.json``): the library's native WordPiece tokenizer
  (:class:`~edgebert_amd.tokenizer.Tokenizer`, default) or the HF
  ``tokenizers`` Tokenizer the reference uses (``tokenizer="hf"``).
* ``Model.score_pair(query, document)`` / ``score_batch(pairs)`` <-
  ``Model::score_pair`` / ``score_batch`` (src/lib.rs:327-383), for models
  loaded with ``classifier.weight`` / ``classifier.bias``; ``score_ids`` takes
  pre-tokenised pairs.

Errors raise :class:`EbhError` carrying the C ABI's code and message.
"""
from __future__ import annotations

import ctypes
import json
import os
import threading
from collections import OrderedDict

import numpy as np

from . import _native as N
from .synth import BertConfig
from .tokenizer import Tokenizer, c_texts, hf_encode_batch_ids, hf_tokenizer

# "fp32-bf16x6": an fp32 model whose GEMMs form each fp32 product from six
# bf16 MFMA products of three-way bf16 splits (include/edgebert_hip.h).
_DTYPES = {"fp32": N.EBH_DTYPE_F32, "f32": N.EBH_DTYPE_F32, "bf16": N.EBH_DTYPE_BF16,
           "fp32-bf16x6": N.EBH_DTYPE_F32_BF16X6}


def _ptr(a: np.ndarray):
    return ctypes.c_void_p(a.ctypes.data)


def _cfg_struct(cfg: BertConfig) -> N.EbhConfig:
    return N.EbhConfig(cfg.hidden_size, cfg.num_attention_heads, cfg.num_hidden_layers,
                       cfg.intermediate_size, cfg.vocab_size, cfg.max_position_embeddings,
                       cfg.type_vocab_size, cfg.layer_norm_eps)


class Model:
    CACHE_CAPACITY = 1000  # src/lib.rs:249-253

    def __init__(self, handle: int, config: BertConfig, dtype: str, tokenizer=None):
        self._h = ctypes.c_void_p(handle)
        self.config = config
        self.dtype = dtype
        self.tokenizer = tokenizer
        self._cache = OrderedDict()
        self._cache_lock = threading.Lock()

    # ---- construction ---------------------------------------------------
    @staticmethod
    def _create(config: BertConfig):
        L = N.lib()
        h = ctypes.c_void_p()
        cs = _cfg_struct(config)
        N.check(L.ebh_create(ctypes.byref(cs), ctypes.byref(h)))
        return h

    @staticmethod
    def _set(h, name: str, arr: np.ndarray):
        a = np.ascontiguousarray(arr, dtype=np.float32)
        shape = (ctypes.c_int64 * max(a.ndim, 1))(*a.shape)
        N.check(N.lib().ebh_set_tensor(h, name.encode(), _ptr(a), shape, a.ndim))

    @classmethod
    def from_weights(cls, weights: dict, config: BertConfig, dtype: str = "fp32",
                     tokenizer=None) -> "Model":
        """Upload HF-named float32 tensors (Linear weights ``[out, in]``) once to HBM."""
        h = cls._create(config)
        try:
            for name, arr in weights.items():
                cls._set(h, name, arr)
            N.check(N.lib().ebh_finalize(h, _DTYPES[dtype]))
        except Exception:
            N.lib().ebh_destroy(h)
            raise
        return cls(h.value, config, dtype, tokenizer)

    @classmethod
    def from_pretrained_path(cls, path: str, dtype: str = "fp32", tokenizer: str = "native") -> "Model":
        """``config.json`` + ``model.safetensors`` (+ ``tokenizer.json`` if present,
        read by the native tokenizer, or by HF ``tokenizers`` when
        ``tokenizer="hf"``)."""
        if tokenizer not in ("native", "hf"):
            raise ValueError("tokenizer must be 'native' or 'hf'")
        with open(os.path.join(path, "config.json")) as f:
            c = json.load(f)
        config = BertConfig(hidden_size=c["hidden_size"],
                            num_attention_heads=c["num_attention_heads"],
                            num_hidden_layers=c["num_hidden_layers"],
                            intermediate_size=c["intermediate_size"],
                            vocab_size=c["vocab_size"],
                            max_position_embeddings=c["max_position_embeddings"],
                            type_vocab_size=c.get("type_vocab_size", 2),
                            layer_norm_eps=c.get("layer_norm_eps", 1e-12),
                            hidden_act=c.get("hidden_act", "gelu"),
                            model_type=c.get("model_type", "bert"))
        tok_path = os.path.join(path, "tokenizer.json")
        tok = None
        if os.path.exists(tok_path):
            tok = Tokenizer.from_file(tok_path) if tokenizer == "native" else hf_tokenizer(tok_path)
        h = cls._create(config)
        try:
            N.check(N.lib().ebh_load_safetensors(h, os.path.join(path, "model.safetensors").encode()))
            N.check(N.lib().ebh_finalize(h, _DTYPES[dtype]))
        except Exception:
            N.lib().ebh_destroy(h)
            raise
        return cls(h.value, config, dtype, tok)

    def close(self):
        if getattr(self, "_h", None) is not None and self._h.value:
            N.lib().ebh_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ---- forward / encode -----------------------------------------------
    def forward(self, input_ids, attention_mask) -> np.ndarray:
        """``Model::forward``: f32 ``[B, S]`` ids and mask -> pooled ``[B, H]``."""
        ids = np.ascontiguousarray(input_ids, dtype=np.float32)
        mask = np.ascontiguousarray(attention_mask, dtype=np.float32)
        if ids.ndim != 2 or mask.shape != ids.shape:
            raise ValueError("input_ids and attention_mask must both be [B, S]")
        B, S = ids.shape
        out = np.zeros((B, self.config.hidden_size), np.float32)
        N.check(N.lib().ebh_forward(self._h, _ptr(ids), _ptr(mask), B, S, _ptr(out)))
        return out

    def encode_ids(self, ids, mask, normalize: bool = True) -> np.ndarray:
        """``encode_uncached`` after tokenisation: u32 ids / mask ``[B, S]``."""
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        mask = np.ascontiguousarray(mask, dtype=np.uint32)
        if ids.ndim != 2 or mask.shape != ids.shape:
            raise ValueError("ids and mask must both be [B, S]")
        B, S = ids.shape
        out = np.zeros((B, self.config.hidden_size), np.float32)
        N.check(N.lib().ebh_encode(self._h, _ptr(ids), _ptr(mask), B, S, int(bool(normalize)),
                                   _ptr(out)))
        return out

    def encode(self, texts, normalize_embeddings: bool = True):
        """``Model::encode`` (src/lib.rs:479-520): cache lookup, tokenise the misses
        (special tokens on, BatchLongest padding), run them, cache the results."""
        if self.tokenizer is None:
            raise RuntimeError("encode(texts) needs a tokenizer (tokenizer.json); "
                               "use encode_ids for pre-tokenised input")
        texts = list(texts)
        if not texts:
            return []
        results = [None] * len(texts)
        miss_idx, miss_txt = [], []
        with self._cache_lock:
            for i, t in enumerate(texts):
                key = f"{t}||{'true' if normalize_embeddings else 'false'}"
                if key in self._cache:
                    self._cache.move_to_end(key)
                    results[i] = list(self._cache[key])
                else:
                    miss_idx.append(i)
                    miss_txt.append(t)
        if miss_txt:
            emb = self.encode_texts(miss_txt, normalize_embeddings)
            with self._cache_lock:
                for r, i in enumerate(miss_idx):
                    vec = emb[r].tolist()
                    key = f"{texts[i]}||{'true' if normalize_embeddings else 'false'}"
                    self._cache[key] = vec
                    self._cache.move_to_end(key)
                    while len(self._cache) > self.CACHE_CAPACITY:
                        self._cache.popitem(last=False)
                    results[i] = list(vec)
        return results

    def encode_texts(self, texts, normalize: bool = True, nthreads: int = 0) -> np.ndarray:
        """``encode_uncached`` (src/lib.rs:573-619): tokenise and run, no cache.
        With the native tokenizer one call does both (``ebh_encode_texts``: host
        threads tokenise into the pinned staging buffers)."""
        texts = list(texts)
        out = np.zeros((len(texts), self.config.hidden_size), np.float32)
        if not texts:
            return out
        if isinstance(self.tokenizer, Tokenizer):
            arr, lens, _keep = c_texts(texts)
            N.check(N.lib().ebh_encode_texts(self._h, self.tokenizer.handle, arr, _ptr(lens), len(texts),
                                             1 if normalize else 0, _ptr(out), nthreads))
            return out
        if self.tokenizer is None:
            raise RuntimeError("encode(texts) needs a tokenizer (tokenizer.json)")
        ids, mask = hf_encode_batch_ids(self.tokenizer, texts)
        return self.encode_ids(ids.astype(np.uint32), mask.astype(np.uint32), normalize)

    def encode_batch(self, batches, normalize_embeddings: bool = True, workers: int = 2):
        """``encode_batch`` (src/lib.rs:438-450): one ``encode`` per sub-batch, the
        sub-batches run concurrently as the reference's rayon ``par_iter`` runs
        them.  The model serialises its forwards, but a sub-batch's
        tokenisation (host threads, outside the model's lock) overlaps the
        previous sub-batch's forward on the GPU."""
        batches = [list(b) for b in batches]
        if workers <= 1 or len(batches) <= 1:
            return [self.encode(b, normalize_embeddings) for b in batches]
        from concurrent.futures import ThreadPoolExecutor
        with ThreadPoolExecutor(max_workers=min(workers, len(batches))) as pool:
            return list(pool.map(lambda b: self.encode(b, normalize_embeddings), batches))

    def encode_texts_many(self, batches, normalize: bool = True, workers: int = 2) -> list:
        """``encode_texts`` of several sub-batches (no cache), run as
        ``encode_batch`` runs them: ``[n_i, H]`` arrays in order."""
        batches = [list(b) for b in batches]
        if workers <= 1 or len(batches) <= 1:
            return [self.encode_texts(b, normalize) for b in batches]
        from concurrent.futures import ThreadPoolExecutor
        with ThreadPoolExecutor(max_workers=min(workers, len(batches))) as pool:
            return list(pool.map(lambda b: self.encode_texts(b, normalize), batches))

    # ---- cross-encoder (score_pair / score_batch) ------------------------
    def score_ids(self, ids, mask) -> np.ndarray:
        """Scores of pre-tokenised pairs: u32 ids / mask ``[B, S]``, each row the
        encoding of one ``"query [SEP] document"`` text -> ``[B]`` (the pooled
        row ``.dot(classifier.weight) + classifier.bias``, src/lib.rs:359-375)."""
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        mask = np.ascontiguousarray(mask, dtype=np.uint32)
        if ids.ndim != 2 or mask.shape != ids.shape:
            raise ValueError("ids and mask must both be [B, S]")
        B, S = ids.shape
        out = np.zeros(B, np.float32)
        N.check(N.lib().ebh_score(self._h, _ptr(ids), _ptr(mask), B, S, _ptr(out)))
        return out

    def _score_texts(self, pairs) -> np.ndarray:
        if self.tokenizer is None:
            raise RuntimeError("score_pair needs a tokenizer (tokenizer.json); use score_ids")
        if isinstance(self.tokenizer, Tokenizer):
            qs, ql, _kq = c_texts([q for q, _ in pairs])
            ds, dl, _kd = c_texts([d for _, d in pairs])
            out = np.zeros(len(pairs), np.float32)
            N.check(N.lib().ebh_score_texts(self._h, self.tokenizer.handle, qs, _ptr(ql), ds, _ptr(dl),
                                            len(pairs), _ptr(out), 0))
            return out
        texts = [f"{q} [SEP] {d}" for q, d in pairs]      # src/lib.rs:332
        ids, mask = hf_encode_batch_ids(self.tokenizer, texts)
        return self.score_ids(ids.astype(np.uint32), mask.astype(np.uint32))

    def score_pair(self, query: str, document: str) -> float:
        """``Model::score_pair`` (src/lib.rs:327-376)."""
        return float(self._score_texts([(query, document)])[0])

    def score_batch(self, pairs) -> list:
        """``Model::score_batch`` (src/lib.rs:381-383).  The reference scores the
        pairs one by one; here they run as one padded batch, which gives each
        pair the score it gets alone (a pad is a masked key and every other step
        is per token)."""
        pairs = list(pairs)
        if not pairs:
            return []
        return [float(x) for x in self._score_texts(pairs)]

    # ---- device-resident path (bench / integration) ----------------------
    def encode_device(self, ids_ptr: int, mask_ptr: int, B: int, S: int, out_ptr: int,
                      normalize: bool = True, stream: int | None = None):
        """Enqueue a forward over device buffers (int32 ids / mask, f32 out)."""
        N.check(N.lib().ebh_encode_device(self._h, ctypes.c_void_p(ids_ptr),
                                          ctypes.c_void_p(mask_ptr), B, S, int(bool(normalize)),
                                          ctypes.c_void_p(out_ptr),
                                          ctypes.c_void_p(stream) if stream else None))

    def score_device(self, ids_ptr: int, mask_ptr: int, B: int, S: int, out_ptr: int,
                     stream: int | None = None):
        """Enqueue cross-encoder scoring over device buffers (int32 ids / mask, f32 [B] out)."""
        N.check(N.lib().ebh_score_device(self._h, ctypes.c_void_p(ids_ptr), ctypes.c_void_p(mask_ptr),
                                         B, S, ctypes.c_void_p(out_ptr),
                                         ctypes.c_void_p(stream) if stream else None))

    def synchronize(self):
        N.check(N.lib().ebh_synchronize(self._h))

    def set_graph_replay(self, enable: bool):
        """Record repeated forwards (same shape and buffers) as HIP graphs and
        replay them (default on); off runs every launch directly."""
        N.check(N.lib().ebh_set_graph_replay(self._h, 1 if enable else 0))

    def last_tokens(self, B: int):
        n = ctypes.c_int32()
        N.check(N.lib().ebh_last_tokens(self._h, None, None, 0, None, 0, ctypes.byref(n)))
        tok_ids = np.zeros(max(n.value, 1), np.int32)
        tok_pos = np.zeros(max(n.value, 1), np.int32)
        cu = np.zeros(B + 1, np.int32)
        N.check(N.lib().ebh_last_tokens(self._h, _ptr(tok_ids), _ptr(tok_pos), tok_ids.size,
                                        _ptr(cu), cu.size, ctypes.byref(n)))
        return tok_ids[:n.value], tok_pos[:n.value], cu

    def profile_enable(self, kernel: str):
        N.check(N.lib().ebh_profile_enable(self._h, N.PROF[kernel]))

    def profile_read(self):
        launches, ms = ctypes.c_int64(), ctypes.c_double()
        N.check(N.lib().ebh_profile_read(self._h, ctypes.byref(launches), ctypes.byref(ms)))
        return launches.value, ms.value


def cosine_similarity(a, b) -> float:
    """``cosine_similarity`` (src/lib.rs:756-789): dot / (|a||b| + 1e-8)."""
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    n = min(a.size, b.size)
    dot = np.float32(np.dot(a[:n], b[:n]))
    return float(dot / (np.float32(np.linalg.norm(a)) * np.float32(np.linalg.norm(b)) + np.float32(1e-8)))
