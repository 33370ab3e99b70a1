"""Host tokenizer of the encode path.

* :class:`Tokenizer` -- the native BERT WordPiece tokenizer of the library
  (``ebh_tokenizer_*``, ``ebh_tokenize``): ``tokenizer.json`` read the way the
  reference reads it (``Tokenizer::from_file`` with padding BatchLongest and
  truncation at 512, src/lib.rs:310-322) and ``encode_batch(texts, true)``
  (src/lib.rs:577-601), on host threads.
* :func:`hf_tokenizer` -- the HF ``tokenizers`` Tokenizer the reference uses,
  configured with the same overrides, for tokenizer.json files outside the
  native tokenizer's BERT subset.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _native as N


def c_texts(texts):
    """(char* array, int64 byte lengths, keep-alive) of UTF-8 encoded texts."""
    enc = [t.encode("utf-8") for t in texts]
    arr = (ctypes.c_char_p * max(len(enc), 1))(*enc)
    lens = np.array([len(e) for e in enc] or [0], np.int64)
    return arr, lens, enc


class Tokenizer:
    """Native BERT WordPiece tokenizer (thread-safe; immutable once loaded)."""

    def __init__(self, handle: int):
        self._h = ctypes.c_void_p(handle)

    @classmethod
    def from_file(cls, path: str) -> "Tokenizer":
        h = ctypes.c_void_p()
        N.check(N.lib().ebh_tokenizer_load(path.encode(), ctypes.byref(h)))
        return cls(h.value)

    @classmethod
    def from_str(cls, text: str) -> "Tokenizer":
        data = text.encode("utf-8")
        h = ctypes.c_void_p()
        N.check(N.lib().ebh_tokenizer_from_json(data, len(data), ctypes.byref(h)))
        return cls(h.value)

    @property
    def handle(self) -> ctypes.c_void_p:
        return self._h

    def encode_batch_ids(self, texts, nthreads: int = 0, cap: int | None = None):
        """int32 ids and 0/1 mask ``[n, S]`` of ``encode_batch(texts, true)`` padded
        to the batch's longest encoding."""
        texts = list(texts)
        n = len(texts)
        if cap is None:
            cap = 512 + 16
            while True:
                ids = np.empty(max(n * cap, 1), np.int32)
                mask = np.empty(max(n * cap, 1), np.int32)
                S = ctypes.c_int32()
                arr, lens, _keep = c_texts(texts)
                rc = N.lib().ebh_tokenize(self._h, arr, lens.ctypes.data, n, cap, ids.ctypes.data,
                                          mask.ctypes.data, ctypes.byref(S), nthreads)
                if rc == N.EBH_ERR_RANGE and cap < (1 << 20):
                    cap *= 4                      # no truncation in the file: longer texts
                    continue
                N.check(rc)
                break
        else:
            ids = np.empty(max(n * cap, 1), np.int32)
            mask = np.empty(max(n * cap, 1), np.int32)
            S = ctypes.c_int32()
            arr, lens, _keep = c_texts(texts)
            N.check(N.lib().ebh_tokenize(self._h, arr, lens.ctypes.data, n, cap, ids.ctypes.data,
                                         mask.ctypes.data, ctypes.byref(S), nthreads))
        S = S.value
        return ids[:n * S].reshape(n, S), mask[:n * S].reshape(n, S)

    def close(self):
        if getattr(self, "_h", None) is not None and self._h.value:
            N.lib().ebh_tokenizer_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def hf_tokenizer(path: str):
    """``tokenizers.Tokenizer.from_file`` with the reference's overrides: the
    file's padding with strategy BatchLongest, the file's truncation with
    max_length 512 (src/lib.rs:314-322)."""
    from tokenizers import Tokenizer as HFTokenizer
    return _reference_overrides(HFTokenizer.from_file(path))


def hf_tokenizer_from_str(text: str):
    """:func:`hf_tokenizer` for tokenizer.json content."""
    from tokenizers import Tokenizer as HFTokenizer
    return _reference_overrides(HFTokenizer.from_str(text))


def _reference_overrides(tok):
    if tok.padding is not None:
        pad = dict(tok.padding)
        tok.enable_padding(**{k: v for k, v in pad.items()
                              if k in ("direction", "pad_id", "pad_type_id", "pad_token",
                                       "pad_to_multiple_of")})
    if tok.truncation is not None:
        tr = dict(tok.truncation)
        tok.enable_truncation(512, stride=tr.get("stride", 0),
                              strategy=tr.get("strategy", "longest_first"),
                              direction=tr.get("direction", "right"))
    return tok


def hf_encode_batch_ids(tok, texts):
    """int32 ids / mask ``[n, S]`` from an HF tokenizer's ``encode_batch(texts, True)``
    (zero-filled past each encoding, as the reference's marshalling does)."""
    encs = tok.encode_batch(list(texts), add_special_tokens=True)
    S = max((len(e.ids) for e in encs), default=0)
    ids = np.zeros((len(encs), S), np.int32)
    mask = np.zeros((len(encs), S), np.int32)
    for r, e in enumerate(encs):
        ids[r, :len(e.ids)] = e.ids
        mask[r, :len(e.attention_mask)] = e.attention_mask
    return ids, mask
