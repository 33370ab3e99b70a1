"""The host parsers that read untrusted bytes, fed mutated inputs: the
safetensors header (ebh_load_safetensors: JSON, dtypes, shapes, offsets) and
the tokenizer (ebh_tokenizer_from_json: tokenizer.json; ebh_tokenize: UTF-8
texts with any bytes).  Every call must return EBH_OK or an EBH_ERR_* code
with a message; none may crash.  CPU only (no call here touches a GPU); run
under the host AddressSanitizer / UndefinedBehaviorSanitizer build by
`make -C edgebert_amd/csrc sanitize-test`."""
import ctypes
import json
import random
import struct

import numpy as np
import pytest

import edgebert_amd as eb
from edgebert_amd import _native as N
from edgebert_amd import synth
from edgebert_amd.model import _cfg_struct

CODES = {N.EBH_OK, N.EBH_ERR_INVALID_ARG, N.EBH_ERR_NOT_FOUND, N.EBH_ERR_SHAPE, N.EBH_ERR_STATE,
         N.EBH_ERR_RANGE}


def _mutate(rng: random.Random, data: bytes, n_edits: int) -> bytes:
    """Byte flips, insertions, deletions, duplicated spans and truncation."""
    b = bytearray(data)
    for _ in range(n_edits):
        op = rng.randrange(6)
        i = rng.randrange(len(b) + 1)
        if op == 0 and b:
            b[min(i, len(b) - 1)] = rng.randrange(256)
        elif op == 1:
            b[i:i] = bytes(rng.randrange(256) for _ in range(rng.randint(1, 8)))
        elif op == 2 and b:
            del b[i:i + rng.randint(1, 16)]
        elif op == 3 and b:
            j = rng.randrange(len(b))
            b[i:i] = b[j:j + rng.randint(1, 32)]
        elif op == 4:
            del b[i:]
        elif op == 5 and b:   # a digit nudged: offsets and shapes one off
            digits = [k for k, c in enumerate(b) if 48 <= c <= 57]
            if digits:
                k = rng.choice(digits)
                b[k] = 48 + (b[k] - 48 + rng.choice([1, 9])) % 10
    return bytes(b)


def _safetensors_bytes(tensors):
    header, blobs, off = {"__metadata__": {"format": "pt"}}, [], 0
    for name, (dt, arr) in tensors.items():
        data = arr.tobytes()
        header[name] = {"dtype": dt, "shape": list(arr.shape), "data_offsets": [off, off + len(data)]}
        blobs.append(data)
        off += len(data)
    h = json.dumps(header).encode()
    return struct.pack("<Q", len(h)) + h + b"".join(blobs)


def test_safetensors_loader_survives_mutated_files(tmp_path, weights_for):
    L = eb.lib()
    w = weights_for(synth.TINY)
    keep = ["embeddings.LayerNorm.weight", "embeddings.LayerNorm.bias", "encoder.layer.0.output.dense.bias",
            "encoder.layer.0.attention.self.query.weight", "embeddings.token_type_embeddings.weight"]
    tensors = {k: ("F32", w[k]) for k in keep}
    tensors["embeddings.LayerNorm.bias"] = ("F16", w["embeddings.LayerNorm.bias"].astype(np.float16))
    tensors["encoder.layer.0.output.dense.bias"] = (
        "BF16", (w["encoder.layer.0.output.dense.bias"].view(np.uint32) >> 16).astype(np.uint16))
    good = _safetensors_bytes(tensors)
    cs = _cfg_struct(synth.TINY)
    rng = random.Random(1234)
    seen = set()
    path = tmp_path / "m.safetensors"
    for case in range(400):
        # mutations aimed at the header most of the time (the data is opaque bytes)
        data = _mutate(rng, good[:8 + 600] if case % 4 else good, rng.randint(1, 6))
        if case % 4:
            data = data + good[8 + 600:]
        path.write_bytes(data)
        h = ctypes.c_void_p()
        assert L.ebh_create(ctypes.byref(cs), ctypes.byref(h)) == N.EBH_OK
        rc = L.ebh_load_safetensors(h, str(path).encode())
        L.ebh_destroy(h)
        assert rc in CODES, rc
        if rc != N.EBH_OK:
            assert N.last_error()
        seen.add(rc)
    assert N.EBH_ERR_SHAPE in seen and len(seen) >= 2


def test_tokenizer_survives_mutated_json_and_texts():
    L = eb.lib()
    good = synth.tokenizer_json(synth.TINY).encode()
    rng = random.Random(99)
    ok_tokenizers = 0
    for case in range(300):
        data = _mutate(rng, good, rng.randint(1, 4))
        h = ctypes.c_void_p()
        rc = L.ebh_tokenizer_from_json(data, len(data), ctypes.byref(h))
        assert rc in CODES, rc
        if rc != N.EBH_OK:
            assert N.last_error()
            continue
        ok_tokenizers += 1
        texts = [bytes(rng.randrange(256) for _ in range(rng.randint(0, 64))) for _ in range(6)]
        texts.append("t12 t7 [SEP] héllo 中文".encode())
        arr = (ctypes.c_char_p * len(texts))(*texts)
        lens = np.array([len(t) for t in texts], np.int64)
        cap = 2048
        ids = np.empty(len(texts) * cap, np.int32)
        mask = np.empty(len(texts) * cap, np.int32)
        S = ctypes.c_int32()
        rc = L.ebh_tokenize(h, arr, lens.ctypes.data, len(texts), cap, ids.ctypes.data, mask.ctypes.data,
                            ctypes.byref(S), 2)
        L.ebh_tokenizer_destroy(h)
        assert rc in CODES, rc
        if rc == N.EBH_OK:
            assert 0 <= S.value <= cap
            assert set(np.unique(mask[:len(texts) * S.value])) <= {0, 1}
    assert ok_tokenizers > 0


@pytest.mark.parametrize("seed", range(4))
def test_tokenizer_survives_arbitrary_utf8_bytes(seed):
    """Invalid UTF-8, NUL bytes, lone surrogates' encodings, overlong forms and
    4-byte sequences beyond U+10FFFF, through a valid tokenizer."""
    L = eb.lib()
    good = synth.tokenizer_json(synth.TINY).encode()
    h = ctypes.c_void_p()
    N.check(L.ebh_tokenizer_from_json(good, len(good), ctypes.byref(h)))
    rng = random.Random(seed)
    special = [b"\xed\xa0\x80", b"\xc0\xaf", b"\xf4\x90\x80\x80", b"\xf8\x88\x80\x80\x80", b"\x00", b"\xff\xfe",
               b"\xe2\x80", b"\xf0\x9f\x98\x80", "İ".encode(), "ﬁ".encode(), "́" .encode() * 40]
    try:
        for _ in range(50):
            texts = [b"".join(rng.choice(special) if rng.random() < 0.3 else bytes([rng.randrange(256)])
                              for _ in range(rng.randint(0, 200))) for _ in range(8)]
            arr = (ctypes.c_char_p * len(texts))(*texts)
            lens = np.array([len(t) for t in texts], np.int64)
            cap = 4096
            ids = np.empty(len(texts) * cap, np.int32)
            mask = np.empty(len(texts) * cap, np.int32)
            S = ctypes.c_int32()
            rc = L.ebh_tokenize(h, arr, lens.ctypes.data, len(texts), cap, ids.ctypes.data, mask.ctypes.data,
                                ctypes.byref(S), 4)
            assert rc == N.EBH_OK, N.last_error()
            assert ((ids[:len(texts) * S.value] >= 0) & (ids[:len(texts) * S.value] < synth.TINY.vocab_size)).all()
    finally:
        L.ebh_tokenizer_destroy(h)
