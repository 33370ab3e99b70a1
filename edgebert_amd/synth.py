"""Deterministic synthetic models and inputs for the EdgeBERT encoder path.

There is no network here, so the real all-MiniLM-L6-v2 checkpoint that the
reference downloads (`src/lib.rs:403-437`) cannot be used.  Every config is
instead driven by a counter-based generator:

* weights: every embedding table, Linear weight and Linear bias is N(0, 0.02);
  LayerNorm gamma = 1, beta = 0 (the shapes and HF tensor names are the ones
  `Model::from_weights` reads, `src/lib.rs:155-238`).  Tensor ``name`` draws
  element i from the splitmix64 outputs at counters (2i, 2i+1) of the stream
  seeded with ``SEED_WEIGHTS ^ fnv1a64(name)``, turned into a normal deviate by
  Box-Muller.
* inputs: ``[CLS]=101``, then uniform ids in [1000, 30521], then ``[SEP]=102``,
  padded with id 0 / mask 0 (the layout `encode_uncached` builds,
  `src/lib.rs:588-601`).

All arithmetic is vectorised numpy uint64 (wrapping), so MiniLM (22.7 M
parameters) generates in about a second.
"""
from __future__ import annotations

import hashlib
from dataclasses import dataclass, field, asdict

import numpy as np

SEED_WEIGHTS = 0x5EED0001
_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
CLS_ID, SEP_ID, PAD_ID = 101, 102, 0


@dataclass(frozen=True)
class BertConfig:
    """Mirror of the reference `Config` (`src/lib.rs:95-106`) plus the token-type
    table size, which the reference takes from the tensor shape."""
    hidden_size: int
    num_attention_heads: int
    num_hidden_layers: int
    intermediate_size: int
    vocab_size: int = 30522
    max_position_embeddings: int = 512
    type_vocab_size: int = 2
    layer_norm_eps: float = 1e-12
    hidden_act: str = "gelu"
    model_type: str = "bert"

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_attention_heads

    def to_dict(self):
        return asdict(self)


MINILM_L6 = BertConfig(hidden_size=384, num_attention_heads=12, num_hidden_layers=6,
                       intermediate_size=1536)
BERT_BASE = BertConfig(hidden_size=768, num_attention_heads=12, num_hidden_layers=12,
                       intermediate_size=3072)
# Small shape used for brute-force and fixture tests.
TINY = BertConfig(hidden_size=64, num_attention_heads=2, num_hidden_layers=2,
                  intermediate_size=256, vocab_size=2048, max_position_embeddings=64)


@dataclass(frozen=True)
class InputSpec:
    """One workload: batch, padded length, and the inclusive range of true lengths."""
    name: str
    model: BertConfig
    batch: int
    seq_len: int
    len_lo: int
    len_hi: int
    seed: int
    dtype: str = "fp32"
    notes: str = field(default="", compare=False)


# BASELINE.json configs[0..4], in order.
CONFIGS = {
    "c1": InputSpec("c1", MINILM_L6, 2, 8, 8, 8, 1, "fp32", "reference CPU-runnable case"),
    "c2": InputSpec("c2", MINILM_L6, 32, 128, 8, 128, 2, "fp32", "padded, key-padding mask"),
    "c3": InputSpec("c3", MINILM_L6, 256, 128, 128, 128, 3, "fp32", "headline throughput"),
    "c4": InputSpec("c4", MINILM_L6, 16, 512, 256, 512, 4, "fp32", "attention-heavy"),
    "c5": InputSpec("c5", BERT_BASE, 1024, 128, 128, 128, 5, "bf16", "BERT-base, bf16 GEMMs"),
}


def _mix(z: np.ndarray) -> np.ndarray:
    """splitmix64 finaliser (Steele, Lea, Flood 2014), on wrapping uint64 arrays."""
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def splitmix64(seed: int, counters: np.ndarray) -> np.ndarray:
    """Output number ``counters`` (0-based) of the splitmix64 sequence seeded with ``seed``."""
    with np.errstate(over="ignore"):
        c = counters.astype(np.uint64) + np.uint64(1)
        return _mix(np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + c * _GAMMA)


def fnv1a64(text: str) -> int:
    h = 0xCBF29CE484222325
    for byte in text.encode():
        h ^= byte
        h = (h * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def normal(seed: int, n: int) -> np.ndarray:
    """n standard normal deviates (float64) by Box-Muller on splitmix64 pairs."""
    idx = np.arange(n, dtype=np.uint64)
    r0 = splitmix64(seed, idx * np.uint64(2))
    r1 = splitmix64(seed, idx * np.uint64(2) + np.uint64(1))
    u1 = ((r0 >> np.uint64(11)).astype(np.float64) + 1.0) * (2.0 ** -53)   # (0, 1]
    u2 = (r1 >> np.uint64(11)).astype(np.float64) * (2.0 ** -53)           # [0, 1)
    return np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)


def tensor_shapes(cfg: BertConfig) -> dict:
    """HF tensor names and shapes the reference loads (`src/lib.rs:161-238`).
    Linear weights are HF ``[out, in]``."""
    H, I = cfg.hidden_size, cfg.intermediate_size
    shapes = {
        "embeddings.word_embeddings.weight": (cfg.vocab_size, H),
        "embeddings.position_embeddings.weight": (cfg.max_position_embeddings, H),
        "embeddings.token_type_embeddings.weight": (cfg.type_vocab_size, H),
        "embeddings.LayerNorm.weight": (H,),
        "embeddings.LayerNorm.bias": (H,),
    }
    for i in range(cfg.num_hidden_layers):
        p = f"encoder.layer.{i}"
        for proj in ("query", "key", "value"):
            shapes[f"{p}.attention.self.{proj}.weight"] = (H, H)
            shapes[f"{p}.attention.self.{proj}.bias"] = (H,)
        shapes[f"{p}.attention.output.dense.weight"] = (H, H)
        shapes[f"{p}.attention.output.dense.bias"] = (H,)
        shapes[f"{p}.attention.output.LayerNorm.weight"] = (H,)
        shapes[f"{p}.attention.output.LayerNorm.bias"] = (H,)
        shapes[f"{p}.intermediate.dense.weight"] = (I, H)
        shapes[f"{p}.intermediate.dense.bias"] = (I,)
        shapes[f"{p}.output.dense.weight"] = (H, I)
        shapes[f"{p}.output.dense.bias"] = (H,)
        shapes[f"{p}.output.LayerNorm.weight"] = (H,)
        shapes[f"{p}.output.LayerNorm.bias"] = (H,)
    return shapes


def make_weights(cfg: BertConfig, seed: int = SEED_WEIGHTS, std: float = 0.02) -> dict:
    """Random-init weights of the architecture, keyed by HF tensor name (float32)."""
    out = {}
    for name, shape in tensor_shapes(cfg).items():
        n = int(np.prod(shape))
        if "LayerNorm.weight" in name:
            arr = np.ones(n, np.float32)
        elif "LayerNorm.bias" in name:
            arr = np.zeros(n, np.float32)
        else:
            arr = (std * normal(seed ^ fnv1a64(name), n)).astype(np.float32)
        out[name] = arr.reshape(shape)
    return out


def weights_sha256(weights: dict) -> str:
    """Digest over names and float32 little-endian bytes, in sorted-name order."""
    h = hashlib.sha256()
    for name in sorted(weights):
        h.update(name.encode())
        h.update(np.ascontiguousarray(weights[name], dtype="<f4").tobytes())
    return h.hexdigest()


def make_inputs(spec: InputSpec):
    """Seeded ids/mask for one workload.

    Returns ``(ids, mask, lengths)``: int32 ``[B, S]`` ids (pads 0), int32
    ``[B, S]`` mask (1 on real tokens), and int64 true lengths.  Length draw b
    uses counter b of stream ``seed*2``; id draw (b, j) uses counter
    ``b*S + j`` of stream ``seed*2+1``.
    """
    B, S = spec.batch, spec.seq_len
    span = spec.len_hi - spec.len_lo + 1
    r_len = splitmix64(spec.seed * 2, np.arange(B, dtype=np.uint64))
    lengths = spec.len_lo + (r_len % np.uint64(span)).astype(np.int64)
    r_id = splitmix64(spec.seed * 2 + 1, np.arange(B * S, dtype=np.uint64)).reshape(B, S)
    id_hi = min(30521, spec.model.vocab_size - 1)       # [1000, 30521] for the 30522 vocab
    body = (1000 + (r_id % np.uint64(id_hi - 1000 + 1)).astype(np.int64)).astype(np.int32)
    pos = np.arange(S)[None, :]
    L = lengths[:, None]
    ids = np.where(pos < L, body, PAD_ID).astype(np.int32)
    ids[:, 0] = CLS_ID
    ids[np.arange(B), lengths - 1] = SEP_ID
    mask = (pos < L).astype(np.int32)
    return ids, mask, lengths


# ---------------------------------------------------------------------------
# Synthetic tokenizer.json and texts: every id from 1000 up is a distinct
# lowercase word, so the texts of a workload tokenise back to its ids exactly
# (each word is a whole vocabulary entry).
# ---------------------------------------------------------------------------
def vocab_word(i: int) -> str:
    """The word of id ``i`` (>= 1000): ``i`` in base 26 over a..z, prefixed
    with 'q' (no single letters, no collisions)."""
    s = ""
    while True:
        s = chr(ord("a") + i % 26) + s
        i //= 26
        if i == 0:
            return "q" + s


def tokenizer_json(cfg: BertConfig) -> str:
    """A BERT uncased tokenizer.json over ``cfg.vocab_size`` ids: [PAD] 0,
    [UNK] 100, [CLS] 101, [SEP] 102, [MASK] 103, [unusedK] up to 999, then
    :func:`vocab_word` words; BertNormalizer + BertPreTokenizer + WordPiece,
    [CLS] $A [SEP], truncation and BatchLongest padding."""
    import json
    special = {0: "[PAD]", 100: "[UNK]", 101: "[CLS]", 102: "[SEP]", 103: "[MASK]"}
    vocab = {}
    for i in range(cfg.vocab_size):
        vocab[special.get(i, f"[unused{i}]") if i < 1000 else vocab_word(i)] = i
    added = [{"id": i, "content": t, "single_word": False, "lstrip": False, "rstrip": False,
              "normalized": False, "special": True} for i, t in sorted(special.items())]
    tmpl = lambda ids: [{"SpecialToken": {"id": ids[0], "type_id": 0}},  # noqa: E731
                        {"Sequence": {"id": "A", "type_id": 0}},
                        {"SpecialToken": {"id": ids[1], "type_id": 0}}]
    doc = {
        "version": "1.0",
        "truncation": {"direction": "Right", "max_length": 128, "strategy": "LongestFirst", "stride": 0},
        "padding": {"strategy": "BatchLongest", "direction": "Right", "pad_to_multiple_of": None,
                    "pad_id": 0, "pad_type_id": 0, "pad_token": "[PAD]"},
        "added_tokens": added,
        "normalizer": {"type": "BertNormalizer", "clean_text": True, "handle_chinese_chars": True,
                       "strip_accents": None, "lowercase": True},
        "pre_tokenizer": {"type": "BertPreTokenizer"},
        "post_processor": {"type": "TemplateProcessing", "single": tmpl(["[CLS]", "[SEP]"]),
                           "pair": tmpl(["[CLS]", "[SEP]"]),
                           "special_tokens": {t: {"id": t, "ids": [i], "tokens": [t]}
                                              for i, t in ((101, "[CLS]"), (102, "[SEP]"))}},
        "decoder": None,
        "model": {"type": "WordPiece", "unk_token": "[UNK]", "continuing_subword_prefix": "##",
                  "max_input_chars_per_word": 100, "vocab": vocab},
    }
    return json.dumps(doc)


def make_texts(ids: np.ndarray, lengths) -> list:
    """The texts whose encodings under :func:`tokenizer_json` are ``ids``
    ([CLS] words [SEP] rows of a workload)."""
    return [" ".join(vocab_word(int(t)) for t in ids[b, 1:int(lengths[b]) - 1]) for b in range(ids.shape[0])]
