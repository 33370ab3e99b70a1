"""edgebert_amd -- MI355X (gfx950) BERT encoder forward behind EdgeBERT's
``Model::forward`` / ``encode`` boundary.

The compute path is ``libedgebert_hip.so`` (hand-written HIP kernels + C ABI,
``include/edgebert_hip.h``); this package is its host-side mirror of the
reference ``Model`` API.  There is no CPU fallback: without the built
library every entry point raises.
"""
from .synth import BertConfig, MINILM_L6, BERT_BASE, TINY, CONFIGS, make_weights, make_inputs
from ._native import EbhError, lib, header_symbols
from .model import Model, cosine_similarity
from .tokenizer import Tokenizer

__all__ = ["BertConfig", "MINILM_L6", "BERT_BASE", "TINY", "CONFIGS", "make_weights",
           "make_inputs", "EbhError", "lib", "header_symbols", "Model", "cosine_similarity",
           "Tokenizer"]
