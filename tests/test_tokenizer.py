"""Native host tokenizer (ebh_tokenize) against the HF ``tokenizers`` library the
reference tokenises with (src/lib.rs:314-322, 577-601): the same tokenizer.json
read both ways, ids and masks compared exactly.  CPU only."""
import ctypes
import random
import string

import numpy as np
import pytest

from edgebert_amd import _native as N
from edgebert_amd.tokenizer import Tokenizer, hf_encode_batch_ids, hf_tokenizer

tokenizers = pytest.importorskip("tokenizers")
from tokenizers import AddedToken, models, normalizers, pre_tokenizers, processors  # noqa: E402

SPECIALS = {"[PAD]": 0, "[UNK]": 100, "[CLS]": 101, "[SEP]": 102, "[MASK]": 103}


def make_vocab():
    rng = random.Random(7)
    toks = ["[PAD]"] + [f"[unused{i}]" for i in range(1, 100)] + ["[UNK]", "[CLS]", "[SEP]", "[MASK]"]
    chars = (list(string.ascii_lowercase + string.ascii_uppercase + string.digits + string.punctuation)
             + list("éèüöäñçåøßæœ") + list("αβγδεζηθλμπσςω") + list("абвгдежзик")
             + list("中文字符日本語한국어") + list("ー。、«»“”¿¡—…€£¥"))
    toks += chars + ["##" + c for c in chars]
    words, pieces = set(), set()
    while len(words) < 3000:
        words.add("".join(rng.choice(string.ascii_lowercase) for _ in range(rng.randint(2, 8))))
    while len(pieces) < 1000:
        pieces.add("##" + "".join(rng.choice(string.ascii_lowercase) for _ in range(rng.randint(2, 5))))
    toks += sorted(words) + sorted(pieces)
    toks += ["café", "naïve", "Über", "straße", "σοφία", "привет", "İ", "i̇", "é"]
    seen, out = set(), []
    for t in toks:
        if t not in seen:
            seen.add(t)
            out.append(t)
    return {t: i for i, t in enumerate(out)}


VOCAB = make_vocab()
WORDS = [w for w in VOCAB if w.isalpha() and w.islower() and len(w) > 1 and w.isascii()]


def build(tmp_path, name="tokenizer.json", *, lowercase=True, strip_accents=None, clean_text=True,
          chinese=True, post="template", truncation=True, trunc_dir="right", padding=True,
          pad_left=False, pad_multiple=None, pad_id=0, added=None, max_chars=100):
    tok = tokenizers.Tokenizer(models.WordPiece(VOCAB, unk_token="[UNK]", max_input_chars_per_word=max_chars))
    tok.normalizer = normalizers.BertNormalizer(clean_text=clean_text, handle_chinese_chars=chinese,
                                                strip_accents=strip_accents, lowercase=lowercase)
    tok.pre_tokenizer = pre_tokenizers.BertPreTokenizer()
    if post == "template":
        tok.post_processor = processors.TemplateProcessing(
            single="[CLS] $A [SEP]", pair="[CLS] $A [SEP] $B:1 [SEP]:1",
            special_tokens=[("[CLS]", 101), ("[SEP]", 102)])
    elif post == "bert":
        tok.post_processor = processors.BertProcessing(("[SEP]", 102), ("[CLS]", 101))
    tok.add_special_tokens(added if added is not None else
                           [AddedToken(t, normalized=False) for t in SPECIALS])
    if truncation:
        tok.enable_truncation(128, direction=trunc_dir)   # the reference raises max_length to 512
    if padding:
        tok.enable_padding(pad_id=pad_id, pad_token="[PAD]", direction="left" if pad_left else "right",
                           pad_to_multiple_of=pad_multiple)
    path = str(tmp_path / name)
    tok.save(path)
    return path


def sentences(n, seed):
    rng = random.Random(seed)
    extra = ["Café", "NAÏVE", "Über", "straße", "ΣΟΦΊΑ", "Привет", "中文", "日本語", "한국어", "İstanbul",
             "éẗe", "¿qué?", "«quoted»", "“smart”", "a—b", "wait…", "€5", "x​y", "tab\there",
             "new\nline", "nb sp", "ideo　space", "[SEP]", "[sep]", "[MASK]", "##ing", "emoji😀ok",
             "\x00nul", "�rep", "soft­hyphen", "zw﻿nb", "x" * 120]
    out = []
    for _ in range(n):
        k = rng.randint(0, 40)
        toks = []
        for _ in range(k):
            r = rng.random()
            if r < 0.6:
                toks.append(rng.choice(WORDS))
            elif r < 0.7:
                toks.append(rng.choice(WORDS).capitalize())
            elif r < 0.8:
                toks.append(rng.choice(string.punctuation))
            else:
                toks.append(rng.choice(extra))
        out.append((" " if rng.random() < 0.8 else "").join(toks))
    return out


def compare(path, texts, nthreads=0):
    nt = Tokenizer.from_file(path)
    got_ids, got_mask = nt.encode_batch_ids(texts, nthreads=nthreads)
    want_ids, want_mask = hf_encode_batch_ids(hf_tokenizer(path), texts)
    assert got_ids.shape == want_ids.shape
    bad = np.nonzero((got_ids != want_ids).any(1) | (got_mask != want_mask).any(1))[0]
    assert bad.size == 0, [(texts[i], got_ids[i][got_mask[i] > 0].tolist(),
                            want_ids[i][want_mask[i] > 0].tolist()) for i in bad[:5]]
    return got_ids, got_mask


VARIANTS = {
    "uncased": {},
    "cased": dict(lowercase=False),
    "cased_strip": dict(lowercase=False, strip_accents=True),
    "lower_keep_accents": dict(strip_accents=False),
    "no_clean_no_cjk": dict(clean_text=False, chinese=False),
    "bert_processing_left_pad_multiple": dict(post="bert", pad_left=True, pad_multiple=8, pad_id=103),
    "no_padding_no_truncation_no_post": dict(post=None, padding=False, truncation=False),
    "short_words": dict(max_chars=6),
    "lstrip_rstrip_mask": dict(added=[AddedToken(t, normalized=False, lstrip=t == "[MASK]",
                                                 rstrip=t == "[MASK]") for t in SPECIALS]),
}


@pytest.mark.parametrize("variant", sorted(VARIANTS))
def test_matches_hf_tokenizers_on_mixed_text(tmp_path, variant):
    path = build(tmp_path, **VARIANTS[variant])
    compare(path, sentences(400, seed=len(variant)))


def test_every_bmp_code_point_and_a_sample_beyond(tmp_path):
    """Each character between letters: its class (dropped, space, CJK, split,
    punctuation, mark) and mapping (NFD, lowercase) end to end."""
    path = build(tmp_path)
    cps = [c for c in range(0x10000) if not 0xD800 <= c <= 0xDFFF] + list(range(0x10000, 0x110000, 97))
    texts = ["ab" + chr(c) + "Cd " + chr(c) for c in cps]
    compare(path, texts)
    cased = build(tmp_path, "cased.json", lowercase=False)
    compare(cased, texts[::5])


def test_combining_mark_runs_are_reordered_then_stripped(tmp_path):
    """NFD puts each run of combining marks in canonical order before the
    non-spacing ones are dropped (cased + strip keeps spacing marks)."""
    rng = random.Random(3)
    marks = [0x0301, 0x0316, 0x0308, 0x0327, 0x031B, 0x0345, 0x05B0, 0x093C, 0x0903, 0x0F71, 0x1D165,
             0x1D16D, 0x0BCD, 0x302A, 0x20D2]
    bases = "aeiouAEIOUnçÅ한가"
    texts = ["".join(rng.choice(bases) + "".join(chr(rng.choice(marks)) for _ in range(rng.randint(0, 4)))
                     for _ in range(rng.randint(1, 8))) for _ in range(500)]
    for kw in ({}, dict(lowercase=False, strip_accents=True)):
        compare(build(tmp_path, f"t{len(kw)}.json", **kw), texts)


def test_truncation_to_512_with_specials(tmp_path):
    path = build(tmp_path)
    long_text = " ".join(random.Random(1).choice(WORDS) for _ in range(900))
    ids, mask = compare(path, [long_text, "short"])
    assert ids.shape == (2, 512) and ids[0, 0] == 101 and ids[0, 511] == 102
    left = build(tmp_path, "left.json", trunc_dir="left")
    ids, _ = compare(left, [long_text])
    assert ids[0, 0] == 101 and ids[0, -1] == 102


def test_threads_do_not_change_results(tmp_path):
    path = build(tmp_path)
    texts = sentences(300, seed=11)
    one, _ = Tokenizer.from_file(path).encode_batch_ids(texts, nthreads=1)
    many, _ = Tokenizer.from_file(path).encode_batch_ids(texts, nthreads=8)
    assert np.array_equal(one, many)


def test_empty_batch_and_empty_texts(tmp_path):
    nt = Tokenizer.from_file(build(tmp_path))
    ids, mask = nt.encode_batch_ids([])
    assert ids.shape == (0, 0)
    ids, mask = nt.encode_batch_ids(["", " \t\n", "\x00"])
    assert ids.tolist() == [[101, 102]] * 3 and mask.tolist() == [[1, 1]] * 3


def test_invalid_utf8_reads_as_replacement_character(tmp_path):
    """A byte that is not UTF-8 reads as U+FFFD, which clean_text drops."""
    nt = Tokenizer.from_file(build(tmp_path))
    L = N.lib()
    texts = (ctypes.c_char_p * 2)(b"ab\xffcd \xe2\x82", b"abcd")
    ids = np.zeros(64, np.int32)
    mask = np.zeros(64, np.int32)
    S = ctypes.c_int32()
    N.check(L.ebh_tokenize(nt.handle, texts, None, 2, 32, ids.ctypes.data, mask.ctypes.data,
                           ctypes.byref(S), 1))
    s = S.value
    assert ids[:s].tolist() == ids[s:2 * s].tolist()


def test_cap_too_small_is_an_error(tmp_path):
    nt = Tokenizer.from_file(build(tmp_path))
    with pytest.raises(N.EbhError) as e:
        nt.encode_batch_ids(["one two three four"], cap=3)
    assert e.value.code == N.EBH_ERR_RANGE


@pytest.mark.parametrize("mutate,what", [
    (lambda d: d.update(normalizer={"type": "Lowercase"}), "normalizer"),
    (lambda d: d.update(pre_tokenizer={"type": "Whitespace"}), "pre_tokenizer"),
    (lambda d: d["model"].update(type="BPE"), "WordPiece"),
    (lambda d: d["added_tokens"][0].update(normalized=True), "normalized"),
    (lambda d: d["model"].update(unk_token="[NOPE]"), "unk token"),
])
def test_unsupported_files_are_rejected(tmp_path, mutate, what):
    import json
    d = json.load(open(build(tmp_path)))
    mutate(d)
    with pytest.raises(N.EbhError) as e:
        Tokenizer.from_str(json.dumps(d))
    assert e.value.code == N.EBH_ERR_SHAPE and what in str(e.value)


def test_missing_file_and_bad_json(tmp_path):
    with pytest.raises(N.EbhError) as e:
        Tokenizer.from_file(str(tmp_path / "nope.json"))
    assert e.value.code == N.EBH_ERR_NOT_FOUND
    with pytest.raises(N.EbhError) as e:
        Tokenizer.from_str('{"model": ')
    assert e.value.code == N.EBH_ERR_SHAPE


def test_json_surrogate_pair_escapes(tmp_path):
    """tokenizer.json written with \\uXXXX escapes (non-BMP as surrogate pairs)."""
    import json
    d = json.load(open(build(tmp_path)))
    d["model"]["vocab"]["😀"] = len(d["model"]["vocab"])
    path = tmp_path / "ascii.json"
    path.write_text(json.dumps(d, ensure_ascii=True))
    compare(str(path), ["ok 😀 ok", "😀😀"])
