// tokenizer.cpp -- native BERT WordPiece tokenizer behind ebh_tokenize,
// ebh_encode_texts and ebh_score_texts.
//
// Replaces the host tokenization of the reference: Tokenizer::from_file
// ("tokenizer.json") with padding switched to BatchLongest and truncation to
// max_length 512 (src/lib.rs:310-322), then encode_batch(texts, true)
// marshalled into [B, max_len] ids / mask (src/lib.rs:577-601; score_pair,
// src/lib.rs:326-340, encodes "query [SEP] document" the same way).  The
// reference's tokenizer is the HF `tokenizers` crate; this is a restatement of
// its BERT pipeline for the tokenizer.json files BERT models ship:
//   * added tokens (normalized = false): matched in the raw text, leftmost
//     longest first, each becoming its id (lstrip / rstrip take the
//     whitespace beside them);
//   * BertNormalizer: clean_text (drop NUL, U+FFFD and "other" characters,
//     whitespace -> ' '), handle_chinese_chars (' ' around CJK ideographs),
//     strip_accents (NFD, then drop non-spacing marks; defaults to
//     `lowercase`), lowercase;
//   * BertPreTokenizer: split on whitespace, isolate punctuation;
//   * WordPiece: greedy longest-prefix match, continuation pieces looked up
//     with the subword prefix ("##"), a word with an unmatched rest or longer
//     than max_input_chars_per_word becomes the unk token;
//   * post-processing: TemplateProcessing / BertProcessing specials around the
//     sequence; truncation of the sequence to max_length minus those specials;
//     padding to the batch's longest (rounded to pad_to_multiple_of).
// Character classes and mappings come from unicode_tables.inc, read off the
// `tokenizers` library itself by gen_unicode_tables.py.  Texts are encoded on
// a pool of host threads; the ids are written straight into the caller's
// (or the model's pinned staging) [B, S] buffers.
#include <algorithm>
#include <atomic>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "../../include/edgebert_hip.h"
#include "internal.hpp"
#include "json.hpp"

struct ebh_tokenizer {
    // normalizer
    bool clean = false, chinese = false, strip = false, lower = false;
    // WordPiece vocabulary: every token, and the continuation tokens keyed
    // without their prefix.
    struct Table {
        struct Slot { uint32_t hash = 0, off = 0; int32_t len = 0, id = -1; };
        std::vector<uint32_t> arena;
        std::vector<Slot> slots;
        uint32_t mask = 0;
        int max_len = 0;

        static uint32_t hash(const uint32_t* s, int n) {
            uint32_t h = 2166136261u;
            for (int i = 0; i < n; ++i) {
                h ^= s[i];
                h *= 16777619u;
                h ^= h >> 15;
            }
            return h;
        }
        void init(size_t n) {
            size_t cap = 16;
            while (cap < 2 * n + 2) cap <<= 1;
            slots.assign(cap, Slot{});
            mask = (uint32_t)cap - 1;
        }
        void insert(const uint32_t* s, int n, int id) {
            const uint32_t h = hash(s, n);
            for (uint32_t i = h & mask;; i = (i + 1) & mask) {
                Slot& sl = slots[i];
                if (sl.id < 0) {
                    sl.hash = h;
                    sl.off = (uint32_t)arena.size();
                    sl.len = n;
                    sl.id = id;
                    arena.insert(arena.end(), s, s + n);
                    max_len = std::max(max_len, n);
                    return;
                }
                if (sl.hash == h && sl.len == n && !memcmp(&arena[sl.off], s, 4 * (size_t)n)) {
                    sl.id = id;
                    return;
                }
            }
        }
        int find(const uint32_t* s, int n) const {
            if (n > max_len || slots.empty()) return -1;
            const uint32_t h = hash(s, n);
            for (uint32_t i = h & mask;; i = (i + 1) & mask) {
                const Slot& sl = slots[i];
                if (sl.id < 0) return -1;
                if (sl.hash == h && sl.len == n && !memcmp(&arena[sl.off], s, 4 * (size_t)n)) return sl.id;
            }
        }
    };
    Table vocab, cont;
    int unk_id = -1;
    int max_chars_per_word = 100;
    // added tokens, matched in the raw text
    struct Added { std::vector<uint32_t> text; int id; bool lstrip, rstrip; };
    std::vector<Added> added;
    // post-processing of a single sequence
    std::vector<int32_t> prefix, suffix;
    bool truncate = false, trunc_left = false;
    int trunc_max = 0;
    int pad_id = 0, pad_multiple = 0;
    bool pad_left = false;
    int vocab_size = 0;
};

namespace {

using ebh::json::JVal;
using ebh::json::get;
int fail(int code, const std::string& msg) { return ebh::set_error(code, "%s", msg.c_str()); }

#include "unicode_tables.inc"

enum : uint16_t {
    C_DROP = 1, C_SPACE = 2, C_CJK = 4, C_SPLIT = 8, C_PUNCT = 16, C_MARK = 32, C_NFD = 64, C_LOWER = 128,
    C_CCC = 256
};
constexpr uint32_t kMaxCp = 0x110000;

// Per-code-point flags of the tables above (2.2 MB, built once).
const uint16_t* char_flags() {
    static std::vector<uint16_t> f;
    static std::once_flag once;
    std::call_once(once, [] {
        f.assign(kMaxCp, 0);
        auto mark = [&](const uint32_t (*r)[2], size_t n, uint16_t bit) {
            for (size_t i = 0; i < n; ++i)
                for (uint32_t c = r[i][0]; c <= r[i][1]; ++c) f[c] |= bit;
        };
#define EBH_MARK(T, B) mark(T, sizeof(T) / sizeof(T[0]), B)
        EBH_MARK(kCleanDrop, C_DROP);
        EBH_MARK(kCleanSpace, C_SPACE);
        EBH_MARK(kChinese, C_CJK);
        EBH_MARK(kSplitSpace, C_SPLIT);
        EBH_MARK(kPunct, C_PUNCT);
        EBH_MARK(kNonspacingMark, C_MARK);
#undef EBH_MARK
        for (const auto& e : kNfd) f[e[0]] |= C_NFD;
        for (uint32_t c = 0xAC00; c <= 0xD7A3; ++c) f[c] |= C_NFD;   // Hangul syllables
        for (const auto& e : kLower) f[e[0]] |= C_LOWER;
        for (const auto& e : kCombiningClass)
            for (uint32_t c = e[0]; c <= e[1]; ++c) f[c] |= C_CCC;
    });
    return f.data();
}

inline uint16_t flags_of(const uint16_t* F, uint32_t c) { return c < kMaxCp ? F[c] : 0; }

template <size_t W>
const uint32_t* find_row(const uint32_t (*t)[W], size_t n, uint32_t cp) {
    size_t lo = 0, hi = n;
    while (lo < hi) {
        const size_t mid = (lo + hi) / 2;
        if (t[mid][0] < cp) lo = mid + 1;
        else hi = mid;
    }
    return lo < n && t[lo][0] == cp ? t[lo] : nullptr;
}

int combining_class(uint32_t cp) {
    size_t lo = 0, hi = sizeof(kCombiningClass) / sizeof(kCombiningClass[0]);
    while (lo < hi) {
        const size_t mid = (lo + hi) / 2;
        if (kCombiningClass[mid][1] < cp) lo = mid + 1;
        else hi = mid;
    }
    return lo < sizeof(kCombiningClass) / sizeof(kCombiningClass[0]) && kCombiningClass[lo][0] <= cp
               ? (int)kCombiningClass[lo][2]
               : 0;
}

// UTF-8 -> code points; an invalid or truncated sequence reads as U+FFFD
// (which clean_text drops), one byte at a time.
void decode_utf8(const char* s, size_t n, std::vector<uint32_t>& out) {
    out.clear();
    const unsigned char* p = reinterpret_cast<const unsigned char*>(s);
    size_t i = 0;
    while (i < n) {
        const unsigned c = p[i];
        if (c < 0x80) { out.push_back(c); ++i; continue; }
        int len = 0;
        uint32_t cp = 0, min = 0;
        if ((c & 0xE0) == 0xC0) { len = 2; cp = c & 0x1F; min = 0x80; }
        else if ((c & 0xF0) == 0xE0) { len = 3; cp = c & 0x0F; min = 0x800; }
        else if ((c & 0xF8) == 0xF0) { len = 4; cp = c & 0x07; min = 0x10000; }
        bool ok = len > 0 && i + len <= n;
        for (int k = 1; ok && k < len; ++k) {
            if ((p[i + k] & 0xC0) != 0x80) ok = false;
            else cp = (cp << 6) | (p[i + k] & 0x3F);
        }
        if (ok && (cp < min || cp >= kMaxCp || (cp >= 0xD800 && cp <= 0xDFFF))) ok = false;
        if (ok) { out.push_back(cp); i += len; }
        else { out.push_back(0xFFFD); ++i; }
    }
}

struct Scratch {
    std::vector<uint32_t> text, a, b;
    std::vector<int32_t> ids;
};

// BertNormalizer over in[0..n) -> out.
void normalize(const ebh_tokenizer& t, const uint16_t* F, const uint32_t* in, size_t n, std::vector<uint32_t>& out,
               std::vector<uint32_t>& tmp) {
    out.clear();
    for (size_t i = 0; i < n; ++i) {
        uint32_t c = in[i];
        const uint16_t f = flags_of(F, c);
        if (t.clean) {
            if (f & C_DROP) continue;
            if (f & C_SPACE) c = ' ';
        }
        if (t.chinese && (f & C_CJK)) {
            out.push_back(' ');
            out.push_back(c);
            out.push_back(' ');
        } else {
            out.push_back(c);
        }
    }
    if (t.strip) {
        // NFD: full canonical decomposition, then each run of combining marks
        // in stable order of combining class; then drop non-spacing marks.
        tmp.clear();
        for (uint32_t c : out) {
            const uint16_t f = flags_of(F, c);
            if (!(f & C_NFD)) { tmp.push_back(c); continue; }
            if (c >= 0xAC00 && c <= 0xD7A3) {
                const uint32_t s = c - 0xAC00;
                tmp.push_back(0x1100 + s / 588);
                tmp.push_back(0x1161 + (s % 588) / 28);
                if (s % 28) tmp.push_back(0x11A7 + s % 28);
                continue;
            }
            const uint32_t* row = find_row(kNfd, sizeof(kNfd) / sizeof(kNfd[0]), c);
            for (int k = 1; k <= kNfdWidth && row[k]; ++k) tmp.push_back(row[k]);
        }
        for (size_t i = 0; i < tmp.size();) {
            if (!(flags_of(F, tmp[i]) & C_CCC)) { ++i; continue; }
            size_t j = i;
            while (j < tmp.size() && (flags_of(F, tmp[j]) & C_CCC)) ++j;
            if (j - i > 1)
                std::stable_sort(tmp.begin() + i, tmp.begin() + j,
                                 [](uint32_t x, uint32_t y) { return combining_class(x) < combining_class(y); });
            i = j;
        }
        out.clear();
        for (uint32_t c : tmp)
            if (!(flags_of(F, c) & C_MARK)) out.push_back(c);
    }
    if (t.lower) {
        bool any = false;
        for (uint32_t c : out)
            if (flags_of(F, c) & C_LOWER) { any = true; break; }
        if (any) {
            tmp.clear();
            for (uint32_t c : out) {
                if (!(flags_of(F, c) & C_LOWER)) { tmp.push_back(c); continue; }
                const uint32_t* row = find_row(kLower, sizeof(kLower) / sizeof(kLower[0]), c);
                for (int k = 1; k <= kLowerWidth && row[k]; ++k) tmp.push_back(row[k]);
            }
            out.swap(tmp);
        }
    }
}

// WordPiece of one word w[0..n) (WordPiece::tokenize of the tokenizers crate).
void wordpiece(const ebh_tokenizer& t, const uint32_t* w, int n, std::vector<int32_t>& ids) {
    if (n > t.max_chars_per_word) { ids.push_back(t.unk_id); return; }
    const size_t mark = ids.size();
    int start = 0;
    while (start < n) {
        const ebh_tokenizer::Table& tab = start == 0 ? t.vocab : t.cont;
        int end = std::min(n, start + tab.max_len);
        int id = -1;
        for (; end > start; --end)
            if ((id = tab.find(w + start, end - start)) >= 0) break;
        if (id < 0) {
            ids.resize(mark);
            ids.push_back(t.unk_id);
            return;
        }
        ids.push_back(id);
        start = end;
    }
}

// Normalised, pre-tokenised and WordPiece'd segment (text between added tokens).
void encode_segment(const ebh_tokenizer& t, const uint16_t* F, const uint32_t* s, size_t n, Scratch& sc) {
    normalize(t, F, s, n, sc.a, sc.b);
    const std::vector<uint32_t>& x = sc.a;
    size_t i = 0;
    while (i < x.size()) {
        const uint16_t f = flags_of(F, x[i]);
        if (f & C_SPLIT) { ++i; continue; }
        if (f & C_PUNCT) {
            wordpiece(t, &x[i], 1, sc.ids);
            ++i;
            continue;
        }
        size_t j = i + 1;
        while (j < x.size() && !(flags_of(F, x[j]) & (C_SPLIT | C_PUNCT))) ++j;
        wordpiece(t, &x[i], (int)(j - i), sc.ids);
        i = j;
    }
}

// Content ids of one text (added tokens split out first), before post-processing.
void encode_text(const ebh_tokenizer& t, const char* text, size_t len, Scratch& sc) {
    const uint16_t* F = char_flags();
    sc.ids.clear();
    decode_utf8(text, len, sc.text);
    const std::vector<uint32_t>& x = sc.text;
    const size_t n = x.size();
    size_t seg = 0;   // start of the pending plain segment
    size_t i = 0;
    while (i < n) {
        int best = -1;
        size_t best_len = 0;
        for (size_t k = 0; k < t.added.size(); ++k) {
            const std::vector<uint32_t>& a = t.added[k].text;
            if (a.size() > best_len && a.size() <= n - i && !memcmp(&x[i], a.data(), 4 * a.size())) {
                best = (int)k;
                best_len = a.size();
            }
        }
        if (best < 0) { ++i; continue; }
        size_t start = i, stop = i + best_len;
        if (t.added[best].lstrip)
            while (start > seg && (flags_of(F, x[start - 1]) & C_SPLIT)) --start;
        if (t.added[best].rstrip)
            while (stop < n && (flags_of(F, x[stop]) & C_SPLIT)) ++stop;
        if (start > seg) encode_segment(t, F, &x[seg], start - seg, sc);
        sc.ids.push_back(t.added[best].id);
        seg = i = stop;
    }
    if (n > seg) encode_segment(t, F, &x[seg], n - seg, sc);
}

// Truncation and specials of one sequence (add_special_tokens = true).
void finish(const ebh_tokenizer& t, const std::vector<int32_t>& content, std::vector<int32_t>& out) {
    size_t lo = 0, hi = content.size();
    if (t.truncate) {
        const int added = (int)(t.prefix.size() + t.suffix.size());
        const size_t keep = (size_t)std::max(0, t.trunc_max - added);
        if (hi > keep) {
            if (t.trunc_left) lo = hi - keep;
            else hi = keep;
        }
    }
    out.clear();
    out.insert(out.end(), t.prefix.begin(), t.prefix.end());
    out.insert(out.end(), content.begin() + lo, content.begin() + hi);
    out.insert(out.end(), t.suffix.begin(), t.suffix.end());
}

int vocab_id(const ebh_tokenizer& t, const std::string& tok) {
    std::vector<uint32_t> u;
    decode_utf8(tok.data(), tok.size(), u);
    return t.vocab.find(u.data(), (int)u.size());
}

bool as_bool(const JVal* v, bool dflt) { return v && v->kind == JVal::BOOL ? v->num != 0 : dflt; }

int build(ebh_tokenizer& t, const JVal& root) {
    if (root.kind != JVal::OBJ) return fail(EBH_ERR_SHAPE, "tokenizer.json: not a JSON object");
    const JVal* model = get(root, "model");
    const JVal* mtype = model ? get(*model, "type") : nullptr;
    if (!model || !mtype || mtype->kind != JVal::STR || mtype->str != "WordPiece")
        return fail(EBH_ERR_SHAPE, "tokenizer.json: model.type must be WordPiece");
    const JVal* vocab = get(*model, "vocab");
    if (!vocab || vocab->kind != JVal::OBJ || vocab->obj.empty())
        return fail(EBH_ERR_SHAPE, "tokenizer.json: model.vocab missing");
    std::string prefix = "##";
    if (const JVal* p = get(*model, "continuing_subword_prefix"); p && p->kind == JVal::STR) prefix = p->str;
    if (const JVal* m = get(*model, "max_input_chars_per_word"); m && m->kind == JVal::NUM)
        t.max_chars_per_word = (int)m->num;
    std::vector<uint32_t> pre, u;
    decode_utf8(prefix.data(), prefix.size(), pre);
    t.vocab.init(vocab->obj.size());
    size_t ncont = 0;
    for (const auto& kv : vocab->obj)
        if (kv.first.compare(0, prefix.size(), prefix) == 0 && !prefix.empty()) ++ncont;
    t.cont.init(ncont);
    for (const auto& kv : vocab->obj) {
        if (kv.second.kind != JVal::NUM || kv.second.num < 0 || kv.second.num > 2147483647.0)
            return fail(EBH_ERR_SHAPE, "tokenizer.json: bad id for vocab entry " + kv.first);
        const int id = (int)kv.second.num;
        t.vocab_size = std::max(t.vocab_size, id + 1);
        decode_utf8(kv.first.data(), kv.first.size(), u);
        t.vocab.insert(u.data(), (int)u.size(), id);
        if (!pre.empty() && u.size() >= pre.size() && std::equal(pre.begin(), pre.end(), u.begin()))
            t.cont.insert(u.data() + pre.size(), (int)(u.size() - pre.size()), id);
    }
    std::string unk = "[UNK]";
    if (const JVal* p = get(*model, "unk_token"); p && p->kind == JVal::STR) unk = p->str;
    if ((t.unk_id = vocab_id(t, unk)) < 0)
        return fail(EBH_ERR_SHAPE, "tokenizer.json: unk token " + unk + " not in the vocabulary");

    const JVal* norm = get(root, "normalizer");
    if (norm && norm->kind != JVal::NUL) {
        const JVal* ty = get(*norm, "type");
        if (!ty || ty->kind != JVal::STR || ty->str != "BertNormalizer")
            return fail(EBH_ERR_SHAPE, "tokenizer.json: unsupported normalizer (supported: BertNormalizer)");
        t.clean = as_bool(get(*norm, "clean_text"), true);
        t.chinese = as_bool(get(*norm, "handle_chinese_chars"), true);
        t.lower = as_bool(get(*norm, "lowercase"), true);
        const JVal* sa = get(*norm, "strip_accents");
        t.strip = sa && sa->kind == JVal::BOOL ? sa->num != 0 : t.lower;
    }
    const JVal* pt = get(root, "pre_tokenizer");
    const JVal* pty = pt ? get(*pt, "type") : nullptr;
    if (!pty || pty->kind != JVal::STR || pty->str != "BertPreTokenizer")
        return fail(EBH_ERR_SHAPE, "tokenizer.json: unsupported pre_tokenizer (supported: BertPreTokenizer)");

    if (const JVal* at = get(root, "added_tokens"); at && at->kind == JVal::ARR) {
        for (const JVal& a : at->arr) {
            const JVal* content = get(a, "content");
            const JVal* id = get(a, "id");
            if (!content || content->kind != JVal::STR || !id || id->kind != JVal::NUM)
                return fail(EBH_ERR_SHAPE, "tokenizer.json: bad added token");
            if (as_bool(get(a, "normalized"), false) || as_bool(get(a, "single_word"), false))
                return fail(EBH_ERR_SHAPE, "tokenizer.json: added token " + content->str +
                                               " is normalized or single_word (not supported)");
            ebh_tokenizer::Added ad;
            decode_utf8(content->str.data(), content->str.size(), ad.text);
            if (ad.text.empty()) continue;
            ad.id = (int)id->num;
            ad.lstrip = as_bool(get(a, "lstrip"), false);
            ad.rstrip = as_bool(get(a, "rstrip"), false);
            t.vocab_size = std::max(t.vocab_size, ad.id + 1);
            t.added.push_back(std::move(ad));
        }
    }

    if (const JVal* pp = get(root, "post_processor"); pp && pp->kind != JVal::NUL) {
        const JVal* ty = get(*pp, "type");
        const std::string kind = ty && ty->kind == JVal::STR ? ty->str : "";
        if (kind == "BertProcessing") {
            const JVal* cls = get(*pp, "cls");
            const JVal* sep = get(*pp, "sep");
            if (!cls || !sep || cls->kind != JVal::ARR || sep->kind != JVal::ARR || cls->arr.size() != 2 ||
                sep->arr.size() != 2)
                return fail(EBH_ERR_SHAPE, "tokenizer.json: bad BertProcessing");
            t.prefix = {(int32_t)cls->arr[1].num};
            t.suffix = {(int32_t)sep->arr[1].num};
        } else if (kind == "TemplateProcessing") {
            const JVal* single = get(*pp, "single");
            const JVal* specials = get(*pp, "special_tokens");
            if (!single || single->kind != JVal::ARR)
                return fail(EBH_ERR_SHAPE, "tokenizer.json: TemplateProcessing without a single template");
            int seqs = 0;
            for (const JVal& piece : single->arr) {
                if (get(piece, "Sequence")) { ++seqs; continue; }
                const JVal* sp = get(piece, "SpecialToken");
                const JVal* sid = sp ? get(*sp, "id") : nullptr;
                const JVal* def = sid && specials ? get(*specials, sid->str.c_str()) : nullptr;
                const JVal* ids = def ? get(*def, "ids") : nullptr;
                if (!ids || ids->kind != JVal::ARR)
                    return fail(EBH_ERR_SHAPE, "tokenizer.json: TemplateProcessing special token without ids");
                for (const JVal& x : ids->arr) (seqs ? t.suffix : t.prefix).push_back((int32_t)x.num);
            }
            if (seqs != 1) return fail(EBH_ERR_SHAPE, "tokenizer.json: single template must hold one sequence");
        } else {
            return fail(EBH_ERR_SHAPE, "tokenizer.json: unsupported post_processor " + kind);
        }
    }
    // The reference keeps the file's truncation with max_length 512 and the
    // file's padding with the BatchLongest strategy (src/lib.rs:317-322).
    if (const JVal* tr = get(root, "truncation"); tr && tr->kind == JVal::OBJ) {
        t.truncate = true;
        t.trunc_max = 512;
        const JVal* dir = get(*tr, "direction");
        t.trunc_left = dir && dir->kind == JVal::STR && dir->str == "Left";
    }
    if (const JVal* pd = get(root, "padding"); pd && pd->kind == JVal::OBJ) {
        if (const JVal* v = get(*pd, "pad_id"); v && v->kind == JVal::NUM) t.pad_id = (int)v->num;
        if (const JVal* v = get(*pd, "pad_to_multiple_of"); v && v->kind == JVal::NUM) t.pad_multiple = (int)v->num;
        const JVal* dir = get(*pd, "direction");
        t.pad_left = dir && dir->kind == JVal::STR && dir->str == "Left";
    }
    return EBH_OK;
}

int load_json(const char* data, size_t n, ebh_tokenizer** out) {
    ebh::json::Parser ps{data, data + n, {}};
    JVal root;
    if (!ps.parse(root)) return fail(EBH_ERR_SHAPE, "tokenizer.json: bad JSON: " + ps.err);
    std::unique_ptr<ebh_tokenizer> t(new ebh_tokenizer);
    int rc = build(*t, root);
    if (rc) return rc;
    char_flags();
    *out = t.release();
    return EBH_OK;
}

}  // namespace

namespace ebh {

int tokenize_batch(const ebh_tokenizer* t, const char* const* texts, const int64_t* lens, int n, int nthreads,
                   std::vector<std::vector<int32_t>>& seqs, int* S_out) {
    if (!t || (n > 0 && !texts)) return fail(EBH_ERR_INVALID_ARG, "null argument");
    if (n < 0) return fail(EBH_ERR_INVALID_ARG, "negative batch");
    for (int i = 0; i < n; ++i) {
        if (!texts[i] && !(lens && lens[i] == 0)) return fail(EBH_ERR_INVALID_ARG, "null text at " + std::to_string(i));
        if (lens && lens[i] < 0) return fail(EBH_ERR_INVALID_ARG, "negative text length at " + std::to_string(i));
    }
    seqs.resize(n);
    int hw = (int)std::thread::hardware_concurrency();
    if (nthreads <= 0) nthreads = std::min(std::max(hw, 1), 16);
    nthreads = std::max(1, std::min(nthreads, (n + 7) / 8));
    std::atomic<int> next{0};
    auto work = [&]() {
        Scratch sc;
        for (;;) {
            const int i0 = next.fetch_add(8);
            if (i0 >= n) break;
            for (int i = i0; i < std::min(n, i0 + 8); ++i) {
                encode_text(*t, texts[i] ? texts[i] : "", lens ? (size_t)lens[i] : strlen(texts[i]), sc);
                finish(*t, sc.ids, seqs[i]);
            }
        }
    };
    if (nthreads == 1) {
        work();
    } else {
        std::vector<std::thread> pool;
        for (int k = 1; k < nthreads; ++k) pool.emplace_back(work);
        work();
        for (auto& th : pool) th.join();
    }
    int S = 0;
    for (const auto& s : seqs) S = std::max(S, (int)s.size());
    if (t->pad_multiple > 0 && S % t->pad_multiple) S += t->pad_multiple - S % t->pad_multiple;
    *S_out = S;
    return EBH_OK;
}

void write_padded(const ebh_tokenizer* t, const std::vector<std::vector<int32_t>>& seqs, int S, int32_t* ids,
                  int32_t* mask) {
    for (size_t b = 0; b < seqs.size(); ++b) {
        const std::vector<int32_t>& s = seqs[b];
        const int len = (int)s.size(), off = t->pad_left ? S - len : 0;
        int32_t* ir = ids + b * (size_t)S;
        int32_t* mr = mask + b * (size_t)S;
        for (int j = 0; j < S; ++j) {
            const bool real = j >= off && j < off + len;
            ir[j] = real ? s[j - off] : t->pad_id;
            mr[j] = real ? 1 : 0;
        }
    }
}

int tokenizer_vocab_size(const ebh_tokenizer* t) { return t->vocab_size; }

}  // namespace ebh

extern "C" {

int ebh_tokenizer_from_json(const char* json, size_t len, ebh_tokenizer** out) {
    if (!json || !out) return fail(EBH_ERR_INVALID_ARG, "null argument");
    *out = nullptr;
    return load_json(json, len, out);
}

int ebh_tokenizer_load(const char* path, ebh_tokenizer** out) {
    if (!path || !out) return fail(EBH_ERR_INVALID_ARG, "null argument");
    *out = nullptr;
    std::unique_ptr<FILE, int (*)(FILE*)> f(fopen(path, "rb"), fclose);
    if (!f) return fail(EBH_ERR_NOT_FOUND, std::string("cannot open ") + path);
    std::string data;
    char buf[1 << 16];
    size_t k;
    while ((k = fread(buf, 1, sizeof buf, f.get())) > 0) data.append(buf, k);
    return load_json(data.data(), data.size(), out);
}

void ebh_tokenizer_destroy(ebh_tokenizer* t) { delete t; }

int ebh_tokenize(const ebh_tokenizer* t, const char* const* texts, const int64_t* lens, int32_t n, int32_t cap,
                 int32_t* ids, int32_t* mask, int32_t* S_out, int32_t nthreads) {
    if (!S_out) return fail(EBH_ERR_INVALID_ARG, "null argument");
    *S_out = 0;
    std::vector<std::vector<int32_t>> seqs;
    int S = 0;
    int rc = ebh::tokenize_batch(t, texts, lens, n, nthreads, seqs, &S);
    if (rc) return rc;
    if (S > cap)
        return fail(EBH_ERR_RANGE, "a sequence needs " + std::to_string(S) + " positions, cap is " +
                                       std::to_string(cap));
    if (n > 0 && (!ids || !mask)) return fail(EBH_ERR_INVALID_ARG, "null output buffer");
    ebh::write_padded(t, seqs, S, ids, mask);
    *S_out = S;
    return EBH_OK;
}

}  // extern "C"
