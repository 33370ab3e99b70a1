// api.cpp -- host side of the C ABI: weight store, workspace, forward.
//
// Mirrors the reference's Model (src/lib.rs:40-106, 155-260, 573-666):
//   ebh_create / ebh_set_tensor / ebh_finalize   <- Model::from_weights
//   ebh_forward                                  <- Model::forward
//   ebh_encode / ebh_encode_device               <- encode_uncached (after tokenisation)
// All device work of one model runs on one HIP stream in this order:
//   pack -> embed+LN -> L x [QKV GEMM, attention, out GEMM(+res), LN,
//   up GEMM(+GELU), down GEMM(+res), LN] -> pool(+normalise).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/edgebert_hip.h"
#include "../../include/edgebert_hip_ops.h"
#include "internal.hpp"
#include "kernels.hpp"

namespace {
thread_local std::string g_err;
}  // namespace

namespace ebh {
int set_error(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}
}  // namespace ebh

namespace {

using ebh::set_error;
#define fail set_error

#define HIP_TRY(expr)                                                                     \
    do {                                                                                  \
        hipError_t e_ = (expr);                                                           \
        if (e_ != hipSuccess)                                                             \
            return fail(EBH_ERR_HIP, "%s failed: %s", #expr, hipGetErrorString(e_));      \
    } while (0)

constexpr size_t kAlign = 256;
size_t align_up(size_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

// A tensor handed over before ebh_finalize, in its checkpoint encoding: a
// copy of the caller's f32 data (ebh_set_tensor), or a view of F32 / F16 /
// BF16 elements inside a mapped safetensors file (`keep` holds the mapping).
// ebh_finalize uploads each one straight into its place in the device block.
struct HostTensor {
    std::vector<int64_t> shape;
    int kind = ebh::TENSOR_F32;
    const void* src = nullptr;
    std::vector<float> own;
    std::shared_ptr<const void> keep;
    int64_t count() const {
        int64_t n = 1;
        for (int64_t d : shape) n *= d;
        return n;
    }
};

struct DevLayer {
    float *wqkv, *bqkv, *wo, *bo, *ln1_g, *ln1_b, *w1, *b1, *w2, *b2, *ln2_g, *ln2_b;
    uint16_t *wqkv16, *wo16, *w116, *w216;
};

struct Workspace {
    void* base = nullptr;
    int64_t tok_cap = 0;  // B*S tokens
    int b_cap = 0;
    int y_parts = 1;      // Y holds y_parts * tok_cap rows (split-K partial products)
    float *X, *Y, *QKV, *CTX, *F;
    uint16_t* X16;  // bf16 copy of X (bf16 models: the GEMM input)
    int *ids, *mask, *counts, *cu, *ntok, *tok_id, *tok_pos, *err;
    int* order;     // [B] sequences by decreasing length (written by launch_pack)
    float* out;
    float* scores;  // [B] cross-encoder scores
};

struct ProfPair {
    hipEvent_t a, b;
};

// A whole forward recorded as a HIP graph, for calls that repeat one shape on
// the same buffers (serving loops, small batches whose forward is mostly
// launch overhead).  Keyed by everything the recorded launches bake in.
struct GraphEntry {
    int B, S, normalize, host;
    const void *ids, *mask;
    void *out, *scores;
    int64_t tokens;                   // host calls: the exact token count; else -1
    int seen;                         // calls with this key; -1: recording failed
    hipGraphExec_t exec;              // recorded at the key's second call
    uint64_t used;
};
constexpr size_t MAX_GRAPHS = 16;

// Pinned host staging of the blocking entry points.  There are two sets, so a
// caller's forward can be enqueued behind another caller's while that one
// still runs or is being copied out.  A caller holds its slot from staging to
// copy-out, and the model's lock only while it stages and enqueues.
struct HostSlot {
    int* ids = nullptr;
    int* mask = nullptr;
    float* out = nullptr;
    int64_t cap = 0, out_cap = 0;
    hipEvent_t done = nullptr;  // completion of this slot's last forward
    std::mutex mu;
};
constexpr int N_HOST_SLOTS = 2;

}  // namespace

struct ebh_model {
    ebh_config cfg{};
    int dtype = EBH_DTYPE_F32;
    int device = -1;
    bool finalized = false;
    std::unordered_map<std::string, HostTensor> host;
    // device weights: one allocation
    void* wbase = nullptr;
    float *word, *pos, *type0, *emb_g, *emb_b;
    std::vector<DevLayer> layers;
    // cross-encoder head (classifier.weight [H], classifier.bias), when loaded
    bool cross_encoder = false;
    float *cls_w = nullptr, *cls_b = nullptr;
    hipStream_t stream = nullptr;
    hipEvent_t done = nullptr;  // completion of the last enqueued forward
    bool has_done = false;
    Workspace ws;
    int last_B = 0;
    // pinned host staging for the blocking API, taken round robin
    HostSlot slots[N_HOST_SLOTS];
    std::atomic<unsigned> slot_rr{0};
    // recorded forwards (GraphEntry), least recently used dropped first
    std::vector<GraphEntry> graphs;
    uint64_t graph_clock = 0;
    bool graph_replay = true;
    // ebh_encode_device_noalloc has run on this model: ebh_synchronize also
    // reads noalloc_err, the id-range flag those forwards raise (a word of
    // the weight block, so each model has its own and the call allocates
    // nothing)
    bool noalloc_used = false;
    int* noalloc_err = nullptr;
    // profiling of one kernel family
    int prof_kind = EBH_PROF_NONE;
    std::vector<ProfPair> prof_events;
    std::vector<hipEvent_t> prof_free;
    std::mutex mu;
};

namespace {

// Expected HF tensor names and shapes (src/lib.rs:161-238).
std::vector<std::pair<std::string, std::vector<int64_t>>> expected_tensors(const ebh_config& c) {
    const int64_t H = c.hidden_size, I = c.intermediate_size;
    std::vector<std::pair<std::string, std::vector<int64_t>>> t = {
        {"embeddings.word_embeddings.weight", {c.vocab_size, H}},
        {"embeddings.position_embeddings.weight", {c.max_position_embeddings, H}},
        {"embeddings.token_type_embeddings.weight", {c.type_vocab_size, H}},
        {"embeddings.LayerNorm.weight", {H}},
        {"embeddings.LayerNorm.bias", {H}},
    };
    for (int i = 0; i < c.num_hidden_layers; ++i) {
        const std::string p = "encoder.layer." + std::to_string(i) + ".";
        for (const char* proj : {"query", "key", "value"}) {
            t.push_back({p + "attention.self." + proj + ".weight", {H, H}});
            t.push_back({p + "attention.self." + proj + ".bias", {H}});
        }
        t.push_back({p + "attention.output.dense.weight", {H, H}});
        t.push_back({p + "attention.output.dense.bias", {H}});
        t.push_back({p + "attention.output.LayerNorm.weight", {H}});
        t.push_back({p + "attention.output.LayerNorm.bias", {H}});
        t.push_back({p + "intermediate.dense.weight", {I, H}});
        t.push_back({p + "intermediate.dense.bias", {I}});
        t.push_back({p + "output.dense.weight", {H, I}});
        t.push_back({p + "output.dense.bias", {H}});
        t.push_back({p + "output.LayerNorm.weight", {H}});
        t.push_back({p + "output.LayerNorm.bias", {H}});
    }
    return t;
}

const std::vector<int64_t>* expected_shape(const ebh_config& c, const std::string& name,
                                           std::vector<int64_t>& storage) {
    for (auto& kv : expected_tensors(c))
        if (kv.first == name) {
            storage = kv.second;
            return &storage;
        }
    return nullptr;
}

std::string shape_str(const int64_t* s, int n) {
    std::string r = "[";
    for (int i = 0; i < n; ++i) r += (i ? ", " : "") + std::to_string(s[i]);
    return r + "]";
}

int check_config(const ebh_config& c) {
    if (c.hidden_size <= 0 || c.num_attention_heads <= 0 || c.num_hidden_layers < 0 ||
        c.intermediate_size <= 0 || c.vocab_size <= 0 || c.max_position_embeddings <= 0 ||
        c.type_vocab_size <= 0 || !(c.layer_norm_eps >= 0.0f))
        return fail(EBH_ERR_INVALID_ARG, "invalid config: sizes must be positive");
    if (c.hidden_size % c.num_attention_heads)
        return fail(EBH_ERR_INVALID_ARG, "hidden_size %d is not a multiple of num_attention_heads %d",
                    c.hidden_size, c.num_attention_heads);
    const int hd = c.hidden_size / c.num_attention_heads;
    if (hd != 32 && hd != 64)
        return fail(EBH_ERR_INVALID_ARG, "head_dim %d unsupported (32 or 64)", hd);
    if (c.hidden_size % 8 || c.intermediate_size % 8)
        return fail(EBH_ERR_INVALID_ARG, "hidden_size and intermediate_size must be multiples of 8");
    if (c.hidden_size > 2048)
        return fail(EBH_ERR_INVALID_ARG, "hidden_size %d above the supported 2048", c.hidden_size);
    return EBH_OK;
}

void prof_begin(ebh_model* m, int active, int kind, hipStream_t s, ProfPair& pp, bool& on) {
    on = (active == kind);
    if (!on) return;
    for (hipEvent_t* e : {&pp.a, &pp.b}) {
        if (!m->prof_free.empty()) {
            *e = m->prof_free.back();
            m->prof_free.pop_back();
        } else {
            (void)hipEventCreate(e);
        }
    }
    (void)hipEventRecord(pp.a, s);
}

void prof_end(ebh_model* m, hipStream_t s, ProfPair& pp, bool on) {
    if (!on) return;
    (void)hipEventRecord(pp.b, s);
    m->prof_events.push_back(pp);
}

void drop_graphs(ebh_model* m) {
    for (auto& g : m->graphs)
        if (g.exec) (void)hipGraphExecDestroy(g.exec);
    m->graphs.clear();
}

// Place a workspace for tcap tokens and bcap sequences at `base` (nullptr:
// only count); returns the bytes it spans.  Few-token fp32 forwards split the
// bias-free projections over K; Y then holds one partial product per split.
size_t layout_workspace(const ebh_model* m, int64_t tcap, int bcap, char* base, Workspace& w) {
    const ebh_config& c = m->cfg;
    const size_t H = c.hidden_size, I = c.intermediate_size;
    const bool b16 = m->dtype == EBH_DTYPE_BF16;
    int yparts = b16 ? 1
                     : std::max(ebh::gemm_f32_splits((int)tcap, (int)H, (int)H),
                                ebh::gemm_f32_splits((int)tcap, (int)H, (int)I));
    // Few-token attention + output projection: one partial per head.
    if (!b16 && ebh::few_attn_fits((int)tcap, (int)H, c.num_attention_heads))
        yparts = std::max(yparts, c.num_attention_heads);
    size_t off = 0;
    auto take = [&](size_t bytes) { size_t o = off; off += align_up(std::max<size_t>(bytes, 1)); return o; };
    const size_t oErr = take(4), oX = take(b16 ? 0 : tcap * H * 4), oX16 = take(b16 ? tcap * H * 2 : 0),
                 oY = take((size_t)yparts * tcap * H * 4), oQKV = take(tcap * 3 * H * 4),
                 oCTX = take(tcap * H * 4), oF = take(tcap * I * 4), oIds = take(tcap * 4),
                 oMask = take(tcap * 4), oCounts = take(bcap * 4), oOrder = take(bcap * 4), oCu = take((bcap + 1) * 4),
                 oNtok = take(4), oTid = take(tcap * 4), oTpos = take(tcap * 4),
                 oOut = take((size_t)bcap * H * 4), oScores = take((size_t)bcap * 4);
    if (!base) return off;
    w.base = base;
    w.tok_cap = tcap;
    w.b_cap = bcap;
    w.y_parts = yparts;
    w.err = (int*)(base + oErr);
    w.X = b16 ? nullptr : (float*)(base + oX);
    w.X16 = b16 ? (uint16_t*)(base + oX16) : nullptr;
    w.Y = (float*)(base + oY);
    w.QKV = (float*)(base + oQKV);
    w.CTX = (float*)(base + oCTX);
    w.F = (float*)(base + oF);
    w.ids = (int*)(base + oIds);
    w.mask = (int*)(base + oMask);
    w.counts = (int*)(base + oCounts);
    w.order = (int*)(base + oOrder);
    w.cu = (int*)(base + oCu);
    w.ntok = (int*)(base + oNtok);
    w.tok_id = (int*)(base + oTid);
    w.tok_pos = (int*)(base + oTpos);
    w.out = (float*)(base + oOut);
    w.scores = (float*)(base + oScores);
    return off;
}

int ensure_workspace(ebh_model* m, int B, int S) {
    const int64_t T = (int64_t)B * S;
    Workspace& w = m->ws;
    if (w.base && T <= w.tok_cap && B <= w.b_cap) return EBH_OK;
    const int64_t tcap = std::max<int64_t>(T, w.tok_cap);
    const int bcap = std::max(B, w.b_cap);
    Workspace nw;
    const size_t bytes = layout_workspace(m, tcap, bcap, nullptr, nw);
    // Work from the previous call may still use the old block, and recorded
    // forwards hold its addresses.  A raised id-range flag is carried over to
    // the new block (it stays raised until ebh_synchronize reads it).
    if (m->has_done) HIP_TRY(hipEventSynchronize(m->done));
    drop_graphs(m);
    int old_err = 0;
    if (w.base) HIP_TRY(hipMemcpy(&old_err, w.err, 4, hipMemcpyDeviceToHost));
    if (w.base) HIP_TRY(hipFree(w.base));
    w = Workspace{};
    void* base = nullptr;
    HIP_TRY(hipMalloc(&base, bytes));
    layout_workspace(m, tcap, bcap, static_cast<char*>(base), w);
    HIP_TRY(hipMemcpy(w.err, &old_err, 4, hipMemcpyHostToDevice));
    // The model's stream does not wait for the null stream: the flag must be
    // written before the first forward on this workspace can set it.
    HIP_TRY(hipStreamSynchronize(nullptr));
    return EBH_OK;
}

// Called with the model's lock and the slot's lock held (so the slot's last
// forward has completed).
int ensure_host_staging(ebh_model* m, HostSlot& hs, int64_t T, int64_t outn) {
    if (T > hs.cap || outn > hs.out_cap) {
        // Recorded host-path forwards copy from / to these buffers.
        if (m->has_done) HIP_TRY(hipEventSynchronize(m->done));
        drop_graphs(m);
    }
    if (T > hs.cap) {
        if (hs.ids) (void)hipHostFree(hs.ids);
        if (hs.mask) (void)hipHostFree(hs.mask);
        hs.ids = hs.mask = nullptr;
        hs.cap = 0;
        HIP_TRY(hipHostMalloc((void**)&hs.ids, std::max<int64_t>(T, 1) * 4, hipHostMallocDefault));
        HIP_TRY(hipHostMalloc((void**)&hs.mask, std::max<int64_t>(T, 1) * 4, hipHostMallocDefault));
        hs.cap = T;
    }
    if (outn > hs.out_cap) {
        if (hs.out) (void)hipHostFree(hs.out);
        hs.out = nullptr;
        hs.out_cap = 0;
        HIP_TRY(hipHostMalloc((void**)&hs.out, std::max<int64_t>(outn, 1) * 4, hipHostMallocDefault));
        hs.out_cap = outn;
    }
    if (!hs.done) HIP_TRY(hipEventCreateWithFlags(&hs.done, hipEventDisableTiming));
    return EBH_OK;
}

// The kernels of one forward on stream s (ids/mask already in device memory).
// d_scores (optional, cross-encoders): score[b] = pooled[b] . w + bias, from
// the un-normalised pooled rows left in d_out.
// tokens: the number of mask == 1 tokens when the host knows it (the
// blocking entry points), else -1.
// w: the workspace to run in (the model's own, or the no-allocation entry
// point's static one); prof: time the profiled kernel family (creates events).
int enqueue_kernels(ebh_model* m, Workspace& w, const int* d_ids, const int* d_mask, int B, int S,
                    int normalize, float* d_out, hipStream_t s, float* d_scores, int64_t tokens,
                    bool prof = true) {
    const ebh_config& c = m->cfg;
    const int H = c.hidden_size, I = c.intermediate_size, nh = c.num_attention_heads;
    const int hd = H / nh;
    const float eps = c.layer_norm_eps;
    const float scale = 1.0f / sqrtf((float)hd);  // src/lib.rs:196-197
    const int prof_kind = prof ? m->prof_kind : EBH_PROF_NONE;
    const int T = B * S;  // rows every kernel is sized for; they read the packed count on the device

    ProfPair pp{};
    bool on = false;
    const bool bf16 = m->dtype == EBH_DTYPE_BF16;
    const bool few_pack = ebh::pack_embed_few_fits(B, S, H);
    const int* seq_order = few_pack ? nullptr : w.order;   // written by launch_pack only
    if (few_pack) {   // a few short sentences: one launch
        prof_begin(m, prof_kind, EBH_PROF_EMBED, s, pp, on);
        HIP_TRY(ebh::launch_pack_embed_few(d_ids, d_mask, B, S, w.cu, w.ntok, w.tok_id, w.tok_pos, w.err,
                                           m->word, m->pos, m->type0, m->emb_g, m->emb_b, c.vocab_size, H,
                                           eps, bf16 ? nullptr : w.X, w.X16, s));
        prof_end(m, s, pp, on);
    } else {
        HIP_TRY(ebh::launch_pack(d_ids, d_mask, B, S, w.counts, w.cu, w.ntok, w.tok_id, w.tok_pos, s, w.order));
        prof_begin(m, prof_kind, EBH_PROF_EMBED, s, pp, on);
        HIP_TRY(ebh::launch_embed_ln(w.tok_id, w.tok_pos, w.ntok, T, m->word, m->pos, m->type0,
                                     m->emb_g, m->emb_b, c.vocab_size, H, eps, bf16 ? nullptr : w.X, w.err,
                                     w.X16, s));
        prof_end(m, s, pp, on);
    }

    // bf16 models keep the residual stream in bf16 (X16, written by each
    // LayerNorm; every sum and statistic stays fp32) and hand the GEMMs bf16
    // operands: X16, q / k / v, the attention context and the GELU output,
    // each of the last three stored as bf16 in the first half of its fp32
    // buffer.
    uint16_t* qkv16 = reinterpret_cast<uint16_t*>(w.QKV);
    uint16_t* ctx16 = reinterpret_cast<uint16_t*>(w.CTX);
    uint16_t* f16 = reinterpret_cast<uint16_t*>(w.F);
    auto gemm = [&](int kind, const void* A, int64_t lda, const float* W32, const uint16_t* W16,
                    const float* bias, void* C, int N, int K, int epi, bool c16, int splits = 1,
                    int rows = -1) -> int {
        if (rows < 0) rows = T;
        ebh::GemmArgs a{};
        a.splits = splits;
        a.split_stride = (int64_t)rows * N;
        a.A = A;
        a.W = bf16 ? (const void*)W16 : (const void*)W32;
        a.bias = bias;
        a.R = nullptr;
        a.C = static_cast<float*>(C);
        a.lda = lda;
        a.ldw = K;
        a.ldr = 0;
        a.ldc = N;
        a.M_max = rows;
        a.M_dev = w.ntok;
        a.N = N;
        a.K = K;
        a.split6 = m->dtype == EBH_DTYPE_F32_BF16X6;
        ProfPair p2{};
        bool on2 = false;
        prof_begin(m, prof_kind, kind, s, p2, on2);
        hipError_t e = bf16 ? ebh::launch_gemm_bf16_act(a, epi, c16, s) : ebh::launch_gemm_f32(a, epi, s);
        prof_end(m, s, p2, on2);
        if (e != hipSuccess) return fail(EBH_ERR_HIP, "gemm launch failed: %s", hipGetErrorString(e));
        return EBH_OK;
    };

    // Per layer (BertLayer::forward, src/lib.rs:669-683): the attention-output and
    // FFN-down projections are written without bias (as bf16 in bf16 models);
    // their bias and the block's residual are added in fp32, in the reference's
    // order, by the LayerNorm that follows.
    // With few tokens (fp32) these two products are split over K into partial
    // outputs that the LayerNorm sums in a fixed order, so the result does not
    // depend on timing.
    // fp32 with at least a 128-row block per CU: the attention-output and
    // FFN-down products end in their bias + residual + LayerNorm inside the
    // GEMM (each workgroup holds whole rows), in place on X.  That form runs
    // one 128-row block per workgroup, so a ragged batch whose packed rows
    // (known here when the host counted them) fill too few blocks takes the
    // split path instead, with these two products and their LayerNorms sized
    // for the packed rows; everything else stays sized for B*S.
    const int T_real = tokens >= 0 && tokens < T ? (int)tokens : T;
    const bool flip = !bf16 && ebh::gemm_f32_add_ln_fits(T, H, H) && !ebh::gemm_f32_add_ln_fits(T_real, H, H);
    const int T_od = flip ? T_real : T;
    const bool fuse_out = !bf16 && ebh::gemm_f32_add_ln_fits(T_od, H, H);
    const bool fuse_down = !bf16 && ebh::gemm_f32_add_ln_fits(T_od, H, I);
    auto add_ln = [&](const float* bias, const float* g, const float* b, int parts) -> hipError_t {
        return bf16 ? ebh::launch_add_layernorm_y16(reinterpret_cast<const uint16_t*>(w.Y), bias, nullptr, g, b, T_od,
                                                    w.ntok, H, eps, w.X16, s)
                    : ebh::launch_add_layernorm(w.Y, bias, w.X, g, b, T_od, w.ntok, H, eps, w.X16, s, parts,
                                                (int64_t)T_od * H);
    };
    const int64_t part_cap = (int64_t)w.y_parts * w.tok_cap / std::max<int64_t>(T_od, 1);
    auto splits_for = [&](int K) {
        if (bf16) return 1;
        int sp = ebh::gemm_f32_splits(T_od, H, K);
        while (sp > 1 && sp > part_cap) sp /= 2;
        return sp;
    };
    const int sp_out = splits_for(H), sp_down = splits_for(I);
    // At most FEW_ATTN_MAX_TOKENS rows (fp32, heads of 32): attention and the
    // output projection run as one launch writing a partial per head.
    const bool few_attn = !bf16 && ebh::few_attn_fits(T, H, nh) && T_od == T && part_cap >= nh;
    auto gemm_ln = [&](int kind, const float* A, const float* W, const float* bias, const float* g,
                       const float* b, int K) -> int {
        ebh::GemmArgs a{};
        a.A = A;
        a.W = W;
        a.bias = bias;
        a.R = w.X;
        a.C = w.X;
        a.lda = K;
        a.ldw = K;
        a.ldr = H;
        a.ldc = H;
        a.M_max = T;
        a.M_dev = w.ntok;
        a.N = H;
        a.K = K;
        a.ln_g = g;
        a.ln_b = b;
        a.ln_eps = eps;
        a.split6 = m->dtype == EBH_DTYPE_F32_BF16X6;
        ProfPair p2{};
        bool on2 = false;
        prof_begin(m, prof_kind, kind, s, p2, on2);
        hipError_t e = ebh::launch_gemm_f32_add_ln(a, s);
        prof_end(m, s, p2, on2);
        if (e != hipSuccess) return fail(EBH_ERR_HIP, "gemm launch failed: %s", hipGetErrorString(e));
        return EBH_OK;
    };
    for (const DevLayer& L : m->layers) {
        int rc;
        if ((rc = gemm(EBH_PROF_GEMM_QKV, bf16 ? (const void*)w.X16 : w.X, H, L.wqkv, L.wqkv16, L.bqkv,
                       bf16 ? (void*)qkv16 : (void*)w.QKV, 3 * H, H, ebh::EPI_BIAS, bf16)))
            return rc;
        prof_begin(m, prof_kind, EBH_PROF_ATTENTION, s, pp, on);
        if (few_attn)
            HIP_TRY(ebh::launch_attn_out_few(w.QKV, L.wo, w.cu, w.ntok, B, T, H, nh, scale, w.Y, (int64_t)T * H,
                                             s));
        else if (bf16)
            HIP_TRY(ebh::launch_attention_bf16(qkv16, w.cu, B, S, H, nh, hd, scale, ctx16, s, seq_order));
        else
            HIP_TRY(ebh::launch_attention(w.QKV, w.cu, B, S, H, nh, hd, scale, w.CTX, s, seq_order));
        prof_end(m, s, pp, on);
        if (few_attn) {
            prof_begin(m, prof_kind, EBH_PROF_LAYERNORM, s, pp, on);
            HIP_TRY(add_ln(L.bo, L.ln1_g, L.ln1_b, nh));
            prof_end(m, s, pp, on);
        } else if (fuse_out) {
            if ((rc = gemm_ln(EBH_PROF_GEMM_OUT, w.CTX, L.wo, L.bo, L.ln1_g, L.ln1_b, H))) return rc;
        } else {
            if ((rc = gemm(EBH_PROF_GEMM_OUT, bf16 ? (const void*)ctx16 : w.CTX, H, L.wo, L.wo16, nullptr,
                           w.Y, H, H, ebh::EPI_NONE, bf16, sp_out, T_od)))
                return rc;
            prof_begin(m, prof_kind, EBH_PROF_LAYERNORM, s, pp, on);
            HIP_TRY(add_ln(L.bo, L.ln1_g, L.ln1_b, sp_out));
            prof_end(m, s, pp, on);
        }
        if ((rc = gemm(EBH_PROF_GEMM_FFN_UP, bf16 ? (const void*)w.X16 : w.X, H, L.w1, L.w116, L.b1,
                       bf16 ? (void*)f16 : (void*)w.F, I, H, ebh::EPI_BIAS_GELU, bf16)))
            return rc;
        if (fuse_down) {
            if ((rc = gemm_ln(EBH_PROF_GEMM_FFN_DOWN, w.F, L.w2, L.b2, L.ln2_g, L.ln2_b, I))) return rc;
        } else {
            if ((rc = gemm(EBH_PROF_GEMM_FFN_DOWN, bf16 ? (const void*)f16 : w.F, I, L.w2, L.w216, nullptr,
                           w.Y, H, I, ebh::EPI_NONE, bf16, sp_down, T_od)))
                return rc;
            prof_begin(m, prof_kind, EBH_PROF_LAYERNORM, s, pp, on);
            HIP_TRY(add_ln(L.b2, L.ln2_g, L.ln2_b, sp_down));
            prof_end(m, s, pp, on);
        }
    }
    prof_begin(m, prof_kind, EBH_PROF_POOL, s, pp, on);
    HIP_TRY(bf16 ? ebh::launch_pool_b16(w.X16, w.cu, B, H, S, normalize, d_out, s)
                 : ebh::launch_pool(w.X, w.cu, B, H, S, normalize, w.Y, d_out, s));
    prof_end(m, s, pp, on);
    if (d_scores) HIP_TRY(ebh::launch_cls_head(d_out, m->cls_w, m->cls_b, B, H, d_scores, s));
    return EBH_OK;
}

// The recorded forward for this call, recording it at the key's second call;
// nullptr: run the launches directly (replay off, profiling on, the caller's
// stream being captured into a graph of its own, or recording failed).
template <class Body>
hipGraphExec_t graph_for(ebh_model* m, const GraphEntry& key, hipStream_t s, Body&& body) {
    if (!m->graph_replay || m->prof_kind != EBH_PROF_NONE) return nullptr;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return nullptr;
    GraphEntry* e = nullptr;
    for (auto& g : m->graphs)
        if (g.B == key.B && g.S == key.S && g.normalize == key.normalize && g.host == key.host &&
            g.tokens == key.tokens &&
            g.ids == key.ids && g.mask == key.mask && g.out == key.out && g.scores == key.scores) {
            e = &g;
            break;
        }
    if (!e) {
        if (m->graphs.size() >= MAX_GRAPHS) {
            auto lru = std::min_element(m->graphs.begin(), m->graphs.end(),
                                        [](const GraphEntry& a, const GraphEntry& b) { return a.used < b.used; });
            // Device-path launches of that recording may still be queued.
            if (lru->exec && m->has_done && hipEventSynchronize(m->done) != hipSuccess) return nullptr;
            if (lru->exec) (void)hipGraphExecDestroy(lru->exec);
            m->graphs.erase(lru);
        }
        m->graphs.push_back(key);
        m->graphs.back().seen = 1;
        m->graphs.back().exec = nullptr;
        m->graphs.back().used = ++m->graph_clock;
        return nullptr;
    }
    e->used = ++m->graph_clock;
    if (e->exec || e->seen < 0) return e->exec;
    // Record on the model's own stream (never the legacy default stream);
    // the graph is then launched on s.
    hipGraph_t g = nullptr;
    bool ok = hipStreamBeginCapture(m->stream, hipStreamCaptureModeThreadLocal) == hipSuccess;
    if (ok) {
        const int rc = body(m->stream);
        ok = hipStreamEndCapture(m->stream, &g) == hipSuccess && rc == EBH_OK && g &&
             hipGraphInstantiate(&e->exec, g, nullptr, nullptr, 0) == hipSuccess;
    }
    if (g) (void)hipGraphDestroy(g);
    if (!ok) {
        e->exec = nullptr;
        e->seen = -1;
        (void)hipGetLastError();
    }
    return e->exec;
}

// One forward on stream s, ordered after the model's previous work.  hs (the
// blocking entry points): ids / mask come from that slot's pinned staging
// buffers, and the result (d_scores if given, else d_out) goes back to it.
// The blocking entry points check every id on the host, so their forwards
// never raise the device's id-range flag; that flag is sticky (kernels only
// set it) and is read and cleared by ebh_synchronize alone.
int run_forward(ebh_model* m, const int* d_ids, const int* d_mask, int B, int S, int normalize,
                float* d_out, hipStream_t s, float* d_scores, HostSlot* hs, int64_t tokens = -1) {
    const bool host = hs != nullptr;
    Workspace& w = m->ws;
    const int64_t T = (int64_t)B * S;
    const size_t n_out = d_scores ? (size_t)B : (size_t)B * m->cfg.hidden_size;
    if (m->has_done) HIP_TRY(hipStreamWaitEvent(s, m->done, 0));
    auto body = [&](hipStream_t st) -> int {
        if (host) {
            HIP_TRY(hipMemcpyAsync(w.ids, hs->ids, T * 4, hipMemcpyHostToDevice, st));
            HIP_TRY(hipMemcpyAsync(w.mask, hs->mask, T * 4, hipMemcpyHostToDevice, st));
        }
        int rc = enqueue_kernels(m, w, d_ids, d_mask, B, S, normalize, d_out, st, d_scores, tokens);
        if (rc) return rc;
        if (host) {
            HIP_TRY(hipMemcpyAsync(hs->out, d_scores ? d_scores : d_out, n_out * 4, hipMemcpyDeviceToHost, st));
        }
        return EBH_OK;
    };
    // Host-path recordings bake in the slot's staging buffers, so each slot
    // has its own.
    const GraphEntry key{B, S, normalize, host ? 1 : 0, host ? (const void*)hs->ids : d_ids,
                         host ? (const void*)hs->mask : d_mask, host ? (void*)hs->out : d_out, d_scores,
                         tokens, 0, nullptr, 0};
    if (hipGraphExec_t exec = graph_for(m, key, s, body)) {
        HIP_TRY(hipGraphLaunch(exec, s));
    } else {
        const int rc = body(s);
        if (rc) return rc;
    }
    HIP_TRY(hipEventRecord(m->done, s));
    if (hs) HIP_TRY(hipEventRecord(hs->done, s));
    m->has_done = true;
    m->last_B = B;
    return EBH_OK;
}

// Blocking forward from host buffers.  `stage(ids, mask)` writes (and
// validates) the caller's ids / mask into a slot's pinned buffers; the forward
// is enqueued under the model's lock, which is released before the wait, so
// the next caller's forward can be queued behind this one while it runs.
// The result ([B, H] vectors, or [B] scores) is copied to out.
template <class Stage>
int host_forward(ebh_model* m, int B, int S, int normalize, float* out, bool score, Stage&& stage) {
    const int H = m->cfg.hidden_size;
    const int64_t T = (int64_t)B * S;
    const size_t n_out = score ? (size_t)B : (size_t)B * H;
    HostSlot& hs = m->slots[m->slot_rr.fetch_add(1) % N_HOST_SLOTS];
    std::lock_guard<std::mutex> slot_lock(hs.mu);
    {
        std::lock_guard<std::mutex> lk(m->mu);
        HIP_TRY(hipSetDevice(m->device));
        int rc = ensure_host_staging(m, hs, T, (int64_t)B * H);
        if (rc) return rc;
        if ((rc = stage(hs.ids, hs.mask))) return rc;
        int64_t tokens = 0;
        for (int64_t i = 0; i < T; ++i) tokens += hs.mask[i] != 0;
        if ((rc = ensure_workspace(m, B, S))) return rc;
        if ((rc = run_forward(m, m->ws.ids, m->ws.mask, B, S, normalize, m->ws.out, m->stream,
                              score ? m->ws.scores : nullptr, &hs, tokens)))
            return rc;
    }
    HIP_TRY(hipEventSynchronize(hs.done));
    memcpy(out, hs.out, n_out * 4);
    return EBH_OK;
}

int check_model_ready(const ebh_model* m) {
    if (!m) return fail(EBH_ERR_INVALID_ARG, "null model");
    if (!m->finalized) return fail(EBH_ERR_STATE, "model is not finalized (call ebh_finalize)");
    return EBH_OK;
}

int check_dims(const ebh_model* m, int B, int S) {
    if (B < 0 || S < 0) return fail(EBH_ERR_INVALID_ARG, "negative batch or sequence length");
    if (S > m->cfg.max_position_embeddings)
        return fail(EBH_ERR_RANGE, "sequence length %d exceeds max_position_embeddings %d", S,
                    m->cfg.max_position_embeddings);
    if ((int64_t)B * S > (int64_t)1 << 30)
        return fail(EBH_ERR_INVALID_ARG, "batch*seq %lld too large", (long long)B * S);
    return EBH_OK;
}

}  // namespace

// ---------------------------------------------------------------------------
// Static scratch workspace of ebh_encode_device_noalloc: the activations of
// one forward (laid out by layout_workspace; the id-range flag is the
// model's own, in its weight block), held by
// every device the library runs on until the process ends.  Host code never
// uses the array's name as an address (on the host it is only a stand-in):
// ebh_finalize looks its device address up once per device with
// hipGetSymbolAddress, and every kernel argument, fill and copy uses that.
// ---------------------------------------------------------------------------
static __device__ __align__(256) unsigned char scratch[EBH_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
char* g_scratch_ptr[MAX_DEVICES] = {};   // device address of `scratch` per device

// Called by ebh_finalize with the model's device current: look the array up
// on this device once.  (Its first word, the id-range flag slot of the
// workspace layout, is unused: each model's no-allocation forwards raise
// that model's own flag.)
int setup_scratch(int dev) {
    if (dev < 0 || dev >= MAX_DEVICES) return fail(EBH_ERR_STATE, "device %d beyond %d devices", dev, MAX_DEVICES);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch_ptr[dev]) return EBH_OK;
    void* p = nullptr;
    HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) return fail(EBH_ERR_HIP, "hipGetSymbolAddress returned no address for the scratch workspace");
    g_scratch_ptr[dev] = static_cast<char*>(p);
    return EBH_OK;
}

char* scratch_ptr(int dev) {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    return dev >= 0 && dev < MAX_DEVICES ? g_scratch_ptr[dev] : nullptr;
}
}  // namespace

namespace ebh {
// Validate one tensor against the a15 layout (name, rank, shape) and keep it
// until ebh_finalize: f32 data is copied; with `keep` (a mapped file), data
// is referenced in place in any encoding.
int put_tensor(ebh_model* m, const char* name, const void* data, int kind, const int64_t* shape, int32_t ndim,
               std::shared_ptr<const void> keep) {
    if (!m || !name || !shape || (!data && ndim > 0) || ndim < 0) return fail(EBH_ERR_INVALID_ARG, "null argument");
    if (m->finalized) return fail(EBH_ERR_STATE, "model already finalized");
    if (kind != TENSOR_F32 && kind != TENSOR_F16 && kind != TENSOR_BF16)
        return fail(EBH_ERR_INVALID_ARG, "unknown tensor encoding %d", kind);
    if (kind != TENSOR_F32 && !keep) return fail(EBH_ERR_INVALID_ARG, "16-bit tensors are taken from files only");
    for (int i = 0; i < ndim; ++i)
        if (shape[i] < 0) return fail(EBH_ERR_SHAPE, "negative dimension for %s", name);
    const std::string nm(name);
    if (nm == "classifier.weight" || nm == "classifier.bias") {
        // Cross-encoder head (from_cross_encoder_weights, src/lib.rs:385-399).
        // The weight is taken as [H] (get_array1, src/weights.rs:47-58) or as
        // the [1, H] a sequence-classification checkpoint stores; the bias must
        // hold exactly one value (get_scalar, src/weights.rs:99-111).
        int64_t n = 1;
        for (int i = 0; i < ndim; ++i) n *= shape[i];
        if (nm == "classifier.weight") {
            const int64_t H = m->cfg.hidden_size;
            const bool ok = (ndim == 1 && shape[0] == H) || (ndim == 2 && shape[0] == 1 && shape[1] == H);
            if (!ok)
                return fail(EBH_ERR_SHAPE, "Expected 1D tensor, got shape %s for %s (hidden size %lld)",
                            shape_str(shape, ndim).c_str(), name, (long long)H);
        } else if (n != 1) {
            return fail(EBH_ERR_SHAPE, "Expected scalar, got %lld elements", (long long)n);
        }
    } else {
        std::vector<int64_t> storage;
        const std::vector<int64_t>* exp = expected_shape(m->cfg, name, storage);
        if (!exp) return fail(EBH_ERR_NOT_FOUND, "unknown tensor %s", name);
        if (exp->size() == 1 && ndim != 1)
            return fail(EBH_ERR_SHAPE, "Expected 1D tensor, got shape %s for %s",
                        shape_str(shape, ndim).c_str(), name);
        if ((int)exp->size() != ndim || !std::equal(exp->begin(), exp->end(), shape))
            return fail(EBH_ERR_SHAPE, "Shape error: %s has shape %s, expected %s", name,
                        shape_str(shape, ndim).c_str(), shape_str(exp->data(), (int)exp->size()).c_str());
    }
    HostTensor t;
    t.shape.assign(shape, shape + ndim);
    t.kind = kind;
    if (keep) {
        t.src = data;
        t.keep = std::move(keep);
    } else {
        const float* f = static_cast<const float*>(data);
        t.own.assign(f, f + t.count());
        t.src = t.own.data();
    }
    m->host[nm] = std::move(t);
    return EBH_OK;
}
}  // namespace ebh

// ===========================================================================
// C ABI
// ===========================================================================
extern "C" {

const char* ebh_last_error(void) { return g_err.c_str(); }

int ebh_create(const ebh_config* cfg, ebh_model** out) {
    if (!cfg || !out) return fail(EBH_ERR_INVALID_ARG, "null argument");
    *out = nullptr;
    int rc = check_config(*cfg);
    if (rc) return rc;
    ebh_model* m = new ebh_model();
    m->cfg = *cfg;
    *out = m;
    return EBH_OK;
}

int ebh_set_tensor(ebh_model* m, const char* name, const float* data, const int64_t* shape,
                   int32_t ndim) {
    return ebh::put_tensor(m, name, data, ebh::TENSOR_F32, shape, ndim, nullptr);
}

// Device resources a failed ebh_finalize had already made (stream, event,
// weight block) are released and the model goes back to its state before the
// call (host tensors kept), so the call can be repeated without leaking them.
static void release_partial_finalize(ebh_model* m) {
    if (m->device < 0) return;
    (void)hipSetDevice(m->device);
    if (m->stream) (void)hipStreamSynchronize(m->stream);
    if (m->wbase) (void)hipFree(m->wbase);
    if (m->done) (void)hipEventDestroy(m->done);
    if (m->stream) (void)hipStreamDestroy(m->stream);
    m->wbase = nullptr;
    m->noalloc_err = nullptr;
    m->done = nullptr;
    m->stream = nullptr;
    m->device = -1;
}

static int finalize_locked(ebh_model* m, int32_t dtype);

int ebh_finalize(ebh_model* m, int32_t dtype) {
    if (!m) return fail(EBH_ERR_INVALID_ARG, "null model");
    std::lock_guard<std::mutex> lk(m->mu);
    const int rc = finalize_locked(m, dtype);
    if (rc != EBH_OK && !m->finalized) release_partial_finalize(m);
    return rc;
}

static int finalize_locked(ebh_model* m, int32_t dtype) {
    if (m->finalized) return fail(EBH_ERR_STATE, "model already finalized");
    if (dtype != EBH_DTYPE_F32 && dtype != EBH_DTYPE_BF16 && dtype != EBH_DTYPE_F32_BF16X6)
        return fail(EBH_ERR_INVALID_ARG, "unknown dtype %d", dtype);
    if (dtype == EBH_DTYPE_BF16 && (m->cfg.hidden_size % 64 || m->cfg.intermediate_size % 64 ||
                                    !ebh::row4_shape_ok(m->cfg.hidden_size)))
        return fail(EBH_ERR_INVALID_ARG,
                    "bf16 models need hidden_size and intermediate_size multiples of 64, and hidden_size "
                    "= 4 * L * n with L in {64, 32, 16} and n in {1, 2, 3, 4, 6, 8}");
    const auto names = expected_tensors(m->cfg);
    for (auto& kv : names)
        if (!m->host.count(kv.first)) return fail(EBH_ERR_NOT_FOUND, "Tensor %s not found", kv.first.c_str());
    const bool has_cw = m->host.count("classifier.weight") > 0, has_cb = m->host.count("classifier.bias") > 0;
    if (has_cw != has_cb)
        return fail(EBH_ERR_NOT_FOUND, "Tensor %s not found", has_cw ? "classifier.bias" : "classifier.weight");

    const ebh_config& c = m->cfg;
    const size_t H = c.hidden_size, I = c.intermediate_size, L = c.num_hidden_layers;
    const bool b16 = dtype == EBH_DTYPE_BF16;
    int rc0;
    // Layout of the single device weight block.  The four GEMM weights of a
    // layer are held once, in the form the forward reads: fp32 for fp32
    // models, bf16 for bf16 models; everything else is fp32.
    size_t off = 0;
    auto take = [&](size_t bytes) { size_t o = off; off += align_up(bytes); return o; };
    const size_t wes = b16 ? 2 : 4;               // bytes per GEMM weight element
    struct Off { size_t wqkv, bqkv, wo, bo, ln1_g, ln1_b, w1, b1, w2, b2, ln2_g, ln2_b; };
    const size_t oWord = take((size_t)c.vocab_size * H * 4), oPos = take((size_t)c.max_position_embeddings * H * 4),
                 oType = take(H * 4), oEg = take(H * 4), oEb = take(H * 4);
    std::vector<Off> lo(L);
    for (size_t l = 0; l < L; ++l) {
        Off& o = lo[l];
        o.wqkv = take(3 * H * H * wes); o.bqkv = take(3 * H * 4);
        o.wo = take(H * H * wes); o.bo = take(H * 4);
        o.ln1_g = take(H * 4); o.ln1_b = take(H * 4);
        o.w1 = take(I * H * wes); o.b1 = take(I * 4);
        o.w2 = take(H * I * wes); o.b2 = take(H * 4);
        o.ln2_g = take(H * 4); o.ln2_b = take(H * 4);
    }
    const size_t oClsW = has_cw ? take(H * 4) : 0, oClsB = has_cw ? take(4) : 0;
    const size_t oNoallocErr = take(4);            // id-range flag of ebh_encode_device_noalloc

    HIP_TRY(hipGetDevice(&m->device));
    HIP_TRY(hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking));
    HIP_TRY(hipEventCreateWithFlags(&m->done, hipEventDisableTiming));
    if ((rc0 = setup_scratch(m->device))) return rc0;
    HIP_TRY(hipMalloc(&m->wbase, off));
    char* b = static_cast<char*>(m->wbase);

    // Upload.  Every tensor goes from its host memory (the caller's copy, or
    // the mapped checkpoint file) straight to its place in the block when the
    // encodings agree (F32 -> fp32, BF16 -> bf16 GEMM weights); otherwise its
    // bytes land in a device scratch buffer and a conversion kernel writes
    // the destination (F16 / BF16 -> fp32 exactly; F16 / F32 -> bf16 with
    // round to nearest even).  All copies and kernels run in order on the
    // model's stream, so the scratch buffer is reused safely.
    size_t scratch_bytes = 0;
    for (auto& kv : m->host) scratch_bytes = std::max(scratch_bytes, (size_t)kv.second.count() * 4);
    void* scratch = nullptr;
    HIP_TRY(hipMalloc(&scratch, std::max<size_t>(scratch_bytes, 4)));
    std::unique_ptr<void, hipError_t (*)(void*)> scratch_guard(scratch, hipFree);
    hipStream_t st = m->stream;
    // Elements [first, first + n) of tensor `name` (n < 0: all of it) to the
    // block at byte offset o, as fp32 or (to16) bf16.
    auto upload = [&](size_t o, const std::string& name, bool to16, int64_t first = 0, int64_t n = -1) -> int {
        const HostTensor& t = m->host.at(name);
        if (n < 0) n = t.count() - first;
        const size_t esz = t.kind == ebh::TENSOR_F32 ? 4 : 2;
        const char* src = static_cast<const char*>(t.src) + (size_t)first * esz;
        void* dst = b + o;
        const bool direct = (t.kind == ebh::TENSOR_F32 && !to16) || (t.kind == ebh::TENSOR_BF16 && to16);
        if (direct) {
            HIP_TRY(hipMemcpyAsync(dst, src, (size_t)n * esz, hipMemcpyHostToDevice, st));
            return EBH_OK;
        }
        HIP_TRY(hipMemcpyAsync(scratch, src, (size_t)n * esz, hipMemcpyHostToDevice, st));
        if (t.kind == ebh::TENSOR_F32)
            HIP_TRY(ebh::launch_f32_to_bf16(static_cast<const float*>(scratch), static_cast<uint16_t*>(dst), n, st));
        else
            HIP_TRY(ebh::launch_widen16(static_cast<const uint16_t*>(scratch), dst, n,
                                        t.kind == ebh::TENSOR_BF16 ? ebh::WIDEN_BF16_F32
                                                                   : (to16 ? ebh::WIDEN_F16_BF16 : ebh::WIDEN_F16_F32),
                                        st));
        return EBH_OK;
    };
    int rc;
#define EBH_UP(...) \
    if ((rc = upload(__VA_ARGS__))) return rc
    EBH_UP(oWord, "embeddings.word_embeddings.weight", false);
    EBH_UP(oPos, "embeddings.position_embeddings.weight", false);
    EBH_UP(oType, "embeddings.token_type_embeddings.weight", false, 0, (int64_t)H);  // row 0 only (src/lib.rs:658)
    EBH_UP(oEg, "embeddings.LayerNorm.weight", false);
    EBH_UP(oEb, "embeddings.LayerNorm.bias", false);
    for (size_t l = 0; l < L; ++l) {
        const std::string p = "encoder.layer." + std::to_string(l) + ".";
        const Off& o = lo[l];
        EBH_UP(o.wqkv, p + "attention.self.query.weight", b16);
        EBH_UP(o.wqkv + H * H * wes, p + "attention.self.key.weight", b16);
        EBH_UP(o.wqkv + 2 * H * H * wes, p + "attention.self.value.weight", b16);
        EBH_UP(o.bqkv, p + "attention.self.query.bias", false);
        EBH_UP(o.bqkv + H * 4, p + "attention.self.key.bias", false);
        EBH_UP(o.bqkv + 2 * H * 4, p + "attention.self.value.bias", false);
        EBH_UP(o.wo, p + "attention.output.dense.weight", b16);
        EBH_UP(o.bo, p + "attention.output.dense.bias", false);
        EBH_UP(o.ln1_g, p + "attention.output.LayerNorm.weight", false);
        EBH_UP(o.ln1_b, p + "attention.output.LayerNorm.bias", false);
        EBH_UP(o.w1, p + "intermediate.dense.weight", b16);
        EBH_UP(o.b1, p + "intermediate.dense.bias", false);
        EBH_UP(o.w2, p + "output.dense.weight", b16);
        EBH_UP(o.b2, p + "output.dense.bias", false);
        EBH_UP(o.ln2_g, p + "output.LayerNorm.weight", false);
        EBH_UP(o.ln2_b, p + "output.LayerNorm.bias", false);
    }
    if (has_cw) {
        EBH_UP(oClsW, "classifier.weight", false);
        EBH_UP(oClsB, "classifier.bias", false);
    }
#undef EBH_UP
    HIP_TRY(ebh::launch_zero_words(b + oNoallocErr, 1, st));
    HIP_TRY(hipStreamSynchronize(st));

    m->word = (float*)(b + oWord);
    m->pos = (float*)(b + oPos);
    m->type0 = (float*)(b + oType);
    m->emb_g = (float*)(b + oEg);
    m->emb_b = (float*)(b + oEb);
    m->cross_encoder = has_cw;
    m->cls_w = has_cw ? (float*)(b + oClsW) : nullptr;
    m->cls_b = has_cw ? (float*)(b + oClsB) : nullptr;
    m->noalloc_err = (int*)(b + oNoallocErr);
    m->layers.resize(L);
    for (size_t l = 0; l < L; ++l) {
        const Off& o = lo[l];
        DevLayer& d = m->layers[l];
        d.bqkv = (float*)(b + o.bqkv); d.bo = (float*)(b + o.bo);
        d.ln1_g = (float*)(b + o.ln1_g); d.ln1_b = (float*)(b + o.ln1_b);
        d.b1 = (float*)(b + o.b1); d.b2 = (float*)(b + o.b2);
        d.ln2_g = (float*)(b + o.ln2_g); d.ln2_b = (float*)(b + o.ln2_b);
        d.wqkv = d.wo = d.w1 = d.w2 = nullptr;
        d.wqkv16 = d.wo16 = d.w116 = d.w216 = nullptr;
        if (b16) {
            d.wqkv16 = (uint16_t*)(b + o.wqkv); d.wo16 = (uint16_t*)(b + o.wo);
            d.w116 = (uint16_t*)(b + o.w1); d.w216 = (uint16_t*)(b + o.w2);
        } else {
            d.wqkv = (float*)(b + o.wqkv); d.wo = (float*)(b + o.wo);
            d.w1 = (float*)(b + o.w1); d.w2 = (float*)(b + o.w2);
        }
    }
    m->dtype = dtype;
    m->finalized = true;
    m->host.clear();  // weights now live in HBM only (and any mapped file is released)
    return EBH_OK;
}

void ebh_destroy(ebh_model* m) {
    if (!m) return;
    if (m->device >= 0) {   // also after a failed ebh_finalize that got as far as the device
        (void)hipSetDevice(m->device);
        if (m->stream) (void)hipStreamSynchronize(m->stream);
        for (auto& p : m->prof_events) { (void)hipEventDestroy(p.a); (void)hipEventDestroy(p.b); }
        for (auto& e : m->prof_free) (void)hipEventDestroy(e);
        drop_graphs(m);
        if (m->ws.base) (void)hipFree(m->ws.base);
        if (m->wbase) (void)hipFree(m->wbase);
        for (HostSlot& hs : m->slots) {
            if (hs.ids) (void)hipHostFree(hs.ids);
            if (hs.mask) (void)hipHostFree(hs.mask);
            if (hs.out) (void)hipHostFree(hs.out);
            if (hs.done) (void)hipEventDestroy(hs.done);
        }
        if (m->done) (void)hipEventDestroy(m->done);
        if (m->stream) (void)hipStreamDestroy(m->stream);
    }
    delete m;
}

int ebh_forward(ebh_model* m, const float* input_ids, const float* attention_mask, int32_t B,
                int32_t S, float* out) {
    int rc = check_model_ready(m);
    if (rc) return rc;
    if ((rc = check_dims(m, B, S))) return rc;
    if (B == 0) return EBH_OK;  // src/lib.rs:480-482
    if (!input_ids || !attention_mask || !out) return fail(EBH_ERR_INVALID_ARG, "null buffer");
    const int H = m->cfg.hidden_size;
    if (S == 0) {  // mean over an empty sequence: zeros (count clamps to 1)
        memset(out, 0, sizeof(float) * (size_t)B * H);
        return EBH_OK;
    }
    const int64_t T = (int64_t)B * S;
    return host_forward(m, B, S, 0, out, false, [&](int* h_ids, int* h_mask) -> int {
        for (int64_t i = 0; i < T; ++i) {
            // `token_id as usize` (src/lib.rs:639): truncation; NaN / negatives -> 0.
            const float f = input_ids[i];
            int64_t id = (f > 0.0f) ? (f >= 9.2e18f ? INT64_MAX : (int64_t)f) : 0;
            if (id >= m->cfg.vocab_size)
                return fail(EBH_ERR_RANGE, "token id %lld at [%lld, %lld] out of range for vocab %d",
                            (long long)id, (long long)(i / S), (long long)(i % S), m->cfg.vocab_size);
            const float mk = attention_mask[i];
            if (mk != 0.0f && mk != 1.0f)
                return fail(EBH_ERR_INVALID_ARG, "attention mask value %g at [%lld, %lld] is not 0 or 1",
                            (double)mk, (long long)(i / S), (long long)(i % S));
            h_ids[i] = (int)id;
            h_mask[i] = mk != 0.0f;
        }
        return EBH_OK;
    });
}

// u32 ids / mask (the tokenizer's output) -> pinned staging, validated.
static int stage_u32(const ebh_model* m, const uint32_t* ids, const uint32_t* mask, int S, int64_t T, int* h_ids,
              int* h_mask) {
    for (int64_t i = 0; i < T; ++i) {
        if (ids[i] >= (uint32_t)m->cfg.vocab_size)
            return fail(EBH_ERR_RANGE, "token id %u at [%lld, %lld] out of range for vocab %d",
                        ids[i], (long long)(i / S), (long long)(i % S), m->cfg.vocab_size);
        if (mask[i] > 1)
            return fail(EBH_ERR_INVALID_ARG, "attention mask value %u at [%lld, %lld] is not 0 or 1",
                        mask[i], (long long)(i / S), (long long)(i % S));
        h_ids[i] = (int)ids[i];
        h_mask[i] = (int)mask[i];
    }
    return EBH_OK;
}

int ebh_encode(ebh_model* m, const uint32_t* ids, const uint32_t* mask, int32_t B, int32_t S,
               int32_t normalize, float* out) {
    int rc = check_model_ready(m);
    if (rc) return rc;
    if ((rc = check_dims(m, B, S))) return rc;
    if (B == 0) return EBH_OK;
    if (!ids || !mask || !out) return fail(EBH_ERR_INVALID_ARG, "null buffer");
    const int H = m->cfg.hidden_size;
    if (S == 0) {
        memset(out, 0, sizeof(float) * (size_t)B * H);
        return EBH_OK;
    }
    const int64_t T = (int64_t)B * S;
    return host_forward(m, B, S, normalize ? 1 : 0, out, false, [&](int* h_ids, int* h_mask) {
        return stage_u32(m, ids, mask, S, T, h_ids, h_mask);
    });
}

int ebh_encode_device(ebh_model* m, const int32_t* ids, const int32_t* mask, int32_t B,
                      int32_t S, int32_t normalize, float* out, void* stream) {
    int rc = check_model_ready(m);
    if (rc) return rc;
    if ((rc = check_dims(m, B, S))) return rc;
    if (B == 0) return EBH_OK;
    if (!ids || !mask || !out) return fail(EBH_ERR_INVALID_ARG, "null buffer");
    std::lock_guard<std::mutex> lk(m->mu);
    HIP_TRY(hipSetDevice(m->device));
    hipStream_t s = stream ? static_cast<hipStream_t>(stream) : m->stream;
    if (S == 0) {   // mean over an empty sequence: zero rows, ordered like a forward
        if (m->has_done) HIP_TRY(hipStreamWaitEvent(s, m->done, 0));
        HIP_TRY(ebh::launch_zero_words(out, (int64_t)B * m->cfg.hidden_size, s));
        HIP_TRY(hipEventRecord(m->done, s));
        m->has_done = true;
        return EBH_OK;
    }
    if ((rc = ensure_workspace(m, B, S))) return rc;
    return run_forward(m, ids, mask, B, S, normalize ? 1 : 0, out, s, nullptr, nullptr);
}

int ebh_encode_device_noalloc(ebh_model* m, const int32_t* ids, const int32_t* mask, int32_t B, int32_t S,
                              int32_t normalize, float* out, void* stream) {
    int rc = check_model_ready(m);
    if (rc) return rc;
    if ((rc = check_dims(m, B, S))) return rc;
    if (B == 0) return EBH_OK;
    if (!ids || !mask || !out) return fail(EBH_ERR_INVALID_ARG, "null buffer");
    Workspace w;
    const int64_t T = (int64_t)B * S;
    const size_t need = layout_workspace(m, T, B, nullptr, w);
    if (need > (size_t)EBH_NOALLOC_SCRATCH_BYTES)
        return fail(EBH_ERR_RANGE,
                    "batch %d x %d needs %zu bytes of workspace, more than the %zu bytes of the static scratch "
                    "of ebh_encode_device_noalloc (use ebh_encode_device)",
                    B, S, need, (size_t)EBH_NOALLOC_SCRATCH_BYTES);
    std::lock_guard<std::mutex> lk(m->mu);
    HIP_TRY(hipSetDevice(m->device));
    char* base = scratch_ptr(m->device);
    if (!base) return fail(EBH_ERR_STATE, "no scratch workspace on device %d", m->device);
    hipStream_t s = stream ? static_cast<hipStream_t>(stream) : m->stream;
    if (m->has_done) HIP_TRY(hipStreamWaitEvent(s, m->done, 0));
    if (S == 0) {
        HIP_TRY(ebh::launch_zero_words(out, (int64_t)B * m->cfg.hidden_size, s));
    } else {
        layout_workspace(m, T, B, base, w);
        w.err = m->noalloc_err;   // this model's flag, not the shared array's
        if ((rc = enqueue_kernels(m, w, ids, mask, B, S, normalize ? 1 : 0, out, s, nullptr, -1, false)))
            return rc;
    }
    HIP_TRY(hipEventRecord(m->done, s));
    m->has_done = true;
    m->noalloc_used = true;
    return EBH_OK;
}

int ebh_score(ebh_model* m, const uint32_t* ids, const uint32_t* mask, int32_t B, int32_t S,
              float* scores) {
    int rc = check_model_ready(m);
    if (rc) return rc;
    if (!m->cross_encoder) return fail(EBH_ERR_STATE, "Model is not a cross-encoder");
    if ((rc = check_dims(m, B, S))) return rc;
    if (B == 0) return EBH_OK;
    if (!ids || !mask || !scores) return fail(EBH_ERR_INVALID_ARG, "null buffer");
    if (S == 0) return fail(EBH_ERR_INVALID_ARG, "empty pair encoding (S == 0)");
    const int64_t T = (int64_t)B * S;
    return host_forward(m, B, S, 0, scores, true, [&](int* h_ids, int* h_mask) {
        return stage_u32(m, ids, mask, S, T, h_ids, h_mask);
    });
}

// Tokenised texts (host threads, outside the model's lock) -> pinned staging -> forward.
static int forward_texts(ebh_model* m, const ebh_tokenizer* t, const char* const* texts, const int64_t* lens,
                         int32_t n, int32_t normalize, float* out, int32_t nthreads, bool score) {
    int rc = check_model_ready(m);
    if (rc) return rc;
    if (score && !m->cross_encoder) return fail(EBH_ERR_STATE, "Model is not a cross-encoder");
    if (!t) return fail(EBH_ERR_INVALID_ARG, "null tokenizer");
    if (n < 0) return fail(EBH_ERR_INVALID_ARG, "negative batch");
    if (n == 0) return EBH_OK;
    if (!texts || !out) return fail(EBH_ERR_INVALID_ARG, "null buffer");
    std::vector<std::vector<int32_t>> seqs;
    int S = 0;
    if ((rc = ebh::tokenize_batch(t, texts, lens, n, nthreads, seqs, &S))) return rc;
    if ((rc = check_dims(m, n, S))) return rc;
    const int64_t T = (int64_t)n * S;
    return host_forward(m, n, S, normalize ? 1 : 0, out, score, [&](int* h_ids, int* h_mask) -> int {
        ebh::write_padded(t, seqs, S, h_ids, h_mask);
        for (int64_t i = 0; i < T; ++i)
            if (h_ids[i] < 0 || h_ids[i] >= m->cfg.vocab_size)
                return fail(EBH_ERR_RANGE, "token id %d at [%lld, %lld] out of range for vocab %d", h_ids[i],
                            (long long)(i / S), (long long)(i % S), m->cfg.vocab_size);
        return EBH_OK;
    });
}

int ebh_encode_texts(ebh_model* m, const ebh_tokenizer* t, const char* const* texts, const int64_t* lens,
                     int32_t n, int32_t normalize, float* out, int32_t nthreads) {
    return forward_texts(m, t, texts, lens, n, normalize, out, nthreads, false);
}

int ebh_score_texts(ebh_model* m, const ebh_tokenizer* t, const char* const* queries, const int64_t* q_lens,
                    const char* const* documents, const int64_t* d_lens, int32_t n, float* scores,
                    int32_t nthreads) {
    if (n > 0 && (!queries || !documents)) return fail(EBH_ERR_INVALID_ARG, "null buffer");
    std::vector<std::string> pairs(n > 0 ? n : 0);
    std::vector<const char*> ptrs(pairs.size());
    std::vector<int64_t> lens(pairs.size());
    for (int32_t i = 0; i < n; ++i) {
        const int64_t ql = q_lens ? q_lens[i] : (queries[i] ? (int64_t)strlen(queries[i]) : -1);
        const int64_t dl = d_lens ? d_lens[i] : (documents[i] ? (int64_t)strlen(documents[i]) : -1);
        if (ql < 0 || dl < 0 || (ql && !queries[i]) || (dl && !documents[i]))
            return fail(EBH_ERR_INVALID_ARG, "null text or negative length at %d", i);
        pairs[i].assign(queries[i] ? queries[i] : "", ql);   // "{query} [SEP] {document}", src/lib.rs:331
        pairs[i] += " [SEP] ";
        pairs[i].append(documents[i] ? documents[i] : "", dl);
        ptrs[i] = pairs[i].data();
        lens[i] = (int64_t)pairs[i].size();
    }
    return forward_texts(m, t, ptrs.data(), lens.data(), n, 0, scores, nthreads, true);
}

int ebh_score_device(ebh_model* m, const int32_t* ids, const int32_t* mask, int32_t B, int32_t S,
                     float* scores, void* stream) {
    int rc = check_model_ready(m);
    if (rc) return rc;
    if (!m->cross_encoder) return fail(EBH_ERR_STATE, "Model is not a cross-encoder");
    if ((rc = check_dims(m, B, S))) return rc;
    if (B == 0) return EBH_OK;
    if (!ids || !mask || !scores) return fail(EBH_ERR_INVALID_ARG, "null buffer");
    if (S == 0) return fail(EBH_ERR_INVALID_ARG, "empty pair encoding (S == 0)");
    std::lock_guard<std::mutex> lk(m->mu);
    HIP_TRY(hipSetDevice(m->device));
    hipStream_t s = stream ? static_cast<hipStream_t>(stream) : m->stream;
    if ((rc = ensure_workspace(m, B, S))) return rc;
    return run_forward(m, ids, mask, B, S, 0, m->ws.out, s, scores, nullptr);
}

int ebh_synchronize(ebh_model* m) {
    int rc = check_model_ready(m);
    if (rc) return rc;
    std::lock_guard<std::mutex> lk(m->mu);
    HIP_TRY(hipSetDevice(m->device));
    if (m->has_done) HIP_TRY(hipEventSynchronize(m->done));
    int err = 0;
    for (int* flag : {m->ws.base ? m->ws.err : nullptr, m->noalloc_used ? m->noalloc_err : nullptr}) {
        if (!flag) continue;
        int e = 0;
        HIP_TRY(hipMemcpy(&e, flag, 4, hipMemcpyDeviceToHost));
        if (e) HIP_TRY(hipMemset(flag, 0, 4));
        err |= e;
    }
    if (err) {
        HIP_TRY(hipStreamSynchronize(nullptr));  // cleared before the next forward can set it
        return fail(EBH_ERR_RANGE, "token id out of range for vocab %d", m->cfg.vocab_size);
    }
    return EBH_OK;
}

int ebh_last_tokens(ebh_model* m, int32_t* tok_ids, int32_t* tok_pos, int64_t tok_capacity,
                    int32_t* cu_seqlens, int64_t cu_capacity, int32_t* n_tokens) {
    int rc = check_model_ready(m);
    if (rc) return rc;
    std::lock_guard<std::mutex> lk(m->mu);
    HIP_TRY(hipSetDevice(m->device));
    if (!m->ws.base || !m->has_done) return fail(EBH_ERR_STATE, "no forward has run");
    HIP_TRY(hipEventSynchronize(m->done));
    int n = 0;
    HIP_TRY(hipMemcpy(&n, m->ws.ntok, 4, hipMemcpyDeviceToHost));
    if (n_tokens) *n_tokens = n;
    if ((tok_ids || tok_pos) && tok_capacity < n)
        return fail(EBH_ERR_INVALID_ARG, "token capacity %lld < %d", (long long)tok_capacity, n);
    if (tok_ids) HIP_TRY(hipMemcpy(tok_ids, m->ws.tok_id, (size_t)n * 4, hipMemcpyDeviceToHost));
    if (tok_pos) HIP_TRY(hipMemcpy(tok_pos, m->ws.tok_pos, (size_t)n * 4, hipMemcpyDeviceToHost));
    if (cu_seqlens) {
        if (cu_capacity < m->last_B + 1)
            return fail(EBH_ERR_INVALID_ARG, "cu_seqlens capacity %lld < %d", (long long)cu_capacity, m->last_B + 1);
        HIP_TRY(hipMemcpy(cu_seqlens, m->ws.cu, (size_t)(m->last_B + 1) * 4, hipMemcpyDeviceToHost));
    }
    return EBH_OK;
}

int ebh_model_info(const ebh_model* m, ebh_config* cfg_out, int32_t* dtype_out) {
    if (!m) return fail(EBH_ERR_INVALID_ARG, "null model");
    if (cfg_out) *cfg_out = m->cfg;
    if (dtype_out) *dtype_out = m->dtype;
    return EBH_OK;
}

int ebh_set_graph_replay(ebh_model* m, int32_t enable) {
    int rc = check_model_ready(m);
    if (rc) return rc;
    std::lock_guard<std::mutex> lk(m->mu);
    HIP_TRY(hipSetDevice(m->device));
    m->graph_replay = enable != 0;
    if (!m->graph_replay) {
        if (m->has_done) HIP_TRY(hipEventSynchronize(m->done));
        drop_graphs(m);
    }
    return EBH_OK;
}

int ebh_profile_enable(ebh_model* m, int32_t kernel) {
    int rc = check_model_ready(m);
    if (rc) return rc;
    if (kernel < EBH_PROF_NONE || kernel > EBH_PROF_POOL)
        return fail(EBH_ERR_INVALID_ARG, "unknown kernel id %d", kernel);
    std::lock_guard<std::mutex> lk(m->mu);
    HIP_TRY(hipSetDevice(m->device));
    if (m->has_done) HIP_TRY(hipEventSynchronize(m->done));
    for (auto& p : m->prof_events) { m->prof_free.push_back(p.a); m->prof_free.push_back(p.b); }
    m->prof_events.clear();
    m->prof_kind = kernel;
    return EBH_OK;
}

int ebh_profile_read(ebh_model* m, int64_t* launches, double* total_ms) {
    int rc = check_model_ready(m);
    if (rc) return rc;
    std::lock_guard<std::mutex> lk(m->mu);
    HIP_TRY(hipSetDevice(m->device));
    double tot = 0.0;
    for (auto& p : m->prof_events) {
        HIP_TRY(hipEventSynchronize(p.b));
        float ms = 0.0f;
        HIP_TRY(hipEventElapsedTime(&ms, p.a, p.b));
        tot += ms;
    }
    if (launches) *launches = (int64_t)m->prof_events.size();
    if (total_ms) *total_ms = tot;
    return EBH_OK;
}

// ---------------------------------------------------------------------------
// op-level entry points (edgebert_hip_ops.h)
// ---------------------------------------------------------------------------
int ebh_op_gemm(const float* A, int64_t lda, const void* W, int64_t ldw, int32_t w_dtype,
                const float* bias, const float* residual, int64_t ldr, float* C, int64_t ldc,
                int32_t M, int32_t N, int32_t K, int32_t epilogue, void* stream) {
    if (!A || !W || !C || (!bias && epilogue != EBH_EPI_NONE))
        return fail(EBH_ERR_INVALID_ARG, "null buffer");
    if (M < 0 || N <= 0 || K <= 0) return fail(EBH_ERR_INVALID_ARG, "bad GEMM shape");
    if (epilogue < EBH_EPI_BIAS || epilogue > EBH_EPI_NONE)
        return fail(EBH_ERR_INVALID_ARG, "unknown epilogue %d", epilogue);
    if (epilogue == EBH_EPI_BIAS_RESID && (!residual || ldr < N))
        return fail(EBH_ERR_INVALID_ARG, "residual epilogue needs a residual of row stride >= N");
    const int q = w_dtype == EBH_DTYPE_BF16 ? 8 : 4;
    if (w_dtype != EBH_DTYPE_F32 && w_dtype != EBH_DTYPE_BF16 && w_dtype != EBH_DTYPE_F32_BF16X6)
        return fail(EBH_ERR_INVALID_ARG, "unknown dtype %d", w_dtype);
    if (K % q || lda % 4 || ldw % q || lda < K || ldw < K || ldc < N)
        return fail(EBH_ERR_INVALID_ARG, "K and strides must be multiples of %d and cover the rows", q);
    if (M == 0) return EBH_OK;
    ebh::GemmArgs a{};
    a.A = A; a.W = W; a.bias = bias; a.R = residual; a.C = C;
    a.lda = lda; a.ldw = ldw; a.ldr = ldr; a.ldc = ldc;
    a.M_max = M; a.M_dev = nullptr; a.N = N; a.K = K;
    a.split6 = w_dtype == EBH_DTYPE_F32_BF16X6;
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipError_t e = w_dtype == EBH_DTYPE_BF16 ? ebh::launch_gemm_bf16(a, epilogue, s)
                                              : ebh::launch_gemm_f32(a, epilogue, s);
    if (e != hipSuccess) return fail(EBH_ERR_HIP, "gemm launch failed: %s", hipGetErrorString(e));
    return EBH_OK;
}

int ebh_op_gemm_bf16(const uint16_t* A, int64_t lda, const uint16_t* W, int64_t ldw,
                     const float* bias, void* C, int64_t ldc, int32_t c_dtype, int32_t M, int32_t N,
                     int32_t K, int32_t epilogue, void* stream) {
    if (!A || !W || !C || (!bias && epilogue != EBH_EPI_NONE)) return fail(EBH_ERR_INVALID_ARG, "null buffer");
    if (M < 0 || N <= 0 || K <= 0) return fail(EBH_ERR_INVALID_ARG, "bad GEMM shape");
    if (epilogue != EBH_EPI_BIAS && epilogue != EBH_EPI_BIAS_GELU && epilogue != EBH_EPI_NONE)
        return fail(EBH_ERR_INVALID_ARG, "epilogue %d not supported with bf16 activations", epilogue);
    if (c_dtype != EBH_DTYPE_F32 && c_dtype != EBH_DTYPE_BF16)
        return fail(EBH_ERR_INVALID_ARG, "unknown output dtype %d", c_dtype);
    if (K % 64 || N % 4 || lda % 8 || ldw % 8 || ldc % 4 || lda < K || ldw < K || ldc < N)
        return fail(EBH_ERR_INVALID_ARG, "K must be a multiple of 64, N of 4, strides of 8 / 8 / 4");
    if (((uintptr_t)A | (uintptr_t)W | (uintptr_t)C | (uintptr_t)bias) & 15)
        return fail(EBH_ERR_INVALID_ARG, "operands must be 16-byte aligned");
    if (!ebh::gemm_offsets_fit32(lda, ldw, 2))
        return fail(EBH_ERR_INVALID_ARG, "row strides lda %lld / ldw %lld too large (at most %lld elements)",
                    (long long)lda, (long long)ldw, (long long)ebh::gemm_stride_max(2));
    if (M == 0) return EBH_OK;
    ebh::GemmArgs a{};
    a.A = A; a.W = W; a.bias = bias; a.R = nullptr; a.C = static_cast<float*>(C);
    a.lda = lda; a.ldw = ldw; a.ldr = 0; a.ldc = ldc;
    a.M_max = M; a.M_dev = nullptr; a.N = N; a.K = K;
    hipError_t e = ebh::launch_gemm_bf16_act(a, epilogue, c_dtype == EBH_DTYPE_BF16,
                                             static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return fail(EBH_ERR_HIP, "gemm launch failed: %s", hipGetErrorString(e));
    return EBH_OK;
}

int ebh_op_attention(const float* qkv, const int32_t* cu_seqlens, int32_t B, int32_t max_len,
                     int32_t hidden, int32_t num_heads, float* ctx, void* stream) {
    if (!qkv || !cu_seqlens || !ctx) return fail(EBH_ERR_INVALID_ARG, "null buffer");
    if (B < 0 || max_len < 0 || hidden <= 0 || num_heads <= 0 || hidden % num_heads)
        return fail(EBH_ERR_INVALID_ARG, "bad attention shape");
    const int hd = hidden / num_heads;
    if (hd != 32 && hd != 64) return fail(EBH_ERR_INVALID_ARG, "head_dim %d unsupported", hd);
    if (reinterpret_cast<uintptr_t>(qkv) % 16 || reinterpret_cast<uintptr_t>(ctx) % 16)
        return fail(EBH_ERR_INVALID_ARG, "qkv and ctx must be 16-byte aligned");
    const float scale = 1.0f / sqrtf((float)hd);
    HIP_TRY(ebh::launch_attention(qkv, cu_seqlens, B, max_len, hidden, num_heads, hd, scale, ctx,
                                  static_cast<hipStream_t>(stream)));
    return EBH_OK;
}

int ebh_op_attention_bf16(const uint16_t* qkv, const int32_t* cu_seqlens, int32_t B,
                          int32_t max_len, int32_t hidden, int32_t num_heads, uint16_t* ctx,
                          void* stream) {
    if (!qkv || !cu_seqlens || !ctx) return fail(EBH_ERR_INVALID_ARG, "null buffer");
    if (B < 0 || max_len < 0 || hidden <= 0 || num_heads <= 0 || hidden % num_heads)
        return fail(EBH_ERR_INVALID_ARG, "bad attention shape");
    const int hd = hidden / num_heads;
    if (hd != 32 && hd != 64) return fail(EBH_ERR_INVALID_ARG, "head_dim %d unsupported", hd);
    if (reinterpret_cast<uintptr_t>(qkv) % 16 || reinterpret_cast<uintptr_t>(ctx) % 8)
        return fail(EBH_ERR_INVALID_ARG, "qkv must be 16-byte and ctx 8-byte aligned");
    const float scale = 1.0f / sqrtf((float)hd);
    HIP_TRY(ebh::launch_attention_bf16(qkv, cu_seqlens, B, max_len, hidden, num_heads, hd, scale,
                                       ctx, static_cast<hipStream_t>(stream)));
    return EBH_OK;
}

int ebh_op_layer_norm(const float* x, const float* gamma, const float* beta, int32_t rows,
                      int32_t H, float eps, float* y, void* stream) {
    if (!x || !gamma || !beta || !y) return fail(EBH_ERR_INVALID_ARG, "null buffer");
    if (rows < 0 || H <= 0 || H > 2048) return fail(EBH_ERR_INVALID_ARG, "bad LayerNorm shape");
    HIP_TRY(ebh::launch_layernorm(x, y, gamma, beta, rows, nullptr, H, eps,
                                  static_cast<hipStream_t>(stream)));
    return EBH_OK;
}

int ebh_op_add_layer_norm(const float* y, const float* bias, float* x, const float* gamma,
                          const float* beta, int32_t rows, int32_t H, float eps, void* stream) {
    if (!y || !bias || !x || !gamma || !beta) return fail(EBH_ERR_INVALID_ARG, "null buffer");
    if (rows < 0 || H <= 0 || H > 2048) return fail(EBH_ERR_INVALID_ARG, "bad LayerNorm shape");
    HIP_TRY(ebh::launch_add_layernorm(y, bias, x, gamma, beta, rows, nullptr, H, eps, nullptr,
                                      static_cast<hipStream_t>(stream)));
    return EBH_OK;
}

int ebh_op_gemm_add_layer_norm(const float* A, int64_t lda, const float* W, int64_t ldw,
                               const float* bias, float* x, const float* gamma, const float* beta,
                               int32_t M, int32_t N, int32_t K, float eps, void* stream) {
    if (!A || !W || !bias || !x || !gamma || !beta) return fail(EBH_ERR_INVALID_ARG, "null buffer");
    if (M < 0 || N != 384 || K <= 0 || K % 32 || lda < K || ldw < K || lda % 4 || ldw % 4)
        return fail(EBH_ERR_INVALID_ARG, "bad fused LayerNorm GEMM shape (N must be 384, K %% 32 == 0)");
    if (!ebh::gemm_offsets_fit32(lda, ldw, 4))
        return fail(EBH_ERR_INVALID_ARG, "row strides lda %lld / ldw %lld too large (at most %lld elements)",
                    (long long)lda, (long long)ldw, (long long)ebh::gemm_stride_max(4));
    ebh::GemmArgs a{};
    a.A = A;
    a.W = W;
    a.bias = bias;
    a.R = x;
    a.C = x;
    a.lda = lda;
    a.ldw = ldw;
    a.ldr = N;
    a.ldc = N;
    a.M_max = M;
    a.M_dev = nullptr;
    a.N = N;
    a.K = K;
    a.ln_g = gamma;
    a.ln_b = beta;
    a.ln_eps = eps;
    HIP_TRY(ebh::launch_gemm_f32_add_ln(a, static_cast<hipStream_t>(stream)));
    return EBH_OK;
}

int ebh_op_add_layer_norm_y16(const uint16_t* y, const float* bias, float* x, const float* gamma,
                              const float* beta, int32_t rows, int32_t H, float eps, void* stream) {
    if (!y || !bias || !x || !gamma || !beta) return fail(EBH_ERR_INVALID_ARG, "null buffer");
    if (rows < 0 || H <= 0 || !ebh::row4_shape_ok(H)) return fail(EBH_ERR_INVALID_ARG, "bad LayerNorm shape");
    HIP_TRY(ebh::launch_add_layernorm_y16(y, bias, x, gamma, beta, rows, nullptr, H, eps, nullptr,
                                          static_cast<hipStream_t>(stream)));
    return EBH_OK;
}

int ebh_op_add_layer_norm_b16(const uint16_t* y, const float* bias, uint16_t* x16, const float* gamma,
                              const float* beta, int32_t rows, int32_t H, float eps, void* stream) {
    if (!y || !bias || !x16 || !gamma || !beta) return fail(EBH_ERR_INVALID_ARG, "null buffer");
    if (rows < 0 || H <= 0 || !ebh::row4_shape_ok(H)) return fail(EBH_ERR_INVALID_ARG, "bad LayerNorm shape");
    HIP_TRY(ebh::launch_add_layernorm_y16(y, bias, nullptr, gamma, beta, rows, nullptr, H, eps, x16,
                                          static_cast<hipStream_t>(stream)));
    return EBH_OK;
}

int ebh_op_pool(const float* x, const int32_t* cu_seqlens, int32_t B, int32_t H, int32_t S,
                int32_t normalize, float* partials, float* out, void* stream) {
    if (!x || !cu_seqlens || !out) return fail(EBH_ERR_INVALID_ARG, "null buffer");
    if (B < 0 || H <= 0 || H > 2048 || S < 0) return fail(EBH_ERR_INVALID_ARG, "bad pool shape");
    auto al16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
    if (ebh::pool_partials_floats(B, H, S) > 0 && al16(x) && al16(out) && (!partials || !al16(partials)))
        return fail(EBH_ERR_INVALID_ARG, "partials: null or not 16-byte aligned");
    HIP_TRY(ebh::launch_pool(x, cu_seqlens, B, H, S, normalize ? 1 : 0, partials, out,
                             static_cast<hipStream_t>(stream)));
    return EBH_OK;
}

int ebh_op_pool_b16(const uint16_t* x16, const int32_t* cu_seqlens, int32_t B, int32_t H, int32_t S,
                    int32_t normalize, float* out, void* stream) {
    if (!x16 || !cu_seqlens || !out) return fail(EBH_ERR_INVALID_ARG, "null buffer");
    if (B < 0 || H <= 0 || H > 2048 || S < 0) return fail(EBH_ERR_INVALID_ARG, "bad pool shape");
    HIP_TRY(ebh::launch_pool_b16(x16, cu_seqlens, B, H, S, normalize ? 1 : 0, out,
                                 static_cast<hipStream_t>(stream)));
    return EBH_OK;
}

int ebh_op_pack(const int32_t* ids, const int32_t* mask, int32_t B, int32_t S, int32_t* counts,
                int32_t* cu_seqlens, int32_t* n_tokens, int32_t* tok_id, int32_t* tok_pos,
                int32_t* err, void* stream) {
    if (!ids || !mask || !counts || !cu_seqlens || !n_tokens || !tok_id || !tok_pos || !err)
        return fail(EBH_ERR_INVALID_ARG, "null buffer");
    if (B < 0 || S < 0) return fail(EBH_ERR_INVALID_ARG, "bad pack shape");
    HIP_TRY(ebh::launch_pack(ids, mask, B, S, counts, cu_seqlens, n_tokens, tok_id, tok_pos,
                             static_cast<hipStream_t>(stream)));
    HIP_TRY(ebh::launch_zero_words(err, 1, static_cast<hipStream_t>(stream)));
    return EBH_OK;
}

int ebh_op_embed_ln(const int32_t* tok_id, const int32_t* tok_pos, const int32_t* n_tokens,
                    int32_t T_max, const float* word, const float* pos, const float* type0,
                    const float* gamma, const float* beta, int32_t V, int32_t H, float eps,
                    float* x, int32_t* err, void* stream) {
    if (!tok_id || !tok_pos || !n_tokens || !word || !pos || !type0 || !gamma || !beta || !x || !err)
        return fail(EBH_ERR_INVALID_ARG, "null buffer");
    if (T_max < 0 || V <= 0 || H <= 0 || H > 2048) return fail(EBH_ERR_INVALID_ARG, "bad embed shape");
    HIP_TRY(ebh::launch_embed_ln(tok_id, tok_pos, n_tokens, T_max, word, pos, type0, gamma, beta,
                                 V, H, eps, x, err, nullptr, static_cast<hipStream_t>(stream)));
    return EBH_OK;
}

int ebh_op_f32_to_bf16(const float* x, uint16_t* y, int64_t n, void* stream) {
    if (!x || !y || n < 0) return fail(EBH_ERR_INVALID_ARG, "bad conversion arguments");
    HIP_TRY(ebh::launch_f32_to_bf16(x, y, n, static_cast<hipStream_t>(stream)));
    return EBH_OK;
}

int ebh_op_widen16(const uint16_t* x, void* y, int64_t n, int32_t mode, void* stream) {
    if (!x || !y || n < 0 || mode < ebh::WIDEN_F16_F32 || mode > ebh::WIDEN_F16_BF16)
        return fail(EBH_ERR_INVALID_ARG, "bad conversion arguments");
    HIP_TRY(ebh::launch_widen16(x, y, n, mode, static_cast<hipStream_t>(stream)));
    return EBH_OK;
}

int ebh_op_gelu(const float* x, float* y, int64_t n, void* stream) {
    if (!x || !y || n < 0) return fail(EBH_ERR_INVALID_ARG, "bad GELU arguments");
    HIP_TRY(ebh::launch_gelu(x, y, n, static_cast<hipStream_t>(stream)));
    return EBH_OK;
}

}  // extern "C"
