/*
 * oracle.c -- CPU restatement of EdgeBERT's BERT encoder forward.
 *
 * TEST INFRASTRUCTURE ONLY: this is the checker (and the "port" CPU baseline)
 * for the HIP path in edgebert_amd/.  Nothing in the product links or calls it.
 * Every function cites the reference lines (under /root/reference) it restates.
 *
 * Arithmetic follows the reference's evaluation order in fp32 and is compiled
 * with -ffp-contract=off, so elementwise steps are not fused.  Two pieces live
 * in third-party crates that are not under /root/reference and are restated
 * from their published algorithms:
 *   - ndarray 0.16 `.dot` -> matrixmultiply 0.3 sgemm (Cargo.toml:35-36): here a
 *     packed 6x16 AVX2/FMA micro-kernel; summation order differs from the crate's
 *     (bit-level parity unpinned, only tolerance-level parity is claimed);
 *   - ndarray 0.16 `sum` (eight-way unrolled fold) and `var_axis` (Welford with
 *     mul_add), used by mean_axis / var_axis / sum_axis.
 * The reference's `openblas` feature (Cargo.toml:14, lib.rs:1-2) turns on
 * ndarray's `blas` feature, which sends `.dot` to cblas_sgemm.  That variant is
 * here too: orc_set_blas_sgemm() hands in a CBLAS (ILP64) sgemm, and every
 * product then goes to it, one call per batch slice as `.dot` makes them, the
 * slices spread over threads as the reference's rayon loops spread them.
 */
#include "oracle.h"

#include <immintrin.h>
#include <math.h>
#include <omp.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static __thread char g_err[512];

static int fail(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return -1;
}

const char* orc_last_error(void) { return g_err; }

static int g_threads = 0;
static orc_cblas_sgemm_fn g_blas = NULL;
void orc_set_blas_sgemm(orc_cblas_sgemm_fn fn) { g_blas = fn; }

/* c[m,n] = a[m,k] . b[k,n] through the CBLAS sgemm (row-major, no transposes,
 * alpha 1, beta 0: ndarray's `dot` into a fresh array). */
enum { CBLAS_ROW_MAJOR = 101, CBLAS_NO_TRANS = 111 };
static void blas_dot(int m, int n, int k, const float* a, int lda, const float* b, int ldb,
                     float* c, int ldc) {
    if (k <= 0) {   /* an empty sum; CBLAS would reject lda = 0 */
        for (int i = 0; i < m; ++i) memset(c + (size_t)i * ldc, 0, sizeof(float) * n);
        return;
    }
    g_blas(CBLAS_ROW_MAJOR, CBLAS_NO_TRANS, CBLAS_NO_TRANS, m, n, k, 1.0f, a, lda, b, ldb, 0.0f,
           c, ldc);
}
void orc_set_num_threads(int n) { g_threads = n > 0 ? n : 0; if (n > 0) omp_set_num_threads(n); }
int orc_get_num_threads(void) { return g_threads > 0 ? g_threads : omp_get_max_threads(); }

/* ------------------------------------------------------------------------- */
/* ndarray numeric helpers                                                    */
/* ------------------------------------------------------------------------- */

/* ndarray `sum()` on a contiguous lane: eight partial accumulators, combined as
 * (p0+p4), (p1+p5), (p2+p6), (p3+p7), then the tail in order. */
static float nd_sum(const float* x, int n) {
    float p[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int i = 0;
    for (; i + 8 <= n; i += 8)
        for (int j = 0; j < 8; ++j) p[j] = p[j] + x[i + j];
    float acc = 0.0f;
    acc = acc + (p[0] + p[4]);
    acc = acc + (p[1] + p[5]);
    acc = acc + (p[2] + p[6]);
    acc = acc + (p[3] + p[7]);
    for (; i < n; ++i) acc = acc + x[i];
    return acc;
}

/* ndarray `var_axis(.., 0.0)`: Welford update with mul_add, population divisor. */
static float nd_var(const float* x, int n) {
    float mean = 0.0f, sum_sq = 0.0f;
    for (int i = 0; i < n; ++i) {
        float count = (float)(i + 1);
        float delta = x[i] - mean;
        mean = mean + delta / count;
        sum_sq = fmaf(x[i] - mean, delta, sum_sq);
    }
    return sum_sq / (float)n;
}

/* ------------------------------------------------------------------------- */
/* sgemm: c[m,n] = a[m,k] . b[k,n], row-major (ndarray `.dot`)                */
/* ------------------------------------------------------------------------- */
#define MR 6
#define NR 16

static void pack_b(int k, int n, const float* b, int ldb, float* bp) {
    int np = (n + NR - 1) / NR;
    for (int p = 0; p < np; ++p) {
        int j0 = p * NR, nc = n - j0 < NR ? n - j0 : NR;
        float* dst = bp + (size_t)p * k * NR;
        for (int kk = 0; kk < k; ++kk) {
            const float* src = b + (size_t)kk * ldb + j0;
            int j = 0;
            for (; j < nc; ++j) dst[(size_t)kk * NR + j] = src[j];
            for (; j < NR; ++j) dst[(size_t)kk * NR + j] = 0.0f;
        }
    }
}

static void micro_full(int k, const float* a, int lda, const float* bp, float* c, int ldc,
                       int nc) {
    __m256 acc[MR][2];
    for (int r = 0; r < MR; ++r) acc[r][0] = acc[r][1] = _mm256_setzero_ps();
    for (int kk = 0; kk < k; ++kk) {
        __m256 b0 = _mm256_loadu_ps(bp + (size_t)kk * NR);
        __m256 b1 = _mm256_loadu_ps(bp + (size_t)kk * NR + 8);
        for (int r = 0; r < MR; ++r) {
            __m256 av = _mm256_broadcast_ss(a + (size_t)r * lda + kk);
            acc[r][0] = _mm256_fmadd_ps(av, b0, acc[r][0]);
            acc[r][1] = _mm256_fmadd_ps(av, b1, acc[r][1]);
        }
    }
    for (int r = 0; r < MR; ++r) {
        float* cr = c + (size_t)r * ldc;
        if (nc == NR) {
            _mm256_storeu_ps(cr, acc[r][0]);
            _mm256_storeu_ps(cr + 8, acc[r][1]);
        } else {
            float tmp[NR];
            _mm256_storeu_ps(tmp, acc[r][0]);
            _mm256_storeu_ps(tmp + 8, acc[r][1]);
            for (int j = 0; j < nc; ++j) cr[j] = tmp[j];
        }
    }
}

static void micro_tail(int mr, int k, const float* a, int lda, const float* bp, float* c,
                       int ldc, int nc) {
    for (int r = 0; r < mr; ++r) {
        __m256 s0 = _mm256_setzero_ps(), s1 = _mm256_setzero_ps();
        for (int kk = 0; kk < k; ++kk) {
            __m256 av = _mm256_broadcast_ss(a + (size_t)r * lda + kk);
            s0 = _mm256_fmadd_ps(av, _mm256_loadu_ps(bp + (size_t)kk * NR), s0);
            s1 = _mm256_fmadd_ps(av, _mm256_loadu_ps(bp + (size_t)kk * NR + 8), s1);
        }
        float tmp[NR];
        _mm256_storeu_ps(tmp, s0);
        _mm256_storeu_ps(tmp + 8, s1);
        for (int j = 0; j < nc; ++j) c[(size_t)r * ldc + j] = tmp[j];
    }
}

/* One panel column block over all rows of a (panel-outer keeps bp in L1). */
static void gemm_panel(int m, int k, const float* a, int lda, const float* bpanel, float* c,
                       int ldc, int nc) {
    int i = 0;
    for (; i + MR <= m; i += MR)
        micro_full(k, a + (size_t)i * lda, lda, bpanel, c + (size_t)i * ldc, ldc, nc);
    if (i < m) micro_tail(m - i, k, a + (size_t)i * lda, lda, bpanel, c + (size_t)i * ldc, ldc, nc);
}

static void gemm_packed_serial(int m, int n, int k, const float* a, int lda, const float* bp,
                               float* c, int ldc) {
    int np = (n + NR - 1) / NR;
    for (int p = 0; p < np; ++p) {
        int j0 = p * NR, nc = n - j0 < NR ? n - j0 : NR;
        gemm_panel(m, k, a, lda, bp + (size_t)p * k * NR, c + j0, ldc, nc);
    }
}

void orc_sgemm(int m, int n, int k, const float* a, int lda, const float* b, int ldb, float* c,
               int ldc) {
    if (m <= 0 || n <= 0) return;
    if (g_blas) {
        blas_dot(m, n, k, a, lda, b, ldb, c, ldc);
        return;
    }
    if (k <= 0) {
        for (int i = 0; i < m; ++i) memset(c + (size_t)i * ldc, 0, sizeof(float) * n);
        return;
    }
    int np = (n + NR - 1) / NR;
    float* bp = (float*)malloc(sizeof(float) * (size_t)np * k * NR);
    pack_b(k, n, b, ldb, bp);
    if (omp_in_parallel()) {
        gemm_packed_serial(m, n, k, a, lda, bp, c, ldc);
    } else {
#pragma omp parallel for schedule(dynamic, 1)
        for (int p = 0; p < np; ++p) {
            int j0 = p * NR, nc = n - j0 < NR ? n - j0 : NR;
            gemm_panel(m, k, a, lda, bp + (size_t)p * k * NR, c + j0, ldc, nc);
        }
    }
    free(bp);
}

/* matmul_3d_2d (src/lib.rs:795-849): c[b] = a[b] . w for every batch slice;
 * sequential over slices when batch <= 4, parallel over slices otherwise.
 * w is packed once and shared by every slice. */
void orc_matmul_3d_2d(const float* a, int batch, int m, int k, const float* b, int n, float* c) {
    if (g_blas) {
#pragma omp parallel for schedule(dynamic, 1) if (batch > 4)
        for (int s = 0; s < batch; ++s)
            blas_dot(m, n, k, a + (size_t)s * m * k, k, b, n, c + (size_t)s * m * n, n);
        return;
    }
    if (batch <= 4) {
        for (int s = 0; s < batch; ++s)
            orc_sgemm(m, n, k, a + (size_t)s * m * k, k, b, n, c + (size_t)s * m * n, n);
        return;
    }
    int np = (n + NR - 1) / NR;
    float* bp = (float*)malloc(sizeof(float) * (size_t)np * k * NR);
    pack_b(k, n, b, n, bp);
#pragma omp parallel for schedule(dynamic, 1)
    for (int s = 0; s < batch; ++s)
        gemm_packed_serial(m, n, k, a + (size_t)s * m * k, k, bp, c + (size_t)s * m * n, n);
    free(bp);
}

/* matmul_4d (src/lib.rs:898-956): batch*heads independent products
 * [seq1,dim] . [dim,seq2]; parallel when batch*heads > 8. */
void orc_matmul_4d(const float* a, const float* b, int batch, int heads, int seq1, int dim,
                   int seq2, float* c) {
    int total = batch * heads;
    if (g_blas) {
#pragma omp parallel for schedule(dynamic, 4) if (total > 8)
        for (int t = 0; t < total; ++t)
            blas_dot(seq1, seq2, dim, a + (size_t)t * seq1 * dim, dim, b + (size_t)t * dim * seq2,
                     seq2, c + (size_t)t * seq1 * seq2, seq2);
        return;
    }
    if (total <= 8) {
        for (int t = 0; t < total; ++t)
            orc_sgemm(seq1, seq2, dim, a + (size_t)t * seq1 * dim, dim,
                      b + (size_t)t * dim * seq2, seq2, c + (size_t)t * seq1 * seq2, seq2);
        return;
    }
    int np = (seq2 + NR - 1) / NR;
#pragma omp parallel
    {
        float* bp = (float*)malloc(sizeof(float) * (size_t)np * (dim > 0 ? dim : 1) * NR);
#pragma omp for schedule(dynamic, 4)
        for (int t = 0; t < total; ++t) {
            float* ct = c + (size_t)t * seq1 * seq2;
            if (dim == 0) {
                memset(ct, 0, sizeof(float) * (size_t)seq1 * seq2);
                continue;
            }
            pack_b(dim, seq2, b + (size_t)t * dim * seq2, seq2, bp);
            gemm_packed_serial(seq1, seq2, dim, a + (size_t)t * seq1 * dim, dim, bp, ct, seq2);
        }
        free(bp);
    }
}

/* softmax (src/lib.rs:851-870): max fold from -inf, x - max, exp, sum over the
 * last axis, divide. */
void orc_softmax(float* x, int64_t rows, int n) {
#pragma omp parallel for schedule(static) if (rows > 64)
    for (int64_t r = 0; r < rows; ++r) {
        float* row = x + r * n;
        float mx = -INFINITY;
        for (int j = 0; j < n; ++j) mx = fmaxf(mx, row[j]);
        for (int j = 0; j < n; ++j) row[j] = expf(row[j] - mx);
        float s = nd_sum(row, n);
        for (int j = 0; j < n; ++j) row[j] = row[j] / s;
    }
}

/* apply_attention_mask (src/lib.rs:872-896): mask [B,S2] broadcast over heads
 * and query rows; scores where mask == 0.0 become -inf. */
void orc_apply_attention_mask(float* scores, const float* mask, int B, int nh, int S1, int S2) {
#pragma omp parallel for collapse(2) schedule(static) if ((int64_t)B * nh * S1 > 64)
    for (int b = 0; b < B; ++b)
        for (int h = 0; h < nh; ++h)
            for (int i = 0; i < S1; ++i) {
                float* row = scores + (((size_t)b * nh + h) * S1 + i) * S2;
                for (int j = 0; j < S2; ++j)
                    if (mask[(size_t)b * S2 + j] == 0.0f) row[j] = -INFINITY;
            }
}

/* gelu (src/lib.rs:958-978) with SQRT_2_OVER_PI / GELU_COEFF (src/lib.rs:151-152). */
void orc_gelu(float* x, int64_t n) {
    const float SQRT_2_OVER_PI = 0.7978845608f;
    const float GELU_COEFF = 0.044715f;
#pragma omp parallel for schedule(static) if (n > 4096)
    for (int64_t i = 0; i < n; ++i) {
        float val = x[i];
        float val_squared = val * val;
        float val_cubed = val_squared * val;
        float inner = SQRT_2_OVER_PI * (val + GELU_COEFF * val_cubed);
        x[i] = val * 0.5f * (1.0f + tanhf(inner));
    }
}

/* apply_layer_norm_3d (src/lib.rs:980-991): mean_axis, var_axis(ddof 0),
 * inv_std = 1/sqrt(var+eps), (x-mean)*inv_std*weight + bias. */
void orc_layer_norm(const float* x, int64_t rows, int H, const float* weight, const float* bias,
                    float eps, float* y) {
#pragma omp parallel for schedule(static) if (rows > 64)
    for (int64_t r = 0; r < rows; ++r) {
        const float* xr = x + r * H;
        float* yr = y + r * H;
        float mean = nd_sum(xr, H) / (float)H;
        float var = nd_var(xr, H);
        float inv_std = 1.0f / sqrtf(var + eps);
        for (int j = 0; j < H; ++j) yr[j] = (xr[j] - mean) * inv_std * weight[j] + bias[j];
    }
}

/* mean_pool (src/lib.rs:993-1010): sum over the sequence of hidden*mask
 * (subview adds in order), divided by max(sum(mask), 1). */
void orc_mean_pool(const float* hidden, const float* mask, int B, int S, int H, float* out) {
    for (int b = 0; b < B; ++b) {
        float* o = out + (size_t)b * H;
        for (int j = 0; j < H; ++j) o[j] = 0.0f;
        for (int s = 0; s < S; ++s) {
            float m = mask[(size_t)b * S + s];
            const float* h = hidden + ((size_t)b * S + s) * H;
            for (int j = 0; j < H; ++j) o[j] = o[j] + h[j] * m;
        }
        float count = nd_sum(mask + (size_t)b * S, S);
        count = fmaxf(count, 1.0f);
        for (int j = 0; j < H; ++j) o[j] = o[j] / count;
    }
}

/* encode_uncached tail (src/lib.rs:605-612): x / max(sqrt(sum x^2), 1e-12).
 * Rust's f32::max returns the non-NaN operand, as fmaxf does. */
void orc_normalize(float* x, int B, int H) {
    float* sq = (float*)malloc(sizeof(float) * (H > 0 ? H : 1));
    for (int b = 0; b < B; ++b) {
        float* r = x + (size_t)b * H;
        for (int j = 0; j < H; ++j) sq[j] = r[j] * r[j];
        float norm = fmaxf(sqrtf(nd_sum(sq, H)), 1e-12f);
        for (int j = 0; j < H; ++j) r[j] = r[j] / norm;
    }
    free(sq);
}

/* Cross-encoder head (Model::score_pair, src/lib.rs:359-375): the pooled row
 * (`forward`, not normalised) `.dot(weight) + bias`.  ndarray 0.16's 1-D `dot`
 * without BLAS is its unrolled_dot: eight partial sums of products, combined
 * as (p0+p4), (p1+p5), (p2+p6), (p3+p7), then the tail in order -- the shape
 * of its `sum` above. */
float orc_dot(const float* a, const float* b, int n) {
    float p[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int i = 0;
    for (; i + 8 <= n; i += 8)
        for (int j = 0; j < 8; ++j) p[j] = p[j] + a[i + j] * b[i + j];
    float acc = 0.0f;
    acc = acc + (p[0] + p[4]);
    acc = acc + (p[1] + p[5]);
    acc = acc + (p[2] + p[6]);
    acc = acc + (p[3] + p[7]);
    for (; i < n; ++i) acc = acc + a[i] * b[i];
    return acc;
}

/* cosine_similarity (src/lib.rs:756-789): eight-wide tree-reduced dot, plain
 * norms, dot / (|a||b| + 1e-8). */
float orc_cosine_similarity(const float* a, const float* b, int n) {
    int nc = n - n % 8;
    float chunk_dot = 0.0f;
    for (int i = 0; i < nc; i += 8) {
        float d0 = a[i] * b[i] + a[i + 1] * b[i + 1];
        float d1 = a[i + 2] * b[i + 2] + a[i + 3] * b[i + 3];
        float d2 = a[i + 4] * b[i + 4] + a[i + 5] * b[i + 5];
        float d3 = a[i + 6] * b[i + 6] + a[i + 7] * b[i + 7];
        chunk_dot = chunk_dot + ((d0 + d1) + (d2 + d3));
    }
    float tail = 0.0f;
    for (int i = nc; i < n; ++i) tail = tail + a[i] * b[i];
    float dot = chunk_dot + tail;
    float na = 0.0f, nb = 0.0f;
    for (int i = 0; i < n; ++i) na = na + a[i] * a[i];
    for (int i = 0; i < n; ++i) nb = nb + b[i] * b[i];
    return dot / (sqrtf(na) * sqrtf(nb) + 1e-8f);
}

/* ------------------------------------------------------------------------- */
/* Model assembly (Model::from_weights, src/lib.rs:155-260)                   */
/* ------------------------------------------------------------------------- */
typedef struct {
    float *wq_t, *bq, *wk_t, *bk, *wv_t, *bv, *wo_t, *bo; /* [H,H] transposed */
    float *ln1_w, *ln1_b;
    float *w1_t, *b1, *w2_t, *b2; /* w1_t [H,I], w2_t [I,H] */
    float *ln2_w, *ln2_b;
} orc_layer;

typedef struct {
    char* name;
    float* data;
    int64_t shape[2];
    int ndim;
} orc_tensor;

struct orc_model {
    int H, nh, L, I, V, P, TV;
    float eps;
    int ntensors, cap;
    orc_tensor* tensors;
    int built;
    float *word, *pos, *type, *emb_ln_w, *emb_ln_b;
    orc_layer* layers;
};

orc_model* orc_model_new(int hidden_size, int num_attention_heads, int num_hidden_layers,
                         int intermediate_size, int vocab_size, int max_position_embeddings,
                         int type_vocab_size, float layer_norm_eps) {
    if (hidden_size <= 0 || num_attention_heads <= 0 || num_hidden_layers < 0 ||
        intermediate_size <= 0 || vocab_size <= 0 || max_position_embeddings <= 0 ||
        type_vocab_size <= 0) {
        fail("invalid config");
        return NULL;
    }
    orc_model* m = (orc_model*)calloc(1, sizeof(orc_model));
    m->H = hidden_size;
    m->nh = num_attention_heads;
    m->L = num_hidden_layers;
    m->I = intermediate_size;
    m->V = vocab_size;
    m->P = max_position_embeddings;
    m->TV = type_vocab_size;
    m->eps = layer_norm_eps;
    return m;
}

int orc_set_tensor(orc_model* m, const char* name, const float* data, const int64_t* shape,
                   int ndim) {
    if (!m || !name || !data || !shape || ndim < 1 || ndim > 2) return fail("bad tensor args");
    int64_t n = 1;
    for (int d = 0; d < ndim; ++d) n *= shape[d];
    orc_tensor* t = NULL;
    for (int i = 0; i < m->ntensors; ++i)
        if (strcmp(m->tensors[i].name, name) == 0) t = &m->tensors[i];
    if (!t) {
        if (m->ntensors == m->cap) {
            m->cap = m->cap ? 2 * m->cap : 64;
            m->tensors = (orc_tensor*)realloc(m->tensors, sizeof(orc_tensor) * m->cap);
        }
        t = &m->tensors[m->ntensors++];
        t->name = strdup(name);
        t->data = NULL;
    }
    free(t->data);
    t->data = (float*)malloc(sizeof(float) * (size_t)n);
    memcpy(t->data, data, sizeof(float) * (size_t)n);
    t->ndim = ndim;
    t->shape[0] = shape[0];
    t->shape[1] = ndim == 2 ? shape[1] : 1;
    return 0;
}

static orc_tensor* find(orc_model* m, const char* name) {
    for (int i = 0; i < m->ntensors; ++i)
        if (strcmp(m->tensors[i].name, name) == 0) return &m->tensors[i];
    return NULL;
}

/* weights.get_array1 (src/weights.rs:47-58): must exist and be 1-D. */
static float* get1(orc_model* m, const char* name, int64_t len, int* rc) {
    orc_tensor* t = find(m, name);
    if (!t) { *rc = fail("Tensor %s not found", name); return NULL; }
    if (t->ndim != 1) { *rc = fail("Expected 1D tensor, got %d-D for %s", t->ndim, name); return NULL; }
    if (t->shape[0] != len) { *rc = fail("Tensor %s has %lld elements, expected %lld", name, (long long)t->shape[0], (long long)len); return NULL; }
    return t->data;
}

/* weights.get_array2 (src/weights.rs:60-69), optionally followed by .t().to_owned(). */
static float* get2(orc_model* m, const char* name, int64_t r, int64_t c, int transpose, int* rc) {
    orc_tensor* t = find(m, name);
    if (!t) { *rc = fail("Tensor %s not found", name); return NULL; }
    if (t->ndim != 2 || t->shape[0] != r || t->shape[1] != c) {
        *rc = fail("Shape error: %s is not [%lld, %lld]", name, (long long)r, (long long)c);
        return NULL;
    }
    float* out = (float*)malloc(sizeof(float) * (size_t)r * c);
    if (!transpose) {
        memcpy(out, t->data, sizeof(float) * (size_t)r * c);
    } else {
        for (int64_t i = 0; i < r; ++i)
            for (int64_t j = 0; j < c; ++j) out[j * r + i] = t->data[i * c + j];
    }
    return out;
}

static float* dup1(const float* p, int64_t n) {
    float* o = (float*)malloc(sizeof(float) * (size_t)n);
    memcpy(o, p, sizeof(float) * (size_t)n);
    return o;
}

int orc_model_build(orc_model* m) {
    if (!m) return fail("null model");
    int rc = 0, H = m->H, I = m->I;
    char nm[256];
    m->word = get2(m, "embeddings.word_embeddings.weight", m->V, H, 0, &rc); if (rc) return rc;
    m->pos = get2(m, "embeddings.position_embeddings.weight", m->P, H, 0, &rc); if (rc) return rc;
    m->type = get2(m, "embeddings.token_type_embeddings.weight", m->TV, H, 0, &rc); if (rc) return rc;
    m->layers = (orc_layer*)calloc(m->L > 0 ? m->L : 1, sizeof(orc_layer));
#define G2(field, suffix, r, c)                                                   \
    snprintf(nm, sizeof nm, "encoder.layer.%d.%s", i, suffix);                    \
    ly->field = get2(m, nm, r, c, 1, &rc);                                        \
    if (rc) return rc;
#define G1(field, suffix, n)                                                      \
    snprintf(nm, sizeof nm, "encoder.layer.%d.%s", i, suffix);                    \
    { float* p_ = get1(m, nm, n, &rc); if (rc) return rc; ly->field = dup1(p_, n); }
    for (int i = 0; i < m->L; ++i) {
        orc_layer* ly = &m->layers[i];
        G2(wq_t, "attention.self.query.weight", H, H);
        G1(bq, "attention.self.query.bias", H);
        G2(wk_t, "attention.self.key.weight", H, H);
        G1(bk, "attention.self.key.bias", H);
        G2(wv_t, "attention.self.value.weight", H, H);
        G1(bv, "attention.self.value.bias", H);
        G2(wo_t, "attention.output.dense.weight", H, H);
        G1(bo, "attention.output.dense.bias", H);
        G2(w1_t, "intermediate.dense.weight", I, H);
        G1(b1, "intermediate.dense.bias", I);
        G2(w2_t, "output.dense.weight", H, I);
        G1(b2, "output.dense.bias", H);
        G1(ln1_w, "attention.output.LayerNorm.weight", H);
        G1(ln1_b, "attention.output.LayerNorm.bias", H);
        G1(ln2_w, "output.LayerNorm.weight", H);
        G1(ln2_b, "output.LayerNorm.bias", H);
    }
#undef G1
#undef G2
    { float* p = get1(m, "embeddings.LayerNorm.weight", H, &rc); if (rc) return rc; m->emb_ln_w = dup1(p, H); }
    { float* p = get1(m, "embeddings.LayerNorm.bias", H, &rc); if (rc) return rc; m->emb_ln_b = dup1(p, H); }
    m->built = 1;
    return 0;
}

void orc_model_free(orc_model* m) {
    if (!m) return;
    for (int i = 0; i < m->ntensors; ++i) {
        free(m->tensors[i].name);
        free(m->tensors[i].data);
    }
    free(m->tensors);
    if (m->layers) {
        for (int i = 0; i < m->L; ++i) {
            orc_layer* l = &m->layers[i];
            float* ps[] = {l->wq_t, l->bq, l->wk_t, l->bk, l->wv_t, l->bv, l->wo_t, l->bo,
                           l->ln1_w, l->ln1_b, l->w1_t, l->b1, l->w2_t, l->b2, l->ln2_w, l->ln2_b};
            for (size_t j = 0; j < sizeof ps / sizeof ps[0]; ++j) free(ps[j]);
        }
        free(m->layers);
    }
    free(m->word); free(m->pos); free(m->type); free(m->emb_ln_w); free(m->emb_ln_b);
    free(m);
}

/* ------------------------------------------------------------------------- */
/* Forward                                                                    */
/* ------------------------------------------------------------------------- */
static void add_bias(float* x, int64_t rows, int n, const float* b) {
#pragma omp parallel for schedule(static) if (rows > 64)
    for (int64_t r = 0; r < rows; ++r)
        for (int j = 0; j < n; ++j) x[r * n + j] = x[r * n + j] + b[j];
}

static void add_inplace(float* x, const float* y, int64_t n) {
#pragma omp parallel for schedule(static) if (n > 4096)
    for (int64_t i = 0; i < n; ++i) x[i] = x[i] + y[i];
}

/* [B,S,nh,hd] -> [B,nh,S,hd] copy (into_shape + permuted_axes + as_standard_layout). */
static void to_heads(const float* x, int B, int S, int nh, int hd, float* out) {
#pragma omp parallel for collapse(2) schedule(static) if (B * nh > 8)
    for (int b = 0; b < B; ++b)
        for (int h = 0; h < nh; ++h)
            for (int s = 0; s < S; ++s)
                memcpy(out + (((size_t)b * nh + h) * S + s) * hd,
                       x + ((size_t)b * S + s) * nh * hd + (size_t)h * hd, sizeof(float) * hd);
}

/* [B,S,nh,hd] -> [B,nh,hd,S] copy: the permuted key operand of q.k^T. */
static void to_heads_t(const float* x, int B, int S, int nh, int hd, float* out) {
#pragma omp parallel for collapse(2) schedule(static) if (B * nh > 8)
    for (int b = 0; b < B; ++b)
        for (int h = 0; h < nh; ++h)
            for (int s = 0; s < S; ++s)
                for (int d = 0; d < hd; ++d)
                    out[(((size_t)b * nh + h) * hd + d) * S + s] =
                        x[((size_t)b * S + s) * nh * hd + (size_t)h * hd + d];
}

/* [B,nh,S,hd] -> [B,S,nh*hd] (src/lib.rs:726-730). */
static void from_heads(const float* x, int B, int S, int nh, int hd, float* out) {
#pragma omp parallel for collapse(2) schedule(static) if (B * nh > 8)
    for (int b = 0; b < B; ++b)
        for (int h = 0; h < nh; ++h)
            for (int s = 0; s < S; ++s)
                memcpy(out + ((size_t)b * S + s) * nh * hd + (size_t)h * hd,
                       x + (((size_t)b * nh + h) * S + s) * hd, sizeof(float) * hd);
}

/* MultiHeadAttention::forward (src/lib.rs:685-736). */
static void mha_forward(const orc_model* m, const orc_layer* ly, const float* x, const float* mask,
                        int B, int S, float* out) {
    int H = m->H, nh = m->nh, hd = H / nh;
    size_t T = (size_t)B * S;
    float* q = (float*)malloc(sizeof(float) * T * H);
    float* k = (float*)malloc(sizeof(float) * T * H);
    float* v = (float*)malloc(sizeof(float) * T * H);
    orc_matmul_3d_2d(x, B, S, H, ly->wq_t, H, q);
    add_bias(q, T, H, ly->bq);
    orc_matmul_3d_2d(x, B, S, H, ly->wk_t, H, k);
    add_bias(k, T, H, ly->bk);
    orc_matmul_3d_2d(x, B, S, H, ly->wv_t, H, v);
    add_bias(v, T, H, ly->bv);

    float* q4 = (float*)malloc(sizeof(float) * T * H);
    float* kt4 = (float*)malloc(sizeof(float) * T * H);
    float* v4 = (float*)malloc(sizeof(float) * T * H);
    to_heads(q, B, S, nh, hd, q4);
    to_heads_t(k, B, S, nh, hd, kt4);
    to_heads(v, B, S, nh, hd, v4);
    free(q); free(k); free(v);

    size_t nscores = (size_t)B * nh * S * S;
    float* scores = (float*)malloc(sizeof(float) * (nscores ? nscores : 1));
    orc_matmul_4d(q4, kt4, B, nh, S, hd, S, scores);
    /* scale_factor = 1 / sqrt(head_dim) (src/lib.rs:196-197), applied after q.k^T. */
    const float scale = 1.0f / sqrtf((float)hd);
#pragma omp parallel for schedule(static) if (nscores > 4096)
    for (size_t i = 0; i < nscores; ++i) scores[i] = scores[i] * scale;
    orc_apply_attention_mask(scores, mask, B, nh, S, S);
    orc_softmax(scores, (int64_t)B * nh * S, S);
    float* ctx4 = (float*)malloc(sizeof(float) * T * H);
    orc_matmul_4d(scores, v4, B, nh, S, S, hd, ctx4);
    free(scores); free(q4); free(kt4); free(v4);
    float* ctx = (float*)malloc(sizeof(float) * T * H);
    from_heads(ctx4, B, S, nh, hd, ctx);
    free(ctx4);
    orc_matmul_3d_2d(ctx, B, S, H, ly->wo_t, H, out);
    add_bias(out, T, H, ly->bo);
    free(ctx);
}

/* FeedForward::forward (src/lib.rs:739-750). */
static void ffn_forward(const orc_model* m, const orc_layer* ly, const float* x, int B, int S,
                        float* out) {
    int H = m->H, I = m->I;
    size_t T = (size_t)B * S;
    float* inter = (float*)malloc(sizeof(float) * T * I);
    orc_matmul_3d_2d(x, B, S, H, ly->w1_t, I, inter);
    add_bias(inter, T, I, ly->b1);
    orc_gelu(inter, (int64_t)T * I);
    orc_matmul_3d_2d(inter, B, S, I, ly->w2_t, H, out);
    add_bias(out, T, H, ly->b2);
    free(inter);
}

/* BertLayer::forward (src/lib.rs:669-683): post-LN residual blocks. */
static void layer_forward(const orc_model* m, const orc_layer* ly, float* x, const float* mask,
                          int B, int S, float* tmp) {
    int H = m->H;
    size_t T = (size_t)B * S;
    mha_forward(m, ly, x, mask, B, S, tmp);
    add_inplace(tmp, x, (int64_t)(T * H));
    orc_layer_norm(tmp, (int64_t)T, H, ly->ln1_w, ly->ln1_b, m->eps, x); /* x := attention_out */
    ffn_forward(m, ly, x, B, S, tmp);
    add_inplace(tmp, x, (int64_t)(T * H));
    orc_layer_norm(tmp, (int64_t)T, H, ly->ln2_w, ly->ln2_b, m->eps, x);
}

/* `token_id as usize` on an f32: truncation, NaN and negatives saturate to 0. */
static int64_t as_usize(float f) {
    if (!(f > 0.0f)) return 0;
    if (f >= 9.2e18f) return INT64_MAX;
    return (int64_t)f;
}

int orc_forward_trace(const orc_model* m, const float* input_ids, const float* attention_mask,
                      int B, int S, float* pooled, float* trace) {
    if (!m || !m->built) return fail("model not built");
    if (B < 0 || S < 0) return fail("negative shape");
    if (B == 0) return 0;
    int H = m->H;
    if (S > m->P) return fail("sequence length %d exceeds max_position_embeddings %d", S, m->P);
    size_t T = (size_t)B * S;
    for (size_t t = 0; t < T; ++t) {
        int64_t id = as_usize(input_ids[t]);
        if (id >= m->V) return fail("token id %lld out of range for vocab %d", (long long)id, m->V);
    }
    float* x = (float*)malloc(sizeof(float) * (T ? T : 1) * H);
    float* tmp = (float*)malloc(sizeof(float) * (T ? T : 1) * H);
    /* Embedding gather (src/lib.rs:630-643), + position rows 0..S (655-656),
     * + token-type row 0 (658-659). */
#pragma omp parallel for schedule(static) if (B > 1)
    for (int b = 0; b < B; ++b)
        for (int s = 0; s < S; ++s) {
            size_t t = (size_t)b * S + s;
            const float* w = m->word + (size_t)as_usize(input_ids[t]) * H;
            for (int j = 0; j < H; ++j) tmp[t * H + j] = w[j];
        }
    for (size_t t = 0; t < T; ++t) {
        const float* p = m->pos + (size_t)(t % S) * H;
        for (int j = 0; j < H; ++j) tmp[t * H + j] = tmp[t * H + j] + p[j];
    }
    for (size_t t = 0; t < T; ++t)
        for (int j = 0; j < H; ++j) tmp[t * H + j] = tmp[t * H + j] + m->type[j];
    orc_layer_norm(tmp, (int64_t)T, H, m->emb_ln_w, m->emb_ln_b, m->eps, x);
    if (trace) memcpy(trace, x, sizeof(float) * T * H);
    for (int l = 0; l < m->L; ++l) {
        layer_forward(m, &m->layers[l], x, attention_mask, B, S, tmp);
        if (trace) memcpy(trace + (size_t)(l + 1) * T * H, x, sizeof(float) * T * H);
    }
    orc_mean_pool(x, attention_mask, B, S, H, pooled);
    free(x);
    free(tmp);
    return 0;
}

int orc_forward(const orc_model* m, const float* input_ids, const float* attention_mask, int B,
                int S, float* pooled) {
    return orc_forward_trace(m, input_ids, attention_mask, B, S, pooled, NULL);
}
