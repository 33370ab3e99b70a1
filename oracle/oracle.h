/*
 * oracle.h -- CPU restatement of EdgeBERT's encoder forward (TEST INFRASTRUCTURE).
 *
 * This library is the checker for the HIP path, never part of it: only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.
 * It restates /root/reference/src/lib.rs op by op in fp32:
 *
 *   orc_forward          Model::forward             src/lib.rs:621-666
 *   orc_layer_forward    BertLayer::forward         src/lib.rs:669-683
 *   orc_mha_forward      MultiHeadAttention::forward src/lib.rs:685-736
 *   orc_ffn_forward      FeedForward::forward       src/lib.rs:739-750
 *   orc_matmul_3d_2d     matmul_3d_2d               src/lib.rs:795-849
 *   orc_softmax          softmax                    src/lib.rs:851-870
 *   orc_apply_attention_mask apply_attention_mask   src/lib.rs:872-896
 *   orc_matmul_4d        matmul_4d                  src/lib.rs:898-956
 *   orc_gelu             gelu (tanh form)           src/lib.rs:958-978, consts 151-152
 *   orc_layer_norm       apply_layer_norm_3d        src/lib.rs:980-991
 *   orc_mean_pool        mean_pool                  src/lib.rs:993-1010
 *   orc_normalize        encode_uncached tail       src/lib.rs:605-612
 *   orc_dot              score_pair head .dot       src/lib.rs:373 (ndarray unrolled_dot)
 *   orc_model_build      Model::from_weights        src/lib.rs:155-260
 *
 * Linear weights are handed over in HF [out,in] layout and transposed at
 * build time, as from_weights does (`.t().to_owned()`, src/lib.rs:172-210).
 * Errors: functions return 0 on success and -1 on failure with a message
 * available from orc_last_error().
 */
#ifndef EDGEBERT_ORACLE_H
#define EDGEBERT_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct orc_model orc_model;

const char* orc_last_error(void);
void orc_set_num_threads(int n);
int orc_get_num_threads(void);

/* The reference's `openblas` feature (Cargo.toml:14): every `.dot` goes to
 * cblas_sgemm.  fn has the ILP64 CBLAS signature; NULL restores the built-in
 * sgemm (the default feature set, matrixmultiply). */
typedef void (*orc_cblas_sgemm_fn)(int order, int trans_a, int trans_b, int64_t m, int64_t n,
                                   int64_t k, float alpha, const float* a, int64_t lda,
                                   const float* b, int64_t ldb, float beta, float* c,
                                   int64_t ldc);
void orc_set_blas_sgemm(orc_cblas_sgemm_fn fn);

orc_model* orc_model_new(int hidden_size, int num_attention_heads, int num_hidden_layers,
                         int intermediate_size, int vocab_size, int max_position_embeddings,
                         int type_vocab_size, float layer_norm_eps);
int orc_set_tensor(orc_model* m, const char* name, const float* data, const int64_t* shape,
                   int ndim);
int orc_model_build(orc_model* m);
void orc_model_free(orc_model* m);

/* ids / mask: the reference's f32 Array2 [B,S]; pooled: [B,H] (not normalised). */
int orc_forward(const orc_model* m, const float* input_ids, const float* attention_mask, int B,
                int S, float* pooled);
/* Same, also writing the hidden state after the embedding LayerNorm and after
 * every layer into trace[(L+1), B, S, H] when trace != NULL. */
int orc_forward_trace(const orc_model* m, const float* input_ids, const float* attention_mask,
                      int B, int S, float* pooled, float* trace);

/* Individual ops (shapes as in the reference). */
void orc_sgemm(int m, int n, int k, const float* a, int lda, const float* b, int ldb, float* c,
               int ldc);
void orc_matmul_3d_2d(const float* a, int batch, int m, int k, const float* b, int n, float* c);
void orc_matmul_4d(const float* a, const float* b, int batch, int heads, int seq1, int dim,
                   int seq2, float* c);
void orc_softmax(float* x, int64_t rows, int n);
void orc_apply_attention_mask(float* scores, const float* mask, int B, int nh, int S1, int S2);
void orc_gelu(float* x, int64_t n);
void orc_layer_norm(const float* x, int64_t rows, int H, const float* weight, const float* bias,
                    float eps, float* y);
void orc_mean_pool(const float* hidden, const float* mask, int B, int S, int H, float* out);
void orc_normalize(float* x, int B, int H);
float orc_cosine_similarity(const float* a, const float* b, int n);
float orc_dot(const float* a, const float* b, int n);

#ifdef __cplusplus
}
#endif
#endif
