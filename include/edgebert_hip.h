/*
 * edgebert_hip.h -- C ABI of the MI355X (gfx950) BERT encoder forward.
 *
 * Drop-in for the body of EdgeBERT's `Model::forward` plus the normalisation
 * tail of `encode_uncached` (/root/reference/src/lib.rs:588-666).  The host
 * tokenizer and the public `encode` / cache logic stay with the caller; a Rust
 * `hip` backend binds these symbols with `extern "C"`, one declaration per
 * function below with the same parameter types in the same order.
 *
 * Conventions
 *  - Every function returns EBH_OK (0) on success or a negative EBH_ERR_*
 *    code; the message of the calling thread's last failure is returned by
 *    ebh_last_error() (thread-local, valid until the next failing call).
 *  - The caller owns every host buffer; the library owns the device weights
 *    and a workspace that grows on demand.  Calls on one model are
 *    serialised internally, so a model may be shared by many host threads
 *    (as `encode(&self)` is under rayon, src/lib.rs:440-451).
 *  - Linear weights are given in the HF [out, in] layout, exactly as stored
 *    in model.safetensors; the library re-lays them out for the GPU.
 */
#ifndef EDGEBERT_HIP_H
#define EDGEBERT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifndef EBH_API
#define EBH_API __attribute__((visibility("default")))
#endif

#ifdef __cplusplus
extern "C" {
#endif

#define EBH_OK 0
#define EBH_ERR_INVALID_ARG (-1) /* null pointer, negative size, bad config     */
#define EBH_ERR_NOT_FOUND (-2)   /* unknown / missing tensor name               */
#define EBH_ERR_SHAPE (-3)       /* tensor rank or shape does not match config  */
#define EBH_ERR_STATE (-4)       /* e.g. forward before finalize                */
#define EBH_ERR_HIP (-5)         /* HIP runtime failure                         */
#define EBH_ERR_RANGE (-6)       /* token id >= vocab, S > max positions, ...   */

#define EBH_DTYPE_F32 0  /* fp32 GEMMs (parity path)                          */
#define EBH_DTYPE_BF16 1 /* bf16 GEMM inputs, fp32 accumulate; LN/softmax fp32 */
/* fp32 model (fp32 weights and activations, everything else as EBH_DTYPE_F32)
 * whose GEMMs form each fp32 product from bf16 MFMA products: both operands
 * are split in registers into three bf16 parts (h + m + l, round to nearest
 * even) and a.b = ah.bh + ah.bm + am.bh + ah.bl + am.bm + al.bh, each product
 * exact in fp32, accumulated in fp32; the terms left out are below 2^-27 of
 * |a.b|.  Measured against fp64 its GEMM errors are no larger than the fp32
 * MFMA path's; its large GEMMs run faster (bf16 matrix rate is 16x fp32's).
 * Products of at most 64 rows keep the fp32 kernels.  Not in the reference:
 * an opt-in for callers that want the fp32 path's accuracy at more speed. */
#define EBH_DTYPE_F32_BF16X6 2

typedef struct ebh_model ebh_model;

/* Mirrors the reference `Config` (src/lib.rs:95-106).  hidden_act is not a
 * field: the reference ignores it and always applies the tanh GELU
 * (src/lib.rs:958-978). type_vocab_size is the row count of
 * embeddings.token_type_embeddings.weight (the reference reads it from the
 * tensor shape). */
typedef struct ebh_config {
    int32_t hidden_size;
    int32_t num_attention_heads;
    int32_t num_hidden_layers;
    int32_t intermediate_size;
    int32_t vocab_size;
    int32_t max_position_embeddings;
    int32_t type_vocab_size;
    float layer_norm_eps;
} ebh_config;

/* Message of this thread's most recent failure ("" if none). */
EBH_API const char* ebh_last_error(void);

/* Model::from_weights, step 1 (src/lib.rs:155-159): validate the config and
 * create an empty model (no HIP call is made before ebh_finalize).
 * hidden_size must be a multiple of num_attention_heads with head_dim 32 or
 * 64, hidden_size <= 2048, and hidden_size / intermediate_size multiples of 8. */
EBH_API int ebh_create(const ebh_config* cfg, ebh_model** out);

/* ModelWeights::get_array1/2 + from_weights field mapping
 * (src/weights.rs:47-69, src/lib.rs:161-238): hand over one tensor by its HF
 * name.  Data is copied; shape must match the config.  Unknown names fail
 * with EBH_ERR_NOT_FOUND, a wrong rank/shape with EBH_ERR_SHAPE
 * ("Expected 1D tensor ..." as in src/weights.rs:53-57).  The optional
 * cross-encoder head (src/lib.rs:385-399) is "classifier.weight", [H] or
 * [1, H], and "classifier.bias" with exactly one value ("Expected scalar"
 * otherwise, src/weights.rs:99-111). */
EBH_API int ebh_set_tensor(ebh_model* m, const char* name, const float* data, const int64_t* shape,
                   int32_t ndim);

/* Load every tensor from a model.safetensors file (src/weights.rs:15-45).
 * F32, F16 and BF16 tensors are taken in their own encoding: the file is
 * mapped, and ebh_finalize uploads each tensor straight from the mapping
 * (F32 into fp32 slots; BF16 GEMM weights straight into a bf16 model's
 * weights; anything else converted on the device: F16 / BF16 -> fp32 exactly,
 * F16 / F32 -> bf16 rounded to nearest even).  The file must stay unchanged
 * until ebh_finalize or ebh_destroy releases the mapping: a file truncated
 * in place meanwhile makes the upload's reads raise SIGBUS.  A
 * classifier.weight / classifier.bias pair is loaded as the cross-encoder
 * head; other tensors the encoder does not use (pooler.*) are skipped. */
EBH_API int ebh_load_safetensors(ebh_model* m, const char* path);

/* End of from_weights: check that every tensor is present (missing ->
 * EBH_ERR_NOT_FOUND "Tensor <name> not found"), bind the model to the
 * current HIP device, upload all weights once into
 * one device-resident HBM block (QKV concatenated to [3H, H]).  With
 * EBH_DTYPE_BF16 the four GEMM weights of each layer are held as bf16 only
 * (round to nearest even from F32 / F16, as-is from BF16). */
EBH_API int ebh_finalize(ebh_model* m, int32_t dtype);

EBH_API void ebh_destroy(ebh_model* m);

/* Model::forward (src/lib.rs:621-666) on host buffers:
 * input_ids / attention_mask are the reference's f32 [B, S] row-major arrays
 * (src/lib.rs:588-601); out is [B, hidden_size] mean-pooled, NOT normalised.
 * ids are converted like `token_id as usize` (truncation, negatives -> 0) and
 * must be < vocab_size (the reference panics otherwise: EBH_ERR_RANGE); mask
 * values must be 0 or 1.  S must be <= max_position_embeddings.  B == 0 is a
 * no-op; S == 0 yields zero rows; an all-zero mask row yields NaN, as the
 * reference's -inf softmax does.  Blocking. */
EBH_API int ebh_forward(ebh_model* m, const float* input_ids, const float* attention_mask, int32_t B,
                int32_t S, float* out);

/* encode_uncached after tokenisation (src/lib.rs:573-619): u32 ids and mask
 * from the tokenizer's encodings, zero-padded to [B, S]; out [B, hidden_size]
 * L2-normalised (x / max(||x||, 1e-12)) when normalize != 0.  Blocking. */
EBH_API int ebh_encode(ebh_model* m, const uint32_t* ids, const uint32_t* mask, int32_t B, int32_t S,
               int32_t normalize, float* out);

/* Device-pointer variant of ebh_encode for callers that keep ids / mask /
 * output in HBM: int32 ids and 0/1 mask [B, S], out [B, hidden_size], all
 * device pointers; enqueued on `stream` (a hipStream_t, NULL = the model's own
 * stream) and returns without waiting.  Ids are range-checked on the device:
 * an id >= vocab_size reads row 0 and is reported by the next
 * ebh_synchronize(), however many forwards follow it.  Successive calls are
 * ordered even across streams (S == 0 included: zero rows, written by a
 * kernel).  No call enqueues a memset, so `stream` may be under capture. */
EBH_API int ebh_encode_device(ebh_model* m, const int32_t* ids, const int32_t* mask, int32_t B,
                      int32_t S, int32_t normalize, float* out, void* stream);

/* No counterpart in the reference: ebh_encode_device for callers that cannot
 * allocate device memory (tight serving loops, harnesses that forbid
 * hipMalloc, code that must not allocate once running).  Same arguments,
 * results and ordering as
 * ebh_encode_device, but the forward's workspace is a static device array of
 * EBH_NOALLOC_SCRATCH_BYTES per device (held from the library's load until the
 * process ends), so the call makes no hipMalloc / hipFree and records no
 * graph.  A batch whose workspace does not fit fails with EBH_ERR_RANGE
 * before anything is enqueued (128 MiB: MiniLM-L6 about 7k tokens in fp32,
 * 9k in bf16, e.g. 56 x 128; BERT-base about 3.5k in fp32, 4.4k in bf16).
 * Every call on one device shares that array: calls that overlap on a device
 * (other models, other streams, other threads) race; calls on one model are
 * ordered as ebh_encode_device's are.  A bad id raises the calling model's
 * own id-range flag (a word ebh_finalize reserves in the model's weight
 * block), which that model's ebh_synchronize reports and clears; other
 * models never see it.  ebh_last_tokens does not cover these forwards. */
#define EBH_NOALLOC_SCRATCH_BYTES (128u << 20)
EBH_API int ebh_encode_device_noalloc(ebh_model* m, const int32_t* ids, const int32_t* mask, int32_t B,
                                      int32_t S, int32_t normalize, float* out, void* stream);

/* Cross-encoder scoring (Model::score_pair / score_batch, src/lib.rs:327-383):
 * each row of ids / mask [B, S] (u32, zero-padded, as ebh_encode) is one
 * tokenised "query [SEP] document" pair; scores[b] = mean_pool(forward)[b] .
 * classifier.weight + classifier.bias, without normalisation.  All pairs run
 * as one batch; a pair's score does not depend on the others (pads are masked
 * keys and every other step is per token).  Needs a model loaded with
 * classifier.weight / classifier.bias (else EBH_ERR_STATE "Model is not a
 * cross-encoder").  Blocking. */
EBH_API int ebh_score(ebh_model* m, const uint32_t* ids, const uint32_t* mask, int32_t B, int32_t S,
              float* scores);

/* Device-pointer variant of ebh_score: int32 ids / 0-1 mask [B, S] and
 * scores [B] in HBM, enqueued on `stream` (NULL = the model's own stream);
 * returns without waiting, as ebh_encode_device. */
EBH_API int ebh_score_device(ebh_model* m, const int32_t* ids, const int32_t* mask, int32_t B, int32_t S,
                     float* scores, void* stream);

/* ---------------------------------------------------------------------------
 * Host tokenizer.  Tokenizer::from_file("tokenizer.json") with the reference's
 * overrides (padding strategy BatchLongest; truncation, when the file has it,
 * at max_length 512: src/lib.rs:310-322) and encode_batch(texts, true)
 * (src/lib.rs:577-601), for the BERT tokenizer.json files of the models this
 * library runs: normalizer BertNormalizer (or none), pre_tokenizer
 * BertPreTokenizer, model WordPiece, post_processor TemplateProcessing /
 * BertProcessing (or none), added tokens with normalized = false and
 * single_word = false.  Other files are rejected with EBH_ERR_SHAPE and a
 * message naming the unsupported part.  Texts are UTF-8 of lens[i] bytes
 * (lens == NULL: NUL-terminated; with lengths a text may hold NUL, which
 * clean_text drops, as Rust strings may); an invalid byte reads as U+FFFD,
 * which clean_text drops too.  A tokenizer is
 * immutable after loading and may be shared by any number of threads.
 * nthreads: host threads to encode on (<= 0: up to 16, one per hardware
 * thread).
 * ------------------------------------------------------------------------- */
typedef struct ebh_tokenizer ebh_tokenizer;
EBH_API int ebh_tokenizer_load(const char* tokenizer_json_path, ebh_tokenizer** out);
EBH_API int ebh_tokenizer_from_json(const char* json, size_t len, ebh_tokenizer** out);
EBH_API void ebh_tokenizer_destroy(ebh_tokenizer* t);

/* encode_batch of n texts, padded to the batch's longest encoding S (rounded
 * up to the file's pad_to_multiple_of): ids and 0/1 mask written as [n, S]
 * row-major into buffers of at least n * cap elements; *S_out = S.
 * EBH_ERR_RANGE if S > cap (nothing written). */
EBH_API int ebh_tokenize(const ebh_tokenizer* t, const char* const* texts, const int64_t* lens, int32_t n,
                 int32_t cap, int32_t* ids, int32_t* mask, int32_t* S_out, int32_t nthreads);

/* Model::encode(texts, normalize) without the reference's LRU cache
 * (encode_uncached, src/lib.rs:573-619): tokenise on the host threads
 * straight into the model's pinned staging buffers, then the forward; out
 * [n, hidden_size].  Blocking. */
EBH_API int ebh_encode_texts(ebh_model* m, const ebh_tokenizer* t, const char* const* texts,
                     const int64_t* lens, int32_t n, int32_t normalize, float* out, int32_t nthreads);

/* Model::score_batch (src/lib.rs:327-383): pair i is encoded as the single
 * text "queries[i] [SEP] documents[i]", as score_pair formats it; scores [n]
 * as ebh_score.  q_lens / d_lens as lens above.  Blocking. */
EBH_API int ebh_score_texts(ebh_model* m, const ebh_tokenizer* t, const char* const* queries,
                    const int64_t* q_lens, const char* const* documents, const int64_t* d_lens,
                    int32_t n, float* scores, int32_t nthreads);

/* Graph replay (no counterpart in the reference, whose forward runs on the
 * CPU; for serving loops and small batches, whose forward is mostly launch
 * overhead).  When on (the default), the second forward with the same batch
 * shape, normalize flag and buffers (ebh_encode / ebh_forward / ebh_score /
 * the text entry points: the model's own staging; the _device entry points:
 * the caller's pointers) is recorded as a HIP graph, and every later one
 * replays it: the same kernels with the same arguments, so results are
 * bit-identical to direct launches.  Up to 16 recordings per model, least
 * recently used dropped first; all are dropped when the model's buffers grow.
 * Forwards run directly while a kernel is being profiled or while the
 * caller's stream is itself being captured.  enable = 0 turns replay off and
 * frees the recordings. */
EBH_API int ebh_set_graph_replay(ebh_model* m, int32_t enable);

/* Wait for the model's outstanding work; EBH_ERR_RANGE if a device-side id
 * check of any _device forward failed since the previous ebh_synchronize.
 * The flag is sticky: later clean forwards do not clear it, only this call
 * does (blocking calls check their ids on the host and leave it alone). */
EBH_API int ebh_synchronize(ebh_model* m);

/* The packed token stream the last forward consumed: n_tokens (mask == 1
 * tokens) ids and original positions, and cu_seqlens [B+1].  Any output
 * pointer may be NULL; capacities are in elements.  Used to check that the
 * ids reaching the GPU are bit-identical to the caller's.  Blocking. */
EBH_API int ebh_last_tokens(ebh_model* m, int32_t* tok_ids, int32_t* tok_pos, int64_t tok_capacity,
                    int32_t* cu_seqlens, int64_t cu_capacity, int32_t* n_tokens);

/* Hidden size / dtype of a finalized model (for bindings that size outputs). */
EBH_API int ebh_model_info(const ebh_model* m, ebh_config* cfg_out, int32_t* dtype_out);

/* Time one kernel family with HIP events during forwards, on the stream the
 * kernels are launched on.  kernel: one of EBH_PROF_* (EBH_PROF_NONE = off).
 * ebh_profile_read returns the accumulated launch count and total ms since the
 * last ebh_profile_enable, after waiting for the model's work. */
#define EBH_PROF_NONE 0
#define EBH_PROF_GEMM_QKV 1
#define EBH_PROF_ATTENTION 2
#define EBH_PROF_GEMM_OUT 3
#define EBH_PROF_GEMM_FFN_UP 4
#define EBH_PROF_GEMM_FFN_DOWN 5
#define EBH_PROF_LAYERNORM 6
#define EBH_PROF_EMBED 7
#define EBH_PROF_POOL 8
EBH_API int ebh_profile_enable(ebh_model* m, int32_t kernel);
EBH_API int ebh_profile_read(ebh_model* m, int64_t* launches, double* total_ms);

#ifdef __cplusplus
}
#endif
#endif /* EDGEBERT_HIP_H */
