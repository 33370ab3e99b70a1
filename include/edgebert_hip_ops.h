/*
 * edgebert_hip_ops.h -- op-level entry points of the gfx950 encoder kernels.
 *
 * Each call enqueues one kernel (family) on `stream` (a hipStream_t; NULL =
 * the null stream) over caller-owned DEVICE buffers and returns without
 * waiting.  They exist so that every kernel can be checked and timed alone
 * against the reference op it replaces; the model-level API in
 * edgebert_hip.h chains the same kernels.  Return codes as in
 * edgebert_hip.h (arguments are validated on the host before any launch).
 */
#ifndef EDGEBERT_HIP_OPS_H
#define EDGEBERT_HIP_OPS_H

#include <stdint.h>

#ifndef EBH_API
#define EBH_API __attribute__((visibility("default")))
#endif

#ifdef __cplusplus
extern "C" {
#endif

#define EBH_EPI_BIAS 0       /* C = A.W^T + b                       */
#define EBH_EPI_BIAS_GELU 1  /* C = gelu_tanh(A.W^T + b)             */
#define EBH_EPI_BIAS_RESID 2 /* C = (A.W^T + b) + R                  */
#define EBH_EPI_NONE 3       /* C = A.W^T (bias may be NULL)         */

/* matmul_3d_2d + bias (+ gelu / + residual) (src/lib.rs:795-849, 691-698,
 * 732-733, 741-747, 673, 678, 958-978), batch folded into M:
 * A [M, K] fp32 (row stride lda), W [N, K] HF layout (row stride ldw), fp32
 * when w_dtype == EBH_DTYPE_F32 or bf16 bits (uint16) when EBH_DTYPE_BF16 (A
 * is then rounded to bf16 on load; accumulation is fp32); w_dtype
 * EBH_DTYPE_F32_BF16X6: fp32 W, products formed as six bf16 MFMA products of
 * three-way bf16 splits of A and W (see edgebert_hip.h).  C [M, N] (ldc);
 * residual [M, N] (ldr) only for EBH_EPI_BIAS_RESID; bias may be NULL for EBH_EPI_NONE.  K and the strides must
 * be multiples of 4 (fp32) / 8 (bf16).  fp32 row strides above 2,796,202
 * elements run on the guarded kernel (64-bit addresses) instead of the
 * persistent ones, whose lane offsets are 32-bit. */
EBH_API int ebh_op_gemm(const float* A, int64_t lda, const void* W, int64_t ldw, int32_t w_dtype,
                const float* bias, const float* residual, int64_t ldr, float* C, int64_t ldc,
                int32_t M, int32_t N, int32_t K, int32_t epilogue, void* stream);

/* The same GEMM with bf16 activations: A [M, K] and W [N, K] bf16 bits, fp32
 * accumulate, C [M, N] fp32 (c_dtype EBH_DTYPE_F32) or bf16 bits
 * (EBH_DTYPE_BF16), epilogue EBH_EPI_BIAS / EBH_EPI_BIAS_GELU / EBH_EPI_NONE.
 * K % 64 == 0, N % 4 == 0, strides of 8 / 8 / 4 elements, 16-byte aligned
 * operands, lda and ldw at most 5,592,405 elements (the kernel's 32-bit lane
 * offsets span 384 rows of a stride; EBH_ERR_INVALID_ARG beyond).  The forward
 * of EBH_DTYPE_BF16 models uses it for every Linear. */
EBH_API int ebh_op_gemm_bf16(const uint16_t* A, int64_t lda, const uint16_t* W, int64_t ldw,
                     const float* bias, void* C, int64_t ldc, int32_t c_dtype, int32_t M, int32_t N,
                     int32_t K, int32_t epilogue, void* stream);

/* Masked multi-head attention (src/lib.rs:700-730 with 851-956) over packed
 * sequences: qkv [T, 3*hidden] rows (q | k | v), sequence b = rows
 * cu_seqlens[b] .. cu_seqlens[b+1]-1 (every row a real token, lengths <=
 * max_len); ctx [T, hidden]; qkv and ctx 16-byte aligned.  head_dim = hidden /
 * num_heads must be 32 or 64;
 * scale is 1/sqrt(head_dim) as the reference computes it (src/lib.rs:196-197). */
EBH_API int ebh_op_attention(const float* qkv, const int32_t* cu_seqlens, int32_t B, int32_t max_len,
                     int32_t hidden, int32_t num_heads, float* ctx, void* stream);

/* The same attention for bf16 models: qkv [T, 3*hidden] and ctx [T, hidden]
 * hold bf16 bit patterns (qkv 16-byte, ctx 8-byte aligned); q.k^T, softmax and the P.V
 * sums accumulate in fp32 (bf16 counterpart of the reference's fp32
 * attention, src/lib.rs:700-730). */
EBH_API int ebh_op_attention_bf16(const uint16_t* qkv, const int32_t* cu_seqlens, int32_t B,
                          int32_t max_len, int32_t hidden, int32_t num_heads, uint16_t* ctx,
                          void* stream);

/* apply_layer_norm_3d (src/lib.rs:980-991) over rows x [rows, H] -> y (may alias). */
EBH_API int ebh_op_layer_norm(const float* x, const float* gamma, const float* beta, int32_t rows,
                      int32_t H, float eps, float* y, void* stream);

/* End of a residual block (src/lib.rs:672-674, 677-679): x = LayerNorm((y + bias)
 * + x) over rows [rows, H], in place on x; y is a projection written without its
 * bias (EBH_EPI_NONE).  The additions follow the reference's order. */
EBH_API int ebh_op_add_layer_norm(const float* y, const float* bias, float* x, const float* gamma,
                          const float* beta, int32_t rows, int32_t H, float eps, void* stream);

/* A residual block's projection and end in one kernel (src/lib.rs:672-674,
 * 677-679 with the Linear of 732-733 / 741-747): x = LayerNorm((A.W^T + bias)
 * + x), in place on x [M, N] (row stride N), A [M, K] fp32 (lda), W [N, K] fp32
 * (ldw).  Each 128-row block is one workgroup that holds whole rows, so N must
 * be 384 (the MiniLM width); K % 32 == 0, strides multiples of 4 and at
 * most 2,796,202 elements (32-bit lane offsets over 384 rows;
 * EBH_ERR_INVALID_ARG beyond), A, W and bias 16-byte aligned.  Same result, within fp32 rounding, as ebh_op_gemm
 * (EBH_EPI_NONE) followed by ebh_op_add_layer_norm; the fp32 forward uses it
 * when there are at least as many 128-row blocks as CUs. */
EBH_API int ebh_op_gemm_add_layer_norm(const float* A, int64_t lda, const float* W, int64_t ldw,
                               const float* bias, float* x, const float* gamma, const float* beta,
                               int32_t M, int32_t N, int32_t K, float eps, void* stream);

/* The same with y stored as bf16 (the projections of bf16 models); the sums,
 * statistics and x stay fp32.  y rows 8-byte aligned, the fp32 operands
 * 16-byte aligned, and H = 4 * L * n with L in {64, 32, 16}, n in
 * {1, 2, 3, 4, 6, 8} (384, 768, 1024, ...). */
EBH_API int ebh_op_add_layer_norm_y16(const uint16_t* y, const float* bias, float* x, const float* gamma,
                              const float* beta, int32_t rows, int32_t H, float eps, void* stream);

/* The same block end over a bf16 residual stream (bf16 models): x16 =
 * bf16(LayerNorm((y + bias) + x16)), in place on x16 [rows, H] (bf16 bits);
 * the sums and statistics are fp32 (src/lib.rs:672-674, 677-679, 980-991).
 * x16 and y rows 8-byte aligned; H as for ebh_op_add_layer_norm_y16. */
EBH_API int ebh_op_add_layer_norm_b16(const uint16_t* y, const float* bias, uint16_t* x16, const float* gamma,
                              const float* beta, int32_t rows, int32_t H, float eps, void* stream);

/* mean_pool (src/lib.rs:993-1010) over packed sequences (+ the normalise tail,
 * src/lib.rs:605-612, when normalize != 0); S is the padded length the caller
 * had (S > 0 and an empty sequence gives NaN, as in the reference).  With
 * H % 4 == 0, H <= 768, x and out 16-byte aligned, S > 32 and fewer
 * sequences than the device has CUs, each sequence's 32-row chunks are summed
 * by workgroups of their own into `partials`: B * ceil(S / 32) * H floats,
 * 16-byte aligned (otherwise unused, and may be null). */
EBH_API int ebh_op_pool(const float* x, const int32_t* cu_seqlens, int32_t B, int32_t H, int32_t S,
                int32_t normalize, float* partials, float* out, void* stream);
/* The same over a bf16 residual stream x16 [T, H] (bf16 bits, 8-byte aligned,
 * H % 4 == 0); sums in fp32. */
EBH_API int ebh_op_pool_b16(const uint16_t* x16, const int32_t* cu_seqlens, int32_t B, int32_t H, int32_t S,
                    int32_t normalize, float* out, void* stream);

/* Token packing: ids / mask [B, S] -> cu_seqlens [B+1], n_tokens [1],
 * tok_id / tok_pos [B*S]; counts [B] is scratch; err [1] is cleared (the
 * forward itself never clears its flag: see ebh_synchronize). */
EBH_API int ebh_op_pack(const int32_t* ids, const int32_t* mask, int32_t B, int32_t S,
                int32_t* counts, int32_t* cu_seqlens, int32_t* n_tokens, int32_t* tok_id,
                int32_t* tok_pos, int32_t* err, void* stream);

/* Embedding rows word[tok_id] + pos[tok_pos] + type0, then LayerNorm
 * (src/lib.rs:628-661), for the first *n_tokens (device) of T_max tokens;
 * ids outside [0, V) read row 0 and set *err |= 1. */
EBH_API int ebh_op_embed_ln(const int32_t* tok_id, const int32_t* tok_pos, const int32_t* n_tokens,
                    int32_t T_max, const float* word, const float* pos, const float* type0,
                    const float* gamma, const float* beta, int32_t V, int32_t H, float eps,
                    float* x, int32_t* err, void* stream);

/* fp32 -> bf16 bits, round to nearest even (weight conversion). */
EBH_API int ebh_op_f32_to_bf16(const float* x, uint16_t* y, int64_t n, void* stream);

/* The device conversion of 16-bit checkpoint tensors (ebh_load_safetensors +
 * ebh_finalize): mode 0 F16 bits -> f32, 1 BF16 bits -> f32 (both exact,
 * y float[n]), 2 F16 bits -> bf16 bits rounded to nearest even (y uint16[n]). */
EBH_API int ebh_op_widen16(const uint16_t* x, void* y, int64_t n, int32_t mode, void* stream);

/* The tanh-form GELU as fused into the FFN-up epilogues, elementwise:
 * y[i] = gelu(x[i]) with the epilogue's exp2 + reciprocal evaluation. */
EBH_API int ebh_op_gelu(const float* x, float* y, int64_t n, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* EDGEBERT_HIP_OPS_H */
