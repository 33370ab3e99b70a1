// kernels.hpp -- device helpers and kernel launchers of the gfx950 encoder path.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ebh {

// GEMM epilogues: bias, then optionally GELU (FFN up) or a residual add; or
// none at all (the forward adds bias and residual of the attention-output and
// FFN-down projections in the LayerNorm that follows them); or bias, residual
// and that LayerNorm in one (EPI_ADD_LN, launch_gemm_f32_add_ln).
enum Epilogue : int { EPI_BIAS = 0, EPI_BIAS_GELU = 1, EPI_BIAS_RESID = 2, EPI_NONE = 3, EPI_ADD_LN = 4 };

struct GemmArgs {
    const void* A;       // [M, K] row-major activations (fp32)
    const void* W;       // [N, K] row-major weights (fp32 or bf16)
    const float* bias;   // [N]
    const float* R;      // [M, N] residual (EPI_BIAS_RESID) or nullptr
    float* C;            // [M, N]
    int64_t lda, ldw, ldr, ldc;
    int M_max;           // grid is sized for this many rows
    const int* M_dev;    // actual rows, read on device (nullptr: M_max)
    int N, K;
    // Split-K (EPI_NONE only): split s of `splits` (0 or 1: no split) sums k in
    // [s*K/splits, (s+1)*K/splits) into C + s * split_stride.
    int splits;
    int64_t split_stride;
    // EPI_ADD_LN: LayerNorm gamma / beta [N] and epsilon.
    const float* ln_g;
    const float* ln_b;
    float ln_eps;
    // fp32 products as six bf16 MFMA products (the persistent kernels; other
    // paths ignore it): each fp32 operand is split in registers into three
    // bf16 parts h + m + l (round to nearest even at each step), and
    // a.b = ah.bh + ah.bm + am.bh + ah.bl + am.bm + al.bh, every product
    // exact in fp32, accumulated in fp32 (the dropped terms are below 2^-27
    // of |a.b|).
    int split6;
};

// The persistent GEMM kernels address each k-tile load as a per-tile base
// plus a 32-bit lane offset, (row within the tile) * stride * element size
// plus the k-chunk.  Their tiles span at most GEMM_TILE_ROWS_MAX rows of A or
// W, so row strides (lda, ldw, in elements of es bytes) must keep that offset
// below 2^32; launch_gemm_f32 sends larger strides to the guarded kernel
// (64-bit addresses), the other persistent launchers reject them.
constexpr int GEMM_TILE_ROWS_MAX = 384;
// Largest row stride (elements of es bytes) the persistent kernels take:
// GEMM_TILE_ROWS_MAX * stride * es + (one k-tile of at most 64 elements) * es
// stays below 2^32.
inline int64_t gemm_stride_max(int es) {
    return ((int64_t(1) << 32) - 1 - 64 * es) / (GEMM_TILE_ROWS_MAX * es);
}
inline bool gemm_offsets_fit32(int64_t lda, int64_t ldw, int es) {
    const int64_t ld = lda > ldw ? lda : ldw;
    return ld >= 0 && ld <= gemm_stride_max(es);
}

// The few-token GEMM path: M_max <= SKINNY_MAX_ROWS rows in 16-row blocks,
// N % 32 == 0, K % 64 == 0, 16-byte aligned rows and operands.
constexpr int SKINNY_MAX_ROWS = 64;
bool gemm_f32_skinny_fits(int M_max, int N, int K);

// Compute units of the current device (queried once).
int device_cu_count();

// Split count launch_gemm_f32 takes best for a bias-free product of this shape
// (1 unless there are too few tiles to fill the chip); the caller provides
// `splits` partial outputs.
int gemm_f32_splits(int M_max, int N, int K);

// C = epi(A . W^T + bias); W fp32 (gemm_f32) or bf16 (gemm_bf16, A rounded to bf16).
hipError_t launch_gemm_f32(const GemmArgs& a, int epi, hipStream_t s);
hipError_t launch_gemm_bf16(const GemmArgs& a, int epi, hipStream_t s);

// Masked multi-head attention over packed sequences: qkv [T, 3H] rows
// (q | k | v), cu_seqlens [B+1]; ctx [T, H].  head_dim 32 or 64.  order
// (nullable): a permutation of the B sequences, the order in which the grid
// takes them (launch_pack writes one by decreasing length).
hipError_t launch_attention(const float* qkv, const int* cu_seqlens, int B, int max_len,
                            int H, int nh, int head_dim, float scale, float* ctx, hipStream_t s,
                            const int* order = nullptr);

// Attention with bf16 q / k / v (qkv [T, 3H] bf16 bits) and bf16 context;
// scores, softmax and accumulation in fp32.  head_dim 32 or 64.
hipError_t launch_attention_bf16(const uint16_t* qkv, const int* cu_seqlens, int B, int max_len,
                                 int H, int nh, int head_dim, float scale, uint16_t* ctx,
                                 hipStream_t s, const int* order = nullptr);

// C = LayerNorm((A . W^T + bias) + R) per row (fp32), C may alias R (each
// element is read and written by the same lane).  One workgroup owns whole rows
// (128 x 384 tiles), so it takes N == 384; gemm_f32_add_ln_fits tells whether
// this fused form is the faster one for the shape (enough rows to give every CU
// a tile).  hipErrorInvalidValue for shapes or alignments it does not take.
bool gemm_f32_add_ln_fits(int M_max, int N, int K);
hipError_t launch_gemm_f32_add_ln(const GemmArgs& a, hipStream_t s);

// bf16 activations and weights, fp32 accumulate: C = epi(A . W^T + bias), A [M,K]
// and W [N,K] bf16 bits, C fp32 or (c_bf16) bf16 bits.  Needs 16-byte aligned
// operands and rows, N % 4 == 0 and K % 64 == 0 (hipErrorInvalidValue otherwise).
hipError_t launch_gemm_bf16_act(const GemmArgs& a, int epi, bool c_bf16, hipStream_t s);

// Row LayerNorm (population variance), y may alias x.
hipError_t launch_layernorm(const float* x, float* y, const float* g, const float* b,
                            int rows_max, const int* rows_dev, int H, float eps, hipStream_t s);

// x = LayerNorm((y + bias) + x) per row, in place on x.  y may come as
// nparts split-K partial products part_stride floats apart; they are summed in
// order (((p0 + p1) + p2) + ...) before the bias.
// x16 (optional): bf16 copy of the result (the input of bf16 GEMMs).
hipError_t launch_add_layernorm(const float* y, const float* bias, float* x, const float* g,
                                const float* b, int rows_max, const int* rows_dev, int H, float eps,
                                uint16_t* x16, hipStream_t s, int nparts = 1,
                                int64_t part_stride = 0);
// The same with y stored as bf16 (bf16 models).  x == nullptr: the residual
// stream is bf16 instead, x16 = bf16(LayerNorm((y + bias) + x16)) in place
// (sums and statistics fp32).  Needs 8-byte aligned bf16 rows, 16-byte aligned
// fp32 operands and row4_shape_ok(H).
// H = 4 * L * n with L lanes per row in {64, 32, 16} and n float4 per lane in
// {1, 2, 3, 4, 6, 8}: the shapes the float4 row kernels take.
bool row4_shape_ok(int H);
hipError_t launch_add_layernorm_y16(const uint16_t* y, const float* bias, float* x, const float* g,
                                    const float* b, int rows_max, const int* rows_dev, int H, float eps,
                                    uint16_t* x16, hipStream_t s);

// Token packing: mask [B,S] -> cu_seqlens [B+1], n_tokens, packed ids/positions;
// with `order` (B ints), also the sequences by decreasing length.
hipError_t launch_pack(const int* ids, const int* mask, int B, int S, int* counts, int* cu,
                       int* n_tokens, int* tok_id, int* tok_pos, hipStream_t s, int* order = nullptr);

// n 32-bit words at p set to zero (a kernel launch, never a memset node).
hipError_t launch_zero_words(void* p, int64_t n, hipStream_t s);

// Packing and embeddings in one launch for B*S <= 64 positions (the float4 row
// shapes): the same outputs as launch_pack followed by launch_embed_ln.
bool pack_embed_few_fits(int B, int S, int H);
hipError_t launch_pack_embed_few(const int* ids, const int* mask, int B, int S, int* cu, int* n_tokens,
                                 int* tok_id, int* tok_pos, int* err, const float* word, const float* pos,
                                 const float* type0, const float* g, const float* b, int V, int H, float eps,
                                 float* x, uint16_t* x16, hipStream_t s);

// Attention + the attention-output projection at a handful of tokens (fp32,
// few.hip): at most FEW_ATTN_MAX_TOKENS rows (T_max, the rows the workspace is
// sized for; the packed count is read from ntok), H = 384 in heads of 32.
// Takes the QKV projection (with its bias, [T, 3H]) and writes nh partial
// attention-output products (each head's context times its 32 columns of Wo;
// no bias) at Y + h * part_stride; launch_add_layernorm with nh parts
// finishes the block.
constexpr int FEW_ATTN_MAX_TOKENS = 64;
bool few_attn_fits(int T_max, int H, int nh);
hipError_t launch_attn_out_few(const float* qkv, const float* wo, const int* cu, const int* ntok, int B,
                              int T_max, int H, int nh, float scale, float* Y, int64_t part_stride,
                              hipStream_t s);

// Embedding gather + position + token type 0 + LayerNorm over packed tokens,
// into x (fp32) and / or x16 (bf16; either may be nullptr, not both).
hipError_t launch_embed_ln(const int* tok_id, const int* tok_pos, const int* n_tokens,
                           int T_max, const float* word, const float* pos, const float* type0,
                           const float* g, const float* b, int V, int H, float eps, float* x,
                           int* err, uint16_t* x16, hipStream_t s);

// Masked mean over each packed sequence, optional L2 normalisation; out [B, H].
// Floats of `partials` the fp32 pool needs: B * ceil(S / 32) * H when it
// sums fewer sequences than CUs, of more than 32 positions and H % 4 == 0,
// H <= 768, in 32-row chunks; else 0 (unused).
int64_t pool_partials_floats(int B, int H, int S);
hipError_t launch_pool(const float* x, const int* cu_seqlens, int B, int H, int S,
                       int normalize, float* partials, float* out, hipStream_t s);
// The same over a bf16 residual stream x16 (sums in fp32).
hipError_t launch_pool_b16(const uint16_t* x16, const int* cu_seqlens, int B, int H, int S,
                           int normalize, float* out, hipStream_t s);

// Cross-encoder head: out[b] = pooled[b] . w + bias[0] (pooled [B, H], w [H]).
hipError_t launch_cls_head(const float* pooled, const float* w, const float* bias, int B, int H,
                           float* out, hipStream_t s);

// fp32 -> bf16 (round to nearest even) for weight upload.
hipError_t launch_f32_to_bf16(const float* x, uint16_t* y, int64_t n, hipStream_t s);

// y = the fused epilogues' tanh-form GELU of x, elementwise (op-level check
// of its error bound).
hipError_t launch_gelu(const float* x, float* y, int64_t n, hipStream_t s);

// Half-precision checkpoint tensors (safetensors F16 / BF16) to device form:
// F16 -> f32 and BF16 -> f32 exactly, F16 -> bf16 rounded to nearest even.
enum Widen16 : int { WIDEN_F16_F32 = 0, WIDEN_BF16_F32 = 1, WIDEN_F16_BF16 = 2 };
hipError_t launch_widen16(const uint16_t* x, void* y, int64_t n, int mode, hipStream_t s);

// ---------------------------------------------------------------------------
// device helpers
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}

// exp(x) = 2^(x * log2 e) on the hardware exp2 (v_exp_f32).  The rounded
// product x log2(e) has relative error <= 2 eps (eps = 2^-24: the constant
// and the product), which exp2 turns into |x| 2 eps relative error of the
// result, plus its own 1 ulp: |fast_exp(x) - e^x| <= (2 |x| + 2) eps e^x.
// The softmax calls it with x = score - row max <= 0, so each unnormalised
// probability is off by at most max over x <= 0 of (2|x| + 2) eps e^x = 2 eps
// absolute (1.2e-7).  Below x = -87.3 the result is 0 (flushed), against a
// true value below 1.2e-38.
__device__ __forceinline__ float fast_exp(float x) {
    return __builtin_amdgcn_exp2f(x * 1.4426950408889634f);
}

// tanh-form GELU of the reference (src/lib.rs:958-978, constants 151-152).
__device__ __forceinline__ float gelu_tanh(float val) {
    const float SQRT_2_OVER_PI = 0.7978845608f;
    const float GELU_COEFF = 0.044715f;
    float val_cubed = val * val * val;
    float inner = SQRT_2_OVER_PI * (val + GELU_COEFF * val_cubed);
    return val * 0.5f * (1.0f + tanhf(inner));
}

// tanh-form GELU of the reference (constants of src/lib.rs:151-152),
// 0.5 x (1 + tanh(u)) with u = sqrt(2/pi) (x + 0.044715 x^3), evaluated as
// x * sigmoid(2u) = x / (1 + e^(-2u)) on the hardware exp2 and reciprocal:
// five VALU operations besides those two, and no cancellation for negative x
// (e^(-2u) = inf gives -0 for finite x; x = +inf gives +inf, -inf gives NaN,
// as the tanh form does).
//
// Error bound (eps = 2^-24, t = x (K1 + K2 x^2) the exponent passed to exp2),
// against the same formula in exact arithmetic with the reference's decimal
// constants: K1 and K2 are rounded products of rounded constants (3 and 5
// eps); s = fma(x^2, K2, K1) adds the rounding of x^2 and its own (its two
// terms have the same sign, so nothing cancels): 7 eps; t = x s: 8 eps.
// exp2 turns a relative error d of t into |t| d ln 2 of e, plus its own
// 1 ulp; 1 + e, the reciprocal and the final product add 4 eps, and e's
// error reaches the result scaled by e / (1 + e) <= 1.  So
//   |gelu_fast(x) - gelu(x)| <= (8 ln2 |t| + 8) eps |gelu(x)|,
// e.g. <= 8.5e-6 relative for x >= -5 (|t| <= 25), <= 6e-7 for x >= 0.
// Where t > 126 (x < -9.7) e leaves the fp32 range and the result is -0 or a
// value below 2^-126, against a true value below 1e-36.
// ebh_op_gelu (test_gpu_ops.py) checks this bound over [-12, 12] against the
// float64 tanh form.
__device__ __forceinline__ float gelu_tanh_fast(float val) {
    // -2 * log2(e) * sqrt(2/pi), and that times 0.044715
    const float K1 = -2.0f * 1.4426950408889634f * 0.7978845608f;
    const float K2 = K1 * 0.044715f;
    const float e = __builtin_amdgcn_exp2f(val * fmaf(val * val, K2, K1));  // e^(-2u)
    return val * __builtin_amdgcn_rcpf(1.0f + e);
}

// One lane's 16 bytes from global memory straight into LDS
// (global_load_lds_dwordx4): lane l of the wave lands at lds + 16 l bytes, so
// `lds` must be the same for every lane.  Issued from inline asm so that the
// compiler's wait-count tracking does not see it (it would otherwise make
// every LDS read wait for every outstanding load); callers wait explicitly
// with wait_vmcnt.  M0 (the instruction's LDS base) is saved and restored.
__device__ __forceinline__ void load_lds16_async(const void* g, const float* lds) {
    const uint32_t base = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds);
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %2\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %1, off\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(g), "s"(base)
        : "memory");
}

// A pointer every lane of the wave holds, as a wave-uniform 64-bit value
// (readfirstlane of each half; the casts keep the low half from being
// sign-extended into the high one).
__device__ __forceinline__ uint64_t uniform_u64(const void* p) {
    const uint64_t b = (uint64_t)(uintptr_t)p;
    return ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32)) << 32) |
           (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b);
}

// load_lds16_async with the global address split as a wave-uniform 64-bit
// base (SGPR pair) plus this lane's 32-bit byte offset: the saddr form of
// global_load_lds_dwordx4.  lds_addr is the LDS byte address (the same for
// every lane).
__device__ __forceinline__ void load_lds16_sbase(uint64_t sbase, uint32_t voff, uint32_t lds_addr) {
    const uint32_t base = __builtin_amdgcn_readfirstlane(lds_addr);
    const void* sb = (const void*)(uintptr_t)sbase;
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %3\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %1, %2\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(voff), "s"(sb), "s"(base)
        : "memory");
}
__device__ __forceinline__ void load_lds16_sbase(uint64_t sbase, uint32_t voff, const float* lds) {
    load_lds16_sbase(sbase, voff, (uint32_t)(uintptr_t)lds);
}

// At most n vector-memory operations of this wave outstanding (n is
// wave-uniform; s_waitcnt takes an immediate, so switch over the counter's
// range, 0..63; larger n waits for everything, which is always safe).
// Vector memory operations complete in issue order.
__device__ __forceinline__ void wait_vmcnt(int n) {
    switch (n) {
#define EBH_VMCNT(k) \
    case k: asm volatile("s_waitcnt vmcnt(" #k ")" ::: "memory"); break;
        EBH_VMCNT(1) EBH_VMCNT(2) EBH_VMCNT(3) EBH_VMCNT(4) EBH_VMCNT(5) EBH_VMCNT(6)
        EBH_VMCNT(7) EBH_VMCNT(8) EBH_VMCNT(9) EBH_VMCNT(10) EBH_VMCNT(11) EBH_VMCNT(12)
        EBH_VMCNT(13) EBH_VMCNT(14) EBH_VMCNT(15) EBH_VMCNT(16) EBH_VMCNT(17) EBH_VMCNT(18)
        EBH_VMCNT(19) EBH_VMCNT(20) EBH_VMCNT(21) EBH_VMCNT(22) EBH_VMCNT(23) EBH_VMCNT(24)
        EBH_VMCNT(25) EBH_VMCNT(26) EBH_VMCNT(27) EBH_VMCNT(28) EBH_VMCNT(29) EBH_VMCNT(30)
        EBH_VMCNT(31) EBH_VMCNT(32) EBH_VMCNT(33) EBH_VMCNT(34) EBH_VMCNT(35) EBH_VMCNT(36)
        EBH_VMCNT(37) EBH_VMCNT(38) EBH_VMCNT(39) EBH_VMCNT(40) EBH_VMCNT(41) EBH_VMCNT(42)
        EBH_VMCNT(43) EBH_VMCNT(44) EBH_VMCNT(45) EBH_VMCNT(46) EBH_VMCNT(47) EBH_VMCNT(48)
        EBH_VMCNT(49) EBH_VMCNT(50) EBH_VMCNT(51) EBH_VMCNT(52) EBH_VMCNT(53) EBH_VMCNT(54)
        EBH_VMCNT(55) EBH_VMCNT(56) EBH_VMCNT(57) EBH_VMCNT(58) EBH_VMCNT(59) EBH_VMCNT(60)
        EBH_VMCNT(61) EBH_VMCNT(62) EBH_VMCNT(63)
#undef EBH_VMCNT
        default: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
    }
}

// wait_vmcnt for a count known to be one of a few values: a descending
// ladder over those values (V0 > V1 > ...) waits until at most the largest
// of them that is <= n is outstanding, else for everything.  That is the
// exact wait when n is one of them and a longer one otherwise, and costs a
// compare per value instead of wait_vmcnt's search over the counter's range.
template <int V, int... Vs>
__device__ __forceinline__ void wait_vmcnt_of(int n) {
    static_assert(V >= 0 && V < 64, "vmcnt range");
    if (n >= V) {
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(V) : "memory");
    } else {
        if constexpr (sizeof...(Vs) > 0) wait_vmcnt_of<Vs...>(n);
        else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
}

// This wave's LDS reads have returned; then the workgroup barrier.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// XOR swizzle of the 16-byte chunk index within an LDS row of CPR chunks
// (tiles stored unpadded, [rows][CPR chunks]): chunk c of row r lives at
// c ^ chunk_swizzle16<CPR>(r).  32 lanes reading one chunk of 32 consecutive
// rows then spread over all banks (checked for 32 and 64 banks).
template <int CPR>
__device__ __forceinline__ int chunk_swizzle16(int r) {
    static_assert(CPR == 4 || CPR == 8 || CPR == 16, "4, 8 or 16 chunks per row");
    if constexpr (CPR == 16) return r & 15;
    else if constexpr (CPR == 8) return (r & 7) ^ ((r >> 3) & 1);
    else return ((r >> 1) & 3) ^ ((r >> 3) & 1);
}

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);  // quiet NaN
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// Two floats to two bf16 (round to nearest even, NaN stays NaN) packed in one
// word, lo in bits 0..15: gfx950's v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    typedef float v2f_t __attribute__((ext_vector_type(2)));
    typedef __bf16 v2bf_t __attribute__((ext_vector_type(2)));
    const v2f_t v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, v2bf_t));
}

}  // namespace ebh
