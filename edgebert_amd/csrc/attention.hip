// attention.hip -- masked multi-head self-attention over packed sequences.
//
// Replaces, per (sequence, head), the reference chain
//   q.k^T (matmul_4d, src/lib.rs:713, 898-956) -> * scale (714) ->
//   key-padding mask to -inf (717, 872-896) -> row softmax (720, 851-870) ->
//   P.V (723) -> permute back (726-730)
// without materialising the [S, S] score matrix in HBM.  Tokens are packed
// (only mask == 1 tokens exist), so the key-padding mask becomes "key index <
// sequence length"; a padded key contributes exactly 0, as exp(-inf) does in
// the reference.
//
// Work split: workgroup = (head, 128-query block, sequence), 4 waves of 32
// queries.  K and V of the sequence stream through LDS in 128-key chunks;
// softmax is online across chunks (one chunk when S <= 128).
//
// Transposed scores: each wave computes S^T = K . Q^T with
// v_mfma_f32_32x32x2_f32, so lane l owns query l%32 and, for each 32-key
// block, keys 8*(r/4) + 4*(l/32) + r%4 (r = 0..15).  Row max / sum are then
// per-lane reductions plus one exchange with lane l^32, and the
// probabilities already sit in the A-operand layout of the P.V MFMA
// (row = query = l%32, k = one key per lane half), so P never leaves
// registers.
#include "kernels.hpp"

namespace ebh {

typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));

template <int HD, bool OUT16>
__global__ __launch_bounds__(256) void attention_kernel(const float* __restrict__ qkv,
                                                        const int* __restrict__ cu_seqlens,
                                                        void* __restrict__ ctx_out, int H,
                                                        float scale) {
    constexpr int KC = 128;        // keys per LDS chunk
    constexpr int KS = HD + 4;     // K row stride (floats): conflict-free 16-B reads
    constexpr int NJ = HD / 32;    // 32-wide output blocks of the context
    __shared__ __attribute__((aligned(16))) float Ks[KC * KS];
    __shared__ __attribute__((aligned(16))) float Vs[KC * HD];

    const int head = blockIdx.x, qb = blockIdx.y, b = blockIdx.z;
    const int start = cu_seqlens[b];
    const int len = cu_seqlens[b + 1] - start;
    if (qb * 128 >= len) return;  // uniform over the workgroup

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, half = lane >> 5;
    const int64_t ld = 3 * (int64_t)H;
    const float* Qg = qkv + (int64_t)start * ld + head * HD;
    const float* Kg = Qg + H;
    const float* Vg = Qg + 2 * H;

    // This lane's query row as the B operand of S^T = K . Q^T.
    const int q0 = qb * 128 + wave * 32;
    const int qi = min(q0 + l32, len - 1);
    v4f qf[HD / 8];
#pragma unroll
    for (int s = 0; s < HD / 8; ++s)
        qf[s] = *reinterpret_cast<const v4f*>(Qg + (int64_t)qi * ld + s * 8 + 4 * half);

    v16f o[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[j][r] = 0.0f;
    float m_run = -INFINITY, l_run = 0.0f;

    const int nchunks = (len + KC - 1) / KC;
    for (int c = 0; c < nchunks; ++c) {
        const int kbase = c * KC;
        __syncthreads();  // previous chunk fully consumed
        constexpr int F4 = KC * HD / 4;
        for (int i = tid; i < F4; i += 256) {
            const int r = i / (HD / 4), cc = i % (HD / 4);
            const int key = kbase + r;
            float4 kv = make_float4(0, 0, 0, 0), vv = make_float4(0, 0, 0, 0);
            if (key < len) {
                kv = *reinterpret_cast<const float4*>(Kg + (int64_t)key * ld + cc * 4);
                vv = *reinterpret_cast<const float4*>(Vg + (int64_t)key * ld + cc * 4);
            }
            *reinterpret_cast<float4*>(&Ks[r * KS + cc * 4]) = kv;
            *reinterpret_cast<float4*>(&Vs[r * HD + cc * 4]) = vv;
        }
        __syncthreads();

        const int nkb = min(4, (len - kbase + 31) / 32);  // 32-key blocks holding real keys
        v16f sc[4];
        float cmax = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            if (kb < nkb) {
#pragma unroll
                for (int r = 0; r < 16; ++r) sc[kb][r] = 0.0f;
                const float* kr = Ks + (kb * 32 + l32) * KS + 4 * half;
#pragma unroll
                for (int s = 0; s < HD / 8; ++s) {
                    const v4f kf = *reinterpret_cast<const v4f*>(kr + s * 8);
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        sc[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(kf[q], qf[s][q], sc[kb], 0, 0, 0);
                }
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key = kbase + kb * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
                    float t = sc[kb][r] * scale;         // scale after q.k^T (src/lib.rs:714)
                    if (key >= len) t = -INFINITY;       // key-padding mask (src/lib.rs:887-891)
                    sc[kb][r] = t;
                    cmax = fmaxf(cmax, t);
                }
            }
        }
        cmax = fmaxf(cmax, __shfl_xor(cmax, 32));
        const float m_new = fmaxf(m_run, cmax);
        const float alpha = fast_exp(m_run - m_new);  // 0 on the first chunk
        float psum = 0.0f;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            if (kb < nkb) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const float pr = fast_exp(sc[kb][r] - m_new);
                    sc[kb][r] = pr;
                    psum += pr;
                }
            }
        }
        l_run = l_run * alpha + psum;
        m_run = m_new;
        if (c > 0) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float ar = __shfl(alpha, 8 * (r >> 2) + 4 * half + (r & 3));
#pragma unroll
                for (int j = 0; j < NJ; ++j) o[j][r] *= ar;
            }
        }
        // context += P . V over this chunk
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            if (kb < nkb) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key = kb * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
#pragma unroll
                    for (int j = 0; j < NJ; ++j)
                        o[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(
                            sc[kb][r], Vs[key * HD + j * 32 + l32], o[j], 0, 0, 0);
                }
            }
        }
    }

    // Normalise by the row sum (both lane halves hold partial sums) and store:
    // lane holds context column j*32 + l32 of query rows 8*(r/4) + 4*half + r%4.
    const float l_tot = l_run + __shfl_xor(l_run, 32);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int qrow = 8 * (r >> 2) + 4 * half + (r & 3);
        const float lq = __shfl(l_tot, qrow);
        const int q = q0 + qrow;
        if (q < len) {
            const int64_t at = (int64_t)(start + q) * H + head * HD + l32;
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                const float c = o[j][r] / lq;
                if constexpr (OUT16) static_cast<uint16_t*>(ctx_out)[at + j * 32] = f32_to_bf16_rne(c);
                else static_cast<float*>(ctx_out)[at + j * 32] = c;
            }
        }
    }
}

hipError_t launch_attention(const float* qkv, const int* cu_seqlens, int B, int max_len, int H,
                            int nh, int head_dim, float scale, void* ctx, bool ctx_bf16,
                            hipStream_t s) {
    if (B <= 0 || max_len <= 0) return hipSuccess;
    const dim3 grid(nh, (max_len + 127) / 128, B), block(256);
    if (head_dim == 32 && !ctx_bf16)
        hipLaunchKernelGGL((attention_kernel<32, false>), grid, block, 0, s, qkv, cu_seqlens, ctx, H, scale);
    else if (head_dim == 32)
        hipLaunchKernelGGL((attention_kernel<32, true>), grid, block, 0, s, qkv, cu_seqlens, ctx, H, scale);
    else if (head_dim == 64 && !ctx_bf16)
        hipLaunchKernelGGL((attention_kernel<64, false>), grid, block, 0, s, qkv, cu_seqlens, ctx, H, scale);
    else if (head_dim == 64)
        hipLaunchKernelGGL((attention_kernel<64, true>), grid, block, 0, s, qkv, cu_seqlens, ctx, H, scale);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace ebh
