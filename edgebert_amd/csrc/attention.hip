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
// probabilities already sit in an operand layout of the P.V MFMA (query =
// l%32, one key per lane half), so P never leaves registers.  The context is
// accumulated transposed too, O^T = V^T . P^T: lane l then holds dims
// 8*(r/4) + 4*(l/32) + r%4 of its own query l%32, so the online-softmax
// rescale and the final division use the lane's own statistics, and the
// context leaves as 16-byte stores of four consecutive dims.
#include "kernels.hpp"

namespace ebh {

typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));

template <int HD>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(HD == 32 ? 3 : 2))) void attention_kernel(const float* __restrict__ qkv,
                                                        const int* __restrict__ cu_seqlens,
                                                        float* __restrict__ ctx_out, int H,
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
        // K and V loads go out in groups of up to 4 + 4 float4 per thread, a
        // group's loads all issued before its LDS writes: the chunk costs one
        // or two memory round trips instead of one per piece.
        constexpr int F4 = KC * HD / 4;       // float4 pieces of K (and of V)
        constexpr int PT = F4 / 256;          // per thread
        constexpr int GP = PT < 4 ? PT : 4;   // per group
        static_assert(PT * 256 == F4 && PT % GP == 0, "whole pieces per thread");
#pragma unroll
        for (int g0 = 0; g0 < PT; g0 += GP) {
            float4 kv[GP], vv[GP];
#pragma unroll
            for (int pi = 0; pi < GP; ++pi) {
                const int i = tid + 256 * (g0 + pi), key = kbase + i / (HD / 4), cc = i % (HD / 4);
                kv[pi] = vv[pi] = make_float4(0, 0, 0, 0);
                if (key < len) {
                    kv[pi] = *reinterpret_cast<const float4*>(Kg + (int64_t)key * ld + cc * 4);
                    vv[pi] = *reinterpret_cast<const float4*>(Vg + (int64_t)key * ld + cc * 4);
                }
            }
#pragma unroll
            for (int pi = 0; pi < GP; ++pi) {
                const int i = tid + 256 * (g0 + pi), r = i / (HD / 4), cc = i % (HD / 4);
                *reinterpret_cast<float4*>(&Ks[r * KS + cc * 4]) = kv[pi];
                *reinterpret_cast<float4*>(&Vs[r * HD + cc * 4]) = vv[pi];
            }
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
            for (int j = 0; j < NJ; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) o[j][r] *= alpha;
        }
        // context^T += V^T . P^T over this chunk: A = V^T (row = dim l32, one
        // key per lane half), B = P^T (that key, column = query l32).
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            if (kb < nkb) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key = kb * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
#pragma unroll
                    for (int j = 0; j < NJ; ++j)
                        o[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(
                            Vs[key * HD + j * 32 + l32], sc[kb][r], o[j], 0, 0, 0);
                }
            }
        }
    }

    // Normalise by the row sum (both lane halves hold partial sums) and store:
    // lane holds dims j*32 + 8*g + 4*half + 0..3 (g = r / 4) of query l32.
    const float l_tot = l_run + __shfl_xor(l_run, 32);
    const int q = q0 + l32;
    if (q < len) {
        const float inv = 1.0f / l_tot;
        const int64_t at = (int64_t)(start + q) * H + head * HD + 4 * half;
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const float c0 = o[j][4 * g] * inv, c1 = o[j][4 * g + 1] * inv;
                const float c2 = o[j][4 * g + 2] * inv, c3 = o[j][4 * g + 3] * inv;
                *reinterpret_cast<float4*>(ctx_out + at + j * 32 + 8 * g) = make_float4(c0, c1, c2, c3);
            }
    }
}

// ---------------------------------------------------------------------------
// bf16 variant (models whose GEMMs run in bf16): Q, K, V and the context are
// bf16; scores, softmax, row sums and the P.V accumulation are fp32.
//
// S^T = K . Q^T on v_mfma_f32_32x32x16_bf16: lane (l%32, half h) supplies
// K row (key) l%32 and Q row (query) l%32, dims 16s + 8h .. +7 of slice s, so
// the score layout is that of the fp32 kernel (lane owns query l%32; keys
// 8*(r/4) + 4h + r%4 of each 32-key block).  For P.V, MFMA m (m = 0, 1) of a
// 32-key block takes r in [8m, 8m+8): lane half h then holds keys
// 16m + 4h + 0..3 and 16m + 8 + 4h + 0..3, which together cover the 16 keys
// of that MFMA, so P goes to the A operand straight from registers (rounded to
// bf16).  The B operand needs, per lane, the same 8 keys at one head dim, so V
// is staged transposed in LDS (Vt[dim][key], two keys per 32-bit word) and
// read as two 8-byte runs.
// ---------------------------------------------------------------------------
typedef short v8s_t __attribute__((ext_vector_type(8)));
typedef __bf16 v8bf_t __attribute__((ext_vector_type(8)));

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

template <int HD>
__global__ __launch_bounds__(256) void attention_bf16_kernel(const uint16_t* __restrict__ qkv,
                                                             const int* __restrict__ cu_seqlens,
                                                             uint16_t* __restrict__ ctx, int H,
                                                             float scale) {
    constexpr int KC = 128;                 // keys per LDS chunk
    constexpr int KRS = HD + 8;             // K row stride (bf16): 16-byte padding, conflict-free b128 reads
    constexpr int VTS = KC + 8;             // Vt row stride (bf16): one row per head dim
    constexpr int NJ = HD / 32;             // 32-wide blocks of the context
    constexpr int NS = HD / 16;             // 16-dim slices of q.k
    __shared__ __attribute__((aligned(16))) uint16_t Ks[KC * KRS];
    __shared__ __attribute__((aligned(16))) uint16_t Vt[HD * VTS];

    const int head = blockIdx.x, qb = blockIdx.y, b = blockIdx.z;
    const int start = cu_seqlens[b];
    const int len = cu_seqlens[b + 1] - start;
    if (qb * 128 >= len) return;  // uniform over the workgroup

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, half = lane >> 5;
    const int64_t ld = 3 * (int64_t)H;
    const uint16_t* Qg = qkv + (int64_t)start * ld + head * HD;
    const uint16_t* Kg = Qg + H;
    const uint16_t* Vg = Qg + 2 * H;

    // This lane's query as the B operand: dims 16s + 8*half .. +7.
    const int q0 = qb * 128 + wave * 32;
    const int qi = min(q0 + l32, len - 1);
    v8s_t qf[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s)
        qf[s] = *reinterpret_cast<const v8s_t*>(Qg + (int64_t)qi * ld + 16 * s + 8 * half);

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
        // Every K and V load of the chunk is issued before the first LDS
        // write (one memory round trip per chunk).  K: 16-byte pieces (8
        // dims) straight into the padded row layout.  V transposed: a thread
        // takes keys (2p, 2p+1) x 8 dims and writes 8 words Vt[d][2p .. 2p+1].
        constexpr int KP = KC * HD / 8, KPT = KP / 256;
        constexpr int VP = (KC / 2) * (HD / 8), VPT = VP / 256;
        static_assert(KPT * 256 == KP && VPT * 256 == VP, "whole pieces per thread");
        uint4 kv[KPT], va[VPT], vb2[VPT];
#pragma unroll
        for (int pi = 0; pi < KPT; ++pi) {
            const int i = tid + 256 * pi, key = kbase + i / (HD / 8), cc = i % (HD / 8);
            kv[pi] = make_uint4(0, 0, 0, 0);
            if (key < len) kv[pi] = *reinterpret_cast<const uint4*>(Kg + (int64_t)key * ld + cc * 8);
        }
#pragma unroll
        for (int pi = 0; pi < VPT; ++pi) {
            const int i = tid + 256 * pi, pr = i % (KC / 2), cc = i / (KC / 2);
            const int k0 = kbase + 2 * pr;
            va[pi] = vb2[pi] = make_uint4(0, 0, 0, 0);
            if (k0 < len) va[pi] = *reinterpret_cast<const uint4*>(Vg + (int64_t)k0 * ld + cc * 8);
            if (k0 + 1 < len) vb2[pi] = *reinterpret_cast<const uint4*>(Vg + (int64_t)(k0 + 1) * ld + cc * 8);
        }
#pragma unroll
        for (int pi = 0; pi < KPT; ++pi) {
            const int i = tid + 256 * pi, r = i / (HD / 8), cc = i % (HD / 8);
            *reinterpret_cast<uint4*>(&Ks[r * KRS + cc * 8]) = kv[pi];
        }
#pragma unroll
        for (int pi = 0; pi < VPT; ++pi) {
            const int i = tid + 256 * pi, pr = i % (KC / 2), cc = i / (KC / 2);
            const uint32_t av[4] = {va[pi].x, va[pi].y, va[pi].z, va[pi].w};
            const uint32_t bv[4] = {vb2[pi].x, vb2[pi].y, vb2[pi].z, vb2[pi].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int d = cc * 8 + 2 * e;
                *reinterpret_cast<uint32_t*>(&Vt[d * VTS + 2 * pr]) = (av[e] & 0xFFFFu) | (bv[e] << 16);
                *reinterpret_cast<uint32_t*>(&Vt[(d + 1) * VTS + 2 * pr]) = (av[e] >> 16) | (bv[e] & 0xFFFF0000u);
            }
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
                const uint16_t* kr = Ks + (kb * 32 + l32) * KRS + 8 * half;
#pragma unroll
                for (int s = 0; s < NS; ++s) {
                    const v8s_t kf = *reinterpret_cast<const v8s_t*>(kr + 16 * s);
                    sc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf_t, kf),
                                                                      __builtin_bit_cast(v8bf_t, qf[s]),
                                                                      sc[kb], 0, 0, 0);
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
            for (int j = 0; j < NJ; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) o[j][r] *= alpha;
        }
        // context^T += V^T . P^T over this chunk, two 16-key MFMAs per 32-key
        // block: A = V^T (row = dim l32, this lane half's 8 keys), B = P^T.
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            if (kb < nkb) {
#pragma unroll
                for (int mm = 0; mm < 2; ++mm) {
                    const float* pf = reinterpret_cast<const float*>(&sc[kb]) + 8 * mm;
                    const v8s_t pa = __builtin_bit_cast(
                        v8s_t, make_uint4(pack_bf16x2(pf[0], pf[1]), pack_bf16x2(pf[2], pf[3]),
                                          pack_bf16x2(pf[4], pf[5]), pack_bf16x2(pf[6], pf[7])));
                    const int kl = kb * 32 + 16 * mm + 4 * half;   // first of this lane's two 4-key runs
#pragma unroll
                    for (int j = 0; j < NJ; ++j) {
                        const uint16_t* vr = Vt + (j * 32 + l32) * VTS + kl;
                        const uint2 lo = *reinterpret_cast<const uint2*>(vr);
                        const uint2 hi = *reinterpret_cast<const uint2*>(vr + 8);
                        v8s_t vb;
                        vb[0] = (short)(lo.x & 0xFFFF); vb[1] = (short)(lo.x >> 16);
                        vb[2] = (short)(lo.y & 0xFFFF); vb[3] = (short)(lo.y >> 16);
                        vb[4] = (short)(hi.x & 0xFFFF); vb[5] = (short)(hi.x >> 16);
                        vb[6] = (short)(hi.y & 0xFFFF); vb[7] = (short)(hi.y >> 16);
                        o[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf_t, vb),
                                                                        __builtin_bit_cast(v8bf_t, pa),
                                                                        o[j], 0, 0, 0);
                    }
                }
            }
        }
    }

    // Lane holds dims j*32 + 8*g + 4*half + 0..3 (g = r / 4) of query l32.
    const float l_tot = l_run + __shfl_xor(l_run, 32);
    const int q = q0 + l32;
    if (q < len) {
        const float inv = 1.0f / l_tot;
        uint16_t* dst = ctx + (int64_t)(start + q) * H + head * HD + 4 * half;
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                *reinterpret_cast<uint2*>(dst + j * 32 + 8 * g) =
                    make_uint2(pack_bf16x2(o[j][4 * g] * inv, o[j][4 * g + 1] * inv),
                               pack_bf16x2(o[j][4 * g + 2] * inv, o[j][4 * g + 3] * inv));
            }
    }
}

hipError_t launch_attention_bf16(const uint16_t* qkv, const int* cu_seqlens, int B, int max_len,
                                 int H, int nh, int head_dim, float scale, uint16_t* ctx,
                                 hipStream_t s) {
    if (B <= 0 || max_len <= 0) return hipSuccess;
    const dim3 grid(nh, (max_len + 127) / 128, B), block(256);
    if (head_dim == 32)
        hipLaunchKernelGGL(attention_bf16_kernel<32>, grid, block, 0, s, qkv, cu_seqlens, ctx, H, scale);
    else if (head_dim == 64)
        hipLaunchKernelGGL(attention_bf16_kernel<64>, grid, block, 0, s, qkv, cu_seqlens, ctx, H, scale);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_attention(const float* qkv, const int* cu_seqlens, int B, int max_len, int H,
                            int nh, int head_dim, float scale, float* ctx, hipStream_t s) {
    if (B <= 0 || max_len <= 0) return hipSuccess;
    const dim3 grid(nh, (max_len + 127) / 128, B), block(256);
    if (head_dim == 32)
        hipLaunchKernelGGL(attention_kernel<32>, grid, block, 0, s, qkv, cu_seqlens, ctx, H, scale);
    else if (head_dim == 64)
        hipLaunchKernelGGL(attention_kernel<64>, grid, block, 0, s, qkv, cu_seqlens, ctx, H, scale);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace ebh
