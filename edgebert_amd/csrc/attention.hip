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
// queries.  K and V of the sequence stream through LDS in 64-key chunks
// (sequences of at most 128 tokens) or 128-key chunks; softmax is online
// across chunks.  The grid's
// sequence index goes through `order` when the caller has one (the packing
// scan writes the sequences longest first), so that the long sequences'
// workgroups start first.
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
#include <algorithm>

#include "kernels.hpp"

namespace ebh {

typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));

// One key chunk (up to 128 keys, in 32-key blocks) of the fp32 kernel below
// for the wave's 32 queries: S^T = K . Q^T, the key-padding mask, the
// online-softmax update and context^T += V^T . P^T.  lim = real keys in the
// chunk (1..128); c2 = scale log2(e).  Fewer VALU instructions matter here: on this chip the VALU does
// not issue while an fp32 MFMA of the same SIMD runs, so the softmax's
// instructions add to the MFMA time instead of hiding behind it.
template <int HD>
__device__ __forceinline__ void attend_chunk(const float* Ks, const float* Vs, const v4f* qf, float c2, int l32,
                                             int half, int lim, v16f* o, float& m_run, float& l_run, bool first) {
    constexpr int KS = HD + 4, NJ = HD / 32;
    v16f sc[4];
    float cmax = -INFINITY;
    const int lim_h = lim - 4 * half;   // key kb*32 + 8(r/4) + r%4 + 4 half is real iff kb*32 + 8(r/4) + r%4 < lim_h
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
        if (kb * 32 < lim) {
#pragma unroll
            for (int r = 0; r < 16; ++r) sc[kb][r] = 0.0f;
            const float* kr = Ks + (kb * 32 + l32) * KS + 4 * half;
#pragma unroll
            for (int s = 0; s < HD / 8; ++s) {
                const v4f kf = *reinterpret_cast<const v4f*>(kr + s * 8);
#pragma unroll
                for (int q = 0; q < 4; ++q) sc[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(kf[q], qf[s][q], sc[kb], 0, 0, 0);
            }
            // Key-padding mask (src/lib.rs:887-891), only in the block that
            // straddles the sequence end; the row max is taken over the raw
            // scores (scale > 0 commutes with max).
            if ((kb + 1) * 32 > lim) {
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (kb * 32 + 8 * (r >> 2) + (r & 3) >= lim_h) sc[kb][r] = -INFINITY;
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) cmax = fmaxf(cmax, sc[kb][r]);
        }
    }
    cmax = fmaxf(cmax, __shfl_xor(cmax, 32));
    // exp(scale (s - m)) as 2^(s c - m c), c = scale log2(e): the scale after
    // q.k^T (src/lib.rs:714) folded into one FMA per score.  m and m_run are
    // raw-score maxima; alpha = 0 on the first chunk.  The exponent is off by
    // at most 3 eps |s c - m c| + eps |m c| (the roundings of c, m c and the
    // FMA; eps = 2^-24), which exp2 turns into a relative error of that times
    // ln 2 plus its own 1 ulp.
    const float m_new = fmaxf(m_run, cmax);
    const float mc = m_new * c2;
    const float alpha = __builtin_amdgcn_exp2f(m_run * c2 - mc);
    float ps[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
        if (kb * 32 < lim) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float pr = __builtin_amdgcn_exp2f(fmaf(sc[kb][r], c2, -mc));
                sc[kb][r] = pr;
                ps[r & 3] += pr;
            }
        }
    }
    l_run = l_run * alpha + ((ps[0] + ps[1]) + (ps[2] + ps[3]));
    m_run = m_new;
    if (!first) {
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) o[j][r] *= alpha;
    }
    // context^T += V^T . P^T: A = V^T (row = dim l32, one key per lane half),
    // B = P^T (that key, column = query l32).
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
        if (kb * 32 < lim) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int key = kb * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
#pragma unroll
                for (int j = 0; j < NJ; ++j)
                    o[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(Vs[key * HD + j * 32 + l32], sc[kb][r], o[j], 0, 0, 0);
            }
        }
    }
}

// KC = keys per LDS chunk.  With 64-key chunks (sequences of at most 128
// tokens) the next chunk's K and V are loaded into registers while the
// current chunk's MFMAs run, and the smaller chunk leaves room for four
// workgroups per CU (c3: 69.5 -> 65.8 us per layer against one 128-key chunk);
// longer sequences keep 128-key chunks, loaded when they are needed, three
// workgroups per CU (c4: 53.1 against 53.9 us with 64-key chunks).
template <int HD, int KC>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(HD == 32 ? (KC == 64 ? 4 : 3) : 2))) void attention_kernel(
    const float* __restrict__ qkv, const int* __restrict__ cu_seqlens, float* __restrict__ ctx_out, int H, float scale,
    const int* __restrict__ order) {
    constexpr bool PREFETCH = KC == 64;
    constexpr int KS = HD + 4;     // K row stride (floats): conflict-free 16-B reads
    constexpr int NJ = HD / 32;    // 32-wide output blocks of the context
    __shared__ __attribute__((aligned(16))) float Ks[KC * KS];
    __shared__ __attribute__((aligned(16))) float Vs[KC * HD];

    const int head = blockIdx.x, qb = blockIdx.y, b = order ? order[blockIdx.z] : (int)blockIdx.z;
    const int start = cu_seqlens[b];
    const int len = cu_seqlens[b + 1] - start;
    if (qb * 128 >= len) return;  // uniform over the workgroup

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, half = lane >> 5;
    const int64_t ld = 3 * (int64_t)H;
    const float* Qg = qkv + (int64_t)start * ld + head * HD;
    const float* Kg = Qg + H;
    const float* Vg = Qg + 2 * H;

    // K and V of a chunk, float4 pieces in registers (with PREFETCH the next
    // chunk's loads go out before the current chunk's MFMAs, so only the first
    // chunk waits for memory).
    constexpr int F4 = KC * HD / 4;       // float4 pieces of K (and of V)
    constexpr int PT = F4 / 256;          // per thread
    static_assert(PT * 256 == F4, "whole pieces per thread");
    float4 kv[PT], vv[PT];
    auto load_chunk = [&](int kbase) {
#pragma unroll
        for (int pi = 0; pi < PT; ++pi) {
            const int i = tid + 256 * pi, key = kbase + i / (HD / 4), cc = i % (HD / 4);
            kv[pi] = vv[pi] = make_float4(0, 0, 0, 0);
            if (key < len) {
                kv[pi] = *reinterpret_cast<const float4*>(Kg + (int64_t)key * ld + cc * 4);
                vv[pi] = *reinterpret_cast<const float4*>(Vg + (int64_t)key * ld + cc * 4);
            }
        }
    };
    if (PREFETCH) load_chunk(0);

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
    const float c_exp = scale * 1.4426950408889634f;   // exponent scale of the softmax (base 2)

    const int nchunks = (len + KC - 1) / KC;
    for (int c = 0; c < nchunks; ++c) {
        __syncthreads();  // previous chunk fully consumed
        if (!PREFETCH) load_chunk(c * KC);
#pragma unroll
        for (int pi = 0; pi < PT; ++pi) {
            const int i = tid + 256 * pi, r = i / (HD / 4), cc = i % (HD / 4);
            *reinterpret_cast<float4*>(&Ks[r * KS + cc * 4]) = kv[pi];
            *reinterpret_cast<float4*>(&Vs[r * HD + cc * 4]) = vv[pi];
        }
        __syncthreads();
        if (PREFETCH && c + 1 < nchunks) load_chunk((c + 1) * KC);
        // A wave whose 32 queries all lie past the sequence end (the last
        // query block of a ragged sequence) only helps load K and V.
        if (q0 < len)
            attend_chunk<HD>(Ks, Vs, qf, c_exp, l32, half, min(len - c * KC, KC), o, m_run, l_run, c == 0);
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
                                                             float scale, const int* __restrict__ order) {
    constexpr int KC = 128;                 // keys per LDS chunk
    constexpr int KRS = HD + 8;             // K row stride (bf16): 16-byte padding, conflict-free b128 reads
    constexpr int VTS = KC + 8;             // Vt row stride (bf16): one row per head dim
    constexpr int NJ = HD / 32;             // 32-wide blocks of the context
    constexpr int NS = HD / 16;             // 16-dim slices of q.k
    __shared__ __attribute__((aligned(16))) uint16_t Ks[KC * KRS];
    __shared__ __attribute__((aligned(16))) uint16_t Vt[HD * VTS];

    const int head = blockIdx.x, qb = blockIdx.y, b = order ? order[blockIdx.z] : (int)blockIdx.z;
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
        // A wave whose 32 queries all lie past the sequence end only helps
        // load K and V.
        if (q0 >= len) continue;

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

// ---------------------------------------------------------------------------
// bf16 attention for sequences of at most 128 tokens: one key chunk and one
// query block per (head, sequence) workgroup.  Q, K and V go straight from
// HBM into LDS (global_load_lds_dwordx4, no staging registers, no transposing
// copy), so a workgroup needs 48 KB of LDS and at most 110 VGPRs: three
// workgroups per CU, whose load phases overlap each other's MFMAs and
// softmax; within a workgroup the scores wait for Q and K only.
//
// K rows sit unpadded with 16-byte chunk c of row r at c ^ chunk_swizzle16(r)
// (conflict-free fragment reads down 32 rows), as the GEMM tiles do.  V stays
// row-major ([key][dim]): the A operand of O^T = V^T . P^T needs, per lane,
// one dim at 8 keys, which ds_read_b64_tr_b16 delivers.  Within each 16-lane
// group that instruction hands lane i element i % 4 of the 8-byte reads of
// lanes i / 4, 4 + i / 4, 8 + i / 4 and 12 + i / 4; so when lane j of the
// group addresses key k0 + j / 4, dims d0 + 4 (j % 4) .. +3, lane i receives
// dim d0 + i at the four keys k0 .. k0 + 3.  Two such reads give a lane its 8
// keys of one MFMA.  V chunk c of row r sits at c ^ 4 ((r >> 1) & 1) (64-dim
// rows), so the four rows a half-wave reads fall in different banks.
// ---------------------------------------------------------------------------
typedef short v4s_t __attribute__((ext_vector_type(4)));

template <int HD>
__device__ __forceinline__ int v_swizzle(int r) {
    return HD == 64 ? 4 * ((r >> 1) & 1) : 0;
}

template <int HD>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3, 3))) void attention_bf16_short_kernel(
    const uint16_t* __restrict__ qkv, const int* __restrict__ cu_seqlens, uint16_t* __restrict__ ctx, int H,
    float scale, const int* __restrict__ order) {
    constexpr int KC = 128;                 // keys (and queries) per sequence at most
    constexpr int CPR = HD / 8;             // 16-byte chunks per K / V row
    constexpr int TILE = KC * HD;           // bf16 elements of the K or V tile
    constexpr int NLD = KC * CPR / 256;     // 16-byte loads per thread per tile
    constexpr int NJ = HD / 32;             // 32-wide blocks of the context
    constexpr int NS = HD / 16;             // 16-dim slices of q.k
    __shared__ __attribute__((aligned(16))) uint16_t Ks[TILE];
    __shared__ __attribute__((aligned(16))) uint16_t Vs[TILE];
    __shared__ __attribute__((aligned(16))) uint16_t Qs[TILE];

    const int head = blockIdx.x, b = order ? order[blockIdx.y] : (int)blockIdx.y;
    const int start = cu_seqlens[b];
    const int len = cu_seqlens[b + 1] - start;
    if (len == 0) return;  // uniform over the workgroup
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, half = lane >> 5;
    const int64_t ld = 3 * (int64_t)H;
    const uint16_t* Qg = qkv + (int64_t)start * ld + head * HD;
    const uint16_t* Kg = Qg + H;
    const uint16_t* Vg = Qg + 2 * H;

    // Q, K and V into LDS, in that order: wave w's load i fills 16-byte slots
    // (4 i + w) * 64 + lane, i.e. row P / CPR, stored chunk P % CPR.  Rows
    // past the sequence re-read its last row (their keys are masked, their V
    // rows meet zero probabilities, their queries are not stored).  The scores
    // wait for Q and K only; V lands while they and the softmax run.
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
        const int P = (i * 4 + wave) * 64 + lane;
        const int r = P / CPR, pc = P % CPR;
        const int64_t row = (int64_t)min(r, len - 1) * ld;
        load_lds16_async(Qg + row + 8 * (pc ^ chunk_swizzle16<CPR>(r)),
                         reinterpret_cast<const float*>(Qs + (i * 4 + wave) * 512));
    }
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
        const int P = (i * 4 + wave) * 64 + lane;
        const int r = P / CPR, pc = P % CPR;
        const int64_t row = (int64_t)min(r, len - 1) * ld;
        load_lds16_async(Kg + row + 8 * (pc ^ chunk_swizzle16<CPR>(r)),
                         reinterpret_cast<const float*>(Ks + (i * 4 + wave) * 512));
    }
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
        const int P = (i * 4 + wave) * 64 + lane;
        const int r = P / CPR, pc = P % CPR;
        const int64_t row = (int64_t)min(r, len - 1) * ld;
        load_lds16_async(Vg + row + 8 * (pc ^ v_swizzle<HD>(r)),
                         reinterpret_cast<const float*>(Vs + (i * 4 + wave) * 512));
    }
    wait_vmcnt(NLD);   // this wave's Q and K loads (its V loads may be in flight)
    __syncthreads();
    // A wave whose 32 queries all lie past the sequence end skips the scores
    // and P.V; it still meets the barrier below.
    const bool active = wave * 32 < len;
    // This lane's query as the B operand: dims 16s + 8*half .. +7.
    const int qr = wave * 32 + l32;
    v8s_t qf[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s)
        qf[s] = *reinterpret_cast<const v8s_t*>(Qs + qr * HD + 8 * ((2 * s + half) ^ chunk_swizzle16<CPR>(qr)));

    const int nkb = active ? (len + 31) / 32 : 0;   // 32-key blocks holding real keys
    // S^T = K . Q^T: the four 32-key blocks' MFMA chains side by side.
    v16f sc[4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) sc[kb][r] = 0.0f;
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
            if (kb < nkb) {
                const int kr = kb * 32 + l32;
                const v8s_t kf = *reinterpret_cast<const v8s_t*>(
                    Ks + kr * HD + 8 * ((2 * s + half) ^ chunk_swizzle16<CPR>(kr)));
                sc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf_t, kf),
                                                                  __builtin_bit_cast(v8bf_t, qf[s]), sc[kb], 0, 0, 0);
            }
    // Row max of the raw scores (scale > 0 commutes with max); keys past the
    // sequence (only in its last block) are masked to -inf (src/lib.rs:887-891).
    float cmax = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
        if (kb < nkb) {
            if ((kb + 1) * 32 > len) {
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (kb * 32 + 8 * (r >> 2) + 4 * half + (r & 3) >= len) sc[kb][r] = -INFINITY;
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) cmax = fmaxf(cmax, sc[kb][r]);
        }
    }
    cmax = fmaxf(cmax, __shfl_xor(cmax, 32));
    // p = exp(scale * (s - max)) as exp2(s * c - max * c), c = scale * log2(e):
    // the scale after q.k^T (src/lib.rs:714) folded into one FMA.
    const float c2 = scale * 1.4426950408889634f, off = -cmax * c2;
    float psum = 0.0f;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
        if (kb < nkb) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float pr = __builtin_amdgcn_exp2f(fmaf(sc[kb][r], c2, off));
                sc[kb][r] = pr;
                psum += pr;
            }
        }
    }
    v16f o[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[j][r] = 0.0f;
    wait_vmcnt(0);     // this wave's V loads
    __syncthreads();   // and everyone else's
    // context^T += V^T . P^T, two 16-key MFMAs per 32-key block.  Lane half h
    // of the B operand (P) holds keys 16 mm + 4 h + 0..3 and 16 mm + 8 + 4 h +
    // 0..3; the A operand (V^T) gets the same keys at dim l32 from two
    // transposing reads.  16-lane group g reads dims 16 (g % 2) .. +15 of its
    // 32-dim block at keys k0 .. k0 + 3.
    const int g16 = lane >> 4, i16 = lane & 15;
    const int vrow = i16 >> 2, vdim = 16 * (g16 & 1) + 4 * (i16 & 3);
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
        if (kb < nkb) {
#pragma unroll
            for (int mm = 0; mm < 2; ++mm) {
                const float* pf = reinterpret_cast<const float*>(&sc[kb]) + 8 * mm;
                const v8s_t pa = __builtin_bit_cast(
                    v8s_t, make_uint4(pack_bf16x2(pf[0], pf[1]), pack_bf16x2(pf[2], pf[3]),
                                      pack_bf16x2(pf[4], pf[5]), pack_bf16x2(pf[6], pf[7])));
                const int k0 = kb * 32 + 16 * mm + 4 * (g16 >> 1);   // this group's first key
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    const int d = j * 32 + vdim;                     // this lane's 4 dims to address
                    const int ra = k0 + vrow, rb = k0 + 8 + vrow;
                    const v4s_t va = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (__attribute__((address_space(3))) v4s_t*)(Vs + ra * HD + 8 * ((d >> 3) ^ v_swizzle<HD>(ra)) + (d & 7)));
                    const v4s_t vb = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (__attribute__((address_space(3))) v4s_t*)(Vs + rb * HD + 8 * ((d >> 3) ^ v_swizzle<HD>(rb)) + (d & 7)));
                    const v8s_t vf = {va[0], va[1], va[2], va[3], vb[0], vb[1], vb[2], vb[3]};
                    o[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf_t, vf),
                                                                    __builtin_bit_cast(v8bf_t, pa), o[j], 0, 0, 0);
                }
            }
        }
    }
    // Lane holds dims j*32 + 8*g + 4*half + 0..3 (g = r / 4) of query l32.
    const float l_tot = psum + __shfl_xor(psum, 32);
    const int q = wave * 32 + l32;
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
                                 hipStream_t s, const int* order) {
    if (B <= 0 || max_len <= 0) return hipSuccess;
    if (max_len <= 128) {
        // One key chunk per sequence: K and V straight into LDS, three
        // workgroups per CU.
        const dim3 grid(nh, B), block(256);
        if (head_dim == 32)
            hipLaunchKernelGGL(attention_bf16_short_kernel<32>, grid, block, 0, s, qkv, cu_seqlens, ctx, H, scale, order);
        else if (head_dim == 64)
            hipLaunchKernelGGL(attention_bf16_short_kernel<64>, grid, block, 0, s, qkv, cu_seqlens, ctx, H, scale, order);
        else
            return hipErrorInvalidValue;
        return hipGetLastError();
    }
    const dim3 grid(nh, (max_len + 127) / 128, B), block(256);
    if (head_dim == 32)
        hipLaunchKernelGGL(attention_bf16_kernel<32>, grid, block, 0, s, qkv, cu_seqlens, ctx, H, scale, order);
    else if (head_dim == 64)
        hipLaunchKernelGGL(attention_bf16_kernel<64>, grid, block, 0, s, qkv, cu_seqlens, ctx, H, scale, order);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_attention(const float* qkv, const int* cu_seqlens, int B, int max_len, int H,
                            int nh, int head_dim, float scale, float* ctx, hipStream_t s, const int* order) {
    if (B <= 0 || max_len <= 0) return hipSuccess;
    const dim3 grid(nh, (max_len + 127) / 128, B), block(256);
    const bool short_seqs = max_len <= 128;
    if (head_dim == 32 && short_seqs)
        hipLaunchKernelGGL((attention_kernel<32, 64>), grid, block, 0, s, qkv, cu_seqlens, ctx, H, scale, order);
    else if (head_dim == 32)
        hipLaunchKernelGGL((attention_kernel<32, 128>), grid, block, 0, s, qkv, cu_seqlens, ctx, H, scale, order);
    else if (head_dim == 64 && short_seqs)
        hipLaunchKernelGGL((attention_kernel<64, 64>), grid, block, 0, s, qkv, cu_seqlens, ctx, H, scale, order);
    else if (head_dim == 64)
        hipLaunchKernelGGL((attention_kernel<64, 128>), grid, block, 0, s, qkv, cu_seqlens, ctx, H, scale, order);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace ebh
