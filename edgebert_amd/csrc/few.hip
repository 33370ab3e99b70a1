// few.hip -- attention and the attention-output projection in one launch at a
// handful of tokens (fp32, head_dim 32).
//
// With at most FEW_ATTN_MAX_TOKENS packed tokens, the attention half of the
// reference's BertLayer::forward (src/lib.rs:669-683) runs as three launches
// instead of four: the QKV projection (691-698) on the few-token GEMM; then
// attn_out_few_kernel, workgroup (head h, third), masked softmax attention of
// head h over each sequence (713-730) and one third of the columns of the
// head's share of the attention-output projection (732), ctx_h . Wo[:, h*32 ..
// h*32+31]^T, stored as partial h of Y; then add_layernorm (rowops.hip), which
// sums the nh partials in head order, adds the output bias and the residual
// and normalises (733-734).
// At these sizes a launch costs a few microseconds however little it does,
// and a compute unit streams only about 10 bytes per clock from beyond its
// cache.  So launches are merged only where the weights stay spread over many
// workgroups: measured at 16 tokens of MiniLM,
//   - this kernel takes 6.6 us against 4.5 (attention) + 3.7 (the split
//     output projection), and the LayerNorm over 12 partials 4.5 against 4.3;
//   - a workgroup per head that also ran the head's QKV projection spent 20k
//     cycles loading its 196 KB of weights (14 us a launch);
//   - FFN up + GELU + the chunk's share of FFN down in one launch (48
//     workgroups of 32 intermediate columns) took 7.6 us against 5.4 + 4.1,
//     but the LayerNorm over its 48 partials 7.4 us against 4.3.
// The kernel issues every global load before its first wait and keeps q, k,
// v, the scores and the context in LDS.
//
// MFMA: v_mfma_f32_16x16x4_f32 with the lane map of the few-token GEMM
// (gemm.hip): lane l supplies A row l % 16 and B row (output column) l % 16 at
// k = kb + 4 (l / 16) + e for element e of one float4, and holds output rows
// 4 (l / 16) + i, i = 0..3, of column l % 16.
#include <algorithm>

#include "kernels.hpp"

namespace ebh {

namespace {

typedef float v4f_t __attribute__((ext_vector_type(4)));

constexpr int FEW_NW = 8;          // waves per workgroup
constexpr int FEW_HD = 32;         // head_dim these kernels take
constexpr int FEW_T = FEW_ATTN_MAX_TOKENS;

__device__ __forceinline__ v4f_t ld4(const float* p) { return *reinterpret_cast<const v4f_t*>(p); }

__device__ __forceinline__ v4f_t mfma4(v4f_t a, v4f_t b, v4f_t c) {
#pragma unroll
    for (int e = 0; e < 4; ++e) c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[e], b[e], c, 0, 0, 0);
    return c;
}

// Workgroup (h, third): attention of head h over every sequence, then columns
// [third * H / 3, (third + 1) * H / 3) of that head's share of the output
// projection.  qkv [M, 3H] (the QKV projection with its bias), Wo [H, H];
// partial h goes to Y + h * part_stride.  The three workgroups of a head
// repeat its (small) attention so that the projection's weights are spread
// over three times as many compute units.
__global__ __launch_bounds__(64 * FEW_NW) void attn_out_few_kernel(
    const float* __restrict__ qkv, const float* __restrict__ Wo, const int* __restrict__ cu,
    const int* __restrict__ ntok, int B, int H, float scale, float* __restrict__ Y, int64_t part_stride) {
    constexpr int QS = 3 * FEW_HD + 4;   // q | k | v row stride in LDS (floats)
    constexpr int PS = FEW_T + 1;        // score row stride
    constexpr int CS = FEW_HD + 4;       // context row stride
    __shared__ __attribute__((aligned(16))) float qkv_s[FEW_T * QS];
    __shared__ __attribute__((aligned(16))) float ps[FEW_T * PS];
    __shared__ __attribute__((aligned(16))) float ctx_s[FEW_T * CS];
    __shared__ float inv_s[FEW_T];
    __shared__ int seq_start[FEW_T], seq_len[FEW_T];

    const int h = blockIdx.x, third = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int M = min(*ntok, FEW_T);
    const int r = lane & 15, q = lane >> 4;

    // Every global load goes out before the first wait: this wave's 16
    // output-projection rows (columns h*32 .. +31), the head's q | k | v rows
    // and the sequence bounds.
    const int n0 = third * (H / 3) + wave * 16;
    v4f_t wf[2];
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) wf[s2] = ld4(Wo + (int64_t)(n0 + r) * H + h * FEW_HD + 16 * s2 + 4 * q);
    constexpr int PIECES = FEW_T * 3 * FEW_HD / 4;    // float4 of q | k | v for FEW_T rows
    constexpr int PPT = PIECES / (64 * FEW_NW);
    v4f_t pv[PPT];
#pragma unroll
    for (int k = 0; k < PPT; ++k) {
        const int e = tid + 64 * FEW_NW * k, t = e / (3 * FEW_HD / 4), c4 = e % (3 * FEW_HD / 4);
        const int part = c4 / (FEW_HD / 4), d4 = c4 % (FEW_HD / 4);
        if (t < M) pv[k] = ld4(qkv + (int64_t)t * 3 * H + part * H + h * FEW_HD + 4 * d4);
    }
    int cb0 = 0, cb1 = 0;
    if (tid < B) {
        cb0 = cu[tid];
        cb1 = cu[tid + 1];
    }
#pragma unroll
    for (int k = 0; k < PPT; ++k) {
        const int e = tid + 64 * FEW_NW * k, t = e / (3 * FEW_HD / 4), c4 = e % (3 * FEW_HD / 4);
        if (t < M) *reinterpret_cast<v4f_t*>(qkv_s + t * QS + 4 * c4) = pv[k];
    }
    // Sequence of each packed token (B <= 64 <= the workgroup's threads).
    if (tid < B)
        for (int t = cb0; t < min(cb1, M); ++t) {
            seq_start[t] = cb0;
            seq_len[t] = cb1 - cb0;
        }
    __syncthreads();

    // Scores of query t against key jj of its own sequence, scaled after q.k
    // (src/lib.rs:713-714); keys past the sequence are masked out below.
    for (int e = tid; e < FEW_T * FEW_T; e += 64 * FEW_NW) {
        const int t = e / FEW_T, jj = e % FEW_T;
        if (t >= M || jj >= seq_len[t]) continue;
        const float* qr = qkv_s + t * QS;
        const float* kr = qkv_s + (seq_start[t] + jj) * QS + FEW_HD;
        float d = 0.0f;
#pragma unroll
        for (int c = 0; c < FEW_HD; c += 4) {
            const v4f_t a = ld4(qr + c), b = ld4(kr + c);
            d = fmaf(a[0], b[0], d);
            d = fmaf(a[1], b[1], d);
            d = fmaf(a[2], b[2], d);
            d = fmaf(a[3], b[3], d);
        }
        ps[t * PS + jj] = d * scale;
    }
    __syncthreads();
    // Row softmax (src/lib.rs:851-870): wave per query row, lane per key.
    for (int t = wave; t < M; t += FEW_NW) {
        const int len = seq_len[t];
        const float v = lane < len ? ps[t * PS + lane] : -INFINITY;
        float m = v;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
        const float p = lane < len ? fast_exp(v - m) : 0.0f;
        float l = p;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) l += __shfl_xor(l, o);
        if (lane < len) ps[t * PS + lane] = p;
        if (lane == 0) inv_s[t] = 1.0f / l;
    }
    __syncthreads();
    // Context = P . V / row sum (src/lib.rs:723); rows past M are zero.
    for (int e = tid; e < FEW_T * FEW_HD; e += 64 * FEW_NW) {
        const int t = e / FEW_HD, d = e % FEW_HD;
        float c = 0.0f;
        if (t < M) {
            const int len = seq_len[t];
            const float* vr = qkv_s + seq_start[t] * QS + 2 * FEW_HD + d;
            for (int jj = 0; jj < len; ++jj) c = fmaf(ps[t * PS + jj], vr[jj * QS], c);
            c *= inv_s[t];
        }
        ctx_s[t * CS + d] = c;
    }
    __syncthreads();

    // Wave w: output columns n0 .. n0 + 15 of partial h.
    float* P = Y + h * part_stride;
    for (int m0 = 0; m0 < M; m0 += 16) {
        v4f_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) acc = mfma4(ld4(ctx_s + (m0 + r) * CS + 16 * s2 + 4 * q), wf[s2], acc);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = m0 + 4 * q + i;
            if (row < M) P[(int64_t)row * H + n0 + r] = acc[i];
        }
    }
}

}  // namespace

bool few_attn_fits(int T_max, int H, int nh) {
    return T_max > 0 && T_max <= FEW_T && H == 3 * 16 * FEW_NW && nh * FEW_HD == H;
}

// H = 384: each wave of a workgroup takes 16 of its 128 output columns.
hipError_t launch_attn_out_few(const float* qkv, const float* wo, const int* cu, const int* ntok, int B,
                              int T_max, int H, int nh, float scale, float* Y, int64_t part_stride,
                              hipStream_t s) {
    if (!few_attn_fits(T_max, H, nh) || B <= 0 || B > FEW_T || part_stride < (int64_t)T_max * H)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(attn_out_few_kernel, dim3(nh, 3), dim3(64 * FEW_NW), 0, s, qkv, wo, cu, ntok, B, H, scale,
                       Y, part_stride);
    return hipGetLastError();
}

}  // namespace ebh
