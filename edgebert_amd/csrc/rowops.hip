// rowops.hip -- HBM-bound row kernels of the encoder path: token packing,
// embedding gather + LayerNorm, LayerNorm, masked mean pool + L2 normalise.
//
// One wave64 owns one row of H floats (NC = ceil(H/64) values per lane,
// element c*64 + lane so every load/store instruction covers 256 contiguous
// bytes); mean and variance are two wave reductions over register-resident
// values, so each row is read once and written once.
#include <algorithm>

#include "kernels.hpp"

namespace ebh {

// ---------------------------------------------------------------------------
// Token packing.  The reference runs every padded position through the
// encoder and only drops pads in the pooling (src/lib.rs:993-1010); a pad
// never influences a real token (it is a masked key, and every other op is
// row-wise), so only mask == 1 tokens are packed, keeping their original
// positions for the position embedding.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void pack_count_kernel(const int* __restrict__ mask, int S,
                                                         int* __restrict__ counts) {
    __shared__ int part[4];
    const int b = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int n = 0;
    for (int s0 = 0; s0 < S; s0 += 256) {
        const int s = s0 + tid;
        const bool on = s < S && mask[(int64_t)b * S + s] != 0;
        const unsigned long long bal = __ballot(on);
        n += __popcll(bal);
    }
    if (lane == 0) part[wave] = n;
    __syncthreads();
    if (tid == 0) counts[b] = part[0] + part[1] + part[2] + part[3];
}

constexpr int ORDER_BINS = 1024;   // length bins of the longest-first order

// Exclusive prefix sum over the 1024 threads of a workgroup (thread order),
// and the total: an inclusive scan within each wave by lane shuffles, then
// the waves' totals added in wave order.  Two barriers; `wsum` holds 16 ints
// of LDS.  Every thread of the workgroup must call it.
__device__ __forceinline__ int block_excl_scan_1024(int v, int* wsum, int& total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int incl = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(incl, o);
        if (lane >= o) incl += y;
    }
    if (lane == 63) wsum[wave] = incl;
    __syncthreads();
    int before = 0, tot = 0;
#pragma unroll
    for (int w = 0; w < 16; ++w) {
        const int c = wsum[w];
        before += w < wave ? c : 0;
        tot += c;
    }
    __syncthreads();   // wsum may be reused
    total = tot;
    return before + incl - v;
}

// order[0..B): the sequences by decreasing length (counts, clamped to
// ORDER_BINS - 1; ties in any order), a counting sort by the 1024 threads of
// one workgroup.  Thread t takes bin 1023 - t, so the scan runs from the
// longest length down and a bin's exclusive value is its first slot.
__device__ __forceinline__ void order_by_length(const int* counts, int B, int* next, int* wsum,
                                                int* __restrict__ order) {
    static_assert(ORDER_BINS == 1024, "one bin per thread");
    const int tid = threadIdx.x;
    next[tid] = 0;
    __syncthreads();
    for (int b = tid; b < B; b += 1024) atomicAdd(&next[min(counts[b], ORDER_BINS - 1)], 1);
    __syncthreads();
    int total;
    const int first = block_excl_scan_1024(next[ORDER_BINS - 1 - tid], wsum, total);
    next[ORDER_BINS - 1 - tid] = first;   // each thread rewrites only its own bin
    __syncthreads();
    for (int b = tid; b < B; b += 1024) order[atomicAdd(&next[min(counts[b], ORDER_BINS - 1)], 1)] = b;
}

// Exclusive scan of counts[0..B) -> cu[0..B], n_tokens = cu[B]; one workgroup.
// With `order`, also the sequences by decreasing length (a counting sort over
// the lengths, clamped to ORDER_BINS - 1; ties in any order): the attention
// grid walks them longest first, so that the long sequences' workgroups start
// first and the short ones fill in around them.
__global__ __launch_bounds__(1024) void pack_scan_kernel(const int* __restrict__ counts, int B,
                                                         int* __restrict__ cu,
                                                         int* __restrict__ n_tokens,
                                                         int* __restrict__ order) {
    __shared__ int wsum[16];
    __shared__ int next[ORDER_BINS];
    const int tid = threadIdx.x;
    const int per = (B + 1023) / 1024;
    const int lo = min(B, tid * per), hi = min(B, lo + per);
    int local = 0;
    for (int i = lo; i < hi; ++i) local += counts[i];
    int total;
    int run = block_excl_scan_1024(local, wsum, total);   // exclusive prefix of this thread's segment
    for (int i = lo; i < hi; ++i) {
        cu[i] = run;
        run += counts[i];
    }
    if (tid == 1023) {
        cu[B] = total;
        *n_tokens = total;
    }
    if (!order) return;   // uniform over the workgroup
    order_by_length(counts, B, next, wsum, order);
}

__global__ __launch_bounds__(256) void pack_scatter_kernel(const int* __restrict__ ids,
                                                           const int* __restrict__ mask, int S,
                                                           const int* __restrict__ cu,
                                                           int* __restrict__ tok_id,
                                                           int* __restrict__ tok_pos) {
    __shared__ int part[4];
    const int b = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int base = cu[b];
    for (int s0 = 0; s0 < S; s0 += 256) {
        const int s = s0 + tid;
        const bool on = s < S && mask[(int64_t)b * S + s] != 0;
        const unsigned long long bal = __ballot(on);
        if (lane == 0) part[wave] = __popcll(bal);
        __syncthreads();
        int before = 0;
        for (int w = 0; w < wave; ++w) before += part[w];
        const int total = part[0] + part[1] + part[2] + part[3];
        const unsigned long long below = lane ? (bal & ((~0ull) >> (64 - lane))) : 0ull;
        if (on) {
            const int dst = base + before + __popcll(below);
            tok_id[dst] = ids[(int64_t)b * S + s];
            tok_pos[dst] = s;
        }
        base += total;
        __syncthreads();
    }
}

// The whole packing in one 1024-thread workgroup, for batches of at most
// PACK1_MAX_POS positions and PACK1_MAX_B sequences (c2, c4: three launches
// made one).  Positions go in rounds of 1024 in order.  Every round's mask
// and ids are loaded first; a ballot per wave and round counts the kept
// tokens, one workgroup scan turns the (round, wave) counts into offsets,
// and each lane adds the kept tokens below it in its wave's ballot, so every
// kept token lands where the three-kernel path puts it.  The thread holding
// position b * S records cu[b], the tokens before it.  The order of the
// sequences by decreasing length is the same counting sort as in
// pack_scan_kernel, over counts held in LDS.  Four barriers before the
// order, three in it.
constexpr int PACK1_MAX_POS = 8192, PACK1_MAX_B = 1024;
__global__ __launch_bounds__(1024) void pack_one_kernel(const int* __restrict__ ids, const int* __restrict__ mask,
                                                        int B, int S, int* __restrict__ counts,
                                                        int* __restrict__ cu, int* __restrict__ n_tokens,
                                                        int* __restrict__ tok_id, int* __restrict__ tok_pos,
                                                        int* __restrict__ order) {
    constexpr int R = PACK1_MAX_POS / 1024;   // rounds of 1024 positions
    __shared__ int wsum[16];
    __shared__ int off_s[16 * R];              // per (round, wave): its count, then the tokens before it
    __shared__ int cu_s[PACK1_MAX_B + 1];
    __shared__ int cnt_s[PACK1_MAX_B];
    __shared__ int next[ORDER_BINS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int P = B * S, nr = (P + 1023) / 1024;
    int mv[R], iv[R];   // every round's mask and id, loaded before the first ranking
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int p = r * 1024 + tid;
        mv[r] = p < P ? mask[p] : 0;
        iv[r] = p < P ? ids[p] : 0;
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
        if (r < nr) {   // uniform
            const int c = __popcll(__ballot(mv[r] != 0));
            if (lane == 0) off_s[r * 16 + wave] = c;
            __builtin_amdgcn_sched_barrier(0);   // one round's mask live at a time
        }
    for (int b = tid; b <= B; b += 1024) cu_s[b] = 0;   // S == 0: every sequence empty
    __syncthreads();
    // The (round, wave) counts in round-major order, scanned: thread i takes entry i.
    int total;
    const int pre = block_excl_scan_1024(tid < 16 * nr ? off_s[tid] : 0, wsum, total);
    if (tid < 16 * nr) off_s[tid] = pre;   // each thread rewrites only its own entry
    __syncthreads();
    // The ballots are taken again below (one instruction each) rather than
    // the counting pass's sixteen 64-bit masks being held across the scan.
#pragma unroll
    for (int r = 0; r < R; ++r) asm volatile("" : "+v"(mv[r]));
#pragma unroll
    for (int r = 0; r < R; ++r)
        if (r < nr) {
            const int p = r * 1024 + tid;
            const bool on = mv[r] != 0;
            const unsigned long long bal = __ballot(on);
            const unsigned long long below = lane ? (bal & ((~0ull) >> (64 - lane))) : 0ull;
            const int dst = off_s[r * 16 + wave] + __popcll(below);
            if (p < P && p % S == 0) cu_s[p / S] = dst;
            if (on) {
                tok_id[dst] = iv[r];
                tok_pos[dst] = p % S;
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    if (tid == 0) {
        cu_s[B] = total;
        *n_tokens = total;
    }
    __syncthreads();
    for (int b = tid; b <= B; b += 1024) cu[b] = cu_s[b];
    for (int b = tid; b < B; b += 1024) {
        const int n = cu_s[b + 1] - cu_s[b];
        cnt_s[b] = n;
        counts[b] = n;
    }
    if (!order) return;   // uniform over the workgroup
    __syncthreads();
    order_by_length(cnt_s, B, next, wsum, order);
}

hipError_t launch_pack(const int* ids, const int* mask, int B, int S, int* counts, int* cu,
                       int* n_tokens, int* tok_id, int* tok_pos, hipStream_t s, int* order) {
    if (B <= 0) return hipSuccess;
    if (B <= PACK1_MAX_B && (int64_t)B * S <= PACK1_MAX_POS) {
        hipLaunchKernelGGL(pack_one_kernel, dim3(1), dim3(1024), 0, s, ids, mask, B, S, counts, cu, n_tokens,
                           tok_id, tok_pos, order);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(pack_count_kernel, dim3(B), dim3(256), 0, s, mask, S, counts);
    hipLaunchKernelGGL(pack_scan_kernel, dim3(1), dim3(1024), 0, s, counts, B, cu, n_tokens, order);
    hipLaunchKernelGGL(pack_scatter_kernel, dim3(B), dim3(256), 0, s, ids, mask, S, cu, tok_id,
                       tok_pos);
    return hipGetLastError();
}

// n 32-bit words of p set to 0: a kernel, not hipMemsetAsync, so that a caller
// capturing its stream into a HIP graph records a kernel node.
__global__ __launch_bounds__(256) void zero_words_kernel(uint32_t* __restrict__ p, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) p[i] = 0u;
}

hipError_t launch_zero_words(void* p, int64_t n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    const int64_t blocks = std::min<int64_t>((n + 255) / 256, 1024);
    hipLaunchKernelGGL(zero_words_kernel, dim3((unsigned)blocks), dim3(256), 0, s, static_cast<uint32_t*>(p), n);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// LayerNorm on a register-resident row (apply_layer_norm_3d, src/lib.rs:980-991):
// mean, population variance, inv_std = 1/sqrt(var + eps),
// y = (x - mean) * inv_std * gamma + beta.
// ---------------------------------------------------------------------------
template <int NC>
__device__ __forceinline__ void ln_row(float (&v)[NC], int lane, int H, const float* g,
                                       const float* b, float eps, float* y,
                                       uint16_t* y16 = nullptr) {
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < NC; ++c) s += v[c];
    const float mean = wave_sum(s) / (float)H;
    float ss = 0.0f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int i = c * 64 + lane;
        const float d = v[c] - mean;
        if (i < H) ss += d * d;
    }
    const float var = wave_sum(ss) / (float)H;
    const float inv_std = 1.0f / sqrtf(var + eps);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int i = c * 64 + lane;
        if (i < H) {
            const float o = (v[c] - mean) * inv_std * g[i] + b[i];
            if (y) y[i] = o;
            if (y16) y16[i] = f32_to_bf16_rne(o);  // bf16 copy for bf16 GEMM inputs
        }
    }
}

template <int NC>
__global__ __launch_bounds__(256) void layernorm_kernel(const float* x, float* y,
                                                        const float* __restrict__ g,
                                                        const float* __restrict__ bta,
                                                        int rows_max, const int* rows_dev, int H,
                                                        float eps) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int rows = rows_dev ? *rows_dev : rows_max;
    if (row >= rows) return;
    const float* xr = x + (int64_t)row * H;
    float v[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int i = c * 64 + lane;
        v[c] = i < H ? xr[i] : 0.0f;
    }
    ln_row<NC>(v, lane, H, g, bta, eps, y + (int64_t)row * H);
}

// Residual block end (BertLayer::forward, src/lib.rs:672-674 and 677-679):
// x = LayerNorm((y + bias) + x), where y is the projection without its bias
// (the GEMM writes it raw), added in the reference's order: the Linear's bias
// first (src/lib.rs:733, 747), then the block input.  In place on x.
template <int NC>
__global__ __launch_bounds__(256) void add_layernorm_kernel(const float* __restrict__ y,
                                                            const float* __restrict__ bias,
                                                            float* x, const float* __restrict__ g,
                                                            const float* __restrict__ bta,
                                                            int rows_max, const int* rows_dev,
                                                            int H, float eps, uint16_t* x16,
                                                            int nparts, int64_t part_stride) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int rows = rows_dev ? *rows_dev : rows_max;
    if (row >= rows) return;
    const float* yr = y + (int64_t)row * H;
    float* xr = x + (int64_t)row * H;
    float v[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int i = c * 64 + lane;
        float yv = 0.0f;
        if (i < H) {
            yv = yr[i];
            for (int q = 1; q < nparts; ++q) yv += yr[q * part_stride + i];
        }
        v[c] = i < H ? (yv + bias[i]) + xr[i] : 0.0f;
    }
    ln_row<NC>(v, lane, H, g, bta, eps, xr, x16 ? x16 + (int64_t)row * H : nullptr);
}

// Embeddings (Model::forward, src/lib.rs:628-661): word[id] + position[pos] +
// token_type[0], then the embeddings LayerNorm.  An id outside [0, V) reads
// row 0 and raises the error flag (the reference panics on such an id).
template <int NC>
__global__ __launch_bounds__(256) void embed_ln_kernel(
    const int* __restrict__ tok_id, const int* __restrict__ tok_pos,
    const int* __restrict__ n_tokens, const float* __restrict__ word,
    const float* __restrict__ pos, const float* __restrict__ type0, const float* __restrict__ g,
    const float* __restrict__ bta, int V, int H, float eps, float* __restrict__ x,
    int* __restrict__ err, uint16_t* __restrict__ x16) {
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (t >= *n_tokens) return;
    int id = tok_id[t];
    if (id < 0 || id >= V) {
        if (lane == 0) atomicOr(err, 1);
        id = 0;
    }
    const float* wr = word + (int64_t)id * H;
    const float* pr = pos + (int64_t)tok_pos[t] * H;
    float v[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int i = c * 64 + lane;
        v[c] = i < H ? (wr[i] + pr[i]) + type0[i] : 0.0f;
    }
    ln_row<NC>(v, lane, H, g, bta, eps, x ? x + (int64_t)t * H : nullptr, x16 ? x16 + (int64_t)t * H : nullptr);
}

// ---------------------------------------------------------------------------
// float4 variants of the LayerNorm row kernels: LPR lanes per row (16, 32 or
// 64, so one wave holds 64 / LPR rows), each lane NV float4 at elements
// 4 * (c * LPR + sub) .. +3, H == 4 * NV * LPR.  Every global access is a
// 16-byte lane access (a wave instruction moves 1 KB), the row stays in
// registers, and mean / variance are reductions over the row's lane group.
// ---------------------------------------------------------------------------
template <int LPR>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int o = LPR / 2; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

template <int NV, int LPR>
__device__ __forceinline__ void ln_row4(float4 (&v)[NV], int sub, int H, const float* g,
                                        const float* b, float eps, float* y, uint16_t* y16) {
    // gamma / beta are loaded first, so their memory round trip overlaps the
    // row reductions instead of following them.
    float4 g4[NV], b4[NV];
#pragma unroll
    for (int c = 0; c < NV; ++c) {
        g4[c] = *reinterpret_cast<const float4*>(g + 4 * (c * LPR + sub));
        b4[c] = *reinterpret_cast<const float4*>(b + 4 * (c * LPR + sub));
    }
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < NV; ++c) s += (v[c].x + v[c].y) + (v[c].z + v[c].w);
    const float mean = group_sum<LPR>(s) / (float)H;
    float ss = 0.0f;
#pragma unroll
    for (int c = 0; c < NV; ++c) {
        const float dx = v[c].x - mean, dy = v[c].y - mean, dz = v[c].z - mean, dw = v[c].w - mean;
        ss += (dx * dx + dy * dy) + (dz * dz + dw * dw);
    }
    const float var = group_sum<LPR>(ss) / (float)H;
    const float inv_std = 1.0f / sqrtf(var + eps);
#pragma unroll
    for (int c = 0; c < NV; ++c) {
        const int i = 4 * (c * LPR + sub);
        float4 o;
        o.x = (v[c].x - mean) * inv_std * g4[c].x + b4[c].x;
        o.y = (v[c].y - mean) * inv_std * g4[c].y + b4[c].y;
        o.z = (v[c].z - mean) * inv_std * g4[c].z + b4[c].z;
        o.w = (v[c].w - mean) * inv_std * g4[c].w + b4[c].w;
        if (y) *reinterpret_cast<float4*>(y + i) = o;
        if (y16) {
            uint2 h;
            h.x = (uint32_t)f32_to_bf16_rne(o.x) | ((uint32_t)f32_to_bf16_rne(o.y) << 16);
            h.y = (uint32_t)f32_to_bf16_rne(o.z) | ((uint32_t)f32_to_bf16_rne(o.w) << 16);
            *reinterpret_cast<uint2*>(y16 + i) = h;
        }
    }
}

// x = LayerNorm((y + bias) + x) on float4 rows.  PB == 0: y is one product;
// otherwise y holds nparts split-K partials part_stride floats apart, added in
// order, with their loads going out PB partials at a time (an index past the
// last partial re-reads the last one and is not added), so a row waits for
// one memory round trip per PB partials rather than one per partial.
template <int NV, int LPR, int PB, int BS = 256>
__device__ __forceinline__ void add_layernorm4_row(const float* __restrict__ y, const float* __restrict__ bias,
                                                   float* x, const float* __restrict__ g,
                                                   const float* __restrict__ bta, int rows_max,
                                                   const int* rows_dev, int H, float eps, uint16_t* x16,
                                                   int nparts, int64_t part_stride) {
    constexpr int RPB = BS / LPR;                 // rows per workgroup
    const int row = blockIdx.x * RPB + threadIdx.x / LPR, sub = threadIdx.x % LPR;
    const int rows = rows_dev ? *rows_dev : rows_max;
    if (row >= rows) return;
    const float* yr = y + (int64_t)row * H;
    float* xr = x + (int64_t)row * H;
    float4 a[NV], bb[NV], r[NV];
#pragma unroll
    for (int c = 0; c < NV; ++c) {
        const int i = 4 * (c * LPR + sub);
        a[c] = *reinterpret_cast<const float4*>(yr + i);
        bb[c] = *reinterpret_cast<const float4*>(bias + i);
        r[c] = *reinterpret_cast<const float4*>(xr + i);
    }
    if constexpr (PB > 0) {
        for (int q0 = 1; q0 < nparts; q0 += PB) {
            float4 pq[PB][NV];
#pragma unroll
            for (int k = 0; k < PB; ++k) {
                const float* pr = yr + (int64_t)min(q0 + k, nparts - 1) * part_stride;
#pragma unroll
                for (int c = 0; c < NV; ++c) pq[k][c] = *reinterpret_cast<const float4*>(pr + 4 * (c * LPR + sub));
            }
#pragma unroll
            for (int k = 0; k < PB; ++k)
                if (q0 + k < nparts) {
#pragma unroll
                    for (int c = 0; c < NV; ++c) {
                        a[c].x += pq[k][c].x; a[c].y += pq[k][c].y; a[c].z += pq[k][c].z; a[c].w += pq[k][c].w;
                    }
                }
        }
    }
    float4 v[NV];
#pragma unroll
    for (int c = 0; c < NV; ++c)
        v[c] = make_float4((a[c].x + bb[c].x) + r[c].x, (a[c].y + bb[c].y) + r[c].y,
                           (a[c].z + bb[c].z) + r[c].z, (a[c].w + bb[c].w) + r[c].w);
    ln_row4<NV, LPR>(v, sub, H, g, bta, eps, xr, x16 ? x16 + (int64_t)row * H : nullptr);
}

#define EBH_ADD_LN4_KERNEL(NAME, PB)                                                                    \
    template <int NV, int LPR>                                                                          \
    __global__ __launch_bounds__(256) void NAME(const float* __restrict__ y, const float* __restrict__ bias, \
                                                float* x, const float* __restrict__ g,                  \
                                                const float* __restrict__ bta, int rows_max,            \
                                                const int* rows_dev, int H, float eps, uint16_t* x16,   \
                                                int nparts, int64_t part_stride) {                      \
        add_layernorm4_row<NV, LPR, PB>(y, bias, x, g, bta, rows_max, rows_dev, H, eps, x16, nparts,    \
                                        part_stride);                                                   \
    }
EBH_ADD_LN4_KERNEL(add_layernorm4_kernel, 0)       // one product
EBH_ADD_LN4_KERNEL(add_layernorm4_p4_kernel, 4)    // split-K partials
// More than 8 partials at a handful of rows (the few-token attention's one
// per head): one row per workgroup (LPR threads), the partials read 16 at a
// time (4 where the row takes more than 3 float4 per lane, for registers).  A
// compute unit streams only about 10 bytes per clock from beyond its cache,
// so the rows' partials are spread over as many of them as there are rows.
template <int NV, int LPR>
__global__ __launch_bounds__(LPR) void add_layernorm4_row1_kernel(
    const float* __restrict__ y, const float* __restrict__ bias, float* x, const float* __restrict__ g,
    const float* __restrict__ bta, int rows_max, const int* rows_dev, int H, float eps, uint16_t* x16, int nparts,
    int64_t part_stride) {
    add_layernorm4_row<NV, LPR, (NV <= 3 ? 16 : 4), LPR>(y, bias, x, g, bta, rows_max, rows_dev, H, eps, x16,
                                                           nparts, part_stride);
}
#undef EBH_ADD_LN4_KERNEL

// The same with the projection y stored as bf16 (bf16 models write the
// attention-output and FFN-down products in bf16); the sum, statistics and
// output stay fp32.
// R16 == false: the residual stream x is fp32 (read, then overwritten with
// the result, with an optional bf16 copy in x16).  R16: the residual stream is
// bf16 (bf16 models): x16 is read as the residual and overwritten with the
// bf16 result; x is not used.  Either way the sums and statistics are fp32.
template <int NV, int LPR, bool R16>
__device__ __forceinline__ void add_layernorm4_y16_row(const uint16_t* __restrict__ y, const float* __restrict__ bias,
                                                       float* x, const float* __restrict__ g,
                                                       const float* __restrict__ bta, int rows_max,
                                                       const int* rows_dev, int H, float eps, uint16_t* x16) {
    constexpr int RPB = 256 / LPR;
    const int row = blockIdx.x * RPB + threadIdx.x / LPR, sub = threadIdx.x % LPR;
    const int rows = rows_dev ? *rows_dev : rows_max;
    if (row >= rows) return;
    const uint16_t* yr = y + (int64_t)row * H;
    float* xr = R16 ? nullptr : x + (int64_t)row * H;
    uint16_t* x16r = x16 ? x16 + (int64_t)row * H : nullptr;
    float4 v[NV];
#pragma unroll
    for (int c = 0; c < NV; ++c) {
        const int i = 4 * (c * LPR + sub);
        const uint2 a = *reinterpret_cast<const uint2*>(yr + i);
        const float4 bb = *reinterpret_cast<const float4*>(bias + i);
        float4 r;
        if constexpr (R16) {
            const uint2 h = *reinterpret_cast<const uint2*>(x16r + i);
            r = make_float4(__uint_as_float(h.x << 16), __uint_as_float(h.x & 0xFFFF0000u),
                            __uint_as_float(h.y << 16), __uint_as_float(h.y & 0xFFFF0000u));
        } else {
            r = *reinterpret_cast<const float4*>(xr + i);
        }
        const float a0 = __uint_as_float(a.x << 16), a1 = __uint_as_float(a.x & 0xFFFF0000u);
        const float a2 = __uint_as_float(a.y << 16), a3 = __uint_as_float(a.y & 0xFFFF0000u);
        v[c] = make_float4((a0 + bb.x) + r.x, (a1 + bb.y) + r.y, (a2 + bb.z) + r.z, (a3 + bb.w) + r.w);
    }
    ln_row4<NV, LPR>(v, sub, H, g, bta, eps, xr, x16r);
}

#define EBH_ADD_LN4_Y16_KERNEL(NAME, R16)                                                                \
    template <int NV, int LPR>                                                                           \
    __global__ __launch_bounds__(256) void NAME(const uint16_t* __restrict__ y, const float* __restrict__ bias, \
                                                float* x, const float* __restrict__ g,                   \
                                                const float* __restrict__ bta, int rows_max,             \
                                                const int* rows_dev, int H, float eps, uint16_t* x16) {  \
        add_layernorm4_y16_row<NV, LPR, R16>(y, bias, x, g, bta, rows_max, rows_dev, H, eps, x16);      \
    }
EBH_ADD_LN4_Y16_KERNEL(add_layernorm4_y16_kernel, false)   // fp32 residual stream
EBH_ADD_LN4_Y16_KERNEL(add_layernorm4_b16_kernel, true)    // bf16 residual stream
#undef EBH_ADD_LN4_Y16_KERNEL

template <int NV, int LPR>
__global__ __launch_bounds__(256) void embed_ln4_kernel(
    const int* __restrict__ tok_id, const int* __restrict__ tok_pos,
    const int* __restrict__ n_tokens, const float* __restrict__ word,
    const float* __restrict__ pos, const float* __restrict__ type0, const float* __restrict__ g,
    const float* __restrict__ bta, int V, int H, float eps, float* __restrict__ x,
    int* __restrict__ err, uint16_t* __restrict__ x16) {
    constexpr int RPB = 256 / LPR;
    const int t = blockIdx.x * RPB + threadIdx.x / LPR, sub = threadIdx.x % LPR;
    if (t >= *n_tokens) return;
    int id = tok_id[t];
    if (id < 0 || id >= V) {
        if (sub == 0) atomicOr(err, 1);
        id = 0;
    }
    const float* wr = word + (int64_t)id * H;
    const float* pr = pos + (int64_t)tok_pos[t] * H;
    float4 v[NV];
#pragma unroll
    for (int c = 0; c < NV; ++c) {
        const int i = 4 * (c * LPR + sub);
        const float4 a = *reinterpret_cast<const float4*>(wr + i);
        const float4 p4 = *reinterpret_cast<const float4*>(pr + i);
        const float4 ty = *reinterpret_cast<const float4*>(type0 + i);
        v[c] = make_float4((a.x + p4.x) + ty.x, (a.y + p4.y) + ty.y, (a.z + p4.z) + ty.z, (a.w + p4.w) + ty.w);
    }
    ln_row4<NV, LPR>(v, sub, H, g, bta, eps, x ? x + (int64_t)t * H : nullptr,
                     x16 ? x16 + (int64_t)t * H : nullptr);
}

// The bf16-residual block end of bf16 models with 16-byte lane accesses:
// LPR lanes per row, each lane NV8 chunks of 8 consecutive elements at
// 8 * (c * LPR + sub) .. +7 (H == 8 * NV8 * LPR), so the bf16 product, the
// bf16 residual and the bf16 result move as uint4 (a wave instruction moves
// 1 KB).  x16 = bf16(LayerNorm((y + bias) + x16)), sums and statistics fp32.
// Each lane group takes RPG rows (rows g, g + RPB, ... of the workgroup's
// block, so every step of the workgroup covers RPB consecutive rows): bias,
// gamma and beta are loaded once for all of them (they are 72 floats a lane,
// 3x the row's own bytes, and would otherwise load again per row through the
// CU's load path), and the next row's product and residual are loaded before
// the current row's sums.
constexpr int LN8_RPG = 4;

template <int NV8, int LPR>
__global__ __launch_bounds__(256) void add_layernorm8_b16_kernel(const uint16_t* __restrict__ y,
                                                                 const float* __restrict__ bias,
                                                                 uint16_t* x16, const float* __restrict__ g,
                                                                 const float* __restrict__ bta, int rows_max,
                                                                 const int* rows_dev, int H, float eps) {
    constexpr int RPB = 256 / LPR;
    const int grp = threadIdx.x / LPR, sub = threadIdx.x % LPR;
    const int row0 = blockIdx.x * RPB * LN8_RPG + grp;
    const int rows = rows_dev ? *rows_dev : rows_max;
    if (row0 >= rows) return;
    float4 bb[NV8][2], g4[NV8][2], b4[NV8][2];
#pragma unroll
    for (int c = 0; c < NV8; ++c) {
        const int i = 8 * (c * LPR + sub);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            bb[c][h] = *reinterpret_cast<const float4*>(bias + i + 4 * h);
            g4[c][h] = *reinterpret_cast<const float4*>(g + i + 4 * h);
            b4[c][h] = *reinterpret_cast<const float4*>(bta + i + 4 * h);
        }
    }
    auto lo = [](uint32_t w) { return __uint_as_float(w << 16); };
    auto hi = [](uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); };
    uint4 ya[NV8], xa[NV8];
    auto load_row = [&](int row) __attribute__((always_inline)) {
#pragma unroll
        for (int c = 0; c < NV8; ++c) {
            const int i = 8 * (c * LPR + sub);
            ya[c] = *reinterpret_cast<const uint4*>(y + (int64_t)row * H + i);
            xa[c] = *reinterpret_cast<const uint4*>(x16 + (int64_t)row * H + i);
        }
    };
    load_row(row0);
#pragma unroll
    for (int r = 0; r < LN8_RPG; ++r) {
        const int row = row0 + r * RPB;
        if (row >= rows) break;  // uniform over the row's lane group
        float v[NV8][8];
        float s = 0.0f;
#pragma unroll
        for (int c = 0; c < NV8; ++c) {
            const uint32_t yw[4] = {ya[c].x, ya[c].y, ya[c].z, ya[c].w};
            const uint32_t xw[4] = {xa[c].x, xa[c].y, xa[c].z, xa[c].w};
            const float bv[8] = {bb[c][0].x, bb[c][0].y, bb[c][0].z, bb[c][0].w,
                                 bb[c][1].x, bb[c][1].y, bb[c][1].z, bb[c][1].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v[c][2 * e] = (lo(yw[e]) + bv[2 * e]) + lo(xw[e]);
                v[c][2 * e + 1] = (hi(yw[e]) + bv[2 * e + 1]) + hi(xw[e]);
            }
#pragma unroll
            for (int e = 0; e < 8; e += 2) s += v[c][e] + v[c][e + 1];
        }
        if (r + 1 < LN8_RPG && row + RPB < rows) load_row(row + RPB);
        const float mean = group_sum<LPR>(s) / (float)H;
        float ss = 0.0f;
#pragma unroll
        for (int c = 0; c < NV8; ++c)
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
                const float d0 = v[c][e] - mean, d1 = v[c][e + 1] - mean;
                ss += d0 * d0 + d1 * d1;
            }
        const float inv_std = 1.0f / sqrtf(group_sum<LPR>(ss) / (float)H + eps);
        uint16_t* xr = x16 + (int64_t)row * H;
#pragma unroll
        for (int c = 0; c < NV8; ++c) {
            const float gv[8] = {g4[c][0].x, g4[c][0].y, g4[c][0].z, g4[c][0].w,
                                 g4[c][1].x, g4[c][1].y, g4[c][1].z, g4[c][1].w};
            const float tv[8] = {b4[c][0].x, b4[c][0].y, b4[c][0].z, b4[c][0].w,
                                 b4[c][1].x, b4[c][1].y, b4[c][1].z, b4[c][1].w};
            uint32_t o[4];
#pragma unroll
            for (int e = 0; e < 4; ++e)
                o[e] = pack_bf16x2((v[c][2 * e] - mean) * inv_std * gv[2 * e] + tv[2 * e],
                                   (v[c][2 * e + 1] - mean) * inv_std * gv[2 * e + 1] + tv[2 * e + 1]);
            *reinterpret_cast<uint4*>(xr + 8 * (c * LPR + sub)) = make_uint4(o[0], o[1], o[2], o[3]);
        }
    }
}

// (LPR, NV8) for add_layernorm8_b16_kernel, or LPR = 0.
static void row8_shape(int H, int& lpr, int& nv8) {
    lpr = 0;
    nv8 = 0;
    const int cands[3] = {64, 32, 16};
    for (int c : cands)
        if (H % (8 * c) == 0 && H / (8 * c) >= 1 && H / (8 * c) <= 4) { lpr = c; nv8 = H / (8 * c); return; }
}

// (LPR, NV) for a row of H floats, or LPR = 0 when the float4 kernels do not apply.
static void row4_shape(int H, int& lpr, int& nv) {
    lpr = 0;
    nv = 0;
    const int cands[3] = {64, 32, 16};
    for (int c : cands)
        if (H % (4 * c) == 0) {
            const int n = H / (4 * c);
            if (n == 1 || n == 2 || n == 3 || n == 4 || n == 6 || n == 8) { lpr = c; nv = n; return; }
        }
}

bool row4_shape_ok(int H) {
    int lpr, nv;
    row4_shape(H, lpr, nv);
    return lpr != 0;
}

#define EBH_ROW4_DISPATCH(KERNEL, LPR, NV, GRIDF, STREAM, ...)                                 \
    do {                                                                                         \
        bool done_ = false;                                                                      \
        EBH_ROW4_L(KERNEL, 64, LPR, NV, GRIDF, STREAM, __VA_ARGS__)                              \
        EBH_ROW4_L(KERNEL, 32, LPR, NV, GRIDF, STREAM, __VA_ARGS__)                              \
        EBH_ROW4_L(KERNEL, 16, LPR, NV, GRIDF, STREAM, __VA_ARGS__)                              \
        if (!done_) return hipErrorInvalidValue;                                                 \
    } while (0)
#define EBH_ROW4_L(KERNEL, L, LPR, NV, GRIDF, STREAM, ...)                                      \
    if (LPR == L) {                                                                              \
        const dim3 grid_((GRIDF + 256 / L - 1) / (256 / L));                                     \
        switch (NV) {                                                                            \
            case 1: hipLaunchKernelGGL((KERNEL<1, L>), grid_, dim3(256), 0, STREAM, __VA_ARGS__); done_ = true; break; \
            case 2: hipLaunchKernelGGL((KERNEL<2, L>), grid_, dim3(256), 0, STREAM, __VA_ARGS__); done_ = true; break; \
            case 3: hipLaunchKernelGGL((KERNEL<3, L>), grid_, dim3(256), 0, STREAM, __VA_ARGS__); done_ = true; break; \
            case 4: hipLaunchKernelGGL((KERNEL<4, L>), grid_, dim3(256), 0, STREAM, __VA_ARGS__); done_ = true; break; \
            case 6: hipLaunchKernelGGL((KERNEL<6, L>), grid_, dim3(256), 0, STREAM, __VA_ARGS__); done_ = true; break; \
            case 8: hipLaunchKernelGGL((KERNEL<8, L>), grid_, dim3(256), 0, STREAM, __VA_ARGS__); done_ = true; break; \
            default: break;                                                                      \
        }                                                                                        \
    }

static bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

#define EBH_ROW_DISPATCH(KERNEL, H, GRID, STREAM, ...)                                       \
    do {                                                                                     \
        const int nc_ = ((H) + 63) / 64;                                                     \
        if (nc_ <= 4) hipLaunchKernelGGL(KERNEL<4>, GRID, dim3(256), 0, STREAM, __VA_ARGS__);  \
        else if (nc_ <= 6) hipLaunchKernelGGL(KERNEL<6>, GRID, dim3(256), 0, STREAM, __VA_ARGS__); \
        else if (nc_ <= 8) hipLaunchKernelGGL(KERNEL<8>, GRID, dim3(256), 0, STREAM, __VA_ARGS__); \
        else if (nc_ <= 12) hipLaunchKernelGGL(KERNEL<12>, GRID, dim3(256), 0, STREAM, __VA_ARGS__); \
        else if (nc_ <= 16) hipLaunchKernelGGL(KERNEL<16>, GRID, dim3(256), 0, STREAM, __VA_ARGS__); \
        else if (nc_ <= 32) hipLaunchKernelGGL(KERNEL<32>, GRID, dim3(256), 0, STREAM, __VA_ARGS__); \
        else return hipErrorInvalidValue;                                                    \
    } while (0)

hipError_t launch_layernorm(const float* x, float* y, const float* g, const float* b,
                            int rows_max, const int* rows_dev, int H, float eps, hipStream_t s) {
    if (rows_max <= 0) return hipSuccess;
    const dim3 grid((rows_max + 3) / 4);
    EBH_ROW_DISPATCH(layernorm_kernel, H, grid, s, x, y, g, b, rows_max, rows_dev, H, eps);
    return hipGetLastError();
}

hipError_t launch_add_layernorm(const float* y, const float* bias, float* x, const float* g,
                                const float* b, int rows_max, const int* rows_dev, int H, float eps,
                                uint16_t* x16, hipStream_t s, int nparts, int64_t part_stride) {
    if (rows_max <= 0) return hipSuccess;
    if (nparts < 1) nparts = 1;
    int lpr, nv;
    row4_shape(H, lpr, nv);
    if (lpr && al16(y) && al16(bias) && al16(x) && al16(g) && al16(b) && (!x16 || ((uintptr_t)x16 & 7) == 0) &&
        part_stride % 4 == 0) {
        // Partials are read PB at a time, each group one memory round trip.
        if (nparts > 8 && rows_max <= 64) {
#define EBH_LN_ROW1(L)                                                                                  \
            if (lpr == L) {                                                                         \
                switch (nv) {                                                                       \
                    case 1: hipLaunchKernelGGL((add_layernorm4_row1_kernel<1, L>), dim3(rows_max), dim3(L), 0, s, \
                                               y, bias, x, g, b, rows_max, rows_dev, H, eps, x16, nparts, part_stride); break; \
                    case 2: hipLaunchKernelGGL((add_layernorm4_row1_kernel<2, L>), dim3(rows_max), dim3(L), 0, s, \
                                               y, bias, x, g, b, rows_max, rows_dev, H, eps, x16, nparts, part_stride); break; \
                    case 3: hipLaunchKernelGGL((add_layernorm4_row1_kernel<3, L>), dim3(rows_max), dim3(L), 0, s, \
                                               y, bias, x, g, b, rows_max, rows_dev, H, eps, x16, nparts, part_stride); break; \
                    default: return hipErrorInvalidValue;                                           \
                }                                                                                   \
                return hipGetLastError();                                                           \
            }
            EBH_LN_ROW1(64) EBH_LN_ROW1(32) EBH_LN_ROW1(16)
#undef EBH_LN_ROW1
        }
        if (nparts > 1)
            EBH_ROW4_DISPATCH(add_layernorm4_p4_kernel, lpr, nv, rows_max, s, y, bias, x, g, b, rows_max,
                              rows_dev, H, eps, x16, nparts, part_stride);
        else
            EBH_ROW4_DISPATCH(add_layernorm4_kernel, lpr, nv, rows_max, s, y, bias, x, g, b, rows_max,
                              rows_dev, H, eps, x16, nparts, part_stride);
        return hipGetLastError();
    }
    const dim3 grid((rows_max + 3) / 4);
    EBH_ROW_DISPATCH(add_layernorm_kernel, H, grid, s, y, bias, x, g, b, rows_max, rows_dev, H, eps, x16,
                     nparts, part_stride);
    return hipGetLastError();
}

hipError_t launch_add_layernorm_y16(const uint16_t* y, const float* bias, float* x, const float* g,
                                    const float* b, int rows_max, const int* rows_dev, int H, float eps,
                                    uint16_t* x16, hipStream_t s) {
    if (rows_max <= 0) return hipSuccess;
    int lpr, nv;
    row4_shape(H, lpr, nv);
    if (!lpr || ((uintptr_t)y & 7) || !al16(bias) || (x && !al16(x)) || !al16(g) || !al16(b) ||
        (x16 && ((uintptr_t)x16 & 7)) || (!x && !x16))
        return hipErrorInvalidValue;
    int lpr8, nv8;
    row8_shape(H, lpr8, nv8);
    if (!x && lpr8 && ((uintptr_t)y & 15) == 0 && ((uintptr_t)x16 & 15) == 0 && ((uintptr_t)g & 15) == 0 &&
        ((uintptr_t)b & 15) == 0 && ((uintptr_t)bias & 15) == 0) {
        const int rows_per_wg = 256 / lpr8 * LN8_RPG;
        const dim3 grid8((rows_max + rows_per_wg - 1) / rows_per_wg);
#define EBH_LN8(L, N)                                                                                  \
        if (lpr8 == L && nv8 == N) {                                                                    \
            hipLaunchKernelGGL((add_layernorm8_b16_kernel<N, L>), grid8, dim3(256), 0, s, y, bias, x16, g, b, \
                               rows_max, rows_dev, H, eps);                                            \
            return hipGetLastError();                                                                  \
        }
        EBH_LN8(64, 1) EBH_LN8(64, 2) EBH_LN8(64, 3) EBH_LN8(64, 4)
        EBH_LN8(32, 1) EBH_LN8(32, 2) EBH_LN8(32, 3) EBH_LN8(32, 4)
        EBH_LN8(16, 1) EBH_LN8(16, 2) EBH_LN8(16, 3) EBH_LN8(16, 4)
#undef EBH_LN8
    }
    if (x)
        EBH_ROW4_DISPATCH(add_layernorm4_y16_kernel, lpr, nv, rows_max, s, y, bias, x, g, b, rows_max,
                          rows_dev, H, eps, x16);
    else
        EBH_ROW4_DISPATCH(add_layernorm4_b16_kernel, lpr, nv, rows_max, s, y, bias, x, g, b, rows_max,
                          rows_dev, H, eps, x16);
    return hipGetLastError();
}

hipError_t launch_embed_ln(const int* tok_id, const int* tok_pos, const int* n_tokens,
                           int T_max, const float* word, const float* pos, const float* type0,
                           const float* g, const float* b, int V, int H, float eps, float* x,
                           int* err, uint16_t* x16, hipStream_t s) {
    if (T_max <= 0) return hipSuccess;
    int lpr, nv;
    row4_shape(H, lpr, nv);
    if (!x && !x16) return hipErrorInvalidValue;
    if (lpr && al16(word) && al16(pos) && al16(type0) && al16(g) && al16(b) && (!x || al16(x)) &&
        (!x16 || ((uintptr_t)x16 & 7) == 0)) {
        EBH_ROW4_DISPATCH(embed_ln4_kernel, lpr, nv, T_max, s, tok_id, tok_pos, n_tokens, word, pos,
                          type0, g, b, V, H, eps, x, err, x16);
        return hipGetLastError();
    }
    const dim3 grid((T_max + 3) / 4);
    EBH_ROW_DISPATCH(embed_ln_kernel, H, grid, s, tok_id, tok_pos, n_tokens, word, pos, type0, g,
                     b, V, H, eps, x, err, x16);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Token packing and embeddings in one launch for at most 64 positions (B*S <=
// 64: a few short sentences, where four separate launches cost more than
// their work).  A token's packed index is the number of mask == 1 positions
// before it in row-major order, so one wave ballot over the <= 64 mask values
// gives every index, cu_seqlens and the count.  Every workgroup takes the
// ballot itself (the mask is at most 64 ints) and embeds its own rows of the
// packed order; workgroup 0 also writes cu_seqlens, n_tokens, tok_id /
// tok_pos and the id-range flag, as a plain store of "some id out of range",
// so no clear has to be ordered before another workgroup's report.
// ---------------------------------------------------------------------------
template <int NV, int LPR>
__global__ __launch_bounds__(256) void pack_embed_few_kernel(
    const int* __restrict__ ids, const int* __restrict__ mask, int B, int S, int* __restrict__ cu,
    int* __restrict__ n_tokens, int* __restrict__ tok_id, int* __restrict__ tok_pos, int* __restrict__ err,
    const float* __restrict__ word, const float* __restrict__ pos, const float* __restrict__ type0,
    const float* __restrict__ g, const float* __restrict__ bta, int V, int H, float eps, float* __restrict__ x,
    uint16_t* __restrict__ x16) {
    const int T = B * S;                          // <= 64
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const bool in = lane < T;
    const int id_l = in ? ids[lane] : 0;
    const bool on = in && mask[lane] != 0;
    const unsigned long long bal = __ballot(on);
    const unsigned long long bad = __ballot(on && (id_l < 0 || id_l >= V));
    const int n = __popcll(bal);
    if (blockIdx.x == 0 && wave == 0) {
        const unsigned long long below = lane ? (bal & (~0ull >> (64 - lane))) : 0ull;
        if (on) {
            const int k = __popcll(below);
            tok_id[k] = id_l;
            tok_pos[k] = lane % S;
        }
        if (lane < B) cu[lane] = __popcll(bal & ((1ull << (lane * S)) - 1));  // lane * S <= 63
        if (lane == 0) {
            cu[B] = n;
            *n_tokens = n;
            if (bad) *err = 1;                    // sticky: only ebh_synchronize clears it
        }
    }
    constexpr int RPB = 256 / LPR;
    const int r = blockIdx.x * RPB + tid / LPR, sub = tid % LPR;
    if (r >= n) return;
    unsigned long long rest = bal;                // position of the r-th mask == 1 entry
    for (int i = 0; i < r; ++i) rest &= rest - 1;
    const int t = __builtin_ctzll(rest);
    int id = ids[t];
    if (id < 0 || id >= V) id = 0;                // reported through err above
    const float* wr = word + (int64_t)id * H;
    const float* pr = pos + (int64_t)(t % S) * H;
    float4 v[NV];
#pragma unroll
    for (int c = 0; c < NV; ++c) {
        const int i = 4 * (c * LPR + sub);
        const float4 a = *reinterpret_cast<const float4*>(wr + i);
        const float4 p4 = *reinterpret_cast<const float4*>(pr + i);
        const float4 ty = *reinterpret_cast<const float4*>(type0 + i);
        v[c] = make_float4((a.x + p4.x) + ty.x, (a.y + p4.y) + ty.y, (a.z + p4.z) + ty.z, (a.w + p4.w) + ty.w);
    }
    ln_row4<NV, LPR>(v, sub, H, g, bta, eps, x ? x + (int64_t)r * H : nullptr, x16 ? x16 + (int64_t)r * H : nullptr);
}

bool pack_embed_few_fits(int B, int S, int H) {
    int lpr, nv;
    row4_shape(H, lpr, nv);
    return B > 0 && S > 0 && B * S <= 64 && lpr != 0;
}

hipError_t launch_pack_embed_few(const int* ids, const int* mask, int B, int S, int* cu, int* n_tokens,
                                 int* tok_id, int* tok_pos, int* err, const float* word, const float* pos,
                                 const float* type0, const float* g, const float* b, int V, int H, float eps,
                                 float* x, uint16_t* x16, hipStream_t s) {
    int lpr, nv;
    row4_shape(H, lpr, nv);
    if (!pack_embed_few_fits(B, S, H) || (!x && !x16) || !al16(word) || !al16(pos) || !al16(type0) || !al16(g) ||
        !al16(b) || (x && !al16(x)) || (x16 && ((uintptr_t)x16 & 7)))
        return hipErrorInvalidValue;
    EBH_ROW4_DISPATCH(pack_embed_few_kernel, lpr, nv, B * S, s, ids, mask, B, S, cu, n_tokens, tok_id, tok_pos,
                      err, word, pos, type0, g, b, V, H, eps, x, x16);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// mean_pool (src/lib.rs:993-1010) + normalise (src/lib.rs:605-612).
//
// One 512-thread workgroup per sequence (pool_kernel): wave w sums tokens w,
// w+8, w+16, ... with four rows in flight per step (the sum is latency-bound
// otherwise); wave 0 then adds the eight partial rows in wave order, divides
// by max(count, 1) and optionally scales by 1 / max(||x||, 1e-12).
//
// Fewer sequences than CUs, of more than POOL_CR positions, with rows of
// H % 4 == 0 floats, H <= 768 (MiniLM, BERT-base): one sequence per
// workgroup would leave most CUs idle while each waits a dozen dependent
// memory round trips (16 sequences of 256-512 tokens: 18.0 us).  There the
// tokens are summed in chunks of POOL_CR rows, a workgroup per chunk
// (pool_chunk_kernel): thread t of 768 owns float4 column t % F of the row
// (F = H / 4) and sums rows r0 + g, r0 + g + RG, ... of the chunk (g = t / F,
// RG = 768 / F >= 4 row groups), all loaded before the first add; the RG
// sums are added in g order into `part` [B, C, H] (C = ceil(S / POOL_CR)),
// and pool_finish_kernel adds a sequence's chunks in order and finishes as
// above (c4: 18.0 -> ~8 us).
//
// Either way the order of additions depends only on the sequence's own
// length and the batch's shape, so a sequence gives the same vector wherever
// it sits in the batch.  A sequence with no real token among S > 0 positions
// is NaN, as the reference's all -inf softmax row makes it.
// ---------------------------------------------------------------------------
constexpr int POOL_CR = 32;    // rows per chunk
constexpr int POOL_NT = 768;   // threads per chunk workgroup: whole rows of float4 for H = 384 and 768

// Divide by the count, then the optional L2 normalisation, for the float4
// column t < F of sequence b (v = its sum); every thread of the workgroup
// takes part (the norm is a workgroup sum, over waves in order).
__device__ __forceinline__ void pool_finish_row(float4 v, int t, int F, int len, int S, int normalize,
                                                float* __restrict__ out_row, float* wsum) {
    const float count = fmaxf((float)len, 1.0f);
    const bool all_masked = (len == 0 && S > 0);
    v.x = v.x / count; v.y = v.y / count; v.z = v.z / count; v.w = v.w / count;
    if (all_masked) v = make_float4(__builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""));
    float ss = t < F ? (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w) : 0.0f;
    ss = wave_sum(ss);
    const int nw = (int)(blockDim.x >> 6);
    if ((t & 63) == 0) wsum[t >> 6] = ss;
    __syncthreads();
    float tot = wsum[0];
    for (int w = 1; w < nw; ++w) tot += wsum[w];
    if (t < F) {
        if (normalize) {
            const float norm = fmaxf(sqrtf(tot), 1e-12f);
            v.x = v.x / norm; v.y = v.y / norm; v.z = v.z / norm; v.w = v.w / norm;
        }
        reinterpret_cast<float4*>(out_row)[t] = v;
    }
}

// This thread's rows r0 + g, r0 + g + RG, ... below r1 (<= r0 + POOL_CR;
// U >= POOL_CR / RG of them), and their sum in that order from 0.
template <int U>
__device__ __forceinline__ void pool_load(float4 (&v)[U], const float4* __restrict__ xp, int F, int RG, int g,
                                          int r0, int r1) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int r = r0 + g + u * RG;
        v[u] = r < r1 ? xp[(int64_t)r * F] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
}
template <int U>
__device__ __forceinline__ float4 pool_add(const float4 (&v)[U], int RG, int g, int r0, int r1) {
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int u = 0; u < U; ++u)
        if (r0 + g + u * RG < r1) {
            acc.x += v[u].x; acc.y += v[u].y; acc.z += v[u].z; acc.w += v[u].w;
        }
    return acc;
}

// The chunk's sum for float4 column t < F: the row groups' sums in g order.
__device__ __forceinline__ float4 pool_groups(const float4* red, int F, int RG, int t) {
    float4 sum = red[t];
    for (int q = 1; q < RG; ++q) {
        const float4 o = red[q * F + t];
        sum.x += o.x; sum.y += o.y; sum.z += o.z; sum.w += o.w;
    }
    return sum;
}

// One chunk of one sequence: grid (C, B), POOL_NT threads, RG >= POOL_CR / U.
template <int U>
__global__ __launch_bounds__(POOL_NT) void pool_chunk_kernel(const float* __restrict__ x, const int* __restrict__ cu,
                                                             int H, int C, float* __restrict__ part) {
    __shared__ float4 red[POOL_NT];
    const int F = H >> 2, RG = POOL_NT / F;
    const int b = blockIdx.y, ch = blockIdx.x, t = threadIdx.x;
    const int start = cu[b], len = cu[b + 1] - start, r0 = ch * POOL_CR;
    if (r0 >= len) return;   // past the sequence: the finish step skips this chunk
    const int col = t % F, g = t / F;
    const float4* xp = reinterpret_cast<const float4*>(x + (int64_t)start * H) + col;
    const int r1 = g < RG ? min(len, r0 + POOL_CR) : r0;   // idle threads: no rows
    float4 v[U];
    pool_load<U>(v, xp, F, RG, g, r0, r1);
    red[t] = pool_add<U>(v, RG, g, r0, r1);
    __syncthreads();
    if (t < F) reinterpret_cast<float4*>(part + ((int64_t)b * C + ch) * H)[t] = pool_groups(red, F, RG, t);
}

// A sequence's chunk sums added in chunk order, then finished: grid B,
// F rounded up to whole waves.
__global__ __launch_bounds__(POOL_NT) void pool_finish_kernel(const float* __restrict__ part,
                                                              const int* __restrict__ cu, int H, int S,
                                                              int normalize, int C, float* __restrict__ out) {
    __shared__ float wsum[POOL_NT / 64];
    const int F = H >> 2, b = blockIdx.x, t = threadIdx.x;
    const int len = cu[b + 1] - cu[b], nch = (len + POOL_CR - 1) / POOL_CR;
    float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (t < F && nch > 0) {
        const float4* pp = reinterpret_cast<const float4*>(part + (int64_t)b * C * H) + t;
        v = pp[0];
        constexpr int U = 8;
        for (int c0 = 1; c0 < nch; c0 += U) {
            float4 q[U];
#pragma unroll
            for (int u = 0; u < U; ++u)
                q[u] = c0 + u < nch ? pp[(int64_t)(c0 + u) * F] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
            for (int u = 0; u < U; ++u)
                if (c0 + u < nch) {
                    v.x += q[u].x; v.y += q[u].y; v.z += q[u].z; v.w += q[u].w;
                }
        }
    }
    pool_finish_row(v, t, F, len, S, normalize, out + (int64_t)b * H, wsum);
}

// One workgroup of POOL_WAVES waves per sequence (batches of at least as many
// sequences as CUs, one chunk, or other widths).
constexpr int POOL_WAVES = 8;

template <int NC>
__global__ __launch_bounds__(64 * POOL_WAVES) void pool_kernel(const float* __restrict__ x,
                                                               const int* __restrict__ cu, int H,
                                                               int S, int normalize,
                                                               float* __restrict__ out) {
    __shared__ float red[POOL_WAVES - 1][NC * 64];
    const int b = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int start = cu[b], len = cu[b + 1] - start;
    float acc[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) acc[c] = 0.0f;
    constexpr int U = 4;  // rows in flight per wave
    int t = wave;
    for (; t + (U - 1) * POOL_WAVES < len; t += U * POOL_WAVES) {
        float v[U][NC];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const float* xr = x + (int64_t)(start + t + u * POOL_WAVES) * H;
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const int i = c * 64 + lane;
                v[u][c] = i < H ? xr[i] : 0.0f;
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int c = 0; c < NC; ++c) acc[c] += v[u][c];
    }
    for (; t < len; t += POOL_WAVES) {
        const float* xr = x + (int64_t)(start + t) * H;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const int i = c * 64 + lane;
            if (i < H) acc[c] += xr[i];
        }
    }
    if (wave > 0) {
#pragma unroll
        for (int c = 0; c < NC; ++c) red[wave - 1][c * 64 + lane] = acc[c];
    }
    __syncthreads();
    if (wave != 0) return;
    const float count = fmaxf((float)len, 1.0f);
    const bool all_masked = (len == 0 && S > 0);
    float ss = 0.0f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int i = c * 64 + lane;
        float v = acc[c];
#pragma unroll
        for (int w = 0; w < POOL_WAVES - 1; ++w) v += red[w][c * 64 + lane];
        v = v / count;
        if (all_masked) v = __builtin_nanf("");
        acc[c] = v;
        if (i < H) ss += v * v;
    }
    const float norm = normalize ? fmaxf(sqrtf(wave_sum(ss)), 1e-12f) : 1.0f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int i = c * 64 + lane;
        if (i < H) out[(int64_t)b * H + i] = normalize ? acc[c] / norm : acc[c];
    }
}

// Chunks per sequence of the chunked path, 0 where pool_kernel runs: H % 4
// == 0 and at least 4 row groups (H <= 768), so a thread's rows of a chunk
// take at most 8 loads; fewer sequences than CUs, more than one chunk.
static int pool_chunks(int B, int H, int S) {
    const int C = (S + POOL_CR - 1) / POOL_CR;
    return H % 4 == 0 && H / 4 <= POOL_NT / 4 && C > 1 && B < device_cu_count() ? C : 0;
}

int64_t pool_partials_floats(int B, int H, int S) { return (int64_t)B * pool_chunks(B, H, S) * H; }

hipError_t launch_pool(const float* x, const int* cu_seqlens, int B, int H, int S, int normalize,
                       float* partials, float* out, hipStream_t s) {
    if (B <= 0) return hipSuccess;
    const int C = pool_chunks(B, H, S);
    if (C > 0 && al16(x) && al16(out)) {
        const bool u4 = POOL_NT / (H / 4) >= POOL_CR / 4;   // 8 or more row groups: 4 rows each
        if (!partials || !al16(partials)) return hipErrorInvalidValue;
        if (u4) hipLaunchKernelGGL(pool_chunk_kernel<4>, dim3(C, B), dim3(POOL_NT), 0, s, x, cu_seqlens, H, C, partials);
        else hipLaunchKernelGGL(pool_chunk_kernel<8>, dim3(C, B), dim3(POOL_NT), 0, s, x, cu_seqlens, H, C, partials);
        hipLaunchKernelGGL(pool_finish_kernel, dim3(B), dim3((H / 4 + 63) / 64 * 64), 0, s, partials,
                           cu_seqlens, H, S, normalize, C, out);
        return hipGetLastError();
    }
    const int nc = (H + 63) / 64;
    const dim3 grid(B), block(64 * POOL_WAVES);
    if (nc <= 4) hipLaunchKernelGGL(pool_kernel<4>, grid, block, 0, s, x, cu_seqlens, H, S, normalize, out);
    else if (nc <= 6) hipLaunchKernelGGL(pool_kernel<6>, grid, block, 0, s, x, cu_seqlens, H, S, normalize, out);
    else if (nc <= 8) hipLaunchKernelGGL(pool_kernel<8>, grid, block, 0, s, x, cu_seqlens, H, S, normalize, out);
    else if (nc <= 12) hipLaunchKernelGGL(pool_kernel<12>, grid, block, 0, s, x, cu_seqlens, H, S, normalize, out);
    else if (nc <= 16) hipLaunchKernelGGL(pool_kernel<16>, grid, block, 0, s, x, cu_seqlens, H, S, normalize, out);
    else if (nc <= 32) hipLaunchKernelGGL(pool_kernel<32>, grid, block, 0, s, x, cu_seqlens, H, S, normalize, out);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

// The same over the bf16 residual stream of bf16 models, with the schedule
// and summation order of pool_kernel, but each lane loads four consecutive
// bf16 values (8 bytes: elements 4 (c * 64 + lane) .. +3) so that a wave
// instruction moves 512 bytes; sums in fp32.
template <int NC4>
__global__ __launch_bounds__(64 * POOL_WAVES) void pool_b16_kernel(const uint16_t* __restrict__ x,
                                                                   const int* __restrict__ cu, int H,
                                                                   int S, int normalize,
                                                                   float* __restrict__ out) {
    __shared__ float4 red[POOL_WAVES - 1][NC4 * 64];
    const int b = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int start = cu[b], len = cu[b + 1] - start;
    float4 acc[NC4];
#pragma unroll
    for (int c = 0; c < NC4; ++c) acc[c] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    auto add_row = [&](float4 (&a)[NC4], const uint2 (&h)[NC4]) __attribute__((always_inline)) {
#pragma unroll
        for (int c = 0; c < NC4; ++c) {
            a[c].x += __uint_as_float(h[c].x << 16);
            a[c].y += __uint_as_float(h[c].x & 0xFFFF0000u);
            a[c].z += __uint_as_float(h[c].y << 16);
            a[c].w += __uint_as_float(h[c].y & 0xFFFF0000u);
        }
    };
    constexpr int U = 4;  // rows in flight per wave
    int t = wave;
    for (; t + (U - 1) * POOL_WAVES < len; t += U * POOL_WAVES) {
        uint2 v[U][NC4];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint16_t* xr = x + (int64_t)(start + t + u * POOL_WAVES) * H;
#pragma unroll
            for (int c = 0; c < NC4; ++c) {
                const int i = 4 * (c * 64 + lane);
                v[u][c] = i < H ? *reinterpret_cast<const uint2*>(xr + i) : make_uint2(0u, 0u);
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) add_row(acc, v[u]);
    }
    for (; t < len; t += POOL_WAVES) {
        const uint16_t* xr = x + (int64_t)(start + t) * H;
        uint2 v[NC4];
#pragma unroll
        for (int c = 0; c < NC4; ++c) {
            const int i = 4 * (c * 64 + lane);
            v[c] = i < H ? *reinterpret_cast<const uint2*>(xr + i) : make_uint2(0u, 0u);
        }
        add_row(acc, v);
    }
    if (wave > 0) {
#pragma unroll
        for (int c = 0; c < NC4; ++c) red[wave - 1][c * 64 + lane] = acc[c];
    }
    __syncthreads();
    if (wave != 0) return;
    const float count = fmaxf((float)len, 1.0f);
    const bool all_masked = (len == 0 && S > 0);
    float ss = 0.0f;
#pragma unroll
    for (int c = 0; c < NC4; ++c) {
        const int i = 4 * (c * 64 + lane);
        float4 v = acc[c];
#pragma unroll
        for (int w = 0; w < POOL_WAVES - 1; ++w) {
            const float4 r = red[w][c * 64 + lane];
            v.x += r.x; v.y += r.y; v.z += r.z; v.w += r.w;
        }
        v.x /= count; v.y /= count; v.z /= count; v.w /= count;
        if (all_masked) v = make_float4(__builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""));
        acc[c] = v;
        if (i < H) ss += (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
    }
    const float norm = normalize ? fmaxf(sqrtf(wave_sum(ss)), 1e-12f) : 1.0f;
#pragma unroll
    for (int c = 0; c < NC4; ++c) {
        const int i = 4 * (c * 64 + lane);
        if (i < H) {
            float4 v = acc[c];
            if (normalize) { v.x /= norm; v.y /= norm; v.z /= norm; v.w /= norm; }
            float* o = out + (int64_t)b * H + i;   // the caller's [B, H] buffer: 4-byte stores
            o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
        }
    }
}

hipError_t launch_pool_b16(const uint16_t* x16, const int* cu_seqlens, int B, int H, int S, int normalize,
                           float* out, hipStream_t s) {
    if (B <= 0) return hipSuccess;
    if (H % 4 || ((uintptr_t)x16 & 7)) return hipErrorInvalidValue;
    const int nc4 = (H + 255) / 256;
    const dim3 grid(B), block(64 * POOL_WAVES);
    if (nc4 <= 2) hipLaunchKernelGGL(pool_b16_kernel<2>, grid, block, 0, s, x16, cu_seqlens, H, S, normalize, out);
    else if (nc4 <= 3) hipLaunchKernelGGL(pool_b16_kernel<3>, grid, block, 0, s, x16, cu_seqlens, H, S, normalize, out);
    else if (nc4 <= 4) hipLaunchKernelGGL(pool_b16_kernel<4>, grid, block, 0, s, x16, cu_seqlens, H, S, normalize, out);
    else if (nc4 <= 8) hipLaunchKernelGGL(pool_b16_kernel<8>, grid, block, 0, s, x16, cu_seqlens, H, S, normalize, out);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

// Cross-encoder head (Model::score_pair, src/lib.rs:363-375): score[b] =
// pooled[b] . w + bias, one wave per row (the products summed in lane order,
// then a butterfly over the wave).
__global__ __launch_bounds__(256) void cls_head_kernel(const float* __restrict__ pooled,
                                                       const float* __restrict__ w,
                                                       const float* __restrict__ bias, int B, int H,
                                                       float* __restrict__ out) {
    const int b = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (b >= B) return;
    const float* x = pooled + (int64_t)b * H;
    float acc = 0.0f;
    for (int i = lane; i < H; i += 64) acc += x[i] * w[i];
    acc = wave_sum(acc);
    if (lane == 0) out[b] = acc + bias[0];
}

hipError_t launch_cls_head(const float* pooled, const float* w, const float* bias, int B, int H,
                           float* out, hipStream_t s) {
    if (B <= 0) return hipSuccess;
    hipLaunchKernelGGL(cls_head_kernel, dim3((B + 3) / 4), dim3(256), 0, s, pooled, w, bias, B, H, out);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
__global__ void f32_to_bf16_kernel(const float* __restrict__ x, uint16_t* __restrict__ y,
                                   int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        y[i] = f32_to_bf16_rne(x[i]);
}

hipError_t launch_f32_to_bf16(const float* x, uint16_t* y, int64_t n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    const int64_t blocks = (n + 255) / 256;
    hipLaunchKernelGGL(f32_to_bf16_kernel, dim3((unsigned)(blocks < 65536 ? blocks : 65536)),
                       dim3(256), 0, s, x, y, n);
    return hipGetLastError();
}

// IEEE binary16 bits -> the float of the same value, exactly: a normal f16
// rebiases its exponent (15 -> 127); a subnormal m * 2^-24 (m < 1024) is
// normalised (shifted until bit 10 is set, the exponent counting down); zero
// keeps its sign; inf and NaN keep the all-ones exponent and the mantissa
// bits (NaN payloads shifted up, as a hardware widening does for quiet NaNs).
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    const uint32_t sign = (h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu, man = h & 0x3FFu;
    if (exp == 0x1Fu) return __uint_as_float(sign | 0x7F800000u | (man << 13));
    if (exp == 0) {
        if (man == 0) return __uint_as_float(sign);
        const int lz = __clz(man) - 21;           // zeros above bit 10 of man (1..10)
        man = (man << lz) & 0x3FFu;
        exp = 1 - lz;                             // f16 exponent of the normalised value
    }
    return __uint_as_float(sign | ((exp + 112u) << 23) | (man << 13));
}

// 16-bit checkpoint tensors to their device form: F16 or BF16 bits -> f32
// (exact), or F16 bits -> bf16 (the exact f32 value rounded to nearest even).
// BF16 bits need no kernel for a bf16 destination.
template <int MODE>   // 0: f16 -> f32, 1: bf16 -> f32, 2: f16 -> bf16
__global__ __launch_bounds__(256) void widen16_kernel(const uint16_t* __restrict__ x, void* __restrict__ y,
                                                      int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
        const uint32_t h = x[i];
        if constexpr (MODE == 0) static_cast<float*>(y)[i] = f16_bits_to_f32(h);
        if constexpr (MODE == 1) static_cast<float*>(y)[i] = __uint_as_float(h << 16);
        if constexpr (MODE == 2) static_cast<uint16_t*>(y)[i] = f32_to_bf16_rne(f16_bits_to_f32(h));
    }
}

hipError_t launch_widen16(const uint16_t* x, void* y, int64_t n, int mode, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    const dim3 grid((unsigned)std::min<int64_t>((n + 255) / 256, 65536)), block(256);
    switch (mode) {
        case WIDEN_F16_F32: hipLaunchKernelGGL(widen16_kernel<0>, grid, block, 0, s, x, y, n); break;
        case WIDEN_BF16_F32: hipLaunchKernelGGL(widen16_kernel<1>, grid, block, 0, s, x, y, n); break;
        case WIDEN_F16_BF16: hipLaunchKernelGGL(widen16_kernel<2>, grid, block, 0, s, x, y, n); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace ebh
