// gemm.hip -- fused-bias GEMM family on CDNA4 MFMA.
//
// Replaces matmul_3d_2d + the bias adds, the GELU pass and the residual adds
// of the reference (src/lib.rs:691-698, 732-733, 741-747, 673, 678,
// 795-849, 958-978).  The reference multiplies by the transposed weight
// (`W.t()`, [in, out]); here both operands stay K-contiguous ("NT"):
//   C[m, n] = epi( sum_k A[m, k] * W[n, k] + bias[n] )
// with W in the HF [out, in] layout.
//
// Tiling (fp32): a 256-thread workgroup (4 wave64) owns a BM x BN tile of C;
// each wave owns (BM/WAVES_M) x (BN/WAVES_N) as 32x32 blocks of
// v_mfma_f32_32x32x2_f32.  A and W tiles of BK columns are staged through
// double-buffered LDS (one barrier per k-tile) with the next tile's global
// loads in flight during the current tile's MFMAs.
//
// K ordering: one 32x32x2 MFMA consumes k in {kA, kB}, lane half h supplying
// one of them.  Within each 8-wide k slice lane half h owns k = 4h..4h+3, so
// each lane fetches its four operands with one 16-byte LDS read and MFMA q
// (q = 0..3) uses k = 4h + q.  A and W use the same map, so the products
// summed are exactly those of the dot product.
#include "kernels.hpp"

namespace ebh {

typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef short v8s __attribute__((ext_vector_type(8)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

// Workgroup -> tile.  Workgroups are dispatched round-robin over the 8 XCDs
// (each with its own L2); remap so that each XCD receives a contiguous run of
// tiles, and order tiles N-fastest so the XCD that loads an A row panel also
// does every N tile of it.
__device__ __forceinline__ void tile_coords(int ntiles_n, int& mt, int& nt) {
    int nb = gridDim.x, bid = blockIdx.x;
    if ((nb & 7) == 0) bid = (bid & 7) * (nb >> 3) + (bid >> 3);
    mt = bid / ntiles_n;
    nt = bid - mt * ntiles_n;
}

template <int EPI>
__device__ __forceinline__ float epilogue(float acc, float bias, const float* R, int64_t ldr,
                                          int row, int col) {
    float v = acc + bias;
    if (EPI == EPI_BIAS_GELU) v = gelu_tanh(v);
    if (EPI == EPI_BIAS_RESID) v = v + R[(int64_t)row * ldr + col];
    return v;
}

// ---------------------------------------------------------------------------
// fp32: v_mfma_f32_32x32x2_f32
// ---------------------------------------------------------------------------
template <int BM, int BN, int BK, int WAVES_M, int WAVES_N, int EPI>
__global__ __launch_bounds__(256) void gemm_f32_kernel(GemmArgs p) {
    static_assert(WAVES_M * WAVES_N == 4, "4 waves per workgroup");
    constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
    constexpr int FM = WM / 32, FN = WN / 32;
    constexpr int LDS_STRIDE = BK + 4;            // floats; 16-B aligned rows, conflict-free b128 reads
    constexpr int KF4 = BK / 4;                   // float4 per tile row
    constexpr int A_LD = BM * KF4 / 256;          // float4 loads per thread per k-tile
    constexpr int W_LD = BN * KF4 / 256;
    static_assert(A_LD * 256 == BM * KF4 && W_LD * 256 == BN * KF4, "tile/thread mismatch");

    __shared__ __attribute__((aligned(16))) float As[2][BM * LDS_STRIDE];
    __shared__ __attribute__((aligned(16))) float Ws[2][BN * LDS_STRIDE];

    const int M = p.M_dev ? *p.M_dev : p.M_max;
    const int ntiles_n = (p.N + BN - 1) / BN;
    int mt, nt;
    tile_coords(ntiles_n, mt, nt);
    const int m0 = mt * BM, n0 = nt * BN;
    if (m0 >= M) return;  // uniform over the workgroup

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;
    const int l32 = lane & 31, half = lane >> 5;
    const int K = p.K, N = p.N;
    const float* __restrict__ A = static_cast<const float*>(p.A);
    const float* __restrict__ W = static_cast<const float*>(p.W);

    // Per-thread global source rows (clamped: rows past M / N are loaded but never stored).
    const float* a_src[A_LD];
    const float* w_src[W_LD];
    int a_lds[A_LD], w_lds[W_LD], a_col[A_LD], w_col[W_LD];
#pragma unroll
    for (int i = 0; i < A_LD; ++i) {
        int idx = tid + 256 * i, r = idx / KF4, c = idx % KF4;
        int gr = min(m0 + r, M - 1);
        a_src[i] = A + (int64_t)gr * p.lda;
        a_col[i] = c * 4;
        a_lds[i] = r * LDS_STRIDE + c * 4;
    }
#pragma unroll
    for (int i = 0; i < W_LD; ++i) {
        int idx = tid + 256 * i, r = idx / KF4, c = idx % KF4;
        int gr = min(n0 + r, N - 1);
        w_src[i] = W + (int64_t)gr * p.ldw;
        w_col[i] = c * 4;
        w_lds[i] = r * LDS_STRIDE + c * 4;
    }

    float4 ra[A_LD], rw[W_LD];
    auto gload = [&](int k0) {
#pragma unroll
        for (int i = 0; i < A_LD; ++i) {
            int k = k0 + a_col[i];
            ra[i] = k < K ? *reinterpret_cast<const float4*>(a_src[i] + k) : make_float4(0, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < W_LD; ++i) {
            int k = k0 + w_col[i];
            rw[i] = k < K ? *reinterpret_cast<const float4*>(w_src[i] + k) : make_float4(0, 0, 0, 0);
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < A_LD; ++i) *reinterpret_cast<float4*>(&As[buf][a_lds[i]]) = ra[i];
#pragma unroll
        for (int i = 0; i < W_LD; ++i) *reinterpret_cast<float4*>(&Ws[buf][w_lds[i]]) = rw[i];
    };

    v16f acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    const int nk = (K + BK - 1) / BK;
    gload(0);
    lstore(0);
    __syncthreads();

    const int a_off = (wm * WM + l32) * LDS_STRIDE + 4 * half;
    const int w_off = (wn * WN + l32) * LDS_STRIDE + 4 * half;
    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < nk) gload((kt + 1) * BK);
        const float* as = As[cur];
        const float* ws = Ws[cur];
#pragma unroll
        for (int s = 0; s < BK / 8; ++s) {
            v4f af[FM], wf[FN];
#pragma unroll
            for (int i = 0; i < FM; ++i)
                af[i] = *reinterpret_cast<const v4f*>(as + a_off + i * 32 * LDS_STRIDE + s * 8);
#pragma unroll
            for (int j = 0; j < FN; ++j)
                wf[j] = *reinterpret_cast<const v4f*>(ws + w_off + j * 32 * LDS_STRIDE + s * 8);
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int i = 0; i < FM; ++i)
#pragma unroll
                    for (int j = 0; j < FN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i][q], wf[j][q],
                                                                         acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) lstore(cur ^ 1);
        __syncthreads();
    }

    // Epilogue: lane holds column l32 of each 32x32 block and rows
    // 8*(r/4) + 4*half + r%4 (r = 0..15).
#pragma unroll
    for (int j = 0; j < FN; ++j) {
        const int col = n0 + wn * WN + j * 32 + l32;
        if (col >= N) continue;
        const float bcol = p.bias[col];
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            const int rbase = m0 + wm * WM + i * 32 + 4 * half;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = rbase + 8 * (r >> 2) + (r & 3);
                if (row < M)
                    p.C[(int64_t)row * p.ldc + col] =
                        epilogue<EPI>(acc[i][j][r], bcol, p.R, p.ldr, row, col);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// bf16 inputs, fp32 accumulate: v_mfma_f32_32x32x16_bf16.
// A (fp32 activations) is rounded to bf16 while it is staged into LDS; W is
// already bf16 in HBM.  Within each 16-wide k slice lane half h owns
// k = 8h..8h+7 (one 16-byte LDS read per operand per MFMA).
// ---------------------------------------------------------------------------
template <int BM, int BN, int BK, int WAVES_M, int WAVES_N, int EPI>
__global__ __launch_bounds__(256) void gemm_bf16_kernel(GemmArgs p) {
    static_assert(WAVES_M * WAVES_N == 4, "4 waves per workgroup");
    constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
    constexpr int FM = WM / 32, FN = WN / 32;
    constexpr int LDS_STRIDE = BK + 8;            // bf16 elements (16-B padding)
    constexpr int A_CH = BK / 4;                  // fp32 float4 chunks per A row
    constexpr int W_CH = BK / 8;                  // 16-B bf16 chunks per W row
    constexpr int A_LD = BM * A_CH / 256;
    constexpr int W_LD = BN * W_CH / 256;
    static_assert(A_LD * 256 == BM * A_CH && W_LD * 256 == BN * W_CH, "tile/thread mismatch");

    __shared__ __attribute__((aligned(16))) uint16_t As[2][BM * LDS_STRIDE];
    __shared__ __attribute__((aligned(16))) uint16_t Ws[2][BN * LDS_STRIDE];

    const int M = p.M_dev ? *p.M_dev : p.M_max;
    const int ntiles_n = (p.N + BN - 1) / BN;
    int mt, nt;
    tile_coords(ntiles_n, mt, nt);
    const int m0 = mt * BM, n0 = nt * BN;
    if (m0 >= M) return;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;
    const int l32 = lane & 31, half = lane >> 5;
    const int K = p.K, N = p.N;
    const float* __restrict__ A = static_cast<const float*>(p.A);
    const uint16_t* __restrict__ W = static_cast<const uint16_t*>(p.W);

    const float* a_src[A_LD];
    const uint16_t* w_src[W_LD];
    int a_lds[A_LD], w_lds[W_LD], a_col[A_LD], w_col[W_LD];
#pragma unroll
    for (int i = 0; i < A_LD; ++i) {
        int idx = tid + 256 * i, r = idx / A_CH, c = idx % A_CH;
        a_src[i] = A + (int64_t)min(m0 + r, M - 1) * p.lda;
        a_col[i] = c * 4;
        a_lds[i] = r * LDS_STRIDE + c * 4;
    }
#pragma unroll
    for (int i = 0; i < W_LD; ++i) {
        int idx = tid + 256 * i, r = idx / W_CH, c = idx % W_CH;
        w_src[i] = W + (int64_t)min(n0 + r, N - 1) * p.ldw;
        w_col[i] = c * 8;
        w_lds[i] = r * LDS_STRIDE + c * 8;
    }

    float4 ra[A_LD];
    uint4 rw[W_LD];
    auto gload = [&](int k0) {
#pragma unroll
        for (int i = 0; i < A_LD; ++i) {
            int k = k0 + a_col[i];
            ra[i] = k < K ? *reinterpret_cast<const float4*>(a_src[i] + k) : make_float4(0, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < W_LD; ++i) {
            int k = k0 + w_col[i];
            rw[i] = k < K ? *reinterpret_cast<const uint4*>(w_src[i] + k) : make_uint4(0, 0, 0, 0);
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < A_LD; ++i) {
            uint2 v;
            v.x = (uint32_t)f32_to_bf16_rne(ra[i].x) | ((uint32_t)f32_to_bf16_rne(ra[i].y) << 16);
            v.y = (uint32_t)f32_to_bf16_rne(ra[i].z) | ((uint32_t)f32_to_bf16_rne(ra[i].w) << 16);
            *reinterpret_cast<uint2*>(&As[buf][a_lds[i]]) = v;
        }
#pragma unroll
        for (int i = 0; i < W_LD; ++i) *reinterpret_cast<uint4*>(&Ws[buf][w_lds[i]]) = rw[i];
    };

    v16f acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    const int nk = (K + BK - 1) / BK;
    gload(0);
    lstore(0);
    __syncthreads();

    const int a_off = (wm * WM + l32) * LDS_STRIDE + 8 * half;
    const int w_off = (wn * WN + l32) * LDS_STRIDE + 8 * half;
    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < nk) gload((kt + 1) * BK);
        const uint16_t* as = As[cur];
        const uint16_t* ws = Ws[cur];
#pragma unroll
        for (int s = 0; s < BK / 16; ++s) {
            v8bf af[FM], wf[FN];
#pragma unroll
            for (int i = 0; i < FM; ++i)
                af[i] = __builtin_bit_cast(v8bf, *reinterpret_cast<const v8s*>(as + a_off + i * 32 * LDS_STRIDE + s * 16));
#pragma unroll
            for (int j = 0; j < FN; ++j)
                wf[j] = __builtin_bit_cast(v8bf, *reinterpret_cast<const v8s*>(ws + w_off + j * 32 * LDS_STRIDE + s * 16));
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], wf[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) lstore(cur ^ 1);
        __syncthreads();
    }

#pragma unroll
    for (int j = 0; j < FN; ++j) {
        const int col = n0 + wn * WN + j * 32 + l32;
        if (col >= N) continue;
        const float bcol = p.bias[col];
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            const int rbase = m0 + wm * WM + i * 32 + 4 * half;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = rbase + 8 * (r >> 2) + (r & 3);
                if (row < M)
                    p.C[(int64_t)row * p.ldc + col] =
                        epilogue<EPI>(acc[i][j][r], bcol, p.R, p.ldr, row, col);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
template <int BM, int BN, int BK, int WAVES_M, int WAVES_N, bool BF16>
static hipError_t launch_tile(const GemmArgs& a, int epi, hipStream_t s) {
    const int mt = (a.M_max + BM - 1) / BM, nt = (a.N + BN - 1) / BN;
    const dim3 grid(mt * nt), block(256);
    if (mt == 0 || nt == 0) return hipSuccess;
    switch (epi) {
#define EBH_CASE(E)                                                                           \
    case E:                                                                                   \
        if (BF16)                                                                             \
            hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, BK, WAVES_M, WAVES_N, E>), grid,     \
                               block, 0, s, a);                                               \
        else                                                                                  \
            hipLaunchKernelGGL((gemm_f32_kernel<BM, BN, BK, WAVES_M, WAVES_N, E>), grid,      \
                               block, 0, s, a);                                               \
        break;
        EBH_CASE(EPI_BIAS)
        EBH_CASE(EPI_BIAS_GELU)
        EBH_CASE(EPI_BIAS_RESID)
#undef EBH_CASE
        default:
            return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_gemm_f32(const GemmArgs& a, int epi, hipStream_t s) {
    return launch_tile<128, 128, 32, 2, 2, false>(a, epi, s);
}

hipError_t launch_gemm_bf16(const GemmArgs& a, int epi, hipStream_t s) {
    return launch_tile<128, 128, 32, 2, 2, true>(a, epi, s);
}

}  // namespace ebh
