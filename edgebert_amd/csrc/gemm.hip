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
#include <algorithm>

#include <type_traits>

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
    float v = EPI == EPI_NONE ? acc : acc + bias;
    if (EPI == EPI_BIAS_GELU) v = gelu_tanh(v);
    if (EPI == EPI_BIAS_RESID) v = v + R[(int64_t)row * ldr + col];
    return v;
}

// ---------------------------------------------------------------------------
// fp32: v_mfma_f32_32x32x2_f32.
// NT = 64 * WAVES_M * WAVES_N threads; wave (wm, wn) owns the (BM/WAVES_M) x
// (BN/WAVES_N) sub-tile as FM x FN blocks of 32x32.  KFULL: the launcher has
// checked that K is a multiple of BK, so the k-tile loads carry no guard.
// ---------------------------------------------------------------------------
template <int BM, int BN, int BK, int WAVES_M, int WAVES_N, int EPI, bool KFULL>
__global__ __launch_bounds__(64 * WAVES_M * WAVES_N) void gemm_f32_kernel(GemmArgs p) {
    constexpr int NT = 64 * WAVES_M * WAVES_N;
    constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
    constexpr int FM = WM / 32, FN = WN / 32;
    static_assert(FM * 32 == WM && FN * 32 == WN, "wave tile must be whole 32x32 blocks");
    constexpr int LDS_STRIDE = BK + 4;            // floats; 16-B aligned rows, conflict-free b128 reads
    constexpr int KF4 = BK / 4;                   // float4 per tile row
    constexpr int A_TOT = BM * KF4, W_TOT = BN * KF4;   // float4 per k-tile
    constexpr int A_LD = (A_TOT + NT - 1) / NT;   // float4 loads per thread per k-tile
    constexpr int W_LD = (W_TOT + NT - 1) / NT;
    // Whether load i of this thread exists (only the last one can be partial).
    auto a_on = [&](int i) { return A_TOT % NT == 0 || i + 1 < A_LD || (int)threadIdx.x + NT * i < A_TOT; };
    auto w_on = [&](int i) { return W_TOT % NT == 0 || i + 1 < W_LD || (int)threadIdx.x + NT * i < W_TOT; };

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
        int idx = tid + NT * i, r = idx / KF4, c = idx % KF4;
        int gr = min(m0 + r, M - 1);
        a_src[i] = A + (int64_t)gr * p.lda + c * 4;
        a_col[i] = c * 4;
        a_lds[i] = r * LDS_STRIDE + c * 4;
    }
#pragma unroll
    for (int i = 0; i < W_LD; ++i) {
        int idx = tid + NT * i, r = idx / KF4, c = idx % KF4;
        int gr = min(n0 + r, N - 1);
        w_src[i] = W + (int64_t)gr * p.ldw + c * 4;
        w_col[i] = c * 4;
        w_lds[i] = r * LDS_STRIDE + c * 4;
    }

    float4 ra[A_LD], rw[W_LD];
    auto gload = [&](int k0) {
#pragma unroll
        for (int i = 0; i < A_LD; ++i) {
            if (!a_on(i)) continue;
            if (KFULL || k0 + a_col[i] < K)
                ra[i] = *reinterpret_cast<const float4*>(a_src[i] + k0);
            else
                ra[i] = make_float4(0, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < W_LD; ++i) {
            if (!w_on(i)) continue;
            if (KFULL || k0 + w_col[i] < K)
                rw[i] = *reinterpret_cast<const float4*>(w_src[i] + k0);
            else
                rw[i] = make_float4(0, 0, 0, 0);
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < A_LD; ++i)
            if (a_on(i)) *reinterpret_cast<float4*>(&As[buf][a_lds[i]]) = ra[i];
#pragma unroll
        for (int i = 0; i < W_LD; ++i)
            if (w_on(i)) *reinterpret_cast<float4*>(&Ws[buf][w_lds[i]]) = rw[i];
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
// fp32, persistent: one workgroup per CU walks a strided list of BM x BN C
// tiles through one flattened (tile, k-tile) pipeline with NSTAGE LDS stages,
// so the loads of the next NSTAGE-1 k-tiles (across tile boundaries) are in
// flight while the MFMAs of the current one run.
//
// Loads are global_load_lds_dwordx4 issued from inline asm: the compiler's
// wait-count tracking does not see them, so it does not make every LDS read
// wait for every outstanding LDS load.  The loop waits explicitly instead:
// before k-tile `it` is used, vmcnt(n) with n = the load instructions this
// wave issued after k-tile it's own (every wave issues the same number, and
// vector memory operations complete in issue order), then the barrier.
// M0 (the LDS destination base of the instruction) is saved and restored
// inside the asm.  The bias row segment of a tile comes the same way, into a
// small per-wave LDS slot, so the epilogue issues no global load.
//
// A tile's epilogue runs at the top of the next tile's first k-tile, after
// that k-tile's wait and before its loads are issued: the C tile is
// transposed through the LDS stage the previous k-tile used (free until the
// loads issued right after the epilogue refill it) and written as
// row-contiguous float4.  Its stores are then older than every load still to
// be waited for, so no later wait depends on them finishing early.
// ---------------------------------------------------------------------------

// Standalone GELU (ebh_op_gelu): gelu_tanh_fast over n floats.
__global__ __launch_bounds__(256) void gelu_kernel(const float* __restrict__ x, float* __restrict__ y, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
        y[i] = gelu_tanh_fast(x[i]);
}

hipError_t launch_gelu(const float* x, float* y, int64_t n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(gelu_kernel, dim3((unsigned)std::min<int64_t>((n + 255) / 256, 65536)), dim3(256), 0, s,
                       x, y, n);
    return hipGetLastError();
}

// Word 3 of a gfx9 buffer resource descriptor for plain dword-addressed
// buffers (32-bit data format; no swizzle, no index stride).  Accesses at or
// past the descriptor's byte count return 0 (loads) or are dropped (stores).
constexpr int BUFFER_RSRC_WORD3 = 0x00020000;

// BF16: A and W are bf16 (16-byte chunk = 8 elements, one
// v_mfma_f32_32x32x16_bf16 per fragment pair and k-slice); otherwise fp32
// (chunk = 4 elements, four v_mfma_f32_32x32x2_f32).  OUT16: C is written as
// bf16 (round to nearest even) instead of fp32, through the packed epilogue:
// the MFMAs take W as their first operand, so each block holds C transposed
// and a lane holds four consecutive columns of one C row per group of four
// accumulators (epilogue_packed).  LDS offsets below are in
// 4-byte words, so both element types share the layout and the swizzle.
// Eight fp32 values (x0, x1) split into three bf16 vectors with
// x = h + m + l: h = bf16(x), m = bf16(x - h), l = bf16(x - h - m), each
// rounded to nearest even; both differences are exact in fp32 (x - h has at
// most 16 significant bits).  |x - h - m - l| <= 2^-26 |x| or so, and the
// split products dropped by the six-product GEMM (m.l, l.m, l.l) are below
// 2^-27 |a.b|.
__device__ __forceinline__ void split3_bf16(const v4f& x0, const v4f& x1, v8bf& h, v8bf& m, v8bf& l) {
    uint32_t hh[4], mm[4], ll[4];
    const float xs[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float a = xs[2 * e], b = xs[2 * e + 1];
        const uint32_t ph = pack_bf16x2(a, b);
        const float ra = a - __uint_as_float(ph << 16), rb = b - __uint_as_float(ph & 0xffff0000u);
        const uint32_t pm = pack_bf16x2(ra, rb);
        const float sa = ra - __uint_as_float(pm << 16), sb = rb - __uint_as_float(pm & 0xffff0000u);
        hh[e] = ph;
        mm[e] = pm;
        ll[e] = pack_bf16x2(sa, sb);
    }
    h = __builtin_bit_cast(v8bf, make_uint4(hh[0], hh[1], hh[2], hh[3]));
    m = __builtin_bit_cast(v8bf, make_uint4(mm[0], mm[1], mm[2], mm[3]));
    l = __builtin_bit_cast(v8bf, make_uint4(ll[0], ll[1], ll[2], ll[3]));
}

template <bool BF16, bool OUT16, int BM, int BN, int BK, int WAVES_M, int WAVES_N, int NSTAGE, int EPI,
          bool SPLIT6 = false, bool MF16 = false>
__global__ __launch_bounds__(64 * WAVES_M * WAVES_N) void gemm_persistent_kernel(GemmArgs p) {
    constexpr int ES = BF16 ? 2 : 4;              // bytes per element
    constexpr int EPC = 16 / ES;                  // elements per 16-byte chunk
    static_assert(EPI == EPI_BIAS || EPI == EPI_BIAS_GELU || EPI == EPI_NONE || EPI == EPI_ADD_LN,
                  "no plain residual here");
    constexpr bool LN = EPI == EPI_ADD_LN;
    static_assert(!LN || (!BF16 && !OUT16 && BM / WAVES_M == 64), "LayerNorm epilogue: fp32, 64-row wave tiles");
    constexpr bool HAS_BIAS = EPI != EPI_NONE;
    constexpr int NT = 64 * WAVES_M * WAVES_N, NW = WAVES_M * WAVES_N;
    constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
    constexpr int FM = WM / 32, FN = WN / 32;
    static_assert(FM * 32 == WM && FN * 32 == WN, "wave tile must be whole 32x32 blocks");
    // MF16 (bf16 operands): v_mfma_f32_16x16x32_bf16 on 16x16 blocks instead
    // of v_mfma_f32_32x32x16_bf16 on 32x32 blocks.  The flops per cycle are
    // the same, but these kernels are power-bound, and measured on MI355X with
    // random operands a stream of the 16x16 form holds a higher clock under
    // sustained load (1.95 against 1.76 GHz from registers; 1.85 against
    // 1.64-1.71 GHz with a GEMM's LDS fragment reads beside them).
    static_assert(!MF16 || (BF16 && !SPLIT6 && EPI != EPI_ADD_LN && (BK == 64 || BK == 32)),
                  "16x16x32 MFMAs: bf16, 32- or 64-deep k-tiles");
    constexpr int FM16 = WM / 16, FN16 = WN / 16;
    static_assert(!MF16 || FM16 % 2 == 0, "16x16 steps take half of the wave tile's row blocks each");
    constexpr int CPR = BK / EPC;                 // 16-byte chunks per tile row
    constexpr int KS = CPR / 2;                   // k-slices (two chunks: one per lane half)
    constexpr int RW = CPR * 4;                   // words per tile row
    constexpr int A_CH = BM * CPR, W_CH = BN * CPR;
    static_assert(A_CH % NT == 0 && W_CH % NT == 0, "every wave issues the same loads");
    constexpr int LA = A_CH / NT, LW = W_CH / NT, NL = LA + LW;
    constexpr int D = NSTAGE - 1;                 // k-tiles in flight ahead
    constexpr int STAGE = (BM + BN) * RW;         // words per stage: A rows, then W rows
    constexpr int C4 = WN / 4;                    // float4 per wave-tile row
    // FLAT: wave tiles too wide for a 32-row transpose per stage, or whose
    // float4 rows do not tile 64 lanes (e.g. 96 columns): C goes through LDS
    // 16 rows at a time and the lanes walk the rows' float4 in order.
    constexpr bool PACKED = OUT16;
    static_assert(!PACKED || (NW * 16 * WN <= STAGE && WN % 64 == 0), "packed epilogue: 32 bf16 rows per wave per stage");
    constexpr bool FLAT = !LN && !PACKED && (64 % C4 != 0 || NW * 32 * WN > STAGE);
    static_assert(LN || FLAT || PACKED || NW * 32 * WN <= STAGE, "each wave transposes 32 C rows at a time through one stage");
    static_assert(!FLAT || (NW * 16 * WN <= STAGE && (4 * WN) % 64 == 0), "16-row transpose shape");
    static_assert(!LN || 2 * WAVES_N * BM + 2 * NW * 64 <= STAGE, "LayerNorm exchange fits one stage");
    constexpr int RPP = FLAT || LN ? 1 : 64 / C4; // wave-tile rows per float4 pass
    static_assert(LN || FLAT || PACKED || (C4 * RPP == 64 && 32 % RPP == 0), "epilogue pass shape");
    constexpr int NPB = 32 / RPP;                 // float4 passes per 32-row block
    constexpr int BIAS_SLOT = 256;                // floats: one wave's 64 x 16-byte bias chunks

    __shared__ __attribute__((aligned(16))) float smem[NSTAGE * STAGE + (HAS_BIAS ? 2 * NW * BIAS_SLOT : 0)];

    const int M = p.M_dev ? *p.M_dev : p.M_max;
    const int N = p.N;
    const int ntiles_n = (N + BN - 1) / BN;
    const int ntiles = ((M + BM - 1) / BM) * ntiles_n;
    // Split-K: work item u covers C tile u % ntiles over k-range u / ntiles
    // (split-major, so an XCD's consecutive items still share A row panels).
    const int S = p.splits > 1 ? p.splits : 1;
    const int nwork = ntiles * S;
    const int nk = p.K / BK / S;                  // k-tiles per work item
    // Workgroup b runs on XCD b % 8, and each XCD's workgroups take
    // consecutive N-fastest tiles, which share A row panels in that XCD's L2.
    // Whole rounds of items: workgroup x * G / 8 + b / 8 of XCD x walks items
    // in steps of G (each round's 32 consecutive tiles per XCD).  Otherwise
    // each XCD takes an eighth of the items as one consecutive range, walked
    // in steps of G / 8, so that the last, partial step spreads over all XCDs
    // (fewer items than workgroups had left whole XCDs idle: c2 QKV 32.7 ->
    // 31.2 us).
    const int G = gridDim.x;
    int u0 = blockIdx.x, ustep = G, uend = nwork;
    if ((G & 7) == 0 && nwork % G == 0) {
        u0 = (blockIdx.x & 7) * (G >> 3) + (blockIdx.x >> 3);
    } else if ((G & 7) == 0) {
        const int x = blockIdx.x & 7;
        ustep = G >> 3;
        u0 = (int)((int64_t)x * nwork / 8) + (blockIdx.x >> 3);
        uend = (int)((int64_t)(x + 1) * nwork / 8);
    }
    const int my_tiles = u0 < uend ? (uend - u0 + ustep - 1) / ustep : 0;
    const int total = my_tiles * nk;
    if (total == 0) return;  // uniform over the workgroup

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // fp32 products take the wave index as a wave-uniform (scalar) value, so
    // that the k-loop's LDS destinations come from scalar arithmetic: fp32
    // MFMAs hold the SIMD's VALU while they run, and VALU address math in
    // the k-loop adds to the MFMA time (c3: QKV 233.7 -> 225.6 us, FFN up
    // 306.7 -> 298.2 us).  bf16 MFMAs leave the VALU free, and there the
    // scalar form was slower (c5 GEMMs +3-4%), as it was for the split
    // products; the LayerNorm instances' epilogue needs the SGPRs.
    const int wave_u = LN || BF16 || SPLIT6 ? wave : __builtin_amdgcn_readfirstlane(wave);
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;
    const int l32 = lane & 31, half = lane >> 5;
    const char* __restrict__ A = static_cast<const char*>(p.A);
    const char* __restrict__ W = static_cast<const char*>(p.W);

    // This lane's share of each k-tile load: row and swizzled k-chunk of LDS chunk i*NT + tid.
    int l_r[NL], l_c[NL];
#pragma unroll
    for (int i = 0; i < NL; ++i) {
        const int P = (i < LA ? i : i - LA) * NT + tid;
        l_r[i] = P / CPR;
        l_c[i] = EPC * ((P % CPR) ^ chunk_swizzle16<CPR>(P / CPR));   // elements
    }
    // Sources of the next k-tile to load (iteration `nit`): the A and W panel
    // bases of that k-tile (wave-uniform, in SGPRs, advanced by BK per k-tile)
    // and this lane's byte offsets from them (32-bit, fixed for a C tile: the
    // row, clamped to the last real row, and the swizzled k-chunk).  Offsets
    // instead of per-load 64-bit addresses keep the k-loop's addressing off
    // the VGPRs.
    uint32_t soff[NL];
    uint64_t abase = 0, wbase = 0;
    const float* bias_src = nullptr;
    int nit = 0;
    auto point_at = [&](int it) {
        const int u = u0 + (it / nk) * ustep, split = u / ntiles, t = u - split * ntiles;
        const int kt = split * nk + it - (it / nk) * nk;
        const int mt = t / ntiles_n, m0 = mt * BM, n0 = (t - mt * ntiles_n) * BN;
#pragma unroll
        for (int i = 0; i < NL; ++i)
            soff[i] = i < LA ? (uint32_t)(((min(m0 + l_r[i], M - 1) - m0) * p.lda + l_c[i]) * ES)
                             : (uint32_t)(((min(n0 + l_r[i], N - 1) - n0) * p.ldw + l_c[i]) * ES);
        abase = uniform_u64(A + ((int64_t)m0 * p.lda + kt * BK) * ES);
        wbase = uniform_u64(W + ((int64_t)n0 * p.ldw + kt * BK) * ES);
        if (HAS_BIAS) bias_src = p.bias + min(n0 + wn * WN + 4 * lane, N - 4);
    };
    // Load instructions of k-tile j (the bias chunk rides with a tile's first k-tile).
    auto n_issued = [&](int j) { return NL + (HAS_BIAS && j % nk == 0 ? 1 : 0); };
    // The loads of a k-tile go out in parts, one before each of the first
    // half of its k-slices' MFMAs (split products: one per 16-deep slice).
    // The CU's vector memory path takes one 1 KB load per 16 cycles, and a
    // wave stalls at issue while it is backed up: one burst after the barrier
    // would idle the MFMA pipes (at bf16 rates a k-tile's loads need half of
    // its MFMA time on that path), while parts spread over all k-slices leave
    // the last loads too little time to land before the next k-tile's wait
    // (fp32 c3 forward 6.115 -> 6.043 ms against the burst).  Part `part` of
    // NPART issues loads [part * PER, (part + 1) * PER); the last part adds the
    // bias chunk and moves on to the next k-tile.
    constexpr int NPART = KS > 1 ? KS / 2 : 1;
    constexpr int PER = (NL + NPART - 1) / NPART;
    // LDS destinations: fp32 products form them as 32-bit integers (no
    // generic 64-bit LDS pointer, fewer VALU instructions in the k-loop:
    // FFN down 297.2 -> 289.2 us at c3); the bf16 and split products keep
    // the pointer form, which measured faster there (c5 GEMMs 3-5%).
    const uint32_t lds_wave = (uint32_t)(uintptr_t)smem + (uint32_t)wave_u * 64 * 16;
    auto issue_part = [&](int part) {
        const uint32_t st = lds_wave + (uint32_t)((nit % NSTAGE) * STAGE) * 4;
        float* stp = smem + (nit % NSTAGE) * STAGE;
#pragma unroll
        for (int i = 0; i < NL; ++i)
            if (i / PER == part) {
                if constexpr (BF16 || SPLIT6)
                    load_lds16_sbase(i < LA ? abase : wbase, soff[i],
                                     stp + (i < LA ? 0 : BM * RW) + ((i < LA ? i : i - LA) * NT + wave * 64) * 4);
                else
                    load_lds16_sbase(i < LA ? abase : wbase, soff[i],
                                     st + (uint32_t)((i < LA ? 0 : BM * RW) + (i < LA ? i : i - LA) * NT * 4) * 4);
            }
        if (part == NPART - 1) {
            if (HAS_BIAS && nit % nk == 0)
                load_lds16_async(bias_src, smem + NSTAGE * STAGE + (((nit / nk) & 1) * NW + wave) * BIAS_SLOT);
            ++nit;
            if (nit < total) {
                if (nit % nk == 0) {
                    point_at(nit);
                } else {
                    abase += BK * ES;
                    wbase += BK * ES;
                }
            }
        }
    };
    auto issue = [&]() {
#pragma unroll
        for (int part = 0; part < NPART; ++part) issue_part(part);
    };

    const int sw = chunk_swizzle16<CPR>(l32);
    const int a_row = (wm * WM + l32) * RW, w_row = BM * RW + (wn * WN + l32) * RW;
    // 16x16x32 blocks: lane (r16, q16) gives row r16 of a block at k-chunk
    // q16 of the 32-deep slice (16 bytes; A and W use the same map), and holds
    // D[4 q16 + e][r16] of D = W.A^T, i.e. C row r16, columns 4 q16 .. +3.
    // Block rows are multiples of 16, so a block's swizzle is that of r16.
    const int r16 = lane & 15, q16 = lane >> 4;
    const int sw16 = chunk_swizzle16<CPR>(r16);
    const int a_row16 = (wm * WM + r16) * RW, w_row16 = BM * RW + (wn * WN + r16) * RW;
    // Epilogue lane map: pass qq of block row i covers wave-tile rows
    // i*32 + qq*RPP + lane / C4, columns 4 * (lane % C4) .. +3.
    const int e_r = lane / C4, e_c = 4 * (lane % C4);

    v16f acc[FM][FN];
    v4f acc16[FM16][FN16];

    // EPI_ADD_LN: the tile spans whole rows (one tile column), so the workgroup
    // holds every value of its rows.  Lane (l32, half) of wave (wm, wn) holds,
    // in acc[i][j][r], row wm*64 + i*32 + 8*(r/4) + 4*half + r%4 of the tile at
    // column wn*WN + j*32 + l32; a row's values lie in the 32 lanes of one
    // half-wave (3 each here) and in the WAVES_N waves of one wave row.
    //
    // Sum of each of this lane's 32 row values q[i*16 + r] over the 32 lanes of
    // its half-wave by recursive halving: at each step a lane keeps the half of
    // its values that its lane bit selects, each plus its partner's copy, so
    // lane l32 ends with the total of value l32.  (Both halves are exchanged and
    // the choice is made between the sums: a choice between two elements of q
    // would index q by lane and keep it out of registers.)
    auto half_wave_sums = [&](float (&q)[32]) __attribute__((always_inline)) -> float {
#pragma unroll
        for (int step = 0; step < 5; ++step) {
            const int m = 16 >> step;
            const bool up = (l32 & m) != 0;
#pragma unroll
            for (int k = 0; k < m; ++k) {
                const float lo = q[k] + __shfl_xor(q[k], m);
                const float hi = q[k + m] + __shfl_xor(q[k + m], m);
                q[k] = up ? hi : lo;
            }
        }
        return q[0];
    };
    // Row index within the wave tile of value v = i*16 + r (held by lane l32 = v
    // after half_wave_sums).
    const int my_row = (l32 >> 4) * 32 + 8 * ((l32 & 15) >> 2) + 4 * half + (l32 & 3);
    // Row totals across the WAVES_N waves of a wave row, through LDS `red`
    // ([WAVES_N][BM]); then each lane's statistic for its own row is handed to
    // the lanes holding the row's values through the wave's slot of `bc`
    // ([NW][64]) and read back as v[i][r].
    auto row_stat = [&](float part, float* red, float* bc, auto&& finish, float (&v)[FM][16])
                        __attribute__((always_inline)) {
        red[wn * BM + wm * WM + my_row] = part;
        lds_barrier();
        float tot = red[wm * WM + my_row];
#pragma unroll
        for (int w = 1; w < WAVES_N; ++w) tot += red[w * BM + wm * WM + my_row];
        bc[wave * 64 + my_row] = finish(tot);
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
                const float4 f = *reinterpret_cast<const float4*>(bc + wave * 64 + i * 32 + 8 * g4 + 4 * half);
                v[i][4 * g4] = f.x; v[i][4 * g4 + 1] = f.y; v[i][4 * g4 + 2] = f.z; v[i][4 * g4 + 3] = f.w;
            }
    };
    // x = LayerNorm((acc + bias) + R) for local tile t, in the order of the
    // unfused add-LayerNorm: mean, then the mean of squared deviations, then
    // (v - mean) * (1 / sqrt(var + eps)) * gamma + beta.  `ex` is a consumed
    // LDS stage (the exchange buffers).
    auto epilogue_ln = [&](int t, float* ex) __attribute__((always_inline)) {
        const int m0 = (u0 + t * ustep) * BM;
        const float* bsl = smem + NSTAGE * STAGE + ((t & 1) * NW + wave) * BIAS_SLOT + l32;
        const int col = wn * WN + l32;
        // R and C are [M, BN] (row stride BN), read and written through buffer
        // descriptors that start at the tile's first row and end at row M.
        // Element (i, j, r) of this lane lies lane_off + 128 j bytes (the
        // lane's part) plus row_off(i, r) bytes (uniform: the scalar offset)
        // from the tile start; a row at or past M gets a lane offset past the
        // descriptor's end, so it reads 0 and is not written.
        const int valid = min(M - m0, BM);
        const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(p.R) + (int64_t)m0 * BN, (short)0, valid * BN * 4, BUFFER_RSRC_WORD3);
        const __amdgpu_buffer_rsrc_t cx = __builtin_amdgcn_make_buffer_rsrc(
            p.C + (int64_t)m0 * BN, (short)0, valid * BN * 4, BUFFER_RSRC_WORD3);
        const int lane_row = wm * WM + 4 * half;
        int lane_off = (lane_row * BN + col) * 4;
        // Opaque per tile: keeps the 96 offsets derived from it from being
        // computed once ahead of the tile loop and held in registers.
        asm volatile("" : "+v"(lane_off));
        auto row_c = [](int i, int r) { return i * 32 + 8 * (r >> 2) + (r & 3); };
        const int lim = valid - lane_row;         // rows row_c < lim of this lane are real
        auto voff = [&](int i, int r) { return row_c(i, r) < lim ? lane_off : (int)0x80000000; };
        float bj[FN], gj[FN], betaj[FN];
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            bj[j] = bsl[j * 32];
            gj[j] = p.ln_g[col + j * 32];
            betaj[j] = p.ln_b[col + j * 32];
        }
        // The residual loads go out one 32-row block at a time (48 registers in
        // flight beside the 96 accumulators).
#pragma unroll
        for (int i = 0; i < FM; ++i) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int vo = voff(i, r), so = row_c(i, r) * BN * 4;
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j][r] = (acc[i][j][r] + bj[j]) +
                                   __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rx, vo + 128 * j, so, 0));
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        float q[32], st[FM][16];
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                float sum = acc[i][0][r];
#pragma unroll
                for (int j = 1; j < FN; ++j) sum += acc[i][j][r];
                q[i * 16 + r] = sum;
            }
        const float inv_n = 1.0f / (float)N;
        row_stat(half_wave_sums(q), ex, ex + 2 * WAVES_N * BM, [&](float tot) { return tot * inv_n; }, st);
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                float sum = 0.0f;
#pragma unroll
                for (int j = 0; j < FN; ++j) {
                    const float d = acc[i][j][r] - st[i][r];
                    acc[i][j][r] = d;
                    sum += d * d;
                }
                q[i * 16 + r] = sum;
            }
        const float eps = p.ln_eps;
        row_stat(half_wave_sums(q), ex + WAVES_N * BM, ex + 2 * WAVES_N * BM + NW * 64,
                 [&](float tot) { return 1.0f / sqrtf(tot * inv_n + eps); }, st);
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int vo = voff(i, r), so = row_c(i, r) * BN * 4;
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    __builtin_amdgcn_raw_buffer_store_b32(
                        __float_as_uint(acc[i][j][r] * st[i][r] * gj[j] + betaj[j]), cx, vo + 128 * j, so, 0);
            }
    };

    // Epilogue of local tile t: bias (+ GELU), C through LDS stage `cs`, float4 stores.
    // One row group's store: the descriptor starts at C row g0 (wave-uniform)
    // and holds min(M - g0, span) rows, so a lane whose row in the group lies
    // past M (or whose offset is the out-of-range value) is not written.
    // The lane offsets are constants of the epilogue: no per-store row
    // arithmetic, which on this chip adds to the fp32 MFMA time.
    constexpr int CES = OUT16 ? 2 : 4;  // bytes per C element
    // wrow, wv: the wave tile's first C row and the rows of it that exist
    // (wave-uniform: a descriptor in VGPRs makes the compiler loop over lanes).
    auto store_group = [&](char* cb, int wrow, int wv, int r0, int span, uint32_t voff, float4 v)
                           __attribute__((always_inline)) {
        const int rowb = p.ldc * CES, left = wv - r0, g0 = wrow + r0;
        const int bytes = left >= span ? span * rowb : (left > 0 ? left * rowb : 0);
        const __amdgpu_buffer_rsrc_t cr =
            __builtin_amdgcn_make_buffer_rsrc(cb + (int64_t)g0 * rowb, (short)0, bytes, BUFFER_RSRC_WORD3);
        typedef unsigned int u4v __attribute__((ext_vector_type(4)));
        typedef unsigned int u2v __attribute__((ext_vector_type(2)));
        if constexpr (OUT16) {
            const u2v h = {(uint32_t)f32_to_bf16_rne(v.x) | ((uint32_t)f32_to_bf16_rne(v.y) << 16),
                           (uint32_t)f32_to_bf16_rne(v.z) | ((uint32_t)f32_to_bf16_rne(v.w) << 16)};
            __builtin_amdgcn_raw_buffer_store_b64(h, cr, voff, 0, 0);
        } else {
            __builtin_amdgcn_raw_buffer_store_b128(
                u4v{__float_as_uint(v.x), __float_as_uint(v.y), __float_as_uint(v.z), __float_as_uint(v.w)}, cr,
                voff, 0, 0);
        }
    };
    // FLAT epilogue: per 16-row half of each 32-row block (MFMA rows r = 8h ..
    // 8h+7 hold rows 16h .. 16h+15), C through the wave's 16 x WN slot of LDS
    // stage `cs`, then float4 q = pass * 64 + lane of those rows in row-major
    // order.  The lane's (row, column) repeats every PP passes (64 PP float4
    // are whole rows), so each of the PP patterns has its own lane constants.
    auto epilogue_flat = [&](int t, const float* cs_base) __attribute__((always_inline)) {
        const int u = u0 + t * ustep, split = u / ntiles, tile = u - split * ntiles;
        char* const cb = reinterpret_cast<char*>(p.C + (int64_t)split * p.split_stride);
        const int m0 = (tile / ntiles_n) * BM, n0 = (tile - (tile / ntiles_n) * ntiles_n) * BN;
        const float* bslot = smem + NSTAGE * STAGE + ((t & 1) * NW + wave) * BIAS_SLOT;
        float* cw = const_cast<float*>(cs_base) + wave * (16 * WN);
        constexpr int NPASS = 4 * WN / 64;
        constexpr int PP = C4 / (C4 % 64 == 0 ? 64 : (C4 % 32 == 0 ? 32 : (C4 % 16 == 0 ? 16 : 8)));
        constexpr int RPG = 64 * PP / C4;              // rows per PP passes
        constexpr int SPAN = 64 / C4 + 2;              // rows one store can touch, at most
        static_assert(C4 % 8 == 0 && NPASS % PP == 0 && (64 * PP) % C4 == 0, "FLAT pass pattern");
        // lane-derived offsets opaque here (formed at the epilogue, not held)
        int fl = lane, fl32 = l32, fhalf = half;
        asm volatile("" : "+v"(fl), "+v"(fl32), "+v"(fhalf));
        const int wrow = __builtin_amdgcn_readfirstlane(m0 + wm * WM), wv = __builtin_amdgcn_readfirstlane(M - wrow);
        int ldo[PP], bo[PP];
        uint32_t vo[PP];
#pragma unroll
        for (int pp = 0; pp < PP; ++pp) {
            const int q = 64 * pp + fl, lr = q / C4, c = 4 * (q - lr * C4);
            const int gc = n0 + wn * WN + c;
            ldo[pp] = lr * WN + c;
            bo[pp] = c;
            vo[pp] = gc < N ? (uint32_t)(((lr - (64 * pp) / C4) * p.ldc + gc) * CES) : 0xFFFFFFF0u;
        }
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
#pragma unroll
                for (int j = 0; j < FN; ++j)
#pragma unroll
                    for (int rr = 0; rr < 8; ++rr)
                        cw[(8 * (rr >> 2) + 4 * fhalf + (rr & 3)) * WN + j * 32 + fl32] = acc[i][j][8 * h + rr];
#pragma unroll
                for (int ps = 0; ps < NPASS; ++ps) {
                    const int pp = ps % PP, k = ps / PP;
                    float4 v = *reinterpret_cast<const float4*>(cw + ldo[pp] + k * RPG * WN);
                    if (HAS_BIAS) {
                        const float4 b4 = *reinterpret_cast<const float4*>(bslot + bo[pp]);
                        v.x += b4.x; v.y += b4.y; v.z += b4.z; v.w += b4.w;
                    }
                    if constexpr (EPI == EPI_BIAS_GELU) {
                        v.x = gelu_tanh_fast(v.x); v.y = gelu_tanh_fast(v.y);
                        v.z = gelu_tanh_fast(v.z); v.w = gelu_tanh_fast(v.w);
                    }
                    store_group(cb, wrow, wv, i * 32 + 16 * h + (64 * pp) / C4 + k * RPG, SPAN, vo[pp], v);
                }
            }
    };
    auto epilogue_tile = [&](int t, const float* cs_base) {
        const int u = u0 + t * ustep, split = u / ntiles, tile = u - split * ntiles;
        char* const cb = reinterpret_cast<char*>(p.C + (int64_t)split * p.split_stride);
        const int m0 = (tile / ntiles_n) * BM, n0 = (tile - (tile / ntiles_n) * ntiles_n) * BN;
        // The lane's place in the tile, opaque here: the offsets derived from
        // it are formed at the epilogue, not held across the k-loop.
        int er = e_r, ec = e_c;
        asm volatile("" : "+v"(er), "+v"(ec));
        const int gc = n0 + wn * WN + ec;
        float4 bias4 = make_float4(0, 0, 0, 0);
        if (HAS_BIAS)
            bias4 = *reinterpret_cast<const float4*>(smem + NSTAGE * STAGE + ((t & 1) * NW + wave) * BIAS_SLOT + ec);
        float* cw = const_cast<float*>(cs_base) + wave * (32 * WN);
        const int wrow = __builtin_amdgcn_readfirstlane(m0 + wm * WM), wv = __builtin_amdgcn_readfirstlane(M - wrow);
        const uint32_t voff = gc < N ? (uint32_t)((er * p.ldc + gc) * CES) : 0xFFFFFFF0u;   // N % 4 == 0
#pragma unroll
        for (int i = 0; i < FM; ++i) {
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    cw[(8 * (r >> 2) + 4 * half + (r & 3)) * WN + j * 32 + l32] = acc[i][j][r];
#pragma unroll
            for (int qq = 0; qq < NPB; ++qq) {
                float4 v = *reinterpret_cast<const float4*>(cw + (qq * RPP + er) * WN + ec);
                if (HAS_BIAS) { v.x += bias4.x; v.y += bias4.y; v.z += bias4.z; v.w += bias4.w; }
                if constexpr (EPI == EPI_BIAS_GELU) {
                    v.x = gelu_tanh_fast(v.x); v.y = gelu_tanh_fast(v.y);
                    v.z = gelu_tanh_fast(v.z); v.w = gelu_tanh_fast(v.w);
                }
                store_group(cb, wrow, wv, i * 32 + qq * RPP, RPP, voff, v);
            }
        }
    };

    // Packed bf16 epilogue.  acc[i][j][4g + e] is C at row i*32 + l32 and
    // column j*32 + 8g + 4*half + e of the wave tile: four consecutive columns,
    // which get their bias (+ GELU) and are rounded into one 8-byte pair of
    // bf16 words.  Per 32-row block, the wave's 32 rows x WN bf16 go through
    // its slot of LDS stage `cs` (16-byte chunk c of row r at c ^ (r & 7), so
    // neither the 8-byte writes down a column nor the 16-byte reads along the
    // rows collide on a bank) and leave as 16-byte row-contiguous stores.
    auto epilogue_packed = [&](int t, const float* cs_base) __attribute__((always_inline)) {
        const int u = u0 + t * ustep, split = u / ntiles, tile = u - split * ntiles;
        uint16_t* const Cs = reinterpret_cast<uint16_t*>(p.C) + (int64_t)split * p.split_stride;
        const int m0 = (tile / ntiles_n) * BM, n0 = (tile - (tile / ntiles_n) * ntiles_n) * BN;
        const float* bslot = smem + NSTAGE * STAGE + ((t & 1) * NW + wave) * BIAS_SLOT;
        char* cw = reinterpret_cast<char*>(const_cast<float*>(cs_base) + wave * (16 * WN));
        constexpr int CPW = WN / 8;               // 16-byte chunks per wave-tile row
        constexpr int NPASS = 32 * CPW / 64;
        const bool wide = (p.ldc & 7) == 0;       // rows 16-byte aligned
#pragma unroll
        for (int i = 0; i < FM; ++i) {
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    float4 v = make_float4(acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]);
                    if (HAS_BIAS) {
                        const float4 b4 = *reinterpret_cast<const float4*>(bslot + j * 32 + 8 * g + 4 * half);
                        v.x += b4.x; v.y += b4.y; v.z += b4.z; v.w += b4.w;
                    }
                    if constexpr (EPI == EPI_BIAS_GELU) {
                        v.x = gelu_tanh_fast(v.x); v.y = gelu_tanh_fast(v.y);
                        v.z = gelu_tanh_fast(v.z); v.w = gelu_tanh_fast(v.w);
                    }
                    const uint2 h = make_uint2(pack_bf16x2(v.x, v.y), pack_bf16x2(v.z, v.w));
                    *reinterpret_cast<uint2*>(cw + l32 * (2 * WN) + (((j * 4 + g) ^ (l32 & 7)) << 4) + 8 * half) = h;
                }
#pragma unroll
            for (int ps = 0; ps < NPASS; ++ps) {
                const int q = ps * 64 + lane, r = q / CPW, c = q - r * CPW;
                const uint4 d = *reinterpret_cast<const uint4*>(cw + r * (2 * WN) + ((c ^ (r & 7)) << 4));
                const int grow = m0 + wm * WM + i * 32 + r, gcol = n0 + wn * WN + 8 * c;
                if (grow < M && gcol < N) {   // N % 4 == 0: the chunk's first 4 columns are in
                    uint16_t* dst = Cs + (int64_t)grow * p.ldc + gcol;
                    if (wide && gcol + 8 <= N) {
                        // Streaming store: the output is consumed by a later
                        // kernel, not this one (bf16 products at c5: QKV 511 ->
                        // 499 us, FFN up 766 -> 749 us; the same hint on the fp32
                        // epilogues measured 1-2% slower and is not used there).
                        typedef unsigned int u4v __attribute__((ext_vector_type(4)));
                        __builtin_nontemporal_store(u4v{d.x, d.y, d.z, d.w}, reinterpret_cast<u4v*>(dst));
                    } else {
                        *reinterpret_cast<uint2*>(dst) = make_uint2(d.x, d.y);
                        if (gcol + 8 <= N) *reinterpret_cast<uint2*>(dst + 4) = make_uint2(d.z, d.w);
                    }
                }
            }
        }
    };

    // Packed bf16 epilogue of the 16x16x32 blocks: acc16[i][j][e] is C at
    // wave-tile row 16 i + r16, column 16 j + 4 q16 + e.  Two row blocks (32
    // rows) at a time go through the wave's LDS slot as in epilogue_packed.
    auto epilogue_packed16 = [&](int t, const float* cs_base) __attribute__((always_inline)) {
        const int u = u0 + t * ustep, split = u / ntiles, tile = u - split * ntiles;
        uint16_t* const Cs = reinterpret_cast<uint16_t*>(p.C) + (int64_t)split * p.split_stride;
        const int m0 = (tile / ntiles_n) * BM, n0 = (tile - (tile / ntiles_n) * ntiles_n) * BN;
        const float* bslot = smem + NSTAGE * STAGE + ((t & 1) * NW + wave) * BIAS_SLOT;
        char* cw = reinterpret_cast<char*>(const_cast<float*>(cs_base) + wave * (16 * WN));
        constexpr int CPW = WN / 8;               // 16-byte chunks per wave-tile row
        constexpr int NPASS = 32 * CPW / 64;
        const bool wide = (p.ldc & 7) == 0;       // rows 16-byte aligned
#pragma unroll
        for (int ip = 0; ip < FM16 / 2; ++ip) {
#pragma unroll
            for (int ii = 0; ii < 2; ++ii)
#pragma unroll
                for (int j = 0; j < FN16; ++j) {
                    const v4f a = acc16[2 * ip + ii][j];
                    float4 v = make_float4(a[0], a[1], a[2], a[3]);
                    if (HAS_BIAS) {
                        const float4 b4 = *reinterpret_cast<const float4*>(bslot + j * 16 + 4 * q16);
                        v.x += b4.x; v.y += b4.y; v.z += b4.z; v.w += b4.w;
                    }
                    if constexpr (EPI == EPI_BIAS_GELU) {
                        v.x = gelu_tanh_fast(v.x); v.y = gelu_tanh_fast(v.y);
                        v.z = gelu_tanh_fast(v.z); v.w = gelu_tanh_fast(v.w);
                    }
                    const uint2 h = make_uint2(pack_bf16x2(v.x, v.y), pack_bf16x2(v.z, v.w));
                    const int r = 16 * ii + r16;
                    *reinterpret_cast<uint2*>(cw + r * (2 * WN) + (((2 * j + (q16 >> 1)) ^ (r & 7)) << 4) +
                                              8 * (q16 & 1)) = h;
                }
#pragma unroll
            for (int ps = 0; ps < NPASS; ++ps) {
                const int q = ps * 64 + lane, r = q / CPW, c = q - r * CPW;
                const uint4 d = *reinterpret_cast<const uint4*>(cw + r * (2 * WN) + ((c ^ (r & 7)) << 4));
                const int grow = m0 + wm * WM + ip * 32 + r, gcol = n0 + wn * WN + 8 * c;
                if (grow < M && gcol < N) {   // N % 4 == 0: the chunk's first 4 columns are in
                    uint16_t* dst = Cs + (int64_t)grow * p.ldc + gcol;
                    if (wide && gcol + 8 <= N) {
                        typedef unsigned int u4v __attribute__((ext_vector_type(4)));
                        __builtin_nontemporal_store(u4v{d.x, d.y, d.z, d.w}, reinterpret_cast<u4v*>(dst));
                    } else {
                        *reinterpret_cast<uint2*>(dst) = make_uint2(d.x, d.y);
                        if (gcol + 8 <= N) *reinterpret_cast<uint2*>(dst + 4) = make_uint2(d.z, d.w);
                    }
                }
            }
        }
    };
    // fp32 output of the 16x16x32 blocks (the op-level bf16 GEMM with an fp32
    // C): each lane's four consecutive columns of a row as one float4 store.
    auto epilogue_direct16 = [&](int t) __attribute__((always_inline)) {
        const int u = u0 + t * ustep, split = u / ntiles, tile = u - split * ntiles;
        float* const Cs = p.C + (int64_t)split * p.split_stride;
        const int m0 = (tile / ntiles_n) * BM, n0 = (tile - (tile / ntiles_n) * ntiles_n) * BN;
        const float* bslot = smem + NSTAGE * STAGE + ((t & 1) * NW + wave) * BIAS_SLOT;
#pragma unroll
        for (int i = 0; i < FM16; ++i)
#pragma unroll
            for (int j = 0; j < FN16; ++j) {
                const v4f a = acc16[i][j];
                float4 v = make_float4(a[0], a[1], a[2], a[3]);
                if (HAS_BIAS) {
                    const float4 b4 = *reinterpret_cast<const float4*>(bslot + j * 16 + 4 * q16);
                    v.x += b4.x; v.y += b4.y; v.z += b4.z; v.w += b4.w;
                }
                if constexpr (EPI == EPI_BIAS_GELU) {
                    v.x = gelu_tanh_fast(v.x); v.y = gelu_tanh_fast(v.y);
                    v.z = gelu_tanh_fast(v.z); v.w = gelu_tanh_fast(v.w);
                }
                const int grow = m0 + wm * WM + 16 * i + r16, gcol = n0 + wn * WN + 16 * j + 4 * q16;
                if (grow < M && gcol < N) *reinterpret_cast<float4*>(Cs + (int64_t)grow * p.ldc + gcol) = v;
            }
    };

    auto finish_tile = [&](int t, float* stage) __attribute__((always_inline)) {
        if constexpr (LN) epilogue_ln(t, stage);
        else if constexpr (MF16 && OUT16) epilogue_packed16(t, stage);
        else if constexpr (MF16) epilogue_direct16(t);
        else if constexpr (PACKED) epilogue_packed(t, stage);
        else if constexpr (FLAT) epilogue_flat(t, stage);
        else epilogue_tile(t, stage);
    };

    // k-slice s + 1's fragments are read while slice s's MFMAs run (two
    // fragment sets in registers).  fp32 c3 forward 6.04 -> 6.00 ms against
    // reading each slice's just before its MFMAs.
    constexpr bool PREF = KS > 1;
    v4f afb[PREF ? 2 : 1][FM], wfb[PREF ? 2 : 1][FN];
    auto mfma_slice = [&](int b) __attribute__((always_inline)) {
        const v4f (&af)[FM] = afb[b];
        const v4f (&wf)[FN] = wfb[b];
        if constexpr (BF16) {
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = PACKED
                        ? __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                              __builtin_bit_cast(v8bf, wf[j]), __builtin_bit_cast(v8bf, af[i]), acc[i][j], 0, 0, 0)
                        : __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                              __builtin_bit_cast(v8bf, af[i]), __builtin_bit_cast(v8bf, wf[j]), acc[i][j], 0, 0, 0);
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int i = 0; i < FM; ++i)
#pragma unroll
                    for (int j = 0; j < FN; ++j)
                        acc[i][j] = PACKED
                            ? __builtin_amdgcn_mfma_f32_32x32x2f32(wf[j][q], af[i][q], acc[i][j], 0, 0, 0)
                            : __builtin_amdgcn_mfma_f32_32x32x2f32(af[i][q], wf[j][q], acc[i][j], 0, 0, 0);
        }
    };
    // The MFMAs of each k-tile's last slice (fragments already in registers,
    // set 1) wait until after the next k-tile's barrier and the issue of its
    // first fragment reads, so the MFMA pipes keep working through the
    // barrier and the latency of those reads.  At a tile's end they run
    // before its epilogue (after the next tile's first barrier, so also
    // there).  The first k-tile of a tile is peeled off, so that no MFMA sits
    // behind a branch on the k-tile index: accumulators merged from two paths
    // cost the register allocator a second copy of them.
    constexpr bool DEFER = PREF && KS % 2 == 0 && !SPLIT6;
    // MF16: a k-tile runs as steps of 16 MFMAs (256 cycles, as one 16-deep
    // slice of the 32x32 form), two per 32-deep slice: step s4 = 2 sl + h
    // multiplies the A blocks of half h of the wave tile's rows by the W
    // blocks of slice sl.  A step's A fragments are read during the previous step (two
    // sets); a slice's W fragments with its first step's A fragments (two
    // sets).  So the fragment registers stay those of the 32x32 form's two
    // sets (plus one W set), within two waves per SIMD.
    v4f a16b[2][FM16 / 2], w16b[2][FN16];
    auto mfma16 = [&](int s4) __attribute__((always_inline)) {
        const int sl = s4 >> 1, h = s4 & 1;
#pragma unroll
        for (int i = 0; i < FM16 / 2; ++i)
#pragma unroll
            for (int j = 0; j < FN16; ++j)
                acc16[h * (FM16 / 2) + i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    __builtin_bit_cast(v8bf, w16b[sl & 1][j]), __builtin_bit_cast(v8bf, a16b[s4 & 1][i]),
                    acc16[h * (FM16 / 2) + i][j], 0, 0, 0);
    };
    // The MFMAs deferred past the next k-tile's barrier: the last slice (or step).
    auto last_step = [&]() __attribute__((always_inline)) {
        if constexpr (MF16) mfma16(KS - 1);
        else mfma_slice(1);
    };
    if constexpr (DEFER) {
        if constexpr (MF16) {
#pragma unroll
            for (int i = 0; i < FM16 / 2; ++i) a16b[1][i] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int j = 0; j < FN16; ++j) w16b[1][j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
        } else {
#pragma unroll
            for (int i = 0; i < FM; ++i) afb[1][i] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int j = 0; j < FN; ++j) wfb[1][j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
        }
    }

    int it = 0;
    // Wait until k-tile `it` has landed in every wave's part: only the loads
    // issued after it may remain outstanding.
    auto enter_ktile = [&]() __attribute__((always_inline)) {
        int after = 0;
        for (int j = it + 1; j < nit; ++j) after += n_issued(j);
        if constexpr (D == 1)   // one k-tile ahead: after is 0, NL or NL + 1
            wait_vmcnt_of<NL + (HAS_BIAS ? 1 : 0), NL>(after);
        else
            wait_vmcnt(after);
        lds_barrier();
    };
    // The MFMAs of k-tile `it` (its loads have landed), and the loads of a
    // later k-tile spread over its first slices.
    auto run_ktile = [&](auto first) __attribute__((always_inline)) {
        const bool refill = nit < total;
        const float* st = smem + (it % NSTAGE) * STAGE;
        auto rd = [&](int s, int b) __attribute__((always_inline)) {
            const int ko = 4 * ((2 * s + half) ^ sw);
#pragma unroll
            for (int i = 0; i < FM; ++i)
                afb[b][i] = *reinterpret_cast<const v4f*>(st + a_row + i * 32 * RW + ko);
#pragma unroll
            for (int j = 0; j < FN; ++j)
                wfb[b][j] = *reinterpret_cast<const v4f*>(st + w_row + j * 32 * RW + ko);
        };
        if constexpr (SPLIT6) {
            static_assert(!BF16 && KS % 2 == 0, "split products: fp32 tiles of whole 16-deep slices");
            // fp32 A and W fragments, split in registers into bf16 parts
            // h + m + l; six bf16 MFMAs per block and 16-deep slice (the
            // smallest products first).  Lane half h takes k = 16 sp +
            // 8 h .. +7: fp32 chunks 4 sp + 2 h and 4 sp + 2 h + 1.
#pragma unroll
            for (int sp = 0; sp < KS / 2; ++sp) {
                if (refill && sp < NPART) issue_part(sp);
                const int c0 = 4 * sp + 2 * half;
                const int ko0 = 4 * (c0 ^ sw), ko1 = 4 * ((c0 + 1) ^ sw);
                v8bf wh[FN], wm[FN], wl[FN];
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    split3_bf16(*reinterpret_cast<const v4f*>(st + w_row + j * 32 * RW + ko0),
                                *reinterpret_cast<const v4f*>(st + w_row + j * 32 * RW + ko1), wh[j], wm[j], wl[j]);
#pragma unroll
                for (int i = 0; i < FM; ++i) {
                    v8bf ah, am, al;
                    split3_bf16(*reinterpret_cast<const v4f*>(st + a_row + i * 32 * RW + ko0),
                                *reinterpret_cast<const v4f*>(st + a_row + i * 32 * RW + ko1), ah, am, al);
#pragma unroll
                    for (int j = 0; j < FN; ++j) {
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, wh[j], acc[i][j], 0, 0, 0);
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(am, wm[j], acc[i][j], 0, 0, 0);
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, wl[j], acc[i][j], 0, 0, 0);
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(am, wh[j], acc[i][j], 0, 0, 0);
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, wm[j], acc[i][j], 0, 0, 0);
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, wh[j], acc[i][j], 0, 0, 0);
                    }
                }
            }
        } else if constexpr (MF16) {
            static_assert(KS == 2 * (BK / 32), "two steps per 32-deep slice");
            auto rd16 = [&](int s4, int b) __attribute__((always_inline)) {
                const int sl = s4 >> 1, h = s4 & 1;
                const int ko = 4 * ((4 * sl + q16) ^ sw16);
#pragma unroll
                for (int i = 0; i < FM16 / 2; ++i)
                    a16b[b][i] = *reinterpret_cast<const v4f*>(st + a_row16 + (h * (FM16 / 2) + i) * 16 * RW + ko);
                if (h == 0) {
#pragma unroll
                    for (int j = 0; j < FN16; ++j)
                        w16b[sl & 1][j] = *reinterpret_cast<const v4f*>(st + w_row16 + j * 16 * RW + ko);
                }
            };
            rd16(0, 0);
            if constexpr (DEFER && !decltype(first)::value) mfma16(KS - 1);   // k-tile it - 1's last step
#pragma unroll
            for (int s4 = 0; s4 < KS; ++s4) {
                if (refill && s4 < NPART) issue_part(s4);
                if (s4 + 1 < KS) rd16(s4 + 1, (s4 + 1) & 1);
                if (!(DEFER && s4 == KS - 1)) mfma16(s4);
            }
        } else {
            if (PREF) rd(0, 0);
            if constexpr (DEFER && !decltype(first)::value) mfma_slice(1);   // k-tile it - 1's last slice
#pragma unroll
            for (int s = 0; s < KS; ++s) {
                if (refill && s < NPART) issue_part(s);
                if (!PREF) rd(s, 0);
                else if (s + 1 < KS) rd(s + 1, (s + 1) & 1);
                if (!(DEFER && s == KS - 1)) mfma_slice(PREF ? (s & 1) : 0);
            }
        }
    };

    point_at(0);
#pragma unroll
    for (int d = 0; d < D; ++d)
        if (nit < total) issue();
    for (int t = 0; t < my_tiles; ++t) {
        enter_ktile();
        if constexpr (DEFER && !LN) last_step();   // the previous tile's last slice (zeros at t = 0)
        if (!LN && t > 0) {
            finish_tile(t - 1, smem + ((it - 1) % NSTAGE) * STAGE);
            lds_barrier();  // the stage is refilled by the loads below
        }
        if constexpr (MF16) {
#pragma unroll
            for (int i = 0; i < FM16; ++i)
#pragma unroll
                for (int j = 0; j < FN16; ++j) acc16[i][j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
        } else {
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
        }
        run_ktile(std::true_type{});
        ++it;
        for (int kt = 1; kt < nk; ++kt, ++it) {
            enter_ktile();
            run_ktile(std::false_type{});
        }
        // EPI_ADD_LN: one epilogue site, at the end of each tile (the next
        // tile's first k-tile is already on its way into the other stage).
        if constexpr (LN) {
            if constexpr (DEFER) mfma_slice(1);
            lds_barrier();  // every wave is done with this tile's last stage
            finish_tile(t, smem + ((it - 1) % NSTAGE) * STAGE);
            lds_barrier();  // that stage is refilled next
        }
    }
    if constexpr (!LN) {
        if constexpr (DEFER) last_step();
        lds_barrier();  // every wave is done with the last k-tile's stage
        finish_tile(my_tiles - 1, smem + ((it - 1) % NSTAGE) * STAGE);
    }
}

// ---------------------------------------------------------------------------
// bf16 products with bf16 outputs (every Linear of a bf16 model): 256 x 256
// C tiles, 64-deep k-tiles, 8 waves of 128 x 64 on v_mfma_f32_16x16x32_bf16,
// persistent over a strided list of tiles (one workgroup per CU).
//
// Measured on MI355X, the 2-stage kernel above loses its time at three places
// besides the MFMAs: waiting for the k-tile's loads (the A panels stream from
// HBM, and one k-tile of lookahead leaves their latency exposed: 9-15% of a
// wave's cycles, up to 37% at a higher clock), the epilogue's stores (a CU
// issues stores at ~25 B/clk, so a 128 KB output tile takes ~5k cycles, and
// the next k-tile's loads queue behind them in the in-order vmcnt), and the
// GELU.  This kernel:
//  * keeps A k-tiles in a ring of three LDS stages (two k-tiles in flight
//    ahead) and W k-tiles, which the L2 / last-level cache holds, in a ring of
//    two: 3 x 32 KB + 2 x 32 KB, the whole 160 KB;
//  * starts each tile's accumulators at its bias (the bias row segment rides
//    into the freed A stage with the tile's first k-tile), so the epilogue
//    adds nothing and needs no LDS of its own beyond that stage;
//  * issues the next W k-tile before the epilogue's stores and counts every
//    vector memory instruction it issues (the stores are buffer stores whose
//    rows past M or columns past N get an offset past the descriptor's end,
//    so every lane issues every store and the count is exact).  The next
//    k-tile then waits for its W without waiting for the stores, which drain
//    during its MFMAs and are only waited for a k-tile later.
// Load order per k-tile j: W(j + 1), then A(j + 2) (at a tile's first k-tile:
// the bias, W(j + 1), the stores, then A(j + 2)).  Waiting for W(j) covers
// A(j) too, which was issued before it.
// ---------------------------------------------------------------------------
template <int EPI>
__global__ __launch_bounds__(512) void gemm_bf16_ring_kernel(GemmArgs p) {
    constexpr int BM = 256, BN = 256, BK = 64, NT = 512, WAVES_N = 4;
    constexpr int WM = 128, WN = 64, FM16 = WM / 16, FN16 = WN / 16, HALF = FM16 / 2;
    constexpr int CPR = BK / 8, RW = 4 * CPR;     // 16-byte chunks / 4-byte words per tile row
    constexpr int SA = BM * RW, SW = BN * RW;     // words per A / W stage
    constexpr int LA = BM * CPR / NT, LW = BN * CPR / NT;
    static_assert(LA == LW, "A and W tiles share the lane load pattern");
    constexpr int EROWS = 16;                     // C rows per epilogue pass (one row block)
    constexpr int CPW = WN / 8;                   // 16-byte chunks per wave-tile row
    constexpr int ST_PASS = EROWS * CPW / 64;     // stores per lane per pass
    constexpr int N_ST = FM16 * ST_PASS;          // stores per lane per tile
    constexpr int STAGE_WORDS = 512, BIAS_WORDS = 256;   // per wave, within the freed A stage
    static_assert(8 * STAGE_WORDS + 8 * BIAS_WORDS <= SA, "epilogue staging and bias fit one A stage");
    constexpr bool HAS_BIAS = EPI != EPI_NONE;
    __shared__ __attribute__((aligned(16))) float smem[3 * SA + 2 * SW];
    float* const sA = smem;
    float* const sW = smem + 3 * SA;

    const int M = p.M_dev ? *p.M_dev : p.M_max;
    const int N = p.N;
    const int ntiles_n = (N + BN - 1) / BN;
    const int ntiles = ((M + BM - 1) / BM) * ntiles_n;
    const int nk = p.K / BK;
    const int G = gridDim.x;
    const int wg = (G & 7) == 0 ? (blockIdx.x & 7) * (G >> 3) + (blockIdx.x >> 3) : blockIdx.x;
    const int my_tiles = wg < ntiles ? (ntiles - wg + G - 1) / G : 0;
    const int total = my_tiles * nk;
    if (total == 0) return;  // uniform over the workgroup

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;
    const char* __restrict__ A = static_cast<const char*>(p.A);
    const char* __restrict__ W = static_cast<const char*>(p.W);

    // Lane share of each k-tile load (A and W alike): LDS chunk i*NT + tid,
    // tile row r, holding global chunk (position ^ swizzle(r)).
    int l_r[LA], l_c[LA];
#pragma unroll
    for (int i = 0; i < LA; ++i) {
        const int P = i * NT + tid;
        l_r[i] = P / CPR;
        l_c[i] = 8 * ((P % CPR) ^ chunk_swizzle16<CPR>(P / CPR));   // elements
    }
    // Load cursors: the next A / W k-tile to load (global iteration index),
    // its panel base (wave-uniform) and this lane's 32-bit byte offsets.
    int ia = 0, iw = 0;
    uint64_t abase = 0, wbase = 0;
    uint32_t aoff[LA], woff[LA];
    auto a_seek = [&](int x) __attribute__((always_inline)) {
        const int ti = x / nk, kt = x - ti * nk;
        const int m0 = ((wg + ti * G) / ntiles_n) * BM;
#pragma unroll
        for (int i = 0; i < LA; ++i) aoff[i] = (uint32_t)(((min(m0 + l_r[i], M - 1) - m0) * p.lda + l_c[i]) * 2);
        abase = uniform_u64(A + ((int64_t)m0 * p.lda + (int64_t)kt * BK) * 2);
    };
    auto w_seek = [&](int x) __attribute__((always_inline)) {
        const int ti = x / nk, kt = x - ti * nk;
        const int n0 = ((wg + ti * G) % ntiles_n) * BN;
#pragma unroll
        for (int i = 0; i < LA; ++i) woff[i] = (uint32_t)(((min(n0 + l_r[i], N - 1) - n0) * p.ldw + l_c[i]) * 2);
        wbase = uniform_u64(W + ((int64_t)n0 * p.ldw + (int64_t)kt * BK) * 2);
    };
    // Vector memory instructions this wave has issued (loads, bias, stores)
    // and the count right after the last W k-tile / bias load.
    int vm = 0, w_mark = 0, b_mark = 0;
    auto issue_a = [&]() __attribute__((always_inline)) {
        if (ia >= total) return;
        float* st = sA + (ia % 3) * SA;
#pragma unroll
        for (int i = 0; i < LA; ++i) load_lds16_sbase(abase, aoff[i], st + (i * NT + wave * 64) * 4);
        vm += LA;
        if (++ia < total) {
            if (ia % nk == 0) a_seek(ia);
            else abase += BK * 2;
        }
    };
    auto issue_w = [&]() __attribute__((always_inline)) {
        if (iw >= total) return;
        float* st = sW + (iw & 1) * SW;
#pragma unroll
        for (int i = 0; i < LA; ++i) load_lds16_sbase(wbase, woff[i], st + (i * NT + wave * 64) * 4);
        vm += LA;
        w_mark = vm;
        if (++iw < total) {
            if (iw % nk == 0) w_seek(iw);
            else wbase += BK * 2;
        }
    };
    // Bias of local tile t, this wave's 64 columns (lanes past them load
    // clamped copies), into the wave's slot of A stage `st`.
    auto issue_bias = [&](int t, float* st) __attribute__((always_inline)) {
        const int n0 = ((wg + t * G) % ntiles_n) * BN;
        load_lds16_async(p.bias + min(n0 + wn * WN + 4 * lane, N - 4), st + 8 * STAGE_WORDS + wave * BIAS_WORDS);
        vm += 1;
        b_mark = vm;
    };

    const int r16 = lane & 15, q16 = lane >> 4;
    const int sw16 = chunk_swizzle16<CPR>(r16);
    const int a_row16 = (wm * WM + r16) * RW, w_row16 = (wn * WN + r16) * RW;
    v4f acc16[FM16][FN16];
    v4f a16b[2][HALF], w16b[2][FN16];
    // Step s4 = 2 sl + h of a k-tile: the A blocks of row half h against the
    // W blocks of 32-deep slice sl (fragments read a step ahead, two sets).
    auto mfma16 = [&](int s4) __attribute__((always_inline)) {
        const int sl = s4 >> 1, h = s4 & 1;
#pragma unroll
        for (int i = 0; i < HALF; ++i)
#pragma unroll
            for (int j = 0; j < FN16; ++j)
                acc16[h * HALF + i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    __builtin_bit_cast(v8bf, w16b[sl & 1][j]), __builtin_bit_cast(v8bf, a16b[s4 & 1][i]),
                    acc16[h * HALF + i][j], 0, 0, 0);
    };
    auto rd16 = [&](const float* stA, const float* stW, int s4, int b) __attribute__((always_inline)) {
        const int sl = s4 >> 1, h = s4 & 1;
        const int ko = 4 * ((4 * sl + q16) ^ sw16);
#pragma unroll
        for (int i = 0; i < HALF; ++i)
            a16b[b][i] = *reinterpret_cast<const v4f*>(stA + a_row16 + (h * HALF + i) * 16 * RW + ko);
        if (h == 0) {
#pragma unroll
            for (int j = 0; j < FN16; ++j)
                w16b[sl & 1][j] = *reinterpret_cast<const v4f*>(stW + w_row16 + j * 16 * RW + ko);
        }
    };
    // The MFMAs of global k-tile j; the last step is left for after the next
    // barrier.  Away from a tile's first k-tile the previous k-tile's last
    // step runs first and the loads W(j + 1), A(j + 2) go out with steps 0, 1.
    auto run_ktile = [&](int j, bool first) __attribute__((always_inline)) {
        const float* stA = sA + (j % 3) * SA;
        const float* stW = sW + (j & 1) * SW;
        rd16(stA, stW, 0, 0);
        if (!first) mfma16(3);
#pragma unroll
        for (int s4 = 0; s4 < 3; ++s4) {
            if (!first && s4 == 0) issue_w();
            if (!first && s4 == 1) issue_a();
            rd16(stA, stW, s4 + 1, (s4 + 1) & 1);
            mfma16(s4);
        }
    };

    // Epilogue of local tile t (GELU or nothing: the bias is in the
    // accumulators), one 16-row block at a time through the wave's 2 KB of
    // the freed A stage `st`, then 16-byte buffer stores of whole row chunks.
    // Every address is a lane constant of the epilogue plus a compile-time
    // step: a store's descriptor starts at its 8-row group and ends at row M,
    // so the lane offset (row within the group, column) is the same for all
    // of the tile's stores, and rows past M fall outside the descriptor.
    static_assert(CPW == 8 && ST_PASS * 64 == EROWS * CPW, "a store pass is 8 rows of 8 chunks");
    auto epilogue = [&](int t, float* st) __attribute__((always_inline)) {
        const int u = wg + t * G;
        const int ws = __builtin_amdgcn_readfirstlane(wave);
        const int wrow = (u / ntiles_n) * BM + (ws / WAVES_N) * WM;   // the wave tile's first C row
        const int n0 = (u % ntiles_n) * BN;
        // Lane-derived values opaque here: formed at the epilogue, not held
        // across the k-loop (the last tile's epilogue follows it).
        int el = lane;
        asm volatile("" : "+v"(el));
        const int er = el & 15, eq = el >> 4;   // C fragment: row er, columns 4 eq .. 4 eq + 3 of a block
        const int sr = el >> 3, sc = el & 7;    // store: row sr of an 8-row group, 16-byte chunk sc
        char* const cw = reinterpret_cast<char*>(st + ws * STAGE_WORDS);
        // Fragment writes: row er, chunk (2 j + eq / 2) ^ (er & 7), half eq & 1;
        // 2 j + b = 2 j ^ b for b < 2, so the chunk's byte offset is wx ^ 32 j.
        char* const wr = cw + er * (2 * WN) + 8 * (eq & 1);
        const int wx = ((eq >> 1) ^ (er & 7)) << 4;
        // Row reads: row 8 ps + sr, chunk sc ^ sr.
        const char* const rd = cw + sr * (2 * WN) + ((sc ^ sr) << 4);
        const int col = n0 + (ws % WAVES_N) * WN + 8 * sc;
        const uint32_t voff = col < N ? (uint32_t)((sr * p.ldc + col) * 2) : 0xFFFFFFF0u;
        // Rows of the wave tile that exist (at most WM; <= 0 past M), and the
        // bytes of a C row: wave-uniform, so the descriptors stay scalar (a
        // descriptor in VGPRs makes the compiler loop over the lanes).
        const int wv = __builtin_amdgcn_readfirstlane(M - wrow);
        const int rowb = p.ldc * 2;
        uint16_t* const cbase = reinterpret_cast<uint16_t*>(p.C);
#pragma unroll
        for (int i = 0; i < FM16; ++i) {
#pragma unroll
            for (int j = 0; j < FN16; ++j) {
                const v4f a = acc16[i][j];
                float4 v = make_float4(a[0], a[1], a[2], a[3]);
                if constexpr (EPI == EPI_BIAS_GELU) {
                    v.x = gelu_tanh_fast(v.x); v.y = gelu_tanh_fast(v.y);
                    v.z = gelu_tanh_fast(v.z); v.w = gelu_tanh_fast(v.w);
                }
                const uint2 h = make_uint2(pack_bf16x2(v.x, v.y), pack_bf16x2(v.z, v.w));
                *reinterpret_cast<uint2*>(wr + (wx ^ (32 * j))) = h;
            }
#pragma unroll
            for (int ps = 0; ps < ST_PASS; ++ps) {
                const uint4 d = *reinterpret_cast<const uint4*>(rd + ps * 8 * (2 * WN));
                const int r0 = i * EROWS + ps * 8;                    // the group's first row in the wave tile
                const int left = wv - r0;
                const int bytes = left >= 8 ? 8 * rowb : (left > 0 ? left * rowb : 0);
                const __amdgpu_buffer_rsrc_t cr = __builtin_amdgcn_make_buffer_rsrc(
                    cbase + (int64_t)(wrow + r0) * p.ldc, (short)0, bytes, BUFFER_RSRC_WORD3);
                typedef unsigned int u4v __attribute__((ext_vector_type(4)));
                __builtin_amdgcn_raw_buffer_store_b128(u4v{d.x, d.y, d.z, d.w}, cr, voff, 0, 2 /* nt */);
            }
        }
        vm += N_ST;
    };

    // Prologue: bias(0) into the stage A(2) will take, A(0), W(0), A(1).
    a_seek(0);
    w_seek(0);
    if (HAS_BIAS) issue_bias(0, sA + 2 * SA);
    issue_a();
    issue_w();
    issue_a();
    int j = 0;
    // Counts that occur after W(j): A(j + 1), and the stores and A(j + 1)
    // when j - 1 was a tile's first k-tile; after the bias: W(j + 1) and the
    // stores.
    auto wait_after = [&](int n) __attribute__((always_inline)) { wait_vmcnt_of<N_ST + LA, N_ST, LA>(n); };
    for (int t = 0; t < my_tiles; ++t) {
        // First k-tile of tile t: W(j) (and so A(j) and the bias) landed.
        wait_after(vm - w_mark);
        lds_barrier();
        float* freed = sA + ((j + 2) % 3) * SA;   // A stage of k-tile j - 1
        if (t > 0) {
            if (HAS_BIAS) issue_bias(t, freed);
            mfma16(3);                 // tile t - 1's last step
        }
        issue_w();                     // W(j + 1), before the stores
        if (t > 0) {
            epilogue(t - 1, freed);
            if (HAS_BIAS) wait_after(vm - b_mark);
        }
        if constexpr (HAS_BIAS) {
            const float* bs = freed + 8 * STAGE_WORDS + wave * BIAS_WORDS;
#pragma unroll
            for (int jj = 0; jj < FN16; ++jj) {
                const v4f b4 = *reinterpret_cast<const v4f*>(bs + 16 * jj + 4 * q16);
#pragma unroll
                for (int i = 0; i < FM16; ++i) acc16[i][jj] = b4;
            }
        } else {
#pragma unroll
            for (int i = 0; i < FM16; ++i)
#pragma unroll
                for (int jj = 0; jj < FN16; ++jj) acc16[i][jj] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
        }
        lds_barrier();                 // the freed stage is refilled next
        issue_a();                     // A(j + 2)
        run_ktile(j, true);
        ++j;
        for (int kt = 1; kt < nk; ++kt, ++j) {
            wait_after(vm - w_mark);
            lds_barrier();
            run_ktile(j, false);
        }
    }
    mfma16(3);
    lds_barrier();
    epilogue(my_tiles - 1, sA + ((j + 2) % 3) * SA);
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
// Few-token products (M_max <= 64: a handful of short sentences).  Such a
// product is a chain of memory round trips rather than MFMA work, so each
// weight byte is read once per 16-row block (the few activation rows stay in
// cache) and the work is spread over as many workgroups as the shape gives:
// workgroup (32-column slice, 16-row block, k split s)
// runs NW waves, wave w taking k in [s*K/S + w*KW, s*K/S + (w+1)*KW), KW =
// K / (NW*S), with all of a wave's loads in flight at once when KW <=
// 16*NSTEP.  v_mfma_f32_16x16x4_f32: lane l gives A row l % 16 and W row
// (output column) l % 16 at k = kb + 4 (l / 16) + e for e = 0..3 of one
// float4, so A and W pair the same k; each lane then holds rows 4 (l / 16) +
// i, i = 0..3, of column l % 16.  The wave sums are added through LDS in wave
// order, then either the bias (+ GELU) is applied (one split), or split s is
// stored at C + s * split_stride (EPI_NONE: the LayerNorm that follows adds
// the splits in order).
// ---------------------------------------------------------------------------
template <int EPI, int NSTEP, int NW>
__global__ __launch_bounds__(64 * NW) void gemm_skinny_kernel(GemmArgs p) {
    typedef float v4f_t __attribute__((ext_vector_type(4)));
    __shared__ __attribute__((aligned(16))) float red[NW][16][32];
    const int M = p.M_dev ? *p.M_dev : p.M_max;
    const int N = p.N, K = p.K;
    const int S = p.splits > 1 ? p.splits : 1;
    const int nslices = N / 32;
    const int blk = blockIdx.x, nb = blk % nslices, m0 = (blk / nslices) * 16, n0 = nb * 32;
    const int split = blockIdx.y;
    if (m0 >= M) return;  // uniform over the workgroup
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r = lane & 15, q = lane >> 4;
    const int KW = K / (NW * S);
    const int kb = split * (K / S) + wave * KW + 4 * q;
    const float* Ar = static_cast<const float*>(p.A) + (int64_t)min(m0 + r, M - 1) * p.lda + kb;
    const float* W0 = static_cast<const float*>(p.W) + (int64_t)(n0 + r) * p.ldw + kb;
    const float* W1 = W0 + 16 * p.ldw;
    v4f_t acc0 = {0.0f, 0.0f, 0.0f, 0.0f}, acc1 = acc0;
    for (int k = 0; k < KW; k += 16 * NSTEP) {
        float4 a[NSTEP], w0[NSTEP], w1[NSTEP];
#pragma unroll
        for (int j = 0; j < NSTEP; ++j) {
            a[j] = *reinterpret_cast<const float4*>(Ar + k + 16 * j);
            w0[j] = *reinterpret_cast<const float4*>(W0 + k + 16 * j);
            w1[j] = *reinterpret_cast<const float4*>(W1 + k + 16 * j);
        }
#pragma unroll
        for (int j = 0; j < NSTEP; ++j) {
            const float av[4] = {a[j].x, a[j].y, a[j].z, a[j].w};
            const float b0[4] = {w0[j].x, w0[j].y, w0[j].z, w0[j].w};
            const float b1[4] = {w1[j].x, w1[j].y, w1[j].z, w1[j].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(av[e], b0[e], acc0, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(av[e], b1[e], acc1, 0, 0, 0);
            }
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        red[wave][4 * q + i][r] = acc0[i];
        red[wave][4 * q + i][16 + r] = acc1[i];
    }
    __syncthreads();
    // Element pairs e = t, t + 64 NW, ... of the 16 x 32 block: row e / 16,
    // columns 2 (e % 16) .. +1.
    for (int e = tid; e < 256; e += 64 * NW) {
        const int row = e >> 4, col = 2 * (e & 15);
        const int grow = m0 + row, gcol = n0 + col;
        if (grow >= M) continue;
        float2 v = *reinterpret_cast<const float2*>(&red[0][row][col]);
#pragma unroll
        for (int w = 1; w < NW; ++w) {
            const float2 pw = *reinterpret_cast<const float2*>(&red[w][row][col]);
            v.x += pw.x;
            v.y += pw.y;
        }
        if constexpr (EPI != EPI_NONE) {
            const float2 b2 = *reinterpret_cast<const float2*>(p.bias + gcol);
            v.x += b2.x;
            v.y += b2.y;
            if constexpr (EPI == EPI_BIAS_GELU) {
                v.x = gelu_tanh_fast(v.x);
                v.y = gelu_tanh_fast(v.y);
            }
        }
        *reinterpret_cast<float2*>(p.C + split * p.split_stride + (int64_t)grow * p.ldc + gcol) = v;
    }
}

bool gemm_f32_skinny_fits(int M_max, int N, int K) {
    return M_max > 0 && M_max <= SKINNY_MAX_ROWS && N % 32 == 0 && K % 64 == 0 && K > 0;
}

template <int EPI, int NW>
static hipError_t launch_skinny_nw(const GemmArgs& a, hipStream_t s) {
    const int S = a.splits > 1 ? a.splits : 1;
    const int steps = a.K / (16 * NW * S);        // 16-deep steps per wave
    const dim3 grid((a.N / 32) * ((a.M_max + 15) / 16), S), block(64 * NW);
    if (steps % 4 == 0) hipLaunchKernelGGL((gemm_skinny_kernel<EPI, 4, NW>), grid, block, 0, s, a);
    else if (steps % 3 == 0) hipLaunchKernelGGL((gemm_skinny_kernel<EPI, 3, NW>), grid, block, 0, s, a);
    else if (steps % 2 == 0) hipLaunchKernelGGL((gemm_skinny_kernel<EPI, 2, NW>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((gemm_skinny_kernel<EPI, 1, NW>), grid, block, 0, s, a);
    return hipGetLastError();
}

// 8 waves when each still gets a whole 16-deep step, else 4 (K % (64 S) == 0).
template <int EPI>
static hipError_t launch_skinny_epi(const GemmArgs& a, hipStream_t s) {
    const int S = a.splits > 1 ? a.splits : 1;
    return a.K % (128 * S) == 0 ? launch_skinny_nw<EPI, 8>(a, s) : launch_skinny_nw<EPI, 4>(a, s);
}

static hipError_t launch_skinny(const GemmArgs& a, int epi, hipStream_t s) {
    switch (epi) {
        case EPI_BIAS: return launch_skinny_epi<EPI_BIAS>(a, s);
        case EPI_BIAS_GELU: return launch_skinny_epi<EPI_BIAS_GELU>(a, s);
        case EPI_NONE: return launch_skinny_epi<EPI_NONE>(a, s);
        default: return hipErrorInvalidValue;
    }
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
template <int BM, int BN, int BK, int WAVES_M, int WAVES_N, bool BF16, bool KFULL = false>
static hipError_t launch_tile(const GemmArgs& a, int epi, hipStream_t s) {
    const int mt = (a.M_max + BM - 1) / BM, nt = (a.N + BN - 1) / BN;
    const dim3 grid(mt * nt), block(64 * WAVES_M * WAVES_N);
    if (mt == 0 || nt == 0) return hipSuccess;
    switch (epi) {
#define EBH_CASE(E)                                                                           \
    case E:                                                                                   \
        if constexpr (BF16)                                                                   \
            hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, BK, WAVES_M, WAVES_N, E>), grid,     \
                               block, 0, s, a);                                               \
        else                                                                                  \
            hipLaunchKernelGGL((gemm_f32_kernel<BM, BN, BK, WAVES_M, WAVES_N, E, KFULL>),     \
                               grid, block, 0, s, a);                                         \
        break;
        EBH_CASE(EPI_BIAS)
        EBH_CASE(EPI_BIAS_GELU)
        EBH_CASE(EPI_BIAS_RESID)
        EBH_CASE(EPI_NONE)
#undef EBH_CASE
        default:
            return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// Persistent launch: min(tiles, CUs) workgroups (one per CU: the two LDS
// stages take 128 KB at BK = 64).
int device_cu_count() {
    static int n = 0;
    if (n == 0) {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
            n = v;
        else
            n = 256;
    }
    return n;
}

static int cu_count() { return device_cu_count(); }

template <int BM, int BN, int BK, int WAVES_M, int WAVES_N, int NSTAGE, bool BF16, bool OUT16, bool SPLIT6,
          bool MF16 = BF16 && !SPLIT6>
static hipError_t launch_persistent_kernel(const GemmArgs& a, int epi, hipStream_t s, int wg_per_cu);

template <int BM, int BN, int BK, int WAVES_M, int WAVES_N, int NSTAGE, bool BF16 = false, bool OUT16 = false>
static hipError_t launch_persistent(const GemmArgs& a, int epi, hipStream_t s, int wg_per_cu = 1) {
    if constexpr (!BF16 && (BK / 4) % 4 == 0)
        if (a.split6) return launch_persistent_kernel<BM, BN, BK, WAVES_M, WAVES_N, NSTAGE, false, OUT16, true>(a, epi, s, wg_per_cu);
    return launch_persistent_kernel<BM, BN, BK, WAVES_M, WAVES_N, NSTAGE, BF16, OUT16, false>(a, epi, s, wg_per_cu);
}

template <int BM, int BN, int BK, int WAVES_M, int WAVES_N, int NSTAGE, bool BF16, bool OUT16, bool SPLIT6,
          bool MF16>
static hipError_t launch_persistent_kernel(const GemmArgs& a, int epi, hipStream_t s, int wg_per_cu) {
    // One work item per tile and k-split.
    const int64_t items = (int64_t)((a.M_max + BM - 1) / BM) * ((a.N + BN - 1) / BN) * (a.splits > 1 ? a.splits : 1);
    if (items == 0) return hipSuccess;
    const int grid = (int)std::min<int64_t>(items, (int64_t)cu_count() * wg_per_cu);
    const dim3 block(64 * WAVES_M * WAVES_N);
    switch (epi) {
        case EPI_BIAS:
            hipLaunchKernelGGL((gemm_persistent_kernel<BF16, OUT16, BM, BN, BK, WAVES_M, WAVES_N, NSTAGE, EPI_BIAS, SPLIT6, MF16>), dim3(grid), block, 0, s, a);
            break;
        case EPI_BIAS_GELU:
            hipLaunchKernelGGL((gemm_persistent_kernel<BF16, OUT16, BM, BN, BK, WAVES_M, WAVES_N, NSTAGE, EPI_BIAS_GELU, SPLIT6, MF16>), dim3(grid), block, 0, s, a);
            break;
        case EPI_NONE:
            hipLaunchKernelGGL((gemm_persistent_kernel<BF16, OUT16, BM, BN, BK, WAVES_M, WAVES_N, NSTAGE, EPI_NONE, SPLIT6, MF16>), dim3(grid), block, 0, s, a);
            break;
        default:
            return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// fp32 dispatch.  The persistent kernels need 16-byte aligned rows and
// operands, N % 4 == 0 (float4 epilogue), K a multiple of their k-tile with
// at least NSTAGE - 1 k-tiles, and no residual operand; anything else takes
// the guarded register-staged kernel.
hipError_t launch_gemm_f32(const GemmArgs& a, int epi, hipStream_t s) {
    const bool ok = epi != EPI_BIAS_RESID && aligned16(a.A) && aligned16(a.W) && aligned16(a.C) &&
                    (epi == EPI_NONE || aligned16(a.bias)) && a.lda % 4 == 0 && a.ldw % 4 == 0 &&
                    a.ldc % 4 == 0 && a.N % 4 == 0 && gemm_offsets_fit32(a.lda, a.ldw, 4);
    // Tile choice measured on MI355X at MiniLM shapes (M = 2.4k .. 32k tokens):
    //  * few tokens (under half a 128 x 128 tile per CU, e.g. the narrow
    //    projections of batch 32 of short sentences): 64 x 64 tiles, two
    //    workgroups per CU, so most CUs have work and their SIMDs a second wave;
    //  * outputs made of whole 256-column panels with at least one 256 x 256
    //    tile per CU (FFN up at 32k tokens): 256 x 256 tiles, 32-deep k-tiles,
    //    8 waves of 128 x 64 (FFN up 321 -> 314 us);
    //  * otherwise outputs made of whole 192-column panels with at least one
    //    256 x 192 tile per CU (QKV at 32k tokens): 256 x 192 tiles, 32-deep
    //    k-tiles, 8 waves of 64 x 96.  Both wide tiles load far fewer bytes per
    //    flop than 128 x 128 (QKV 297 -> 262 us at 128 x 384, 252 -> 243 us
    //    at 256 x 192; FFN up 338 -> 319 us at 128 x 384);
    //  * but where either wide tile would make fewer than two rounds of
    //    workgroups by the padded row count, and N is whole 96-column panels:
    //    128 x 96 tiles, 32-deep k-tiles, 4 waves of 32 x 96, two workgroups
    //    per CU.  A wide tile's round is all or nothing: 1.1 rounds cost two
    //    (FFN up at 9,216 rows: 145.8 us on 256 x 192, 101.8 on 128 x 96; QKV
    //    at 12,288: 142.0 against 94.1), and a padded batch whose real rows
    //    fill three quarters of one round still takes the whole round (FFN up
    //    at 6,124 of 8,192 rows: 80.1 against 66.0 us).  The wide tiles are
    //    ahead only on a round filled exactly (FFN up at 8,192 dense rows:
    //    83.8 against 88.1 us);
    //  * wide outputs over a short K with many tiles per CU: 32-deep k-tiles,
    //    two workgroups per CU, so one workgroup's GELU epilogue runs beside
    //    the other's MFMAs;
    //  * where 128 x 128 tiles would need more than one round by the padded
    //    row count but 128 x 96 tiles come to at most 1.5 per CU (N whole
    //    96-column panels): those, two workgroups per CU.  The busiest CU then
    //    has 0.75 of a 128 x 128 tile's work if the real rows fill one round,
    //    1.5 of it if they fill more, against 1 or 2 (QKV at 4,096 padded
    //    rows: 53.0 -> 41.8 us dense, 31.2 -> 28.7 us for c2's 2,424 rows);
    //  * otherwise 128 x 128 tiles, 64-deep k-tiles, 8 waves (two per SIMD).
    //  * split-K (a.splits > 1, bias-free products only): each split is a work
    //    item of its own, written to its own partial output; mid-size split
    //    products run 128 x 96 x 32 tiles where N is whole 96-column panels
    //    and there are fewer 128 x 128 tiles than CUs, else 128 x 128 x 32,
    //    two workgroups per CU (mid_splits picks the split count to match).
    const int S = a.splits > 1 ? a.splits : 1;
    //  * at most 64 rows: the few-token kernel (gemm_skinny_kernel); bias-free
    //    products split over K as below.
    if (ok && gemm_f32_skinny_fits(a.M_max, a.N, a.K) && a.K % (64 * S) == 0 && (S == 1 || epi == EPI_NONE))
        return launch_skinny(a, epi, s);
    if (S > 1 && (epi != EPI_NONE || !ok || a.K % (32 * S))) return hipErrorInvalidValue;
    const int64_t tiles128 = (int64_t)((a.M_max + 127) / 128) * ((a.N + 127) / 128);
    if (ok && a.K % (64 * S) == 0 && 2 * tiles128 < (int64_t)cu_count())
        return launch_persistent<64, 64, 64, 2, 2, 2>(a, epi, s, 2);
    if (ok && S > 1 && a.K % (32 * S) == 0 && a.N % 96 == 0 && tiles128 < (int64_t)cu_count())
        return launch_persistent<128, 96, 32, 4, 1, 2>(a, epi, s, 2);   // mid-size split products (mid_splits)
    if (ok && S > 1 && a.K % (32 * S) == 0)
        return launch_persistent<128, 128, 32, 2, 2, 2>(a, epi, s, 2);
    const int64_t rows256 = (a.M_max + 255) / 256, cus = cu_count();
    const bool wide256 = ok && S == 1 && a.N % 256 == 0 && a.K % 32 == 0 && rows256 * (a.N / 256) >= cus;
    const bool wide192 = ok && S == 1 && a.N % 192 == 0 && a.K % 32 == 0 && rows256 * (a.N / 192) >= cus;
    if (ok && S == 1 && a.N % 96 == 0 && a.K % 32 == 0 &&
        ((wide256 && rows256 * (a.N / 256) < 2 * cus) || (!wide256 && wide192 && rows256 * (a.N / 192) < 2 * cus)))
        return launch_persistent<128, 96, 32, 4, 1, 2>(a, epi, s, 2);
    if (wide256) return launch_persistent<256, 256, 32, 2, 4, 2>(a, epi, s, 1);
    if (wide192) return launch_persistent<256, 192, 32, 4, 2, 2>(a, epi, s, 1);
    if (ok && a.K % 32 == 0 && a.N >= 1536 && a.K < 1024 && tiles128 >= 8 * (int64_t)cu_count() && S == 1)
        return launch_persistent<128, 128, 32, 2, 2, 2>(a, epi, s, 2);
    if (ok && S == 1 && a.N % 96 == 0 && a.K % 32 == 0 && tiles128 > (int64_t)cu_count() &&
        2 * (int64_t)((a.M_max + 127) / 128) * (a.N / 96) <= 3 * (int64_t)cu_count())
        return launch_persistent<128, 96, 32, 4, 1, 2>(a, epi, s, 2);
    if (ok && a.K % (64 * S) == 0)
        return launch_persistent<128, 128, 64, 2, 4, 2>(a, epi, s, 1);
    if (ok && a.K % (32 * S) == 0)
        return launch_persistent<128, 128, 32, 2, 2, 2>(a, epi, s, 2);
    return launch_tile<128, 128, 32, 2, 2, false>(a, epi, s);
}

static int mid_splits(int M_max, int N, int K);

int gemm_f32_splits(int M_max, int N, int K) {
    const int64_t tiles128 = (int64_t)((M_max + 127) / 128) * ((N + 127) / 128);
    if (2 * tiles128 >= (int64_t)cu_count()) return mid_splits(M_max, N, K);
    // The few-token path runs 64 x 64 tiles two workgroups per CU: the most
    // splits (of at least two 64-deep k-tiles each) whose work items fit two
    // rounds of workgroups (M_max counts padding the packed forward does not
    // compute, so one round by M_max is often half a round in fact).
    // Measured at 16 tokens, FFN down: 37.8 us unsplit, 11.7 at 4 splits, 7.3
    // at 8; at 2.4k tokens (4k padded), 2 splits are best.
    const int64_t tiles64 = (int64_t)((M_max + 63) / 64) * ((N + 63) / 64);
    for (int S : {8, 6, 4, 3, 2})
        if (K % (64 * S) == 0 && K / S >= 128 && tiles64 * S <= 4 * (int64_t)cu_count()) return S;
    return 1;
}

// Mid-size products (half to two 128 x 128 tiles per CU, e.g. 16 long
// sentences): two workgroups per CU, split over K.
//  * N whole 96-column panels (MiniLM's 384) and fewer 128 x 128 tiles than
//    CUs: 128 x 96 tiles, as many splits (4, 3 or 2) as keep at least six
//    32-deep k-tiles per work item and at most two rounds of workgroups by
//    M_max.  Measured at 6,124 of 8,192 tokens: FFN down 69.2 us (128 x 128,
//    3 splits) -> 62.0 us (4 splits); the attention-output projection takes 2
//    splits, 27.0 us, and its LayerNorm then sums two partials instead of
//    three (c4 9.3k -> 9.6k sentences/s).  With 4 splits it took 24.8 us, but
//    the LayerNorm's two extra partial reads cost as much.  At 8,192 dense
//    tokens: out 42.1 -> 27.9 us, FFN down 127.6 -> 79.8 us.  With more
//    128 x 128 tiles (16,384 padded positions) a ragged batch's items came to
//    just over one round (8,585 tokens: 544 items for 512 workgroups), slower
//    than the unsplit product (FFN down 99.8 -> 112.1 us), so those keep the
//    rule below;
//  * otherwise 128 x 128 tiles, split so that the work items come to about
//    one round of workgroups (counted by M_max, which includes padding).
//    Measured at 6.1k of 8k tokens, FFN down: 103.6 us unsplit, 72.0 us in
//    3 splits; the attention-output projection 30.5 -> 24.4.
static int mid_splits(int M_max, int N, int K) {
    const int64_t tiles128 = (int64_t)((M_max + 127) / 128) * ((N + 127) / 128);
    const int64_t slots = 2 * (int64_t)cu_count();
    if (2 * tiles128 < (int64_t)cu_count() || tiles128 >= slots) return 1;
    if (N % 96 == 0 && tiles128 < (int64_t)cu_count()) {
        const int64_t tiles96 = (int64_t)((M_max + 127) / 128) * (N / 96);
        for (int S : {4, 3, 2})
            if (K % (32 * S) == 0 && K / S >= 192 && tiles96 * S <= 2 * slots) return S;
        return 1;
    }
    for (int S : {4, 3, 2})
        if (K % (32 * S) == 0 && K / S >= 128 && 5 * tiles128 * S <= 6 * slots) return S;
    return 1;
}

// Fused projection + bias + residual + LayerNorm: 128 x 384 tiles (whole rows
// of a 384-wide output), 32-deep k-tiles, 8 waves of 64 x 96, two LDS stages
// (2 x 64 KB) plus the bias slots, one workgroup per CU.  Measured on MI355X
// at 32k tokens of MiniLM width, this tile's main loop runs the attention-output
// and FFN-down products faster than 128 x 128 tiles do, and the LayerNorm pass
// that would follow (a read of the product and the residual, a write of x) is
// gone; with fewer row blocks than CUs part of the chip would idle, so the
// split 128 x 128 path and its separate LayerNorm stay the choice there.
constexpr int ADD_LN_BM = 128, ADD_LN_BN = 384, ADD_LN_BK = 32;

bool gemm_f32_add_ln_fits(int M_max, int N, int K) {
    return N == ADD_LN_BN && K % ADD_LN_BK == 0 && K >= ADD_LN_BK &&
           (M_max + ADD_LN_BM - 1) / ADD_LN_BM >= cu_count();
}

hipError_t launch_gemm_f32_add_ln(const GemmArgs& a, hipStream_t s) {
    const bool ok = a.N == ADD_LN_BN && a.K % ADD_LN_BK == 0 && a.K >= ADD_LN_BK && a.splits <= 1 &&
                    aligned16(a.A) && aligned16(a.W) && aligned16(a.bias) && a.R && a.C && a.ln_g &&
                    a.ln_b && a.lda % 4 == 0 && a.ldw % 4 == 0 && a.M_max >= 0 &&
                    gemm_offsets_fit32(a.lda, a.ldw, 4);
    if (!ok) return hipErrorInvalidValue;
    const int tiles = (a.M_max + ADD_LN_BM - 1) / ADD_LN_BM;
    if (tiles == 0) return hipSuccess;
    const int grid = std::min(tiles, cu_count());
    if (a.split6)
        hipLaunchKernelGGL((gemm_persistent_kernel<false, false, ADD_LN_BM, ADD_LN_BN, ADD_LN_BK, 2, 4, 2, EPI_ADD_LN, true>),
                           dim3(grid), dim3(512), 0, s, a);
    else
        hipLaunchKernelGGL((gemm_persistent_kernel<false, false, ADD_LN_BM, ADD_LN_BN, ADD_LN_BK, 2, 4, 2, EPI_ADD_LN>),
                           dim3(grid), dim3(512), 0, s, a);
    return hipGetLastError();
}

// bf16 activations: 256 x 256 tiles, 64-deep k-tiles (8 chunks of 8), 8 waves
// of 128 x 64, two LDS stages (2 x 64 KB), one workgroup per CU.
hipError_t launch_gemm_bf16_act(const GemmArgs& a, int epi, bool c_bf16, hipStream_t s) {
    const bool ok = epi != EPI_BIAS_RESID && a.splits <= 1 && aligned16(a.A) && aligned16(a.W) && aligned16(a.C) &&
                    (epi == EPI_NONE || aligned16(a.bias)) && a.lda % 8 == 0 && a.ldw % 8 == 0 &&
                    a.ldc % 4 == 0 && a.N % 4 == 0 && a.K % 64 == 0 && a.K > 0 &&
                    gemm_offsets_fit32(a.lda, a.ldw, 2);
    if (!ok) return hipErrorInvalidValue;
    if (c_bf16 && a.N % 8 == 0 && a.ldc % 8 == 0 && (epi == EPI_NONE || aligned16(a.bias))) {
        const int64_t tiles = (int64_t)((a.M_max + 255) / 256) * ((a.N + 255) / 256);
        if (tiles == 0) return hipSuccess;
        const dim3 grid((unsigned)std::min<int64_t>(tiles, cu_count())), block(512);
        switch (epi) {
            case EPI_BIAS: hipLaunchKernelGGL(gemm_bf16_ring_kernel<EPI_BIAS>, grid, block, 0, s, a); break;
            case EPI_BIAS_GELU: hipLaunchKernelGGL(gemm_bf16_ring_kernel<EPI_BIAS_GELU>, grid, block, 0, s, a); break;
            case EPI_NONE: hipLaunchKernelGGL(gemm_bf16_ring_kernel<EPI_NONE>, grid, block, 0, s, a); break;
            default: return hipErrorInvalidValue;
        }
        return hipGetLastError();
    }
    if (c_bf16) return launch_persistent<256, 256, 64, 2, 4, 2, true, true>(a, epi, s, 1);
    return launch_persistent<256, 256, 64, 2, 4, 2, true, false>(a, epi, s, 1);
}

hipError_t launch_gemm_bf16(const GemmArgs& a, int epi, hipStream_t s) {
    return launch_tile<128, 128, 32, 2, 2, true>(a, epi, s);
}

}  // namespace ebh
