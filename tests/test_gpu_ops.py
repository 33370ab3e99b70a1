"""Each HIP kernel alone, through the op-level C ABI (include/edgebert_hip_ops.h),
against a float64 reference of the reference op it replaces; then the
model-level edge cases of the forward (empty batch, S = 0, all-masked row,
masks with holes, ids out of range, concurrent callers, workspace growth,
safetensors loading).  Device memory comes from torch; every call is
enqueued on torch's current stream."""
import ctypes
import json
import os
import threading

import numpy as np
import pytest

from conftest import cosine_rows

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "encoder_golden.npz")


@pytest.fixture(scope="module")
def env():
    import torch
    import edgebert_amd as eb
    from edgebert_amd import _native as N
    assert torch.cuda.is_available(), "gpu tests need a GPU"
    return torch, eb, N, eb.lib()


def vp(t):
    """Device address of a tensor the caller keeps alive until the work is done
    (a temporary would return its block to torch's allocator at once, and the
    next allocation could take it over before the kernel reads it)."""
    return ctypes.c_void_p(t.data_ptr())


def stream(torch):
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


# ---------------------------------------------------------------------------
# GEMM family (matmul_3d_2d + bias / GELU / residual)
# ---------------------------------------------------------------------------
def gelu64(x):
    return 0.5 * x * (1 + np.tanh(0.7978845608 * (x + 0.044715 * x ** 3)))


GEMM_SHAPES = [(1, 8, 4), (7, 40, 12), (130, 1152, 384), (257, 384, 1536), (64, 96, 64),
               (300, 1536, 384), (33, 768, 3072)]


@pytest.mark.parametrize("M,N,K", GEMM_SHAPES)
@pytest.mark.parametrize("epi", [0, 1, 2, 3])
def test_gemm_f32(env, M, N, K, epi):
    torch, eb, Nn, L = env
    rng = np.random.default_rng(M * 7 + N + K + epi)
    lda = K + 4                                   # a row stride above K
    A = rng.standard_normal((M, lda)).astype(np.float32)
    W = (0.05 * rng.standard_normal((N, K))).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    R = rng.standard_normal((M, N)).astype(np.float32)
    dA, dW, db, dR = dev(torch, A), dev(torch, W), dev(torch, bias), dev(torch, R)
    dC = torch.full((M, N), float("nan"), device="cuda")
    Nn.check(L.ebh_op_gemm(vp(dA), lda, vp(dW), K, Nn.EBH_DTYPE_F32, vp(db) if epi != 3 else None,
                           vp(dR) if epi == 2 else None, N, vp(dC), N, M, N, K, epi, stream(torch)))
    torch.cuda.synchronize()
    want = A[:, :K].astype(np.float64) @ W.T.astype(np.float64) + (bias if epi != 3 else 0.0)
    if epi == 1:
        want = gelu64(want)
    if epi == 2:
        want = want + R
    got = dC.cpu().numpy()
    tol = 2e-6 * np.sqrt(K) * (np.abs(A[:, :K]).max() * np.abs(W).max() * np.sqrt(K)) + 1e-5
    np.testing.assert_allclose(got, want, rtol=0, atol=tol)


def test_gemm_f32_row_stride_past_32bit_offsets(env):
    """A rows 17.1M floats apart (a 4.4 GB operand): 63 rows of that stride lie
    past 2^32 bytes, beyond the 32-bit lane offsets of the persistent kernels'
    64-row tiles that this shape would otherwise take, so the op runs the
    guarded kernel (64-bit addresses).  Against the float64 product of the rows
    used."""
    torch, eb, Nn, L = env
    M, N, K, lda = 65, 128, 64, 17_100_000
    assert 63 * lda * 4 >= 2 ** 32
    rng = np.random.default_rng(17)
    A = rng.standard_normal((M, K)).astype(np.float32)
    W = (0.05 * rng.standard_normal((N, K))).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    big = torch.zeros(M * lda, device="cuda")
    big.view(M, lda)[:, :K] = torch.from_numpy(A).cuda()
    dW, db = dev(torch, W), dev(torch, bias)
    dC = torch.full((M, N), float("nan"), device="cuda")
    Nn.check(L.ebh_op_gemm(vp(big), lda, vp(dW), K, Nn.EBH_DTYPE_F32, vp(db), None, N, vp(dC), N,
                           M, N, K, 0, stream(torch)))
    torch.cuda.synchronize()
    want = A.astype(np.float64) @ W.T.astype(np.float64) + bias
    np.testing.assert_allclose(dC.cpu().numpy(), want, rtol=0, atol=1e-4)
    del big
    torch.cuda.empty_cache()


@pytest.mark.parametrize("M,N,K,epi", [
    (4100, 1152, 384, 0),      # 128 x 128 tiles, 8 waves (row tail of 4)
    (8192, 384, 1536, 3),      # 8 waves, long K, no bias
    (33000, 1536, 384, 1),     # 256 x 256 tiles (GELU), ragged last row block: FFN up
    (32768, 1152, 384, 0),     # 256 x 192 tiles (bias): QKV at 256 x 128 tokens
    (33000, 1152, 384, 1),     # 256 x 192 tiles (GELU), ragged last row block
    (90000, 576, 256, 3),      # 256 x 192 tiles, no bias, 8 k-tiles
    (8100, 1536, 384, 1),      # 128 x 96 tiles in place of one round of 256 x 192 (GELU), ragged rows
    (12000, 1152, 384, 0),     # 128 x 96 tiles in place of 1.1 rounds of 256 x 192 (bias)
    (20000, 1536, 384, 3),     # 128 x 96 tiles in place of 1.8 rounds of 256 x 256 (no bias)
    (40000, 576, 256, 1),      # 128 x 96 tiles, 8 k-tiles, ragged last row block (GELU)
    (4000, 1152, 384, 0),      # 128 x 96 tiles in place of 1.1 rounds of 128 x 128 (bias), ragged rows
    (3000, 1536, 384, 1),      # the same with GELU
    (40000, 512, 160, 3),      # 256 x 256 tiles, no bias, 5 k-tiles
    (9000, 1024, 384, 1),      # 128 x 128 tiles beside the 128 x 384 case (N not whole panels)
    (500, 256, 96, 0),         # K % 64 != 0: 32-deep k-tiles
    (4100, 1000, 384, 1),      # 128 x 128 tiles, N past the last whole panel, ragged rows (GELU)
    (1000, 200, 256, 3),       # 64 x 64 tiles (few per CU), N past the last whole panel
])
def test_gemm_f32_dispatch_paths(env, M, N, K, epi):
    """The tile configurations chosen for many tokens, each against the float64
    product (the small shapes above all take the few-token or guarded kernels)."""
    torch, eb, Nn, L = env
    rng = np.random.default_rng(M + N + K)
    A = rng.standard_normal((M, K)).astype(np.float32)
    W = (0.05 * rng.standard_normal((N, K))).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    dA, dW, db = dev(torch, A), dev(torch, W), dev(torch, bias)
    dC = torch.full((M, N), float("nan"), device="cuda")
    Nn.check(L.ebh_op_gemm(vp(dA), K, vp(dW), K, Nn.EBH_DTYPE_F32, vp(db) if epi != 3 else None,
                           None, N, vp(dC), N, M, N, K, epi, stream(torch)))
    torch.cuda.synchronize()
    want = A.astype(np.float64) @ W.T.astype(np.float64) + (bias if epi != 3 else 0.0)
    if epi == 1:
        want = gelu64(want)
    tol = 2e-6 * np.sqrt(K) * (np.abs(A).max() * np.abs(W).max() * np.sqrt(K)) + 1e-5
    np.testing.assert_allclose(dC.cpu().numpy(), want, rtol=0, atol=tol)


@pytest.mark.parametrize("M,N,K,epi", [
    (4100, 1152, 384, 0), (8192, 384, 1536, 3), (33000, 1536, 384, 1), (32768, 1152, 384, 0),
    (33000, 1152, 384, 1), (90000, 576, 256, 3), (40000, 512, 160, 3), (9000, 1024, 384, 1),
    (500, 256, 96, 0), (2000, 384, 1536, 3), (8100, 1536, 384, 1), (12000, 1152, 384, 0),
    (4000, 1152, 384, 0)])
def test_gemm_f32_split_products(env, M, N, K, epi):
    """EBH_DTYPE_F32_BF16X6: fp32 products formed from six bf16 MFMA products
    of three-way bf16 splits, on every tile configuration of the fp32
    dispatch.  Against the float64 product it meets the fp32 tolerance, and
    its largest error is at most that of the fp32 MFMA path on the same data
    (times 1.5, for the different summation order)."""
    torch, eb, Nn, L = env
    rng = np.random.default_rng(M + N + K + 7)
    A = rng.standard_normal((M, K)).astype(np.float32)
    W = (0.05 * rng.standard_normal((N, K))).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    dA, dW, db = dev(torch, A), dev(torch, W), dev(torch, bias)
    want = A.astype(np.float64) @ W.T.astype(np.float64) + (bias if epi != 3 else 0.0)
    if epi == 1:
        want = gelu64(want)
    errs = {}
    for wd in (Nn.EBH_DTYPE_F32, Nn.EBH_DTYPE_F32_BF16X6):
        dC = torch.full((M, N), float("nan"), device="cuda")
        Nn.check(L.ebh_op_gemm(vp(dA), K, vp(dW), K, wd, vp(db) if epi != 3 else None,
                               None, N, vp(dC), N, M, N, K, epi, stream(torch)))
        torch.cuda.synchronize()
        errs[wd] = float(np.abs(dC.cpu().numpy() - want).max())
    tol = 2e-6 * np.sqrt(K) * (np.abs(A).max() * np.abs(W).max() * np.sqrt(K)) + 1e-5
    print(f"max |err| fp32 MFMA {errs[Nn.EBH_DTYPE_F32]:.3e}, bf16x6 {errs[Nn.EBH_DTYPE_F32_BF16X6]:.3e}", flush=True)
    assert errs[Nn.EBH_DTYPE_F32_BF16X6] <= tol
    assert errs[Nn.EBH_DTYPE_F32_BF16X6] <= 1.5 * errs[Nn.EBH_DTYPE_F32] + 1e-7


@pytest.mark.parametrize("M,N,K", [(1, 32, 64), (16, 1152, 384), (33, 384, 1536), (64, 3072, 768),
                                   (50, 96, 192), (7, 64, 320)])
@pytest.mark.parametrize("epi", [0, 1, 3])
def test_gemm_f32_few_tokens(env, M, N, K, epi):
    """At most 64 rows: the few-token kernel (4 or 8 waves, 1 to 4 16-deep
    steps per load batch, 1 to 4 row blocks with a ragged last one, a row
    stride above K) against the float64 product."""
    torch, eb, Nn, L = env
    rng = np.random.default_rng(3 * M + N + K + epi)
    lda = K + 4
    A = rng.standard_normal((M, lda)).astype(np.float32)
    W = (0.05 * rng.standard_normal((N, K))).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    dA, dW, db = dev(torch, A), dev(torch, W), dev(torch, bias)
    dC = torch.full((M + 3, N), float("nan"), device="cuda")
    Nn.check(L.ebh_op_gemm(vp(dA), lda, vp(dW), K, Nn.EBH_DTYPE_F32, vp(db) if epi != 3 else None,
                           None, N, vp(dC), N, M, N, K, epi, stream(torch)))
    torch.cuda.synchronize()
    want = A[:, :K].astype(np.float64) @ W.T.astype(np.float64) + (bias if epi != 3 else 0.0)
    if epi == 1:
        want = gelu64(want)
    got = dC.cpu().numpy()
    assert np.isnan(got[M:]).all(), "rows past M were written"
    tol = 2e-6 * np.sqrt(K) * (np.abs(A[:, :K]).max() * np.abs(W).max() * np.sqrt(K)) + 1e-5
    np.testing.assert_allclose(got[:M], want, rtol=0, atol=tol)


def _bf16_round(x):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.bfloat16).float().numpy()


@pytest.mark.parametrize("M,N,K", [(5, 16, 8), (130, 2304, 768), (257, 768, 3072), (64, 1536, 384)])
@pytest.mark.parametrize("epi", [0, 1, 2])
def test_gemm_bf16(env, M, N, K, epi):
    """bf16 inputs (A rounded on load, W pre-converted), fp32 accumulate: equal to
    the float64 product of the bf16-rounded operands up to fp32 summation."""
    torch, eb, Nn, L = env
    rng = np.random.default_rng(M + N + K + epi)
    A = rng.standard_normal((M, K)).astype(np.float32)
    W = (0.05 * rng.standard_normal((N, K))).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    R = rng.standard_normal((M, N)).astype(np.float32)
    dA, dW32, db, dR = dev(torch, A), dev(torch, W), dev(torch, bias), dev(torch, R)
    dW16 = torch.empty((N, K), dtype=torch.int16, device="cuda")
    Nn.check(L.ebh_op_f32_to_bf16(vp(dW32), vp(dW16), N * K, stream(torch)))
    dC = torch.empty((M, N), device="cuda")
    Nn.check(L.ebh_op_gemm(vp(dA), K, vp(dW16), K, Nn.EBH_DTYPE_BF16, vp(db),
                           vp(dR) if epi == 2 else None, N, vp(dC), N, M, N, K, epi, stream(torch)))
    torch.cuda.synchronize()
    want = _bf16_round(A).astype(np.float64) @ _bf16_round(W).T.astype(np.float64) + bias
    if epi == 1:
        want = gelu64(want)
    if epi == 2:
        want = want + R
    np.testing.assert_allclose(dC.cpu().numpy(), want, rtol=0, atol=2e-5 * np.sqrt(K))


@pytest.mark.parametrize("M,N,K", [(5, 16, 64), (300, 2304, 768), (257, 768, 3072), (1000, 3072, 768),
                                   (130, 100, 128)])
@pytest.mark.parametrize("epi", [0, 1, 3])
@pytest.mark.parametrize("c16", [False, True])
def test_gemm_bf16_activations(env, M, N, K, epi, c16):
    """bf16 A and W (the forward of bf16 models): equal to the float64 product of
    the same bf16 values up to fp32 summation; a bf16 C is that, rounded."""
    torch, eb, Nn, L = env
    rng = np.random.default_rng(M + N + K + epi + int(c16))
    A = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).to(torch.bfloat16)
    W = torch.from_numpy((0.05 * rng.standard_normal((N, K))).astype(np.float32)).to(torch.bfloat16)
    bias = rng.standard_normal(N).astype(np.float32)
    dA, dW, db = A.cuda(), W.cuda(), dev(torch, bias)
    dC = torch.full((M, N), float("nan"), device="cuda", dtype=torch.bfloat16 if c16 else torch.float32)
    Nn.check(L.ebh_op_gemm_bf16(vp(dA), K, vp(dW), K, vp(db) if epi != 3 else None, vp(dC), N,
                                Nn.EBH_DTYPE_BF16 if c16 else Nn.EBH_DTYPE_F32, M, N, K, epi, stream(torch)))
    torch.cuda.synchronize()
    want = A.double().numpy() @ W.double().numpy().T + (bias if epi != 3 else 0.0)
    if epi == 1:
        want = gelu64(want)
    got = dC.float().cpu().numpy()
    if c16:   # one bf16 rounding of the fp32 result (relative 2^-8)
        np.testing.assert_allclose(got, want, rtol=2 ** -8, atol=1e-4 * np.sqrt(K))
    else:
        np.testing.assert_allclose(got, want, rtol=0, atol=2e-5 * np.sqrt(K))


@pytest.mark.parametrize("M,N,K,epi,pad", [
    (20000, 3072, 768, 1, 0),    # 79 x 12 tiles: several per workgroup, ragged last row block, GELU
    (70001, 256, 64, 0, 8),      # one k-tile per tile, 274 tiles, odd M, C rows 8 elements apart beyond N
    (9000, 2304, 768, 3, 0),     # no bias
    (33000, 768, 3072, 0, 0),    # long K: 48 k-tiles per tile
])
def test_gemm_bf16_ring_many_tiles(env, M, N, K, epi, pad):
    """bf16 products with bf16 outputs over more tiles than workgroups: each
    workgroup walks several tiles, so every tile boundary (the previous
    tile's epilogue and buffer stores, the next tile's bias in its
    accumulators, the three-stage A ring) is exercised.  Against torch's fp32
    product of the same bf16 values (TF32 off), within one bf16 rounding;
    the row padding past N must stay untouched."""
    torch, eb, Nn, L = env
    g = torch.Generator(device="cuda").manual_seed(M + N + K)
    A = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
    W = (0.05 * torch.randn(N, K, device="cuda", generator=g)).to(torch.bfloat16)
    bias = torch.randn(N, device="cuda", generator=g)
    ldc = N + pad
    C = torch.full((M, ldc), float("nan"), device="cuda", dtype=torch.bfloat16)
    Nn.check(L.ebh_op_gemm_bf16(vp(A), K, vp(W), K, vp(bias) if epi != 3 else None, vp(C), ldc,
                                Nn.EBH_DTYPE_BF16, M, N, K, epi, stream(torch)))
    torch.cuda.synchronize()
    prev = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    try:
        want = A.float() @ W.float().t()
    finally:
        torch.backends.cuda.matmul.allow_tf32 = prev
    if epi != 3:
        want = want + bias
    if epi == 1:
        want = torch.nn.functional.gelu(want, approximate="tanh")
    got = C[:, :N].float()
    err = (got - want).abs()
    tol = 2 ** -8 * want.abs() + 1e-4 * K ** 0.5
    assert bool((err <= tol).all()), f"max err {float(err.max()):.3e}"
    if pad:
        assert bool(torch.isnan(C[:, N:].float()).all())


def test_f32_to_bf16_round_to_nearest_even(env):
    torch, eb, Nn, L = env
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.standard_normal(10000).astype(np.float32) * 100,
                        np.array([0.0, -0.0, np.inf, -np.inf, 1e-40, -1e-39, 3.4e38, 1.0 + 2 ** -8,
                                  1.0 + 3 * 2 ** -8, np.nan], np.float32)])
    dx = dev(torch, x)
    dy = torch.empty(x.size, dtype=torch.int16, device="cuda")
    Nn.check(L.ebh_op_f32_to_bf16(vp(dx), vp(dy), x.size, stream(torch)))
    torch.cuda.synchronize()
    got = dy.cpu().numpy().view(np.uint16)
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    fin = ~np.isnan(x)
    np.testing.assert_array_equal(got[fin], want[fin])
    assert np.isnan(np.frombuffer((got[~fin].astype(np.uint32) << 16).tobytes(), np.float32)).all()


def _all_16bit_patterns():
    return np.arange(65536, dtype=np.uint32).astype(np.uint16)


@pytest.mark.parametrize("mode", [0, 1, 2])
def test_widen16_every_bit_pattern(env, mode):
    """The device conversion of F16 / BF16 checkpoint tensors, on all 65536
    bit patterns (zeros of both signs, every subnormal, +-inf, NaNs):
    F16 -> f32 equals numpy's float16 widening, BF16 -> f32 the 16-bit shift,
    F16 -> bf16 torch's round-to-nearest-even of that f32 value; a NaN stays a
    NaN of the same sign."""
    torch, eb, Nn, L = env
    x = _all_16bit_patterns()
    dx = dev(torch, x.view(np.int16))
    if mode == 2:
        dy = torch.empty(x.size, dtype=torch.int16, device="cuda")
    else:
        dy = torch.empty(x.size, dtype=torch.float32, device="cuda")
    Nn.check(L.ebh_op_widen16(vp(dx), vp(dy), x.size, mode, stream(torch)))
    torch.cuda.synchronize()
    f16 = x.view(np.float16).astype(np.float32)
    if mode == 0:
        got, want = dy.cpu().numpy(), f16
    elif mode == 1:
        got, want = dy.cpu().numpy(), (x.astype(np.uint32) << 16).view(np.float32)
    else:
        got_b = dy.cpu().numpy().view(np.uint16)
        want_b = torch.from_numpy(f16).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
        got = (got_b.astype(np.uint32) << 16).view(np.float32)
        want = (want_b.astype(np.uint32) << 16).view(np.float32)
    nan = np.isnan(want)
    assert nan.sum() == (2046 if mode != 1 else 254)
    np.testing.assert_array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    assert np.isnan(got[nan]).all()
    assert (np.signbit(got[nan]) == (x[nan] >= 0x8000)).all()   # torch's own bf16 NaN is unsigned


def test_gelu_error_bound(env):
    """The fused GELU (exp2 + reciprocal form) against the float64 tanh form of
    the reference (src/lib.rs:958-978) over [-12, 12] in steps of 2^-12 and
    2^20 random values, within its stated bound
    |err| <= (8 ln2 |t| + 8) 2^-24 |gelu(x)|, t = x (K1 + K2 x^2) (plus 2e-37
    absolute where the result leaves the normal fp32 range)."""
    torch, eb, Nn, L = env
    rng = np.random.default_rng(17)
    x = np.concatenate([np.arange(-12 * 4096, 12 * 4096 + 1) / 4096.0,
                        rng.standard_normal(1 << 20) * 3.0, [0.0, -0.0]]).astype(np.float32)
    dx = dev(torch, x)
    dy = torch.empty_like(dx)
    Nn.check(L.ebh_op_gelu(vp(dx), vp(dy), x.size, stream(torch)))
    torch.cuda.synchronize()
    got = dy.cpu().numpy().astype(np.float64)
    x64 = x.astype(np.float64)
    # 0.5 (1 + tanh u) = 1 / (1 + e^(-2u)): the second form has no cancellation
    # in float64 where tanh u -> -1 (x < -5); the two agree elsewhere.
    u = 0.7978845608 * (x64 + 0.044715 * x64 ** 3)
    with np.errstate(over="ignore"):
        want = x64 / (1.0 + np.exp(-2.0 * u))
    well = x64 > -3
    np.testing.assert_allclose(want[well], gelu64(x64[well]), rtol=1e-13, atol=1e-300)
    k1 = -2.0 * np.log2(np.e) * 0.7978845608
    t = x64 * (k1 + k1 * 0.044715 * x64 * x64)
    bound = (8 * np.log(2) * np.abs(t) + 8) * 2.0 ** -24 * np.abs(want) + 2e-37
    err = np.abs(got - want)
    worst = float((err / bound).max())
    print(f"gelu: max abs err {err.max():.3e}, max err / bound {worst:.3f}, "
          f"max rel err (x >= -5) {float((err / np.maximum(np.abs(want), 1e-30))[x64 >= -5].max()):.3e}")
    assert worst <= 1.0
    assert np.isfinite(got).all()


# ---------------------------------------------------------------------------
# attention (QK^T, scale, key-padding mask, softmax, PV) over packed sequences
# ---------------------------------------------------------------------------
def attention64(qkv, cu, H, nh):
    hd = H // nh
    out = np.zeros((qkv.shape[0], H))
    for b in range(len(cu) - 1):
        s, e = cu[b], cu[b + 1]
        if e == s:
            continue
        for h in range(nh):
            q = qkv[s:e, h * hd:(h + 1) * hd].astype(np.float64)
            k = qkv[s:e, H + h * hd:H + (h + 1) * hd].astype(np.float64)
            v = qkv[s:e, 2 * H + h * hd:2 * H + (h + 1) * hd].astype(np.float64)
            sc = (q @ k.T) * (1.0 / np.sqrt(hd))
            p = np.exp(sc - sc.max(1, keepdims=True))
            out[s:e, h * hd:(h + 1) * hd] = (p / p.sum(1, keepdims=True)) @ v
    return out


@pytest.mark.parametrize("H,nh,lengths", [
    (384, 12, [1, 2, 31, 32, 33, 127, 128, 129]),
    (384, 12, [256, 300, 511, 512]),
    (768, 12, [1, 64, 128, 130, 257]),
    (64, 2, [5, 17]),
    # at most 128 tokens: 64-key chunks, the second one prefetched
    (384, 12, [1, 63, 64, 65, 100, 127, 128]),
    (768, 12, [1, 65, 128]),
    # BERT-base heads (head_dim 64) up to max_position_embeddings = 512
    # (src/lib.rs:100, 655): four 128-key chunks, the last one partial
    (768, 12, [384, 511, 512]),
    (768, 12, [512, 0, 300, 1, 449]),
])
def test_attention(env, H, nh, lengths):
    torch, eb, Nn, L = env
    rng = np.random.default_rng(sum(lengths) + H)
    T = sum(lengths)
    qkv = rng.standard_normal((T, 3 * H)).astype(np.float32)
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    dq, dcu = dev(torch, qkv), dev(torch, cu)
    dctx = torch.full((T, H), float("nan"), device="cuda")
    Nn.check(L.ebh_op_attention(vp(dq), vp(dcu), len(lengths), max(lengths), H, nh, vp(dctx),
                                stream(torch)))
    torch.cuda.synchronize()
    np.testing.assert_allclose(dctx.cpu().numpy(), attention64(qkv, cu, H, nh), rtol=0, atol=2e-5)


_SHORT_RAGGED = [int(x) for x in np.random.default_rng(7).integers(1, 129, 120)]


@pytest.mark.parametrize("H,nh,lengths", [
    (384, 12, [1, 2, 31, 32, 33, 127, 128, 129]),
    (384, 12, [256, 300, 511, 512]),
    (768, 12, [1, 64, 128, 130, 257]),
    (64, 2, [5, 17]),
    (768, 12, [128, 1, 64, 100, 0, 77, 128, 33]),
    (384, 12, [1, 2, 31, 32, 33, 127, 128, 0]),
    (384, 12, _SHORT_RAGGED),
    (768, 12, _SHORT_RAGGED[:60]),
    # BERT-base heads (head_dim 64) up to max_position_embeddings = 512
    # (src/lib.rs:100, 655)
    (768, 12, [384, 511, 512]),
    (768, 12, [512, 0, 300, 1, 449]),
])
def test_attention_bf16(env, H, nh, lengths):
    """bf16 q / k / v and context: the float64 attention of the same bf16 values,
    within the bf16 rounding of the probabilities and of the result.  Batches
    whose sequences all have at most 128 tokens take the short-sequence kernel:
    one workgroup per (head, sequence), Q, K and V loaded straight into LDS,
    the scores waiting for Q and K only; the ragged cases (120 and 60
    sequences of 1-128 tokens) and the ones with an empty sequence run that
    path, the others the chunked kernel for longer sequences (128-key chunks
    through registers, online softmax)."""
    torch, eb, Nn, L = env
    rng = np.random.default_rng(sum(lengths) + H + 1)
    T = sum(lengths)
    qkv = torch.from_numpy(rng.standard_normal((T, 3 * H)).astype(np.float32)).to(torch.bfloat16)
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    dq, dcu = qkv.cuda(), dev(torch, cu)
    dctx = torch.full((T, H), float("nan"), device="cuda", dtype=torch.bfloat16)
    Nn.check(L.ebh_op_attention_bf16(vp(dq), vp(dcu), len(lengths), max(lengths), H, nh, vp(dctx),
                                     stream(torch)))
    torch.cuda.synchronize()
    want = attention64(qkv.float().numpy(), cu, H, nh)
    # |ctx| <= max|v| ~ 4; probabilities carry 2^-9 relative error, the output one
    # more bf16 rounding.
    np.testing.assert_allclose(dctx.float().cpu().numpy(), want, rtol=2 ** -8, atol=1e-2)


def test_attention_empty_sequence_writes_nothing(env):
    torch, eb, Nn, L = env
    H, nh = 384, 12
    cu = np.array([0, 3, 3, 5], np.int32)            # middle sequence empty
    qkv = np.random.default_rng(0).standard_normal((5, 3 * H)).astype(np.float32)
    dctx = torch.zeros((5, H), device="cuda")
    dq, dcu = dev(torch, qkv), dev(torch, cu)
    Nn.check(L.ebh_op_attention(vp(dq), vp(dcu), 3, 3, H, nh, vp(dctx),
                                stream(torch)))
    torch.cuda.synchronize()
    np.testing.assert_allclose(dctx.cpu().numpy(), attention64(qkv, cu, H, nh), rtol=0, atol=2e-5)


# ---------------------------------------------------------------------------
# row kernels
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("H", [64, 384, 768, 1000])
def test_layer_norm(env, H):
    torch, eb, Nn, L = env
    import oracle
    rng = np.random.default_rng(H)
    x = (3 * rng.standard_normal((333, H)) + 1).astype(np.float32)
    g = rng.standard_normal(H).astype(np.float32)
    b = rng.standard_normal(H).astype(np.float32)
    dx, dg, db = dev(torch, x), dev(torch, g), dev(torch, b)
    dy = torch.empty_like(dx)
    Nn.check(L.ebh_op_layer_norm(vp(dx), vp(dg), vp(db), 333, H,
                                 ctypes.c_float(1e-12), vp(dy), stream(torch)))
    Nn.check(L.ebh_op_layer_norm(vp(dx), vp(dg), vp(db), 333, H,
                                 ctypes.c_float(1e-12), vp(dx), stream(torch)))    # in place
    torch.cuda.synchronize()
    want = oracle.layer_norm(x, g, b, 1e-12)
    np.testing.assert_allclose(dy.cpu().numpy(), want, rtol=0, atol=1e-5)
    np.testing.assert_array_equal(dx.cpu().numpy(), dy.cpu().numpy())


@pytest.mark.parametrize("H", [64, 384, 768])
def test_add_layer_norm(env, H):
    """x = LN((y + b) + x), the residual-block end the forward uses."""
    torch, eb, Nn, L = env
    import oracle
    rng = np.random.default_rng(H + 1)
    rows = 517
    y = rng.standard_normal((rows, H)).astype(np.float32)
    x = rng.standard_normal((rows, H)).astype(np.float32)
    b = rng.standard_normal(H).astype(np.float32)
    g = rng.standard_normal(H).astype(np.float32)
    beta = rng.standard_normal(H).astype(np.float32)
    dy, dx, db, dg, dbeta = (dev(torch, a) for a in (y, x, b, g, beta))
    Nn.check(L.ebh_op_add_layer_norm(vp(dy), vp(db), vp(dx), vp(dg), vp(dbeta), rows, H,
                                     ctypes.c_float(1e-12), stream(torch)))
    torch.cuda.synchronize()
    want = oracle.layer_norm(((y + b) + x).astype(np.float32), g, beta, 1e-12)
    np.testing.assert_allclose(dx.cpu().numpy(), want, rtol=0, atol=1e-5)


@pytest.mark.parametrize("M,K", [
    (32768, 384),     # attention-output shape at 256 x 128 tokens: one row block per CU
    (32768, 1536),    # FFN-down shape
    (33000, 384),     # more row blocks than CUs: a second round and a ragged last block
    (1000, 1536),     # few rows (the op takes any M; the forward would not fuse here)
    (5, 64),
])
def test_gemm_add_layer_norm(env, M, K):
    """x = LN((A.W^T + b) + x) in one kernel: against the float64 product and
    LayerNorm, and against the unfused GEMM + add-LayerNorm pair on the GPU."""
    torch, eb, Nn, L = env
    rng = np.random.default_rng(M + K)
    H = 384
    A = rng.standard_normal((M, K)).astype(np.float32)
    W = (rng.standard_normal((H, K)) / np.sqrt(K)).astype(np.float32)
    b = rng.standard_normal(H).astype(np.float32)
    x = rng.standard_normal((M, H)).astype(np.float32)
    g = rng.standard_normal(H).astype(np.float32)
    beta = rng.standard_normal(H).astype(np.float32)
    dA, dW, db, dg, dbeta = (dev(torch, a) for a in (A, W, b, g, beta))
    dx, dx2 = dev(torch, x), dev(torch, x)
    eps = ctypes.c_float(1e-12)
    Nn.check(L.ebh_op_gemm_add_layer_norm(vp(dA), K, vp(dW), K, vp(db), vp(dx), vp(dg), vp(dbeta),
                                          M, H, K, eps, stream(torch)))
    dy = torch.empty((M, H), device="cuda")
    Nn.check(L.ebh_op_gemm(vp(dA), K, vp(dW), K, Nn.EBH_DTYPE_F32, None, None, H, vp(dy), H, M, H, K, 3,
                           stream(torch)))
    Nn.check(L.ebh_op_add_layer_norm(vp(dy), vp(db), vp(dx2), vp(dg), vp(dbeta), M, H, eps, stream(torch)))
    torch.cuda.synchronize()
    v = (A.astype(np.float64) @ W.T.astype(np.float64) + b) + x
    mu = v.mean(1, keepdims=True)
    var = ((v - mu) ** 2).mean(1, keepdims=True)
    want = (v - mu) / np.sqrt(var + 1e-12) * g + beta
    got = dx.cpu().numpy()
    # v has unit-order spread per row; fp32 GEMM and statistics errors reach
    # the output scaled by |gamma| (up to about 4 here).
    np.testing.assert_allclose(got, want, rtol=0, atol=5e-5)
    np.testing.assert_allclose(got, dx2.cpu().numpy(), rtol=0, atol=5e-5)


def test_gemm_add_layer_norm_rejects_other_widths(env):
    torch, eb, Nn, L = env
    t = torch.zeros(1024, device="cuda")
    rc = L.ebh_op_gemm_add_layer_norm(vp(t), 64, vp(t), 64, vp(t), vp(t), vp(t), vp(t), 2, 8, 64,
                                      ctypes.c_float(1e-12), stream(torch))
    assert rc == Nn.EBH_ERR_INVALID_ARG


@pytest.mark.parametrize("H", [384, 768])
def test_add_layer_norm_bf16_projection(env, H):
    """The same block end with y held as bf16 (bf16 models): equal to the fp32
    kernel on the bf16 values of y; the error path rejects an unsupported H."""
    torch, eb, Nn, L = env
    import oracle
    rng = np.random.default_rng(H + 2)
    rows = 517
    y16 = torch.from_numpy(rng.standard_normal((rows, H)).astype(np.float32)).to(torch.bfloat16)
    x = rng.standard_normal((rows, H)).astype(np.float32)
    b = rng.standard_normal(H).astype(np.float32)
    g = rng.standard_normal(H).astype(np.float32)
    beta = rng.standard_normal(H).astype(np.float32)
    dy, dx, db, dg, dbeta = y16.cuda(), dev(torch, x), dev(torch, b), dev(torch, g), dev(torch, beta)
    Nn.check(L.ebh_op_add_layer_norm_y16(vp(dy), vp(db), vp(dx), vp(dg), vp(dbeta), rows, H,
                                         ctypes.c_float(1e-12), stream(torch)))
    torch.cuda.synchronize()
    y = y16.float().numpy()
    want = oracle.layer_norm(((y + b) + x).astype(np.float32), g, beta, 1e-12)
    np.testing.assert_allclose(dx.cpu().numpy(), want, rtol=0, atol=1e-5)
    assert L.ebh_op_add_layer_norm_y16(vp(dy), vp(db), vp(dx), vp(dg), vp(dbeta), rows, 100,
                                       ctypes.c_float(1e-12), stream(torch)) == Nn.EBH_ERR_INVALID_ARG


@pytest.mark.parametrize("H", [384, 768])
def test_add_layer_norm_bf16_residual(env, H):
    """The block end of bf16 models, whose residual stream is bf16: x16 =
    bf16(LayerNorm((y + b) + x16)) in place, the sums and statistics in fp32.
    Against the oracle's LayerNorm of the same bf16 values, to bf16 rounding."""
    torch, eb, Nn, L = env
    import oracle
    rng = np.random.default_rng(H + 7)
    rows = 333
    y16 = torch.from_numpy(rng.standard_normal((rows, H)).astype(np.float32)).to(torch.bfloat16)
    x16 = torch.from_numpy(rng.standard_normal((rows, H)).astype(np.float32)).to(torch.bfloat16)
    b = rng.standard_normal(H).astype(np.float32)
    g = rng.standard_normal(H).astype(np.float32)
    beta = rng.standard_normal(H).astype(np.float32)
    dy, dx16, db, dg, dbeta = y16.cuda(), x16.cuda(), dev(torch, b), dev(torch, g), dev(torch, beta)
    Nn.check(L.ebh_op_add_layer_norm_b16(vp(dy), vp(db), vp(dx16), vp(dg), vp(dbeta), rows, H,
                                         ctypes.c_float(1e-12), stream(torch)))
    torch.cuda.synchronize()
    want = oracle.layer_norm(((y16.float().numpy() + b) + x16.float().numpy()).astype(np.float32), g, beta, 1e-12)
    got = dx16.cpu().float().numpy()
    np.testing.assert_allclose(got, want, rtol=2.0 ** -8, atol=1e-6)   # bf16: 8 significant bits
    assert L.ebh_op_add_layer_norm_b16(vp(dy), vp(db), vp(dx16), vp(dg), vp(dbeta), rows, 100,
                                       ctypes.c_float(1e-12), stream(torch)) == Nn.EBH_ERR_INVALID_ARG


@pytest.mark.parametrize("normalize", [0, 1])
def test_pool_bf16(env, normalize):
    """mean_pool + normalise over a bf16 residual stream: fp32 sums of the bf16
    values, against float64 on the same values."""
    torch, eb, Nn, L = env
    H, S = 768, 64
    lengths = [1, 5, 64, 0, 33]
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    x16 = torch.from_numpy(np.random.default_rng(2).standard_normal((cu[-1], H)).astype(np.float32)).to(torch.bfloat16)
    x = x16.float().numpy()
    dout = torch.empty((len(lengths), H), device="cuda")
    dx16, dcu = x16.cuda(), dev(torch, cu)
    Nn.check(L.ebh_op_pool_b16(vp(dx16), vp(dcu), len(lengths), H, S, normalize, vp(dout), stream(torch)))
    torch.cuda.synchronize()
    got = dout.cpu().numpy()
    for bi, n in enumerate(lengths):
        if n == 0:
            assert np.isnan(got[bi]).all()
            continue
        want = x[cu[bi]:cu[bi + 1]].astype(np.float64).mean(0)
        if normalize:
            want = want / max(np.linalg.norm(want), 1e-12)
        np.testing.assert_allclose(got[bi], want, rtol=0, atol=2e-6)


def run_pool(torch, Nn, L, x, lengths, H, S, normalize):
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    dout = torch.full((len(lengths), H), float("nan"), device="cuda")
    part = torch.full((len(lengths) * max(1, -(-S // 32)) * H,), float("nan"), device="cuda")
    dx, dcu = dev(torch, x), dev(torch, cu)
    Nn.check(L.ebh_op_pool(vp(dx), vp(dcu), len(lengths), H, S, normalize, vp(part),
                           vp(dout), stream(torch)))
    torch.cuda.synchronize()
    return dout.cpu().numpy(), cu


@pytest.mark.parametrize("normalize", [0, 1])
@pytest.mark.parametrize("H,S,lengths", [
    (384, 64, [1, 5, 64, 0, 33]),                       # two 32-row chunks
    (384, 32, [1, 32, 0, 17]),                          # one chunk: one workgroup per sequence
    (384, 512, [512, 1, 33, 0, 300, 32, 64, 65, 511]),  # up to 16 chunks (c4's lengths)
    (768, 512, [512, 100, 31, 0, 257]),                 # BERT-base width: 4 row groups, 8 rows each
    (100, 96, [96, 7, 0, 50]),                          # 25 float4 columns, 30 row groups, idle threads
    (1024, 128, [128, 3, 0, 97]),                       # H > 768: one workgroup per sequence
    (90, 64, [64, 1, 0, 40]),                           # H % 4 != 0: the same
])
def test_pool(env, normalize, H, S, lengths):
    """mean_pool + normalise against float64: a few sequences, so those of
    more than 32 positions, H % 4 == 0 and H <= 768 are summed by a workgroup
    per 32-row chunk."""
    torch, eb, Nn, L = env
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    x = np.random.default_rng(H + S).standard_normal((max(cu[-1], 1), H)).astype(np.float32)
    got, cu = run_pool(torch, Nn, L, x, lengths, H, S, normalize)
    for b, n in enumerate(lengths):
        if n == 0:
            assert np.isnan(got[b]).all()            # all-masked sequence: NaN, as the reference
            continue
        want = x[cu[b]:cu[b + 1]].astype(np.float64).mean(0)
        if normalize:
            want = want / max(np.linalg.norm(want), 1e-12)
        np.testing.assert_allclose(got[b], want, rtol=0, atol=2e-6)


def test_pool_order_depends_on_the_sequence_only(env):
    """A sequence's vector is the same bits wherever it sits in the batch and
    whatever padded length S the batch has (chunks past its end are skipped),
    on the chunked path and on the one-workgroup-per-sequence path (a batch of
    more sequences than CUs)."""
    torch, eb, Nn, L = env
    H = 384
    rng = np.random.default_rng(9)
    seqs = [rng.standard_normal((n, H)).astype(np.float32) for n in (300, 33, 512, 1)]
    a, _ = run_pool(torch, Nn, L, np.concatenate(seqs), [len(q) for q in seqs], H, 512, 1)
    order = [3, 1, 0, 2]
    b, _ = run_pool(torch, Nn, L, np.concatenate([seqs[i] for i in order]), [len(seqs[i]) for i in order],
                    H, 1024, 1)
    np.testing.assert_array_equal(b, a[order])
    many = [seqs[i % 4] for i in range(320)]
    c, _ = run_pool(torch, Nn, L, np.concatenate(many), [len(q) for q in many], H, 512, 1)
    for i in range(4):
        np.testing.assert_array_equal(c[i::4], np.broadcast_to(c[i], c[i::4].shape))
        np.testing.assert_allclose(c[i], a[i], rtol=0, atol=2e-7)


@pytest.mark.parametrize("B,S", [
    (37, 200),     # 7,400 positions: the one-workgroup packing
    (16, 512),     # 8,192 (c4's shape): its largest batch
    (1, 1),
    (1025, 8),     # more sequences than it takes: count, scan and scatter kernels
    (37, 300),     # 11,100 positions: the same
])
def test_pack_with_holes(env, B, S):
    """Masks need not be a prefix: every mask==1 token is kept with its position."""
    torch, eb, Nn, L = env
    rng = np.random.default_rng(5 + B + S)
    ids = rng.integers(0, 30522, (B, S)).astype(np.int32)
    mask = (rng.random((B, S)) < 0.6).astype(np.int32)
    mask[3 % B] = 0
    mask[4 % B] = 1
    d = {k: torch.zeros(n, dtype=torch.int32, device="cuda")
         for k, n in [("counts", B), ("cu", B + 1), ("n", 1), ("tid", B * S), ("tpos", B * S), ("err", 1)]}
    d["err"].fill_(7)
    dids, dmask = dev(torch, ids), dev(torch, mask)
    Nn.check(L.ebh_op_pack(vp(dids), vp(dmask), B, S, vp(d["counts"]),
                           vp(d["cu"]), vp(d["n"]), vp(d["tid"]), vp(d["tpos"]), vp(d["err"]),
                           stream(torch)))
    torch.cuda.synchronize()
    n = int(d["n"].item())
    assert n == mask.sum()
    np.testing.assert_array_equal(d["tid"].cpu().numpy()[:n], ids[mask != 0])
    np.testing.assert_array_equal(d["tpos"].cpu().numpy()[:n], np.nonzero(mask)[1])
    np.testing.assert_array_equal(d["cu"].cpu().numpy(), np.concatenate([[0], np.cumsum(mask.sum(1))]))
    np.testing.assert_array_equal(d["counts"].cpu().numpy(), mask.sum(1))
    assert int(d["err"].item()) == 0


def test_embed_ln_flags_bad_ids(env, weights_for):
    torch, eb, Nn, L = env
    import oracle
    cfg = eb.MINILM_L6
    w = weights_for(cfg)
    H, V = cfg.hidden_size, cfg.vocab_size
    tok = np.array([101, 5, V - 1, 102, V + 3, -2], np.int32)
    pos = np.array([0, 1, 2, 3, 511, 7], np.int32)
    T = len(tok)
    dn = dev(torch, np.array([T], np.int32))
    derr = torch.zeros(1, dtype=torch.int32, device="cuda")
    dx = torch.empty((T, H), device="cuda")
    dw = {k: dev(torch, w[k]) for k in ("embeddings.word_embeddings.weight",
                                        "embeddings.position_embeddings.weight",
                                        "embeddings.token_type_embeddings.weight",
                                        "embeddings.LayerNorm.weight", "embeddings.LayerNorm.bias")}
    dtok, dpos = dev(torch, tok), dev(torch, pos)
    Nn.check(L.ebh_op_embed_ln(vp(dtok), vp(dpos), vp(dn), T,
                               vp(dw["embeddings.word_embeddings.weight"]),
                               vp(dw["embeddings.position_embeddings.weight"]),
                               vp(dw["embeddings.token_type_embeddings.weight"]),
                               vp(dw["embeddings.LayerNorm.weight"]), vp(dw["embeddings.LayerNorm.bias"]),
                               V, H, ctypes.c_float(1e-12), vp(dx), vp(derr), stream(torch)))
    torch.cuda.synchronize()
    assert int(derr.item()) == 1
    safe = np.where((tok >= 0) & (tok < V), tok, 0)
    e = (w["embeddings.word_embeddings.weight"][safe] + w["embeddings.position_embeddings.weight"][pos]
         + w["embeddings.token_type_embeddings.weight"][0])
    want = oracle.layer_norm(e.astype(np.float32), w["embeddings.LayerNorm.weight"],
                             w["embeddings.LayerNorm.bias"], 1e-12)
    np.testing.assert_allclose(dx.cpu().numpy(), want, rtol=0, atol=1e-5)


# ---------------------------------------------------------------------------
# model-level edge cases
# ---------------------------------------------------------------------------
_M = {}


@pytest.fixture(scope="module")
def minilm(env, weights_for):
    torch, eb, Nn, L = env
    if "m" not in _M:
        _M["m"] = eb.Model.from_weights(weights_for(eb.MINILM_L6), eb.MINILM_L6, "fp32")
    return _M["m"]


@pytest.fixture(scope="module")
def orc(weights_for):
    import oracle
    from edgebert_amd import synth
    return oracle.OracleModel(synth.MINILM_L6, weights_for(synth.MINILM_L6))


def test_golden_fixtures(env, minilm):
    with np.load(GOLDEN, allow_pickle=False) as g:
        for case in ("c1", "c2"):
            got = minilm.encode_ids(g[f"{case}_ids"], g[f"{case}_mask"], normalize=True)
            assert np.abs(got - g[f"{case}_out"]).max() <= 1e-4
            assert cosine_rows(got, g[f"{case}_out"]).min() >= 0.99999
        got = minilm.forward(g["c1_ids"].astype(np.float32), g["c1_mask"].astype(np.float32))
        assert np.abs(got - g["c1_pooled"]).max() <= 1e-4


def test_empty_batch_and_empty_sequence(env, minilm):
    torch, eb, Nn, L = env
    assert minilm.encode_ids(np.zeros((0, 5), np.uint32), np.zeros((0, 5), np.uint32)).shape == (0, 384)
    out = minilm.encode_ids(np.zeros((3, 0), np.uint32), np.zeros((3, 0), np.uint32), normalize=False)
    assert out.shape == (3, 384) and (out == 0).all()


def test_all_masked_row_is_nan_others_unchanged(env, minilm, orc):
    ids = np.array([[101, 2000, 3000, 102], [101, 2500, 102, 0], [101, 7, 8, 102]], np.uint32)
    mask = np.array([[1, 1, 1, 1], [0, 0, 0, 0], [1, 1, 1, 1]], np.uint32)
    got = minilm.encode_ids(ids, mask, normalize=True)
    assert np.isnan(got[1]).all()
    want = orc.encode(ids, mask, normalize=True)
    assert np.isnan(want[1]).all()
    assert np.abs(got[[0, 2]] - want[[0, 2]]).max() <= 1e-4


@pytest.mark.parametrize("B,S", [(6, 40), (4, 16), (3, 7)])
def test_mask_with_holes_matches_padded_oracle(env, minilm, orc, B, S):
    """Left padding and holes: positions stay absolute, as in the reference.
    At most 64 positions (4 x 16, 3 x 7) the packing runs in the fused
    packing + embeddings kernel."""
    rng = np.random.default_rng(9 + B * S)
    ids = rng.integers(1000, 30522, (B, S)).astype(np.float32)
    mask = (rng.random((B, S)) < 0.7).astype(np.float32)
    mask[0, :S // 4] = 0      # left padded
    mask[:, S // 2] = 1
    got = minilm.forward(ids, mask)
    want = orc.forward(ids, mask)
    assert np.abs(got - want).max() <= 1e-4
    assert cosine_rows(got, want).min() >= 0.99999


def test_out_of_range_inputs(env, minilm):
    torch, eb, Nn, L = env
    ids = np.full((2, 4), 101, np.uint32)
    mask = np.ones((2, 4), np.uint32)
    ids[1, 2] = 30522
    with pytest.raises(eb.EbhError, match="out of range") as e:
        minilm.encode_ids(ids, mask)
    assert e.value.code == Nn.EBH_ERR_RANGE
    with pytest.raises(eb.EbhError, match="max_position_embeddings"):
        minilm.encode_ids(np.full((1, 513), 101, np.uint32), np.ones((1, 513), np.uint32))
    with pytest.raises(eb.EbhError, match="not 0 or 1"):
        minilm.forward(np.full((1, 3), 101, np.float32), np.array([[1, 0.5, 1]], np.float32))
    # float ids as the reference casts them (`as usize`): 101.7 -> 101, -3 -> 0
    a = minilm.forward(np.array([[101.7, -3.0, 102.2]], np.float32), np.ones((1, 3), np.float32))
    b = minilm.forward(np.array([[101, 0, 102]], np.float32), np.ones((1, 3), np.float32))
    np.testing.assert_array_equal(a, b)


def test_device_path_reports_bad_id_on_synchronize(env, minilm):
    torch, eb, Nn, L = env
    ids = torch.full((2, 8), 101, dtype=torch.int32, device="cuda")
    ids[1, 3] = 40000
    mask = torch.ones_like(ids)
    out = torch.empty((2, 384), device="cuda")
    minilm.encode_device(ids.data_ptr(), mask.data_ptr(), 2, 8, out.data_ptr(), True,
                         torch.cuda.current_stream().cuda_stream)
    with pytest.raises(eb.EbhError, match="out of range") as e:
        minilm.synchronize()
    assert e.value.code == Nn.EBH_ERR_RANGE
    ids[1, 3] = 2000
    minilm.encode_device(ids.data_ptr(), mask.data_ptr(), 2, 8, out.data_ptr(), True,
                         torch.cuda.current_stream().cuda_stream)
    minilm.synchronize()                             # flag cleared, no error
    host = minilm.encode_ids(ids.cpu().numpy().astype(np.uint32), mask.cpu().numpy().astype(np.uint32))
    np.testing.assert_array_equal(out.cpu().numpy(), host)


@pytest.mark.parametrize("B,S", [(2, 8), (4, 40)])
def test_bad_id_flag_is_sticky_across_later_forwards(env, minilm, B, S):
    """A bad id in one queued device forward is still reported after clean
    forwards follow it (pipelined use), after a blocking call, and after the
    workspace grows; ebh_synchronize reports it once and clears it.  (2, 8)
    packs and embeds in one launch, (4, 40) in the separate kernels."""
    torch, eb, Nn, L = env
    s = torch.cuda.current_stream().cuda_stream
    ids = torch.full((B, S), 101, dtype=torch.int32, device="cuda")
    mask = torch.ones_like(ids)
    out = torch.empty((B, 384), device="cuda")
    bad = ids.clone()
    bad[B - 1, 3] = 40000
    good_host = ids.cpu().numpy().astype(np.uint32)
    minilm.synchronize()
    for after in ("device", "blocking", "grow"):
        minilm.encode_device(bad.data_ptr(), mask.data_ptr(), B, S, out.data_ptr(), True, s)
        if after == "device":
            for _ in range(3):
                minilm.encode_device(ids.data_ptr(), mask.data_ptr(), B, S, out.data_ptr(), True, s)
        elif after == "blocking":
            got = minilm.encode_ids(good_host, good_host * 0 + 1)
            assert np.isfinite(got).all()
        else:
            # 160 x 300 tokens: more than any other test of this module runs
            big = torch.full((160, 300), 101, dtype=torch.int32, device="cuda")
            big_mask = torch.ones_like(big)
            big_out = torch.empty((160, 384), device="cuda")
            minilm.encode_device(big.data_ptr(), big_mask.data_ptr(), 160, 300,
                                 big_out.data_ptr(), True, s)
        with pytest.raises(eb.EbhError, match="out of range") as e:
            minilm.synchronize()
        assert e.value.code == Nn.EBH_ERR_RANGE, after
        minilm.synchronize()                         # read once, then clear


def test_empty_sequence_device_call_is_ordered_after_earlier_forwards(env, minilm, weights_for):
    """S == 0 on the device path writes zero rows with a kernel, ordered after
    the model's earlier work on another stream and before later work: a long
    forward into `out` on stream A, then S == 0 into the same `out` on stream
    B, leaves zeros; a forward after it leaves vectors again."""
    torch, eb, Nn, L = env
    spec = eb.CONFIGS["c3"]
    ids_np, mask_np, _ = eb.make_inputs(spec)
    ids = torch.from_numpy(ids_np.astype(np.int32)).cuda()
    mask = torch.from_numpy(mask_np.astype(np.int32)).cuda()
    out = torch.full((spec.batch, 384), 7.0, device="cuda")
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    for _ in range(2):
        minilm.encode_device(ids.data_ptr(), mask.data_ptr(), spec.batch, 128, out.data_ptr(), True,
                             sa.cuda_stream)
        minilm.encode_device(ids.data_ptr(), mask.data_ptr(), spec.batch, 0, out.data_ptr(), True,
                             sb.cuda_stream)
        minilm.synchronize()
        assert (out.cpu().numpy() == 0).all()
    minilm.encode_device(ids.data_ptr(), mask.data_ptr(), spec.batch, 128, out.data_ptr(), True,
                         sb.cuda_stream)
    minilm.synchronize()
    norms = np.linalg.norm(out.cpu().numpy().astype(np.float64), axis=1)
    np.testing.assert_allclose(norms, 1.0, atol=1e-5)


def test_concurrent_callers_and_workspace_growth(env, minilm):
    """encode(&self) is shared by rayon workers (src/lib.rs:440-451): many host
    threads on one model give the results of serial calls, across workspace growth."""
    from edgebert_amd import synth
    cases = []
    for i, (B, lo, hi) in enumerate([(3, 4, 10), (40, 8, 128), (2, 300, 512), (17, 2, 60)]):
        spec = synth.InputSpec(f"t{i}", synth.MINILM_L6, B, hi, lo, hi, 100 + i)
        ids, mask, _ = synth.make_inputs(spec)
        cases.append((ids, mask))
    serial = [minilm.encode_ids(i, m) for i, m in cases]
    results = {}

    def run(k):
        for rep in range(3):
            for j, (i, m) in enumerate(cases):
                results[(k, rep, j)] = minilm.encode_ids(i, m)

    ts = [threading.Thread(target=run, args=(k,)) for k in range(4)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert len(results) == 4 * 3 * len(cases)
    for (k, rep, j), v in results.items():
        np.testing.assert_array_equal(v, serial[j])


def test_from_pretrained_path_safetensors(env, tmp_path, weights_for):
    """config.json + model.safetensors (written by the safetensors library) -> the
    vectors of the same tensors handed over one by one."""
    torch, eb, Nn, L = env
    from safetensors.numpy import save_file
    from edgebert_amd import synth
    cfg = synth.TINY
    w = weights_for(cfg)
    st = {k: np.ascontiguousarray(v) for k, v in w.items()}
    st["pooler.dense.weight"] = np.zeros((cfg.hidden_size, cfg.hidden_size), np.float32)
    save_file(st, str(tmp_path / "model.safetensors"))
    with open(tmp_path / "config.json", "w") as f:
        json.dump({"hidden_size": cfg.hidden_size, "num_attention_heads": cfg.num_attention_heads,
                   "num_hidden_layers": cfg.num_hidden_layers, "intermediate_size": cfg.intermediate_size,
                   "vocab_size": cfg.vocab_size, "max_position_embeddings": cfg.max_position_embeddings,
                   "layer_norm_eps": cfg.layer_norm_eps, "hidden_act": "gelu", "model_type": "bert"}, f)
    m1 = eb.Model.from_pretrained_path(str(tmp_path))
    m2 = eb.Model.from_weights(w, cfg)
    ids, mask, _ = synth.make_inputs(synth.InputSpec("t", cfg, 5, 20, 3, 20, 4))
    np.testing.assert_array_equal(m1.encode_ids(ids, mask), m2.encode_ids(ids, mask))
    m1.close()
    m2.close()


def _write_pretrained_dir(path, cfg, tensors):
    from safetensors.torch import save_file
    save_file(tensors, str(path / "model.safetensors"))
    with open(path / "config.json", "w") as f:
        json.dump({"hidden_size": cfg.hidden_size, "num_attention_heads": cfg.num_attention_heads,
                   "num_hidden_layers": cfg.num_hidden_layers, "intermediate_size": cfg.intermediate_size,
                   "vocab_size": cfg.vocab_size, "max_position_embeddings": cfg.max_position_embeddings,
                   "layer_norm_eps": cfg.layer_norm_eps, "hidden_act": "gelu", "model_type": "bert"}, f)


@pytest.mark.parametrize("file_dtype", ["F16", "BF16"])
@pytest.mark.parametrize("model_dtype", ["fp32", "bf16"])
def test_from_pretrained_path_half_precision(env, tmp_path, weights_for, orc, file_dtype, model_dtype):
    """A model.safetensors holding F16 or BF16 tensors (MiniLM shape) is
    uploaded in its own encoding and converted on the device.  Its vectors are
    bit-identical to those of the same values handed over as f32 (widened in
    torch), for fp32 and bf16 models; the fp32 model also matches the oracle
    run on the widened weights."""
    torch, eb, Nn, L = env
    from edgebert_amd import synth
    cfg = synth.MINILM_L6
    w = weights_for(cfg)
    tdt = torch.float16 if file_dtype == "F16" else torch.bfloat16
    half = {k: torch.from_numpy(np.ascontiguousarray(v)).to(tdt) for k, v in w.items()}
    widened = {k: v.float().numpy() for k, v in half.items()}
    _write_pretrained_dir(tmp_path, cfg, half)
    m_file = eb.Model.from_pretrained_path(str(tmp_path), dtype=model_dtype)
    m_ref = eb.Model.from_weights(widened, cfg, model_dtype)
    try:
        spec = synth.CONFIGS["c2"]
        ids, mask, _ = synth.make_inputs(spec)
        got = m_file.encode_ids(ids, mask)
        np.testing.assert_array_equal(got, m_ref.encode_ids(ids, mask))
        if model_dtype == "fp32":
            import oracle
            sel = np.arange(0, spec.batch, 4)
            want = oracle.OracleModel(cfg, widened).encode_unpadded(ids[sel], mask[sel], normalize=True)
            assert np.abs(got[sel] - want).max() <= 1e-4
            assert cosine_rows(got[sel], want).min() >= 0.99999
    finally:
        m_file.close()
        m_ref.close()


def test_bf16_minilm_c3(env, weights_for, orc):
    """bf16 GEMMs at the headline shape: cosine >= 0.999 against the fp32 oracle."""
    torch, eb, Nn, L = env
    spec = eb.CONFIGS["c3"]
    ids, mask, _ = eb.make_inputs(spec)
    m16 = eb.Model.from_weights(weights_for(spec.model), spec.model, "bf16")
    got = m16.encode_ids(ids, mask)
    sel = np.arange(0, spec.batch, 32)
    want = orc.encode(ids[sel], mask[sel])
    assert cosine_rows(got[sel], want).min() >= 0.999
    m16.close()
