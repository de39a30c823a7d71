"""GPU parity: every hot-path kernel, called through the C ABI, against the oracle.

Tolerances (stated per test):
  * int4/int8 unpack, block and zero-point indexing, KV-cache row copies and
    paged slot writes: bit-exact.
  * fp32 outputs: max abs diff <= 6e-5 (plus the fp32-accumulation term for long
    reductions where noted).
  * fp16 outputs: |got - exact| <= 1e-3 + 1 fp16 ULP of the exact value (the
    output is itself rounded to fp16, so a correctly rounded result is within half
    an ULP; at |y| >= 2 one ULP exceeds 1e-3). The MFMA prefill GEMM also rounds
    each dequantised weight to fp16 (fp16((q - zp) * s)); its rigorous bound
    2^-11 * sum_k |a_k * w_nk| is added for that path and reported.
"""

from __future__ import annotations

import numpy as np
import pytest
import refs

pytestmark = pytest.mark.gpu


def dev(x, dtype=None):
    import torch

    t = torch.from_numpy(np.ascontiguousarray(x))
    if dtype is not None:
        t = t.to(dtype)
    return t.cuda()


def host(t):
    import torch

    torch.cuda.synchronize()
    return t.float().cpu().numpy() if t.is_floating_point() else t.cpu().numpy()


def ulp16(x):
    x = np.abs(np.asarray(x, np.float64))
    e = np.floor(np.log2(np.maximum(x, 2.0 ** -14)))
    return 2.0 ** (e - 10)


def assert_f16_close(got, exact, extra=0.0, what=""):
    got = np.asarray(got, np.float64)
    exact = np.asarray(exact, np.float64)
    tol = 1e-3 + ulp16(exact) + extra
    bad = np.abs(got - exact) > tol
    assert not bad.any(), (f"{what}: {bad.sum()} of {bad.size} beyond tolerance; max diff "
                           f"{np.abs(got - exact).max():.3e}, max ulp "
                           f"{refs.max_ulp_f16(got, exact):.2f}")


# ------------------------------------------------------------------ MatMulNBits --

def _mnb_inputs(rng, M, N, K, block, bits=4, asym=True, zp_all8=False, dtype=np.float32):
    nb = (K + block - 1) // block
    q = rng.integers(0, 1 << bits, size=(N, nb, block), dtype=np.uint8)
    import oracle

    B = oracle.pack_nibbles(q) if bits == 4 else q
    s = (np.abs(rng.standard_normal(N * nb) * 0.02) + 1e-4).astype(dtype)
    zp = None
    if zp_all8:
        zp = np.full(N * ((nb + 1) // 2), 0x88, np.uint8)
    elif asym:
        zp = oracle.pack_zero_points(rng.integers(0, 1 << bits, size=(N, nb), dtype=np.uint8), bits)
    A = rng.standard_normal((M, K)).astype(dtype)
    return A, B, s, zp


@pytest.mark.parametrize("K,N,block,skip,pair", [
    (1536, 2048, 32, False, False), (1536, 1536, 32, True, False), (1536, 17920, 32, True, True),
    (8960, 1536, 32, True, False), (4096, 512, 128, True, True), (1000, 64, 64, False, True),
    (1536, 24576, 32, True, False), (1536, 45056, 32, False, True),
    (14336, 512, 32, True, False), (4096, 1024, 32, True, True), (8192, 768, 32, True, False)])
def test_mnb_decode_fused(ortmi, oracle, K, N, block, skip, pair):
    """Norm prologue and SwiGLU-pair epilogue of the decode GEMV against the unfused
    ops of the oracle (norm rounded to fp16, matmul in fp64, SwiGLU op by op)."""
    import ctypes

    import torch

    rng = np.random.default_rng(K + N + block)
    A, B, s, zp = _mnb_inputs(rng, 1, N, K, block, asym=N % 3 == 0, dtype=np.float16)
    x = A[0]
    sk = rng.standard_normal(K).astype(np.float16) if skip else None
    gamma = (1 + 0.2 * rng.standard_normal(K)).astype(np.float16)
    y, r = oracle.rms_norm(x, gamma, 1e-6, skip=sk, round16=True)
    a16 = oracle.round_f16(y)
    exact = oracle.mnb_matmul(a16, B, s, zp, N, K, 4, block)
    lib = ortmi.load_kernels()
    dx, dB, ds, dg = dev(x), dev(B), dev(s), dev(gamma)
    dz = dev(zp) if zp is not None else None
    dsk = dev(sk) if skip else None
    res = torch.empty(K, dtype=torch.float16, device="cuda") if skip else None
    out = torch.empty(N // 2 if pair else N, dtype=torch.float16, device="cuda")
    p = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())  # noqa: E731
    flags = 1 | (2 if pair else 0)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    ortmi.check(lib.ortmi_matmul_nbits_decode_fused(
        p(dx), p(dsk), p(dg), 1e-6, p(res), p(dB), p(ds), p(dz), p(out), N, K, block,
        flags, 10, st))
    got = host(out)
    if skip:
        np.testing.assert_array_equal(host(res), r)
    W = oracle.mnb_dequant(B, s, zp, N, K, 4, block)
    # The normalised activations may differ from the oracle's by one fp16 rounding.
    extra = np.abs(W) @ (np.abs(a16) * 2.0 ** -10)
    if not pair:
        assert_f16_close(got, exact, extra=extra, what="fused norm GEMV")
        return
    g, u = oracle.round_f16(exact[0::2]), oracle.round_f16(exact[1::2])
    sig = oracle.round_f16(1.0 / (1.0 + np.exp(-g.astype(np.float64))))
    ref = oracle.round_f16(oracle.round_f16(g * sig) * u)
    # g and u each carry the GEMV tolerance; propagate it through silu(g) * u.
    eg = 1e-3 + ulp16(g) + extra[0::2]
    eu = 1e-3 + ulp16(u) + extra[1::2]
    dsilu = np.abs(sig * (1 + g * (1 - sig)))
    bound = eg * dsilu * np.abs(u) + eu * np.abs(g * sig) + eg * eu * 1.2 + 2 * ulp16(ref)
    assert (np.abs(got - ref) <= 1e-3 + bound).all(), np.abs(got - ref).max()


@pytest.mark.parametrize("K,N,block,skip,pair", [
    (1536, 2048, 32, False, False), (1536, 17920, 32, True, True), (4096, 512, 128, True, True),
    (8960, 1536, 32, True, False)])
def test_mnb_decode_fused_bf16(ortmi, oracle, K, N, block, skip, pair):
    """The fused decode GEMV with bf16 tensors (norm prologue in fp32 rounded to
    bf16, the fp8-convert dot product, SwiGLU op by op in bf16) against the
    oracle's unfused ops on the same bf16 inputs."""
    import ctypes

    import torch

    def rb(a):  # round to bf16 (RNE) and widen back
        return torch.from_numpy(np.asarray(a, np.float32)).to(torch.bfloat16).float().numpy()

    def tb(a):
        return torch.from_numpy(np.asarray(a, np.float32)).to(torch.bfloat16).cuda()

    rng = np.random.default_rng(K + N + block + 1)
    A, B, s, zp = _mnb_inputs(rng, 1, N, K, block, asym=N % 3 == 0)
    x, s_r = rb(A[0]), rb(s)
    sk = rb(rng.standard_normal(K)) if skip else None
    gamma = rb(1 + 0.2 * rng.standard_normal(K))
    y, r = oracle.rms_norm(x, gamma, 1e-6, skip=sk)
    a_b = rb(y)
    exact = oracle.mnb_matmul(a_b[None], B, s_r, zp, N, K, 4, block)[0]
    lib = ortmi.load_kernels()
    # Every device tensor is held by a name until the kernel has run (a temporary
    # would go back to the allocator and its block could be handed out again).
    dx, dg, ds, dB = tb(x), tb(gamma), tb(s_r), dev(B)
    dz = dev(zp) if zp is not None else None
    dsk = tb(sk) if skip else None
    res = torch.empty(K, dtype=torch.bfloat16, device="cuda") if skip else None
    out = torch.empty(N // 2 if pair else N, dtype=torch.bfloat16, device="cuda")
    p = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())  # noqa: E731
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    ortmi.check(lib.ortmi_matmul_nbits_decode_fused(
        p(dx), p(dsk), p(dg), 1e-6, p(res), p(dB), p(ds), p(dz), p(out), N, K,
        block, 1 | (2 if pair else 0), 16, st))  # 16: bf16
    got = host(out)
    if skip:
        np.testing.assert_array_equal(host(res), rb(r))
    W = oracle.mnb_dequant(B, s_r, zp, N, K, 4, block)
    # The normalised activations may differ by one bf16 rounding; fp32 accumulation.
    extra = np.abs(W) @ (np.abs(a_b) * 2.0 ** -7) + 2.0 ** -18 * (np.abs(W) @ np.abs(a_b))
    if not pair:
        assert (np.abs(got - exact) <= 2.0 ** -8 * np.abs(exact) + extra).all(), \
            np.abs(got - exact).max()
        return
    g, u = rb(exact[0::2]), rb(exact[1::2])
    sig = rb(1.0 / (1.0 + np.exp(-g.astype(np.float64))))
    ref = rb(rb(g * sig) * u)
    eg = 2.0 ** -8 * np.abs(g) + extra[0::2]
    eu = 2.0 ** -8 * np.abs(u) + extra[1::2]
    dsilu = np.abs(sig * (1 + g * (1 - sig)))
    bound = eg * dsilu * np.abs(u) + eu * np.abs(g * sig) + eg * eu * 1.2 + 2.0 ** -7 * np.abs(ref)
    assert (np.abs(got - ref) <= 1e-6 + bound).all(), np.abs(got - ref).max()


@pytest.mark.parametrize("K,block", [(256, 32), (1176, 32), (256, 64), (512, 128), (8960, 32),
                                     (1536, 32)])
@pytest.mark.parametrize("asym", [False, True])
def test_mnb_gemv_fp32(ortmi, oracle, K, block, asym):
    import torch

    rng = np.random.default_rng(K + block + asym)
    N = 200
    A, B, s, zp = _mnb_inputs(rng, 1, N, K, block, asym=asym)
    Y = ortmi.matmul_nbits(dev(A), dev(B), dev(s), None if zp is None else dev(zp), K=K, N=N,
                           block_size=block)
    ref = oracle.mnb_matmul(A, B, s, zp, N, K, 4, block)
    got = host(Y)
    # fp32: 6e-5 plus fp32 accumulation over K terms (bounded by K * eps32 * sum|a*w|).
    W = refs.dequant_ref(B, s, zp, N, K, 4, block)
    acc_bound = K * 2.0 ** -24 * (np.abs(A.astype(np.float64)) @ np.abs(W).T)
    assert np.all(np.abs(got - ref) <= 6e-5 + acc_bound), np.abs(got - ref).max()
    assert Y.dtype == torch.float32


def test_mnb_gemv_config1_shape(ortmi, oracle):
    """K=4096, N=11008, fp32, block 32, zero points all 8 (the single-node config)."""
    rng = np.random.default_rng(2024)
    K, N = 4096, 11008
    A, B, s, zp = _mnb_inputs(rng, 1, N, K, 32, zp_all8=True)
    got = host(ortmi.matmul_nbits(dev(A), dev(B), dev(s), dev(zp), K=K, N=N))
    ref = oracle.mnb_matmul(A, B, s, zp, N, K, 4, 32)
    diff = np.abs(got - ref).max()
    assert diff <= 6e-5, diff


@pytest.mark.parametrize("K,block,N", [(1536, 32, 300), (8960, 32, 300), (4096, 64, 300),
                                       (1536, 32, 20700), (520, 32, 21001), (1000, 64, 20481),
                                       (11008, 32, 300), (14336, 32, 300), (12000, 64, 257),
                                       (16384, 128, 200), (2048, 32, 999), (4096, 32, 4096),
                                       (8192, 32, 3072), (16384, 32, 515)])
def test_mnb_gemv_fp16(ortmi, oracle, K, block, N):
    """Includes long walks over short rows (N beyond 80 rows per CU, K <= 1536),
    which take four rows per wave, with an odd N and a partial final block, the
    long rows of 7B-class down projections (K = 11008, 14336, up to 16384: six to
    eight 32-code chunks per lane), and rows of whole 64-chunk runs at block 32,
    which take interleaved chunks (K = 2048 to 16384, one to eight per lane)."""
    import torch

    rng = np.random.default_rng(K * 3 + block + N)
    A, B, s, zp = _mnb_inputs(rng, 1, N, K, block, dtype=np.float16)
    Y = ortmi.matmul_nbits(dev(A), dev(B), dev(s), dev(zp), K=K, N=N, block_size=block)
    assert Y.dtype == torch.float16
    ref = oracle.mnb_matmul(A, B, s, zp, N, K, 4, block)
    assert_f16_close(host(Y), ref, what="gemv fp16")


@pytest.mark.parametrize("K,N", [(4096, 1000), (8192, 700), (14336, 257), (2048, 64)])
def test_mnb_gemv_fp16_interleaved_symmetric(ortmi, oracle, K, N):
    """Interleaved chunks (block 32, rows of whole 64-chunk runs) without zero
    points, the decoder's symmetric form: every code is offset by 8."""
    rng = np.random.default_rng(K + N + 7)
    A, B, s, zp = _mnb_inputs(rng, 1, N, K, 32, asym=False, dtype=np.float16)
    assert zp is None
    Y = ortmi.matmul_nbits(dev(A), dev(B), dev(s), None, K=K, N=N, block_size=32)
    ref = oracle.mnb_matmul(A, B, s, None, N, K, 4, 32)
    assert_f16_close(host(Y), ref, what="gemv fp16 symmetric")


@pytest.mark.parametrize("M", [2, 8, 64, 130])
@pytest.mark.parametrize("K,N,block", [(256, 192, 32), (512, 256, 64), (384, 160, 128),
                                       (1176, 64, 32)])
def test_mnb_gemm_fp16(ortmi, oracle, M, K, N, block):
    rng = np.random.default_rng(M * 11 + K + N + block)
    A, B, s, zp = _mnb_inputs(rng, M, N, K, block, dtype=np.float16)
    got = host(ortmi.matmul_nbits(dev(A), dev(B), dev(s), dev(zp), K=K, N=N, block_size=block))
    ref = oracle.mnb_matmul(A, B, s, zp, N, K, 4, block)
    W = refs.dequant_ref(B, s, zp, N, K, 4, block)
    bound = 2.0 ** -11 * (np.abs(A.astype(np.float64)) @ np.abs(W).T)
    assert_f16_close(got, ref, extra=bound, what="gemm fp16")
    # Structure check with the weight rounding modelled: exact to output rounding.
    W16 = W.astype(np.float16).astype(np.float64)
    ref16 = A.astype(np.float64) @ W16.T
    assert_f16_close(got, ref16, what="gemm fp16 (fp16 weights)")


def _check_gemm_rows(oracle, got_rows, A_rows, B, s, zp, N, K, block, what):
    """Two checks of MFMA-GEMM output rows. Primary: against fp64 A . W16^T with the
    dequantised weights rounded to fp16 once (what the kernel feeds the matrix cores),
    within the plain fp16 bar (1e-3 + 1 ULP). Secondary: against the oracle's exact
    fp64 dequantisation, within the bar plus the rigorous bound 2^-11 sum |a w| of
    that one weight rounding."""
    W = refs.dequant_ref(B, s, zp, N, K, 4, block)
    W16 = W.astype(np.float16).astype(np.float64)
    assert_f16_close(got_rows, A_rows.astype(np.float64) @ W16.T, what=what + " (fp16 weights)")
    ref = oracle.mnb_matmul(A_rows, B, s, zp, N, K, 4, block)
    bound = 2.0 ** -11 * (np.abs(A_rows.astype(np.float64)) @ np.abs(W).T)
    assert_f16_close(got_rows, ref, extra=bound, what=what)


@pytest.mark.parametrize("M,N,K", [
    (512, 4096, 4096),   # the prefill GEMM config
    (512, 1536, 8960),   # the decoder prefill's down_proj (64x64 tiles, k split)
    (512, 2048, 1536),   # the decoder prefill's merged QKV
])
def test_mnb_gemm_config2_shape(ortmi, oracle, M, N, K):
    """Prefill GEMM shapes at full size, fp16, block 32, zero points U{0..15}. The
    prefill GEMM config (512 x 4096 x 4096) is checked on all 512 rows; the two
    decoder shapes on a sample of rows, which keeps the CPU side short."""
    rng = np.random.default_rng(M + N + K)
    A, B, s, zp = _mnb_inputs(rng, M, N, K, 32, dtype=np.float16)
    got = host(ortmi.matmul_nbits(dev(A), dev(B), dev(s), dev(zp), K=K, N=N))
    rows = np.arange(M) if (N, K) == (4096, 4096) else np.r_[np.arange(0, M, 37), M - 1]
    _check_gemm_rows(oracle, got[rows], A[rows], B, s, zp, N, K, 32, f"gemm {M}x{N}x{K}")


@pytest.mark.parametrize("M,N,K,block", [(1030, 8200, 1000, 64), (1024, 8192, 1536, 32)])
def test_mnb_gemm_large_tiles(ortmi, oracle, M, N, K, block):
    """Shapes that fill the CUs twice with 128x128 tiles (the weights-in-registers
    tile): ragged M, N and K edges, and the aligned case, on a sample of rows."""
    rng = np.random.default_rng(M + N + K)
    A, B, s, zp = _mnb_inputs(rng, M, N, K, block, dtype=np.float16)
    got = host(ortmi.matmul_nbits(dev(A), dev(B), dev(s), dev(zp), K=K, N=N, block_size=block))
    rows = np.r_[np.arange(0, M, 41), M - 1]
    _check_gemm_rows(oracle, got[rows], A[rows], B, s, zp, N, K, block, "gemm large tiles")


@pytest.mark.parametrize("M,N,K,block", [(37, 400, 1536, 32), (512, 2048, 1536, 32),
                                         (512, 17920, 1536, 32), (64, 256, 1000, 64)])
def test_mnb_gemm_swiglu_pairs(ortmi, oracle, M, N, K, block):
    """SwiGLU in the GEMM epilogue over interleaved gate/up rows equals the GEMM
    followed by the SwiGLU-pairs kernel bit for bit (the same tile walk), and the
    oracle's unfused ops (fp16 matmul outputs, SwiGLU op by op) within tolerance.
    The shapes cover the 64x64, 64x128 and 128x128 tile forms and K % 64 != 0."""
    import ctypes

    import torch

    rng = np.random.default_rng(M + N + K)
    A, B, s, zp = _mnb_inputs(rng, M, N, K, block, dtype=np.float16)
    dA, dB, ds, dz = dev(A), dev(B), dev(s), dev(zp)
    lib = ortmi.load_kernels()
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    y = torch.empty((M, N // 2), dtype=torch.float16, device="cuda")
    ortmi.check(lib.ortmi_matmul_nbits_swiglu_pairs(p(dA), p(dB), p(ds), p(dz), p(y), M, N, K,
                                                    block, 10, st))
    full = ortmi.matmul_nbits(dA, dB, ds, dz, K=K, N=N, block_size=block)
    y2 = torch.empty((M, N // 2), dtype=torch.float16, device="cuda")
    ortmi.check(lib.ortmi_swiglu_pairs(p(full), p(y2), M, N // 2, 10, st))
    torch.cuda.synchronize()
    assert torch.equal(y, y2), "epilogue SwiGLU differs from the unfused pair"
    rows = np.arange(0, M, max(1, M // 16))
    mm = oracle.mnb_matmul(A[rows], B, s, zp, N, K, 4, block)
    g = oracle.round_f16(mm[:, 0::2])
    u = oracle.round_f16(mm[:, 1::2])
    sig = oracle.round_f16(1.0 / (1.0 + np.exp(-g.astype(np.float64))))
    ref = oracle.round_f16(oracle.round_f16(g * sig) * u)
    W = refs.dequant_ref(B, s, zp, N, K, 4, block)
    bound = 2.0 ** -11 * (np.abs(A[rows].astype(np.float64)) @ np.abs(W).T)
    # a 1-ulp difference in g or u moves the result by about that much times |u| or |g|
    extra = 4.0 * (bound[:, 0::2] * np.abs(u) + bound[:, 1::2] * np.abs(g) + bound[:, 0::2])
    assert_f16_close(host(y)[rows], ref, extra=extra, what="gemm swiglu pairs")


@pytest.mark.parametrize("M", [1, 5])
@pytest.mark.parametrize("K,N,block,asym", [(1536, 300, 32, True), (4096, 257, 64, False),
                                            (1000, 130, 128, True), (8960, 64, 32, False)])
def test_mnb_bf16(ortmi, oracle, M, K, N, block, asym):
    """bf16 activations and scales (M = 1: the decode GEMV and its fp8-convert dot
    product; M > 1: the matrix-core GEMM, which rounds each dequantised weight to
    bf16 once) against the oracle run on the same bf16 values: within the output's
    bf16 rounding plus fp32 accumulation, plus 2^-9 sum |a w| for that weight
    rounding when M > 1."""
    import torch

    rng = np.random.default_rng(M * 7 + K + N + block)
    A, B, s, zp = _mnb_inputs(rng, M, N, K, block, asym=asym)
    tA = torch.from_numpy(A).to(torch.bfloat16)
    ts = torch.from_numpy(s).to(torch.bfloat16)
    A_r, s_r = tA.float().numpy(), ts.float().numpy()
    got = host(ortmi.matmul_nbits(tA.cuda(), dev(B), ts.cuda(), dev(zp) if asym else None,
                                  K=K, N=N, block_size=block))
    ref = oracle.mnb_matmul(A_r, B, s_r, zp if asym else None, N, K, 4, block)
    W = refs.dequant_ref(B, s_r, zp if asym else None, N, K, 4, block)
    accum = 2.0 ** -18 * (np.abs(A_r.astype(np.float64)) @ np.abs(W).T)
    wround = 2.0 ** -9 * (np.abs(A_r.astype(np.float64)) @ np.abs(W).T) if M > 1 else 0.0
    bound = 2.0 ** -8 * np.abs(ref) + accum + wround
    assert (np.abs(got - ref) <= bound).all(), np.abs(got - ref).max()


@pytest.mark.parametrize("M,K,N,block", [(64, 512, 256, 32), (130, 1176, 64, 32),
                                         (40, 1024, 384, 64), (96, 768, 200, 128),
                                         (512, 4096, 4096, 32)])
def test_mnb_gemm_bf16(ortmi, oracle, M, K, N, block):
    """bf16 prefill on the matrix cores (v_mfma_f32_32x32x16_bf16), zero points
    U{0..15}. Primary check: against fp64 A . Wbf16^T with the dequantised weights
    rounded to bf16 once, as the kernel feeds them, within the output's bf16
    rounding plus fp32 accumulation. Secondary: against the oracle's exact
    dequantisation, plus the rigorous bound 2^-9 sum |a w| of that rounding."""
    import torch

    rng = np.random.default_rng(M + K + N + block)
    A, B, s, zp = _mnb_inputs(rng, M, N, K, block)
    tA = torch.from_numpy(A).to(torch.bfloat16)
    ts = torch.from_numpy(s).to(torch.bfloat16)
    A_r, s_r = tA.float().numpy(), ts.float().numpy()
    got = host(ortmi.matmul_nbits(tA.cuda(), dev(B), ts.cuda(), dev(zp), K=K, N=N,
                                  block_size=block))
    rows = np.r_[np.arange(0, M, max(1, M // 24)), M - 1]
    W = refs.dequant_ref(B, s_r, zp, N, K, 4, block)
    Wb = torch.from_numpy(W.astype(np.float32)).to(torch.bfloat16).double().numpy()
    Ar = A_r[rows].astype(np.float64)
    accum = 2.0 ** -18 * (np.abs(Ar) @ np.abs(W).T)
    want = Ar @ Wb.T
    bound = 2.0 ** -8 * np.abs(want) + accum + 1e-30
    bad = np.abs(got[rows] - want) > bound
    assert not bad.any(), f"bf16 gemm (bf16 weights): max diff {np.abs(got[rows] - want).max():.3e}"
    ref = oracle.mnb_matmul(A_r[rows], B, s_r, zp, N, K, 4, block)
    bound2 = 2.0 ** -8 * np.abs(ref) + accum + 2.0 ** -9 * (np.abs(Ar) @ np.abs(W).T)
    assert (np.abs(got[rows] - ref) <= bound2).all(), np.abs(got[rows] - ref).max()


@pytest.mark.parametrize("M,bits,block", [(1, 8, 32), (3, 8, 64), (1, 4, 16), (5, 4, 16)])
def test_mnb_generic_forms_fp32(ortmi, oracle, M, bits, block):
    rng = np.random.default_rng(M + bits + block)
    K, N = 3 * block + 5, 70
    A, B, s, zp = _mnb_inputs(rng, M, N, K, block, bits=bits)
    got = host(ortmi.matmul_nbits(dev(A), dev(B), dev(s), dev(zp), K=K, N=N, bits=bits,
                                  block_size=block))
    ref = oracle.mnb_matmul(A, B, s, zp, N, K, bits, block)
    assert np.abs(got - ref).max() <= 6e-5


@pytest.mark.parametrize("dtype", [np.float16, np.float32, "bf16"])
@pytest.mark.parametrize("V,D,block,asym,i64", [(2, 32, 16, False, True), (300, 1536, 32, True, True),
                                                (97, 200, 64, True, False), (151, 1024, 128, False, False)])
def test_gather_block_quantized(ortmi, oracle, dtype, V, D, block, asym, i64):
    """GatherBlockQuantized on the GPU equals the oracle bit for bit (fp32, fp16 and
    bf16 scales; symmetric and packed zero points; int32/int64 ids with negative and
    out-of-range ids; a partial final block when D % block != 0)."""
    import torch

    rng = np.random.default_rng(V + D + block + asym)
    nb = (D + block - 1) // block
    q = rng.integers(0, 16, size=(V, D), dtype=np.uint8)
    data = (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8)
    s32 = (np.abs(rng.standard_normal((V, nb))) * 0.05 + 1e-3).astype(np.float32)
    zp = oracle.pack_zero_points(rng.integers(0, 16, size=(V, nb), dtype=np.uint8), 4) if asym else None
    ids = rng.integers(-V, V, size=(3, 7)).astype(np.int64 if i64 else np.int32)
    ids[0, 0], ids[2, 6] = V + 3, -V - 1  # out of range: zero rows
    if dtype == "bf16":
        ts = torch.from_numpy(s32).to(torch.bfloat16)
        s_ref = ts.to(torch.float32).numpy()
        ts = ts.cuda()
    else:
        s_np = s32.astype(dtype)
        ts, s_ref = dev(s_np), s_np.astype(np.float32)
    got = ortmi.gather_block_quantized(dev(data), ts, dev(ids), dev(zp) if asym else None,
                                       block_size=block)
    assert tuple(got.shape) == (3, 7, D)
    ref = oracle.gather_block_quantized(data, s_ref, zp, ids, block, np.float32)
    if dtype == "bf16":
        ref = torch.from_numpy(ref).to(torch.bfloat16).to(torch.float32).numpy()
        got = got.to(torch.float32)
    elif dtype == np.float16:
        ref = ref.astype(np.float16).astype(np.float32)
    np.testing.assert_array_equal(host(got).astype(np.float32), ref)
    assert not host(got)[0, 0].any() and not host(got)[2, 6].any()


def test_mnb_dequant_indexing_bit_exact(ortmi, oracle):
    """One-hot activations read single dequantised columns: (q - zp) * s must be
    exact in fp32 for every code, block and zero-point nibble."""
    rng = np.random.default_rng(5)
    N, K, block = 64, 256, 32
    _, B, s, zp = _mnb_inputs(rng, 1, N, K, block)
    W = oracle.mnb_dequant(B, s, zp, N, K, 4, block)
    Bd, sd, zd = dev(B), dev(s), dev(zp)
    for k in (0, 1, 30, 31, 32, 33, 127, 128, 255):
        e = np.zeros((1, K), np.float32)
        e[0, k] = 1
        got = host(ortmi.matmul_nbits(dev(e), Bd, sd, zd, K=K, N=N))
        np.testing.assert_array_equal(got[0], W[:, k])


# ------------------------------------------------------------ GroupQueryAttention --

def _gqa_inputs(rng, B, S, H, KV, hd, cap, rope=True, base=10000.0, max_pos=8192):
    q = rng.standard_normal((B, S, H * hd)).astype(np.float16)
    k = rng.standard_normal((B, S, KV * hd)).astype(np.float16)
    v = rng.standard_normal((B, S, KV * hd)).astype(np.float16)
    pk = rng.standard_normal((B, KV, cap, hd)).astype(np.float16)
    pv = rng.standard_normal((B, KV, cap, hd)).astype(np.float16)
    cos = sin = None
    if rope:
        c, s_ = refs.rotary_caches(max_pos, hd, base)
        cos, sin = c.astype(np.float16), s_.astype(np.float16)
    return q, k, v, pk, pv, cos, sin


def _run_gqa(ortmi, oracle, B, S, H, KV, hd, cap, past, rope=True, interleaved=False,
             inplace=False, seed=0, base=10000.0):
    import torch

    rng = np.random.default_rng(seed)
    q, k, v, pk, pv, cos, sin = _gqa_inputs(rng, B, S, H, KV, hd, cap, rope, base)
    total = past + S
    dq, dk, dv, dpk, dpv = dev(q), dev(k), dev(v), dev(pk), dev(pv)
    kw = {}
    if inplace:
        kw = dict(present_key=dpk, present_value=dpv)
    out, prk, prv = ortmi.group_query_attention(
        dq, dk, dv, dpk, dpv, dev(np.full(B, total - 1, np.int32)), total,
        None if cos is None else dev(cos), None if sin is None else dev(sin), num_heads=H,
        kv_num_heads=KV, do_rotary=int(rope), rotary_interleaved=int(interleaved), **kw)
    ro, rk, rv, shared = oracle.gqa(q, k, v, pk, pv, total, H, KV, cos=cos, sin=sin,
                                    interleaved=interleaved, round16=True)
    assert_f16_close(host(out), ro, what="gqa output")
    got_k, got_v = host(prk), host(prv)
    vp = past if (0 <= past <= cap) else cap
    # Rows other than the new ones are bit-exact copies; new V rows are copies of
    # the input; new K rows are RoPE outputs rounded once (<= 1 fp16 ULP).
    old = np.ones(got_k.shape[2], bool)
    old[vp:vp + S] = False
    np.testing.assert_array_equal(got_k[:, :, old], rk[:, :, old].astype(np.float16).astype(np.float32))
    np.testing.assert_array_equal(got_v, rv.astype(np.float16).astype(np.float32))
    dk_new = np.abs(got_k[:, :, vp:vp + S] - rk[:, :, vp:vp + S])
    assert (dk_new <= ulp16(rk[:, :, vp:vp + S])).all()
    assert prk.dtype == torch.float16
    return shared


@pytest.mark.parametrize("interleaved", [False, True])
def test_gqa_decode_growing(ortmi, oracle, interleaved):
    assert not _run_gqa(ortmi, oracle, B=2, S=1, H=8, KV=2, hd=128, cap=300, past=300,
                        interleaved=interleaved, seed=1)


def test_gqa_decode_shared_inplace(ortmi, oracle):
    assert _run_gqa(ortmi, oracle, B=2, S=1, H=12, KV=2, hd=128, cap=512, past=200, inplace=True,
                    seed=2, base=1e6)


@pytest.mark.parametrize("H,KV,hd", [(14, 2, 64), (6, 2, 128), (5, 1, 128), (24, 3, 128)])
def test_gqa_decode_group_sizes(ortmi, oracle, H, KV, hd):
    """Every query-heads-per-KV-head ratio 1..8 has a decode kernel (G = 7, 3, 5, 8 here)."""
    assert _run_gqa(ortmi, oracle, B=2, S=1, H=H, KV=KV, hd=hd, cap=700, past=650, inplace=True,
                    seed=H * 10 + KV, base=1e6)


@pytest.mark.parametrize("H,KV,hd", [(12, 2, 128), (32, 8, 128), (8, 8, 64), (32, 32, 96)])
def test_gqa_decode_capturable(ortmi, oracle, H, KV, hd):
    """Device-resident total_sequence_length: equal to the oracle, and a HIP graph
    captured at one length and replayed at others equals eager calls bit for bit."""
    import torch

    rng = np.random.default_rng(H + KV + hd)
    B, cap, past = 2, 300, 140
    q, k, v, pk, pv, cos, sin = _gqa_inputs(rng, B, 1, H, KV, hd, cap, True, 1e6)
    dcos, dsin = dev(cos), dev(sin)
    tot = torch.tensor([past + 1], dtype=torch.int32, device="cuda")
    dpk, dpv = dev(pk), dev(pv)
    out = ortmi.group_query_attention_decode_capturable(
        dev(q), dev(k), dev(v), dpk, dpv, tot, dcos, dsin, num_heads=H, kv_num_heads=KV)
    ro, rk, rv, shared = oracle.gqa(q, k, v, pk, pv, past + 1, H, KV, cos=cos, sin=sin,
                                    round16=True)
    assert shared
    assert_f16_close(host(out), ro, what="capturable gqa")
    np.testing.assert_array_equal(host(dpv), rv.astype(np.float16).astype(np.float32))
    old = np.ones(cap, bool)
    old[past] = False
    np.testing.assert_array_equal(host(dpk)[:, :, old], pk.astype(np.float32)[:, :, old])

    # Graph captured at total = 61, replayed at 62..64 with eager work in between.
    sq, sk, sv = dev(q), dev(k), dev(v)
    kg, vg = dev(pk), dev(pv)
    ke, ve = dev(pk), dev(pv)
    ws = torch.empty(ortmi.load_kernels().ortmi_group_query_attention_workspace_size(
        B, 1, H, hd, cap), dtype=torch.uint8, device="cuda")
    tg = torch.tensor([61], dtype=torch.int32, device="cuda")
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        gout = ortmi.group_query_attention_decode_capturable(
            sq, sk, sv, kg, vg, tg, dcos, dsin, num_heads=H, kv_num_heads=KV, workspace=ws)
    for t in (62, 63, 64):
        step = rng.standard_normal((3, B, 1, max(H, KV) * hd)).astype(np.float16)
        sq.copy_(dev(step[0][..., :H * hd]))
        sk.copy_(dev(step[1][..., :KV * hd]))
        sv.copy_(dev(step[2][..., :KV * hd]))
        tg.fill_(t)
        graph.replay()
        torch.cuda.synchronize()
        te = torch.tensor([t], dtype=torch.int32, device="cuda")
        eout = ortmi.group_query_attention_decode_capturable(
            sq, sk, sv, ke, ve, te, dcos, dsin, num_heads=H, kv_num_heads=KV)
        torch.cuda.synchronize()
        assert torch.equal(gout, eout), f"replay at total={t} differs from eager"
        assert torch.equal(kg, ke) and torch.equal(vg, ve)


@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("H,KV,hd,past", [(12, 2, 128, 140), (8, 8, 64, 5), (16, 4, 128, 299),
                                         (32, 8, 128, 290)])
def test_gqa_partials_merge_gemv(ortmi, oracle, H, KV, hd, past, dt):
    """One-token attention left as split partials and merged in the o_proj GEMV's
    prologue equals the capturable attention followed by the plain GEMV (same KV
    append, bit for bit; outputs within the GEMV tolerance plus one rounding of
    each activation to the dtype). bf16 runs the merge GEMV's fp8-convert dot
    product."""
    import ctypes

    import torch

    bf = dt == "bf16"
    code = 16 if bf else 10
    tdt = torch.bfloat16 if bf else torch.float16

    def rnd(a):  # round to the dtype and widen back
        return torch.from_numpy(np.asarray(a, np.float32)).to(tdt).float().numpy()

    def td(a):
        return torch.from_numpy(np.asarray(a, np.float32)).to(tdt).cuda()

    rng = np.random.default_rng(H * 3 + hd + past)
    B, cap = 1, 300
    q, k, v, pk, pv, cos, sin = _gqa_inputs(rng, B, 1, H, KV, hd, cap, True, 1e6)
    if bf:
        q, k, v, pk, pv, cos, sin = (rnd(x) for x in (q, k, v, pk, pv, cos, sin))
    dq, dk, dv, dcos, dsin = (td(x) for x in (q, k, v, cos, sin))
    tot = torch.tensor([past + 1], dtype=torch.int32, device="cuda")
    ka, va, kb, vb = td(pk), td(pv), td(pk), td(pv)
    ref = ortmi.group_query_attention_decode_capturable(
        dq, dk, dv, ka, va, tot, dcos, dsin, num_heads=H, kv_num_heads=KV)
    K, N, block = H * hd, 1536, 32
    _, W, s_, zp = _mnb_inputs(rng, 1, N, K, block, asym=True)
    s_ = rnd(s_)
    dW, ds, dz = dev(W), td(s_), dev(zp)
    y_ref = ortmi.matmul_nbits(ref.reshape(1, K), dW, ds, dz, K=K, N=N, bits=4, block_size=block)
    lib = ortmi.load_kernels()
    ns = lib.ortmi_group_query_attention_decode_splits(B, H, KV, hd, cap)
    assert ns >= 1
    part = torch.empty(B * H * ns * (hd + 2), dtype=torch.float32, device="cuda")
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    ortmi.check(lib.ortmi_group_query_attention_decode_partials(
        p(dq), p(dk), p(dv), p(kb), p(vb), cap, p(tot), p(dcos), p(dsin), cos.shape[1],
        cos.shape[0], p(part), B, H, KV, hd, 0.0, 0, code, st))
    y = torch.empty(N, dtype=tdt, device="cuda")
    ortmi.check(lib.ortmi_matmul_nbits_decode_merge(
        p(part), ns, hd, p(dW), p(ds), p(dz), p(y), N, K, block, code, st))
    torch.cuda.synchronize()
    assert torch.equal(ka, kb) and torch.equal(va, vb)
    a = host(ref).reshape(K)
    Wd = oracle.mnb_dequant(W, s_, zp, N, K, 4, block)
    exact = oracle.mnb_matmul(rnd(a)[None], W, s_, zp, N, K, 4, block)[0]
    if not bf:
        extra = np.abs(Wd) @ (np.abs(a) * 2.0 ** -10)
        assert_f16_close(host(y), exact, extra=extra, what="merged o_proj GEMV")
        assert_f16_close(host(y_ref).reshape(N), exact, extra=extra, what="unfused o_proj GEMV")
        return
    # bf16: output rounding (2^-8 relative), one bf16 rounding of each merged
    # activation, fp32 accumulation.
    extra = np.abs(Wd) @ (np.abs(a) * 2.0 ** -7) + 2.0 ** -18 * (np.abs(Wd) @ np.abs(a))
    for got, what in ((host(y), "merged"), (host(y_ref).reshape(N), "unfused")):
        assert (np.abs(got - exact) <= 2.0 ** -8 * np.abs(exact) + extra).all(), \
            (what, np.abs(got - exact).max())


@pytest.mark.parametrize("S,past,cap", [(1, 40, 64), (9, 10, 64)])
def test_gqa_packed_qkv(ortmi, oracle, S, past, cap):
    """Packed [B, S, (H + 2 KV) hd] input (key = value = None) equals separate Q/K/V."""
    rng = np.random.default_rng(S * 7 + past)
    B, H, KV, hd = 2, 12, 2, 128
    q, k, v, pk, pv, cos, sin = _gqa_inputs(rng, B, S, H, KV, hd, cap, True, 1e6)
    packed = np.concatenate([q, k, v], axis=-1)
    total = past + S
    dpk, dpv = dev(pk), dev(pv)
    out, _, _ = ortmi.group_query_attention(
        dev(packed), None, None, dpk, dpv, dev(np.full(B, total - 1, np.int32)), total,
        dev(cos), dev(sin), num_heads=H, kv_num_heads=KV, do_rotary=1, present_key=dpk,
        present_value=dpv)
    ro, rk, rv, _ = oracle.gqa(q, k, v, pk, pv, total, H, KV, cos=cos, sin=sin, round16=True)
    assert_f16_close(host(out), ro, what="packed gqa")
    np.testing.assert_array_equal(host(dpv), rv.astype(np.float16).astype(np.float32))


def test_gqa_decode_shared_separate_present(ortmi, oracle):
    assert _run_gqa(ortmi, oracle, B=3, S=1, H=4, KV=4, hd=64, cap=100, past=37, seed=3)


@pytest.mark.parametrize("B,S,H,KV,cap,past,inplace", [
    (2, 1, 32, 32, 700, 650, True),    # Phi-3.5-mini's heads: one query head per KV head
    (2, 1, 12, 4, 300, 300, False),    # growing contract (past rows copied by the kernel)
    (3, 1, 16, 2, 8192, 8000, True),   # long context: many key splits
    (2, 40, 12, 4, 100, 30, True),     # prefill chunk after cached rows (matrix-core tiles)
    (1, 300, 32, 32, 300, 0, True),    # a prompt into an empty buffer
])
def test_gqa_head96(ortmi, oracle, B, S, H, KV, cap, past, inplace):
    """Head size 96 (Phi-3.5-mini) on the fast kernels: one-token decode on 16-lane
    groups whose last 4 lanes are padding, prefill on the matrix-core tiles; the
    output within the fp16 tolerance, every cached row bit-exact, the new K rows
    within one fp16 ulp (full rotary over the 96 dims, half 48)."""
    _run_gqa(ortmi, oracle, B=B, S=S, H=H, KV=KV, hd=96, cap=cap, past=past, inplace=inplace,
             seed=96 + S + past, base=1e4)


def test_gqa_decode_config3_shape(ortmi, oracle):
    """B=8, H=32, KV=8, hd=128, past 4096, growing contract (the decode config):
    every present row bit-exact (the new K row within one fp16 ulp), the output
    within the fp16 tolerance."""
    assert not _run_gqa(ortmi, oracle, B=8, S=1, H=32, KV=8, hd=128, cap=4096, past=4096, seed=4)


@pytest.mark.parametrize("S,past,cap", [(16, 0, 0), (5, 7, 7), (33, 10, 64)])
def test_gqa_prefill(ortmi, oracle, S, past, cap):
    _run_gqa(ortmi, oracle, B=2, S=S, H=8, KV=2, hd=128, cap=cap, past=past, seed=S + past)


@pytest.mark.parametrize("S,past,cap,H", [(200, 150, 400, 8), (512, 0, 512, 12)])
def test_gqa_prefill_key_splits(ortmi, oracle, S, past, cap, H):
    """Prompts whose tiles are split over keys (chunks of 128 keys crossing the
    causal diagonal of several tiles) and merged per (token, head) row."""
    _run_gqa(ortmi, oracle, B=1 if S == 512 else 2, S=S, H=H, KV=2, hd=128, cap=cap,
             past=past, inplace=past == 0, seed=S + 7, base=1e6)


def test_gqa_prefill_decoder_shape(ortmi, oracle):
    """Prompt of 128 tokens into an empty shared buffer, 12 query / 2 kv heads, base 1e6."""
    _run_gqa(ortmi, oracle, B=1, S=128, H=12, KV=2, hd=128, cap=256, past=0, inplace=True,
             seed=9, base=1e6)


@pytest.mark.parametrize("scale,amp", [(-0.06, 1.0), (0.35, 1.0), (0.09, 3.0)])
def test_gqa_prefill_scale_and_score_range(ortmi, oracle, scale, amp):
    """Prefill tiles with an explicit scale attribute: a negative one (the tile stages Q
    with its sign flipped and scales by the magnitude), and wide score ranges whose
    running maxima grow along the key walk (cached keys scaled up with their position,
    up to 3x): the block maxima then pass the tile's lazy-rescale threshold of 8 log2
    units several times per query. Output within the fp16 tolerance of the oracle at
    the same scale."""
    rng = np.random.default_rng(int(1000 * abs(scale)) + int(amp))
    B, S, H, KV, hd, cap, past = 2, 200, 8, 2, 128, 400, 150
    q, k, v, pk, pv, cos, sin = _gqa_inputs(rng, B, S, H, KV, hd, cap, True, 1e6)
    q = (q.astype(np.float32) * amp).astype(np.float16)
    ramp = (1.0 + 2.0 * np.arange(cap) / cap).astype(np.float32)[None, None, :, None]
    pk = (pk.astype(np.float32) * ramp).astype(np.float16)
    total = past + S
    dpk, dpv = dev(pk), dev(pv)
    out, _, _ = ortmi.group_query_attention(
        dev(q), dev(k), dev(v), dpk, dpv, dev(np.full(B, total - 1, np.int32)), total, dev(cos),
        dev(sin), num_heads=H, kv_num_heads=KV, scale=scale, do_rotary=1, present_key=dpk,
        present_value=dpv)
    ro, _, _, shared = oracle.gqa(q, k, v, pk, pv, total, H, KV, cos=cos, sin=sin, scale=scale,
                                  round16=True)
    assert shared
    assert_f16_close(host(out), ro, what=f"gqa prefill scale {scale} x{amp}")


@pytest.mark.parametrize("scale,amp", [(-0.08, 1.0), (0.1, 3.0)])
def test_paged_prefill_scale_and_score_range(ortmi, oracle, scale, amp):
    """The paged tile body with an explicit scale: negative, and a wide score range
    that moves the lazy reference point several times per walk (as for GQA above).
    Long prefill chunks, so every sequence takes the matrix-core tiles over several
    key blocks."""
    rng = np.random.default_rng(77 + int(amp))
    H, KV, d, blk, batch, maxb = 8, 2, 128, 16, 3, 40
    nb = maxb * batch
    new = np.array([150, 97, 64], np.int32)
    past = np.array([300, 0, 511], np.int32)
    cum = np.concatenate([[0], np.cumsum(new)]).astype(np.int32)
    nt = int(cum[-1])
    q = (rng.standard_normal((nt, H * d)) * amp).astype(np.float16)
    k = rng.standard_normal((nt, KV * d)).astype(np.float16)
    v = rng.standard_normal((nt, KV * d)).astype(np.float16)
    kc = rng.standard_normal((nb, blk, KV, d)).astype(np.float16)
    vc = rng.standard_normal((nb, blk, KV, d)).astype(np.float16)
    bt = rng.permutation(nb).astype(np.int32).reshape(batch, maxb)
    # Cached keys grow with their position in the sequence (up to 3x), so the walk's
    # block maxima keep passing the lazy-rescale threshold.
    for b in range(batch):
        for lb in range(maxb):
            kc[bt[b, lb]] = (kc[bt[b, lb]].astype(np.float32) * (1 + 2 * lb / maxb)).astype(
                np.float16)
    out = ortmi.paged_attention(dev(q), dev(k), dev(v), dev(kc), dev(vc), dev(cum), dev(past),
                                dev(bt), num_heads=H, kv_num_heads=KV, scale=scale)
    ro, _, _ = oracle.paged_attention(q, k, v, kc, vc, cum, past, bt, H, KV, scale=scale,
                                      round16=True)
    assert_f16_close(host(out), ro, what=f"paged prefill scale {scale} x{amp}")


@pytest.mark.parametrize("dt", ["bf16"])
@pytest.mark.parametrize("past", [250, 4])
def test_gqa_decode_dtypes(ortmi, oracle, dt, past):
    """One-token GQA with bf16 tensors (the decode kernel's FMA score path, its
    RoPE on bf16 table entries): within bf16 rounding of the fp32 oracle run on
    the same values. (The op takes fp16 and bf16.)"""
    import torch

    rng = np.random.default_rng(90 + past + len(dt))
    B, H, KV, hd, cap = 2, 8, 2, 128, 300
    tdt = torch.float32 if dt == "f32" else torch.bfloat16
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(tdt)  # noqa: E731
    q = t(rng.standard_normal((B, 1, H * hd)))
    k = t(rng.standard_normal((B, 1, KV * hd)))
    v = t(rng.standard_normal((B, 1, KV * hd)))
    pk = t(rng.standard_normal((B, KV, cap, hd)))
    pv = t(rng.standard_normal((B, KV, cap, hd)))
    c, s_ = refs.rotary_caches(1024, hd, 10000.0)
    cos, sin = t(c), t(s_)
    total = past + 1
    out, prk, prv = ortmi.group_query_attention(
        q.cuda(), k.cuda(), v.cuda(), pk.cuda(), pv.cuda(),
        dev(np.full(B, total - 1, np.int32)), total, cos.cuda(), sin.cuda(), num_heads=H,
        kv_num_heads=KV, do_rotary=1)
    f = lambda x: x.float().numpy()  # noqa: E731
    ro, rk, rv, _ = oracle.gqa(f(q), f(k), f(v), f(pk), f(pv), total, H, KV, cos=f(cos),
                               sin=f(sin))
    got = out.float().cpu().numpy()
    rel = 2.0 ** -22 if dt == "f32" else 2.0 ** -6
    tol = (6e-5 if dt == "f32" else 4e-3) + rel * np.abs(ro)
    assert (np.abs(got - ro) <= tol).all(), f"gqa {dt}: max diff {np.abs(got - ro).max():.3e}"
    gv = prv.float().cpu().numpy()
    np.testing.assert_array_equal(gv[:, :, :total], rv[:, :, :total])


def test_gqa_no_rotary(ortmi, oracle):
    _run_gqa(ortmi, oracle, B=1, S=1, H=8, KV=8, hd=64, cap=40, past=40, rope=False, seed=12)


# ------------------------------------------------------------------ PagedAttention --

def _run_paged(ortmi, oracle, H, KV, d, nb, blk, batch, seed, rope=False, interleaved=0,
               new_max=4, slot_mapping=None, head_sink=None, qk_norm=False, latent=False,
               v_head_size=0, rotary_offset=0):
    rng = np.random.default_rng(seed)
    maxb = nb // batch
    cap = maxb * blk
    new_lens = rng.integers(1, min(new_max, cap) + 1, size=batch).astype(np.int32)
    past = np.array([rng.integers(0, cap - nl + 1) for nl in new_lens], np.int32)
    cum = np.concatenate([[0], np.cumsum(new_lens)]).astype(np.int32)
    nt = int(cum[-1])
    q = (rng.standard_normal((nt, H * d)) * 0.3).astype(np.float16)
    k = (rng.standard_normal((nt, KV * d)) * 0.3).astype(np.float16)
    v = (rng.standard_normal((nt, KV * d)) * 0.3).astype(np.float16)
    kc = (rng.standard_normal((nb, blk, KV, d)) * 0.3).astype(np.float16)
    vc = (rng.standard_normal((nb, blk, KV, d)) * 0.3).astype(np.float16)
    bt = rng.permutation(nb).astype(np.int32).reshape(batch, maxb)
    cos = sin = None
    if rope:
        # With a rotary_offset the rotated dims are [offset, offset + d/2).
        c, s_ = refs.rotary_caches(cap, d // 2 if rotary_offset else d)
        cos, sin = c.astype(np.float16), s_.astype(np.float16)
    if latent:
        v = vc = None
    qw = kw = None
    if qk_norm:
        qw = np.linspace(0.75, 1.25, d).astype(np.float16)
        kw = np.linspace(1.25, 0.75, d).astype(np.float16)
    sm = None if slot_mapping is None else slot_mapping(cum, past, bt, blk)
    dkc = dev(kc)
    dvc = None if latent else dev(vc)
    out = ortmi.paged_attention(
        dev(q), dev(k), None if latent else dev(v), dkc, dvc, dev(cum), dev(past), dev(bt),
        None if cos is None else dev(cos), None if sin is None else dev(sin),
        None if sm is None else dev(sm), None if head_sink is None else dev(head_sink),
        None if qw is None else dev(qw), None if kw is None else dev(kw), num_heads=H,
        kv_num_heads=KV, do_rotary=int(rope), rotary_interleaved=interleaved,
        qk_norm_epsilon=1e-5, kv_cache_layout="LATENT" if latent else "SEPARATE",
        v_head_size=v_head_size, rotary_offset=rotary_offset)
    ro, rkc, rvc = oracle.paged_attention(q, k, v, kc, vc, cum, past, bt, H, KV, cos=cos, sin=sin,
                                          interleaved=interleaved, rotary_offset=rotary_offset,
                                          slot_mapping=sm, head_sink=head_sink, q_norm=qw,
                                          k_norm=kw, qk_eps=1e-5, v_head_size=v_head_size,
                                          round16=True)
    assert out.shape == (int(cum[-1]), H * (v_head_size or d))
    assert_f16_close(host(out), ro, what="paged output")
    gk = host(dkc)
    if not latent:
        np.testing.assert_array_equal(host(dvc), rvc)  # slot writes of V are bit-exact copies
    # K slots: untouched rows bit-exact, written rows within 1 ULP (rounded RoPE/norm).
    assert (np.abs(gk - rkc) <= ulp16(rkc)).all()
    return out


@pytest.mark.parametrize("H,KV", [(4, 2), (4, 4), (8, 2), (2, 1)])
@pytest.mark.parametrize("batch", [1, 3])
def test_paged_core(ortmi, oracle, H, KV, batch):
    _run_paged(ortmi, oracle, H, KV, 64, nb=8 * batch, blk=4, batch=batch, seed=H * 10 + KV + batch)


@pytest.mark.parametrize("blk", [2, 16])
def test_paged_multiblock_long(ortmi, oracle, blk):
    # Long pasts force the split-K path for single-token sequences.
    _run_paged(ortmi, oracle, 8, 2, 128, nb=96 * 2, blk=blk, batch=2, seed=blk + 7, new_max=1)


@pytest.mark.parametrize("interleaved", [0, 1])
def test_paged_rotary(ortmi, oracle, interleaved):
    _run_paged(ortmi, oracle, 4, 2, 64, nb=16, blk=4, batch=2, seed=31 + interleaved, rope=True,
               interleaved=interleaved)


@pytest.mark.parametrize("vhd", [64, 128])
def test_paged_latent_layout(ortmi, oracle, vhd):
    """LATENT cache layout (rust/src/ops/attention.rs:2500-2505, 2624-2628): no value
    input or value cache; values are the first v_head_size dims of each cached key
    (head size 128, v_head_size 64 or 128), with a multi-token chunk and RoPE."""
    _run_paged(ortmi, oracle, 8, 2, 128, nb=24, blk=4, batch=3, seed=300 + vhd, new_max=6,
               rope=True, latent=True, v_head_size=vhd)


@pytest.mark.parametrize("interleaved", [0, 1])
@pytest.mark.parametrize("d,offset", [(64, 16), (128, 8)])
def test_paged_rotary_offset(ortmi, oracle, interleaved, d, offset):
    """rotary_offset (rust/src/ops/attention.rs:2455-2493, 2620): RoPE rotates head
    dims [offset, offset + rotary_dim) and passes the dims before and after through;
    here rotary_dim = head_size / 2."""
    _run_paged(ortmi, oracle, 4, 2, d, nb=16, blk=4, batch=2, seed=41 + interleaved + d,
               rope=True, interleaved=interleaved, new_max=5, rotary_offset=offset)


def test_paged_optional_inputs(ortmi, oracle):
    def slots(cum, past, bt, blk):
        nt = int(cum[-1])
        s = np.full(nt, -1, np.int32)
        for b in range(len(cum) - 1):
            for i in range(cum[b], cum[b + 1]):
                p = past[b] + (i - cum[b])
                s[i] = bt[b, p // blk] * blk + p % blk
        s[0] = -1
        return s
    sink = np.array([-0.5, 0.25, 1.0, -1.0], np.float16)
    _run_paged(ortmi, oracle, 4, 2, 64, nb=8, blk=4, batch=2, seed=129, slot_mapping=slots,
               head_sink=sink, qk_norm=True)


@pytest.mark.parametrize("new_max,nbs", [(5, 8), (1, 96)])
def test_paged_bf16(ortmi, oracle, new_max, nbs):
    """bf16 caches and activations (the VALU tile and the bf16 decode kernel): the
    oracle runs in fp32 on the same bf16 values; outputs within bf16 rounding, V
    slots bit-exact, K slots within one bf16 ulp."""
    import torch

    rng = np.random.default_rng(71 + new_max)
    H, KV, d, blk, batch = 8, 2, 128, 4, 2
    nb = nbs * batch
    maxb = nb // batch
    cap = maxb * blk
    new_lens = rng.integers(1, new_max + 1, size=batch).astype(np.int32)
    past = np.array([rng.integers(0, cap - nl + 1) for nl in new_lens], np.int32)
    cum = np.concatenate([[0], np.cumsum(new_lens)]).astype(np.int32)
    nt = int(cum[-1])
    bf = lambda a: torch.from_numpy((a * 0.3).astype(np.float32)).to(torch.bfloat16)  # noqa: E731
    q, k, v = (bf(rng.standard_normal((nt, n * d))) for n in (H, KV, KV))
    kc, vc = (bf(rng.standard_normal((nb, blk, KV, d))) for _ in range(2))
    bt = rng.permutation(nb).astype(np.int32).reshape(batch, maxb)
    dkc, dvc = kc.cuda(), vc.cuda()
    out = ortmi.paged_attention(q.cuda(), k.cuda(), v.cuda(), dkc, dvc, dev(cum), dev(past),
                                dev(bt), num_heads=H, kv_num_heads=KV)
    f = lambda t: t.float().numpy()  # noqa: E731
    ro, rkc, rvc = oracle.paged_attention(f(q), f(k), f(v), f(kc), f(vc), cum, past, bt, H, KV)
    got = out.float().cpu().numpy()
    assert out.dtype == torch.bfloat16
    tol = 2e-3 + 2.0 ** -7 * np.abs(ro)
    assert (np.abs(got - ro) <= tol).all(), f"paged bf16: max diff {np.abs(got - ro).max():.3e}"
    np.testing.assert_array_equal(dvc.float().cpu().numpy(), rvc)
    gk = dkc.float().cpu().numpy()
    assert (np.abs(gk - rkc) <= 2.0 ** -7 * np.abs(rkc) + 1e-30).all()


def _bf16_tile_tol(ro, vmax):
    """bf16 matrix-core tile bound: the output's bf16 rounding (2^-8 relative, with
    margin 2^-7), fp32 accumulation (2e-3), and P rounded to bf16 once before the
    P V product: each weight moves by at most 2^-9 relative, which moves a weighted
    average of values within [-vmax, vmax] by at most 2^-8 * 2 vmax."""
    return 2e-3 + 2.0 ** -7 * np.abs(ro) + 2.0 ** -7 * vmax


@pytest.mark.parametrize("B,S,H,KV,past,cap,inplace", [
    (1, 512, 12, 2, 0, 640, True),     # the decoder's 512-token prompt
    (2, 300, 32, 8, 200, 600, True),   # a chunk after cached rows, shared buffer
    (1, 96, 8, 2, 40, 40, False),      # growing contract
])
def test_gqa_prefill_bf16_matrix_cores(ortmi, oracle, B, S, H, KV, past, cap, inplace):
    """bf16 GQA prefill on the matrix cores (S^T = K Q^T and O^T += V^T P^T with
    v_mfma_f32_32x32x16_bf16) at the decoder's size, RoPE in the op, against the
    oracle run in fp32 on the same bf16 values with bf16 rounding of the RoPE'd
    rows: outputs within _bf16_tile_tol, cached and new V rows bit-exact, new K rows
    within one bf16 ulp."""
    import torch

    rng = np.random.default_rng(500 + S + past)
    hd = 128
    bf = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16)  # noqa: E731
    q, k, v = (bf(0.5 * rng.standard_normal((B, S, n * hd))) for n in (H, KV, KV))
    pk, pv = (bf(0.5 * rng.standard_normal((B, KV, cap, hd))) for _ in range(2))
    c, s_ = refs.rotary_caches(4096, hd, 1e6)
    cos, sin = bf(c), bf(s_)
    total = past + S
    dpk, dpv = pk.cuda(), pv.cuda()
    kw = dict(present_key=dpk, present_value=dpv) if inplace else {}
    out, prk, prv = ortmi.group_query_attention(
        q.cuda(), k.cuda(), v.cuda(), dpk, dpv, dev(np.full(B, total - 1, np.int32)), total,
        cos.cuda(), sin.cuda(), num_heads=H, kv_num_heads=KV, do_rotary=1, **kw)
    f = lambda x: x.float().numpy()  # noqa: E731
    ro, rk, rv, _ = oracle.gqa(f(q), f(k), f(v), f(pk), f(pv), total, H, KV, cos=f(cos),
                               sin=f(sin), round16=2)
    assert out.dtype == torch.bfloat16
    got = out.float().cpu().numpy()
    tol = _bf16_tile_tol(ro, max(np.abs(f(v)).max(), np.abs(f(pv)).max()))
    assert (np.abs(got - ro) <= tol).all(), f"gqa bf16 prefill: max diff {np.abs(got - ro).max():.3e}"
    gv, gk = prv.float().cpu().numpy(), prk.float().cpu().numpy()
    np.testing.assert_array_equal(gv[:, :, :total], rv[:, :, :total])
    assert (np.abs(gk[:, :, :total] - rk[:, :, :total]) <= _ulp_bf16(rk[:, :, :total])).all()


def test_paged_prefill_bf16_matrix_cores(ortmi, oracle):
    """bf16 PagedAttention at the mixed-batch shape's head layout (H 32, KV 8, head
    128, block 16): four sequences prefill 256-token chunks on the matrix-core tiles
    and eight decode one token, against the oracle in fp32 on the same bf16 values:
    outputs within _bf16_tile_tol, the written cache slots bit-exact."""
    import torch

    rng = np.random.default_rng(77)
    H, KV, d, blk = 32, 8, 128, 16
    new_lens = np.array([256] * 4 + [1] * 8, np.int32)
    batch = len(new_lens)
    past = rng.integers(0, 700, size=batch).astype(np.int32)
    maxb = int((past + new_lens).max() + blk - 1) // blk
    nb = batch * maxb
    cum = np.concatenate([[0], np.cumsum(new_lens)]).astype(np.int32)
    nt = int(cum[-1])
    bf = lambda a: torch.from_numpy((a * 0.5).astype(np.float32)).to(torch.bfloat16)  # noqa: E731
    q, k, v = (bf(rng.standard_normal((nt, n * d))) for n in (H, KV, KV))
    kc, vc = (bf(rng.standard_normal((nb, blk, KV, d))) for _ in range(2))
    bt = rng.permutation(nb).astype(np.int32).reshape(batch, maxb)
    dkc, dvc = kc.cuda(), vc.cuda()
    out = ortmi.paged_attention(q.cuda(), k.cuda(), v.cuda(), dkc, dvc, dev(cum), dev(past),
                                dev(bt), num_heads=H, kv_num_heads=KV)
    f = lambda t: t.float().numpy()  # noqa: E731
    ro, rkc, rvc = oracle.paged_attention(f(q), f(k), f(v), f(kc), f(vc), cum, past, bt, H, KV)
    got = out.float().cpu().numpy()
    assert out.dtype == torch.bfloat16
    tol = _bf16_tile_tol(ro, max(np.abs(f(v)).max(), np.abs(f(vc)).max()))
    assert (np.abs(got - ro) <= tol).all(), f"paged bf16: max diff {np.abs(got - ro).max():.3e}"
    np.testing.assert_array_equal(dvc.float().cpu().numpy(), rvc)
    np.testing.assert_array_equal(dkc.float().cpu().numpy(), rkc)


def test_paged_mixed_batch_reduced(ortmi, oracle):
    """Mixed prefill + decode: 2 sequences prefill 40-token chunks, 6 decode one token,
    block 16, 32/8 heads, hd 128 (a reduced form of the mixed-batch config)."""
    rng = np.random.default_rng(55)
    H, KV, d, blk = 32, 8, 128, 16
    ctx = rng.integers(64, 700, size=8)
    new = np.array([40, 40, 1, 1, 1, 1, 1, 1])
    past = (ctx - new).astype(np.int32)
    nblocks = [int((c + blk - 1) // blk) for c in ctx]
    nb = sum(nblocks)
    maxb = max(nblocks)
    perm = rng.permutation(nb).astype(np.int32)
    bt = np.zeros((8, maxb), np.int32)
    o = 0
    for b, n in enumerate(nblocks):
        bt[b, :n] = perm[o:o + n]
        o += n
    cum = np.concatenate([[0], np.cumsum(new)]).astype(np.int32)
    nt = int(cum[-1])
    q = rng.standard_normal((nt, H * d)).astype(np.float16)
    k = rng.standard_normal((nt, KV * d)).astype(np.float16)
    v = rng.standard_normal((nt, KV * d)).astype(np.float16)
    kc = rng.standard_normal((nb, blk, KV, d)).astype(np.float16)
    vc = rng.standard_normal((nb, blk, KV, d)).astype(np.float16)
    dkc, dvc = dev(kc), dev(vc)
    out = ortmi.paged_attention(dev(q), dev(k), dev(v), dkc, dvc, dev(cum), dev(past), dev(bt),
                                num_heads=H, kv_num_heads=KV)
    ro, rkc, rvc = oracle.paged_attention(q, k, v, kc, vc, cum, past, bt, H, KV, round16=True)
    assert_f16_close(host(out), ro, what="paged mixed")
    np.testing.assert_array_equal(host(dkc), rkc)
    np.testing.assert_array_equal(host(dvc), rvc)


def test_paged_mixed_batch_full_size(ortmi, oracle):
    """The benchmarked mixed batch at full size: 32 sequences with contexts U[256, 8192],
    4 prefill 256-token chunks and 28 one-token decodes, block 16, 32/8 heads, hd 128
    (block tables of up to 512 entries, prefill tiles crossing the causal diagonal,
    8K-context split counts). Every written K/V slot is bit-exact and every output row
    of all 32 sequences is within the fp16 tolerance."""
    import importlib

    wl = importlib.import_module(ortmi.__name__ + ".workloads")
    cfg = wl.paged_mixed_config()
    print(f"cfg5: ctx {cfg['ctx'].min()}..{cfg['ctx'].max()}, tokens {int(cfg['cum'][-1])}, "
          f"blocks {cfg['kc'].shape[0]}, max table {cfg['bt'].shape[1]}", flush=True)
    dkc, dvc = dev(cfg["kc"]), dev(cfg["vc"])
    out = ortmi.paged_attention(dev(cfg["q"]), dev(cfg["k"]), dev(cfg["v"]), dkc, dvc,
                                dev(cfg["cum"]), dev(cfg["past"]), dev(cfg["bt"]),
                                num_heads=cfg["H"], kv_num_heads=cfg["KV"])
    got, gk, gv = host(out), host(dkc), host(dvc)
    ro, rkc, rvc = oracle.paged_attention(cfg["q"], cfg["k"], cfg["v"], cfg["kc"], cfg["vc"],
                                          cfg["cum"], cfg["past"], cfg["bt"], cfg["H"], cfg["KV"],
                                          round16=True)
    np.testing.assert_array_equal(gk, rkc)
    np.testing.assert_array_equal(gv, rvc)
    cum = cfg["cum"]
    for b in range(len(cum) - 1):
        assert_f16_close(got[cum[b]:cum[b + 1]], ro[cum[b]:cum[b + 1]],
                         what=f"cfg5 sequence {b} (ctx {cfg['ctx'][b]}, new {cfg['new'][b]})")


# ---------------------------------------------------------------- RotaryEmbedding --

@pytest.mark.parametrize("form", ["bsnd_ids", "bsnd_offset", "bnsd_ids", "per_token"])
@pytest.mark.parametrize("interleaved", [0, 1])
def test_rotary_embedding(ortmi, oracle, form, interleaved):
    import torch

    rng = np.random.default_rng(["bsnd_ids", "bsnd_offset", "bnsd_ids", "per_token"].index(form)
                                * 10 + interleaved)
    B, S, NH, hd = 2, 7, 4, 64
    c, s_ = refs.rotary_caches(64, hd)
    cos, sin = c.astype(np.float16), s_.astype(np.float16)
    x = rng.standard_normal((B, S, NH * hd)).astype(np.float16)
    if form == "bsnd_offset":
        pos = np.array([5], np.int64)
        rows = np.broadcast_to(5 + np.arange(S), (B, S))
    elif form == "per_token":
        pos = None
        rows = np.arange(B * S).reshape(B, S)
        cos = cos[:B * S].reshape(B, S, hd // 2)
        sin = sin[:B * S].reshape(B, S, hd // 2)
    else:
        pos = rng.integers(0, 64, size=(B, S)).astype(np.int64)
        rows = pos
    xin = x
    if form == "bnsd_ids":
        xin = x.reshape(B, S, NH, hd).transpose(0, 2, 1, 3).copy()
    y = ortmi.rotary_embedding(dev(xin), None if pos is None else dev(pos), dev(cos), dev(sin),
                               interleaved=interleaved, num_heads=NH)
    ref = oracle.rotary(x, rows, cos.reshape(-1, hd // 2), sin.reshape(-1, hd // 2),
                        interleaved=bool(interleaved), num_heads=NH, round16=True)
    got = host(y)
    if form == "bnsd_ids":
        got = got.transpose(0, 2, 1, 3).reshape(B, S, NH * hd)
    assert (np.abs(got - ref) <= ulp16(ref)).all()
    assert y.dtype == torch.float16


def _ulp_bf16(x):
    x = np.abs(np.asarray(x, np.float64))
    return 2.0 ** (np.floor(np.log2(np.maximum(x, 2.0 ** -126))) - 7)


def rotary_case(dt, rng, shape, max_pos, hd, half):
    """Inputs of one RotaryEmbedding case in dtype `dt` ("f16", "bf16", "f32"): the
    device tensors (x, cos, sin), their float32 values (what the oracle rotates),
    the oracle's rounding mode and a tolerance function of the exact result."""
    import torch

    tdt = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}[dt]
    c, s_ = refs.rotary_caches(max_pos, 2 * half, 10000.0)
    xs = torch.from_numpy(rng.standard_normal(shape).astype(np.float32)).to(tdt)
    cs, sn = torch.from_numpy(c.astype(np.float32)).to(tdt), torch.from_numpy(s_.astype(np.float32)).to(tdt)
    vals = [t.float().numpy() for t in (xs, cs, sn)]
    mode = {"f16": 1, "bf16": 2, "f32": 0}[dt]
    tol = {"f16": lambda r: ulp16(r), "bf16": _ulp_bf16,
           "f32": lambda r: 1e-6 + 1e-6 * np.abs(r)}[dt]
    return [t.cuda() for t in (xs, cs, sn)], vals, mode, tol


@pytest.mark.parametrize("dt", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("half,interleaved,layout", [
    (16, 0, "bsnd"), (16, 1, "bsnd"), (24, 0, "bnsd"), (32, 1, "bnsd"), (32, 0, "bsnd")])
def test_rotary_embedding_dtypes_partial(ortmi, oracle, dt, half, interleaved, layout):
    """Standalone RotaryEmbedding in fp16, bf16 and fp32, with partial rotary (a
    cos/sin cache narrower than head_size / 2: only dims [0, 2 * half) rotate, the
    tail keeps its values bit for bit, rust/src/ops/attention.rs:1234-1282) and
    full rotary, both pair layouts and both tensor layouts, against the oracle on
    the same rounded inputs (one rounding of the rotated value to the dtype)."""
    rng = np.random.default_rng(half * 10 + interleaved + 3 * ("f16", "bf16", "f32").index(dt))
    B, S, NH, hd, max_pos = 2, 9, 4, 64, 96
    shape = (B, S, NH * hd) if layout == "bsnd" else (B, NH, S, hd)
    (dx, dc, ds), (x, c, s_), mode, tol = rotary_case(dt, rng, shape, max_pos, hd, half)
    pos = rng.integers(0, max_pos, size=(B, S)).astype(np.int64)
    y = ortmi.rotary_embedding(dx, dev(pos), dc, ds, interleaved=interleaved,
                               num_heads=NH if layout == "bsnd" else 0)
    ref = oracle.rotary(x, pos, c, s_, interleaved=bool(interleaved), round16=mode,
                        layout=layout, num_heads=NH if layout == "bsnd" else None)
    got = host(y)
    assert y.dtype == dx.dtype
    assert (np.abs(got - ref) <= tol(ref)).all(), f"max diff {np.abs(got - ref).max():.3e}"
    if layout == "bsnd":
        g4, x4 = got.reshape(B, S, NH, hd), x.reshape(B, S, NH, hd)
    else:
        g4, x4 = got, x
    np.testing.assert_array_equal(g4[..., 2 * half:], x4[..., 2 * half:])


# ------------------------------------------------------------ (Skip)SimplifiedLN --

@pytest.mark.parametrize("dtype", [np.float32, np.float16])
@pytest.mark.parametrize("skip", [False, True])
def test_rms_norm(ortmi, oracle, dtype, skip):
    rng = np.random.default_rng(int(skip) + (dtype == np.float16))
    x = rng.standard_normal((9, 1536)).astype(dtype)
    sk = rng.standard_normal((9, 1536)).astype(dtype)
    g = rng.standard_normal(1536).astype(dtype)
    r16 = dtype == np.float16
    if skip:
        y, r = ortmi.skip_simplified_layer_norm(dev(x), dev(sk), dev(g), epsilon=1e-6)
        ry, rr = oracle.rms_norm(x, g, 1e-6, skip=sk, round16=r16)
        np.testing.assert_array_equal(host(r), rr)  # residual: one rounding of x + skip
    else:
        y = ortmi.simplified_layer_norm(dev(x), dev(g), epsilon=1e-5)
        ry, _ = oracle.rms_norm(x, g, 1e-5, round16=r16)
    if r16:
        assert_f16_close(host(y), ry, what="rms fp16")
    else:
        assert np.abs(host(y) - ry).max() <= 6e-5


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_skip_rms_norm_bias(ortmi, oracle, dtype):
    """SkipSimplifiedLayerNormalization with its optional bias input ([D], the same for
    every row): the residual output is x + skip + bias rounded once to the dtype
    (bit-exact against the oracle), the normalised output within the dtype's bar; and
    a zero bias gives exactly the bias-free results."""
    rng = np.random.default_rng(31 + (dtype == np.float16))
    rows, D = 7, 1536
    x = rng.standard_normal((rows, D)).astype(dtype)
    sk = rng.standard_normal((rows, D)).astype(dtype)
    b = rng.standard_normal(D).astype(dtype)
    g = rng.standard_normal(D).astype(dtype)
    r16 = dtype == np.float16
    y, r = ortmi.skip_simplified_layer_norm(dev(x), dev(sk), dev(g), dev(b), epsilon=1e-6)
    ry, rr = oracle.rms_norm(x, g, 1e-6, skip=sk, bias=b, round16=r16)
    np.testing.assert_array_equal(host(r), rr)
    if r16:
        assert_f16_close(host(y), ry, what="skip rms + bias fp16")
    else:
        assert np.abs(host(y) - ry).max() <= 6e-5
    y0, r0 = ortmi.skip_simplified_layer_norm(dev(x), dev(sk), dev(g), dev(np.zeros_like(b)),
                                              epsilon=1e-6)
    y1, r1 = ortmi.skip_simplified_layer_norm(dev(x), dev(sk), dev(g), epsilon=1e-6)
    np.testing.assert_array_equal(host(r0), host(r1))
    np.testing.assert_array_equal(host(y0), host(y1))


# ------------------------------------------------------------------------- glue --

def test_glue_kernels(ortmi):
    import ctypes

    import torch

    lib = ortmi.load_kernels()
    rng = np.random.default_rng(77)
    g = rng.standard_normal(5000).astype(np.float16)
    u = rng.standard_normal(5000).astype(np.float16)
    dg, du = dev(g), dev(u)
    out = torch.empty_like(dg)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    ortmi.check(lib.ortmi_swiglu(ctypes.c_void_p(dg.data_ptr()), ctypes.c_void_p(du.data_ptr()),
                                 ctypes.c_void_p(out.data_ptr()), 5000, 10, st))
    g32 = g.astype(np.float32)
    sig = (1.0 / (1.0 + np.exp(-g32.astype(np.float64)))).astype(np.float16).astype(np.float32)
    t = (g32 * sig).astype(np.float16).astype(np.float32)
    ref = (t * u.astype(np.float32)).astype(np.float16).astype(np.float32)
    assert (np.abs(host(out) - ref) <= ulp16(ref)).all()
    # argmax: first index on ties, one-pass and two-pass (the tie straddles partials)
    x = rng.standard_normal((3, 151936)).astype(np.float16)
    x[1, 17] = x[1, 99] = 100.0
    x[2, 4000] = x[2, 151935] = 100.0
    idx = torch.empty(3, dtype=torch.int64, device="cuda")
    dx = dev(x)
    wsz = lib.ortmi_argmax_rows_workspace_size(3, 151936)
    ws = torch.empty(wsz, dtype=torch.uint8, device="cuda")
    for w, wb in ((None, 0), (ctypes.c_void_p(ws.data_ptr()), wsz)):
        idx.fill_(-5)
        ortmi.check(lib.ortmi_argmax_rows(ctypes.c_void_p(dx.data_ptr()),
                                          ctypes.c_void_p(idx.data_ptr()), 3, 151936, 10, w, wb,
                                          st))
        np.testing.assert_array_equal(host(idx), np.argmax(x.astype(np.float32), axis=1))
    # the same rows in fp32, fp16 rows of 200000 columns with NaNs that never win, and
    # rows of 4099 columns (not whole 16-byte vectors: the element-wise partial pass)
    odd = rng.standard_normal((2, 4099)).astype(np.float16)
    odd[0, 4098] = odd[1, 2048] = 30.0
    for xs, dt in ((x.astype(np.float32), 1), (None, 10), (odd, 10)):
        if xs is None:
            xs = rng.standard_normal((2, 200000)).astype(np.float16)
            xs[0, 199999] = 50.0
            xs[1, 5] = np.nan
            xs[1, 199990] = xs[1, 196610] = 60.0
        r = xs.shape[0]
        wsz2 = lib.ortmi_argmax_rows_workspace_size(r, xs.shape[1])
        ws2 = torch.empty(max(wsz2, 1), dtype=torch.uint8, device="cuda")
        i2 = torch.full((r,), -5, dtype=torch.int64, device="cuda")
        dxs = dev(xs)
        ortmi.check(lib.ortmi_argmax_rows(ctypes.c_void_p(dxs.data_ptr()),
                                          ctypes.c_void_p(i2.data_ptr()), r, xs.shape[1], dt,
                                          ctypes.c_void_p(ws2.data_ptr()), wsz2, st))
        expect = np.argmax(np.where(np.isnan(xs), -np.inf, xs.astype(np.float32)), axis=1)
        np.testing.assert_array_equal(host(i2), expect)
    # gather rows with a negative id
    table = rng.standard_normal((100, 64)).astype(np.float16)
    ids = np.array([3, -1, 50], np.int64)
    dt_, di = dev(table), dev(ids)
    o = torch.empty((3, 64), dtype=torch.float16, device="cuda")
    ortmi.check(lib.ortmi_gather_rows(ctypes.c_void_p(dt_.data_ptr()), ctypes.c_void_p(di.data_ptr()),
                                      ctypes.c_void_p(o.data_ptr()), 3, 100, 64, 10, st))
    np.testing.assert_array_equal(host(o), table[[3, 99, 50]].astype(np.float32))


# ------------------------------------------------------ PagedAttention, generic ---


def _run_paged_generic(ortmi, oracle, dt, H, KV, d, nb, blk, batch, seed, rope=False,
                       interleaved=0, new_max=4, latent=False, v_head_size=0, rotary_offset=0,
                       head_sink=False, qk_norm=False):
    """The forms the generic kernels serve (fp32, head sizes other than 64/128, LATENT
    value sizes other than 64/128, odd rotary offsets) against the oracle on the same
    rounded inputs. Tolerances: fp32 1e-5 + 1e-5 |exact|, fp16 1e-3 + 2 ULP, bf16
    4e-3 + 2^-6 |exact|; V slots exact, K slots within one rounding of the oracle."""
    import torch

    tdt = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}[dt]

    def cast(a):
        t = torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(tdt)
        return t.cuda(), t.float().numpy()

    rng = np.random.default_rng(seed)
    maxb = nb // batch
    cap = maxb * blk
    new_lens = rng.integers(1, min(new_max, cap) + 1, size=batch).astype(np.int32)
    past = np.array([rng.integers(0, cap - nl + 1) for nl in new_lens], np.int32)
    cum = np.concatenate([[0], np.cumsum(new_lens)]).astype(np.int32)
    nt = int(cum[-1])
    vd = v_head_size or d
    q, nq = cast(rng.standard_normal((nt, H * d)) * 0.3)
    k, nk = cast(rng.standard_normal((nt, KV * d)) * 0.3)
    v, nv = cast(rng.standard_normal((nt, KV * d)) * 0.3)
    kc, nkc = cast(rng.standard_normal((nb, blk, KV, d)) * 0.3)
    vc, nvc = cast(rng.standard_normal((nb, blk, KV, d)) * 0.3)
    bt = rng.permutation(nb).astype(np.int32).reshape(batch, maxb)
    cos = sin = ncos = nsin = None
    if rope:
        c, s_ = refs.rotary_caches(cap, d // 2 if rotary_offset else d)
        cos, ncos = cast(c)
        sin, nsin = cast(s_)
    if latent:
        v = vc = nv = nvc = None
    sink = nsink = qw = nqw = kw = nkw = None
    if head_sink:
        sink, nsink = cast(rng.uniform(-1, 1, H))
    if qk_norm:
        qw, nqw = cast(np.linspace(0.75, 1.25, d))
        kw, nkw = cast(np.linspace(1.25, 0.75, d))
    out = ortmi.paged_attention(
        q, k, v, kc, vc, dev(cum), dev(past), dev(bt), cos, sin, None, sink, qw, kw,
        num_heads=H, kv_num_heads=KV, do_rotary=int(rope), rotary_interleaved=interleaved,
        qk_norm_epsilon=1e-5, kv_cache_layout="LATENT" if latent else "SEPARATE",
        v_head_size=v_head_size, rotary_offset=rotary_offset)
    torch.cuda.synchronize()
    r16 = {"f32": 0, "f16": 1, "bf16": 2}[dt]
    ro, rkc, rvc = oracle.paged_attention(nq, nk, nv, nkc, nvc, cum, past, bt, H, KV, cos=ncos,
                                          sin=nsin, interleaved=interleaved,
                                          rotary_offset=rotary_offset, head_sink=nsink,
                                          q_norm=nqw, k_norm=nkw, qk_eps=1e-5,
                                          v_head_size=v_head_size, round16=r16)
    got = out.float().cpu().numpy()
    assert got.shape == (nt, H * vd) and out.dtype == tdt
    if dt == "f32":
        tol = 1e-5 + 1e-5 * np.abs(ro)
    elif dt == "f16":
        tol = 1e-3 + 2 * ulp16(ro)
    else:
        tol = 4e-3 + 2.0 ** -6 * np.abs(ro)
    bad = ~(np.abs(got - ro) <= tol)
    assert not bad.any(), (f"{dt} paged output: {bad.sum()} of {bad.size} beyond tolerance, "
                           f"max diff {np.nanmax(np.abs(got - ro)):.3e}")
    if not latent:
        np.testing.assert_array_equal(vc.float().cpu().numpy(), rvc)
    gk = kc.float().cpu().numpy()
    mant = {"f32": 23, "f16": 10, "bf16": 7}[dt]
    ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(rkc), 2.0 ** -24))) - mant)
    assert (np.abs(gk - rkc) <= (2 if qk_norm else 1) * ulp + (1e-6 if dt == "f32" else 0)).all()


@pytest.mark.parametrize("rope,interleaved", [(False, 0), (True, 0), (True, 1)])
def test_paged_generic_fp32(ortmi, oracle, rope, interleaved):
    _run_paged_generic(ortmi, oracle, "f32", 8, 2, 128, nb=24, blk=4, batch=3, seed=500 + rope,
                       rope=rope, interleaved=interleaved, new_max=6)


@pytest.mark.parametrize("dt,d", [("f16", 96), ("bf16", 256), ("f16", 32)])
def test_paged_generic_head_sizes(ortmi, oracle, dt, d):
    _run_paged_generic(ortmi, oracle, dt, 4, 2, d, nb=16, blk=4, batch=2, seed=510 + d,
                       rope=True, new_max=5, head_sink=True, qk_norm=True)


def test_paged_generic_latent_and_offset(ortmi, oracle):
    """LATENT with v_head_size 96 of head 128, and a rotary_offset of 4 (fp16)."""
    _run_paged_generic(ortmi, oracle, "f16", 8, 1, 128, nb=24, blk=4, batch=3, seed=520,
                       rope=True, new_max=6, latent=True, v_head_size=96)
    _run_paged_generic(ortmi, oracle, "f16", 4, 2, 64, nb=16, blk=4, batch=2, seed=521,
                       rope=True, interleaved=1, new_max=5, rotary_offset=4)


@pytest.mark.parametrize("path", ["fused", "generic"])
def test_paged_attention_malformed_control_tensors(ortmi, oracle, path):
    """Malformed control tensors stay in bounds and read as clamped: a negative first
    cum_seqlens entry is the sequence start 0 (outputs and caches bit-identical to
    cum_seqlens[0] = 0); a past length of 2^31 - 1 reads as max_context (identical to
    past = max_context: every key from the cache, none beyond max_context); unsorted
    cum_seqlens with negative and huge past lengths and out-of-range block ids
    complete, and a well-formed call on the same buffers afterwards equals the
    oracle. path: fp16 head 128 (the tile and single-token kernels) or fp32 head 64
    (the generic kernel)."""
    import torch

    dtype, d = (np.float16, 128) if path == "fused" else (np.float32, 64)
    rng = np.random.default_rng(5 if path == "fused" else 6)
    H, KV, blk, batch, maxb = 4, 2, 16, 3, 4
    nb = batch * maxb
    max_ctx = maxb * blk
    T = 6
    kc0 = rng.standard_normal((nb, blk, KV, d)).astype(dtype)
    vc0 = rng.standard_normal((nb, blk, KV, d)).astype(dtype)
    bt = rng.permutation(nb).astype(np.int32).reshape(batch, maxb)
    q, k, v = (rng.standard_normal((T, n * d)).astype(dtype) for n in (H, KV, KV))
    i32 = lambda a: dev(np.asarray(a, np.int32))  # noqa: E731

    def call(cum, past, table=bt):
        kc, vc = dev(kc0), dev(vc0)
        o = ortmi.paged_attention(dev(q), dev(k), dev(v), kc, vc, i32(cum), i32(past), i32(table),
                                  num_heads=H, kv_num_heads=KV)
        torch.cuda.synchronize()
        return host(o), host(kc), host(vc)

    def same(a, b):
        for x, y in zip(a, b):
            np.testing.assert_array_equal(x, y)

    ok = call([0, 3, 4, 6], [5, 20, 0])
    same(call([-6, 3, 4, 6], [5, 20, 0]), ok)
    same(call([0, 3, 4, 6], [5, 2 ** 31 - 1, 0]), call([0, 3, 4, 6], [5, max_ctx, 0]))
    bad_bt = bt.copy()
    bad_bt[0, 1], bad_bt[2, 0] = -1, nb + 5
    call([0, 5, 2, 6], [-3, 5, 99999], bad_bt)
    call([3, -2 ** 31, 2 ** 31 - 1, 1], [2 ** 31 - 1, -1, 7], bad_bt)
    got = call([0, 3, 4, 6], [5, 20, 0])
    same(got, ok)
    ro, rk, rv = oracle.paged_attention(q, k, v, kc0.astype(np.float32), vc0.astype(np.float32),
                                        np.array([0, 3, 4, 6], np.int32),
                                        np.array([5, 20, 0], np.int32), bt, H, KV)
    if dtype == np.float16:
        assert_f16_close(got[0], ro, what="paged after malformed calls")
        np.testing.assert_array_equal(got[1], oracle.round_f16(rk))
    else:
        assert np.abs(got[0] - ro).max() <= 6e-5
        np.testing.assert_array_equal(got[1], rk)


def test_copy_small_h2d(ortmi):
    """ortmi_copy_small_h2d (the data transfer's one-launch path for a run's small
    feeds): every byte of up to 16 host buffers (pageable numpy memory, 1024 bytes in
    all) lands at its device destination, at any offset and alignment, bit-exact;
    zero-length copies and bytes around the destinations are left alone; more than 16
    copies or 1024 bytes are rejected before anything is launched."""
    import ctypes

    import torch

    lib = ortmi.load_kernels()
    rng = np.random.default_rng(91)
    sizes = [8, 4, 4, 0, 37, 1, 200, 3, 16, 90, 64, 2, 5, 8, 7, 574]
    assert sum(sizes) == 1023
    srcs = [rng.integers(0, 256, size=n, dtype=np.uint8) for n in sizes]
    buf = torch.full((4096,), 0xA5, dtype=torch.uint8, device="cuda")
    offs, o = [], 3
    for n in sizes:
        offs.append(o)
        o += n + 5  # a gap of untouched bytes after each destination
    base = buf.data_ptr()
    n = len(sizes)
    dst = (ctypes.c_void_p * n)(*[base + x for x in offs])
    src = (ctypes.c_void_p * n)(*[s.ctypes.data if len(s) else None for s in srcs])
    nb = (ctypes.c_size_t * n)(*sizes)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert lib.ortmi_copy_small_h2d(n, dst, src, nb, st) == 0
    got = host(buf)
    want = np.full(4096, 0xA5, np.uint8)
    for x, s in zip(offs, srcs):
        want[x:x + len(s)] = s
    np.testing.assert_array_equal(got, want)
    assert lib.ortmi_copy_small_h2d(0, None, None, None, st) == 0
    big = (ctypes.c_size_t * n)(*(sizes[:-1] + [sizes[-1] + 2]))  # 1025 bytes
    assert lib.ortmi_copy_small_h2d(n, dst, src, big, st) == 1
    assert b"1024" in lib.ortmi_last_error()
    d17 = (ctypes.c_void_p * 17)(*([base] * 17))
    s17 = (ctypes.c_void_p * 17)(*([srcs[0].ctypes.data] * 17))
    n17 = (ctypes.c_size_t * 17)(*([1] * 17))
    assert lib.ortmi_copy_small_h2d(17, d17, s17, n17, st) == 1
    np.testing.assert_array_equal(host(buf), want)
