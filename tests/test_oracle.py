"""Pin the C oracle (oracle/oracle.c) before it is trusted as the parity target.

Each check is chosen so that a plausible mistake in the oracle (nibble order, zero
point column, block index, sign of the rotation, GQA head mapping, causal offset,
cache slot arithmetic) fails it: closed forms, known-answer data from the
reference's own tests, and independent numpy restatements of the reference
tests' numpy references (tests/refs.py). CPU only.
"""

from __future__ import annotations

import json
import os

import numpy as np
import pytest
import refs

# --------------------------------------------------------------------- fp16 ---


def test_f16_conversions_match_ieee(oracle):
    bits = np.arange(65536, dtype=np.uint16)
    f = oracle.f16_bits_to_f32(bits)
    ref = bits.view(np.float16).astype(np.float32)
    same = (f.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(f) & np.isnan(ref))
    assert same.all()
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(200_000) * np.exp(rng.uniform(-25, 12, 200_000))).astype(np.float32)
    edge = np.array([65504, 65519.99, 65520, 2.0**-24, 2.0**-25, 3 * 2.0**-26, -0.0, np.inf],
                    np.float32)
    x = np.concatenate([x, edge])
    with np.errstate(over="ignore"):
        assert (oracle.f32_to_f16_bits(x) == x.astype(np.float16).view(np.uint16)).all()


# -------------------------------------------------------------- MatMulNBits ---


def _gbq_fixture():
    """Known-answer case of tests/ops/_models.py:558-580 as committed in
    tests/golden/gbq_kat.json (packed bytes, scales, indices and the expected
    gathered rows written from the definition of the codes)."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "gbq_kat.json")
    with open(path) as f:
        kat = json.load(f)
    return (np.array(kat["data_uint8"], np.uint8), np.array(kat["scales_f32"], np.float32),
            np.array(kat["indices_int64"], np.int64), np.array(kat["expected_f32"], np.float32))


def test_mnb_dequant_known_answer(oracle):
    qdata, scales, indices, expected = _gbq_fixture()
    W = oracle.mnb_dequant(qdata, scales, None, N=2, K=32, bits=4, block=16)
    # GatherBlockQuantized gathers rows [1, -2] -> [1, 0] of the dequantised table.
    np.testing.assert_array_equal(W[indices % 2], expected)
    # A nibble-order mistake would not pass: swapping nibbles changes the table.
    swapped = ((qdata & 0x0F) << 4) | (qdata >> 4)
    assert not np.array_equal(oracle.mnb_dequant(swapped, scales, None, 2, 32, 4, 16)[indices % 2],
                              expected)


def test_gather_block_quantized_known_answer(oracle):
    """The oracle's GatherBlockQuantized on the reference's known-answer case, bit
    for bit, plus its index rules: a negative id counts from the end, an id out of
    range gives a zero row, zero points 8 equal the symmetric form."""
    qdata, scales, indices, expected = _gbq_fixture()
    np.testing.assert_array_equal(oracle.gather_block_quantized(qdata, scales, None, indices, 16),
                                  expected)
    zp8 = np.full((2, 1), 0x88, np.uint8)
    np.testing.assert_array_equal(oracle.gather_block_quantized(qdata, scales, zp8, indices, 16),
                                  expected)
    got = oracle.gather_block_quantized(qdata, scales, None, np.array([[0, 5], [-1, -3]]), 16)
    assert got.shape == (2, 2, 32)
    np.testing.assert_array_equal(got[0, 0], expected[1])  # row 0 is the KAT's second row
    np.testing.assert_array_equal(got[1, 0], expected[0])  # -1 -> row 1
    assert not got[0, 1].any() and not got[1, 1].any()     # 5 and -3 are out of range


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("block", [16, 32, 64, 128])
@pytest.mark.parametrize("asym", [False, True])
def test_mnb_dequant_matches_numpy_unpack(oracle, bits, block, asym):
    rng = np.random.default_rng(bits * 1000 + block + asym)
    N, K = 5, block * 3 - (7 if block > 16 else 0)  # includes a partial final block
    nb = (K + block - 1) // block
    q = rng.integers(0, 1 << bits, size=(N, nb, block), dtype=np.uint8)
    B = oracle.pack_nibbles(q) if bits == 4 else q
    s = (rng.standard_normal(N * nb) * 0.05).astype(np.float32)
    zp = None
    if asym:
        zp = oracle.pack_zero_points(rng.integers(0, 1 << bits, size=(N, nb), dtype=np.uint8), bits)
    W = oracle.mnb_dequant(B, s, zp, N, K, bits, block)
    np.testing.assert_array_equal(W, refs.dequant_ref(B, s, zp, N, K, bits, block).astype(np.float32))


def test_mnb_special_cases(oracle):
    rng = np.random.default_rng(7)
    N, K, bs = 6, 96, 32
    nb = K // bs
    q = rng.integers(0, 16, size=(N, nb, bs), dtype=np.uint8)
    B = oracle.pack_nibbles(q)
    s = np.abs(rng.standard_normal(N * nb)).astype(np.float32) + 0.1
    # All-8 zero points are the symmetric form (config-1 zero points are all 0x88).
    zp8 = np.full(N * ((nb + 1) // 2), 0x88, np.uint8)
    A = rng.standard_normal((3, K)).astype(np.float32)
    np.testing.assert_array_equal(oracle.mnb_matmul(A, B, s, zp8, N, K),
                                  oracle.mnb_matmul(A, B, s, None, N, K))
    # Codes equal to their zero point dequantise to exactly zero.
    zq = oracle.pack_zero_points(q[:, :, 0], 4)
    q_eq = np.repeat(q[:, :, :1], bs, axis=2)
    assert not oracle.mnb_matmul(A, oracle.pack_nibbles(q_eq), s, zq, N, K).any()
    # A one-hot activation row selects one dequantised column.
    W = refs.dequant_ref(B, s, None, N, K, 4, bs)
    for k in (0, 31, 32, 95):
        e = np.zeros((1, K), np.float32)
        e[0, k] = 1
        np.testing.assert_array_equal(oracle.mnb_matmul(e, B, s, None, N, K)[0], W[:, k])


@pytest.mark.parametrize("M", [1, 8])
@pytest.mark.parametrize("K,block", [(128, 32), (1176, 32), (192, 64), (384, 128), (48, 16)])
def test_mnb_matmul_matches_fp64_gemm(oracle, M, K, block):
    rng = np.random.default_rng(M * 7 + K)
    N = 33
    nb = (K + block - 1) // block
    B = oracle.pack_nibbles(rng.integers(0, 16, size=(N, nb, block), dtype=np.uint8))
    s = (rng.standard_normal(N * nb) * 0.05).astype(np.float32)
    zp = oracle.pack_zero_points(rng.integers(0, 16, size=(N, nb), dtype=np.uint8), 4)
    A = rng.standard_normal((M, K)).astype(np.float32)
    Y = oracle.mnb_matmul(A, B, s, zp, N, K, 4, block)
    ref = A.astype(np.float64) @ refs.dequant_ref(B, s, zp, N, K, 4, block).T
    np.testing.assert_allclose(Y, ref, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("K,block,asym,f16", [(4096, 32, True, False), (1536, 32, False, True),
                                              (8960, 32, True, True), (1024, 64, True, False),
                                              (2048, 128, False, False)])
def test_mnb_matmul_fast_matches_fp64(oracle, K, block, asym, f16):
    """The CPU baseline's fp32 AVX2 GEMV against the fp64 restatement, within an
    fp32 accumulation bound: the kernel sums a*q and a*z per block before subtracting,
    so its error is bounded by 2^-20 * sum_k |a_k| (q_k + z) s < 2^-15 * sum_k |a_k| s
    per row (sums of <= 8960 terms), for fp32 and fp16 scales, with and without zero
    points. A swapped nibble order fails by orders of magnitude more."""
    try:
        probe = oracle.mnb_matmul_fast(np.zeros(32, np.float32), np.zeros((1, 1, 16), np.uint8),
                                       np.ones(1, np.float32), None, 1, 32, 32)
    except ValueError:
        pytest.skip("no AVX2/FMA on this CPU")
    assert probe[0] == 0
    rng = np.random.default_rng(K + block)
    N, nb = 97, K // block
    B = oracle.pack_nibbles(rng.integers(0, 16, size=(N, nb, block), dtype=np.uint8))
    s = (np.abs(rng.standard_normal(N * nb)) * 0.02 + 1e-3).astype(np.float16 if f16 else np.float32)
    zp = (oracle.pack_zero_points(rng.integers(0, 16, size=(N, nb), dtype=np.uint8), 4)
          if asym else None)
    a = rng.standard_normal(K).astype(np.float32)
    y = oracle.mnb_matmul_fast(a, B, s, zp, N, K, block)
    s32 = s.astype(np.float32)
    ref = oracle.mnb_matmul(a[None], B, s32, zp, N, K, 4, block)[0]
    abs_blocks = np.abs(a.astype(np.float64)).reshape(nb, block).sum(axis=1)
    bound = 2.0 ** -15 * (s32.astype(np.float64).reshape(N, nb) @ abs_blocks)
    assert (np.abs(y - ref) <= bound).all(), float(np.max(np.abs(y - ref) / bound))
    # The bound is far below the error of a swapped nibble order.
    swapped = oracle.mnb_matmul(a[None], (B >> 4) | ((B & 15) << 4), s32, zp, N, K, 4, block)[0]
    assert (np.abs(swapped - ref) > 100 * bound).mean() > 0.9
    # Several activation rows at once (the prefill form) give each row's GEMV.
    A = rng.standard_normal((3, K)).astype(np.float32)
    Y = oracle.mnb_matmul_fast(A, B, s, zp, N, K, block)
    for m in range(3):
        np.testing.assert_array_equal(Y[m], oracle.mnb_matmul_fast(A[m], B, s, zp, N, K, block))


# ---------------------------------------------------------------------- RoPE ---


@pytest.mark.parametrize("interleaved", [False, True])
def test_rotary_closed_forms(oracle, interleaved):
    rng = np.random.default_rng(3)
    B, S, NH, hd = 2, 5, 3, 16
    cos, sin = refs.rotary_caches(64, hd)
    x = rng.standard_normal((B, S, NH * hd)).astype(np.float32)
    rows = np.arange(S)[None, :] + np.array([[0], [7]])
    y = oracle.rotary(x, rows, cos, sin, interleaved=interleaved, num_heads=NH)
    # Position 0 is the identity (cos 1, sin 0).
    np.testing.assert_allclose(y[0, 0], x[0, 0], rtol=0, atol=1e-7)
    # Each rotated pair keeps its norm.
    xr = x.reshape(B, S, NH, hd).astype(np.float64)
    yr = y.reshape(B, S, NH, hd).astype(np.float64)
    if interleaved:
        nx = xr[..., 0::2] ** 2 + xr[..., 1::2] ** 2
        ny = yr[..., 0::2] ** 2 + yr[..., 1::2] ** 2
    else:
        nx = xr[..., :8] ** 2 + xr[..., 8:] ** 2
        ny = yr[..., :8] ** 2 + yr[..., 8:] ** 2
    np.testing.assert_allclose(ny, nx, rtol=1e-5)
    # Against the numpy restatement (sign of the rotation, pair layout).
    for b in range(B):
        ref = refs.apply_rope(xr[b], cos, sin, rows[b], interleaved)
        np.testing.assert_allclose(yr[b], ref, rtol=1e-5, atol=1e-6)
    # Rotation by p1 then p2 equals rotation by p1 + p2 (exact caches).
    y1 = oracle.rotary(x, np.full((B, S), 3), cos, sin, interleaved=interleaved, num_heads=NH)
    y2 = oracle.rotary(y1, np.full((B, S), 4), cos, sin, interleaved=interleaved, num_heads=NH)
    y7 = oracle.rotary(x, np.full((B, S), 7), cos, sin, interleaved=interleaved, num_heads=NH)
    np.testing.assert_allclose(y2, y7, rtol=1e-5, atol=1e-5)


def test_rotary_partial_dims_pass_through(oracle):
    rng = np.random.default_rng(4)
    x = rng.standard_normal((1, 3, 2 * 32)).astype(np.float32)
    cos, sin = refs.rotary_caches(16, 16)  # rotary dim 16 of head 32
    y = oracle.rotary(x, np.arange(3)[None], cos, sin, num_heads=2)
    np.testing.assert_array_equal(y.reshape(1, 3, 2, 32)[..., 16:], x.reshape(1, 3, 2, 32)[..., 16:])


# ----------------------------------------------------------------------- GQA ---


@pytest.mark.parametrize("S,past,cap", [(1, 12, 12), (1, 12, 20), (5, 0, 0), (4, 6, 16), (3, 8, 8)])
@pytest.mark.parametrize("rope", [False, True])
def test_gqa_matches_numpy(oracle, S, past, cap, rope):
    rng = np.random.default_rng(S * 100 + past * 10 + cap + rope)
    B, H, KV, hd = 2, 8, 2, 16
    q = rng.standard_normal((B, S, H * hd)).astype(np.float32)
    k = rng.standard_normal((B, S, KV * hd)).astype(np.float32)
    v = rng.standard_normal((B, S, KV * hd)).astype(np.float32)
    pk = rng.standard_normal((B, KV, cap, hd)).astype(np.float32)
    pv = rng.standard_normal((B, KV, cap, hd)).astype(np.float32)
    total = past + S
    cos = sin = None
    if rope:
        cos, sin = refs.rotary_caches(64, hd)
    out, pres_k, pres_v, shared = oracle.gqa(q, k, v, pk, pv, total, H, KV, cos=cos, sin=sin)
    ro, rk, rv = refs.gqa_ref(q, k, v, pk, pv, total, H, KV, cos=cos, sin=sin)
    assert shared == (cap > past)
    np.testing.assert_allclose(out, ro, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(pres_k, rk, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(pres_v, rv, rtol=0, atol=0)


def test_gqa_packed_equals_separate(oracle):
    rng = np.random.default_rng(5)
    B, S, H, KV, hd, cap = 1, 3, 4, 2, 8, 5
    q = rng.standard_normal((B, S, H * hd)).astype(np.float32)
    k = rng.standard_normal((B, S, KV * hd)).astype(np.float32)
    v = rng.standard_normal((B, S, KV * hd)).astype(np.float32)
    pk = rng.standard_normal((B, KV, cap, hd)).astype(np.float32)
    pv = rng.standard_normal((B, KV, cap, hd)).astype(np.float32)
    a = oracle.gqa(q, k, v, pk, pv, cap + S, H, KV)
    packed = np.concatenate([q, k, v], axis=-1)
    b = oracle.gqa(packed, None, None, pk, pv, cap + S, H, KV)
    np.testing.assert_array_equal(a[0], b[0])


@pytest.mark.parametrize("total", [1, 33, 600])
def test_gqa_step_fast_matches_gqa(oracle, total):
    """The CPU baseline's one-token attention (fp32 numpy) against the oracle's GQA
    on the shared buffer: the new K/V rows identical, the output within one fp16
    ULP (fp32 against fp64 softmax sums, both rounded to fp16). A rotation applied to the wrong
    half of the head, or the new row written at total instead of total - 1, fails."""
    rng = np.random.default_rng(total)
    H, KV, hd, cap = 12, 2, 128, 640
    f16 = lambda *s: rng.standard_normal(s).astype(np.float16).astype(np.float32)  # noqa: E731
    ang = np.arange(1024)[:, None] / (10000.0 ** (np.arange(hd // 2) / (hd // 2)))
    cos, sin = np.cos(ang).astype(np.float16), np.sin(ang).astype(np.float16)
    pk, pv = f16(1, KV, cap, hd), f16(1, KV, cap, hd)
    q, k, v = f16(1, 1, H * hd), f16(1, 1, KV * hd), f16(1, 1, KV * hd)
    ref, rk, rv, shared = oracle.gqa(q, k, v, pk, pv, total, H, KV, cos, sin, round16=True)
    assert shared
    fk, fv = pk.copy(), pv.copy()
    got = oracle._gqa_step_fast(q, k, v, fk, fv, total, H, KV, cos, sin)
    np.testing.assert_array_equal(fk[0, :, :total], rk[0, :, :total])
    np.testing.assert_array_equal(fv[0, :, :total], rv[0, :, :total])
    assert refs.max_ulp_f16(got, ref) <= 1.0


def test_gqa_single_key_returns_value(oracle):
    # With no past and S = 1 the only key is the new one: softmax = 1, out = V.
    rng = np.random.default_rng(6)
    B, H, KV, hd = 1, 4, 1, 8
    q = rng.standard_normal((B, 1, H * hd)).astype(np.float32)
    k = rng.standard_normal((B, 1, KV * hd)).astype(np.float32)
    v = rng.standard_normal((B, 1, KV * hd)).astype(np.float32)
    empty = np.zeros((B, KV, 0, hd), np.float32)
    out, *_ = oracle.gqa(q, k, v, empty, empty, 1, H, KV)
    np.testing.assert_allclose(out.reshape(H, hd), np.tile(v.reshape(1, hd), (H, 1)), rtol=1e-6)


def test_gqa_head_mapping_sensitivity(oracle):
    # Query head h must read kv head h // (H/KV); an h % KV mapping would differ.
    rng = np.random.default_rng(8)
    B, S, H, KV, hd, cap = 1, 1, 4, 2, 8, 6
    q = rng.standard_normal((B, S, H * hd)).astype(np.float32)
    k = rng.standard_normal((B, S, KV * hd)).astype(np.float32)
    v = rng.standard_normal((B, S, KV * hd)).astype(np.float32)
    pk = rng.standard_normal((B, KV, cap, hd)).astype(np.float32)
    pv = rng.standard_normal((B, KV, cap, hd)).astype(np.float32)
    out, *_ = oracle.gqa(q, k, v, pk, pv, cap + 1, H, KV)
    ref, *_ = refs.gqa_ref(q, k, v, pk, pv, cap + 1, H, KV)
    np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-6)
    swapped_kv = pk[:, ::-1].copy(), pv[:, ::-1].copy()
    other, *_ = oracle.gqa(q, k[..., ::-1].copy(), v, *swapped_kv, cap + 1, H, KV)
    assert not np.allclose(other, out)


def _gqa_case(rng, B=2, S=3, H=4, KV=2, hd=16, cap=6):
    q = rng.standard_normal((B, S, H * hd)).astype(np.float32)
    k = rng.standard_normal((B, S, KV * hd)).astype(np.float32)
    v = rng.standard_normal((B, S, KV * hd)).astype(np.float32)
    pk = rng.standard_normal((B, KV, cap, hd)).astype(np.float32)
    pv = rng.standard_normal((B, KV, cap, hd)).astype(np.float32)
    return q, k, v, pk, pv


def test_gqa_qk_norm_is_rms_norm_before_rope(oracle):
    """QK-norm (inputs 14/15) equals normalising q and k per head with numpy first;
    normalising after RoPE instead (weights are not rotation invariant) differs."""
    rng = np.random.default_rng(21)
    B, S, H, KV, hd, cap = 2, 3, 4, 2, 16, 6
    q, k, v, pk, pv = _gqa_case(rng, B, S, H, KV, hd, cap)
    qw = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    kw = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    cos, sin = refs.rotary_caches(32, hd)
    out, prk, prv, _ = oracle.gqa(q, k, v, pk, pv, cap + S, H, KV, cos=cos, sin=sin,
                                  q_norm=qw, k_norm=kw, qk_eps=1e-5)
    qn = refs.rms_norm_ref(q.reshape(B, S, H, hd), qw, 1e-5).reshape(q.shape)
    kn = refs.rms_norm_ref(k.reshape(B, S, KV, hd), kw, 1e-5).reshape(k.shape)
    want, wk, wv, _ = oracle.gqa(qn, kn, v, pk, pv, cap + S, H, KV, cos=cos, sin=sin)
    np.testing.assert_allclose(out, want, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(prk, wk, rtol=1e-5, atol=1e-6)
    np.testing.assert_array_equal(prv, wv)
    ro, rk, _ = refs.gqa_ref(qn, kn, v, pk, pv, cap + S, H, KV, cos=cos, sin=sin)
    np.testing.assert_allclose(out, ro, rtol=1e-5, atol=1e-6)
    # Norm after RoPE: a different result, so the order is pinned.
    pos = np.arange(cap, cap + S)
    qr = np.stack([refs.apply_rope(q.reshape(B, S, H, hd)[b], cos, sin, pos, False)
                   for b in range(B)])
    qrn = refs.rms_norm_ref(qr, qw, 1e-5)
    qh = qn.reshape(B, S, H, hd)
    qrot = np.stack([refs.apply_rope(qh[b], cos, sin, pos, False) for b in range(B)])
    assert not np.allclose(qrn, qrot, atol=1e-3)


def test_gqa_bias_zero_and_constant_rows_change_nothing(oracle):
    rng = np.random.default_rng(22)
    B, S, H, KV, hd, cap = 2, 3, 4, 2, 16, 6
    q, k, v, pk, pv = _gqa_case(rng, B, S, H, KV, hd, cap)
    total = cap + S
    base, *_ = oracle.gqa(q, k, v, pk, pv, total, H, KV)
    zero = np.zeros((1, 1, S, total), np.float32)
    got, *_ = oracle.gqa(q, k, v, pk, pv, total, H, KV, bias=zero)
    np.testing.assert_array_equal(got, base)
    # A per-row constant shifts every score of the row alike: softmax is unchanged.
    const = np.broadcast_to(rng.uniform(-3, 3, (B, H, S, 1)), (B, H, S, total + 2))
    got, *_ = oracle.gqa(q, k, v, pk, pv, total, H, KV, bias=np.ascontiguousarray(const))
    np.testing.assert_allclose(got, base, rtol=1e-5, atol=1e-6)


def test_gqa_bias_one_hot_selects_a_value_row(oracle):
    """A bias of -inf everywhere but key j[b,h,s] makes the softmax one-hot: the
    output row is that key's value row (indexing by batch, head, query and key)."""
    rng = np.random.default_rng(23)
    B, S, H, KV, hd, cap = 2, 3, 4, 2, 16, 6
    q, k, v, pk, pv = _gqa_case(rng, B, S, H, KV, hd, cap)
    total = cap + S
    bias = np.full((B, H, S, total), -np.inf, np.float32)
    pick = np.zeros((B, H, S), np.int64)
    for b in range(B):
        for h in range(H):
            for s in range(S):
                pick[b, h, s] = rng.integers(0, cap + s + 1)  # causal: keys <= cap + s
                bias[b, h, s, pick[b, h, s]] = 0.0
    out, _, prv, _ = oracle.gqa(q, k, v, pk, pv, total, H, KV, bias=bias)
    out = out.reshape(B, S, H, hd)
    g = H // KV
    for b in range(B):
        for h in range(H):
            for s in range(S):
                want = prv[b, h // g, pick[b, h, s]]
                np.testing.assert_allclose(out[b, s, h], want, rtol=1e-6, atol=1e-7)


def test_gqa_bias_broadcast_equals_tiled(oracle):
    rng = np.random.default_rng(24)
    B, S, H, KV, hd, cap = 2, 2, 4, 2, 8, 5
    q, k, v, pk, pv = _gqa_case(rng, B, S, H, KV, hd, cap)
    total = cap + S
    small = rng.standard_normal((1, 1, S, total)).astype(np.float32)
    a, *_ = oracle.gqa(q, k, v, pk, pv, total, H, KV, bias=small)
    b, *_ = oracle.gqa(q, k, v, pk, pv, total, H, KV,
                       bias=np.ascontiguousarray(np.broadcast_to(small, (B, H, S, total))))
    np.testing.assert_array_equal(a, b)
    # A bias does change the result (it is not silently dropped).
    base, *_ = oracle.gqa(q, k, v, pk, pv, total, H, KV)
    assert not np.allclose(a, base, atol=1e-3)


def test_gqa_bf16_rounding_matches_torch(oracle):
    """round16=2 rounds the roped K rows to bfloat16 exactly as torch does (an identity
    rotation, cos = 1 and sin = 0, leaves only the rounding)."""
    import torch

    rng = np.random.default_rng(25)
    B, S, H, KV, hd, cap = 1, 4, 2, 1, 16, 0
    q, k, v, pk, pv = _gqa_case(rng, B, S, H, KV, hd, cap)
    k = k * np.float32(1 + 2.0 ** -9)  # push values off the bf16 grid, including ties
    cos = np.ones((8, hd // 2), np.float32)
    sin = np.zeros((8, hd // 2), np.float32)
    _, prk, _, _ = oracle.gqa(q, k, v, pk, pv, S, H, KV, cos=cos, sin=sin, round16=2)
    want = torch.from_numpy(k).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(prk[0].transpose(1, 0, 2).reshape(S, KV * hd), want[0])


# ---------------------------------------------------- GQA sliding window cache ---


def _sliding_history(rng, N, H, KV, hd, max_pos, interleaved):
    """Queries, keys and values for N absolute positions, and the cos/sin cache."""
    q = (rng.standard_normal((N, H * hd)) * 0.5).astype(np.float32)
    k = (rng.standard_normal((N, KV * hd)) * 0.5).astype(np.float32)
    v = rng.standard_normal((N, KV * hd)).astype(np.float32)
    c, s_ = refs.rotary_caches(max_pos, hd)
    return q, k, v, c.astype(np.float32), s_.astype(np.float32)


def _windowed_attention(oracle, q, k, v, cos, sin, H, KV, hd, t, window, interleaved):
    """Query at absolute position t over the keys at positions (t - window, t], each
    key RoPE'd at its own position: the window read off the whole history, with no
    cache in between."""
    lo = max(0, t - window + 1)
    pos = np.arange(lo, t + 1)
    kr = oracle.rotary(k[None, lo:t + 1], pos[None], cos, sin, interleaved,
                       num_heads=KV)[0].reshape(-1, KV, hd).astype(np.float64)
    qr = oracle.rotary(q[None, t:t + 1], np.array([[t]]), cos, sin, interleaved,
                       num_heads=H)[0].reshape(H, hd).astype(np.float64)
    vv = v[lo:t + 1].reshape(-1, KV, hd).astype(np.float64)
    out = np.zeros((H, hd))
    for h in range(H):
        kv = h // (H // KV)
        sc = kr[:, kv] @ qr[h] / np.sqrt(hd)
        e = np.exp(sc - sc.max())
        out[h] = e @ vv[:, kv] / e.sum()
    return out.reshape(-1)


@pytest.mark.parametrize("cap,window,chunks,interleaved", [
    (5, 3, [1] * 12, 0),            # the reference's sliding-decode (past 8, cap 5, window 3)
    (5, 4, [5, 3, 1, 2, 1, 4], 1),  # sliding-chunk-staging: 3 new rows on a full cache
    (6, 4, [7, 1, 1, 3, 1], 0),     # sliding-batched-rope: past 7 on capacity 6
    (8, 8, [2, 3, 3, 1, 1], 0),     # window = capacity: one row reclaimed at a time
    (4, 1, [3, 2, 1], 1),           # window 1: each query sees only itself
])
def test_gqa_sliding_matches_windowed_history(oracle, cap, window, chunks, interleaved):
    """Chunks fed one after the other, present back into past: every output row equals
    attention over the window of the full history, and present holds the last
    sliding_cache_end(length) keys (RoPE'd at their positions) and values in order,
    zeros after. This pins the cache bookkeeping (the reclaim arithmetic, which rows
    survive, the staging form) and the window bound independently of the reference's
    working-buffer construction that the oracle restates."""
    H, KV, hd = 4, 2, 16
    N = sum(chunks)
    rng = np.random.default_rng(cap * 100 + window * 10 + len(chunks))
    q, k, v, cos, sin = _sliding_history(rng, N, H, KV, hd, N + 4, interleaved)
    pk = rng.standard_normal((1, KV, cap, hd)).astype(np.float32)  # garbage past the valid rows
    pv = rng.standard_normal((1, KV, cap, hd)).astype(np.float32)
    length = 0
    for S in chunks:
        sl = slice(length, length + S)
        out, pk, pv = oracle.gqa_sliding(q[None, sl], k[None, sl], v[None, sl], pk, pv,
                                         [length + S - 1], H, KV, window, cos=cos, sin=sin,
                                         interleaved=bool(interleaved))
        for i in range(S):
            want = _windowed_attention(oracle, q, k, v, cos, sin, H, KV, hd, length + i, window,
                                       interleaved)
            np.testing.assert_allclose(out[0, i], want, rtol=1e-5, atol=1e-6)
        length += S
        end = oracle.sliding_cache_end(length, cap, window)
        first = length - end
        krot = oracle.rotary(k[None, first:length], np.arange(first, length)[None], cos, sin,
                             bool(interleaved), num_heads=KV)[0]
        np.testing.assert_allclose(pk[0, :, :end].transpose(1, 0, 2).reshape(end, -1), krot,
                                   rtol=1e-6, atol=1e-6)
        np.testing.assert_array_equal(pv[0, :, :end].transpose(1, 0, 2).reshape(end, -1),
                                      v[first:length])
        assert not pk[0, :, end:].any() and not pv[0, :, end:].any()


def test_gqa_sliding_cache_end_closed_form(oracle):
    """Reclaim arithmetic against a step-by-step simulation: append one row at a time
    and drop the oldest cap - window + 1 rows whenever a row would not fit."""
    for cap in range(1, 9):
        for window in range(1, cap + 1):
            rows = 0
            for length in range(1, 40):
                if rows == cap:
                    rows -= cap - window + 1
                rows += 1
                assert oracle.sliding_cache_end(length, cap, window) == rows


def test_gqa_sliding_without_eviction_is_plain_gqa(oracle):
    """No row reclaimed and a window covering every key: the shared-buffer GQA of
    oracle.gqa, present included (its rows past the valid ones are old past rows
    there and zeros here)."""
    rng = np.random.default_rng(31)
    B, S, H, KV, hd, cap, past = 2, 3, 6, 2, 32, 16, 7
    q = rng.standard_normal((B, S, H * hd)).astype(np.float32)
    k = rng.standard_normal((B, S, KV * hd)).astype(np.float32)
    v = rng.standard_normal((B, S, KV * hd)).astype(np.float32)
    pk = rng.standard_normal((B, KV, cap, hd)).astype(np.float32)
    pv = rng.standard_normal((B, KV, cap, hd)).astype(np.float32)
    cos, sin = refs.rotary_caches(32, hd)
    total = past + S
    out, prk, prv = oracle.gqa_sliding(q, k, v, pk, pv, [total - 1] * B, H, KV, cap, cos=cos,
                                       sin=sin)
    ro, rk, rv, shared = oracle.gqa(q, k, v, pk, pv, total, H, KV, cos=cos, sin=sin)
    assert shared
    np.testing.assert_allclose(out, ro, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(prk[:, :, :total], rk[:, :, :total], rtol=1e-6, atol=1e-6)
    np.testing.assert_array_equal(prv[:, :, :total], rv[:, :, :total])
    assert not prk[:, :, total:].any()


def test_gqa_sliding_batches_keep_their_own_geometry(oracle):
    """Two sequences at different lengths in one call equal the two run alone, also
    when only one of them needs the staging form (a global switch in the reference)."""
    rng = np.random.default_rng(32)
    H, KV, hd, cap, window, S = 4, 2, 16, 5, 4, 3
    q = rng.standard_normal((2, S, H * hd)).astype(np.float32)
    k = rng.standard_normal((2, S, KV * hd)).astype(np.float32)
    v = rng.standard_normal((2, S, KV * hd)).astype(np.float32)
    pk = rng.standard_normal((2, KV, cap, hd)).astype(np.float32)
    pv = rng.standard_normal((2, KV, cap, hd)).astype(np.float32)
    cos, sin = refs.rotary_caches(32, hd)
    seqlens = [5 + S - 1, 1 + S - 1]  # past 5 (staging) and past 1 (no eviction)
    both = oracle.gqa_sliding(q, k, v, pk, pv, seqlens, H, KV, window, cos=cos, sin=sin)
    for b in range(2):
        one = oracle.gqa_sliding(q[b:b + 1], k[b:b + 1], v[b:b + 1], pk[b:b + 1], pv[b:b + 1],
                                 [seqlens[b]], H, KV, window, cos=cos, sin=sin)
        for x, y in zip(both, one):
            np.testing.assert_allclose(x[b], y[0], rtol=1e-6, atol=1e-7)


# ------------------------------------------------------------ PagedAttention ---


def _paged_case(rng, H, KV, d, nb, blk, batch, new_max=4):
    maxb = nb // batch
    cap = maxb * blk
    new_lens = rng.integers(1, min(new_max, cap) + 1, size=batch).astype(np.int32)
    past = np.array([rng.integers(0, cap - nl + 1) for nl in new_lens], np.int32)
    cum = np.concatenate([[0], np.cumsum(new_lens)]).astype(np.int32)
    nt = int(cum[-1])
    q = (rng.standard_normal((nt, H * d)) * 0.3).astype(np.float32)
    k = (rng.standard_normal((nt, KV * d)) * 0.3).astype(np.float32)
    v = (rng.standard_normal((nt, KV * d)) * 0.3).astype(np.float32)
    kc = (rng.standard_normal((nb, blk, KV, d)) * 0.3).astype(np.float32)
    vc = (rng.standard_normal((nb, blk, KV, d)) * 0.3).astype(np.float32)
    bt = rng.permutation(nb).astype(np.int32).reshape(batch, maxb)
    return q, k, v, kc, vc, cum, past, bt


@pytest.mark.parametrize("H,KV", [(4, 2), (4, 4), (8, 2), (2, 1)])
@pytest.mark.parametrize("rope,interleaved", [(False, 0), (True, 0), (True, 1)])
def test_paged_matches_numpy(oracle, H, KV, rope, interleaved):
    rng = np.random.default_rng(H * 10 + KV + rope * 3 + interleaved)
    d, blk, batch = 16, 4, 3
    q, k, v, kc, vc, cum, past, bt = _paged_case(rng, H, KV, d, 8 * batch, blk, batch)
    cos = sin = None
    if rope:
        cos, sin = refs.rotary_caches(8 * blk, d)
    out, okc, ovc = oracle.paged_attention(q, k, v, kc, vc, cum, past, bt, H, KV, cos=cos, sin=sin,
                                           interleaved=interleaved)
    ref, rkc, rvc = refs.paged_ref(q, k, v, kc, vc, cum, past, bt, H, KV, d, cos=cos, sin=sin,
                                   interleaved=interleaved)
    np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(okc, rkc, rtol=1e-6, atol=1e-6)
    np.testing.assert_array_equal(ovc, rvc)


def test_paged_optional_inputs(oracle):
    # slot_mapping (with a skipped slot), head_sink and QK-norm together
    # (tests/ops/test_paged_attention.py:290-457 form).
    rng = np.random.default_rng(129)
    h, kv, d, nb, blk = 4, 2, 8, 4, 4
    q = rng.standard_normal((3, h * d)).astype(np.float32)
    k = rng.standard_normal((3, kv * d)).astype(np.float32)
    v = rng.standard_normal((3, kv * d)).astype(np.float32)
    kc = rng.standard_normal((nb, blk, kv, d)).astype(np.float32)
    vc = rng.standard_normal((nb, blk, kv, d)).astype(np.float32)
    cum = np.array([0, 3], np.int32)
    past = np.array([3], np.int32)
    bt = np.array([[2, 0, 1, 3]], np.int32)
    slots = np.array([3, -1, 9], np.int32)
    sink = np.array([-0.5, 0.25, 1.0, -1.0], np.float32)
    qw = np.linspace(0.75, 1.25, d).astype(np.float32)
    kw = np.linspace(1.25, 0.75, d).astype(np.float32)
    out, okc, ovc = oracle.paged_attention(q, k, v, kc, vc, cum, past, bt, h, kv,
                                           slot_mapping=slots, head_sink=sink, q_norm=qw,
                                           k_norm=kw, qk_eps=1e-5)
    ref, rkc, rvc = refs.paged_ref(q, k, v, kc, vc, cum, past, bt, h, kv, d, slot_mapping=slots,
                                   head_sink=sink, q_norm=qw, k_norm=kw, norm_eps=1e-5)
    np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(okc, rkc, rtol=1e-6, atol=1e-6)
    np.testing.assert_array_equal(ovc, rvc)


def test_paged_latent_layout_and_offset(oracle):
    rng = np.random.default_rng(291)
    h, kv, d, vd, nb, blk = 2, 1, 16, 8, 3, 4
    q = (rng.standard_normal((2, h * d)) * 0.2).astype(np.float32)
    k = (rng.standard_normal((2, d)) * 0.2).astype(np.float32)
    kc = (rng.standard_normal((nb, blk, kv, d)) * 0.2).astype(np.float32)
    cum, past, bt = np.array([0, 2], np.int32), np.array([3], np.int32), np.array([[1, 0, 2]], np.int32)
    cos, sin = refs.rotary_caches(nb * blk, 8)
    out, okc, _ = oracle.paged_attention(q, k, None, kc, None, cum, past, bt, h, kv, cos=cos,
                                         sin=sin, rotary_offset=8, v_head_size=vd, scale=0.2)
    ref, rkc, _ = refs.paged_ref(q, k, None, kc, None, cum, past, bt, h, kv, d, cos=cos, sin=sin,
                                 rotary_offset=8, vd=vd, scale=0.2)
    np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(okc, rkc, rtol=1e-6, atol=1e-6)


def test_paged_equals_dense_gqa_and_is_permutation_invariant(oracle):
    # Identity block table over a contiguous cache is dense GQA; relabelling the
    # physical blocks (and the table) must not change the output.
    rng = np.random.default_rng(11)
    H, KV, d, blk, past, nq = 4, 2, 16, 4, 9, 3
    nblk = 4
    q = rng.standard_normal((nq, H * d)).astype(np.float32)
    k = rng.standard_normal((nq, KV * d)).astype(np.float32)
    v = rng.standard_normal((nq, KV * d)).astype(np.float32)
    kc = rng.standard_normal((nblk, blk, KV, d)).astype(np.float32)
    vc = rng.standard_normal((nblk, blk, KV, d)).astype(np.float32)
    cum, pastv = np.array([0, nq], np.int32), np.array([past], np.int32)
    ident = np.arange(nblk, dtype=np.int32)[None]
    out, *_ = oracle.paged_attention(q, k, v, kc, vc, cum, pastv, ident, H, KV)
    dense_pk = kc.reshape(nblk * blk, KV, d)[:past].transpose(1, 0, 2)[None]
    dense_pv = vc.reshape(nblk * blk, KV, d)[:past].transpose(1, 0, 2)[None]
    g, *_ = oracle.gqa(q[None], k[None], v[None], dense_pk.copy(), dense_pv.copy(), past + nq, H, KV)
    np.testing.assert_allclose(out, g[0], rtol=1e-5, atol=1e-6)
    perm = rng.permutation(nblk)
    inv = np.argsort(perm)
    kc2, vc2 = kc[perm], vc[perm]  # physical block i now holds old block perm[i]
    table2 = inv[ident].astype(np.int32)
    out2, *_ = oracle.paged_attention(q, k, v, kc2, vc2, cum, pastv, table2, H, KV)
    np.testing.assert_allclose(out2, out, rtol=1e-6, atol=1e-7)


# ------------------------------------------------------------------ RMS norm ---


def test_rms_norm_closed_form_and_numpy(oracle):
    D = 64
    gamma = np.linspace(0.5, 1.5, D).astype(np.float32)
    x = np.full((2, D), 3.0, np.float32)
    y, _ = oracle.rms_norm(x, gamma, 1e-6)
    np.testing.assert_allclose(y, np.broadcast_to(3.0 / np.sqrt(9.0 + 1e-6) * gamma, (2, D)),
                               rtol=1e-6)
    rng = np.random.default_rng(9)
    x = rng.standard_normal((5, D)).astype(np.float32)
    skip = rng.standard_normal((5, D)).astype(np.float32)
    y, r = oracle.rms_norm(x, gamma, 1e-6, skip=skip)
    np.testing.assert_allclose(r, x + skip, rtol=1e-6)
    np.testing.assert_allclose(y, refs.rms_norm_ref(x + skip, gamma), rtol=1e-5, atol=1e-6)
    # fp16 residual rounding: the norm is taken of the rounded residual.
    y16, r16 = oracle.rms_norm(x, gamma, 1e-6, skip=skip, round16=True)
    np.testing.assert_array_equal(r16, (x + skip).astype(np.float16).astype(np.float32))
    np.testing.assert_allclose(y16, refs.rms_norm_ref(r16, gamma), rtol=1e-5, atol=1e-6)
    # The skip variant's optional bias [D] joins every row's residual sum (ORT's
    # input_skip_bias_sum) and a zero bias changes nothing.
    bias = rng.standard_normal(D).astype(np.float32)
    yb, rb = oracle.rms_norm(x, gamma, 1e-6, skip=skip, bias=bias)
    np.testing.assert_allclose(rb, x + skip + bias[None, :], rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(yb, refs.rms_norm_ref(x + skip + bias, gamma), rtol=1e-5, atol=1e-6)
    y0, r0 = oracle.rms_norm(x, gamma, 1e-6, skip=skip, bias=np.zeros(D, np.float32))
    np.testing.assert_array_equal(r0, r)
    np.testing.assert_array_equal(y0, y)
    # The sum is formed in fp32 left to right, as ORT's CPU kernel forms it: 1 + 2^-24
    # rounds (to even) to 1, and 1 + 2^-24 again stays 1, where a single rounding of
    # the exact sum 1 + 2^-23 would keep it.
    one = np.ones((1, D), np.float32)
    tiny = np.full((1, D), 2.0 ** -24, np.float32)
    _, rt = oracle.rms_norm(one, gamma, 1e-6, skip=tiny, bias=tiny[0])
    np.testing.assert_array_equal(rt, one)


def test_decoder_forward_cached_weights_match_per_row_form(oracle):
    """The decoder oracle's fast form (weights dequantised once, fp64 products summed
    by BLAS) equals the per-row C form (fp64 products summed in order) to fp16 output
    rounding, over a prompt and two decode steps of a small 2-layer decoder; the
    logit_rows selection returns exactly the selected rows."""
    from conftest import load_package

    pkg = load_package()
    from importlib import import_module

    dec = import_module(pkg.__name__ + ".decoder")
    cfg = dec.DecoderConfig(layers=2, hidden=256, heads=4, kv_heads=2, head_dim=64, inter=512,
                            vocab=1024, max_pos=128)
    w = dec.make_weights(cfg, seed=3)
    wc = oracle.dequant_cache(w, cfg)
    assert set(wc) == {f"l{i}.{n}" for i in range(2) for n, _, _ in cfg.linear_shapes()} | \
        {"lm_head"}
    ids = np.random.default_rng(4).integers(0, cfg.vocab, size=9)

    def run(cache):
        kr = [np.zeros((1, 2, 32, 64), np.float32) for _ in range(2)]
        vr = [np.zeros_like(k) for k in kr]
        out = [oracle.decoder_forward(w, cfg, ids, kr, vr, 9, wcache=cache)]
        for step, tok in enumerate((5, 77)):
            out.append(oracle.decoder_forward(w, cfg, [tok], kr, vr, 10 + step, wcache=cache))
        return out, kr

    slow, ks = run(None)
    fast, kf = run(wc)
    for a, b in zip(slow, fast):
        ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(a), 2.0 ** -14))) - 10)
        assert (np.abs(a - b) <= ulp).all()
    for a, b in zip(ks, kf):
        assert np.abs(a - b).max() <= 2.0 ** -9 * max(1.0, np.abs(a).max())
    kr = [np.zeros((1, 2, 32, 64), np.float32) for _ in range(2)]
    vr = [np.zeros_like(k) for k in kr]
    last = oracle.decoder_forward(w, cfg, ids, kr, vr, 9, wcache=wc, logit_rows=[8, 2])
    np.testing.assert_array_equal(last, fast[0][[8, 2]])
