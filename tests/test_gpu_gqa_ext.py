"""GroupQueryAttention forms served by the generic kernels
(ortmi_group_query_attention_ex): fp32 tensors, QK-norm (inputs 14/15), an
additive attention_bias (input 10) and head sizes other than 64/128, against the
oracle on the same rounded inputs.

Tolerances: fp32 1e-5 + 1e-5 |exact|; fp16 1e-3 + 2 ULP of the exact value
(one ULP for the output rounding, one for an intermediate that rounds the other
way); bf16 4e-3 + 2^-6 |exact| (the bf16 decode-kernel bound). New fp16/bf16 K
rows are within one ULP of the oracle's (RoPE outputs rounded once; two with
QK-norm, whose rounded output feeds the RoPE), fp32 ones within 1e-6 (1 + |x|);
old K rows and all V rows are exact copies.
"""

from __future__ import annotations

import numpy as np
import pytest
import refs
from test_gpu_ops import ulp16

pytestmark = pytest.mark.gpu

_ROUND = {"f32": 0, "f16": 1, "bf16": 2}


def _tdt(dt):
    import torch

    return {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}[dt]


def _cast(a, dt):
    """(device tensor, float32 numpy of the same rounded values)."""
    import torch

    t = torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(_tdt(dt))
    return t.cuda(), t.float().numpy()


def _ulp(x, dt):
    x = np.abs(np.asarray(x, np.float64))
    if dt == "f16":
        return ulp16(x)
    mant = 23 if dt == "f32" else 7
    e = np.floor(np.log2(np.maximum(x, 2.0 ** -126)))
    return 2.0 ** (e - mant)


def _window_bias(B, S, total, vp, window):
    """Causal + sliding-window additive mask [B, 1, S, total] (0 or -inf)."""
    bias = np.full((B, 1, S, total), -np.inf, np.float32)
    for s in range(S):
        p = vp + s
        bias[:, :, s, max(0, p - window + 1):p + 1] = 0.0
    return bias


def _run(ortmi, oracle, dt, B, S, H, KV, hd, cap, past, *, rope=True, interleaved=False,
         rot_half=None, qk_norm=False, bias=None, packed=False, inplace=False, seed=0,
         scale=0.0):
    import torch

    rng = np.random.default_rng(seed)
    total = past + S
    shared = 0 <= past <= cap and cap > past
    vp = past if 0 <= past <= cap else cap
    q, nq = _cast(rng.standard_normal((B, S, H * hd)), dt)
    k, nk = _cast(rng.standard_normal((B, S, KV * hd)), dt)
    v, nv = _cast(rng.standard_normal((B, S, KV * hd)), dt)
    pk, npk = _cast(rng.standard_normal((B, KV, cap, hd)), dt)
    pv, npv = _cast(rng.standard_normal((B, KV, cap, hd)), dt)
    cos = sin = ncos = nsin = None
    if rope:
        c, s_ = refs.rotary_caches(max(total, 16) + 8, 2 * (rot_half or hd // 2), 10000.0)
        cos, ncos = _cast(c, dt)
        sin, nsin = _cast(s_, dt)
    qn = kn = nqn = nkn = None
    if qk_norm:
        qn, nqn = _cast(rng.uniform(0.5, 1.5, hd), dt)
        kn, nkn = _cast(rng.uniform(0.5, 1.5, hd), dt)
    db = nb = None
    if bias is not None:
        db, nb = _cast(bias, dt)
    if packed:
        qin = torch.cat([q, k, v], dim=-1).contiguous()
        kin = vin = None
    else:
        qin, kin, vin = q, k, v
    kw = dict(present_key=pk, present_value=pv) if inplace else {}
    out, prk, prv = ortmi.group_query_attention(
        qin, kin, vin, pk, pv, torch.full((B,), total - 1, dtype=torch.int32, device="cuda"),
        total, cos, sin, num_heads=H, kv_num_heads=KV, do_rotary=int(rope),
        rotary_interleaved=int(interleaved), attention_bias=db, q_norm_weight=qn,
        k_norm_weight=kn, qk_norm_epsilon=1e-5, scale=scale, **kw)
    torch.cuda.synchronize()
    ro, rk, rv, rshared = oracle.gqa(nq, nk, nv, npk, npv, total, H, KV, cos=ncos, sin=nsin,
                                     interleaved=interleaved, scale=scale, round16=_ROUND[dt],
                                     q_norm=nqn, k_norm=nkn, qk_eps=1e-5, bias=nb)
    assert rshared == shared
    got = out.float().cpu().numpy()
    assert out.dtype == _tdt(dt) and got.shape == ro.shape
    if dt == "f32":
        tol = 1e-5 + 1e-5 * np.abs(ro)
    elif dt == "f16":
        tol = 1e-3 + 2 * ulp16(ro)
    else:
        tol = 4e-3 + 2.0 ** -6 * np.abs(ro)
    bad = ~(np.abs(got - ro) <= tol)
    assert not bad.any(), (f"{dt} output: {bad.sum()} of {bad.size} beyond tolerance, max diff "
                           f"{np.nanmax(np.abs(got - ro)):.3e}")
    gk, gv = prk.float().cpu().numpy(), prv.float().cpu().numpy()
    old = np.ones(gk.shape[2], bool)
    old[vp:vp + S] = False
    np.testing.assert_array_equal(gk[:, :, old], rk[:, :, old])
    np.testing.assert_array_equal(gv, rv)
    new_k = gk[:, :, vp:vp + S]
    # RoPE (and QK-norm) outputs rounded once; after QK-norm an intermediate that
    # rounds the other way moves the result by at most two ULPs.
    # fp32 rows are not rounded to a storage grid: the kernel's fp32 products and
    # difference against the oracle's fp64 ones (|x| ~ 1 here).
    ulps = 2 if qk_norm else 1
    want_k = rk[:, :, vp:vp + S]
    tol_k = 1e-6 + 1e-6 * np.abs(want_k) if dt == "f32" else ulps * _ulp(want_k, dt)
    assert (np.abs(new_k - want_k) <= tol_k).all(), \
        f"new K rows: max diff {np.abs(new_k - want_k).max():.3e}"
    return got, gv


@pytest.mark.parametrize("interleaved", [False, True])
def test_gqa_fp32_decode_growing(ortmi, oracle, interleaved):
    _run(ortmi, oracle, "f32", B=2, S=1, H=8, KV=2, hd=128, cap=300, past=300,
         interleaved=interleaved, seed=1)


def test_gqa_fp32_decode_shared_inplace(ortmi, oracle):
    _run(ortmi, oracle, "f32", B=1, S=1, H=16, KV=4, hd=128, cap=512, past=200, inplace=True,
         seed=2)


def test_gqa_fp32_prefill_packed_growing(ortmi, oracle):
    _run(ortmi, oracle, "f32", B=1, S=37, H=4, KV=2, hd=64, cap=5, past=5, packed=True,
         interleaved=True, seed=3)


def test_gqa_fp32_prefill_no_past_custom_scale(ortmi, oracle):
    _run(ortmi, oracle, "f32", B=2, S=19, H=6, KV=3, hd=64, cap=0, past=0, rope=False,
         scale=0.05, seed=4)


@pytest.mark.parametrize("dt", ["f16", "bf16", "f32"])
def test_gqa_qk_norm_prefill_shared(ortmi, oracle, dt):
    _run(ortmi, oracle, dt, B=2, S=16, H=8, KV=2, hd=128, cap=64, past=20, qk_norm=True,
         inplace=True, seed=5)


def test_gqa_qk_norm_decode_head256(ortmi, oracle):
    _run(ortmi, oracle, "bf16", B=1, S=1, H=16, KV=8, hd=256, cap=128, past=100, qk_norm=True,
         inplace=True, seed=6)


@pytest.mark.parametrize("S,past,cap", [(24, 0, 64), (1, 40, 64), (9, 30, 30)])
def test_gqa_bias_sliding_window_mask(ortmi, oracle, S, past, cap):
    """The Gemma3n form: do_rotary = 0, a causal + sliding-window additive mask as
    attention_bias [B, 1, S, total], head size 256."""
    vp = past if past <= cap else cap
    bias = _window_bias(1, S, past + S, vp, window=8)
    got, _ = _run(ortmi, oracle, "f16", B=1, S=S, H=4, KV=1, hd=256, cap=cap, past=past,
                  rope=False, bias=bias, seed=7)
    assert np.isfinite(got).all()


def test_gqa_bias_per_head_batch_wider_rows(ortmi, oracle):
    """attention_bias [B, H, S, total + 3] (rows wider than the attended keys) with a
    different random bias per batch, head and query."""
    B, S, H, past = 2, 5, 8, 17
    bias = np.random.default_rng(8).standard_normal((B, H, S, past + S + 3)).astype(np.float32)
    _run(ortmi, oracle, "f16", B=B, S=S, H=H, KV=2, hd=128, cap=past, past=past, bias=bias,
         seed=9)


def test_gqa_bias_broadcast_fp32(ortmi, oracle):
    B, S, past = 2, 3, 40
    bias = np.random.default_rng(10).standard_normal((1, 1, S, past + S)).astype(np.float32)
    _run(ortmi, oracle, "f32", B=B, S=S, H=8, KV=4, hd=64, cap=64, past=past, bias=bias,
         inplace=True, seed=11)


def test_gqa_bias_one_hot_selects_value_rows(ortmi, oracle):
    """-inf everywhere but one key per (head, query): each output row is that key's
    V row, rounded once."""
    B, S, H, KV, hd, past = 1, 4, 4, 2, 64, 12
    total = past + S
    rng = np.random.default_rng(12)
    bias = np.full((B, H, S, total), -np.inf, np.float32)
    pick = np.zeros((H, S), np.int64)
    for h in range(H):
        for s in range(S):
            pick[h, s] = rng.integers(0, past + s + 1)
            bias[0, h, s, pick[h, s]] = 0.0
    got, gv = _run(ortmi, oracle, "f16", B=B, S=S, H=H, KV=KV, hd=hd, cap=past, past=past,
                   bias=bias, seed=13)
    got = got.reshape(S, H, hd)
    for h in range(H):
        for s in range(S):
            np.testing.assert_array_equal(got[s, h], gv[0, h // (H // KV), pick[h, s]])


def test_gqa_head96_partial_rotary(ortmi, oracle):
    """Head size 96 (no fused kernel) with RoPE on the first 64 dims only."""
    _run(ortmi, oracle, "f16", B=2, S=7, H=6, KV=2, hd=96, cap=32, past=10, rot_half=32,
         inplace=True, seed=14)


@pytest.mark.parametrize("dt", ["f16", "f32"])
def test_ep_gqa_node_bias_and_qk_norm(ortmi, oracle, dt):
    """A 16-input GroupQueryAttention node (attention_bias, QK-norm weights as
    initializers, in-op RoPE) through the plugin EP: two decode steps with present
    bound to past, against the oracle."""
    from importlib import import_module

    import torch

    hx = import_module(ortmi.__name__ + ".harness")
    H, KV, hd, cap, past = 8, 2, 128, 48, 20
    et = hx.FLOAT16 if dt == "f16" else hx.FLOAT
    rng = np.random.default_rng(15)
    c, s_ = refs.rotary_caches(128, hd, 1e6)
    _, ncos = _cast(c, dt)
    _, nsin = _cast(s_, dt)
    _, nqn = _cast(rng.uniform(0.5, 1.5, hd), dt)
    _, nkn = _cast(rng.uniform(0.5, 1.5, hd), dt)
    npdt = np.float16 if dt == "f16" else np.float32
    g = hx.Graph()
    g.value("q", et, [1, 1, H * hd])
    g.value("k", et, [1, 1, KV * hd])
    g.value("v", et, [1, 1, KV * hd])
    for n in ("pk", "pv", "ok", "ov"):
        g.value(n, et, [1, KV, cap, hd])
    g.value("sl", hx.INT32, [1])
    g.value("tot", hx.INT32, [1])
    g.value("bias", et, [1, 1, 1, -1])
    g.value("o", et, [1, 1, H * hd])
    g.initializer("cos", ncos.astype(npdt))
    g.initializer("sin", nsin.astype(npdt))
    g.initializer("qn", nqn.astype(npdt))
    g.initializer("kn", nkn.astype(npdt))
    ins = ["q", "k", "v", "pk", "pv", "sl", "tot", "cos", "sin", "", "bias", "", "", "", "qn",
           "kn"]
    g.node("GroupQueryAttention", ins, ["o", "ok", "ov"], domain="com.microsoft", num_heads=H,
           kv_num_heads=KV, do_rotary=1, qk_norm_epsilon=1e-5)
    g.io(["q", "k", "v", "pk", "pv", "sl", "tot", "bias"], ["o", "ok", "ov"])
    sess = hx.Session(g)
    assert sess.partitions() == [[0]]
    pk, npk = _cast(np.concatenate([rng.standard_normal((1, KV, past, hd)),
                                    np.zeros((1, KV, cap - past, hd))], axis=2), dt)
    pv, npv = _cast(np.concatenate([rng.standard_normal((1, KV, past, hd)),
                                    np.zeros((1, KV, cap - past, hd))], axis=2), dt)
    sess.bind_output("ok", pk)
    sess.bind_output("ov", pv)
    out = torch.empty((1, 1, H * hd), dtype=_tdt(dt), device="cuda")
    sess.bind_output("o", out)
    for step in range(2):
        total = past + step + 1
        q, nq = _cast(rng.standard_normal((1, 1, H * hd)), dt)
        k, nk = _cast(rng.standard_normal((1, 1, KV * hd)), dt)
        v, nv = _cast(rng.standard_normal((1, 1, KV * hd)), dt)
        b, nb = _cast(rng.standard_normal((1, 1, 1, total)) * 2, dt)
        sess.run({"q": (q, et), "k": (k, et), "v": (v, et), "pk": (pk, et), "pv": (pv, et),
                  "sl": (torch.tensor([total - 1], dtype=torch.int32, device="cuda"), hx.INT32),
                  "tot": (torch.tensor([total], dtype=torch.int32), hx.INT32),
                  "bias": (b, et)})
        torch.cuda.synchronize()
        ro, rk, rv, shared = oracle.gqa(nq, nk, nv, npk, npv, total, H, KV, cos=ncos, sin=nsin,
                                        round16=_ROUND[dt], q_norm=nqn, k_norm=nkn,
                                        qk_eps=1e-5, bias=nb)
        assert shared
        got = out.float().cpu().numpy()
        tol = 1e-3 + 2 * ulp16(ro) if dt == "f16" else 1e-5 + 1e-5 * np.abs(ro)
        assert (np.abs(got - ro) <= tol).all(), f"EP GQA step {step}: max diff " \
            f"{np.abs(got - ro).max():.3e}"
        gk = pk.float().cpu().numpy()
        np.testing.assert_array_equal(pv.float().cpu().numpy(), rv)
        tol_k = 1e-6 + 1e-6 * np.abs(rk) if dt == "f32" else 2 * _ulp(rk, dt)
        assert (np.abs(gk - rk) <= tol_k).all()
        npk, npv = gk, rv


# ------------------------------------------------------- sliding-window cache ---


def _run_sliding(ortmi, oracle, dt, B, S, H, KV, hd, cap, window, seqlens, *, rope=True,
                 interleaved=False, qk_norm=False, packed=False, inplace=False, seed=0,
                 past=None):
    """One sliding-cache step through ortmi.group_query_attention_sliding against
    oracle.gqa_sliding on the same rounded inputs; returns the device present
    (key, value) for the next step. past: (key, value) device tensors, or None for
    random ones."""
    import torch

    rng = np.random.default_rng(seed)
    q, nq = _cast(rng.standard_normal((B, S, H * hd)), dt)
    k, nk = _cast(rng.standard_normal((B, S, KV * hd)), dt)
    v, nv = _cast(rng.standard_normal((B, S, KV * hd)), dt)
    if past is None:
        pk, npk = _cast(rng.standard_normal((B, KV, cap, hd)), dt)
        pv, npv = _cast(rng.standard_normal((B, KV, cap, hd)), dt)
    else:
        pk, pv = past
        npk, npv = pk.float().cpu().numpy(), pv.float().cpu().numpy()
    cos = sin = ncos = nsin = None
    if rope:
        c, s_ = refs.rotary_caches(max(seqlens) + S + 8, hd, 10000.0)
        cos, ncos = _cast(c, dt)
        sin, nsin = _cast(s_, dt)
    qn = kn = nqn = nkn = None
    if qk_norm:
        qn, nqn = _cast(rng.uniform(0.5, 1.5, hd), dt)
        kn, nkn = _cast(rng.uniform(0.5, 1.5, hd), dt)
    if packed:
        qin, kin, vin = torch.cat([q, k, v], dim=-1).contiguous(), None, None
    else:
        qin, kin, vin = q, k, v
    kw = dict(present_key=pk, present_value=pv) if inplace else {}
    sl = torch.tensor(seqlens, dtype=torch.int32, device="cuda")
    out, prk, prv = ortmi.group_query_attention_sliding(
        qin, kin, vin, pk, pv, sl, cos, sin, num_heads=H, kv_num_heads=KV,
        local_window_size=window, do_rotary=int(rope), rotary_interleaved=int(interleaved),
        q_norm_weight=qn, k_norm_weight=kn, qk_norm_epsilon=1e-5, **kw)
    torch.cuda.synchronize()
    ro, rk, rv = oracle.gqa_sliding(nq, nk, nv, npk, npv, seqlens, H, KV, window, cos=ncos,
                                    sin=nsin, interleaved=interleaved, round16=_ROUND[dt],
                                    q_norm=nqn, k_norm=nkn, qk_eps=1e-5)
    got = out.float().cpu().numpy()
    if dt == "f32":
        tol = 1e-5 + 1e-5 * np.abs(ro)
    elif dt == "f16":
        tol = 1e-3 + 2 * ulp16(ro)
    else:
        tol = 4e-3 + 2.0 ** -6 * np.abs(ro)
    bad = ~(np.abs(got - ro) <= tol)
    assert not bad.any(), (f"{dt} sliding output: {bad.sum()} of {bad.size} beyond tolerance, "
                           f"max diff {np.nanmax(np.abs(got - ro)):.3e}")
    gk, gv = prk.float().cpu().numpy(), prv.float().cpu().numpy()
    np.testing.assert_array_equal(gv, rv)
    ulps = 2 if qk_norm else 1
    for b in range(B):
        p = max(seqlens[b] + 1 - S, 0)
        after = oracle.sliding_cache_end(p + S, cap, window)
        first_new = max(after - S, 0)  # rows [first_new, after) are this step's keys
        np.testing.assert_array_equal(gk[b, :, :first_new], rk[b, :, :first_new])
        np.testing.assert_array_equal(gk[b, :, after:], 0)
        new_k, want_k = gk[b, :, first_new:after], rk[b, :, first_new:after]
        tol_k = 1e-6 + 1e-6 * np.abs(want_k) if dt == "f32" else ulps * _ulp(want_k, dt)
        assert (np.abs(new_k - want_k) <= tol_k).all(), \
            f"new K rows: max diff {np.abs(new_k - want_k).max():.3e}"
    return prk, prv


# The reference's sliding_window_cache cases (tests/ops/test_mlx_ops.py:245-300).
_SLIDING_REF = [
    ("sliding-decode", dict(B=1, H=4, KV=2, hd=16, S=1, past=8, cap=5, rope=False, window=3)),
    ("sliding-chunk-staging", dict(B=1, H=4, KV=2, hd=16, S=3, past=5, cap=5, rope=False,
                                   window=4)),
    ("sliding-batched-rope", dict(B=2, H=4, KV=2, hd=16, S=1, past=7, cap=6, rope=True,
                                  window=4)),
]


@pytest.mark.parametrize("inplace", [False, True])
@pytest.mark.parametrize("name,g", _SLIDING_REF, ids=[c[0] for c in _SLIDING_REF])
def test_gqa_sliding_reference_cases(ortmi, oracle, name, g, inplace):
    seqlens = [g["past"] + g["S"] - 1] * g["B"]
    _run_sliding(ortmi, oracle, "f32", g["B"], g["S"], g["H"], g["KV"], g["hd"], g["cap"],
                 g["window"], seqlens, rope=g["rope"], inplace=inplace, seed=11)


@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_gqa_sliding_steps_in_place(ortmi, oracle, dt):
    """Chunks and single tokens fed one after the other into one cache compacted in
    place (present bound to past), through several reclaims: head 128, RoPE."""
    past = None
    length = 0
    for i, S in enumerate([9, 3, 1, 1, 4, 1, 1, 1, 7, 1]):
        past = _run_sliding(ortmi, oracle, dt, 1, S, 8, 2, 128, 12, 8, [length + S - 1],
                            interleaved=True, inplace=True, seed=20 + i, past=past)
        length += S


def test_gqa_sliding_batches_qk_norm_packed(ortmi, oracle):
    """Two sequences at different lengths (one needing the staging form, one not
    yet full), packed QKV, QK-norm, head 64, fp16, separate present."""
    _run_sliding(ortmi, oracle, "f16", 2, 3, 6, 3, 64, 5, 4, [5 + 3 - 1, 1 + 3 - 1],
                 qk_norm=True, packed=True, seed=30)
