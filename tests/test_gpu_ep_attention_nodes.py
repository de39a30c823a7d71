"""PagedAttention and RotaryEmbedding nodes through the plugin-EP boundary
(CreateEpFactories -> GetCapability -> Compile -> Compute) on device tensors,
against the oracle. Tolerance as the kernel tests: fp16 1e-3 + 1 ULP of the exact
value; rotated rows (RoPE outputs rounded once) within 1 ULP; copied rows exact.
"""

from __future__ import annotations

from importlib import import_module

import numpy as np
import pytest
import refs
from test_gpu_ops import assert_f16_close, dev, host, ulp16

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hx(ortmi):
    return import_module(ortmi.__name__ + ".harness")


@pytest.mark.parametrize("interleaved,offset", [(0, 0), (1, 0), (0, 32)])
def test_ep_paged_attention_rope_qk_norm_device_caches(ortmi, oracle, hx, interleaved, offset):
    """PagedAttention with in-op RoPE (optionally interleaved, or on dims past a
    rotary_offset) and QK-norm weights as initializers, caches in device memory
    updated in place, over two calls (a mixed prefill/decode batch, then decode)."""
    import torch

    rng = np.random.default_rng(100 + interleaved + offset)
    H, KV, d, blk, batch, maxb = 8, 2, 128, 16, 3, 5
    nb = maxb * batch + 2
    c, s_ = refs.rotary_caches(256, 64, 10000.0)  # rotary dim 64 of head 128
    cos, sin = c.astype(np.float16), s_.astype(np.float16)
    qn = rng.uniform(0.5, 1.5, d).astype(np.float16)
    kn = rng.uniform(0.5, 1.5, d).astype(np.float16)
    g = hx.Graph()
    g.value("q", hx.FLOAT16, [-1, H * d])
    g.value("k", hx.FLOAT16, [-1, KV * d])
    g.value("v", hx.FLOAT16, [-1, KV * d])
    g.value("kc", hx.FLOAT16, [nb, blk, KV, d])
    g.value("vc", hx.FLOAT16, [nb, blk, KV, d])
    g.value("cum", hx.INT32, [batch + 1])
    g.value("past", hx.INT32, [batch])
    g.value("bt", hx.INT32, [batch, maxb])
    g.value("o", hx.FLOAT16, [-1, H * d])
    g.initializer("cos", cos)
    g.initializer("sin", sin)
    g.initializer("qn", qn)
    g.initializer("kn", kn)
    ins = ["q", "k", "v", "kc", "vc", "cum", "past", "bt", "cos", "sin", "", "", "qn", "kn"]
    g.node("PagedAttention", ins, ["o"], domain="com.microsoft", num_heads=H, kv_num_heads=KV,
           do_rotary=1, rotary_interleaved=interleaved, rotary_offset=offset,
           qk_norm_epsilon=1e-5)
    g.io(["q", "k", "v", "kc", "vc", "cum", "past", "bt"], ["o"])
    sess = hx.Session(g)
    assert sess.partitions() == [[0]]
    kc = rng.standard_normal((nb, blk, KV, d)).astype(np.float16)
    vc = rng.standard_normal((nb, blk, KV, d)).astype(np.float16)
    dkc, dvc = dev(kc), dev(vc)
    bt = rng.permutation(nb)[:batch * maxb].astype(np.int32).reshape(batch, maxb)
    ref_k, ref_v = kc.astype(np.float32), vc.astype(np.float32)
    past = np.array([7, 0, 40], np.int32)
    for call, new in enumerate(([5, 23, 1], [1, 1, 1])):
        new = np.array(new, np.int32)
        cum = np.concatenate([[0], np.cumsum(new)]).astype(np.int32)
        nt = int(cum[-1])
        q, k, v = (rng.standard_normal((nt, n * d)).astype(np.float16) for n in (H, KV, KV))
        o = torch.empty((nt, H * d), dtype=torch.float16, device="cuda")
        sess.bind_output("o", o)
        F, I = hx.FLOAT16, hx.INT32
        sess.run({"q": (dev(q), F), "k": (dev(k), F), "v": (dev(v), F), "kc": (dkc, F),
                  "vc": (dvc, F), "cum": (dev(cum), I), "past": (dev(past), I),
                  "bt": (dev(bt), I)})
        torch.cuda.synchronize()
        ro, rk, rv = oracle.paged_attention(q, k, v, ref_k, ref_v, cum, past, bt, H, KV, cos=cos,
                                            sin=sin, interleaved=bool(interleaved),
                                            rotary_offset=offset, q_norm=qn, k_norm=kn,
                                            qk_eps=1e-5, round16=True)
        assert_f16_close(host(o), ro, extra=ulp16(ro),
                         what=f"EP PagedAttention call {call} (interleaved {interleaved}, "
                              f"offset {offset})")
        gk, gv = host(dkc), host(dvc)
        np.testing.assert_array_equal(gv, oracle.round_f16(rv))
        # New K rows: QK-norm then RoPE, each rounded once (an intermediate that
        # rounds the other way moves the result by at most two ULPs).
        assert (np.abs(gk - rk) <= 2 * ulp16(rk)).all(), "new K rows beyond two fp16 ULPs"
        ref_k, ref_v = gk, gv
        past = past + new


@pytest.mark.parametrize("domain,layout,interleaved,pos_form", [
    ("com.microsoft", "bsnd", 0, "ids"),
    ("com.microsoft", "bsnd", 1, "offset"),
    ("com.microsoft", "bnsd", 0, "ids"),
    ("", "bnsd", 1, "ids"),
    ("", "bsnd", 0, "ids"),
])
def test_ep_rotary_embedding_node(ortmi, oracle, hx, domain, layout, interleaved, pos_form):
    """A RotaryEmbedding node (com.microsoft: x, position_ids, cos, sin; ai.onnx: x,
    cos, sin, position_ids) on device tensors, against the oracle's rotation of
    the same fp16 values."""
    import torch

    rng = np.random.default_rng(200 + 100 * len(domain) + 10 * (layout == "bnsd") +
                                2 * interleaved + (pos_form == "offset"))
    B, S, NH, hd, max_pos = 2, 11, 4, 64, 128
    c, s_ = refs.rotary_caches(max_pos, hd, 10000.0)
    cos, sin = c.astype(np.float16), s_.astype(np.float16)
    shape = [B, S, NH * hd] if layout == "bsnd" else [B, NH, S, hd]
    x = rng.standard_normal(shape).astype(np.float16)
    if pos_form == "offset":
        pos = np.array([17], np.int64)
        rows = np.broadcast_to(17 + np.arange(S), (B, S))
    else:
        pos = rng.integers(0, max_pos, size=(B, S)).astype(np.int64)
        rows = pos
    g = hx.Graph()
    g.value("x", hx.FLOAT16, shape)
    g.value("pos", hx.INT64, list(pos.shape))
    g.value("y", hx.FLOAT16, shape)
    g.initializer("cos", cos)
    g.initializer("sin", sin)
    ins = ["x", "pos", "cos", "sin"] if domain else ["x", "cos", "sin", "pos"]
    attrs = dict(interleaved=interleaved)
    if layout == "bsnd":
        attrs["num_heads"] = NH
    g.node("RotaryEmbedding", ins, ["y"], domain=domain, **attrs)
    g.io(["x", "pos"], ["y"])
    sess = hx.Session(g)
    assert sess.partitions() == [[0]]
    y = torch.empty(shape, dtype=torch.float16, device="cuda")
    sess.bind_output("y", y)
    sess.run({"x": (dev(x), hx.FLOAT16), "pos": (dev(pos), hx.INT64)})
    torch.cuda.synchronize()
    want = oracle.rotary(x, rows, cos, sin, interleaved=bool(interleaved), layout=layout,
                         num_heads=NH if layout == "bsnd" else None)
    got = host(y)
    assert (np.abs(got - want) <= ulp16(want)).all(), \
        f"max diff {np.abs(got - want).max():.3e}"


@pytest.mark.parametrize("dt", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("domain", ["com.microsoft", ""])
def test_ep_rotary_embedding_node_partial_dtypes(ortmi, oracle, hx, dt, domain):
    """A RotaryEmbedding node in both domains with partial rotary (a cos/sin cache of
    width 16 for head size 64: dims [0, 32) rotate, the tail passes through bit for
    bit) in fp16, bf16 and fp32, on device tensors, against the oracle on the same
    rounded inputs."""
    import torch
    from test_gpu_ops import rotary_case

    rng = np.random.default_rng(300 + 7 * ("f16", "bf16", "f32").index(dt) + len(domain))
    B, S, NH, hd, half, max_pos = 2, 5, 4, 64, 16, 64
    shape = [B, S, NH * hd]
    (dx, dc, ds), (x, c, s_), mode, tol = rotary_case(dt, rng, tuple(shape), max_pos, hd, half)
    et = {"f16": hx.FLOAT16, "bf16": hx.BFLOAT16, "f32": hx.FLOAT}[dt]
    pos = rng.integers(0, max_pos, size=(B, S)).astype(np.int64)
    g = hx.Graph()
    g.value("x", et, shape)
    g.value("pos", hx.INT64, [B, S])
    g.value("cos", et, [max_pos, half])
    g.value("sin", et, [max_pos, half])
    g.value("y", et, shape)
    ins = ["x", "pos", "cos", "sin"] if domain else ["x", "cos", "sin", "pos"]
    g.node("RotaryEmbedding", ins, ["y"], domain=domain, num_heads=NH, interleaved=0)
    g.io(["x", "pos", "cos", "sin"], ["y"])
    sess = hx.Session(g)
    assert sess.partitions() == [[0]]
    y = torch.empty(shape, dtype=dx.dtype, device="cuda")
    sess.bind_output("y", y)
    sess.run({"x": (dx, et), "pos": (dev(pos), hx.INT64), "cos": (dc, et), "sin": (ds, et)})
    torch.cuda.synchronize()
    want = oracle.rotary(x, pos, c, s_, round16=mode, num_heads=NH)
    got = host(y)
    assert (np.abs(got - want) <= tol(want)).all(), f"max diff {np.abs(got - want).max():.3e}"
    np.testing.assert_array_equal(got.reshape(B, S, NH, hd)[..., 2 * half:],
                                  x.reshape(B, S, NH, hd)[..., 2 * half:])
