"""GPU parity through the plugin-EP boundary: graphs loaded by the harness host
(CreateEpFactories -> GetCapability -> Compile -> Compute) against the oracle.

Per-op tolerances are those of the kernel tests (fp16: 1e-3 + 1 ULP of the exact
value). The decoder is checked end to end the way the north-star bar states it:
identical greedy tokens. Logits of a many-layer fp16 graph differ from the
fp64-accumulating oracle by accumulated fp16 rounding of intermediates, so the
token check is made teacher-forced: at every step the oracle runs on the same
tokens as the GPU, and the GPU's greedy token must equal the oracle's argmax
unless the oracle's own top-1 margin over the GPU token is within the measured
logit error (a near tie, which the test reports).
"""

from __future__ import annotations

from importlib import import_module

import numpy as np
import pytest
from test_gpu_ops import _mnb_inputs, assert_f16_close, dev, host

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hx(ortmi):
    return import_module(ortmi.__name__ + ".harness")


@pytest.fixture(scope="module")
def dec(ortmi):
    return import_module(ortmi.__name__ + ".decoder")


@pytest.mark.parametrize("M", [1, 9])
def test_ep_matmulnbits_node(ortmi, oracle, hx, M):
    import torch

    rng = np.random.default_rng(40 + M)
    N, K = 384, 1536
    A, B, s, zp = _mnb_inputs(rng, M, N, K, 32, dtype=np.float16)
    g = hx.Graph()
    g.value("x", hx.FLOAT16, [1, -1, K])
    g.value("y", hx.FLOAT16, [1, -1, N])
    g.initializer("B", B)
    g.initializer("s", s)
    g.initializer("zp", zp)
    g.node("MatMulNBits", ["x", "B", "s", "zp"], ["y"], domain="com.microsoft", K=K, N=N, bits=4,
           block_size=32)
    g.io(["x"], ["y"])
    sess = hx.Session(g)
    assert sess.partitions() == [[0]]
    y = torch.empty((1, M, N), dtype=torch.float16, device="cuda")
    sess.bind_output("y", y)
    sess.run({"x": (dev(A.reshape(1, M, K)), hx.FLOAT16)})
    ptr, shape = sess.output("y")
    assert ptr == y.data_ptr() and shape == (1, M, N)
    exact = oracle.mnb_matmul(A, B, s, zp, N, K)
    extra = 0.0
    if M > 1:  # MFMA path: fp16-rounded dequantised weights
        W = oracle.mnb_dequant(B, s, zp, N, K)
        extra = 2.0 ** -11 * (np.abs(A.astype(np.float64)) @ np.abs(W.T))
    assert_f16_close(host(y).reshape(M, N), exact, extra=extra, what="EP MatMulNBits")


@pytest.mark.parametrize("asym", [False, True])
def test_ep_gather_block_quantized_node(ortmi, oracle, hx, asym):
    """An int4 embedding (GatherBlockQuantized, block 32, fp16 scales) claimed and
    run by the EP equals the oracle bit for bit, including a negative id."""
    import torch

    rng = np.random.default_rng(77 + asym)
    V, D, block = 1000, 256, 32
    nb = D // block
    q = rng.integers(0, 16, size=(V, D), dtype=np.uint8)
    data = (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8)
    sc = (np.abs(rng.standard_normal((V, nb))) * 0.05 + 1e-3).astype(np.float16)
    zp = oracle.pack_zero_points(rng.integers(0, 16, size=(V, nb), dtype=np.uint8), 4) if asym else None
    g = hx.Graph()
    g.value("ids", hx.INT64, [1, -1])
    g.value("emb", hx.FLOAT16, [1, -1, D])
    g.initializer("table", data)
    g.initializer("scales", sc)
    inputs = ["table", "ids", "scales"]
    if asym:
        g.initializer("zp", zp.reshape(V, -1))
        inputs.append("zp")
    g.node("GatherBlockQuantized", inputs, ["emb"], domain="com.microsoft", bits=4,
           block_size=block, gather_axis=0, quantize_axis=1)
    g.io(["ids"], ["emb"])
    sess = hx.Session(g)
    assert sess.partitions() == [[0]]
    ids = np.array([[3, V - 1, -2, 0, 517]], np.int64)
    emb = torch.empty((1, ids.shape[1], D), dtype=torch.float16, device="cuda")
    sess.bind_output("emb", emb)
    sess.run({"ids": (dev(ids), hx.INT64)})
    ref = oracle.gather_block_quantized(data, sc.astype(np.float32), zp, ids, block, np.float16)
    np.testing.assert_array_equal(host(emb), ref.astype(np.float32))


def test_ep_output_binding_and_rerun(ortmi, oracle, hx):
    """A bound output receives the result in place; a second run with new input
    values recomputes (nothing is cached between Compute calls)."""
    import torch

    D = 1536
    rng = np.random.default_rng(7)
    g = hx.Graph()
    g.value("x", hx.FLOAT16, [1, -1, D])
    g.value("r", hx.FLOAT16, [1, -1, D])
    g.value("y", hx.FLOAT16, [1, -1, D])
    g.value("res", hx.FLOAT16, [1, -1, D])
    gamma = (1 + 0.1 * rng.standard_normal(D)).astype(np.float16)
    g.initializer("w", gamma)
    g.node("SkipSimplifiedLayerNormalization", ["x", "r", "w"], ["y", "", "", "res"],
           domain="com.microsoft", epsilon=1e-6)
    g.io(["x", "r"], ["y", "res"])
    sess = hx.Session(g)
    y = torch.empty((1, 5, D), dtype=torch.float16, device="cuda")
    res = torch.empty_like(y)
    sess.bind_output("y", y)
    sess.bind_output("res", res)
    for trial in range(2):
        x = rng.standard_normal((1, 5, D)).astype(np.float16)
        r = rng.standard_normal((1, 5, D)).astype(np.float16)
        sess.run({"x": (dev(x), hx.FLOAT16), "r": (dev(r), hx.FLOAT16)})
        ey, er = oracle.rms_norm(x, gamma, 1e-6, skip=r, round16=True)
        np.testing.assert_array_equal(host(res), er)
        assert_f16_close(host(y), ey, what=f"EP SkipSimplifiedLayerNorm run {trial}")


def test_ep_gqa_decode_steps_shared_kv(ortmi, oracle, hx):
    """Three decode steps through GroupQueryAttention with present bound to past."""
    import torch

    H, KV, hd, cap = 12, 2, 128, 64
    rng = np.random.default_rng(11)
    import refs

    c, s_ = refs.rotary_caches(256, hd, 1e6)
    cos, sin = c.astype(np.float16), s_.astype(np.float16)
    g = hx.Graph()
    g.value("q", hx.FLOAT16, [1, 1, H * hd])
    g.value("k", hx.FLOAT16, [1, 1, KV * hd])
    g.value("v", hx.FLOAT16, [1, 1, KV * hd])
    for n in ("pk", "pv", "ok", "ov"):
        g.value(n, hx.FLOAT16, [1, KV, cap, hd])
    g.value("sl", hx.INT32, [1])
    g.value("tot", hx.INT32, [1])
    g.value("o", hx.FLOAT16, [1, 1, H * hd])
    g.initializer("cos", cos)
    g.initializer("sin", sin)
    g.node("GroupQueryAttention", ["q", "k", "v", "pk", "pv", "sl", "tot", "cos", "sin"],
           ["o", "ok", "ov"], domain="com.microsoft", num_heads=H, kv_num_heads=KV, do_rotary=1)
    g.io(["q", "k", "v", "pk", "pv", "sl", "tot"], ["o", "ok", "ov"])
    sess = hx.Session(g)
    past = 20
    pk = np.zeros((1, KV, cap, hd), np.float16)
    pv = np.zeros_like(pk)
    pk[:, :, :past] = rng.standard_normal((1, KV, past, hd))
    pv[:, :, :past] = rng.standard_normal((1, KV, past, hd))
    dpk, dpv = dev(pk), dev(pv)
    sess.bind_output("ok", dpk)
    sess.bind_output("ov", dpv)
    out = torch.empty((1, 1, H * hd), dtype=torch.float16, device="cuda")
    sess.bind_output("o", out)
    ref_k, ref_v = pk.astype(np.float32), pv.astype(np.float32)
    for step in range(3):
        q = rng.standard_normal((1, 1, H * hd)).astype(np.float16)
        k = rng.standard_normal((1, 1, KV * hd)).astype(np.float16)
        v = rng.standard_normal((1, 1, KV * hd)).astype(np.float16)
        total = past + step + 1
        tot = torch.tensor([total], dtype=torch.int32)  # host input, as ONNX Runtime keeps it
        sess.run({"q": (dev(q), hx.FLOAT16), "k": (dev(k), hx.FLOAT16),
                  "v": (dev(v), hx.FLOAT16), "pk": (dpk, hx.FLOAT16), "pv": (dpv, hx.FLOAT16),
                  "sl": (dev(np.array([total - 1], np.int32)), hx.INT32),
                  "tot": (tot, hx.INT32)})
        ro, rk, rv, shared = oracle.gqa(q, k, v, ref_k, ref_v, total, H, KV, cos=cos, sin=sin,
                                        round16=True)
        assert shared
        ref_k, ref_v = oracle.round_f16(rk), oracle.round_f16(rv)
        assert_f16_close(host(out), ro, what=f"EP GQA step {step}")
        np.testing.assert_array_equal(host(dpv), ref_v)


def _small_cfg(dec, hd=64):
    return dec.DecoderConfig(layers=2, hidden=256, heads=4 if hd == 64 else 12, kv_heads=2,
                             head_dim=hd, inter=512, vocab=2048, max_pos=512)


def _teacher_forced_check(oracle, runner, cfg, w, prompt, steps):
    """Run greedy on the GPU and the oracle on the GPU's tokens; returns stats."""
    S = len(prompt)
    kr = [np.zeros((1, cfg.kv_heads, runner.cap, cfg.head_dim), np.float32)
          for _ in range(cfg.layers)]
    vr = [np.zeros_like(k) for k in kr]
    runner.reset()
    runner.prefill(np.asarray(prompt))
    gpu_logits = host(runner.logits[0, :S])
    ref = oracle.decoder_forward(w, cfg, prompt, kr, vr, S)
    max_err = float(np.abs(gpu_logits - ref).max())
    rows = [(gpu_logits[-1], ref[-1], int(runner.next_id.item()))]
    length = S
    for _ in range(steps):
        tok = rows[-1][2]
        runner.decode_step()
        length += 1
        g = host(runner.logits[0, :1])[0]
        r = oracle.decoder_forward(w, cfg, [tok], kr, vr, length)[0]
        max_err = max(max_err, float(np.abs(g - r).max()))
        rows.append((g, r, int(runner.next_id.item())))
    agree, ties = 0, 0
    for g, r, tok in rows:
        assert np.isfinite(g).all() and np.isfinite(r).all(), "non-finite logits"
        assert tok == int(np.argmax(g)), "device argmax disagrees with the logits it read"
        best = int(np.argmax(r))
        if tok == best:
            agree += 1
        else:
            margin = float(r[best] - r[tok])
            assert margin <= 2 * max_err, (
                f"GPU token {tok} vs oracle {best}: margin {margin:.4g} > 2 x logit error "
                f"{max_err:.4g}")
            ties += 1
    return agree, ties, max_err, float(np.abs(rows[0][1]).max())


@pytest.mark.parametrize("hd", [64, 128])
def test_ep_decoder_small_greedy_matches_oracle(ortmi, oracle, dec, hd):
    cfg = _small_cfg(dec, hd)
    w = dec.make_weights(cfg, seed=hd)
    runner = dec.DecoderRunner(cfg, w, cap=64, max_prompt=32)
    rng = np.random.default_rng(hd + 1)
    prompt = rng.integers(0, cfg.vocab, size=24).tolist()
    agree, ties, err, scale = _teacher_forced_check(oracle, runner, cfg, w, prompt, steps=12)
    print(f"decoder hd={hd}: {agree} tokens agree, {ties} near ties; max logit err {err:.3e} "
          f"(|logit| up to {scale:.2f})")
    assert err <= 0.05 * max(1.0, scale)
    assert agree >= 11


def test_ep_decoder_full_size_short_prompt(ortmi, oracle, dec):
    """The 28-layer, hidden-1536, vocab-151936 decoder: an 8-token prompt and 4 greedy
    steps teacher-forced against the oracle (the full 512 + 128 run is the benchmark)."""
    cfg = dec.DecoderConfig()
    w = dec.make_weights(cfg, seed=4)
    runner = dec.DecoderRunner(cfg, w, cap=64, max_prompt=16)
    assert len(runner.session.partitions()) == 1
    prompt = np.random.default_rng(5).integers(0, cfg.vocab, size=8).tolist()
    agree, ties, err, scale = _teacher_forced_check(oracle, runner, cfg, w, prompt, steps=4)
    print(f"full decoder: {agree} agree, {ties} near ties; max logit err {err:.3e} "
          f"(|logit| up to {scale:.2f})")
    assert err <= 0.05 * max(1.0, scale)
    assert agree >= 4


def test_ep_decoder_prefill_matches_incremental_decode(ortmi, dec):
    """KV-cache consistency at full size: logits of a token decoded incrementally
    equal those of the same position in one prefill of the whole sequence."""
    import torch

    cfg = dec.DecoderConfig()
    w = dec.make_weights(cfg, seed=4)
    runner = dec.DecoderRunner(cfg, w, cap=160, max_prompt=144)
    prompt = np.random.default_rng(6).integers(0, cfg.vocab, size=128).tolist()
    tokens, _, _ = runner.generate(np.asarray(prompt), steps=9)
    inc = host(runner.logits[0, :1])[0]
    full = prompt + tokens[:-1]
    runner.reset()
    runner.prefill(np.asarray(full))
    torch.cuda.synchronize()
    pre = host(runner.logits[0, len(full) - 1])
    scale = float(np.abs(pre).max())
    err = float(np.abs(pre - inc).max())
    assert err <= 0.05 * max(1.0, scale)
    tok = int(runner.next_id.item())
    if tok != tokens[-1]:  # prefill (MFMA GEMM) and decode (GEMV) may split a near tie
        assert float(pre[tok] - pre[tokens[-1]]) <= 2 * err


def test_ep_decode_graph_replay_matches_eager(ortmi, dec, monkeypatch):
    """Decode steps replayed from the EP's captured HIP graph equal eager steps bit
    for bit (same kernels), across a fresh prefill between generations."""
    cfg = _small_cfg(dec, 128)
    w = dec.make_weights(cfg, seed=21)
    prompt = np.random.default_rng(22).integers(0, cfg.vocab, size=20)

    def run(graphs):
        monkeypatch.setenv("ORTMI_EP_GRAPH", "1" if graphs else "0")
        r = dec.DecoderRunner(cfg, w, cap=64, max_prompt=32)
        seen = []
        for rep in range(2):
            r.reset()
            r.prefill(prompt[: 20 - 4 * rep])
            seen.append(host(r.logits[0, :1]))
            for _ in range(8):
                r.decode_step()
                seen.append(host(r.logits[0, :1]))
        return np.stack(seen)

    eager = run(False)
    graphed = run(True)
    np.testing.assert_array_equal(graphed, eager)


def test_ep_decoder_fusions_match_unfused(ortmi, dec, monkeypatch):
    """The decode rewrites (QKV and gate/up merges, norm prologues, SwiGLU
    epilogue) against the same graph run op by op: logits within the fp16
    tolerance carried through two layers, the same greedy tokens."""
    cfg = _small_cfg(dec, 128)
    w = dec.make_weights(cfg, seed=31)
    prompt = np.random.default_rng(32).integers(0, cfg.vocab, size=12)

    def run(fuse):
        monkeypatch.setenv("ORTMI_EP_FUSE", "1" if fuse else "0")
        r = dec.DecoderRunner(cfg, w, cap=64, max_prompt=32)
        r.prefill(prompt)
        logits, toks = [host(r.logits[0, :12])], [int(r.next_id.item())]
        for _ in range(6):
            r.decode_step()
            logits.append(host(r.logits[0, :1]))
            toks.append(int(r.next_id.item()))
        return logits, toks

    fl, ft = run(True)
    ul, ut = run(False)
    for a, b in zip(fl, ul):
        assert np.abs(a - b).max() <= 0.02 * max(1.0, np.abs(b).max())
    assert ft == ut
