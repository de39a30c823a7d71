"""GPU parity through the plugin-EP boundary: graphs loaded by the harness host
(CreateEpFactories -> GetCapability -> Compile -> Compute) against the oracle.

Per-op tolerances are those of the kernel tests (fp16: 1e-3 + 1 ULP of the exact
value). The decoder is checked end to end on identical greedy tokens. Logits of
a many-layer fp16 graph differ from the fp64-accumulating oracle by accumulated
fp16 rounding of intermediates, so the token check is made teacher-forced: at every step the oracle runs on the same
tokens as the GPU, and the GPU's greedy token must equal the oracle's argmax
unless the oracle's own top-1 margin over the GPU token is within TIE_ULPS fp16
ULPs of the row's largest |logit| (a near tie, which the test prints). There is
no agreement quota, and the logits themselves must agree within TIE_ULPS ULPs of
the row max.
"""

from __future__ import annotations

from importlib import import_module

import numpy as np
import pytest
from test_gpu_ops import _mnb_inputs, assert_f16_close, dev, host, ulp16

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


# Stated tie bound of the strict greedy check: a GPU token may differ from the
# oracle's argmax only where the oracle's own top-1 margin over that token is at
# most TIE_ULPS fp16 ULPs of the row's largest |logit| (the fp16 logits of two
# implementations that round 28 layers of fp16 intermediates differently).
TIE_ULPS = 16


@pytest.mark.parametrize("dtype,V,keepdims", [
    (np.float16, 151936, 0),
    (np.float32, 1000, 1),
    (np.float16, 77, 1),
])
def test_ep_argmax_node(ortmi, hx, dtype, V, keepdims):
    """ArgMax over the last axis through the EP against numpy's argmax (the lowest
    index wins ties, as ONNX ArgMax with select_last_index=0 defines it; a NaN never
    wins). Rows carry planted ties, a NaN and a maximum in the last column; the
    keepdims=1 cases write into a host-memory output."""
    import torch

    rng = np.random.default_rng(V + keepdims)
    x = rng.standard_normal((2, 3, V)).astype(dtype)
    x[0, 0, 5] = x[0, 0, 7] = 9.0
    x[0, 1, 0] = np.nan
    x[0, 1, V - 1] = 9.0
    x[0, 2, V - 2] = x[0, 2, V - 1] = 9.0
    x[1, 0, :] = 1.0
    onnx_dt = hx.FLOAT16 if dtype == np.float16 else hx.FLOAT
    g = hx.Graph()
    g.value("x", onnx_dt, [-1, -1, V])
    g.value("y", hx.INT64, [-1, -1, 1] if keepdims else [-1, -1])
    g.node("ArgMax", ["x"], ["y"], axis=-1, keepdims=keepdims)
    g.io(["x"], ["y"])
    sess = hx.Session(g)
    assert sess.partitions() == [[0]]
    shape = (2, 3, 1) if keepdims else (2, 3)
    if keepdims:
        y = torch.full(shape, -1, dtype=torch.int64)
    else:
        y = torch.full(shape, -1, dtype=torch.int64, device="cuda")
    sess.bind_output("y", y)
    sess.run({"x": (dev(x), onnx_dt)})
    torch.cuda.synchronize()
    want = np.argmax(np.where(np.isnan(x), -np.inf, x), axis=-1).reshape(shape)
    assert want[0, 0].item() == 5 and want[0, 1].item() == V - 1 and want[0, 2].item() == V - 2
    assert want[1, 0].item() == 0
    np.testing.assert_array_equal(y.cpu().numpy(), want)


@pytest.mark.parametrize("dtype,axis,keepdims,last", [
    (np.float16, 0, 1, 0),
    (np.float32, 1, 0, 1),
    (np.float16, -1, 1, 1),
    ("bf16", 1, 1, 0),
    (np.float32, -1, 0, 1),
])
def test_ep_argmax_node_any_axis_and_tie_rule(ortmi, hx, dtype, axis, keepdims, last):
    """ArgMax over a leading, middle or last axis, with select_last_index 0 (the
    first maximum) and 1 (the last), through the EP against numpy: argmax of the
    values with NaN read as -inf, on the reversed axis for the last index. Values
    are drawn from 7 levels so that most slices tie; a NaN is planted."""
    import torch

    rng = np.random.default_rng(31 + axis + 3 * last)
    shape = (6, 50, 37)
    x = rng.integers(0, 7, size=shape).astype(np.float32)
    x[1, 2, 3] = np.nan
    if dtype == "bf16":
        onnx_dt, xt = hx.BFLOAT16, torch.from_numpy(x).to(torch.bfloat16).cuda()
    else:
        onnx_dt = hx.FLOAT16 if dtype == np.float16 else hx.FLOAT
        xt = torch.from_numpy(x.astype(dtype)).cuda()
    ax = axis % 3
    oshape = tuple(1 if i == ax else d for i, d in enumerate(shape)) if keepdims else \
        tuple(d for i, d in enumerate(shape) if i != ax)
    g = hx.Graph()
    g.value("x", onnx_dt, list(shape))
    g.value("y", hx.INT64, list(oshape))
    g.node("ArgMax", ["x"], ["y"], axis=axis, keepdims=keepdims, select_last_index=last)
    g.io(["x"], ["y"])
    sess = hx.Session(g)
    assert sess.partitions() == [[0]]
    y = torch.full(oshape, -1, dtype=torch.int64, device="cuda")
    sess.bind_output("y", y)
    sess.run({"x": (xt, onnx_dt)})
    torch.cuda.synchronize()
    xv = np.where(np.isnan(x), -np.inf, x)
    if last:
        want = shape[ax] - 1 - np.argmax(np.flip(xv, axis=ax), axis=ax)
    else:
        want = np.argmax(xv, axis=ax)
    np.testing.assert_array_equal(y.cpu().numpy(), want.reshape(oshape))


def test_ep_decode_program_argmax_node(ortmi, dec, monkeypatch):
    """A decoder graph that ends in ArgMax: its one-token steps run as the decode
    program with the program's argmax written to the ArgMax output (ORTMI_EP_PROGRAM
    =require), giving the tokens and logits of the graph without ArgMax (the runner
    taking the argmax itself) and of the op-by-op path; one step writes the ArgMax
    output into host memory."""
    import torch

    cfg = _small_cfg(dec, 128)
    w = dec.make_weights(cfg, seed=43)
    prompt = np.random.default_rng(44).integers(0, cfg.vocab, size=13)

    def run(mode, argmax_node, host_last=False):
        monkeypatch.setenv("ORTMI_EP_PROGRAM", mode)
        r = dec.DecoderRunner(cfg, w, cap=64, max_prompt=32, argmax_node=argmax_node)
        r.prefill(prompt)
        toks, logits = [int(r.next_id.item())], []
        for i in range(8):
            if host_last and i == 7:
                buf = torch.full((1, 32), -1, dtype=torch.int64)
                r.tokens[r._flip], r._first[r._flip] = buf, buf[:, :1]
            r.decode_step()
            logits.append(host(r.logits[0, :1])[0])
            toks.append(int(r.next_id.item()))
        return toks, logits

    base_t, base_l = run("require", False)
    prog_t, prog_l = run("require", True, host_last=True)
    op_t, _ = run("0", True)
    print(f"tokens {base_t}", flush=True)
    assert prog_t == base_t and op_t == base_t
    for a, b in zip(prog_l, base_l):
        np.testing.assert_array_equal(a, b)


def _fp16_ulp(x):
    return 2.0 ** (np.floor(np.log2(max(abs(float(x)), 2.0 ** -14))) - 10)


def _assert_greedy_strict(rows, what):
    """rows: (GPU logits, oracle logits, GPU token) per step. Every GPU token is its
    own logits' argmax and the oracle's argmax, except where the oracle's margin over
    it is within TIE_ULPS fp16 ULPs of the row's max |logit| (printed); the logits
    agree within TIE_ULPS ULPs of the row max. Returns (ties, max ULPs)."""
    worst, ties = 0.0, []
    for i, (g, r, tok) in enumerate(rows):
        assert np.isfinite(g).all() and np.isfinite(r).all(), f"{what} step {i}: non-finite logits"
        assert tok == int(np.argmax(g)), f"{what} step {i}: device argmax disagrees with its logits"
        ulp = _fp16_ulp(np.abs(r).max())
        worst = max(worst, float(np.abs(g - r).max()) / ulp)
        best = int(np.argmax(r))
        if tok != best:
            margin = float(r[best] - r[tok])
            print(f"{what} step {i}: GPU {tok} vs oracle {best}, oracle margin {margin:.4g} "
                  f"(bound {TIE_ULPS * ulp:.4g})", flush=True)
            assert margin <= TIE_ULPS * ulp, (f"{what} step {i}: GPU token {tok} vs oracle {best}:"
                                              f" margin {margin:.4g} > {TIE_ULPS} ULPs")
            ties.append(i)
    print(f"{what}: {len(rows) - len(ties)} of {len(rows)} tokens equal the oracle's argmax; "
          f"near ties {len(ties)} (steps {ties}); max |logit diff| {worst:.1f} fp16 ULPs of "
          f"the row max", flush=True)
    assert worst <= TIE_ULPS, f"{what}: logits differ by {worst:.1f} ULPs of the row max"
    return ties, worst


def _small_cfg(dec, hd=64):
    heads = {64: 4, 96: 8}.get(hd, 12)
    return dec.DecoderConfig(layers=2, hidden=256, heads=heads, kv_heads=2,
                             head_dim=hd, inter=512, vocab=2048, max_pos=512)


def _teacher_forced_check(oracle, runner, cfg, w, prompt, steps):
    """Run greedy on the GPU and the oracle on the GPU's tokens; returns the
    (GPU logits, oracle logits, GPU token) rows."""
    S = len(prompt)
    kr = [np.zeros((1, cfg.kv_heads, runner.cap, cfg.head_dim), np.float32)
          for _ in range(cfg.layers)]
    vr = [np.zeros_like(k) for k in kr]
    runner.reset()
    runner.prefill(np.asarray(prompt))
    gpu_logits = host(runner.logits[0, :S])
    ref = oracle.decoder_forward(w, cfg, prompt, kr, vr, S)
    rows = [(gpu_logits[-1], ref[-1], int(runner.next_id.item()))]
    length = S
    for _ in range(steps):
        tok = rows[-1][2]
        runner.decode_step()
        length += 1
        g = host(runner.logits[0, :1])[0]
        r = oracle.decoder_forward(w, cfg, [tok], kr, vr, length)[0]
        rows.append((g, r, int(runner.next_id.item())))
    return rows


@pytest.mark.parametrize("hd", [64, 96, 128])
def test_ep_decoder_small_greedy_matches_oracle(ortmi, oracle, dec, hd):
    cfg = _small_cfg(dec, hd)
    w = dec.make_weights(cfg, seed=hd)
    runner = dec.DecoderRunner(cfg, w, cap=64, max_prompt=32)
    rng = np.random.default_rng(hd + 1)
    prompt = rng.integers(0, cfg.vocab, size=24).tolist()
    rows = _teacher_forced_check(oracle, runner, cfg, w, prompt, steps=12)
    _assert_greedy_strict(rows, f"decoder hd={hd}")


def test_ep_decoder_full_size_short_prompt(ortmi, oracle, dec):
    """The 28-layer, hidden-1536, vocab-151936 decoder: an 8-token prompt and 4 greedy
    steps teacher-forced against the oracle (the full 512 + 128 run is the benchmark)."""
    cfg = dec.DecoderConfig()
    w = dec.make_weights(cfg, seed=4)
    runner = dec.DecoderRunner(cfg, w, cap=64, max_prompt=16)
    assert len(runner.session.partitions()) == 1
    prompt = np.random.default_rng(5).integers(0, cfg.vocab, size=8).tolist()
    rows = _teacher_forced_check(oracle, runner, cfg, w, prompt, steps=4)
    _assert_greedy_strict(rows, "full decoder, short prompt")


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


def test_ep_decoder_layer_partitions_match_whole(ortmi, oracle, dec, monkeypatch):
    """A 4-layer decoder whose metadata names its layer boundaries, split two layers
    per fused node (ONNXRUNTIME_EP_MLX_LAYER_PARTITIONS=2): three fused nodes, and
    the same logits (within the fp16 tolerance of the fusions that cannot cross a
    cut) and greedy tokens as the whole graph; tokens teacher-forced against the
    oracle."""
    cfg = dec.DecoderConfig(layers=4, hidden=256, heads=4, kv_heads=2, head_dim=64, inter=512,
                            vocab=2048, max_pos=512)
    w = dec.make_weights(cfg, seed=41)
    prompt = np.random.default_rng(42).integers(0, cfg.vocab, size=14)
    monkeypatch.setenv("ORTMI_EP_PROGRAM", "0")

    def run(span):
        if span:
            monkeypatch.setenv("ONNXRUNTIME_EP_MLX_LAYER_PARTITIONS", str(span))
        else:
            monkeypatch.delenv("ONNXRUNTIME_EP_MLX_LAYER_PARTITIONS", raising=False)
        r = dec.DecoderRunner(cfg, w, cap=64, max_prompt=32, layer_metadata=True)
        nparts = len(r.session.partitions())
        rows = _teacher_forced_check(oracle, r, cfg, w, prompt.tolist(), steps=6)
        return nparts, rows

    n_whole, whole = run(0)
    n_split, split = run(2)
    assert (n_whole, n_split) == (1, 3)
    for (a, _, ta), (b, _, tb) in zip(split, whole):
        assert np.abs(a - b).max() <= 0.02 * max(1.0, np.abs(b).max())
        assert ta == tb
    _assert_greedy_strict(split, "decoder split in layer groups")


# ------------------------------------------------------------- boundary slots --

def _one_node_mnb_graph(hx, rng, N=256, K=512):
    A, B, s, zp = _mnb_inputs(rng, 1, N, K, 32, dtype=np.float16)
    g = hx.Graph()
    g.value("x", hx.FLOAT16, [1, 1, K])
    g.value("y", hx.FLOAT16, [1, 1, N])
    g.initializer("B", B)
    g.initializer("s", s)
    g.initializer("zp", zp)
    g.node("MatMulNBits", ["x", "B", "s", "zp"], ["y"], domain="com.microsoft", K=K, N=N, bits=4,
           block_size=32)
    g.io(["x"], ["y"])
    return g, (A, B, s, zp, N, K)


def test_ep_memory_device_allocator_and_data_transfer(ortmi, hx, monkeypatch):
    """GetDefaultMemoryDevice reports the HBM memory device the EP device registered
    (GPU, AMD's vendor id, GPU 0), or CPU memory with ORTMI_EP_MEMORY=cpu;
    CreateAllocator hands out an HBM allocator only for the EP's own memory info
    (MI355X_HBM, a visible GPU id), whose Alloc/Reserve/Free/Info work;
    CreateDataTransfer copies host<->device and device<->device bit for bit, on each
    of its paths: small host-to-device copies in one launch, device-to-pageable-host
    copies through its pinned staging buffer, and plain asynchronous copies for
    larger tensors and pinned destinations."""
    import torch

    g, _ = _one_node_mnb_graph(hx, np.random.default_rng(1))
    monkeypatch.setenv("ORTMI_EP_MEMORY", "cpu")
    cpu_sess = hx.Session(g)
    assert cpu_sess.default_memory_device_is_cpu()
    assert cpu_sess.memory_device() == (0, 0, 0)
    cpu_sess.close()
    monkeypatch.delenv("ORTMI_EP_MEMORY")
    sess = hx.Session(g)
    assert not sess.default_memory_device_is_cpu()
    assert sess.memory_device() == (1, 0x1002, 0)
    assert sess.allocator_check("MI355X_HBM", 0, 3 << 20) is True
    assert sess.allocator_check("Cpu", 0) is None
    with pytest.raises(RuntimeError, match="GPU 4096"):
        sess.allocator_check("MI355X_HBM", 4096)
    src = torch.arange(3 * 5 * 7, dtype=torch.float32).reshape(3, 5, 7) * 0.25 - 9
    d1 = torch.empty_like(src, device="cuda")
    d2 = torch.empty_like(d1)
    back = torch.empty_like(src)
    sess.data_transfer_copy(src, d1, hx.FLOAT)    # host -> device
    sess.data_transfer_copy(d1, d2, hx.FLOAT)     # device -> device
    sess.data_transfer_copy(d2, back, hx.FLOAT)   # device -> host
    torch.cuda.synchronize()
    assert torch.equal(back, src)
    # Larger than the one-launch (1 KiB) and staging (1 MiB) bounds, and a pinned
    # destination.
    big = torch.randn(3, 1000, 100, dtype=torch.float32)  # 1.2 MB
    db = torch.empty_like(big, device="cuda")
    sess.data_transfer_copy(big, db, hx.FLOAT)
    big_back = torch.empty_like(big)
    sess.data_transfer_copy(db, big_back, hx.FLOAT)
    pinned = torch.empty_like(src).pin_memory()
    sess.data_transfer_copy(d2, pinned, hx.FLOAT)
    torch.cuda.synchronize()
    assert torch.equal(big_back, big) and torch.equal(pinned, src)


@pytest.mark.parametrize("memory", ["hbm", "cpu"])
def test_ep_host_memory_input_and_output(ortmi, oracle, hx, monkeypatch, memory):
    """Host-memory input and output buffers. With the HBM memory device the harness
    applies ORT's placement rule (the feed copied to HBM and the output produced
    there and copied back, through the EP's data transfer); with CPU memory
    (ORTMI_EP_MEMORY=cpu, what ORT hands an EP whose default memory device is the
    CPU) the EP gets the host buffers and stages them itself. Either way the caller's
    host buffer receives the result, identical to the device-bound run."""
    import torch

    g, (A, B, s, zp, N, K) = _one_node_mnb_graph(hx, np.random.default_rng(2))
    monkeypatch.setenv("ORTMI_EP_MEMORY", memory)
    sess = hx.Session(g)
    x_host = torch.from_numpy(A.reshape(1, 1, K).copy())
    y_host = torch.full((1, 1, N), float("nan"), dtype=torch.float16)
    sess.bind_output("y", y_host)
    sess.run({"x": (x_host, hx.FLOAT16)})
    # HBM: one copy in (the feed), one out (the output); CPU: the EP's own staging.
    assert sess.copies() == (2 if memory == "hbm" else 0)
    y_dev = torch.empty((1, 1, N), dtype=torch.float16, device="cuda")
    sess.bind_output("y", y_dev)
    sess.run({"x": (x_host.cuda(), hx.FLOAT16)})
    torch.cuda.synchronize()
    assert torch.equal(y_host, y_dev.cpu())
    assert_f16_close(y_host.float().numpy().reshape(1, N), oracle.mnb_matmul(A, B, s, zp, N, K),
                     what="host-memory MatMulNBits")


def _gqa_graph(hx, H, KV, hd, cap, cos, sin):
    g = hx.Graph()
    g.value("q", hx.FLOAT16, [1, -1, H * hd])
    g.value("k", hx.FLOAT16, [1, -1, KV * hd])
    g.value("v", hx.FLOAT16, [1, -1, KV * hd])
    for n in ("pk", "pv", "ok", "ov"):
        g.value(n, hx.FLOAT16, [1, KV, cap, hd])
    g.value("sl", hx.INT32, [1])
    g.value("tot", hx.INT32, [1])
    g.value("o", hx.FLOAT16, [1, -1, H * hd])
    g.initializer("cos", cos)
    g.initializer("sin", sin)
    g.node("GroupQueryAttention", ["q", "k", "v", "pk", "pv", "sl", "tot", "cos", "sin"],
           ["o", "ok", "ov"], domain="com.microsoft", num_heads=H, kv_num_heads=KV, do_rotary=1)
    g.io(["q", "k", "v", "pk", "pv", "sl", "tot"], ["o", "ok", "ov"])
    return g


def test_ep_gqa_host_kv_delta_write_back(ortmi, hx, monkeypatch):
    """A KV cache in host memory shared by past and present (the reference's
    shared-buffer contract with a CPU-memory EP): a 5-token prompt then 6 decode
    steps give outputs and cache contents identical to the same steps over device
    buffers, and the rows past the live length keep the caller's sentinel (only
    the new rows are written back)."""
    import refs
    import torch

    H, KV, hd, cap = 12, 2, 128, 48
    c, s_ = refs.rotary_caches(256, hd, 1e6)
    cos, sin = c.astype(np.float16), s_.astype(np.float16)
    rng = np.random.default_rng(12)
    steps = [5] + [1] * 6
    feeds = [tuple(rng.standard_normal((1, S, n * hd)).astype(np.float16) for n in (H, KV, KV))
             for S in steps]
    sentinel = np.float16(-7.5)

    def run(on_device):
        # Device buffers with the HBM EP; host buffers with an EP that reports CPU
        # memory, which ORT hands the host buffers themselves.
        monkeypatch.setenv("ORTMI_EP_MEMORY", "hbm" if on_device else "cpu")
        sess = hx.Session(_gqa_graph(hx, H, KV, hd, cap, cos, sin))
        kc = torch.full((1, KV, cap, hd), float(sentinel), dtype=torch.float16)
        vc = torch.full_like(kc, float(sentinel))
        if on_device:
            kc, vc = kc.cuda(), vc.cuda()
        sess.bind_output("ok", kc)
        sess.bind_output("ov", vc)
        outs, total = [], 0
        for (q, k, v), S in zip(feeds, steps):
            total += S
            o = torch.empty((1, S, H * hd), dtype=torch.float16,
                            device="cuda" if on_device else "cpu")
            sess.bind_output("o", o)
            t = (lambda a: torch.from_numpy(a).cuda()) if on_device else torch.from_numpy
            sess.run({"q": (t(q), hx.FLOAT16), "k": (t(k), hx.FLOAT16),
                      "v": (t(v), hx.FLOAT16), "pk": (kc, hx.FLOAT16), "pv": (vc, hx.FLOAT16),
                      "sl": (torch.tensor([total - 1], dtype=torch.int32), hx.INT32),
                      "tot": (torch.tensor([total], dtype=torch.int32), hx.INT32)})
            torch.cuda.synchronize()
            outs.append(o.cpu().clone())
        sess.close()
        return outs, kc.cpu(), vc.cpu(), total

    dev_outs, dk, dv, total = run(True)
    host_outs, hk, hv, _ = run(False)
    for a, b in zip(host_outs, dev_outs):
        assert torch.equal(a, b)
    assert torch.equal(hk, dk) and torch.equal(hv, dv)
    assert (hk[:, :, total:] == float(sentinel)).all() and (hv[:, :, total:] == float(sentinel)).all()
    assert not (hk[:, :, :total] == float(sentinel)).all()


def test_ep_paged_attention_host_caches_written_back(ortmi, oracle, hx, monkeypatch):
    """PagedAttention through an EP that reports CPU memory (ORTMI_EP_MEMORY=cpu),
    with its caches in host memory: the new K/V rows land in the caller's cache
    buffers (in place, as the reference writes them back,
    rust/src/ops/attention.rs:2728-2742), and output and caches equal the oracle's
    over two consecutive calls."""
    import torch

    monkeypatch.setenv("ORTMI_EP_MEMORY", "cpu")
    rng = np.random.default_rng(90)
    H, KV, d, blk, batch = 8, 2, 64, 4, 3
    maxb = 6
    nb = maxb * batch
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
    g.node("PagedAttention", ["q", "k", "v", "kc", "vc", "cum", "past", "bt"], ["o"],
           domain="com.microsoft", num_heads=H, kv_num_heads=KV)
    g.io(["q", "k", "v", "kc", "vc", "cum", "past", "bt"], ["o"])
    sess = hx.Session(g)
    assert sess.partitions() == [[0]]
    kc = torch.from_numpy(rng.standard_normal((nb, blk, KV, d)).astype(np.float16))
    vc = torch.from_numpy(rng.standard_normal((nb, blk, KV, d)).astype(np.float16))
    bt = rng.permutation(nb).astype(np.int32).reshape(batch, maxb)
    ref_k, ref_v = kc.float().numpy(), vc.float().numpy()
    past = np.array([3, 0, 10], np.int32)
    for call, new in enumerate(([4, 5, 1], [1, 1, 1])):
        new = np.array(new, np.int32)
        cum = np.concatenate([[0], np.cumsum(new)]).astype(np.int32)
        nt = int(cum[-1])
        q, k, v = (rng.standard_normal((nt, n * d)).astype(np.float16) for n in (H, KV, KV))
        o = torch.empty((nt, H * d), dtype=torch.float16)
        sess.bind_output("o", o)
        tt = torch.from_numpy
        sess.run({"q": (tt(q), hx.FLOAT16), "k": (tt(k), hx.FLOAT16), "v": (tt(v), hx.FLOAT16),
                  "kc": (kc, hx.FLOAT16), "vc": (vc, hx.FLOAT16), "cum": (tt(cum), hx.INT32),
                  "past": (tt(past), hx.INT32), "bt": (tt(bt), hx.INT32)})
        torch.cuda.synchronize()
        ro, ref_k, ref_v = oracle.paged_attention(q, k, v, ref_k, ref_v, cum, past, bt, H, KV)
        ref_k, ref_v = oracle.round_f16(ref_k), oracle.round_f16(ref_v)
        assert_f16_close(o.float().numpy(), ro, what=f"host-cache PagedAttention call {call}")
        np.testing.assert_array_equal(kc.float().numpy(), ref_k)
        np.testing.assert_array_equal(vc.float().numpy(), ref_v)
        past = past + new


def test_ep_decoder_config4_greedy_tokens_strict(ortmi, oracle, dec, monkeypatch, capsys):
    """The benchmarked int4 decoder end to end: 28 layers, vocab 151936, a 512-token
    prompt then 128 greedy decode steps (129 tokens), every token checked against
    the oracle teacher-forced: the oracle runs the prompt, then the GPU's 128 fed-back
    tokens in one causal pass, and each GPU token must be the oracle's argmax, or the
    oracle's margin over it must be within TIE_ULPS fp16 ULPs of the row's max |logit|
    (each such step is printed, and their count). No agreement quota.
    Fed the way a stock ONNX Runtime feeds an EP whose memory device is HBM: input
    ids, seqlens_k and total_sequence_length are host tensors that the harness copies
    to HBM through the EP's data transfer each step (the KV cache and logits bound to
    device buffers), and every one-token step must run as the decode program
    (ORTMI_EP_PROGRAM=require)."""
    import time

    monkeypatch.setenv("ORTMI_EP_PROGRAM", "require")
    cfg = dec.DecoderConfig()
    w = dec.make_weights(cfg, seed=4)
    P, steps = 512, 128
    runner = dec.DecoderRunner(cfg, w, cap=P + steps, max_prompt=P, host_feeds=True)
    assert runner.session.memory_device() == (1, 0x1002, 0)
    prompt = np.random.default_rng(44).integers(0, cfg.vocab, size=P)
    runner.reset()
    runner.prefill(prompt)
    gpu = [host(runner.logits[0, P - 1])]
    toks = [int(runner.next_id.item())]
    copies0 = runner.session.copies()
    for _ in range(steps):
        runner.decode_step()
        gpu.append(host(runner.logits[0, 0]))
        toks.append(int(runner.next_id.item()))
    # One data-transfer call per step: the host feeds (ids, seqlens_k, total) to HBM.
    assert runner.session.copies() - copies0 == steps
    print(f"GPU tokens {toks[:8]} ... ({len(toks)})", flush=True)
    t0 = time.time()
    wc = oracle.dequant_cache(w, cfg)
    kr = [np.zeros((1, cfg.kv_heads, P + steps, cfg.head_dim), np.float32)
          for _ in range(cfg.layers)]
    vr = [np.zeros_like(k) for k in kr]
    r0 = oracle.decoder_forward(w, cfg, prompt, kr, vr, P, wcache=wc, logit_rows=[P - 1])
    r1 = oracle.decoder_forward(w, cfg, toks[:steps], kr, vr, P + steps, wcache=wc)
    ref = np.concatenate([r0, r1])
    del wc
    print(f"oracle: {time.time() - t0:.1f} s", flush=True)
    assert ref.shape == (steps + 1, cfg.vocab)
    ties, worst = _assert_greedy_strict(list(zip(gpu, ref, toks)), "cfg4 512+128")
    with capsys.disabled():  # the near-tie count belongs in the run's own output
        print(f"\ncfg4 512+128 (host feeds, decode program): {len(toks) - len(ties)} of "
              f"{len(toks)} tokens equal the oracle's argmax, near ties {len(ties)} {ties}, "
              f"max |logit diff| {worst:.1f} fp16 ULPs of the row max", flush=True)


def test_ep_decode_program_matches_op_path(ortmi, oracle, dec, monkeypatch):
    """One-token steps of a fused decoder run as one launch of the decode program
    (ORTMI_EP_PROGRAM=require makes any other path an error) against the same steps
    op by op (ORTMI_EP_PROGRAM=0): logits within the fp16 tolerance carried through
    the layers, identical greedy tokens; and the program's steps teacher-forced
    against the oracle with the strict token rule."""
    cfg = _small_cfg(dec, 128)
    w = dec.make_weights(cfg, seed=41)
    prompt = np.random.default_rng(42).integers(0, cfg.vocab, size=17)

    def run(mode):
        monkeypatch.setenv("ORTMI_EP_PROGRAM", mode)
        r = dec.DecoderRunner(cfg, w, cap=64, max_prompt=32)
        r.prefill(prompt)
        logits, toks = [], [int(r.next_id.item())]
        for _ in range(10):
            r.decode_step()
            logits.append(host(r.logits[0, :1])[0])
            toks.append(int(r.next_id.item()))
        return logits, toks

    pl, pt = run("require")
    ol, ot = run("0")
    for i, (a, b) in enumerate(zip(pl, ol)):
        err = float(np.abs(a - b).max())
        print(f"step {i}: program vs op path max |logit diff| {err:.3e}", flush=True)
        assert err <= 2.0 ** -7 * max(1.0, float(np.abs(b).max()))
    assert pt == ot

    monkeypatch.setenv("ORTMI_EP_PROGRAM", "require")
    runner = dec.DecoderRunner(cfg, w, cap=64, max_prompt=32)
    rows = _teacher_forced_check(oracle, runner, cfg, w, prompt.tolist(), steps=10)
    _assert_greedy_strict(rows, "decode program through the EP")


def test_ep_gqa_sliding_window_cache(ortmi, oracle, hx, monkeypatch):
    """GroupQueryAttention with sliding_window_cache = 1 through the EP: a 5-token
    prompt, a 3-token chunk and single tokens into a capacity-6, window-4 cache
    that present compacts in place, each step against oracle.gqa_sliding on the
    cache the step read; the same steps with the cache in host memory give
    identical outputs and caches."""
    import refs
    import torch

    H, KV, hd, cap, window = 4, 2, 64, 6, 4
    c, s_ = refs.rotary_caches(64, hd, 1e4)
    cos, sin = c.astype(np.float16), s_.astype(np.float16)
    rng = np.random.default_rng(13)
    steps = [5, 3, 1, 1, 2, 1, 1]
    feeds = [tuple(rng.standard_normal((1, S, n * hd)).astype(np.float16) for n in (H, KV, KV))
             for S in steps]

    def run(on_device, check):
        monkeypatch.setenv("ORTMI_EP_MEMORY", "hbm" if on_device else "cpu")
        g = hx.Graph()
        g.value("q", hx.FLOAT16, [1, -1, H * hd])
        g.value("k", hx.FLOAT16, [1, -1, KV * hd])
        g.value("v", hx.FLOAT16, [1, -1, KV * hd])
        for n in ("pk", "pv", "ok", "ov"):
            g.value(n, hx.FLOAT16, [1, KV, cap, hd])
        g.value("sl", hx.INT32, [1])
        g.value("tot", hx.INT32, [1])
        g.value("o", hx.FLOAT16, [1, -1, H * hd])
        g.initializer("cos", cos)
        g.initializer("sin", sin)
        g.node("GroupQueryAttention", ["q", "k", "v", "pk", "pv", "sl", "tot", "cos", "sin"],
               ["o", "ok", "ov"], domain="com.microsoft", num_heads=H, kv_num_heads=KV,
               do_rotary=1, sliding_window_cache=1, local_window_size=window)
        g.io(["q", "k", "v", "pk", "pv", "sl", "tot"], ["o", "ok", "ov"])
        sess = hx.Session(g)
        assert sess.partitions() == [[0]]
        kc = torch.zeros((1, KV, cap, hd), dtype=torch.float16)
        vc = torch.zeros_like(kc)
        if on_device:
            kc, vc = kc.cuda(), vc.cuda()
        sess.bind_output("ok", kc)
        sess.bind_output("ov", vc)
        outs, total = [], 0
        for (q, k, v), S in zip(feeds, steps):
            past_k, past_v = kc.float().cpu().numpy(), vc.float().cpu().numpy()
            total += S
            o = torch.empty((1, S, H * hd), dtype=torch.float16,
                            device="cuda" if on_device else "cpu")
            sess.bind_output("o", o)
            t = (lambda a: torch.from_numpy(a).cuda()) if on_device else torch.from_numpy
            sess.run({"q": (t(q), hx.FLOAT16), "k": (t(k), hx.FLOAT16),
                      "v": (t(v), hx.FLOAT16), "pk": (kc, hx.FLOAT16), "pv": (vc, hx.FLOAT16),
                      "sl": (torch.tensor([total - 1], dtype=torch.int32), hx.INT32),
                      "tot": (torch.tensor([total], dtype=torch.int32), hx.INT32)})
            torch.cuda.synchronize()
            outs.append(o.cpu().clone())
            if check:
                ro, rk, rv = oracle.gqa_sliding(q, k, v, past_k, past_v, [total - 1], H, KV,
                                                window, cos=cos, sin=sin, round16=1)
                assert_f16_close(outs[-1].float().numpy().reshape(S, -1), ro.reshape(S, -1),
                                 extra=ulp16(ro.reshape(S, -1)),
                                 what=f"sliding step S={S} total={total}")
                gk, gv = kc.float().cpu().numpy(), vc.float().cpu().numpy()
                np.testing.assert_array_equal(gv, rv)
                assert (np.abs(gk - rk) <= ulp16(rk)).all()
        sess.close()
        return outs, kc.cpu(), vc.cpu()

    dev_outs, dk, dv = run(True, True)
    host_outs, hk, hv = run(False, False)
    for a, b in zip(host_outs, dev_outs):
        assert torch.equal(a, b)
    assert torch.equal(hk, dk) and torch.equal(hv, dv)


def test_ep_decode_program_abort_falls_back_to_op_path(ortmi, dec, monkeypatch):
    """A one-token step the decode program does not complete runs op by op: the
    program's third launch is aborted before it starts (ORTMI_EP_PROGRAM_ABORT=3,
    through the workspace's abort word), and the run still returns that step's
    tokens, equal to an unaborted run's. With ORTMI_EP_PROGRAM=require the same
    abort is an error naming the status."""
    cfg = _small_cfg(dec, 128)
    w = dec.make_weights(cfg, seed=71)
    prompt = np.random.default_rng(72).integers(0, cfg.vocab, size=11)

    def run(abort, mode):
        monkeypatch.setenv("ORTMI_EP_PROGRAM", mode)
        if abort:
            monkeypatch.setenv("ORTMI_EP_PROGRAM_ABORT", str(abort))
        else:
            monkeypatch.delenv("ORTMI_EP_PROGRAM_ABORT", raising=False)
        r = dec.DecoderRunner(cfg, w, cap=64, max_prompt=32)
        r.prefill(prompt)
        toks, logits = [int(r.next_id.item())], []
        for _ in range(6):
            r.decode_step()
            logits.append(host(r.logits[0, :1])[0])
            toks.append(int(r.next_id.item()))
        r.session.close()
        return toks, logits

    base_toks, base_logits = run(0, "1")
    toks, logits = run(3, "1")
    assert toks == base_toks
    for i, (a, b) in enumerate(zip(logits, base_logits)):
        err = float(np.abs(a - b).max())
        if i < 2:  # before the abort: the same program launches, bit for bit
            assert err == 0.0, f"step {i}: {err}"
        else:      # the op path's step (and its K/V row) from then on: fp16 tolerance
            assert err <= 2.0 ** -7 * max(1.0, float(np.abs(b).max())), f"step {i}: {err}"
    with pytest.raises(RuntimeError, match="decode program failed"):
        run(3, "require")


def test_ep_decoder_with_declared_norm_stats(ortmi, oracle, dec, monkeypatch):
    """A decoder whose SkipSimplifiedLayerNormalization nodes declare their mean and
    inv_std_var outputs, read by nothing (the transformers.js / Mobius export form,
    claimed as rust/src/ops/norm.rs:586-594 claims it): the graph stays one fused node,
    its one-token steps run as the decode program (ORTMI_EP_PROGRAM=require), and the
    greedy tokens pass the strict teacher-forced check against the oracle."""
    monkeypatch.setenv("ORTMI_EP_PROGRAM", "require")
    cfg = _small_cfg(dec, 128)
    w = dec.make_weights(cfg, seed=81)
    runner = dec.DecoderRunner(cfg, w, cap=64, max_prompt=32, norm_stats=True)
    assert len(runner.session.partitions()) == 1
    assert all(runner.session.claimed(i) for i in range(runner.graph.n_nodes))
    prompt = np.random.default_rng(82).integers(0, cfg.vocab, size=15).tolist()
    rows = _teacher_forced_check(oracle, runner, cfg, w, prompt, steps=8)
    _assert_greedy_strict(rows, "decoder with declared norm stats")
