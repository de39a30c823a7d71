"""The one-launch decode step (ortmi_decoder_decode_step) against the op-by-op EP
path and the oracle.

Each decode step runs both ways on the same KV cache: the EP graph (one kernel per
fused op) and the decode program (one launch). They round at the same
op boundaries but sum in different orders, so logits are compared within the fp16
tolerance carried through the layers, the appended K/V rows within one fp16 ULP of
the rows' scale, and the program's greedy token must be the argmax of its own
logits. At full size the program's tokens are checked teacher-forced against the
oracle with the strict rule of the decoder tests (no agreement quota).
"""

from __future__ import annotations

from importlib import import_module

import numpy as np
import pytest
from test_gpu_ep import _assert_greedy_strict
from test_gpu_ops import host

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dec(ortmi):
    return import_module(ortmi.__name__ + ".decoder")


@pytest.fixture(scope="module")
def dprog(ortmi):
    return import_module(ortmi.__name__ + ".decode_program")


def _step_both(runner, prog, length):
    """One decode step through the EP and, on the same KV cache, through the program.
    Returns (ep logits, program logits, ep token, program token, per-layer max |K/V
    row diff|); the cache ends up holding the program's new rows."""
    import torch

    tok = runner.next_id.clone().view(1)
    snap = [(k.clone(), v.clone()) for k, v in runner.kv]
    runner.decode_step()
    torch.cuda.synchronize()
    ep_logits = host(runner.logits[0, 0])
    ep_tok = int(runner.next_id.item())
    ep_rows = [(k[:, :, length].float().clone(), v[:, :, length].float().clone())
               for k, v in runner.kv]
    for (k, v), (ks, vs) in zip(runner.kv, snap):
        k.copy_(ks)
        v.copy_(vs)
    prog.total.fill_(length + 1)
    prog.step(token=tok, total=prog.total)
    torch.cuda.synchronize()
    assert int(prog.status.item()) == 0, f"decode program status {int(prog.status.item())}"
    rows = [(k[:, :, length].float(), v[:, :, length].float()) for k, v in runner.kv]
    kv_diff = max(float(torch.max(torch.abs(a - b)).item())
                  for (ka, va), (kb, vb) in zip(rows, ep_rows) for a, b in ((ka, kb), (va, vb)))
    runner.next_id.copy_(prog.next_id.view(1, 1))
    return ep_logits, host(prog.logits), ep_tok, int(prog.next_id.item()), kv_diff


@pytest.mark.parametrize("shape", [
    dict(G=2),
    dict(G=6),
    # head 64 (16 query heads over 4 KV heads, hidden 1024)
    dict(G=4, heads=16, kv_heads=4, head_dim=64, hidden=1024, inter=2816),
    # the Qwen2.5-0.5B layout: hidden 896 (not a multiple of 256), head 64, 14/2 heads
    dict(G=7, heads=14, kv_heads=2, head_dim=64, hidden=896, inter=4864),
    # the Llama-3.2-1B layout: hidden 2048, 32/8 heads of 64, SwiGLU 8192 (two down
    # rows per wave, gate/up rows beyond the prefetched ones read in the phase)
    dict(G=4, heads=32, kv_heads=8, head_dim=64, hidden=2048, inter=8192),
    # the Phi-4-mini layout: hidden 3072, 24/8 heads of 128, SwiGLU 8192 (6 chunks per
    # lane, one prefetched gate/up group); a 400-row cache asks for 3 key splits and
    # gets 2, the most that leave each projection workgroup at most 16 down rows
    dict(G=3, heads=24, kv_heads=8, head_dim=128, hidden=3072, inter=8192, cap=400),
    # the same layout with one key split (a 64-row cache)
    dict(G=3, heads=24, kv_heads=8, head_dim=128, hidden=3072, inter=8192),
    # the Phi-3.5-mini layout: 32/32 heads of 96 (16-lane key rows, 4 lanes idle),
    # 9216 QKV rows (a second QKV group per wave in registers), one key split
    dict(G=1, heads=32, kv_heads=32, head_dim=96, hidden=3072, inter=8192),
    # the same with two key splits (a 400-row cache)
    dict(G=1, heads=32, kv_heads=32, head_dim=96, hidden=3072, inter=8192, cap=400),
    # head 96 with 4 query heads per KV head at hidden 1536
    dict(G=4, heads=16, kv_heads=4, head_dim=96, hidden=1536, inter=4096),
])
def test_decode_program_matches_ep_steps(ortmi, dec, dprog, monkeypatch, shape):
    """2-layer decoders (head 128 with G query heads per KV head; head 64 at hidden
    1024 and at the Qwen2.5-0.5B and Llama-3.2-1B layouts; the Phi-4-mini layout at
    hidden 3072): 10 decode steps after a 19-token prompt, the program against the
    EP's op-by-op path (ORTMI_EP_PROGRAM=0) on the same cache."""
    monkeypatch.setenv("ORTMI_EP_PROGRAM", "0")
    G = shape["G"]
    H = shape.get("heads", 2 * G)
    hd = shape.get("head_dim", 128)
    cfg = dec.DecoderConfig(layers=2, hidden=shape.get("hidden", H * 128), heads=H,
                            kv_heads=shape.get("kv_heads", 2), head_dim=hd,
                            inter=shape.get("inter", 512), vocab=4096, max_pos=512)
    w = dec.make_weights(cfg, seed=50 + G + hd)
    cap = shape.get("cap", 64)
    runner = dec.DecoderRunner(cfg, w, cap=cap, max_prompt=32)
    prog = dprog.DecodeProgram(cfg, w, runner.kv, cap)
    prompt = np.random.default_rng(G).integers(0, cfg.vocab, size=19)
    runner.reset()
    runner.prefill(prompt)
    length = len(prompt)
    for step in range(10):
        el, pl, et, pt, kvd = _step_both(runner, prog, length)
        runner.length = length + 1
        length += 1
        scale = float(np.abs(el).max())
        err = float(np.abs(el - pl).max())
        print(f"G={G} hd={hd} step {step}: max |logit diff| {err:.3e} (|logit| up to {scale:.2f}), "
              f"K/V row diff {kvd:.3e}, tokens ep {et} program {pt}", flush=True)
        assert np.isfinite(pl).all()
        assert pt == int(np.argmax(pl)), "program token is not the argmax of its logits"
        assert err <= 2.0 ** -7 * max(1.0, scale)
        assert kvd <= 2.0 ** -7 * 4


@pytest.mark.parametrize("layout", [
    dict(heads=24, kv_heads=8, head_dim=128, vocab=200064),  # Phi-4-mini
    dict(heads=32, kv_heads=32, head_dim=96, vocab=32064),  # Phi-3.5-mini
])
def test_decode_program_wide_layout_long_context(ortmi, dec, dprog, monkeypatch, layout):
    """The Phi-4-mini layout (hidden 3072, 24/8 heads of 128, SwiGLU 8192, vocab
    200064) and the Phi-3.5-mini layout (32/32 heads of 96, vocab 32064) with 4
    layers: a 512-token prompt, then 8 decode steps teacher-forced against the op
    path on the same cache. Two key splits of about 260 keys take the register ring
    past the LDS-resident keys, and at Phi-4-mini's vocabulary each wave streams
    about 25 lm_head row groups through its two-entry ring. A token may differ only
    where the op path's top two logits lie within the logit tolerance."""
    monkeypatch.setenv("ORTMI_EP_PROGRAM", "0")
    cfg = dec.DecoderConfig(layers=4, hidden=3072, inter=8192, max_pos=1024, **layout)
    w = dec.make_weights(cfg, seed=8)
    cap = 640
    runner = dec.DecoderRunner(cfg, w, cap=cap, max_prompt=512)
    prog = dprog.DecodeProgram(cfg, w, runner.kv, cap)
    prompt = np.random.default_rng(9).integers(0, cfg.vocab, size=512)
    runner.reset()
    runner.prefill(prompt)
    length = len(prompt)
    for step in range(8):
        el, pl, et, pt, kvd = _step_both(runner, prog, length)
        runner.length = length + 1
        length += 1
        scale = float(np.abs(el).max())
        err = float(np.abs(el - pl).max())
        tol = 2.0 ** -7 * max(1.0, scale)
        top2 = np.sort(el.astype(np.float32))[-2:]
        margin = float(top2[1] - top2[0])
        print(f"step {step}: max |logit diff| {err:.3e} (|logit| up to {scale:.2f}), K/V row diff "
              f"{kvd:.3e}, tokens ep {et} program {pt}, op-path top-2 margin {margin:.4f}", flush=True)
        assert np.isfinite(pl).all()
        assert pt == int(np.argmax(pl)), "program token is not the argmax of its logits"
        assert err <= tol
        assert kvd <= 2.0 ** -7 * 4
        assert pt == et or margin <= 2 * tol


def test_decode_program_full_size_greedy_strict(ortmi, oracle, dec, dprog, capsys):
    """The 28-layer decoder: 512-token prompt through the EP, then 128 greedy steps
    through the decode program; every token teacher-forced against the oracle."""
    import time

    import torch

    cfg = dec.DecoderConfig()
    w = dec.make_weights(cfg, seed=4)
    P, steps = 512, 128
    runner = dec.DecoderRunner(cfg, w, cap=P + steps, max_prompt=P)
    prog = dprog.DecodeProgram(cfg, w, runner.kv, P + steps)
    prompt = np.random.default_rng(44).integers(0, cfg.vocab, size=P)
    runner.reset()
    runner.prefill(prompt)
    gpu = [host(runner.logits[0, P - 1])]
    toks = [int(runner.next_id.item())]
    prog.next_id.copy_(runner.next_id.view(1))
    for i in range(steps):
        prog.total.fill_(P + i + 1)
        prog.step()
        torch.cuda.synchronize()
        assert int(prog.status.item()) == 0
        gpu.append(host(prog.logits))
        toks.append(int(prog.next_id.item()))
    print(f"program tokens {toks[:8]} ... ({len(toks)})", flush=True)
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
    ties, worst = _assert_greedy_strict(list(zip(gpu, ref, toks)), "decode program 512+128")
    with capsys.disabled():  # the near-tie count belongs in the run's own output
        print(f"\ndecode program 512+128: {len(toks) - len(ties)} of {len(toks)} tokens equal "
              f"the oracle's argmax, near ties {len(ties)} {ties}, max |logit diff| "
              f"{worst:.1f} fp16 ULPs of the row max", flush=True)


def test_decode_program_abort_word(ortmi, dec, dprog):
    """A launch aborted before it starts (its launch index + 1 written to the
    workspace's abort word by the host) reads and writes nothing: status stays -1,
    the KV caches, logits and next id are bit-identical to before, and every
    workgroup exits normally. The next launch is not affected: it completes with
    status 0 and gives the bit-identical results of the same step run again from the
    same cache."""
    import torch

    cfg = dec.DecoderConfig(layers=2, hidden=768, heads=6, kv_heads=2, head_dim=128, inter=512,
                            vocab=4096, max_pos=512)
    w = dec.make_weights(cfg, seed=61)
    runner = dec.DecoderRunner(cfg, w, cap=64, max_prompt=32)
    prog = dprog.DecodeProgram(cfg, w, runner.kv, 64)
    prompt = np.random.default_rng(62).integers(0, cfg.vocab, size=17)
    runner.reset()
    runner.prefill(prompt)
    tok = runner.next_id.clone().view(1)
    prog.total.fill_(len(prompt) + 1)
    prog.logits.fill_(float("nan"))
    prog.next_id.fill_(-5)
    torch.cuda.synchronize()
    snap = [(k.clone(), v.clone()) for k, v in runner.kv]
    prog.abort_next()
    prog.step(token=tok, total=prog.total)
    torch.cuda.synchronize()
    assert int(prog.status.item()) == -1
    assert torch.isnan(prog.logits).all() and int(prog.next_id.item()) == -5
    for (k, v), (ks, vs) in zip(runner.kv, snap):
        assert torch.equal(k, ks) and torch.equal(v, vs)
    results = []
    for _ in range(2):
        for (k, v), (ks, vs) in zip(runner.kv, snap):
            k.copy_(ks)
            v.copy_(vs)
        prog.step(token=tok, total=prog.total)
        torch.cuda.synchronize()
        assert int(prog.status.item()) == 0
        results.append((prog.logits.clone(), int(prog.next_id.item()),
                        [(k.clone(), v.clone()) for k, v in runner.kv]))
    (l0, t0, kv0), (l1, t1, kv1) = results
    assert torch.equal(l0, l1) and t0 == t1 == int(torch.argmax(l0.float()).item())
    for (a, b), (c, d) in zip(kv0, kv1):
        assert torch.equal(a, c) and torch.equal(b, d)
