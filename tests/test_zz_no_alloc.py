"""The no-allocation GroupQueryAttention entry point against the workspace one.

ortmi_group_query_attention_noalloc runs the same kernels as
ortmi_group_query_attention with the library's fixed per-GPU scratch in place of a
caller-owned workspace. Both are called through the C ABI on the same inputs and
their outputs and present caches must be bit-identical. Two no-alloc calls run in
a row, the second on a smaller problem, so a stale scratch from the first call
would show. A problem whose workspace exceeds the scratch is rejected on the host.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

F16 = 10


def _problem(rng, B, S, H, KV, hd, cap, total):
    import torch

    f = lambda *s: torch.from_numpy(rng.standard_normal(s).astype(np.float16)).cuda()  # noqa: E731
    q, k, v = f(B, S, H * hd), f(B, S, KV * hd), f(B, S, KV * hd)
    pk, pv = f(B, KV, cap, hd), f(B, KV, cap, hd)
    half = hd // 2
    inv = 1.0 / (1e4 ** (np.arange(half) / half))
    ang = np.arange(8192)[:, None] * inv[None, :]
    cos = torch.from_numpy(np.cos(ang).astype(np.float16)).cuda()
    sin = torch.from_numpy(np.sin(ang).astype(np.float16)).cuda()
    return dict(q=q, k=k, v=v, pk=pk, pv=pv, cos=cos, sin=sin, B=B, S=S, H=H, KV=KV, hd=hd,
                cap=cap, total=total)


def _present_cap(p):
    vp = p["total"] - p["S"]
    shared = 0 <= vp <= p["cap"] and p["cap"] > vp
    return p["cap"] if shared else p["cap"] + p["S"]


def _run(lib, p, noalloc):
    import torch

    ptr = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    B, S, H, KV, hd = p["B"], p["S"], p["H"], p["KV"], p["hd"]
    pcap = _present_cap(p)
    out = torch.full((B, S, H * hd), float("nan"), dtype=torch.float16, device="cuda")
    prk = torch.full((B, KV, pcap, hd), float("nan"), dtype=torch.float16, device="cuda")
    prv = torch.full_like(prk, float("nan"))
    if pcap == p["cap"]:  # shared contract: present starts as a copy of past
        prk.copy_(p["pk"])
        prv.copy_(p["pv"])
    common = [ptr(p["q"]), ptr(p["k"]), ptr(p["v"]), ptr(p["pk"]), ptr(p["pv"]), p["cap"],
              p["total"], ptr(p["cos"]), ptr(p["sin"]), hd // 2, 8192, ptr(out), ptr(prk),
              ptr(prv), B, S, H, KV, hd, 0.0, 0, F16]
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    if noalloc:
        rc = lib.ortmi_group_query_attention_noalloc(*common, st)
    else:
        nkeys = p["total"] if 0 <= p["total"] - S <= p["cap"] else p["cap"] + S
        wsb = lib.ortmi_group_query_attention_workspace_size(B, S, H, hd, nkeys)
        ws = torch.empty(wsb, dtype=torch.uint8, device="cuda")
        rc = lib.ortmi_group_query_attention(*common, ptr(ws), wsb, st)
    assert rc == 0, lib.ortmi_last_error().decode()
    torch.cuda.synchronize()
    return out.cpu().numpy(), prk.cpu().numpy(), prv.cpu().numpy()


def _same(a, b, what):
    a16, b16 = a.view(np.uint16), b.view(np.uint16)
    assert np.array_equal(a16, b16), f"{what}: {np.count_nonzero(a16 != b16)} elements differ"


@pytest.mark.parametrize("first,second", [
    # decode, growing contract, 4K context -> decode, shared contract, 640-row buffer
    ((8, 1, 32, 8, 128, 4096, 4097), (1, 1, 12, 2, 128, 640, 300)),
    # prefill 256 tokens over a 512-row past (splits, merge) -> prefill 40 tokens, hd 64
    ((2, 256, 32, 8, 128, 512, 768), (1, 40, 8, 2, 64, 96, 40)),
])
def test_noalloc_matches_workspace_entry(ortmi, first, second):
    lib = ortmi.load_kernels()
    rng = np.random.default_rng(7)
    for shape in (first, second):
        B, S, H, KV, hd, cap, total = shape
        print(f"no-alloc GQA B={B} S={S} H={H} KV={KV} hd={hd} cap={cap} total={total}",
              flush=True)
        p = _problem(rng, B, S, H, KV, hd, cap, total)
        ref = _run(lib, p, noalloc=False)
        got = _run(lib, p, noalloc=True)
        for r, g, what in zip(ref, got, ("output", "present_key", "present_value")):
            _same(g, r, what)
        assert np.isfinite(got[0]).all()


def test_noalloc_rejects_oversize_on_host(ortmi):
    lib = ortmi.load_kernels()
    cap = lib.ortmi_group_query_attention_noalloc_max_workspace()
    assert cap == 32 << 20
    # 64 sequences x 1024 prompt tokens x 32 heads: the workspace is far above 32 MiB.
    need = lib.ortmi_group_query_attention_workspace_size(64, 1024, 32, 128, 1024)
    assert need > cap
    p = ctypes.c_void_p(256)
    rc = lib.ortmi_group_query_attention_noalloc(p, p, p, None, None, 0, 1024, None, None, 0, 0,
                                                 p, p, p, 64, 1024, 32, 8, 128, 0.0, 0, F16, None)
    assert rc == 3 and "scratch" in lib.ortmi_last_error().decode()
