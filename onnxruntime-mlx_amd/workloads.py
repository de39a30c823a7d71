"""Seeded synthetic inputs for the benchmark configurations (numpy, host side).

Each generator draws its arrays in the order listed, from numpy default_rng(seed),
so CPU and GPU runs see byte-identical inputs.
"""

from __future__ import annotations

import numpy as np


def mnb_gemv_config(seed: int = 1, K: int = 4096, N: int = 11008, block: int = 32):
    """Single MatMulNBits node, bits 4, block 32, K=4096, N=11008, fp32.
    A ~N(0,1) [1,K]; B uint8 [N, K/32, 16] with uniform nibbles; scales
    |N(0,0.02)| + 1e-4 [N*K/32]; zero points all 8 (bytes 0x88)."""
    rng = np.random.default_rng(seed)
    nb = K // block
    A = rng.standard_normal((1, K)).astype(np.float32)
    B = rng.integers(0, 256, size=(N, nb, block // 2), dtype=np.uint8)
    s = (np.abs(rng.standard_normal(N * nb) * 0.02) + 1e-4).astype(np.float32)
    zp = np.full(N * ((nb + 1) // 2), 0x88, np.uint8)
    return A, B, s, zp


def mnb_gemm_config(seed: int = 2, M: int = 512, K: int = 4096, N: int = 4096, block: int = 32):
    """MatMulNBits prefill GEMM: A fp16 [M,K] ~N(0,1), N=4096, block 32, fp16 scales
    |N(0,0.02)| + 1e-4, zero points uniform in 0..15 (packed)."""
    rng = np.random.default_rng(seed)
    nb = K // block
    A = rng.standard_normal((M, K)).astype(np.float16)
    B = rng.integers(0, 256, size=(N, nb, block // 2), dtype=np.uint8)
    s = (np.abs(rng.standard_normal(N * nb) * 0.02) + 1e-4).astype(np.float16)
    z = rng.integers(0, 16, size=(N, (nb + 1) // 2 * 2), dtype=np.uint8)
    zp = (z[:, 0::2] | (z[:, 1::2] << 4)).astype(np.uint8).reshape(-1)
    return A, B, s, zp


def rotary_cache(max_pos: int, head_size: int, base: float, dtype=np.float16):
    half = head_size // 2
    inv = 1.0 / (base ** (np.arange(half, dtype=np.float64) / half))
    ang = np.arange(max_pos, dtype=np.float64)[:, None] * inv[None, :]
    return np.cos(ang).astype(dtype), np.sin(ang).astype(dtype)


def gqa_decode_config(seed: int = 3, B: int = 8, H: int = 32, KV: int = 8, hd: int = 128,
                      past: int = 4096):
    """GroupQueryAttention decode step: fp16, past K/V [B,KV,past,hd] ~N(0,1), new
    Q/K/V for one token, seqlens_k = past for all, total = past + 1, rotary
    (non-interleaved) from [8192, hd/2] caches with base 10000."""
    rng = np.random.default_rng(seed)
    pk = rng.standard_normal((B, KV, past, hd)).astype(np.float16)
    pv = rng.standard_normal((B, KV, past, hd)).astype(np.float16)
    q = rng.standard_normal((B, 1, H * hd)).astype(np.float16)
    k = rng.standard_normal((B, 1, KV * hd)).astype(np.float16)
    v = rng.standard_normal((B, 1, KV * hd)).astype(np.float16)
    seqlens = np.full(B, past, np.int32)
    total = past + 1
    cos, sin = rotary_cache(8192, hd, 10000.0)
    return dict(q=q, k=k, v=v, pk=pk, pv=pv, seqlens=seqlens, total=total, cos=cos, sin=sin)


def paged_mixed_config(seed: int = 5, nseq: int = 32, H: int = 32, KV: int = 8, hd: int = 128,
                       blk: int = 16, n_prefill: int = 4, chunk: int = 256, lo: int = 256,
                       hi: int = 8192):
    """PagedAttention mixed batch: contexts U[lo, hi]; the first n_prefill
    sequences prefill `chunk`-token chunks (past = ctx - chunk), the rest decode one
    token (past = ctx - 1). Block size 16, cache sized to the total block count,
    block table = a random permutation of the physical blocks (rows padded with
    block 0). Q/K/V/caches ~N(0,1), fp16, no rotary."""
    rng = np.random.default_rng(seed)
    ctx = rng.integers(lo, hi + 1, size=nseq)
    new = np.array([chunk] * n_prefill + [1] * (nseq - n_prefill))
    past = (ctx - new).astype(np.int32)
    nblocks = [(int(c) + blk - 1) // blk for c in ctx]
    nb = int(sum(nblocks))
    maxb = max(nblocks)
    perm = rng.permutation(nb).astype(np.int32)
    bt = np.zeros((nseq, maxb), np.int32)
    o = 0
    for b, n in enumerate(nblocks):
        bt[b, :n] = perm[o:o + n]
        o += n
    cum = np.concatenate([[0], np.cumsum(new)]).astype(np.int32)
    T = int(cum[-1])
    q = rng.standard_normal((T, H * hd)).astype(np.float16)
    k = rng.standard_normal((T, KV * hd)).astype(np.float16)
    v = rng.standard_normal((T, KV * hd)).astype(np.float16)
    kc = rng.standard_normal((nb, blk, KV, hd)).astype(np.float16)
    vc = rng.standard_normal((nb, blk, KV, hd)).astype(np.float16)
    return dict(q=q, k=k, v=v, kc=kc, vc=vc, cum=cum, past=past, bt=bt, ctx=ctx, new=new,
                H=H, KV=KV, hd=hd, blk=blk)


def paged_work(cfg) -> tuple[int, int]:
    """(algorithmic HBM bytes, flops) of one PagedAttention step over `cfg`."""
    H, KV, hd = cfg["H"], cfg["KV"], cfg["hd"]
    ctx, new = cfg["ctx"].astype(np.int64), cfg["new"].astype(np.int64)
    T = int(new.sum())
    kv_read = int(ctx.sum()) * KV * hd * 2 * 2          # K and V rows, fp16
    kv_write = T * KV * hd * 2 * 2                       # new K/V rows
    qo = T * H * hd * 2 * 2                              # Q read + output write
    # causal: query i of a sequence attends past + i + 1 keys
    keys = 0
    for c, n in zip(ctx, new):
        p = c - n
        keys += int(n * p + n * (n + 1) // 2)
    flops = 4 * H * hd * keys
    return kv_read + kv_write + qo, flops
