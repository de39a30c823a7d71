"""Independent numpy restatements used to pin the C oracle (test infrastructure).

These follow the numpy references in the reference repository's own tests,
written here in vectorised numpy (a different code path from oracle.c):
  * gqa_ref      - tests/ops/test_gqa11.py:98-112 (repeat heads, causal mask,
                   softmax) plus RoPE per tests/ops/test_paged_attention.py:29-47;
  * paged_ref    - tests/ops/test_paged_attention.py:63-143 (_paged_ref);
  * rms_norm_ref - tests/ops/_models.py:176-177 (np_rms_norm);
  * rotary caches - tests/ops/_models.py:180-185 (base parameterised);
  * dequant_ref  - unpacks with numpy bit operations, independent of oracle.c.
"""

from __future__ import annotations

import math

import numpy as np


def dequant_ref(B, scales, zp, N, K, bits, block):
    nb = (K + block - 1) // block
    B = np.asarray(B, np.uint8).reshape(N, nb, block * bits // 8)
    if bits == 4:
        q = np.stack([B & 0x0F, B >> 4], axis=-1).reshape(N, nb * block)
    else:
        q = B.reshape(N, nb * block)
    if zp is None:
        z = np.full((N, nb), 1 << (bits - 1), np.int32)
    elif bits == 4:
        zc = (nb + 1) // 2
        zb = np.asarray(zp, np.uint8).reshape(N, zc)
        z = np.stack([zb & 0x0F, zb >> 4], axis=-1).reshape(N, 2 * zc)[:, :nb].astype(np.int32)
    else:
        z = np.asarray(zp, np.uint8).reshape(N, nb).astype(np.int32)
    s = np.asarray(scales, np.float64).reshape(N, nb)
    w = (q.astype(np.int32) - np.repeat(z, block, axis=1)) * np.repeat(s, block, axis=1)
    return w[:, :K]


def rotary_caches(max_seq, rotary_dim, base=10000.0):
    half = rotary_dim // 2
    inv_freq = 1.0 / (base ** (np.arange(0, half, dtype=np.float64) / half))
    ang = np.arange(max_seq, dtype=np.float64)[:, None] * inv_freq[None, :]
    return np.cos(ang), np.sin(ang)


def rotate_half(x, interleaved):
    if not interleaved:
        d = x.shape[-1] // 2
        return np.concatenate([-x[..., d:], x[..., :d]], axis=-1)
    out = np.empty_like(x)
    out[..., 0::2] = -x[..., 1::2]
    out[..., 1::2] = x[..., 0::2]
    return out


def apply_rope(x, cos, sin, pos, interleaved, offset=0):
    """x [..., seq, heads, d]; rotates dims [offset, offset + 2*half)."""
    half = cos.shape[-1]
    c, s = cos[pos], sin[pos]
    if not interleaved:
        c = np.concatenate([c, c], axis=-1)
        s = np.concatenate([s, s], axis=-1)
    else:
        c = np.repeat(c, 2, axis=-1)
        s = np.repeat(s, 2, axis=-1)
    out = np.array(x, dtype=np.float64, copy=True)
    seg = out[..., offset:offset + 2 * half]
    out[..., offset:offset + 2 * half] = seg * c[:, None, :] + rotate_half(seg, interleaved) * s[:, None, :]
    return out


def gqa_ref(q, k, v, pk, pv, total, H, KV, cos=None, sin=None, interleaved=False, scale=None):
    """Dense GQA: returns (out [B,S,H*hd], present_k, present_v) in float64."""
    q, k, v = (np.asarray(a, np.float64) for a in (q, k, v))
    pk, pv = np.asarray(pk, np.float64), np.asarray(pv, np.float64)
    B, S, _ = q.shape
    cap, hd = pk.shape[2], pk.shape[3]
    vp = total - S
    shared = 0 <= vp <= cap and cap > vp
    if not (0 <= vp <= cap):
        vp = cap
    qh = q.reshape(B, S, H, hd)
    kh = k.reshape(B, S, KV, hd)
    vh = v.reshape(B, S, KV, hd)
    if cos is not None:
        pos = np.arange(vp, vp + S)
        qh = np.stack([apply_rope(qh[b], cos, sin, pos, interleaved) for b in range(B)])
        kh = np.stack([apply_rope(kh[b], cos, sin, pos, interleaved) for b in range(B)])
    kh = kh.transpose(0, 2, 1, 3)
    vh = vh.transpose(0, 2, 1, 3)
    if shared:
        present_k, present_v = pk.copy(), pv.copy()
        present_k[:, :, vp:vp + S] = kh
        present_v[:, :, vp:vp + S] = vh
    else:
        present_k = np.concatenate([pk, kh], axis=2)
        present_v = np.concatenate([pv, vh], axis=2)
    nk = vp + S
    keys = np.repeat(present_k[:, :, :nk], H // KV, axis=1)
    vals = np.repeat(present_v[:, :, :nk], H // KV, axis=1)
    sc = scale if scale else 1.0 / math.sqrt(hd)
    scores = np.matmul(qh.transpose(0, 2, 1, 3), keys.transpose(0, 1, 3, 2)) * sc
    causal = np.arange(nk)[None, :] <= (vp + np.arange(S))[:, None]
    scores = np.where(causal[None, None], scores, -np.inf)
    probs = np.exp(scores - scores.max(axis=-1, keepdims=True))
    probs /= probs.sum(axis=-1, keepdims=True)
    out = np.matmul(probs, vals).transpose(0, 2, 1, 3).reshape(B, S, H * hd)
    return out, present_k, present_v


def paged_ref(q, k, v, kc, vc, cum, past, bt, H, KV, d, cos=None, sin=None, interleaved=0,
              slot_mapping=None, head_sink=None, q_norm=None, k_norm=None, norm_eps=1e-6,
              rotary_offset=0, vd=None, scale=None):
    """Restatement of _paged_ref; v/vc None = LATENT (values are the first vd key dims)."""
    batch = len(cum) - 1
    vd = vd or d
    sc = scale if scale else 1.0 / math.sqrt(d)
    out = np.zeros((q.shape[0], H * vd), np.float64)
    block_size = kc.shape[1]
    kc = np.array(kc, np.float64, copy=True)
    latent = v is None
    vc = None if latent else np.array(vc, np.float64, copy=True)
    g = H // KV
    for b in range(batch):
        s0, s1 = int(cum[b]), int(cum[b + 1])
        nq = s1 - s0
        if nq == 0:
            continue
        pastb = int(past[b])
        total = pastb + nq
        qb = np.asarray(q[s0:s1], np.float64).reshape(nq, H, d)
        kb = np.asarray(k[s0:s1], np.float64).reshape(nq, KV, d)
        vb = None if latent else np.asarray(v[s0:s1], np.float64).reshape(nq, KV, vd)
        if q_norm is not None:
            qb = qb / np.sqrt(np.mean(qb * qb, axis=-1, keepdims=True) + norm_eps) * q_norm
            kb = kb / np.sqrt(np.mean(kb * kb, axis=-1, keepdims=True) + norm_eps) * k_norm
        if cos is not None:
            pos = np.arange(pastb, total)
            qb = apply_rope(qb, cos, sin, pos, interleaved, rotary_offset)
            kb = apply_rope(kb, cos, sin, pos, interleaved, rotary_offset)
        if latent:
            vb = kb[..., :vd]
        for i in range(nq):
            p = pastb + i
            if slot_mapping is None:
                phys, off = int(bt[b, p // block_size]), p % block_size
            else:
                slot = int(slot_mapping[s0 + i])
                if slot < 0:
                    continue
                phys, off = divmod(slot, block_size)
            kc[phys, off] = kb[i]
            if not latent:
                vc[phys, off] = vb[i]
        keys = np.zeros((total, KV, d))
        vals = np.zeros((total, KV, vd))
        for p in range(total):
            if p < pastb:
                phys, off = int(bt[b, p // block_size]), p % block_size
                keys[p] = kc[phys, off]
                vals[p] = kc[phys, off][..., :vd] if latent else vc[phys, off]
            else:
                keys[p], vals[p] = kb[p - pastb], vb[p - pastb]
        keys, vals = np.repeat(keys, g, 1), np.repeat(vals, g, 1)
        qh, kh, vh = qb.transpose(1, 0, 2), keys.transpose(1, 0, 2), vals.transpose(1, 0, 2)
        scores = np.einsum("hqd,hkd->hqk", qh, kh) * sc
        col = np.arange(total)[None, :]
        row = (pastb + np.arange(nq))[:, None]
        scores = np.where((col > row)[None], -np.inf, scores)
        if head_sink is None:
            scores -= scores.max(-1, keepdims=True)
            e = np.exp(scores)
            attn = e / e.sum(-1, keepdims=True)
        else:
            hs = np.asarray(head_sink, np.float64)
            mx = np.maximum(scores.max(-1, keepdims=True), hs[:, None, None])
            e = np.exp(scores - mx)
            attn = e / (e.sum(-1, keepdims=True) + np.exp(hs[:, None, None] - mx))
        out[s0:s1] = np.einsum("hqk,hkd->hqd", attn, vh).transpose(1, 0, 2).reshape(nq, H * vd)
    return out, kc, vc


def rms_norm_ref(x, scale, eps=1e-6):
    x = np.asarray(x, np.float64)
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * np.asarray(scale, np.float64)


def max_ulp_f16(got, want):
    """Max distance in fp16 ULPs (of the reference value's binade)."""
    want = np.asarray(want, np.float64)
    got = np.asarray(got, np.float64)
    exp = np.floor(np.log2(np.maximum(np.abs(want), 2.0 ** -14)))
    ulp = 2.0 ** (exp - 10)
    return float(np.max(np.abs(got - want) / ulp)) if want.size else 0.0
