"""Python face of the CPU oracle (oracle.c), plus numpy helpers.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, always as the checker (or the timed CPU baseline), never by the
shipped library.

All float inputs are taken as numpy arrays of any float dtype; fp16 inputs are
widened exactly to fp32 before the C code sees them. Results are fp64/fp32 arrays
that the caller rounds to the op dtype.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None


def build() -> str:
    """Compile liboracle.so with the committed Makefile (gcc + OpenMP)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_i32p = ctypes.POINTER(ctypes.c_int32)
_i64p = ctypes.POINTER(ctypes.c_int64)
_i64 = ctypes.c_int64
_int = ctypes.c_int
_flt = ctypes.c_float


def _declare(L: ctypes.CDLL) -> None:
    L.orc_f16_to_f32_n.argtypes = [_u16p, _f32p, _i64]
    L.orc_f32_to_f16_n.argtypes = [_f32p, _u16p, _i64]
    L.orc_mnb_dequant.argtypes = [_u8p, _f32p, _u8p, _i64, _i64, _int, _int, _f32p]
    L.orc_mnb_matmul.argtypes = [_f32p, _u8p, _f32p, _u8p, _i64, _i64, _i64, _int, _int,
                                 _f64p, _int]
    L.orc_rotary.argtypes = [_f32p, _f32p, _int, _int, _int, _int, _i64, _i64, _i64, _i64p,
                             _f32p, _f32p, _int, _int, _int, _int]
    L.orc_rotary.restype = None
    L.orc_gqa_contract.argtypes = [_int, _int, _i64, _i32p, _i64p]
    L.orc_gqa.argtypes = [_f32p, _f32p, _f32p, _f32p, _f32p, _i64, _int, _f32p, _f32p, _int,
                          _int, _int, _int, _int, _int, _int, _flt, _int, _f32p, _f32p, _f32p]
    L.orc_gqa_ex.argtypes = [_f32p, _f32p, _f32p, _f32p, _f32p, _i64, _int, _f32p, _f32p,
                             _int, _int, _int, _int, _int, _int, _int, _flt, _int, _f32p, _f32p,
                             _flt, _f32p, _i64, _i64, _i64, _f32p, _f32p, _f32p]
    L.orc_paged_attention.argtypes = [_f32p, _f32p, _f32p, _f32p, _f32p, _i64, _int, _i32p,
                                      _i32p, _i32p, _int, _int, _f32p, _f32p, _int, _int, _int,
                                      _i32p, _f32p, _f32p, _f32p, _flt, _int, _int, _int, _int,
                                      _flt, _int, _f32p]
    L.orc_rms_norm.argtypes = [_f32p, _f32p, _f32p, _f32p, _i64, _i64, _flt, _int, _f32p,
                               _f32p]
    L.orc_rms_norm.restype = None
    L.orc_mnb_matmul_fast.argtypes = [_f32p, _i64, _u8p, ctypes.c_void_p, _int, _u8p, _i64, _i64,
                                      _int, _f32p, _int]


def _p(a, t):
    if a is None:
        return None
    return a.ctypes.data_as(t)


def _f32(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.float32)


# ------------------------------------------------------------------ fp16 ----
def f16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(bits.shape, np.float32)
    lib().orc_f16_to_f32_n(_p(bits, _u16p), _p(out, _f32p), bits.size)
    return out


def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_f16_n(_p(x, _f32p), _p(out, _u16p), x.size)
    return out


# ------------------------------------------------------------ MatMulNBits ----
def pack_nibbles(vals: np.ndarray) -> np.ndarray:
    """Pack 4-bit values along the last axis, low nibble first.

    Restates the packing the reference's tests feed MatMulNBits
    (tests/ops/test_matmulnbits_asym.py:23-27)."""
    vals = np.asarray(vals, dtype=np.uint8)
    return (vals[..., 0::2] | (vals[..., 1::2] << 4)).astype(np.uint8)


def pack_zero_points(zp: np.ndarray, bits: int) -> np.ndarray:
    """[N, nb] zero points -> the ORT input layout (tests/ops/test_matmulnbits_asym.py:48-58):
    4-bit values are padded to an even count per row and packed, 8-bit ones kept."""
    zp = np.asarray(zp, dtype=np.uint8)
    if bits == 8:
        return zp.reshape(-1).copy()
    if zp.shape[1] % 2:
        zp = np.concatenate([zp, np.zeros((zp.shape[0], 1), np.uint8)], axis=1)
    return pack_nibbles(zp).reshape(-1)


def mnb_dequant(B, scales, zp, N, K, bits=4, block=32) -> np.ndarray:
    B = np.ascontiguousarray(B, dtype=np.uint8)
    s = _f32(scales)
    z = None if zp is None else np.ascontiguousarray(zp, dtype=np.uint8)
    W = np.empty((N, K), np.float32)
    rc = lib().orc_mnb_dequant(_p(B, _u8p), _p(s, _f32p), _p(z, _u8p), N, K, bits, block,
                               _p(W, _f32p))
    if rc:
        raise ValueError("oracle: unsupported MatMulNBits form")
    return W


def mnb_matmul(A, B, scales, zp, N, K, bits=4, block=32, nthreads=0) -> np.ndarray:
    A2 = _f32(A).reshape(-1, K)
    B = np.ascontiguousarray(B, dtype=np.uint8)
    s = _f32(scales)
    z = None if zp is None else np.ascontiguousarray(zp, dtype=np.uint8)
    Y = np.empty((A2.shape[0], N), np.float64)
    rc = lib().orc_mnb_matmul(_p(A2, _f32p), _p(B, _u8p), _p(s, _f32p), _p(z, _u8p),
                              A2.shape[0], N, K, bits, block, _p(Y, _f64p), nthreads)
    if rc:
        raise ValueError("oracle: unsupported MatMulNBits form")
    return Y.reshape(tuple(np.shape(A)[:-1]) + (N,))


def mnb_matmul_fast(A, B, scales, zp, N, K, block=32, nthreads=0) -> np.ndarray:
    """The CPU baseline's int4 MatMulNBits (fast.c): fp32 accumulation with
    AVX2/FMA, scales fp32 or fp16 (used as stored). A [..., K]; returns float32
    [..., N]. Timing baseline only: the parity reference is mnb_matmul."""
    A2 = _f32(A).reshape(-1, K)
    B = np.ascontiguousarray(B, dtype=np.uint8)
    s = np.ascontiguousarray(scales)
    if s.dtype not in (np.float32, np.float16):
        s = s.astype(np.float32)
    z = None if zp is None else np.ascontiguousarray(zp, dtype=np.uint8)
    Y = np.empty((A2.shape[0], N), np.float32)
    rc = lib().orc_mnb_matmul_fast(_p(A2, _f32p), A2.shape[0], _p(B, _u8p),
                                   s.ctypes.data_as(ctypes.c_void_p), int(s.dtype == np.float16),
                                   _p(z, _u8p), N, K, block, _p(Y, _f32p), nthreads)
    if rc:
        raise ValueError("oracle: form outside the fast MatMulNBits (4-bit, block 32-128, AVX2)")
    return Y.reshape(tuple(np.shape(A)[:-1]) + (N,))


def gather_block_quantized(data, scales, zp, indices, block, out_dtype=np.float32) -> np.ndarray:
    """GatherBlockQuantized, 4-bit, gather_axis 0, quantize_axis 1
    (rust/src/ops/quant.rs:1134-1199): rows of the dequantised table
    (q - zp) * scale (the MatMulNBits byte layout with N = rows, K = D), indexed
    with negative ids counting from the end; ids outside [-V, V) give zero rows.
    (q - zp) * scale is formed in fp32 (exact for fp16/bf16 scales), then rounded
    to out_dtype."""
    data = np.asarray(data, np.uint8)
    V, D = data.shape[0], data.shape[1] * 2
    # Rows are D/2 bytes (no padding to whole blocks, unlike MatMulNBits' B): pad
    # them to whole blocks for the dequantisation, which then ignores the padding.
    nb = (D + block - 1) // block
    padded = np.zeros((V, nb * block // 2), np.uint8)
    padded[:, :D // 2] = data
    W = mnb_dequant(padded, np.asarray(scales, np.float32).reshape(-1), zp, V, D, 4, block)
    idx = np.asarray(indices, np.int64).reshape(-1)
    rows = np.where(idx < 0, idx + V, idx)
    ok = (rows >= 0) & (rows < V)
    out = np.zeros((idx.size, D), np.float64)
    out[ok] = W[rows[ok]]
    return out.reshape(tuple(np.shape(indices)) + (D,)).astype(out_dtype)


# ------------------------------------------------------------------ RoPE ----
def rotary(x, rows, cos, sin, interleaved=False, offset=0, round16=False, layout="bsnd",
           num_heads=None):
    """Rotary embedding. x is [B,S,NH*hd] (layout 'bsnd' with num_heads given) or
    [B,NH,S,hd] (layout 'bnsd'); rows[b,s] is the cos/sin cache row of token (b,s)."""
    x = _f32(x)
    cos, sin = _f32(cos), _f32(sin)
    half = cos.shape[-1]
    if layout == "bnsd":
        B, NH, S, hd = x.shape
        sb, ss, sn = NH * S * hd, hd, S * hd
    else:
        B, S, hidden = x.shape
        NH = num_heads
        hd = hidden // NH
        sb, ss, sn = S * hidden, hidden, hd
    rows = np.ascontiguousarray(np.broadcast_to(np.asarray(rows, np.int64), (B, S)))
    y = np.empty_like(x)
    lib().orc_rotary(_p(x, _f32p), _p(y, _f32p), B, S, NH, hd, sb, ss, sn, _p(rows, _i64p),
                     _p(cos, _f32p), _p(sin, _f32p), half, int(interleaved), offset,
                     int(round16))
    return y


# ------------------------------------------------------------------- GQA ----
def gqa_contract(total_seq_len: int, S: int, cap: int):
    vp = ctypes.c_int32(0)
    pcap = ctypes.c_int64(0)
    shared = lib().orc_gqa_contract(total_seq_len, S, cap, ctypes.byref(vp), ctypes.byref(pcap))
    return bool(shared), vp.value, pcap.value


def gqa(q, k, v, past_k, past_v, total_seq_len, num_heads, kv_heads, cos=None, sin=None,
        interleaved=False, scale=0.0, round16=False, q_norm=None, k_norm=None, qk_eps=1e-6,
        bias=None):
    """GroupQueryAttention; returns (out [B,S,H*hd] f32, present_k, present_v, shared).

    q_norm/k_norm: [hd] QK-norm weights; bias: additive mask of rank 4
    [B or 1, H or 1, >= S, >= total] indexed by key position. round16: False/1 = fp16
    rounding when true, 2 = bf16 rounding."""
    q = _f32(q)
    B, S, _ = q.shape
    past_k, past_v = _f32(past_k), _f32(past_v)
    _, KV, cap, hd = past_k.shape
    k, v = _f32(k), _f32(v)
    shared, vp, pcap = gqa_contract(total_seq_len, S, cap)
    out = np.zeros((B, S, num_heads * hd), np.float32)
    pk = np.zeros((B, KV, pcap, hd), np.float32)
    pv = np.zeros((B, KV, pcap, hd), np.float32)
    cos, sin = _f32(cos), _f32(sin)
    half = 0 if cos is None else cos.shape[-1]
    sb = sh = ss = 0
    if bias is not None:
        bias = _f32(bias)
        if bias.ndim != 4 or bias.shape[0] not in (1, B) or bias.shape[1] not in (1, num_heads) \
                or bias.shape[2] < S or bias.shape[3] < vp + S:
            raise ValueError(f"oracle: attention_bias shape {bias.shape} does not cover "
                             f"[{B}, {num_heads}, {S}, {vp + S}]")
        sb = bias.strides[0] // 4 if bias.shape[0] > 1 else 0
        sh = bias.strides[1] // 4 if bias.shape[1] > 1 else 0
        ss = bias.strides[2] // 4
    rc = lib().orc_gqa_ex(_p(q, _f32p), _p(k, _f32p), _p(v, _f32p), _p(past_k, _f32p),
                          _p(past_v, _f32p), cap, total_seq_len, _p(cos, _f32p), _p(sin, _f32p),
                          half, int(interleaved), B, S, num_heads, KV, hd, scale, int(round16),
                          _p(_f32(q_norm), _f32p), _p(_f32(k_norm), _f32p), qk_eps,
                          _p(bias, _f32p), sb, sh, ss, _p(out, _f32p), _p(pk, _f32p),
                          _p(pv, _f32p))
    if rc < 0:
        raise ValueError("oracle: bad GroupQueryAttention arguments")
    return out, pk, pv, shared


def _round_mode(x, mode):
    """Rounds fp32 values to fp16 (mode 1) or bf16 (mode 2, nearest even); mode 0
    keeps them."""
    x = np.ascontiguousarray(x, np.float32)
    if mode == 1:
        return x.astype(np.float16).astype(np.float32)
    if mode == 2:
        b = x.view(np.uint32).astype(np.uint64)
        b = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16) << 16
        return b.astype(np.uint32).view(np.float32)
    return x


def sliding_cache_end(length: int, cap: int, window: int) -> int:
    """Rows a sliding-window cache of capacity `cap` holds after `length` tokens: once
    full it drops its oldest cap - window + 1 rows at a time
    (rust/src/ops/attention.rs:736-745)."""
    gap = cap - window + 1
    if length <= cap:
        return length
    return length - gap * ((length - cap + gap - 1) // gap)


def gqa_sliding(q, k, v, past_k, past_v, seqlens_k, num_heads, kv_heads, window, cos=None,
                sin=None, interleaved=False, scale=0.0, round16=0, q_norm=None, k_norm=None,
                qk_eps=1e-6):
    """GroupQueryAttention with sliding_window_cache = 1, restated from
    rust/src/ops/attention.rs:725-880 (numpy, fp64 products).

    Per batch b: p = max(seqlens_k[b] + 1 - S, 0) tokens precede the new ones, of
    which the cache holds the last before = sliding_cache_end(p) in rows [0, before).
    The working keys are the seed rows past[seed_start:before] followed by the S new
    (RoPE'd at positions p..p+S-1) rows, seed_start = before - kept unless some batch
    keeps fewer rows than its window needs (then 0, the staging form); query i
    attends working key j when seed_rows + i - window < j <= seed_rows + i
    (causal_window_mask, attention.rs:191-219). present = working rows from
    write_start (the staging form drops the seed rows the cache does not keep),
    zero rows after. Returns (out [B,S,H*hd] f32, present_k, present_v) with present
    [B, KV, cap, hd]. round16: 0 fp32, 1 fp16, 2 bf16 rounding of the RoPE/QK-norm
    outputs, as the op materialises them."""
    q = _f32(q)
    B, S, _ = q.shape
    past_k, past_v = _f32(past_k), _f32(past_v)
    _, KV, cap, hd = past_k.shape
    H = num_heads
    G = H // KV
    k = _f32(k).reshape(B, S, KV, hd)
    v = _f32(v).reshape(B, S, KV, hd)
    qh = q.reshape(B, S, H, hd)
    if not 0 < window <= cap:
        raise ValueError("oracle: sliding cache requires 0 < local_window_size <= capacity")
    sc = scale if scale != 0.0 else 1.0 / np.sqrt(hd)
    seq = np.asarray(seqlens_k, np.int64).reshape(-1)

    def qk_norm(x, w):
        if w is None:
            return x
        x64 = x.astype(np.float64)
        inv = 1.0 / np.sqrt((x64 * x64).mean(axis=-1, keepdims=True) + qk_eps)
        return _round_mode((x64 * inv * _f32(w)).astype(np.float32), round16)

    qh = qk_norm(qh, q_norm)
    k = qk_norm(k, k_norm)
    geo = []
    staging = False
    for b in range(B):
        p = max(int(seq[b]) + 1 - S, 0)
        before = sliding_cache_end(p, cap, window)
        after = sliding_cache_end(p + S, cap, window)
        kept = after - S
        staging |= kept < min(p, window - 1)
        geo.append((p, before, after, before - kept))
    out = np.zeros((B, S, H, hd), np.float32)
    pk = np.zeros((B, KV, cap, hd), np.float32)
    pv = np.zeros((B, KV, cap, hd), np.float32)
    for b, (p, before, after, seed_off) in enumerate(geo):
        rows = np.arange(p, p + S)[None, :]
        qb, kb = qh[b:b + 1].reshape(1, S, H * hd), k[b:b + 1].reshape(1, S, KV * hd)
        if cos is not None:
            qb = rotary(qb, rows, cos, sin, interleaved, round16=round16, num_heads=H)
            kb = rotary(kb, rows, cos, sin, interleaved, round16=round16, num_heads=KV)
        qb = qb.reshape(S, H, hd).astype(np.float64)
        kb = kb.reshape(S, KV, hd)
        seed_start = 0 if staging else seed_off
        work_k = np.concatenate([past_k[b, :, seed_start:before], kb.transpose(1, 0, 2)], axis=1)
        work_v = np.concatenate([past_v[b, :, seed_start:before],
                                 v[b].transpose(1, 0, 2)], axis=1)
        seed_rows = before - seed_start
        k_len = seed_rows + S
        j = np.arange(k_len)[None, :]
        qpos = seed_rows + np.arange(S)[:, None]
        allow = (j <= qpos) & (j >= qpos - window + 1)
        for h in range(H):
            kv = h // G
            sco = (qb[:, h] @ work_k[kv].astype(np.float64).T) * sc
            sco = np.where(allow, sco, -np.inf)
            m = sco.max(axis=1, keepdims=True)
            e = np.exp(sco - m)
            out[b, :, h] = (e @ work_v[kv].astype(np.float64)) / e.sum(axis=1, keepdims=True)
        write_start = seed_off if staging else 0
        n = k_len - write_start
        pk[b, :, :n] = work_k[:, write_start:]
        pv[b, :, :n] = work_v[:, write_start:]
    return out.reshape(B, S, H * hd), pk, pv


# -------------------------------------------------------- PagedAttention ----
def paged_attention(q, k, v, kcache, vcache, cum, past, block_table, num_heads, kv_heads,
                    cos=None, sin=None, interleaved=False, rotary_offset=0, slot_mapping=None,
                    head_sink=None, q_norm=None, k_norm=None, qk_eps=1e-6, v_head_size=0,
                    scale=0.0, round16=False):
    """PagedAttention; returns (out [T,H*vhd] f32, kcache', vcache'). v/vcache None = LATENT."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    kc = _f32(kcache).copy()
    vc = None if vcache is None else _f32(vcache).copy()
    nblk, blk, KV, hd = kc.shape
    vhd = v_head_size or hd
    cum = np.ascontiguousarray(cum, np.int32)
    past = np.ascontiguousarray(past, np.int32)
    bt = np.ascontiguousarray(block_table, np.int32)
    batch = cum.shape[0] - 1
    maxb = bt.shape[1] if bt.ndim == 2 else 0
    T = int(cum[-1])
    out = np.zeros((T, num_heads * vhd), np.float32)
    cos, sin = _f32(cos), _f32(sin)
    half = 0 if cos is None else cos.shape[-1]
    sm = None if slot_mapping is None else np.ascontiguousarray(slot_mapping, np.int32)
    rc = lib().orc_paged_attention(
        _p(q, _f32p), _p(k, _f32p), _p(v, _f32p), _p(kc, _f32p), _p(vc, _f32p), nblk, blk,
        _p(cum, _i32p), _p(past, _i32p), _p(bt, _i32p), batch, maxb, _p(cos, _f32p),
        _p(sin, _f32p), half, int(interleaved), rotary_offset, _p(sm, _i32p),
        _p(_f32(head_sink), _f32p), _p(_f32(q_norm), _f32p), _p(_f32(k_norm), _f32p), qk_eps,
        num_heads, KV, hd, vhd, scale, int(round16), _p(out, _f32p))
    if rc:
        raise ValueError("oracle: bad PagedAttention arguments")
    return out, kc, vc


# --------------------------------------------------------------- RMS norm ----
def rms_norm(x, gamma, eps, skip=None, bias=None, round16=False):
    """(Skip)SimplifiedLayerNormalization; returns (y f32, residual f32)."""
    x = _f32(x)
    D = x.shape[-1]
    rows = x.size // D
    y = np.empty_like(x)
    r = np.empty_like(x)
    lib().orc_rms_norm(_p(x, _f32p), _p(_f32(skip), _f32p), _p(_f32(bias), _f32p),
                       _p(_f32(gamma), _f32p), rows, D, eps, int(round16), _p(y, _f32p),
                       _p(r, _f32p))
    return y, r


def round_f16(x) -> np.ndarray:
    """Round to fp16 (RNE) and widen back to fp32."""
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)


# ------------------------------------------------------- int4 decoder -------
def dequant_cache(w, cfg):
    """Every linear layer of a decoder weight dict dequantised once by the C
    restatement (orc_mnb_dequant: (q - 8) * s, exact in fp32) and widened to fp64,
    for decoder_forward(..., wcache=...). About 8 bytes per weight."""
    out = {}
    for key in list(w):
        if key.endswith(".B"):
            name = key[:-2]
            B = w[key]
            N = B.shape[0]
            K = B.shape[1] * cfg.block
            out[name] = mnb_dequant(B, w[name + ".s"], None, N, K, 4, cfg.block).astype(np.float64)
    return out


def _gqa_step_fast(q, k, v, past_k, past_v, total, H, KV, cos, sin):
    """One-token GroupQueryAttention on the shared KV buffer in fp32 numpy (the CPU
    baseline's form of gqa() at S = 1 with non-interleaved rotary over the whole
    head): RoPE of q and the new key at position total - 1, the new K/V row written
    in place, then per KV head softmax(q K^T * scale) V over the total keys."""
    hd = past_k.shape[-1]
    half, pos, G = hd // 2, total - 1, H // KV
    c, s = cos[pos].astype(np.float32), sin[pos].astype(np.float32)

    def rope(x):
        x1, x2 = x[:, :half], x[:, half:]
        return np.concatenate([x1 * c - x2 * s, x1 * s + x2 * c], axis=1)

    qh = round_f16(rope(np.asarray(q, np.float32).reshape(H, hd)))
    past_k[0, :, pos] = round_f16(rope(np.asarray(k, np.float32).reshape(KV, hd)))
    past_v[0, :, pos] = np.asarray(v, np.float32).reshape(KV, hd)
    out = np.empty((H, hd), np.float32)
    for g in range(KV):
        sc = (qh[g * G:(g + 1) * G] @ past_k[0, g, :total].T) * np.float32(1.0 / np.sqrt(hd))
        sc = np.exp(sc - sc.max(axis=1, keepdims=True))
        out[g * G:(g + 1) * G] = (sc @ past_v[0, g, :total]) / sc.sum(axis=1, keepdims=True)
    return round_f16(out).reshape(1, 1, H * hd)


def decoder_forward(w, cfg, ids, past_k, past_v, total, wcache=None, logit_rows=None,
                    fast=False):
    """One forward of the int4 Llama-style decoder graph, op by op in fp16.

    The graph is the ONNX Runtime GenAI q4f16 decoder (op histogram in
    examples/traces/qwen2.5-0.5b-decode.json): Gather -> per layer
    (Skip)SimplifiedLayerNormalization, MatMulNBits q/k/v, GroupQueryAttention
    with rotary on a shared KV buffer, MatMulNBits o, SkipSimplifiedLayerNorm,
    gate/up MatMulNBits, Sigmoid/Mul/Mul, down MatMulNBits -> final
    SkipSimplifiedLayerNorm -> lm_head MatMulNBits. Every op output is rounded
    to fp16, as the fp16 graph stores it.

    w: weight dict (int4 codes [N, K/32, 16], fp16 scales, embed, norms, cos/sin);
    cfg: an object with layers, hidden, heads, kv_heads, head_dim, inter, vocab,
    eps, block; ids: int array [S]; past_k/past_v: per-layer f32 [1, KV, cap, hd]
    arrays, updated in place; total: total sequence length after this call.
    wcache: optional dequant_cache(w, cfg); the linear layers are then fp64 matrix
    products with the cached fp64 weights (the same exact products as the per-row
    C loop, summed in BLAS order). logit_rows: optional row indices of the logits
    to compute (default all S). fast: the linear layers go through the CPU
    baseline's fp32 AVX2 MatMulNBits (fast.c) and one-token attention through
    _gqa_step_fast instead, for timing a CPU decoder; its logits are not a parity
    reference. Returns fp16-rounded logits [rows, vocab] as
    f32.
    """
    r16 = round_f16
    S = len(ids)
    D, H, KV, hd = cfg.hidden, cfg.heads, cfg.kv_heads, cfg.head_dim

    def mm(x, key, N, K):
        if fast:
            return r16(mnb_matmul_fast(x, w[key + ".B"], w[key + ".s"], None, N, K, cfg.block))
        if wcache is not None:
            x2 = np.asarray(x, np.float32).reshape(-1, K).astype(np.float64)
            return r16((x2 @ wcache[key].T).reshape(tuple(np.shape(x)[:-1]) + (N,)))
        return r16(mnb_matmul(x, w[key + ".B"], w[key + ".s"], None, N, K, 4, cfg.block))

    h = w["embed"][np.asarray(ids)].astype(np.float32).reshape(1, S, D)
    cos, sin = w["cos"], w["sin"]
    down, residual = None, h
    for layer in range(cfg.layers):
        p = f"l{layer}"
        if layer == 0:
            x, _ = rms_norm(h, w[p + ".ln1"], cfg.eps, round16=True)
        else:
            x, residual = rms_norm(down, w[p + ".ln1"], cfg.eps, skip=residual, round16=True)
        x = r16(x)
        q = mm(x, p + ".q", H * hd, D)
        k = mm(x, p + ".k", KV * hd, D)
        v = mm(x, p + ".v", KV * hd, D)
        if fast and S == 1:
            out = _gqa_step_fast(q, k, v, past_k[layer], past_v[layer], total, H, KV, cos, sin)
        else:
            out, pk, pv, shared = gqa(q, k, v, past_k[layer], past_v[layer], total, H, KV, cos,
                                      sin, round16=True)
            assert shared, "the decoder runs the shared-buffer KV contract"
            past_k[layer][...] = pk
            past_v[layer][...] = pv
        o = mm(r16(out), p + ".o", D, H * hd)
        x2, residual = rms_norm(o, w[p + ".ln2"], cfg.eps, skip=residual, round16=True)
        x2 = r16(x2)
        gate = mm(x2, p + ".gate", cfg.inter, D)
        up = mm(x2, p + ".up", cfg.inter, D)
        sig = r16(1.0 / (1.0 + np.exp(-gate.astype(np.float64))))
        act = r16(r16(gate * sig) * up)
        down = mm(act, p + ".down", D, cfg.inter)
    xf, _ = rms_norm(down, w["final_ln"], cfg.eps, skip=residual, round16=True)
    xf = r16(xf).reshape(S, D)
    if logit_rows is not None:
        xf = xf[np.asarray(logit_rows)]
    logits = mm(xf, "lm_head", cfg.vocab, D)
    return logits.reshape(-1, cfg.vocab)
