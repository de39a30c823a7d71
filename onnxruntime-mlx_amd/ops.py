"""Op-level host interface over the kernel C ABI (torch tensors in, torch tensors out).

Each function mirrors one ONNX contrib op on the int4-decoder path, with the
reference EP's input order, attribute names and defaults; the reference
translator each follows is cited in its docstring.
"""

from __future__ import annotations

import ctypes

import torch

from . import ORTMI_BF16, ORTMI_F16, ORTMI_F32, check, load_kernels

_DT = {torch.float32: ORTMI_F32, torch.float16: ORTMI_F16, torch.bfloat16: ORTMI_BF16}


def _dt(t: torch.Tensor) -> int:
    try:
        return _DT[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {t.dtype}") from None


def _p(t):
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("MI355X EP ops take device tensors")
    if not t.is_contiguous():
        raise ValueError("MI355X EP ops take contiguous tensors")
    return ctypes.c_void_p(t.data_ptr())


def _stream(stream):
    if stream is not None:
        return ctypes.c_void_p(int(stream))
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _workspace(nbytes: int, device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


# ------------------------------------------------------------------ MatMulNBits
def matmul_nbits(A, B, scales, zero_points=None, *, K, N, bits=4, block_size=32, out=None,
                 stream=None):
    """com.microsoft MatMulNBits: Y[..., N] = A[..., K] . dequant(B)^T.

    Follows matmulnbits_op (rust/src/ops/quant.rs:986-1130) and its claim
    (quant.rs:1655-1711): A, scales and Y share one float dtype, B and zero points
    are uint8, bits in {4, 8}, block_size in {16, 32, 64, 128}.
    """
    if A.shape[-1] != K:
        raise ValueError(f"MatMulNBits: A's last dim {A.shape[-1]} != K={K}")
    if A.dtype != scales.dtype:
        raise TypeError("MatMulNBits: activation and scales must share one float dtype")
    if B.dtype != torch.uint8 or (zero_points is not None and zero_points.dtype != torch.uint8):
        raise TypeError("MatMulNBits: packed weights and zero points must be uint8")
    nb = (K + block_size - 1) // block_size
    if B.numel() != N * nb * block_size * bits // 8:
        raise ValueError("MatMulNBits: B does not hold N * ceil(K/bs) * bs*bits/8 bytes")
    if scales.numel() != N * nb:
        raise ValueError("MatMulNBits: scale count does not match N * nblocks")
    if zero_points is not None:
        zcols = (nb + 1) // 2 if bits == 4 else nb
        if zero_points.numel() != N * zcols:
            raise ValueError("MatMulNBits: zero point count mismatch")
    M = A.numel() // K if K else 0
    Y = out if out is not None else torch.empty(tuple(A.shape[:-1]) + (N,), dtype=A.dtype,
                                                device=A.device)
    check(load_kernels().ortmi_matmul_nbits(_p(A), _p(B), _p(scales), _p(zero_points), _p(Y), M,
                                            N, K, bits, block_size, _dt(A), _stream(stream)))
    return Y


# --------------------------------------------------------- GatherBlockQuantized
def gather_block_quantized(data, scales, indices, zero_points=None, *, block_size=128, bits=4,
                           gather_axis=0, quantize_axis=1, out=None, stream=None):
    """com.microsoft GatherBlockQuantized: rows of an int4 block-quantised table.

    Follows gather_block_quantized_op (rust/src/ops/quant.rs:1134-1199) and its
    claim (quant.rs:1713-1749): data uint8 [V, D/2], indices int32/int64, scales
    [V, ceil(D/block)] in the output dtype, optional uint8 packed zero points; bits
    4, gather_axis 0, quantize_axis 1, block_size >= 16. Output indices.shape + [D].
    """
    if bits != 4 or gather_axis != 0 or quantize_axis != 1 or block_size < 16:
        raise ValueError("GatherBlockQuantized: bits 4, gather_axis 0, quantize_axis 1, "
                         "block_size >= 16 only")
    if data.dtype != torch.uint8 or data.dim() != 2:
        raise TypeError("GatherBlockQuantized: data must be uint8 [V, D/2]")
    if indices.dtype not in (torch.int32, torch.int64):
        raise TypeError("GatherBlockQuantized: indices must be int32 or int64")
    V, D = data.shape[0], data.shape[1] * 2
    nb = (D + block_size - 1) // block_size
    if scales.numel() != V * nb:
        raise ValueError("GatherBlockQuantized: scales must be [V, ceil(D/block_size)]")
    if zero_points is not None and (zero_points.dtype != torch.uint8 or
                                    zero_points.numel() != V * ((nb + 1) // 2)):
        raise ValueError("GatherBlockQuantized: zero points must be uint8 [V, ceil(nblocks/2)]")
    n = indices.numel()
    Y = out if out is not None else torch.empty(tuple(indices.shape) + (D,), dtype=scales.dtype,
                                                device=data.device)
    check(load_kernels().ortmi_gather_block_quantized(
        _p(data), _p(scales), _p(zero_points), _p(indices), int(indices.dtype == torch.int64),
        _p(Y), n, V, D, block_size, bits, _dt(scales), _stream(stream)))
    return Y


# ------------------------------------------------------------ GroupQueryAttention
def gqa_contract(total_sequence_length: int, seq_len: int, past_cap: int):
    """(shared, valid_past, present_cap) per rust/src/ops/attention.rs:636-651."""
    vp = total_sequence_length - seq_len
    if vp < 0 or vp > past_cap:
        return False, past_cap, past_cap + seq_len
    shared = past_cap > vp
    return shared, vp, (past_cap if shared else past_cap + seq_len)


def group_query_attention(query, key, value, past_key, past_value, seqlens_k,
                          total_sequence_length, cos_cache=None, sin_cache=None, *, num_heads,
                          kv_num_heads, scale=0.0, do_rotary=0, rotary_interleaved=0,
                          present_key=None, present_value=None, attention_bias=None,
                          q_norm_weight=None, k_norm_weight=None, qk_norm_epsilon=1e-6,
                          stream=None):
    """com.microsoft GroupQueryAttention (decode and prefill, in-op RoPE).

    Follows group_query_attention_op (rust/src/ops/attention.rs:556-952): one
    valid_past = total_sequence_length - S for the batch (seqlens_k is not
    consulted, attention.rs:642-651); shared-buffer contract when the past buffer
    is longer than valid_past, growing contract otherwise. Pass
    present_key=past_key / present_value=past_value to update a shared buffer in
    place. attention_bias (input 10, rank 4 [B or 1, H or 1, >= S, >= total]) is
    added to the scaled scores; q_norm_weight / k_norm_weight (inputs 14/15, [head])
    RMS-normalise q and k per head before RoPE (attention.rs:663-670). fp32 tensors,
    those inputs and head sizes other than 64/96/128 run the generic kernels
    (ortmi_group_query_attention_ex). Returns (output, present_key, present_value).
    """
    del seqlens_k  # not consulted outside sliding-window mode, as in the reference
    total = int(total_sequence_length)
    B, S, hidden = query.shape
    packed = key is None
    hd = hidden // (num_heads + 2 * kv_num_heads) if packed else hidden // num_heads
    cap = past_key.shape[2]
    shared, vp, pcap = gqa_contract(total, S, cap)
    if shared and vp + S > cap:
        raise ValueError("GroupQueryAttention: total_sequence_length exceeds the KV buffer "
                         "capacity")
    if present_key is None:
        present_key = torch.empty((B, kv_num_heads, pcap, hd), dtype=query.dtype,
                                  device=query.device)
    if present_value is None:
        present_value = torch.empty((B, kv_num_heads, pcap, hd), dtype=query.dtype,
                                    device=query.device)
    if tuple(present_key.shape) != (B, kv_num_heads, pcap, hd):
        raise ValueError("GroupQueryAttention: present_key has the wrong shape for the contract")
    out = torch.empty((B, S, num_heads * hd), dtype=query.dtype, device=query.device)
    lib = load_kernels()
    use_rope = bool(do_rotary) and cos_cache is not None
    half = cos_cache.shape[1] if use_rope else 0
    max_pos = cos_cache.shape[0] if use_rope else 0
    rope = (_p(cos_cache) if use_rope else None, _p(sin_cache) if use_rope else None, half,
            max_pos)
    generic = (query.dtype == torch.float32 or attention_bias is not None
               or q_norm_weight is not None or k_norm_weight is not None
               or hd not in (64, 96, 128))
    if generic:
        ws = _workspace(lib.ortmi_group_query_attention_ex_workspace_size(B, S, num_heads, hd),
                        query.device)
        bdims = (0, 0, 0, 0)
        if attention_bias is not None:
            if attention_bias.dim() != 4 or attention_bias.dtype != query.dtype:
                raise ValueError("GroupQueryAttention: attention_bias must be rank 4 in the "
                                 "output dtype")
            attention_bias = attention_bias.contiguous()
            bdims = tuple(attention_bias.shape)
        check(lib.ortmi_group_query_attention_ex(
            _p(query), _p(key), _p(value), _p(past_key), _p(past_value), cap, total, *rope,
            _p(q_norm_weight), _p(k_norm_weight), float(qk_norm_epsilon), _p(attention_bias),
            *bdims, _p(out), _p(present_key), _p(present_value), B, S, num_heads, kv_num_heads,
            hd, float(scale), int(rotary_interleaved), _dt(query), _p(ws), ws.numel(),
            _stream(stream)))
        return out, present_key, present_value
    ws_bytes = lib.ortmi_group_query_attention_workspace_size(B, S, num_heads, hd, vp + S)
    ws = _workspace(ws_bytes, query.device)
    check(lib.ortmi_group_query_attention(
        _p(query), _p(key), _p(value), _p(past_key), _p(past_value), cap, total, *rope,
        _p(out), _p(present_key), _p(present_value), B, S, num_heads, kv_num_heads, hd,
        float(scale), int(rotary_interleaved), _dt(query), _p(ws), ws.numel(), _stream(stream)))
    return out, present_key, present_value


def group_query_attention_sliding(query, key, value, past_key, past_value, seqlens_k,
                                  cos_cache=None, sin_cache=None, *, num_heads, kv_num_heads,
                                  local_window_size, scale=0.0, do_rotary=0,
                                  rotary_interleaved=0, present_key=None, present_value=None,
                                  q_norm_weight=None, k_norm_weight=None, qk_norm_epsilon=1e-6,
                                  stream=None):
    """GroupQueryAttention with sliding_window_cache = 1 (rust/src/ops/attention.rs:725-880):
    past_key/past_value [B, KV, cap, hd] are a compacting cache, seqlens_k (device
    int32 [B]) gives each sequence's length minus one. Pass present_key=past_key /
    present_value=past_value to compact in place. Returns (output, present_key,
    present_value), present at capacity cap with zero rows after the kept ones."""
    B, S, hidden = query.shape
    packed = key is None
    hd = hidden // (num_heads + 2 * kv_num_heads) if packed else hidden // num_heads
    cap = past_key.shape[2]
    if present_key is None:
        present_key = torch.empty_like(past_key)
    if present_value is None:
        present_value = torch.empty_like(past_value)
    out = torch.empty((B, S, num_heads * hd), dtype=query.dtype, device=query.device)
    lib = load_kernels()
    use_rope = bool(do_rotary) and cos_cache is not None
    half = cos_cache.shape[1] if use_rope else 0
    max_pos = cos_cache.shape[0] if use_rope else 0
    ws = _workspace(lib.ortmi_group_query_attention_sliding_workspace_size(
        B, S, num_heads, kv_num_heads, hd, cap), query.device)
    check(lib.ortmi_group_query_attention_sliding(
        _p(query), _p(key), _p(value), _p(past_key), _p(past_value), cap, _p(seqlens_k),
        _p(cos_cache) if use_rope else None, _p(sin_cache) if use_rope else None, half, max_pos,
        _p(q_norm_weight), _p(k_norm_weight), float(qk_norm_epsilon), int(local_window_size),
        _p(out), _p(present_key), _p(present_value), B, S, num_heads, kv_num_heads, hd,
        float(scale), int(rotary_interleaved), _dt(query), _p(ws), ws.numel(), _stream(stream)))
    return out, present_key, present_value


def group_query_attention_decode_capturable(query, key, value, kv_key, kv_value,
                                            total_sequence_length_device, cos_cache=None,
                                            sin_cache=None, *, num_heads, kv_num_heads,
                                            scale=0.0, rotary_interleaved=0, workspace=None,
                                            stream=None):
    """One-token GroupQueryAttention step, shared KV buffer updated in place, with
    total_sequence_length read from a device int32 tensor (graph-capturable: the
    launches depend only on the buffer capacity). Returns the output [B, 1, H*hd].

    Equal to group_query_attention(..., present_key=kv_key, present_value=kv_value)
    for S = 1 under the shared-buffer contract; the caller keeps
    1 <= total <= capacity. Pass a preallocated `workspace` (uint8 device tensor)
    when capturing, so no allocation happens inside the capture."""
    B, S, hidden = query.shape
    if S != 1:
        raise ValueError("capturable GroupQueryAttention decodes one token")
    hd = hidden // num_heads
    cap = kv_key.shape[2]
    out = torch.empty((B, 1, num_heads * hd), dtype=query.dtype, device=query.device)
    lib = load_kernels()
    ws_bytes = lib.ortmi_group_query_attention_workspace_size(B, 1, num_heads, hd, cap)
    ws = workspace if workspace is not None else _workspace(ws_bytes, query.device)
    half = cos_cache.shape[1] if cos_cache is not None else 0
    max_pos = cos_cache.shape[0] if cos_cache is not None else 0
    check(lib.ortmi_group_query_attention_decode_capturable(
        _p(query), _p(key), _p(value), _p(kv_key), _p(kv_value), cap,
        _p(total_sequence_length_device), _p(cos_cache) if cos_cache is not None else None,
        _p(sin_cache) if sin_cache is not None else None, half, max_pos, _p(out), B, num_heads,
        kv_num_heads, hd, float(scale), int(rotary_interleaved), _dt(query), _p(ws), ws.numel(),
        _stream(stream)))
    return out


# --------------------------------------------------------------- PagedAttention
def paged_attention(query, key, value, key_cache, value_cache, cumulative_sequence_length,
                    past_seqlens, block_table, cos_cache=None, sin_cache=None, slot_mapping=None,
                    head_sink=None, q_norm_weight=None, k_norm_weight=None, *, num_heads,
                    kv_num_heads, scale=0.0, do_rotary=0, rotary_interleaved=0, rotary_offset=0,
                    v_head_size=0, kv_cache_layout="SEPARATE", qk_norm_epsilon=1e-6,
                    max_context=None, stream=None):
    """com.microsoft PagedAttention over a block-paged KV cache (updated in place).

    Follows paged_attention_op (rust/src/ops/attention.rs:2495-2744) with RoPE read
    from the cache rows (tests/ops/test_paged_attention.py:29-47). All control
    tensors stay on the device. Returns the output [T, H*vhd].
    """
    latent = kv_cache_layout == "LATENT"
    if latent:
        value = None
        value_cache = None
    T = query.shape[0]
    nblk, blk, KV, hd = key_cache.shape
    if KV != kv_num_heads:
        raise ValueError("PagedAttention: key_cache head count != kv_num_heads")
    vhd = v_head_size or hd
    batch = cumulative_sequence_length.shape[0] - 1
    maxb = block_table.shape[1]
    if max_context is None:
        max_context = maxb * blk
    out = torch.empty((T, num_heads * vhd), dtype=query.dtype, device=query.device)
    lib = load_kernels()
    ws = _workspace(lib.ortmi_paged_attention_workspace_size(T, batch, num_heads, KV, hd, vhd,
                                                             max_context), query.device)
    use_rope = bool(do_rotary) and cos_cache is not None
    half = cos_cache.shape[1] if use_rope else 0
    max_pos = cos_cache.shape[0] if use_rope else 0
    for name, t in (("cumulative_sequence_length", cumulative_sequence_length),
                    ("past_seqlens", past_seqlens), ("block_table", block_table)):
        if t.dtype != torch.int32:
            raise TypeError(f"PagedAttention: {name} must be int32")
    check(lib.ortmi_paged_attention(
        _p(query), _p(key), _p(value), _p(key_cache), _p(value_cache), nblk, blk,
        _p(cumulative_sequence_length), _p(past_seqlens), _p(block_table), batch, maxb, T,
        max_context, _p(cos_cache) if use_rope else None, _p(sin_cache) if use_rope else None,
        half, max_pos, int(rotary_interleaved), int(rotary_offset), _p(slot_mapping),
        _p(head_sink), _p(q_norm_weight), _p(k_norm_weight), float(qk_norm_epsilon), _p(out),
        num_heads, kv_num_heads, hd, vhd, float(scale), _dt(query), _p(ws), ws.numel(),
        _stream(stream)))
    return out


# -------------------------------------------------------------- RotaryEmbedding
def rotary_embedding(x, position_ids, cos_cache, sin_cache, *, interleaved=0, num_heads=0,
                     rotary_embedding_dim=0, stream=None):
    """com.microsoft RotaryEmbedding (inputs x, position_ids, cos_cache, sin_cache).

    Follows rotary_embedding_op (rust/src/ops/attention.rs:1317-1411): x is
    [B,S,N*hd] or [B,N,S,hd]; position_ids [B,S], an offset [1], or None (then
    cos/sin are per-token [B,S,half]).
    """
    if x.dim() == 4:
        B, NH, S, hd = x.shape
        bnsd = 1
    else:
        B, S, hidden = x.shape
        hd = hidden // num_heads if num_heads > 0 else 2 * cos_cache.shape[-1]
        NH = hidden // hd
        bnsd = 0
    half = cos_cache.shape[-1]
    if rotary_embedding_dim:
        half = min(half, rotary_embedding_dim // 2)
    if position_ids is None:
        cos2 = cos_cache.reshape(-1, cos_cache.shape[-1]).contiguous()
        sin2 = sin_cache.reshape(-1, sin_cache.shape[-1]).contiguous()
        pos_is_offset = 0
    else:
        cos2, sin2 = cos_cache, sin_cache
        pos_is_offset = 1 if position_ids.numel() == 1 else 0
        if position_ids.dtype != torch.int64:
            position_ids = position_ids.to(torch.int64)
    if cos2.shape[-1] != half:
        cos2 = cos2[:, :half].contiguous()
        sin2 = sin2[:, :half].contiguous()
    y = torch.empty_like(x)
    check(load_kernels().ortmi_rotary_embedding(
        _p(x), _p(position_ids), pos_is_offset, _p(cos2), _p(sin2), cos2.shape[0], _p(y), B, S,
        NH, hd, half, bnsd, int(interleaved), _dt(x), _stream(stream)))
    return y


# ------------------------------------------------------- (Skip)SimplifiedLayerNorm
def simplified_layer_norm(x, scale, *, epsilon=1e-5, stream=None):
    """com.microsoft SimplifiedLayerNormalization (rust/src/ops/norm.rs:175-185)."""
    D = x.shape[-1]
    y = torch.empty_like(x)
    check(load_kernels().ortmi_rms_norm(_p(x), None, None, _p(scale), _p(y), None,
                                        x.numel() // D, D, float(epsilon), _dt(x),
                                        _stream(stream)))
    return y


def skip_simplified_layer_norm(x, skip, gamma, bias=None, *, epsilon=1e-6, stream=None):
    """com.microsoft SkipSimplifiedLayerNormalization (rust/src/ops/norm.rs:231-248).

    Returns (normalized, residual) - output 0 and the last output."""
    D = x.shape[-1]
    y = torch.empty_like(x)
    r = torch.empty_like(x)
    check(load_kernels().ortmi_rms_norm(_p(x), _p(skip), _p(bias), _p(gamma), _p(y), _p(r),
                                        x.numel() // D, D, float(epsilon), _dt(x),
                                        _stream(stream)))
    return y, r
