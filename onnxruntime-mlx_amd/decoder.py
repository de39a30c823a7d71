"""Int4 Llama-style decoder expressed as an ONNX contrib-op graph, run through the EP.

The graph mirrors what ONNX Runtime GenAI exports for a q4f16 decoder (the op
histogram the reference records for Qwen2.5-0.5B decode,
examples/traces/qwen2.5-0.5b-decode.json): an embedding Gather, per layer
(Skip)SimplifiedLayerNormalization, seven MatMulNBits, GroupQueryAttention with
in-op rotary, and a Sigmoid/Mul/Mul SwiGLU, then a final norm and the lm_head
MatMulNBits. Weights are random (seeded); every linear layer is 4-bit, block 32,
symmetric, with fp16 scales |N(0, 0.02)|.

The KV cache is device resident with a fixed capacity: each layer's present
output is bound to its past input buffer, so GroupQueryAttention writes the new
rows in place (the shared-buffer contract, rust/src/ops/attention.rs:893-902).
Greedy decoding takes the argmax on the device and feeds it back as the next
input id, so a decode step reads nothing back to the host but total_sequence_length.
"""

from __future__ import annotations

import ctypes
import json
import time
from dataclasses import dataclass

import numpy as np

from . import check, load_kernels
from . import harness as hx


@dataclass
class DecoderConfig:
    layers: int = 28
    hidden: int = 1536
    heads: int = 12
    kv_heads: int = 2
    head_dim: int = 128
    inter: int = 8960
    vocab: int = 151936
    rope_base: float = 1e6
    eps: float = 1e-6
    block: int = 32
    max_pos: int = 4096

    def linear_shapes(self):
        """(name, N, K) of every MatMulNBits in one layer."""
        H, KV, hd, D, I = self.heads, self.kv_heads, self.head_dim, self.hidden, self.inter
        return [("q", H * hd, D), ("k", KV * hd, D), ("v", KV * hd, D), ("o", D, H * hd),
                ("gate", I, D), ("up", I, D), ("down", D, I)]

    def weight_bytes(self) -> int:
        """int4 codes + fp16 scales of all linear layers (the per-token weight stream)."""
        total = 0
        for _, N, K in self.linear_shapes():
            total += N * K // 2 + N * (K // self.block) * 2
        total *= self.layers
        total += self.vocab * self.hidden // 2 + self.vocab * (self.hidden // self.block) * 2
        return total


# Byte -> two codes 8 + popcount(nibble) - 2 (binomial(4, 1/2) around the default zero
# point 8, variance 1), packed low nibble first.
_BINOMIAL_BYTE = np.array(
    [(8 + bin(b & 15).count("1") - 2) | ((8 + bin(b >> 4).count("1") - 2) << 4)
     for b in range(256)], np.uint8)


def _quant_linear(rng, N, K, block):
    """Symmetric int4 weights (default zero point 8), fp16 scales |N(0, 0.02)|.

    Codes are 8 + Binomial(4, 1/2) - 2 rather than uniform over 0..15: with uniform
    codes (effective weight rms 0.09) the fp16 residual stream of this 28-layer
    graph overflows to inf by the seventh layer (down_proj outputs reach 1.6e4 per
    layer), so every implementation, fp16 CPU included, returns NaN logits. The
    byte stream the kernels read is the same size either way."""
    nb = K // block
    B = _BINOMIAL_BYTE[rng.integers(0, 256, size=(N, nb, block // 2), dtype=np.uint8)]
    s = np.abs(rng.standard_normal(N * nb, dtype=np.float32) * 0.02).astype(np.float16)
    return B, s


def make_weights(cfg: DecoderConfig, seed: int = 4):
    rng = np.random.default_rng(seed)
    w = {"embed": rng.standard_normal((cfg.vocab, cfg.hidden), dtype=np.float32).astype(np.float16)}
    for layer in range(cfg.layers):
        for name, N, K in cfg.linear_shapes():
            B, s = _quant_linear(rng, N, K, cfg.block)
            w[f"l{layer}.{name}.B"] = B
            w[f"l{layer}.{name}.s"] = s
        w[f"l{layer}.ln1"] = np.ones(cfg.hidden, np.float16)
        w[f"l{layer}.ln2"] = np.ones(cfg.hidden, np.float16)
    w["final_ln"] = np.ones(cfg.hidden, np.float16)
    B, s = _quant_linear(rng, cfg.vocab, cfg.hidden, cfg.block)
    w["lm_head.B"], w["lm_head.s"] = B, s
    half = cfg.head_dim // 2
    inv = 1.0 / (cfg.rope_base ** (np.arange(half, dtype=np.float64) / half))
    ang = np.arange(cfg.max_pos, dtype=np.float64)[:, None] * inv[None, :]
    w["cos"] = np.cos(ang).astype(np.float16)
    w["sin"] = np.sin(ang).astype(np.float16)
    return w


def build_graph(cfg: DecoderConfig, w, cap: int, layer_metadata: bool = False,
                argmax: bool = False, norm_stats: bool = False) -> hx.Graph:
    """Decoder graph with symbolic sequence length S and KV capacity `cap`.

    argmax: end the graph with ArgMax(logits, axis=-1, keepdims=0) -> next_tokens
    (int64 [1, S]), so greedy decoding takes its next id from the graph itself.

    norm_stats: every SkipSimplifiedLayerNormalization also declares its mean and
    inv_std_var outputs (read by nothing), as transformers.js / Mobius exports do.

    layer_metadata: also record the residual stream after each layer (the last one's
    is the final norm's residual output) under the model metadata key
    onnxruntime_ep_mlx.layer_boundary_outputs, as the reference's exporters do
    (README.md "Large-decoder partition metadata")."""
    g = hx.Graph()
    F16, I32, I64 = hx.FLOAT16, hx.INT32, hx.INT64
    D, H, KV, hd = cfg.hidden, cfg.heads, cfg.kv_heads, cfg.head_dim
    S = -1
    g.value("input_ids", I64, [1, S])
    g.value("seqlens_k", I32, [1])
    g.value("total_sequence_length", I32, [1])
    g.value("logits", F16, [1, S, cfg.vocab])
    g.initializer("embed", w["embed"])
    g.initializer("cos_cache", w["cos"])
    g.initializer("sin_cache", w["sin"])
    inputs = ["input_ids", "seqlens_k", "total_sequence_length"]
    outputs = ["logits"]

    def linear(x, name, wkey, N, K, out):
        g.initializer(f"{wkey}.B", w[f"{wkey}.B"])
        g.initializer(f"{wkey}.s", w[f"{wkey}.s"])
        g.value(out, F16, [1, S, N])
        g.node("MatMulNBits", [x, f"{wkey}.B", f"{wkey}.s"], [out], domain="com.microsoft",
               name=name, K=K, N=N, bits=4, block_size=cfg.block)

    g.value("h0", F16, [1, S, D])
    g.node("Gather", ["embed", "input_ids"], ["h0"], name="embed_gather", axis=0)
    prev_out, residual = None, "h0"

    def skip_norm(x, skip, gamma, y, res, name):
        stats = ["", ""]
        if norm_stats:
            stats = [f"{name}.mean", f"{name}.inv_std"]
            for v in stats:
                g.value(v, hx.FLOAT, [1, S, 1])
        g.node("SkipSimplifiedLayerNormalization", [x, skip, gamma], [y] + stats + [res],
               domain="com.microsoft", name=name, epsilon=cfg.eps)

    for layer in range(cfg.layers):
        p = f"l{layer}"
        g.initializer(f"{p}.ln1", w[f"{p}.ln1"])
        g.initializer(f"{p}.ln2", w[f"{p}.ln2"])
        g.value(f"{p}.x", F16, [1, S, D])
        if layer == 0:
            g.node("SimplifiedLayerNormalization", ["h0", f"{p}.ln1"], [f"{p}.x"],
                   name=f"{p}.ln1", epsilon=cfg.eps, axis=-1)
        else:
            g.value(f"{p}.res1", F16, [1, S, D])
            skip_norm(prev_out, residual, f"{p}.ln1", f"{p}.x", f"{p}.res1", f"{p}.ln1")
            residual = f"{p}.res1"
        for name, N, K in cfg.linear_shapes()[:3]:
            linear(f"{p}.x", f"{p}.{name}_proj", f"{p}.{name}", N, K, f"{p}.{name}")
        for kv in ("key", "value"):
            g.value(f"past_key_values.{layer}.{kv}", F16, [1, KV, cap, hd])
            g.value(f"present.{layer}.{kv}", F16, [1, KV, cap, hd])
            inputs.append(f"past_key_values.{layer}.{kv}")
            outputs.append(f"present.{layer}.{kv}")
        g.value(f"{p}.attn", F16, [1, S, H * hd])
        g.node("GroupQueryAttention",
               [f"{p}.q", f"{p}.k", f"{p}.v", f"past_key_values.{layer}.key",
                f"past_key_values.{layer}.value", "seqlens_k", "total_sequence_length",
                "cos_cache", "sin_cache"],
               [f"{p}.attn", f"present.{layer}.key", f"present.{layer}.value"],
               domain="com.microsoft", name=f"{p}.gqa", num_heads=H, kv_num_heads=KV,
               do_rotary=1, rotary_interleaved=0, scale=0.0)
        linear(f"{p}.attn", f"{p}.o_proj", f"{p}.o", D, H * hd, f"{p}.o")
        g.value(f"{p}.x2", F16, [1, S, D])
        g.value(f"{p}.res2", F16, [1, S, D])
        skip_norm(f"{p}.o", residual, f"{p}.ln2", f"{p}.x2", f"{p}.res2", f"{p}.ln2")
        residual = f"{p}.res2"
        linear(f"{p}.x2", f"{p}.gate_proj", f"{p}.gate", cfg.inter, D, f"{p}.gate")
        linear(f"{p}.x2", f"{p}.up_proj", f"{p}.up", cfg.inter, D, f"{p}.up")
        for v in ("sig", "silu", "act"):
            g.value(f"{p}.{v}", F16, [1, S, cfg.inter])
        g.node("Sigmoid", [f"{p}.gate"], [f"{p}.sig"], name=f"{p}.sigmoid")
        g.node("Mul", [f"{p}.gate", f"{p}.sig"], [f"{p}.silu"], name=f"{p}.silu")
        g.node("Mul", [f"{p}.silu", f"{p}.up"], [f"{p}.act"], name=f"{p}.gated")
        linear(f"{p}.act", f"{p}.down_proj", f"{p}.down", D, cfg.inter, f"{p}.down")
        prev_out = f"{p}.down"
    g.initializer("final_ln", w["final_ln"])
    g.value("xf", F16, [1, S, D])
    g.value("resf", F16, [1, S, D])
    skip_norm(prev_out, residual, "final_ln", "xf", "resf", "final_ln")
    g.initializer("lm_head.B", w["lm_head.B"])
    g.initializer("lm_head.s", w["lm_head.s"])
    g.node("MatMulNBits", ["xf", "lm_head.B", "lm_head.s"], ["logits"], domain="com.microsoft",
           name="lm_head", K=D, N=cfg.vocab, bits=4, block_size=cfg.block)
    if argmax:
        g.value("next_tokens", I64, [1, S])
        g.node("ArgMax", ["logits"], ["next_tokens"], name="greedy", axis=-1, keepdims=0)
        outputs.append("next_tokens")
    if layer_metadata:
        names = [f"l{layer}.res1" for layer in range(1, cfg.layers)] + ["resf"]
        g.metadata("onnxruntime_ep_mlx.layer_boundary_outputs", json.dumps(names))
    g.io(inputs, outputs)
    return g


class DecoderRunner:
    """Greedy generation through the EP with a device-resident KV cache.

    seqlens_k and total_sequence_length are host inputs (pinned), as ONNX Runtime
    keeps them; logits and KV are bound to device buffers (IOBinding).

    argmax_node: build the graph with its ArgMax (build_graph's argmax) and feed its
    output back as the next input id; otherwise the runner takes the argmax of the
    last logits row with ortmi_argmax_rows after each run.

    host_feeds: the input ids are a host tensor too, as an application without
    IOBinding feeds them (ONNX Runtime GenAI's loop): each step reads the greedy id
    back to the host and feeds it, and the harness copies every host feed to the
    EP's memory device (HBM) through the EP's data transfer before Compute. With
    argmax_node the ArgMax output is bound to host memory, where a serving loop
    reads the token. Otherwise the ids stay in HBM and the argmax output is fed
    back in place.
    """

    def __init__(self, cfg: DecoderConfig, weights, cap: int, max_prompt: int,
                 layer_metadata: bool = False, argmax_node: bool = False,
                 host_feeds: bool = False, norm_stats: bool = False):
        import torch

        self.torch = torch
        self.cfg = cfg
        self.cap = cap
        self.argmax_node = argmax_node
        self.host_feeds = host_feeds
        self.ids_host = torch.zeros((1, max_prompt), dtype=torch.int64, pin_memory=True)
        self.graph = build_graph(cfg, weights, cap, layer_metadata, argmax=argmax_node,
                                 norm_stats=norm_stats)
        self.session = hx.Session(self.graph)
        dev = "cuda"
        self.kv = []
        for layer in range(cfg.layers):
            k = torch.zeros((1, cfg.kv_heads, cap, cfg.head_dim), dtype=torch.float16, device=dev)
            v = torch.zeros_like(k)
            self.kv.append((k, v))
            # present bound to past: GroupQueryAttention appends in place
            self.session.bind_output(f"present.{layer}.key", k)
            self.session.bind_output(f"present.{layer}.value", v)
        self.logits = torch.empty((1, max_prompt, cfg.vocab), dtype=torch.float16, device=dev)
        self.session.bind_output("logits", self.logits)
        self.ids = torch.zeros((1, max_prompt), dtype=torch.int64, device=dev)
        self.next_id = torch.zeros((1, 1), dtype=torch.int64, device=dev)
        # ArgMax outputs alternate between two buffers, so a step's input id (the
        # previous step's output) is never the buffer it writes.
        tok_dev = "cpu" if (host_feeds and argmax_node) else dev
        self.tokens = [torch.zeros((1, max_prompt), dtype=torch.int64, device=tok_dev)
                       for _ in range(2)]
        self._first = [t[:, :1] for t in self.tokens]
        self._flip = 0
        # seqlens_k and total_sequence_length live in (pinned) host memory, as ONNX
        # Runtime keeps them.
        self.seqlens = torch.zeros(1, dtype=torch.int32, pin_memory=True)
        self.total = torch.zeros(1, dtype=torch.int32, pin_memory=True)
        self._host = np.frombuffer(
            (ctypes.c_int32 * 1).from_address(self.seqlens.data_ptr()), np.int32), np.frombuffer(
            (ctypes.c_int32 * 1).from_address(self.total.data_ptr()), np.int32)
        self.length = 0
        self.lib = load_kernels()
        self.argmax_ws = torch.empty(
            max(1, self.lib.ortmi_argmax_rows_workspace_size(1, cfg.vocab)), dtype=torch.uint8,
            device=dev)
        # Inputs that keep their buffers for the whole generation are bound once.
        self.session.set_input("seqlens_k", self.seqlens, hx.INT32)
        self.session.set_input("total_sequence_length", self.total, hx.INT32)
        for layer, (k, v) in enumerate(self.kv):
            self.session.set_input(f"past_key_values.{layer}.key", k, hx.FLOAT16)
            self.session.set_input(f"past_key_values.{layer}.value", v, hx.FLOAT16)

    def reset(self):
        self.length = 0

    def run(self, ids, S: int):
        """Forward S new tokens (device int64 [1, S]); logits land in self.logits[:, :S]."""
        if self.length + S > self.cap:
            raise ValueError(f"KV capacity {self.cap} exceeded")
        # The EP is not stream aware: like ONNX Runtime, hand it inputs that are ready.
        self.torch.cuda.current_stream().synchronize()
        self._host[0][0] = self.length + S - 1
        self._host[1][0] = self.length + S
        if self.argmax_node:
            out = self.tokens[self._flip]
            self.session.bind_output("next_tokens", out)
        self.session.run({"input_ids": (ids, hx.INT64)})
        self.length += S
        if self.argmax_node:
            self.next_id = self._first[self._flip] if S == 1 else out[:, S - 1:S]
            self._flip ^= 1

    def argmax_last(self, S: int):
        if self.argmax_node:
            return  # the graph's ArgMax already wrote next_id
        st = ctypes.c_void_p(self.torch.cuda.current_stream().cuda_stream)
        last = self.logits[0, S - 1]
        check(self.lib.ortmi_argmax_rows(ctypes.c_void_p(last.data_ptr()),
                                         ctypes.c_void_p(self.next_id.data_ptr()), 1,
                                         self.cfg.vocab, 10,
                                         ctypes.c_void_p(self.argmax_ws.data_ptr()),
                                         self.argmax_ws.numel(), st))

    def prefill(self, prompt: np.ndarray):
        S = int(prompt.shape[-1])
        ids = self.torch.from_numpy(np.asarray(prompt, np.int64).reshape(-1))
        if self.host_feeds:
            self.ids_host[0, :S].copy_(ids)
            self.run(self.ids_host[:, :S], S)
        else:
            self.ids[0, :S].copy_(ids)
            self.run(self.ids[:, :S], S)
        self.argmax_last(S)

    def decode_step(self):
        if self.host_feeds:
            # The greedy id back to the host (the stream is synchronised by the copy),
            # then fed as a host input.
            self.ids_host[0, 0] = int(self.next_id.reshape(-1)[0].item())
            self.run(self.ids_host[:, :1], 1)
        else:
            self.run(self.next_id, 1)
        self.argmax_last(1)

    def generate(self, prompt: np.ndarray, steps: int):
        """Greedy: returns (tokens, prefill seconds, per-decode-step seconds)."""
        torch = self.torch
        self.reset()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        self.prefill(prompt)
        torch.cuda.synchronize()
        ttft = time.perf_counter() - t0
        tokens = [int(self.next_id.item())]
        times = []
        for _ in range(steps - 1):
            t1 = time.perf_counter()
            self.decode_step()
            torch.cuda.synchronize()
            times.append(time.perf_counter() - t1)
            tokens.append(int(self.next_id.item()))
        return tokens, ttft, times
