"""Host face of the one-launch decode step (ortmi_decoder_decode_step).

Builds the device layer table of an int4 Llama-style decoder from its weights
(the layout the EP's decode rewrites produce: q/k/v rows merged into one
projection, gate/up rows interleaved) and runs greedy decode steps with the KV
cache, token id, total length, logits and next id all in device memory.
"""

from __future__ import annotations

import ctypes

import numpy as np

from . import ORTMI_F16, check, load_kernels

_vp, _f32, _i32 = ctypes.c_void_p, ctypes.c_float, ctypes.c_int32


class Layer(ctypes.Structure):
    """OrtmiDecoderLayer (include/ortmi_kernels.h)."""

    _fields_ = [("qkv_weight", _vp), ("qkv_scales", _vp), ("ln1_gamma", _vp),
                ("ln1_epsilon", _f32), ("reserved0", _i32), ("o_weight", _vp), ("o_scales", _vp),
                ("ln2_gamma", _vp), ("ln2_epsilon", _f32), ("reserved1", _i32),
                ("gate_up_weight", _vp), ("gate_up_scales", _vp), ("down_weight", _vp),
                ("down_scales", _vp), ("k_cache", _vp), ("v_cache", _vp)]


class Dims(ctypes.Structure):
    """OrtmiDecoderDims (include/ortmi_kernels.h)."""

    _fields_ = [(n, _i32) for n in ("layers", "hidden", "num_heads", "kv_num_heads", "head_size",
                                    "intermediate", "vocab", "kv_capacity", "max_position",
                                    "rotary_half", "rotary_interleaved", "block_size",
                                    "dtype")] + [("scale", _f32), ("cooperative", _i32)]


def merge_qkv(w, prefix):
    """q, k, v rows of one layer as one MatMulNBits weight (rows concatenated)."""
    B = np.concatenate([w[f"{prefix}.{n}.B"] for n in ("q", "k", "v")])
    s = np.concatenate([w[f"{prefix}.{n}.s"] for n in ("q", "k", "v")])
    return B, s


def interleave_gate_up(w, prefix):
    """gate and up rows interleaved (row 2i gate i, row 2i+1 up i), scales likewise."""
    g, u = w[f"{prefix}.gate.B"], w[f"{prefix}.up.B"]
    B = np.stack([g, u], axis=1).reshape((-1,) + g.shape[1:])
    N, nb = g.shape[0], g.shape[1]
    gs, us = w[f"{prefix}.gate.s"].reshape(N, nb), w[f"{prefix}.up.s"].reshape(N, nb)
    s = np.stack([gs, us], axis=1).reshape(-1)
    return B, s


class DecodeProgram:
    """Device-resident weights and layer table of a decoder for the one-launch step.

    `kv` is a list of (k_cache, v_cache) device tensors [1, KV, cap, hd] shared
    with whoever fills the prompt (the EP's prefill writes them in place)."""

    def __init__(self, cfg, w, kv, cap):
        import torch

        self.torch = torch
        self.cfg = cfg
        dev = "cuda"
        t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
        self._hold = []
        layers = (Layer * cfg.layers)()
        for i in range(cfg.layers):
            p = f"l{i}"
            qB, qs = merge_qkv(w, p)
            gB, gs = interleave_gate_up(w, p)
            bufs = dict(qB=t(qB), qs=t(qs), g1=t(w[f"{p}.ln1"]), oB=t(w[f"{p}.o.B"]),
                        os=t(w[f"{p}.o.s"]), g2=t(w[f"{p}.ln2"]), gB=t(gB), gs=t(gs),
                        dB=t(w[f"{p}.down.B"]), ds=t(w[f"{p}.down.s"]))
            self._hold.append(bufs)
            P = lambda x: x.data_ptr()  # noqa: E731
            layers[i] = Layer(P(bufs["qB"]), P(bufs["qs"]), P(bufs["g1"]), cfg.eps, 0,
                              P(bufs["oB"]), P(bufs["os"]), P(bufs["g2"]), cfg.eps, 0,
                              P(bufs["gB"]), P(bufs["gs"]), P(bufs["dB"]), P(bufs["ds"]),
                              kv[i][0].data_ptr(), kv[i][1].data_ptr())
        raw = np.frombuffer(bytes(layers), np.uint8)
        self.table = t(raw)
        self.embed = t(w["embed"])
        self.cos, self.sin = t(w["cos"]), t(w["sin"])
        self.final_gamma = t(w["final_ln"])
        self.lmB, self.lms = t(w["lm_head.B"]), t(w["lm_head.s"])
        self.dims = Dims(cfg.layers, cfg.hidden, cfg.heads, cfg.kv_heads, cfg.head_dim,
                         cfg.inter, cfg.vocab, cap, cfg.max_pos, cfg.head_dim // 2, 0,
                         cfg.block, ORTMI_F16, 0.0, 1)
        lib = load_kernels()
        self.lib = lib
        nbytes = lib.ortmi_decoder_decode_step_workspace_size(ctypes.byref(self.dims))
        self.ws = torch.zeros(nbytes + 256, dtype=torch.uint8, device=dev)
        self.ws_off = (-self.ws.data_ptr()) % 256
        self.ws_bytes = nbytes
        self.logits = torch.empty(cfg.vocab, dtype=torch.float16, device=dev)
        self.next_id = torch.zeros(1, dtype=torch.int64, device=dev)
        self.token = torch.zeros(1, dtype=torch.int64, device=dev)
        self.total = torch.zeros(1, dtype=torch.int32, device=dev)
        self.status = torch.full((1,), -1, dtype=torch.int32, device=dev)

    def abort_next(self):
        """Abort the next step before it starts, through the workspace's abort word
        (byte 128: launch index + 1; launch index = the 64-bit started-workgroup
        count at byte 0 / the grid, the CU count rounded down to a multiple of 8).
        The aborted step reads and writes nothing and leaves status at -1."""
        torch = self.torch
        torch.cuda.synchronize()
        base = self.ws[self.ws_off:self.ws_off + 256]
        started = int(base[0:8].view(torch.int64).item())
        cus = torch.cuda.get_device_properties(self.ws.device).multi_processor_count
        word = (started // (cus - cus % 8) + 1) & 0xFFFFFFFF
        base[128:132].view(torch.int32).fill_(word - (1 << 32) if word >= 1 << 31 else word)

    def step(self, token=None, total=None, stream=None):
        """One decode step: token (device int64 [1], default the last next_id) at
        position total - 1 (device int32 [1]); logits and next_id are written."""
        torch = self.torch
        tok = self.next_id if token is None else token
        tot = self.total if total is None else total
        # Every step starts from "not completed": a launch that stops early (or is
        # aborted before it starts) leaves -1, not the previous step's 0.
        self.status.fill_(-1)
        st = ctypes.c_void_p(stream if stream is not None else
                             torch.cuda.current_stream().cuda_stream)
        check(self.lib.ortmi_decoder_decode_step(
            _vp(self.table.data_ptr()), ctypes.byref(self.dims), _vp(self.embed.data_ptr()),
            self.cfg.vocab, _vp(tok.data_ptr()), _vp(tot.data_ptr()), _vp(self.cos.data_ptr()),
            _vp(self.sin.data_ptr()), _vp(self.final_gamma.data_ptr()), self.cfg.eps,
            _vp(self.lmB.data_ptr()), _vp(self.lms.data_ptr()), _vp(self.logits.data_ptr()),
            _vp(self.next_id.data_ptr()), _vp(self.status.data_ptr()),
            _vp(self.ws.data_ptr() + self.ws_off), self.ws_bytes, st))
