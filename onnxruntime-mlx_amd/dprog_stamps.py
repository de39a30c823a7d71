"""Per-phase timing of the one-launch decode step, from timestamps compiled into a
variant of the program (libortmi_dprog_stamps.so, `build.py stamps`).

    python onnxruntime-mlx_amd/dprog_stamps.py [--total 576] [--layers 28]

Runs the benchmark decoder's shape (hidden 1536, 12/2 heads, head 128, SwiGLU
8960, vocab 151936; or the shape --hidden/--heads/... give; random weights) as the
decode program at a given context and
prints, as medians over layers 1..L-1, the time each phase of the dataflow takes:
per projection phase from its input being ready to its output stored, per
producer -> consumer hop from the last producer's store to the consumer's input
ready, and the attention steps. The clock is the GPU's 100 MHz realtime counter
(10 ns ticks). The product library has no stamps; this variant adds one store per
phase per workgroup.
"""

from __future__ import annotations

import argparse
import ctypes
import importlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
SLOTS = 256


def _package():
    if "ortmi" in sys.modules:
        return sys.modules["ortmi"]
    spec = importlib.util.spec_from_file_location(
        "ortmi", os.path.join(HERE, "__init__.py"), submodule_search_locations=[HERE])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["ortmi"] = mod
    spec.loader.exec_module(mod)
    return mod


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--total", type=int, default=576, help="total_sequence_length of the step")
    ap.add_argument("--layers", type=int, default=28,
                    help="at most 31: each layer takes 8 of the 256 stamp slots per workgroup")
    ap.add_argument("--hidden", type=int)
    ap.add_argument("--heads", type=int)
    ap.add_argument("--kv-heads", type=int)
    ap.add_argument("--head-dim", type=int)
    ap.add_argument("--inter", type=int)
    ap.add_argument("--vocab", type=int)
    ap.add_argument("--reps", type=int, default=20)
    ap.add_argument("--cooperative", type=int, default=0,
                    help="1: cooperative launch; 0: plain launch of the same grid")
    args = ap.parse_args()
    import torch

    ortmi = _package()
    dec = importlib.import_module("ortmi.decoder")
    dp = importlib.import_module("ortmi.decode_program")
    path = os.path.join(HERE, "lib", "libortmi_dprog_stamps.so")
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} is missing: run onnxruntime-mlx_amd/build.py stamps")
    lab = ctypes.CDLL(path)
    for n in ("ortmi_decoder_decode_step_workspace_size", "ortmi_decoder_decode_step"):
        f = getattr(lab, n)
        f.restype, f.argtypes = ortmi.SIGNATURES[n]
    lab.ortmi_decoder_decode_step_stamps.argtypes = [ctypes.c_void_p, ctypes.c_int]
    lab.ortmi_decoder_decode_step_stamps.restype = ctypes.c_int

    if not 1 <= args.layers <= 31:
        raise SystemExit("--layers must be 1..31 (8 stamp slots per layer, 256 per workgroup)")
    shape = {k: v for k, v in (("hidden", args.hidden), ("heads", args.heads),
                               ("kv_heads", args.kv_heads), ("head_dim", args.head_dim),
                               ("inter", args.inter), ("vocab", args.vocab)) if v is not None}
    cfg = dec.DecoderConfig(layers=args.layers, **shape)
    w = dec.make_weights(cfg, seed=4)
    cap = max(640, args.total)
    kv = [(torch.randn((1, cfg.kv_heads, cap, cfg.head_dim), dtype=torch.float16, device="cuda"),
           torch.randn((1, cfg.kv_heads, cap, cfg.head_dim), dtype=torch.float16, device="cuda"))
          for _ in range(cfg.layers)]
    prog = dp.DecodeProgram(cfg, w, kv, cap)
    del w
    prog.lib = lab
    prog.dims.cooperative = args.cooperative
    prog.total.fill_(args.total)
    for _ in range(args.reps):
        prog.step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    prog.step()
    e1.record()
    torch.cuda.synchronize()
    status = int(prog.status.item())
    nwg = torch.cuda.get_device_properties(0).multi_processor_count
    nwg -= nwg % 8
    ts = np.zeros((nwg, SLOTS), np.uint64)
    if lab.ortmi_decoder_decode_step_stamps(ts.ctypes.data, nwg):
        raise RuntimeError("stamps read failed")
    base = int(ts[:, SLOTS - 1].min())  # the first workgroup's entry
    T = (ts.astype(np.int64) - base) * 10  # ns
    L, H = cfg.layers, cfg.heads
    attn = np.where(ts[:, 1] == 0)[0]  # no A stamp: attention workgroup
    proj = np.setdiff1d(np.arange(nwg), attn)
    NS = max(1, len(attn) // H)
    split0 = attn[::NS]
    print(f"decode program, {L} layers, total {args.total}, "
          f"{'cooperative' if args.cooperative else 'plain'} launch: status {status}, launch "
          f"{e0.elapsed_time(e1) * 1e3:.1f} us (HIP events); {len(proj)} projection and "
          f"{len(attn)} attention workgroups ({NS} key splits per head)")
    med = np.median
    rows = []
    for l in range(1, L):
        b = 1 + 8 * l
        prev_e = T[proj, b - 1].max()  # last E output stored, previous layer
        r = {
            "hop E->A": med(T[proj, b]) - prev_e,
            "A (norm + QKV)": med(T[proj, b + 1] - T[proj, b]),
            "hop A->attention": med(T[attn, b + 2]) - T[proj, b + 1].max(),
            "attend (RoPE, append, keys)": med(T[attn, b + 4] - T[attn, b + 2]),
            "merge in workgroup": med(T[attn, b + 5] - T[attn, b + 4]),
        }
        if NS > 1:
            r["split 0 waits for partials"] = med(T[split0, b + 6] - T[split0, b + 5])
            r["split 0 merge + store"] = med(T[split0, b + 3] - T[split0, b + 6])
        else:
            r["store"] = med(T[attn, b + 3] - T[attn, b + 5])
        r.update({
            "hop attention->C": med(T[proj, b + 2]) - T[split0, b + 3].max(),
            "C (o_proj)": med(T[proj, b + 3] - T[proj, b + 2]),
            "hop C->D": med(T[proj, b + 4]) - T[proj, b + 3].max(),
            "D (norm + gate/up + SwiGLU)": med(T[proj, b + 5] - T[proj, b + 4]),
            "hop D->E": med(T[proj, b + 6]) - T[proj, b + 5].max(),
            "E (down)": med(T[proj, b + 7] - T[proj, b + 6]),
            "layer (A ready to next A ready)": (med(T[proj, b + 8]) - med(T[proj, b])) if l + 1 < L
            else np.nan,
        })
        rows.append(r)
    keys = list(rows[0])
    print("| step | median over layers 1..L-1 (us) |")
    print("|---|---|")
    for k in keys:
        v = np.nanmedian([r[k] for r in rows]) / 1e3
        print(f"| {k} | {v:.2f} |")
    lm = med(T[:, 2 + 8 * L] - T[:, 1 + 8 * L]) / 1e3
    print(f"| lm_head phase | {lm:.2f} |")
    print(f"| whole launch (first start to last lm_head stamp) | "
          f"{(T[:, 2 + 8 * L].max() - T[:, 0].min()) / 1e3:.1f} |")
    entry = T[:, SLOTS - 1]
    print(f"| workgroup entries spread (first to last entry) | {(entry.max() - entry.min()) / 1e3:.2f} |")
    print(f"| entry to start (layer table, launch index) | {med(T[:, 0] - entry) / 1e3:.2f} |")
    print(f"| last lm_head stamp to greedy id written | "
          f"{(T[0, SLOTS - 2] - T[:, 2 + 8 * L].max()) / 1e3:.2f} |")
    print(f"| first entry to greedy id written | {(T[0, SLOTS - 2] - entry.min()) / 1e3:.1f} |")


if __name__ == "__main__":
    main()
