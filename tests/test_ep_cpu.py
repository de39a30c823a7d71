"""Plugin-EP boundary on the CPU: library loading, CreateEpFactories, GetCapability.

The harness host loads libonnxruntime_mi355x_ep.so exactly as ONNX Runtime's
plugin loader would (dlopen, CreateEpFactories, GetSupportedDevices, CreateEp,
GetCapability). Without a GPU the factory offers no device, so these sessions
are created with force_device and stop after GetCapability: they check which
nodes the EP claims and how it groups them into fused nodes (the reference's
claim tests, rust/src/ep.rs:119-895 and its #[cfg(test)] partition cases).
"""

import ctypes
import subprocess

import numpy as np
import pytest

from conftest import load_package

pkg = load_package()
from importlib import import_module  # noqa: E402

hx = import_module(pkg.__name__ + ".harness")
dec = import_module(pkg.__name__ + ".decoder")

F16, I32, I64, U8, F32 = hx.FLOAT16, hx.INT32, hx.INT64, hx.UINT8, hx.FLOAT


def session(g):
    return hx.Session(g, compile=False, force_device=True)


def mnb_node(g, x, out, N, K, name, bits=4, block=32, zp=False, dtype=F16):
    nb = K // block
    blob = block * bits // 8
    g.initializer(f"{name}.B", np.zeros((N, nb, blob), np.uint8))
    g.initializer(f"{name}.s", np.ones(N * nb, np.float16 if dtype == F16 else np.float32))
    ins = [x, f"{name}.B", f"{name}.s"]
    if zp:
        g.initializer(f"{name}.zp", np.zeros(N * ((nb * bits + 7) // 8), np.uint8))
        ins.append(f"{name}.zp")
    g.value(out, dtype, [1, -1, N])
    return g.node("MatMulNBits", ins, [out], domain="com.microsoft", name=name, K=K, N=N,
                  bits=bits, block_size=block)


def test_ep_exports_only_plugin_entry_points():
    out = subprocess.run(["nm", "-D", "--defined-only", pkg.EP_LIB], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    assert exported == {"CreateEpFactories", "ReleaseEpFactory"}


def test_create_ep_factories_contract():
    L = ctypes.CDLL(pkg.EP_LIB)
    create = L.CreateEpFactories
    create.restype = ctypes.c_void_p
    create.argtypes = [ctypes.c_char_p, ctypes.c_void_p, ctypes.c_void_p,
                       ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t,
                       ctypes.POINTER(ctypes.c_size_t)]
    release = L.ReleaseEpFactory
    release.restype = ctypes.c_void_p
    release.argtypes = [ctypes.c_void_p]
    h = hx.lib()
    h.hx_api_base.restype = ctypes.c_void_p
    base = h.hx_api_base()
    facs = (ctypes.c_void_p * 2)()
    n = ctypes.c_size_t(99)
    # No room for a factory: an error status, zero factories.
    st = create(b"MI355XExecutionProvider", base, None, facs, 0, ctypes.byref(n))
    assert st and n.value == 0
    # Normal registration: exactly one factory, released through ReleaseEpFactory.
    st = create(b"MI355XExecutionProvider", base, None, facs, 2, ctypes.byref(n))
    assert not st and n.value == 1 and facs[0]
    assert not release(facs[0])
    # A null API base yields no factory rather than a crash.
    n.value = 99
    assert not create(b"x", None, None, facs, 2, ctypes.byref(n)) and n.value == 0


def test_no_device_offered_without_gpu_blocks_compile():
    g = hx.Graph()
    g.value("x", F16, [1, 1, 64])
    mnb_node(g, "x", "y", 32, 64, "mm")
    g.io(["x"], ["y"])
    try:
        import torch
        has_gpu = torch.cuda.is_available()
    except Exception:
        has_gpu = False
    if has_gpu:
        pytest.skip("a GPU is visible")
    with pytest.raises(RuntimeError, match="offered no device"):
        hx.Session(g, compile=True)


def test_single_matmulnbits_is_one_partition():
    g = hx.Graph()
    g.value("x", F16, [1, -1, 64])
    mnb_node(g, "x", "y", 32, 64, "mm")
    g.io(["x"], ["y"])
    s = session(g)
    assert s.partitions() == [[0]]


@pytest.mark.parametrize("kw,claimed", [
    (dict(bits=4, block=32), True),
    (dict(bits=8, block=64), True),
    (dict(bits=4, block=16, zp=True), True),
    (dict(bits=4, block=128, dtype=F32), True),
    (dict(bits=3, block=32), False),     # quant.rs:1697-1703 rejects other widths
    (dict(bits=4, block=256), False),
])
def test_matmulnbits_claim_predicate(kw, claimed):
    g = hx.Graph()
    dtype = kw.get("dtype", F16)
    g.value("x", dtype, [1, 1, 256])
    mnb_node(g, "x", "y", 16, 256, "mm", **kw)
    g.io(["x"], ["y"])
    assert session(g).claimed(0) is claimed


def test_matmulnbits_bias_input_declined():
    g = hx.Graph()
    g.value("x", F16, [1, 1, 64])
    g.initializer("B", np.zeros((8, 2, 16), np.uint8))
    g.initializer("s", np.ones(16, np.float16))
    g.initializer("bias", np.ones(8, np.float16))
    g.value("y", F16, [1, 1, 8])
    g.node("MatMulNBits", ["x", "B", "s", "", "", "bias"], ["y"], domain="com.microsoft",
           K=64, N=8, bits=4, block_size=32)
    g.io(["x"], ["y"])
    assert not session(g).claimed(0)


def gbq_graph(bits=4, block=16, gather_axis=0, quantize_axis=1, sdtype=F16, odtype=F16,
              idtype=I64, zp=False):
    g = hx.Graph()
    g.value("ids", idtype, [1, -1])
    g.initializer("table", np.zeros((40, 16), np.uint8))  # V=40, D=32
    g.initializer("scales", np.ones((40, 32 // block if block <= 32 else 1),
                                    np.float16 if sdtype == F16 else np.float32))
    inputs = ["table", "ids", "scales"]
    if zp:
        g.initializer("zp", np.full((40, 1), 0x88, np.uint8))
        inputs.append("zp")
    g.value("emb", odtype, [1, -1, 32])
    g.node("GatherBlockQuantized", inputs, ["emb"], domain="com.microsoft", bits=bits,
           block_size=block, gather_axis=gather_axis, quantize_axis=quantize_axis)
    g.io(["ids"], ["emb"])
    return g


@pytest.mark.parametrize("kw,claimed", [
    (dict(), True),
    (dict(idtype=I32, zp=True), True),
    (dict(block=32, sdtype=F32, odtype=F32), True),
    (dict(bits=8), False),                 # quant.rs:1736-1739: 4-bit only
    (dict(gather_axis=1), False),          # quant.rs:1740-1743
    (dict(quantize_axis=0), False),
    (dict(block=8), False),                # quant.rs:1744-1747: block >= 16
    (dict(sdtype=F32, odtype=F16), False), # quant.rs:1723-1730: scales dtype = output dtype
    (dict(idtype=F32), False),
])
def test_gather_block_quantized_claim_predicate(kw, claimed):
    """Claim contract of gather_block_quantized_claim (rust/src/ops/quant.rs:1713-1749)."""
    assert session(gbq_graph(**kw)).claimed(0) is claimed


def gqa_graph(hd=64, extra=None, inputs_extra=(), dtype=F16, at=None):
    """One GroupQueryAttention node (decode, in-op RoPE). inputs_extra are appended
    after sin (from input 9); `at` maps an input index >= 9 to (name, dtype, dims)."""
    g = hx.Graph()
    H, KV, cap = 4, 2, 32
    npdt = np.float16 if dtype == F16 else np.float32
    g.value("q", dtype, [1, 1, H * hd])
    g.value("k", dtype, [1, 1, KV * hd])
    g.value("v", dtype, [1, 1, KV * hd])
    g.value("pk", dtype, [1, KV, cap, hd])
    g.value("pv", dtype, [1, KV, cap, hd])
    g.value("sl", I32, [1])
    g.value("tot", I32, [1])
    g.initializer("cos", np.ones((64, hd // 2), npdt))
    g.initializer("sin", np.zeros((64, hd // 2), npdt))
    for name, dt, dims in inputs_extra:
        g.value(name, dt, dims)
    g.value("o", dtype, [1, 1, H * hd])
    g.value("ok", dtype, [1, KV, cap, hd])
    g.value("ov", dtype, [1, KV, cap, hd])
    ins = ["q", "k", "v", "pk", "pv", "sl", "tot", "cos", "sin"] + [n for n, _, _ in inputs_extra]
    for i, (name, dt, dims) in sorted((at or {}).items()):
        g.value(name, dt, dims)
        ins += [""] * (i - len(ins)) + [name]
    attrs = dict(num_heads=H, kv_num_heads=KV, do_rotary=1)
    attrs.update(extra or {})
    g.node("GroupQueryAttention", ins, ["o", "ok", "ov"], domain="com.microsoft", **attrs)
    g.io([n for n in ins if n and n not in ("cos", "sin")], ["o", "ok", "ov"])
    return g


@pytest.mark.parametrize("hd,extra,ins,claimed", [
    (128, None, (), True),
    (64, None, (), True),
    (96, None, (), True),                                   # generic kernels: multiples of 16
    (72, None, (), False),                                  # head size without a kernel
    (128, dict(softcap=30.0), (), False),
    (128, dict(local_window_size=128), (), False),          # window with no bias to carry it
    (128, dict(sliding_window_cache=1, local_window_size=16), (), True),   # cap 32 >= 16
    (128, dict(sliding_window_cache=1, local_window_size=64), (), False),  # window > capacity
    (128, dict(sliding_window_cache=1), (), False),         # no window
    (128, dict(smooth_softmax=1), (), False),
    (128, dict(kv_num_heads=3), (), False),                 # 4 % 3 != 0
    (128, None, (("pos", I64, [1, 1]),), False),            # position_ids with in-op rotary
    (128, dict(do_rotary=0), (("pos", I64, [1, 1]),), True),  # ignored without it
])
def test_gqa_claim_predicate(hd, extra, ins, claimed):
    assert session(gqa_graph(hd, extra, ins)).claimed(0) is claimed


HD = 64


@pytest.mark.parametrize("dtype,extra,at,claimed", [
    (F32, None, {}, True),                                                     # fp32 tensors
    (F16, None, {10: ("bias", F16, [1, 1, 1, 32])}, True),                     # attention_bias
    (F16, None, {10: ("bias", F16, [1, 4, 1, 32])}, True),                     # per-head bias
    (F16, None, {10: ("bias", F16, [1, 3, 1, 32])}, False),                    # 3 heads of 4
    (F16, None, {10: ("bias", F16, [1, 32])}, False),                          # rank 2
    (F16, None, {10: ("bias", F32, [1, 1, 1, 32])}, False),                    # dtype mismatch
    (F16, dict(local_window_size=8), {10: ("bias", F16, [1, 1, 1, 32])}, True),  # bias carries it
    (F16, None, {14: ("qn", F16, [HD]), 15: ("kn", F16, [HD])}, True),         # QK-norm
    (F32, None, {14: ("qn", F32, [HD]), 15: ("kn", F32, [HD])}, True),
    (F16, None, {14: ("qn", F16, [HD])}, False),                               # q without k
    (F16, None, {14: ("qn", F16, [HD // 2]), 15: ("kn", F16, [HD // 2])}, False),
    (F16, None, {11: ("sink", F16, [4])}, False),                              # head_sink
    (F16, None, {12: ("ks", F32, [1]), 13: ("vs", F32, [1])}, False),          # quantized KV
    (F16, dict(k_quant_type="PER_TENSOR"), {}, False),
    (F32, dict(sliding_window_cache=1, local_window_size=8), {}, True),        # fp32 sliding
    (F16, dict(sliding_window_cache=1, local_window_size=8),                   # with a bias
     {10: ("bias", F16, [1, 1, 1, 32])}, False),
])
def test_gqa_claim_optional_inputs(dtype, extra, at, claimed):
    """The optional GroupQueryAttention inputs the reference claims
    (rust/src/ops/attention.rs:1520-1745): attention_bias (input 10, rank 4, output
    dtype), QK-norm weights (inputs 14/15, together, shape [head_size]), fp32; and
    the ones it declines (head_sink, quantized KV, ...)."""
    assert session(gqa_graph(HD, extra, (), dtype, at)).claimed(0) is claimed


def test_unsupported_node_splits_partitions():
    # mm0 -> Softmax (no kernel) -> mm1: two fused nodes around the declined op.
    g = hx.Graph()
    g.value("x", F16, [1, 1, 64])
    mnb_node(g, "x", "a", 64, 64, "mm0")
    g.value("b", F16, [1, 1, 64])
    g.node("Softmax", ["a"], ["b"], axis=-1)
    mnb_node(g, "b", "y", 32, 64, "mm1")
    g.io(["x"], ["y"])
    s = session(g)
    assert not s.claimed(1)
    assert sorted(s.partitions()) == [[0], [2]]


def test_clusters_stay_convex():
    # a = mm0(x); b = Softmax(a) [declined]; y = Add(a, c) with c = mm1(b).
    # mm0 and the Add cannot share a fused node: the path mm0 -> Softmax -> mm1 -> Add
    # leaves the cluster and re-enters it, which would make the fused graph cyclic.
    g = hx.Graph()
    g.value("x", F16, [1, 1, 64])
    mnb_node(g, "x", "a", 64, 64, "mm0")
    g.value("b", F16, [1, 1, 64])
    g.node("Softmax", ["a"], ["b"], axis=-1)
    mnb_node(g, "b", "c", 64, 64, "mm1")
    g.value("y", F16, [1, 1, 64])
    g.node("Add", ["a", "c"], ["y"])
    g.io(["x"], ["y"])
    s = session(g)
    parts = s.partitions()
    assert not s.claimed(1)
    where = {n: i for i, p in enumerate(parts) for n in p}
    assert where[0] != where[3]
    # every claimed node is in exactly one partition
    assert sorted(n for p in parts for n in p) == [0, 2, 3]


def test_independent_branches_fuse_together():
    g = hx.Graph()
    g.value("x", F16, [1, 1, 64])
    mnb_node(g, "x", "a", 64, 64, "mm0")
    mnb_node(g, "x", "b", 64, 64, "mm1")
    g.value("y", F16, [1, 1, 64])
    g.node("Add", ["a", "b"], ["y"])
    g.io(["x"], ["y"])
    assert [sorted(p) for p in session(g).partitions()] == [[0, 1, 2]]


def test_broadcasting_add_declined():
    g = hx.Graph()
    g.value("a", F16, [1, 4, 64])
    g.value("b", F16, [1, 1, 64])
    g.value("y", F16, [1, 4, 64])
    g.node("Add", ["a", "b"], ["y"])
    g.io(["a", "b"], ["y"])
    assert not session(g).claimed(0)


def test_norm_claims():
    g = hx.Graph()
    g.value("x", F16, [1, -1, 1536])
    g.value("r", F16, [1, -1, 1536])
    g.initializer("w", np.ones(1536, np.float16))
    for v in ("y0", "y1", "res", "y2", "mean"):
        g.value(v, F16, [1, -1, 1536])
    g.node("SimplifiedLayerNormalization", ["x", "w"], ["y0"], epsilon=1e-6, axis=-1)
    g.node("SkipSimplifiedLayerNormalization", ["x", "r", "w"], ["y1", "", "", "res"],
           domain="com.microsoft", epsilon=1e-6)
    g.node("SkipSimplifiedLayerNormalization", ["x", "r", "w"], ["y2", "mean"],
           domain="com.microsoft", epsilon=1e-6)
    # mean / inv_std_var declared but read by nobody (a transformers.js / Mobius
    # export): claimed, as rust/src/ops/norm.rs:586-594 claims it.
    for v in ("y3", "mean3", "istd3", "res3", "y4", "istd4", "res4", "z4"):
        g.value(v, F16, [1, -1, 1536])
    g.node("SkipSimplifiedLayerNormalization", ["x", "r", "w"], ["y3", "mean3", "istd3", "res3"],
           domain="com.microsoft", epsilon=1e-6)
    # inv_std_var read by another node: declined (it is not produced).
    g.node("SkipSimplifiedLayerNormalization", ["x", "r", "w"], ["y4", "", "istd4", "res4"],
           domain="com.microsoft", epsilon=1e-6)
    g.node("Add", ["y4", "istd4"], ["z4"])
    g.io(["x", "r"], ["y0", "y1", "res", "y2", "mean", "y3", "res3", "z4", "res4"])
    s = session(g)
    assert s.claimed(0) and s.claimed(1) and not s.claimed(2)
    assert s.claimed(3) and not s.claimed(4)


@pytest.mark.parametrize("dtype,attrs,out_dtype,claimed", [
    (F16, dict(axis=-1, keepdims=0), I64, True),
    (F16, dict(axis=2, keepdims=1), I64, True),
    (F32, dict(axis=-1), I64, True),          # keepdims defaults to 1
    (hx.BFLOAT16, dict(axis=2, keepdims=0, select_last_index=0), I64, True),
    (F16, dict(axis=1), I64, True),           # any axis (reduction.rs:582-630)
    (F16, dict(axis=0), I64, True),           # the default axis is 0
    (F16, dict(axis=3), I64, False),          # out of range (reduction.rs:610-617)
    (F16, dict(axis=-1, keepdims=2), I64, False),
    (F16, dict(axis=-1, select_last_index=1), I64, True),
    (F16, dict(axis=-1, select_last_index=2), I64, False),
    (I32, dict(axis=-1), I64, False),         # float inputs only
])
def test_argmax_claim_predicate(dtype, attrs, out_dtype, claimed):
    g = hx.Graph()
    g.value("x", dtype, [1, -1, 1000])
    g.value("y", out_dtype, [1, -1] if attrs.get("keepdims", 1) == 0 else [1, -1, 1])
    g.node("ArgMax", ["x"], ["y"], **attrs)
    g.io(["x"], ["y"])
    assert session(g).claimed(0) is claimed


def test_decoder_graph_with_argmax_fully_claimed():
    cfg = dec.DecoderConfig(layers=2, hidden=256, heads=4, kv_heads=2, head_dim=64, inter=512,
                            vocab=1000, max_pos=256)
    w = dec.make_weights(cfg, seed=0)
    g = dec.build_graph(cfg, w, cap=64, argmax=True)
    parts = session(g).partitions()
    assert len(parts) == 1 and len(parts[0]) == g.n_nodes
    assert g.n_nodes == 1 + cfg.layers * 13 + 3


def test_decoder_graph_with_declared_norm_stats_fully_claimed():
    """Declared-but-unread mean / inv_std_var outputs of every SkipSimplifiedLayerNorm
    keep the decoder one fused node (rust/src/ops/norm.rs:586-594)."""
    cfg = dec.DecoderConfig(layers=3, hidden=256, heads=4, kv_heads=2, head_dim=64, inter=512,
                            vocab=1000, max_pos=256)
    w = dec.make_weights(cfg, seed=0)
    g = dec.build_graph(cfg, w, cap=64, norm_stats=True)
    parts = session(g).partitions()
    assert len(parts) == 1 and len(parts[0]) == g.n_nodes


def test_decoder_graph_fully_claimed_as_one_fused_node():
    cfg = dec.DecoderConfig(layers=2, hidden=256, heads=4, kv_heads=2, head_dim=64, inter=512,
                            vocab=1000, max_pos=256)
    w = dec.make_weights(cfg, seed=0)
    g = dec.build_graph(cfg, w, cap=64)
    s = session(g)
    parts = s.partitions()
    assert len(parts) == 1
    assert len(parts[0]) == g.n_nodes
    # the ops of one layer: 2 norms, 7 MatMulNBits, GQA, Sigmoid + 2 Mul
    assert g.n_nodes == 1 + cfg.layers * 13 + 2


def test_decoder_graph_with_layer_metadata_splits_by_span(monkeypatch):
    """The decoder's residual outputs named in metadata (one per layer, the last
    being the final norm's): span 2 over 5 layers cuts after layers 2 and 4."""
    cfg = dec.DecoderConfig(layers=5, hidden=256, heads=4, kv_heads=2, head_dim=64, inter=512,
                            vocab=1000, max_pos=256)
    w = dec.make_weights(cfg, seed=0)
    g = dec.build_graph(cfg, w, cap=64, layer_metadata=True)
    monkeypatch.delenv("ONNXRUNTIME_EP_MLX_LAYER_PARTITIONS", raising=False)
    assert [len(p) for p in session(g).partitions()] == [g.n_nodes]
    monkeypatch.setenv("ONNXRUNTIME_EP_MLX_LAYER_PARTITIONS", "2")
    parts = session(g).partitions()
    # gather + 13 nodes per layer; layer l's residual comes out of layer l+1's first
    # norm, so a cut after two layers holds 1 + 2*13 + 1 nodes.
    assert [len(p) for p in parts] == [28, 26, 14]
    assert sum(len(p) for p in parts) == g.n_nodes


def test_default_memory_device_slot_matches_reference_binding():
    """OrtEp::GetDefaultMemoryDevice is bound by the reference as
    fn(*const OrtEp, *mut *const OrtMemoryDevice) -> *mut OrtStatus
    (rust/src/ep.rs:104-113): a status return and an out-parameter."""
    import os
    import re

    text = open(os.path.join(os.path.dirname(pkg.EP_LIB), "..", "..", "include",
                             "ort_plugin_ep_abi.h")).read()
    m = re.search(r"(\w+\s*\*)\s*\(\*GetDefaultMemoryDevice\)\(([^)]*)\)", text)
    assert m, "GetDefaultMemoryDevice slot missing from the OrtEp declaration"
    ret, params = m.group(1).replace(" ", ""), " ".join(m.group(2).split())
    assert ret == "OrtStatus*"
    assert params == "const struct OrtEp* this_ptr, const OrtMemoryDevice** device"


def test_default_memory_device_is_cpu_and_foreign_allocators_declined():
    """The EP reports CPU memory as its default device (the reference's answer) and
    hands out no allocator for a memory info that is not its own."""
    g = hx.Graph()
    mnb_node(g, "x", "y", 64, 64, "l")
    g.value("x", F16, [1, -1, 64])
    g.io(["x"], ["y"])
    s = session(g)
    assert s.default_memory_device_is_cpu()
    assert s.allocator_check("Cpu", 0) is None
    assert s.allocator_check("Cuda", 0) is None


@pytest.mark.parametrize("qwidth,packed,claimed", [
    (4 * 128, False, True),
    (4 * 128 + 8, False, False),        # query width not a multiple of num_heads
    (4 * 72, False, False),             # head size 72 has no kernel
    ((4 + 2 * 2) * 64, True, True),     # packed QKV, head size 64
    ((4 + 2 * 2) * 64 + 2, True, False),
])
def test_gqa_claim_checks_head_size_without_past(qwidth, packed, claimed):
    """Without past inputs the head size comes from the query width and the head
    counts (rust/src/ops/attention.rs:1667-1683): a width that does not divide, or
    a head size the kernels lack, is declined at claim time instead of failing in
    Compute."""
    H, KV = 4, 2
    g = hx.Graph()
    g.value("q", F16, [1, 7, qwidth])
    hd = qwidth // (H + 2 * KV) if packed else qwidth // H
    if not packed:
        g.value("k", F16, [1, 7, KV * hd])
        g.value("v", F16, [1, 7, KV * hd])
    g.value("sl", I32, [1])
    g.value("tot", I32, [1])
    g.value("o", F16, [1, 7, H * hd])
    ins = ["q", "", "", "", "", "sl", "tot"] if packed else ["q", "k", "v", "", "", "sl", "tot"]
    g.node("GroupQueryAttention", ins, ["o"], domain="com.microsoft", num_heads=H,
           kv_num_heads=KV, do_rotary=0)
    g.io([n for n in ins if n], ["o"])
    assert session(g).claimed(0) is claimed


# ------------------------------------------------- layer groups of large decoders ---

def layered_graph(layers, residual="add", metadata=None):
    """A decoder-shaped graph, per layer: q/k/v MatMulNBits -> GroupQueryAttention
    (present key/value outputs) -> o_proj MatMulNBits -> Add (residual) ->
    MatMulNBits -> Add (residual, the layer's output x{l+1}). residual="skipnorm"
    puts a SkipSimplifiedLayerNormalization in place of the first Add;
    residual="none" replaces both Adds by such norms (no Add in the layer)."""
    g = hx.Graph()
    H, KV, hd, cap = 2, 1, 64, 16
    D = H * hd
    g.value("x0", F16, [1, 1, D])
    g.value("sl", I32, [1])
    g.value("tot", I32, [1])
    g.value("gamma", F16, [D])
    g.initializer("gamma", np.ones(D, np.float16))
    inputs = ["x0", "sl", "tot"]
    outputs = []
    for l in range(layers):
        x = f"x{l}"
        mnb_node(g, x, f"q{l}", D, D, f"L{l}.q")
        mnb_node(g, x, f"k{l}", KV * hd, D, f"L{l}.k")
        mnb_node(g, x, f"v{l}", KV * hd, D, f"L{l}.v")
        for n in (f"pk{l}", f"pv{l}", f"ok{l}", f"ov{l}"):
            g.value(n, F16, [1, KV, cap, hd])
        g.value(f"a{l}", F16, [1, 1, D])
        g.node("GroupQueryAttention", [f"q{l}", f"k{l}", f"v{l}", f"pk{l}", f"pv{l}", "sl", "tot"],
               [f"a{l}", f"ok{l}", f"ov{l}"], domain="com.microsoft", num_heads=H,
               kv_num_heads=KV, name=f"L{l}.attn")
        mnb_node(g, f"a{l}", f"o{l}", D, D, f"L{l}.o")
        g.value(f"h{l}", F16, [1, 1, D])
        if residual == "add":
            g.node("Add", [x, f"o{l}"], [f"h{l}"], name=f"L{l}.add1")
        else:
            g.value(f"n{l}", F16, [1, 1, D])
            g.node("SkipSimplifiedLayerNormalization", [f"o{l}", x, "gamma"],
                   [f"n{l}", "", "", f"h{l}"], domain="com.microsoft", name=f"L{l}.norm")
        mnb_node(g, f"h{l}", f"m{l}", D, D, f"L{l}.mlp")
        g.value(f"x{l + 1}", F16, [1, 1, D])
        if residual == "none":
            g.node("SkipSimplifiedLayerNormalization", [f"m{l}", f"h{l}", "gamma"],
                   [f"y{l}", "", "", f"x{l + 1}"], domain="com.microsoft", name=f"L{l}.norm2")
            g.value(f"y{l}", F16, [1, 1, D])
            outputs.append(f"y{l}")
        else:
            g.node("Add", [f"h{l}", f"m{l}"], [f"x{l + 1}"], name=f"L{l}.add2")
        inputs += [f"pk{l}", f"pv{l}"]
        outputs += [f"ok{l}", f"ov{l}"]
    outputs.append(f"x{layers}")
    if metadata is not None:
        g.metadata("onnxruntime_ep_mlx.layer_boundary_outputs", metadata)
    g.io(inputs, outputs)
    return g


NODES_PER_LAYER = 8


def _sizes(g):
    return [len(p) for p in session(g).partitions()]


def test_layer_partitions_auto_keeps_decoder_whole(monkeypatch):
    """Unset / "auto": one fused node at any depth (the reference splits decoders
    of 23+ layers, rust/src/ep.rs:365-374; on MI355X the whole-step decode program
    needs the whole decoder in one fused node)."""
    monkeypatch.delenv("ONNXRUNTIME_EP_MLX_LAYER_PARTITIONS", raising=False)
    assert _sizes(layered_graph(24)) == [24 * NODES_PER_LAYER]
    monkeypatch.setenv("ONNXRUNTIME_EP_MLX_LAYER_PARTITIONS", "auto")
    assert _sizes(layered_graph(24)) == [24 * NODES_PER_LAYER]


@pytest.mark.parametrize("value,sizes", [
    ("5", [40, 40, 40, 40, 32]),   # 23 inferred boundaries (between 24 attention nodes)
    (" 8 ", [64, 64, 64]),
    ("+12", [96, 96]),
    ("1", [8] * 23 + [8]),
    ("0", [192]), ("off", [192]), ("false", [192]), ("invalid", [192]), ("-3", [192]),
])
def test_layer_partitions_inferred_boundaries_span(monkeypatch, value, sizes):
    """Inferred boundaries are each layer's last residual Add (the reference's
    structural test, rust/src/ep.rs:539-569); the span override follows
    select_layer_span's grammar (rust/src/ep.rs:360-375, tests 522-537)."""
    monkeypatch.setenv("ONNXRUNTIME_EP_MLX_LAYER_PARTITIONS", value)
    assert _sizes(layered_graph(24)) == sizes


def test_layer_partitions_split_after_the_last_residual_add(monkeypatch):
    monkeypatch.setenv("ONNXRUNTIME_EP_MLX_LAYER_PARTITIONS", "2")
    g = layered_graph(4)
    parts = session(g).partitions()
    # Node order of the graph: 8 per layer, add2 last; the cut follows L1.add2 and
    # the last layer (no attention after it) stays with the remainder.
    assert [len(p) for p in parts] == [16, 16]
    assert parts[0] == list(range(16)) and parts[1] == list(range(16, 32))


def test_layer_partitions_metadata_takes_precedence(monkeypatch):
    """Metadata names the boundaries (here the first residual Add of every layer,
    which inference would not pick) and is used instead of inference."""
    import json

    monkeypatch.setenv("ONNXRUNTIME_EP_MLX_LAYER_PARTITIONS", "3")
    names = [f"h{layer}" for layer in range(9)]
    parts = session(layered_graph(9, metadata=json.dumps(names))).partitions()
    assert [len(p) for p in parts] == [22, 24, 24, 2]
    # Each cut follows an add1 node (index 5 of its layer).
    assert [p[-1] % NODES_PER_LAYER for p in parts[:-1]] == [5, 5, 5]


@pytest.mark.parametrize("metadata,sizes", [
    ('["x1", "x3"]', [8, 16, 8]),                       # span 1: cut after each named output
    ('[]', [32]),                                       # empty list: no boundaries, no inference
    ('not json', [32]),                                 # invalid: ignored, no inference
    ('["x1", 3]', [32]),                                # not all strings
    ('["x\\u0031", "x\\u00333"]', [8, 24]),            # \u escapes decode ("x1", "x33" absent)
    (' [ "x2" , "" ] ', [16, 16]),                      # whitespace; empty names dropped
])
def test_layer_partitions_metadata_parsing(monkeypatch, metadata, sizes):
    monkeypatch.setenv("ONNXRUNTIME_EP_MLX_LAYER_PARTITIONS", "1")
    assert _sizes(layered_graph(4, metadata=metadata)) == sizes


@pytest.mark.parametrize("residual", ["skipnorm", "none"])
def test_layer_partitions_inference_needs_a_residual_add_in_every_layer(monkeypatch, residual):
    """With SkipSimplifiedLayerNormalization carrying the residual the second Add
    is still found ("skipnorm"); with no Add between two attention nodes
    ("none") inference yields no boundaries and the graph stays whole."""
    monkeypatch.setenv("ONNXRUNTIME_EP_MLX_LAYER_PARTITIONS", "2")
    sizes = _sizes(layered_graph(6, residual=residual))
    if residual == "skipnorm":
        assert sizes == [16, 16, 16]
    else:
        assert sizes == [48]


@pytest.mark.parametrize("dtype,d,attrs,claimed", [
    (F16, 128, {}, True),
    (F32, 128, {}, True),                                  # fp32: the generic kernels
    (F16, 96, {}, True),                                   # head sizes 16k <= 256
    (F16, 72, {}, False),
    (F16, 512, {}, False),
    (F16, 128, dict(local_window_size=64), False),         # declined by the reference too
    (F16, 128, dict(softcap=30.0), False),
    # cache dtype names: the caches are the activation dtype, only sub-byte packings
    # are declined (attention.rs:2759-2765)
    (F16, 128, dict(k_cache_dtype="int8", v_cache_dtype="float8e4m3fn"), True),
    (F16, 128, dict(k_cache_dtype="int4"), False),
    (F16, 128, dict(v_cache_dtype="float4e2m1"), False),
    (F16, 128, dict(cache_tensor=hx.INT8), False),         # caches must share the dtype
    (F16, 128, dict(cache_tensor=hx.BFLOAT16), False),
])
def test_paged_attention_claim_forms(dtype, d, attrs, claimed):
    """PagedAttention claim (rust/src/ops/attention.rs:2746-2977): any float dtype, the
    head sizes the kernels take, caches in the activation dtype."""
    g = hx.Graph()
    H, KV, nb, blk, batch, maxb = 4, 2, 8, 4, 2, 4
    attrs = dict(attrs)
    cdt = attrs.pop("cache_tensor", dtype)
    g.value("q", dtype, [-1, H * d])
    g.value("k", dtype, [-1, KV * d])
    g.value("v", dtype, [-1, KV * d])
    g.value("kc", cdt, [nb, blk, KV, d])
    g.value("vc", cdt, [nb, blk, KV, d])
    g.value("cum", I32, [batch + 1])
    g.value("past", I32, [batch])
    g.value("bt", I32, [batch, maxb])
    g.value("o", dtype, [-1, H * d])
    g.node("PagedAttention", ["q", "k", "v", "kc", "vc", "cum", "past", "bt"], ["o"],
           domain="com.microsoft", num_heads=H, kv_num_heads=KV, **attrs)
    g.io(["q", "k", "v", "kc", "vc", "cum", "past", "bt"], ["o"])
    assert session(g).claimed(0) is claimed


@pytest.mark.parametrize("domain,xshape,pos,cos_shape,attrs,claimed", [
    ("com.microsoft", [2, 7, 256], ("pos", I64, [2, 7]), [64, 32], dict(num_heads=4), True),
    # partial rotary: a cache narrower than head_size / 2, the tail keeps its values
    ("com.microsoft", [2, 7, 256], ("pos", I64, [2, 7]), [64, 16], dict(num_heads=4), True),
    ("com.microsoft", [2, 7, 256], ("pos", I64, [1]), [64, 16], dict(num_heads=4), True),
    ("", [2, 4, 7, 64], ("pos", I64, [2, 7]), [64, 8], {}, True),
    ("", [2, 7, 256], None, [2, 7, 32], dict(num_heads=4), True),   # per-token cache
    ("", [2, 7, 256], ("pos", I64, [1]), [64, 32], dict(num_heads=4), False),  # [1]: ms only
    ("com.microsoft", [2, 7, 256], None, [2, 7, 32], dict(num_heads=4), False),  # ms needs ids
    ("com.microsoft", [2, 7, 256], ("pos", I32, [2, 7]), [64, 32], dict(num_heads=4), False),
    ("com.microsoft", [2, 7, 256], ("pos", I64, [2, 7]), [64, 64], dict(num_heads=4), False),
    ("com.microsoft", [2, 7, 256], ("pos", I64, [2, 7]), [64, 16],
     dict(num_heads=0, rotary_embedding_dim=32), False),  # head size not inferable
    ("com.microsoft", [2, 7, 256], ("pos", I64, [2, 7]), [64, 32], dict(num_heads=0), True),
])
def test_rotary_claim_predicate(domain, xshape, pos, cos_shape, attrs, claimed):
    """The RotaryEmbedding claim contract of rust/src/ops/attention.rs:2158-2264: the
    two input orders, position_ids [B,S] (or [1] in com.microsoft) or absent with a
    per-token cache, the head size inferred from the cache when num_heads = 0, and a
    cache narrower than head_size / 2 (partial rotary). position_ids must be int64,
    the type both ONNX schemas give it."""
    g = hx.Graph()
    g.value("x", F16, xshape)
    g.value("y", F16, xshape)
    g.value("cos", F16, cos_shape)
    g.value("sin", F16, cos_shape)
    ins = ["x", "", "cos", "sin"] if domain else ["x", "cos", "sin"]
    io_in = ["x", "cos", "sin"]
    if pos is not None:
        g.value(*pos)
        io_in.append(pos[0])
        if domain:
            ins[1] = pos[0]
        else:
            ins.append(pos[0])
    g.node("RotaryEmbedding", ins, ["y"], domain=domain, **attrs)
    g.io(io_in, ["y"])
    assert session(g).claimed(0) is claimed
