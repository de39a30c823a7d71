"""Python face of the harness host (libortmi_harness.so).

The harness stands in for ONNX Runtime's plugin loader: it builds a graph, loads
the EP library through CreateEpFactories and drives GetCapability / Compile /
Compute over the plugin C ABI. Values are placed as ONNX Runtime places them for
a fused node: on the EP's default memory device (HBM for this EP; CPU memory with
ORTMI_EP_MEMORY=cpu). Feeds and bound outputs on that side (device tensors with
the HBM EP: the IOBinding case) are used in place; feeds on the other side are
copied over through the EP's data transfer before Compute, outputs bound on the
other side are produced there and copied back after it, and outputs nobody binds
are allocated on the EP's side.
"""

from __future__ import annotations

import ctypes
import os

import numpy as np

from . import EP_LIB, LIB_DIR

HARNESS_LIB = os.path.join(LIB_DIR, "libortmi_harness.so")

FLOAT, UINT8, INT8, INT32, INT64, FLOAT16, BFLOAT16 = 1, 2, 3, 6, 7, 10, 16
_NP = {np.dtype(np.float32): FLOAT, np.dtype(np.uint8): UINT8, np.dtype(np.int8): INT8,
       np.dtype(np.int32): INT32, np.dtype(np.int64): INT64, np.dtype(np.float16): FLOAT16}
_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(HARNESS_LIB):
            raise FileNotFoundError(f"{HARNESS_LIB} is missing: run onnxruntime-mlx_amd/build.py")
        L = ctypes.CDLL(HARNESS_LIB)
        vp, i64p, cp = ctypes.c_void_p, ctypes.POINTER(ctypes.c_int64), ctypes.c_char_p
        cpp = ctypes.POINTER(ctypes.c_char_p)
        sig = {
            "hx_last_error": (cp, []),
            "hx_graph_new": (vp, []),
            "hx_graph_free": (None, [vp]),
            "hx_graph_add_value": (ctypes.c_int, [vp, cp, ctypes.c_int, ctypes.c_int, i64p]),
            "hx_graph_add_initializer": (ctypes.c_int, [vp, cp, ctypes.c_int, ctypes.c_int, i64p,
                                                        vp, ctypes.c_size_t]),
            "hx_graph_add_node": (ctypes.c_int, [vp, cp, cp, cp, ctypes.c_int, ctypes.c_int, cpp,
                                                 ctypes.c_int, cpp]),
            "hx_node_attr_int": (ctypes.c_int, [vp, ctypes.c_int, cp, ctypes.c_int64]),
            "hx_node_attr_float": (ctypes.c_int, [vp, ctypes.c_int, cp, ctypes.c_float]),
            "hx_node_attr_string": (ctypes.c_int, [vp, ctypes.c_int, cp, cp]),
            "hx_node_attr_ints": (ctypes.c_int, [vp, ctypes.c_int, cp, ctypes.c_int, i64p]),
            "hx_graph_set_io": (ctypes.c_int, [vp, ctypes.c_int, cpp, ctypes.c_int, cpp]),
            "hx_graph_set_metadata": (ctypes.c_int, [vp, cp, cp]),
            "hx_session_new": (vp, [vp, cp, cp, ctypes.c_int, ctypes.c_int]),
            "hx_session_free": (None, [vp]),
            "hx_session_num_partitions": (ctypes.c_int, [vp]),
            "hx_session_partition_size": (ctypes.c_int, [vp, ctypes.c_int]),
            "hx_session_partition_node": (ctypes.c_int, [vp, ctypes.c_int, ctypes.c_int]),
            "hx_session_node_claimed": (ctypes.c_int, [vp, ctypes.c_int]),
            "hx_session_bind_output": (ctypes.c_int, [vp, cp, vp]),
            "hx_session_set_input": (ctypes.c_int, [vp, cp, vp, ctypes.c_int, ctypes.c_int, i64p]),
            "hx_session_run": (ctypes.c_int, [vp]),
            "hx_session_get_output": (ctypes.c_int, [vp, cp, ctypes.POINTER(vp),
                                                     ctypes.POINTER(ctypes.c_int), i64p]),
            "hx_session_default_memory_device": (ctypes.c_int, [vp, ctypes.POINTER(ctypes.c_int)]),
            "hx_session_memory_device": (ctypes.c_int, [vp, ctypes.POINTER(ctypes.c_int),
                                                        ctypes.POINTER(ctypes.c_uint32),
                                                        ctypes.POINTER(ctypes.c_int)]),
            "hx_session_copies": (ctypes.c_int64, [vp]),
            "hx_factory_allocator_check": (ctypes.c_int, [vp, cp, ctypes.c_int, ctypes.c_size_t]),
            "hx_factory_data_transfer_copy": (ctypes.c_int, [vp, vp, vp, ctypes.c_int,
                                                             ctypes.c_int, i64p]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _err() -> str:
    return lib().hx_last_error().decode(errors="replace")


def _dims(d):
    arr = (ctypes.c_int64 * max(1, len(d)))(*[int(x) for x in d])
    return arr


def _strs(names):
    arr = (ctypes.c_char_p * max(1, len(names)))(*[(n or "").encode() for n in names])
    return arr


class Graph:
    """An in-memory graph in ONNX terms (value infos, initializers, nodes)."""

    def __init__(self):
        self._free = lib().hx_graph_free  # held so teardown never needs module globals
        self.h = lib().hx_graph_new()
        self.n_nodes = 0

    def __del__(self):
        if getattr(self, "h", None):
            self._free(self.h)
            self.h = None

    def value(self, name, dtype, dims):
        lib().hx_graph_add_value(self.h, name.encode(), dtype, len(dims), _dims(dims))

    def initializer(self, name, array: np.ndarray):
        a = np.ascontiguousarray(array)
        lib().hx_graph_add_initializer(self.h, name.encode(), _NP[a.dtype], a.ndim,
                                       _dims(a.shape), a.ctypes.data_as(ctypes.c_void_p), a.nbytes)

    def node(self, op, inputs, outputs, domain="", name=None, since=1, **attrs):
        idx = lib().hx_graph_add_node(self.h, op.encode(), domain.encode(),
                                      (name or f"{op}_{self.n_nodes}").encode(), since,
                                      len(inputs), _strs(inputs), len(outputs), _strs(outputs))
        self.n_nodes += 1
        for k, v in attrs.items():
            if isinstance(v, bool) or isinstance(v, (int, np.integer)):
                lib().hx_node_attr_int(self.h, idx, k.encode(), int(v))
            elif isinstance(v, float):
                lib().hx_node_attr_float(self.h, idx, k.encode(), v)
            elif isinstance(v, str):
                lib().hx_node_attr_string(self.h, idx, k.encode(), v.encode())
            else:
                vals = [int(x) for x in v]
                lib().hx_node_attr_ints(self.h, idx, k.encode(), len(vals), _dims(vals))
        return idx

    def metadata(self, key, value):
        """Set one entry of the model's custom metadata map."""
        lib().hx_graph_set_metadata(self.h, key.encode(), value.encode())

    def io(self, inputs, outputs):
        lib().hx_graph_set_io(self.h, len(inputs), _strs(inputs), len(outputs), _strs(outputs))


class Session:
    """A graph loaded through the EP library (CreateEpFactories ... Compile)."""

    def __init__(self, graph: Graph, ep_path: str = EP_LIB, compile: bool = True,
                 force_device: bool = False, name: str = "MI355XExecutionProvider"):
        self.graph = graph  # keeps the graph alive
        self._free = lib().hx_session_free
        self.h = lib().hx_session_new(graph.h, ep_path.encode(), name.encode(), int(compile),
                                      int(force_device))
        if not self.h:
            raise RuntimeError(_err())

    def close(self):
        if getattr(self, "h", None):
            self._free(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def partitions(self):
        L = lib()
        return [[L.hx_session_partition_node(self.h, i, j)
                 for j in range(L.hx_session_partition_size(self.h, i))]
                for i in range(L.hx_session_num_partitions(self.h))]

    def claimed(self, node_index: int) -> bool:
        return bool(lib().hx_session_node_claimed(self.h, node_index))

    def bind_output(self, name, tensor):
        lib().hx_session_bind_output(self.h, name.encode(),
                                     None if tensor is None else ctypes.c_void_p(tensor.data_ptr()))

    def set_input(self, name, tensor, dtype):
        lib().hx_session_set_input(self.h, name.encode(), ctypes.c_void_p(tensor.data_ptr()),
                                   dtype, tensor.dim(), _dims(tensor.shape))

    def run(self, feeds: dict):
        """feeds: name -> (device tensor, ONNX dtype)."""
        for name, (t, dt) in feeds.items():
            self.set_input(name, t, dt)
        if lib().hx_session_run(self.h):
            raise RuntimeError(_err())

    def default_memory_device_is_cpu(self) -> bool:
        """OrtEp::GetDefaultMemoryDevice: True when the EP reports CPU memory."""
        flag = ctypes.c_int(-1)
        if lib().hx_session_default_memory_device(self.h, ctypes.byref(flag)):
            raise RuntimeError(_err())
        return bool(flag.value)

    def memory_device(self):
        """(OrtMemoryInfoDeviceType, vendor id, device id) of the EP's default memory
        device as the session places values: (0, 0, 0) for CPU memory, (1, 0x1002, 0)
        for HBM of GPU 0."""
        t, v, i = ctypes.c_int(), ctypes.c_uint32(), ctypes.c_int()
        lib().hx_session_memory_device(self.h, ctypes.byref(t), ctypes.byref(v), ctypes.byref(i))
        return t.value, v.value, i.value

    def copies(self) -> int:
        """Data-transfer calls the placement rule made in this session's runs."""
        return int(lib().hx_session_copies(self.h))

    def allocator_check(self, memory_info_name: str, device_id: int = 0, nbytes: int = 1 << 20):
        """OrtEpFactory::CreateAllocator for (name, id): None when the EP gives no
        allocator, True when it gave one that allocated, filled and freed HBM."""
        rc = lib().hx_factory_allocator_check(self.h, memory_info_name.encode(), device_id, nbytes)
        if rc < 0:
            raise RuntimeError(_err())
        return True if rc == 1 else None

    def data_transfer_copy(self, src, dst, dtype):
        """OrtEpFactory::CreateDataTransfer + CopyTensors of one tensor (torch tensors,
        host or device, same shape)."""
        if lib().hx_factory_data_transfer_copy(self.h, ctypes.c_void_p(src.data_ptr()),
                                               ctypes.c_void_p(dst.data_ptr()), dtype, src.dim(),
                                               _dims(src.shape)):
            raise RuntimeError(_err())

    def output(self, name):
        """(device pointer, shape) of a value produced by the last run."""
        ptr = ctypes.c_void_p()
        rank = ctypes.c_int()
        dims = (ctypes.c_int64 * 8)()
        if lib().hx_session_get_output(self.h, name.encode(), ctypes.byref(ptr),
                                       ctypes.byref(rank), dims):
            raise RuntimeError(_err())
        return ptr.value, tuple(dims[i] for i in range(rank.value))
