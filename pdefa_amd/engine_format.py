"""`.engine` model file format: writer and reader (numpy).

The byte layout is the one the reference loader parses
(PDEFA1.0/src/loader/custom_loader.cpp:62-214) and its converter writes
(pdefa/tools/onnx_to_engine.py:312-333, 747-818):

header   u32 magic 0x4E474E45 ("ENGN"), u32 version (1|2), u32 n_weights,
         u32 n_nodes, u32 n_inputs, u32 n_outputs, char brand[64]
weights  n_weights x { u32 name_len, name, u8 dtype (12 F32, 8 I64, 6 I32), u8 rank,
                       i64 dims[rank], u64 offset, u64 size }
nodes    n_nodes x { u8 op, u32 name_len, name, u16 n_in, u16 n_out,
                     i32 in[n_in], i32 out[n_out], 128-byte OpParams }
graph    i32 graph_inputs[n_inputs], i32 graph_outputs[n_outputs]
v2 only  TensorInfo per input then per output:
         { u32 name_len, name, u8 ndim, i64 dims[ndim], u8 dtype }
data     the weight blobs, at data_start + offset

Node input references: idx >= 0 is an intermediate tensor, idx <= -1000 is
weight (-1000 - idx), -1..-999 is external input (-1 - idx)
(PDEFA1.0/src/core/session_parts/session_helpers.inc:6-25).

OpParams is 128 bytes: <7q (stride_h, stride_w, pad_h, pad_w, dil_h, dil_w,
groups) 2q (kernel_h, kernel_w) i (axis) 4x 4q (scale_h, scale_w, target_h,
target_w) B (upsample_mode) 3x f (eps) B (fused_activation) 3x f (leaky_slope)
then zero padding (PDEFA1.0/include/engine/graph.hpp:78-95).
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field
from typing import Dict, List, Optional

import numpy as np

MAGIC = 0x4E474E45
DT_F32 = 12
DT_I64 = 8
DT_I32 = 6
PARAMS_SIZE = 128
# weight dtypes (PDEFA1.0/include/engine/dtype.hpp:36-53 codes) <-> numpy
_NP_OF_DT = {DT_F32: np.float32, DT_I64: np.int64, DT_I32: np.int32}
_DT_OF_NP = {np.dtype(np.int64): DT_I64, np.dtype(np.int32): DT_I32}

# OpType codes (PDEFA1.0/include/engine/graph.hpp:20-73)
OP = {
    "Conv": 1, "MatMul": 2, "Add": 3, "Mul": 4, "Sub": 5, "Div": 6,
    "Relu": 10, "LeakyRelu": 11, "Sigmoid": 12, "Tanh": 13, "SiLU": 14, "GELU": 15,
    "MaxPool": 20, "AveragePool": 21, "BatchNormalization": 22,
    "Softmax": 30, "Concat": 31, "Upsample": 32, "Resize": 33,
    "Input": 40, "Output": 41, "Reshape": 42, "Transpose": 43, "Slice": 44,
    "TopK": 50, "GatherElements": 51,
}
OP_NAME = {v: k for k, v in OP.items()}

_PARAM_FIELDS = ("stride_h", "stride_w", "pad_h", "pad_w", "dil_h", "dil_w", "groups",
                 "kernel_h", "kernel_w", "axis", "scale_h", "scale_w", "target_h",
                 "target_w", "upsample_mode", "eps", "fused_activation", "leaky_slope")

# Defaults the reference converter packs when an attribute is absent
# (onnx_to_engine.py:312-318).
_PARAM_DEFAULTS = dict(stride_h=1, stride_w=1, pad_h=0, pad_w=0, dil_h=1, dil_w=1, groups=1,
                       kernel_h=0, kernel_w=0, axis=-1, scale_h=0, scale_w=0, target_h=0,
                       target_w=0, upsample_mode=0, eps=1e-5, fused_activation=0,
                       leaky_slope=0.01)


def pack_params(**kw) -> bytes:
    p = dict(_PARAM_DEFAULTS)
    for k, v in kw.items():
        if k not in p:
            raise KeyError(f"unknown OpParams field {k!r}")
        p[k] = v
    buf = struct.pack("<7q", p["stride_h"], p["stride_w"], p["pad_h"], p["pad_w"],
                      p["dil_h"], p["dil_w"], p["groups"])
    buf += struct.pack("<2q", p["kernel_h"], p["kernel_w"])
    buf += struct.pack("<i4x", p["axis"])
    buf += struct.pack("<4q", p["scale_h"], p["scale_w"], p["target_h"], p["target_w"])
    buf += struct.pack("<B3xf", p["upsample_mode"], p["eps"])
    buf += struct.pack("<B3xf", p["fused_activation"], p["leaky_slope"])
    return buf + b"\x00" * (PARAMS_SIZE - len(buf))


def unpack_params(raw: bytes) -> Dict[str, float]:
    v = struct.unpack_from("<7q2qi4x4qB3xfB3xf", raw)
    return dict(zip(_PARAM_FIELDS, v))


@dataclass
class Node:
    op: int
    name: str
    inputs: List[int]
    outputs: List[int]
    params: Dict[str, float] = field(default_factory=dict)

    @property
    def op_name(self) -> str:
        return OP_NAME.get(self.op, f"op{self.op}")


@dataclass
class TensorInfo:
    name: str
    shape: List[int]
    dtype: int = DT_F32


@dataclass
class EngineModel:
    weights: List[np.ndarray]
    weight_names: List[str]
    nodes: List[Node]
    graph_inputs: List[int]
    graph_outputs: List[int]
    input_infos: List[TensorInfo] = field(default_factory=list)
    output_infos: List[TensorInfo] = field(default_factory=list)
    version: int = 2
    brand: bytes = b"pdefa-amd"

    def weight(self, ref: int) -> np.ndarray:
        return self.weights[-1000 - ref]


def write_engine(path: str, m: EngineModel) -> None:
    out = bytearray()
    out += struct.pack("<6I", MAGIC, m.version, len(m.weights), len(m.nodes),
                       len(m.graph_inputs), len(m.graph_outputs))
    brand = m.brand[:63]
    out += brand + b"\x00" * (64 - len(brand))
    cursor = 0
    blobs = []
    for name, arr in zip(m.weight_names, m.weights):
        # int64 / int32 arrays keep their type; everything else is F32, as the
        # reference converter writes every initializer (onnx_to_engine.py:428)
        arr = np.asarray(arr)
        dt = _DT_OF_NP.get(arr.dtype, DT_F32)
        arr = np.ascontiguousarray(arr, dtype=_NP_OF_DT[dt])
        nb = name.encode()
        out += struct.pack("<I", len(nb)) + nb
        out += struct.pack("<BB", dt, arr.ndim)
        for d in arr.shape:
            out += struct.pack("<q", int(d))
        out += struct.pack("<QQ", cursor, arr.nbytes)
        cursor += arr.nbytes
        blobs.append(arr.tobytes())
    for n in m.nodes:
        nb = n.name.encode()
        out += struct.pack("<BI", n.op, len(nb)) + nb
        out += struct.pack("<HH", len(n.inputs), len(n.outputs))
        out += struct.pack(f"<{len(n.inputs)}i", *n.inputs)
        out += struct.pack(f"<{len(n.outputs)}i", *n.outputs)
        out += pack_params(**n.params)
    out += struct.pack(f"<{len(m.graph_inputs)}i", *m.graph_inputs)
    out += struct.pack(f"<{len(m.graph_outputs)}i", *m.graph_outputs)
    if m.version >= 2:
        for info in list(m.input_infos) + list(m.output_infos):
            nb = info.name.encode()
            out += struct.pack("<I", len(nb)) + nb
            out += struct.pack("<B", len(info.shape))
            for d in info.shape:
                out += struct.pack("<q", int(d))
            out += struct.pack("<B", info.dtype)
    with open(path, "wb") as f:
        f.write(bytes(out))
        for b in blobs:
            f.write(b)


class FormatError(ValueError):
    pass


def read_engine(path: str) -> EngineModel:
    with open(path, "rb") as f:
        raw = f.read()
    pos = 0

    def take(fmt):
        nonlocal pos
        sz = struct.calcsize(fmt)
        if pos + sz > len(raw):
            raise FormatError("truncated .engine file")
        v = struct.unpack_from(fmt, raw, pos)
        pos += sz
        return v

    magic, version = take("<2I")
    if magic != MAGIC or version not in (1, 2):
        raise FormatError("bad magic or version")
    nw, nn, ni, no = take("<4I")
    brand = take("64s")[0].rstrip(b"\x00")
    wmeta = []
    for _ in range(nw):
        (ln,) = take("<I")
        name = take(f"{ln}s")[0].decode()
        dt, rank = take("<BB")
        dims = take(f"<{rank}q") if rank else ()
        off, size = take("<QQ")
        wmeta.append((name, dt, dims, off, size))
    nodes = []
    for _ in range(nn):
        op, ln = take("<BI")
        name = take(f"{ln}s")[0].decode()
        nin, nout = take("<HH")
        ins = list(take(f"<{nin}i")) if nin else []
        outs = list(take(f"<{nout}i")) if nout else []
        params = unpack_params(raw[pos:pos + PARAMS_SIZE])
        pos += PARAMS_SIZE
        nodes.append(Node(op, name, ins, outs, params))
    gin = list(take(f"<{ni}i")) if ni else []
    gout = list(take(f"<{no}i")) if no else []
    iinfo, oinfo = [], []
    if version >= 2:
        for lst, cnt in ((iinfo, ni), (oinfo, no)):
            for _ in range(cnt):
                (ln,) = take("<I")
                name = take(f"{ln}s")[0].decode()
                (nd,) = take("<B")
                dims = list(take(f"<{nd}q")) if nd else []
                (dt,) = take("<B")
                lst.append(TensorInfo(name, dims, dt))
    data_start = pos
    weights, names = [], []
    for name, dt, dims, off, size in wmeta:
        if dt not in _NP_OF_DT:
            raise FormatError(f"weight {name}: dtype {dt} unsupported")
        npdt = np.dtype(_NP_OF_DT[dt])
        a = np.frombuffer(raw, dtype=npdt, count=size // npdt.itemsize, offset=data_start + off)
        weights.append(a.reshape(dims).copy())
        names.append(name)
    return EngineModel(weights, names, nodes, gin, gout, iinfo, oinfo, version, brand)
