"""A hand-written ONNX (protobuf wire format) encoder for the importer tests — no onnx or protobuf
package is installed here, so the test models are encoded field by field from the ONNX schema:

  ModelProto      1 ir_version, 2 producer_name, 7 graph, 8 opset_import {1 domain, 2 version}
  GraphProto      1 node, 2 name, 5 initializer, 11 input, 12 output, 13 value_info
  NodeProto       1 input, 2 output, 3 name, 4 op_type, 5 attribute
  AttributeProto  1 name, 2 f, 3 i, 4 s, 5 t, 7 floats, 8 ints, 20 type
  TensorProto     1 dims, 2 data_type, 4 float_data, 5 int32_data, 7 int64_data, 8 name, 9 raw_data,
                  10 double_data, 13 external_data {1 key, 2 value}, 14 data_location
  ValueInfoProto  1 name, 2 type {1 tensor_type {1 elem_type, 2 shape {1 dim {1 dim_value, 2 dim_param}}}}

`zoo_to_onnx` turns a graph written by the library as ".vxm" (the VXM2 layout: the zoo model as
built, before any pass) into an ONNX model of the same network, so the ONNX import path can be
compared with the directly built graph on every model the benchmarks use.
"""
import os
import struct

import numpy as np

# ONNX TensorProto.DataType
FLOAT, UINT8, INT8, INT32, INT64, FLOAT16, DOUBLE = 1, 2, 3, 6, 7, 10, 11
_NP = {FLOAT: np.float32, FLOAT16: np.float16, DOUBLE: np.float64, INT64: np.int64, INT32: np.int32, INT8: np.int8,
       UINT8: np.uint8}


# ---------------------------------------------------------------- wire primitives
def varint(v):
    v &= (1 << 64) - 1  # negative int64 values are encoded as their 64-bit two's complement
    out = bytearray()
    while True:
        b = v & 0x7F
        v >>= 7
        if v:
            out.append(b | 0x80)
        else:
            out.append(b)
            return bytes(out)


def key(field, wt):
    return varint((field << 3) | wt)


def f_varint(field, v):
    return key(field, 0) + varint(int(v))


def f_bytes(field, b):
    if isinstance(b, str):
        b = b.encode()
    return key(field, 2) + varint(len(b)) + bytes(b)


def f_fixed32(field, f):
    return key(field, 5) + struct.pack("<f", f)


def f_packed_varints(field, vals):
    return f_bytes(field, b"".join(varint(int(v)) for v in vals))


def f_packed_floats(field, vals):
    return f_bytes(field, struct.pack("<%df" % len(vals), *vals))


# ---------------------------------------------------------------- messages
def tensor(name, arr, dtype=FLOAT, store="raw", packed=True, external=None):
    """A TensorProto. store: "raw" (raw_data), "typed" (float_data / int64_data / int32_data /
    double_data by dtype), or "external" with external=(location, offset, length)."""
    arr = np.asarray(arr)
    b = b""
    dims = list(arr.shape)
    if dims:
        b += f_packed_varints(1, dims) if packed else b"".join(f_varint(1, d) for d in dims)
    b += f_varint(2, dtype) + f_bytes(8, name)
    data = np.ascontiguousarray(arr.astype(_NP[dtype]))
    if store == "raw":
        b += f_bytes(9, data.tobytes())
    elif store == "external":
        loc, off, ln = external
        for k, v in (("location", loc), ("offset", str(off)), ("length", str(ln))):
            b += f_bytes(13, f_bytes(1, k) + f_bytes(2, v))
        b += f_varint(14, 1)
    elif dtype == FLOAT:
        flat = data.ravel().tolist()
        b += f_packed_floats(4, flat) if packed else b"".join(f_fixed32(4, v) for v in flat)
    elif dtype == INT64:
        flat = data.ravel().tolist()
        b += f_packed_varints(7, flat) if packed else b"".join(f_varint(7, v) for v in flat)
    elif dtype == FLOAT16:  # the half's bit pattern in int32_data
        b += f_packed_varints(5, data.view(np.uint16).ravel().tolist())
    elif dtype == INT32:
        b += f_packed_varints(5, data.ravel().tolist())
    elif dtype == DOUBLE:
        b += f_bytes(10, data.tobytes())
    else:
        raise ValueError("typed storage for dtype %d" % dtype)
    return b


def attr(name, v):
    """An AttributeProto from a Python value: int, float, str/bytes, list of ints, list of floats,
    or ("tensor", TensorProto bytes)."""
    b = f_bytes(1, name)
    if isinstance(v, tuple) and v[0] == "tensor":
        return b + f_bytes(5, v[1]) + f_varint(20, 4)
    if isinstance(v, bool) or isinstance(v, (int, np.integer)):
        return b + f_varint(3, int(v)) + f_varint(20, 2)
    if isinstance(v, float):
        return b + f_fixed32(2, v) + f_varint(20, 1)
    if isinstance(v, (str, bytes)):
        return b + f_bytes(4, v) + f_varint(20, 3)
    v = list(v)
    if v and all(isinstance(x, (int, np.integer)) for x in v):
        return b + f_packed_varints(8, v) + f_varint(20, 7)
    return b + f_packed_floats(7, [float(x) for x in v]) + f_varint(20, 6)


def node(op_type, inputs, outputs, name=None, **attrs):
    b = b"".join(f_bytes(1, i) for i in inputs) + b"".join(f_bytes(2, o) for o in outputs)
    if name is not None:
        b += f_bytes(3, name)
    b += f_bytes(4, op_type)
    for k in sorted(attrs):
        b += f_bytes(5, attr(k, attrs[k]))
    return b


def value_info(name, shape=None, elem=FLOAT):
    tt = f_varint(1, elem)
    if shape is not None:
        dims = b""
        for d in shape:
            dims += f_bytes(1, f_bytes(2, d) if isinstance(d, str) else f_varint(1, d))
        tt += f_bytes(2, dims)
    return f_bytes(1, name) + f_bytes(2, f_bytes(1, tt))


def graph(nodes, inputs, outputs, initializers=(), value_infos=(), name="g"):
    b = b"".join(f_bytes(1, n) for n in nodes) + f_bytes(2, name)
    b += b"".join(f_bytes(5, t) for t in initializers)
    b += b"".join(f_bytes(11, v) for v in inputs) + b"".join(f_bytes(12, v) for v in outputs)
    b += b"".join(f_bytes(13, v) for v in value_infos)
    return b


def model(graph_bytes, opset=17):
    return f_varint(1, 8) + f_bytes(2, "vknn-tests") + f_bytes(7, graph_bytes) + f_bytes(8, f_bytes(1, "") + f_varint(2, opset))


# ---------------------------------------------------------------- VXM2 reader
class _Rd:
    def __init__(self, b):
        self.b, self.o = b, 0

    def take(self, n):
        v = self.b[self.o:self.o + n]
        assert len(v) == n, "truncated VXM2"
        self.o += n
        return v

    def u32(self):
        return struct.unpack("<I", self.take(4))[0]

    def i64(self):
        return struct.unpack("<q", self.take(8))[0]

    def f32(self):
        return struct.unpack("<f", self.take(4))[0]

    def str(self):
        return self.take(self.u32()).decode()

    def vec(self, fmt, size):
        n = self.u32()
        return list(struct.unpack("<%d%s" % (n, fmt), self.take(n * size)))


def read_vxm(path):
    """The graph of a VXM2 file as plain Python data (tensors, nodes, inputs, outputs, initializers)."""
    r = _Rd(open(path, "rb").read())
    assert r.u32() == 0x324D5856, "not a VXM2 file"
    tensors = []
    for _ in range(r.u32()):
        name, shape = r.str(), r.vec("q", 8)
        dtype, fmt, flags = r.u32(), r.u32(), r.u32()
        tensors.append(dict(name=name, shape=shape, dtype=dtype, flags=flags))
    nodes = []
    for _ in range(r.u32()):
        nd = dict(type=r.u32(), name=r.str(), inputs=r.vec("i", 4), outputs=r.vec("i", 4), act=r.u32(), lo=r.f32(),
                  hi=r.f32(), sub=r.i64(), res=r.i64(), bias=r.i64(), attrs={})
        for _ in range(r.u32()):
            k, kind, i, f = r.str(), r.u32(), r.i64(), r.f32()
            ints, floats, s = r.vec("q", 8), r.vec("f", 4), r.str()
            nd["attrs"][k] = (kind, i, f, ints, floats, s)
        nodes.append(nd)
    inputs, outputs = r.vec("i", 4), r.vec("i", 4)
    inits = {}
    for _ in range(r.u32()):
        tid = r.i64()
        inits[tid] = r.take(r.u32())
    return dict(tensors=tensors, nodes=nodes, inputs=inputs, outputs=outputs, inits=inits)


# vknn OpType / UnaryType / BinaryType codes (the reference's enumerators) -> ONNX op_type
OPTYPES = ["Unknown", "Conv", "ConvTranspose", "Clip", "Relu", "Add", "GlobalAvgPool", "AvgPool", "MaxPool", "Gemm",
           "MatMul", "Einsum", "Reshape", "Expand", "Tile", "Squeeze", "Flatten", "Softmax", "LayerNorm", "BatchNorm",
           "Concat", "Pad", "Identity", "Constant", "Shape", "Gather", "Unsqueeze", "Unary", "Binary", "PRelu", "Resize"]
_ONNX_OP = {"GlobalAvgPool": "GlobalAveragePool", "AvgPool": "AveragePool", "BatchNorm": "BatchNormalization",
            "Split": "Split"}
UNARY = ["Sigmoid", "Tanh", "HardSwish", "HardSigmoid", "LeakyRelu", "Elu", "Abs", "Neg", "Exp", "Log", "Sqrt", "Floor",
         "Ceil", "Relu", "SiLU", "Erf", "Cos", "Sin", "Reciprocal", "Softplus"]
BINARY = ["Mul", "Sub", "Div", "Max", "Min", "Pow", "Add"]
_SPLIT = 37
_ATTR_INT, _ATTR_FLOAT, _ATTR_INTS, _ATTR_FLOATS, _ATTR_STRING = 1, 2, 3, 4, 5


def zoo_to_onnx(vxm_path, onnx_path, weights="raw", external_file=None, reduce_mean_gap=False):
    """Write the ONNX form of a VXM2 graph (a zoo model before passes).

    weights: "raw" stores every fp32 initializer as raw_data, "typed" as float_data, "external"
    in one data file beside the model (external_file names it). reduce_mean_gap writes global
    average pools as ReduceMean(axes 2,3, keepdims 1)."""
    g = read_vxm(vxm_path)
    T = g["tensors"]
    tname = lambda i: "" if i < 0 else T[i]["name"]
    nodes = []
    for nd in g["nodes"]:
        op = OPTYPES[nd["type"]] if nd["type"] < len(OPTYPES) else ("Split" if nd["type"] == _SPLIT else None)
        assert op is not None and nd["act"] == 0 and nd["res"] < 0 and nd["bias"] < 0, nd
        attrs = {}
        for k, (kind, i, f, ints, floats, s) in nd["attrs"].items():
            attrs[k] = {_ATTR_INT: i, _ATTR_FLOAT: f, _ATTR_INTS: ints, _ATTR_FLOATS: floats, _ATTR_STRING: s}[kind]
        ins, outs = [tname(i) for i in nd["inputs"]], [tname(o) for o in nd["outputs"]]
        if op == "Unary":
            op = UNARY[nd["sub"]]
            if op == "HardSigmoid":
                attrs.update(alpha=nd["lo"], beta=nd["hi"])
            assert op not in ("SiLU", "Relu"), op
        elif op == "Binary":
            op = BINARY[nd["sub"]]
        elif op == "GlobalAvgPool" and reduce_mean_gap:
            op, attrs = "ReduceMean", dict(axes=[2, 3], keepdims=1)
        nodes.append((_ONNX_OP.get(op, op), ins, outs, nd["name"], attrs))
    inits, blob = [], bytearray()
    for tid, raw in sorted(g["inits"].items()):
        t = T[tid]
        if t["dtype"] == 5:  # int64
            arr = np.frombuffer(raw, dtype=np.int64).reshape(t["shape"])
            inits.append(tensor(t["name"], arr, INT64))
            continue
        arr = np.frombuffer(raw, dtype=np.float32).reshape(t["shape"]) if t["shape"] else np.frombuffer(raw, dtype=np.float32)[:1].reshape(())
        if weights == "external":
            off = len(blob)
            blob += arr.tobytes()
            blob += b"\0" * (-len(blob) % 64)
            inits.append(tensor(t["name"], arr, FLOAT, store="external", external=(external_file, off, arr.nbytes)))
        else:
            inits.append(tensor(t["name"], arr, FLOAT, store="raw" if weights == "raw" else "typed"))
    onnx_nodes = [node(op, ins, outs, name=nm, **attrs) for op, ins, outs, nm, attrs in nodes]
    inputs = [value_info(T[i]["name"], T[i]["shape"]) for i in g["inputs"]]
    outputs = [value_info(T[o]["name"], T[o]["shape"] or None) for o in g["outputs"]]
    data = model(graph(onnx_nodes, inputs, outputs, inits))
    with open(onnx_path, "wb") as f:
        f.write(data)
    if weights == "external":
        with open(os.path.join(os.path.dirname(onnx_path), external_file), "wb") as f:
            f.write(bytes(blob))
    return onnx_path


# ---------------------------------------------------------------- hand-built models
def _rng(seed):
    return np.random.default_rng(seed)


def edge_model(path, seed=3):
    """A small network that both the HIP backend and the reference CPU backend run, written in the
    forms real exporters produce and the zoo export does not: a symbolic batch dimension, fp16 and
    double initializers, float_data weights without packing, Clip bounds from a Constant node and
    an initializer, a reused output name, Split sizes as an int64 input, Resize scales from a
    Constant node, ReduceMean as the global pool, HardSigmoid with its default alpha/beta, a
    broadcast Mul, and nodes without names. Input x [N,8,12,12] -> y [N,10]."""
    r = _rng(seed)
    w1 = (r.standard_normal((12, 8, 3, 3)) * 0.2).astype(np.float16)
    b1 = r.standard_normal(12) * 0.1
    w2 = (r.standard_normal((4, 8, 1, 1)) * 0.3).astype(np.float32)
    wf = (r.standard_normal((10, 8)) * 0.3).astype(np.float32)
    bf = (r.standard_normal(10) * 0.1).astype(np.float32)
    inits = [
        tensor("w1", w1, FLOAT16),
        tensor("b1", b1, DOUBLE),
        tensor("cmax", np.array(6.0, np.float32)),
        tensor("w2", w2, FLOAT, store="typed", packed=False),
        tensor("sizes", np.array([4, 8], np.int64), INT64, store="typed", packed=False),
        tensor("wf", wf),
        tensor("bf", bf, FLOAT, store="typed"),
    ]
    nodes = [
        node("Conv", ["x", "w1", "b1"], ["t"], name="conv1", kernel_shape=[3, 3], pads=[1, 1, 1, 1], strides=[1, 1]),
        node("Constant", [], ["cmin"], value=("tensor", tensor("", np.array(0.0, np.float32)))),
        node("Clip", ["t", "cmin", "cmax"], ["t"]),  # reuses the name "t"
        node("Split", ["t", "sizes"], ["a", "b"], name="split", axis=1),
        node("HardSigmoid", ["a"], ["a2"]),
        node("Conv", ["b", "w2"], ["b2"], name="conv2", kernel_shape=[1, 1]),
        node("Relu", ["b2"], ["b3"]),
        node("Concat", ["a2", "b3"], ["c"], name="cat", axis=1),
        node("Constant", [], ["scales"], name="scales_const", value=("tensor", tensor("", np.array([1, 1, 2, 2], np.float32)))),
        node("Resize", ["c", "", "scales"], ["d"], name="up", mode="nearest", coordinate_transformation_mode="asymmetric",
             nearest_mode="floor"),
        node("MaxPool", ["d"], ["e"], name="pool", kernel_shape=[2, 2], strides=[2, 2]),
        node("Add", ["e", "x"], ["f"], name="res"),
        node("ReduceMean", ["f"], ["g"], name="gap", axes=[2, 3], keepdims=1),
        node("Sigmoid", ["g"], ["s"]),
        node("Mul", ["f", "s"], ["f2"], name="scale"),
        node("GlobalAveragePool", ["f2"], ["g2"], name="gap2"),
        node("Flatten", ["g2"], ["h"], name="flat", axis=1),
        node("Gemm", ["h", "wf", "bf"], ["y"], name="fc", transB=1, alpha=1.0, beta=1.0),
    ]
    g = graph(nodes, [value_info("x", ["N", 8, 12, 12])], [value_info("y", ["N", 10])], inits,
              value_infos=[value_info("c", [1, 8, 12, 12])])
    with open(path, "wb") as f:
        f.write(model(g))
    return path


def import_case(path, case):
    """Small graphs, one import rule each (the graphs need not run):
      ssa            two nodes writing one name, the declared output re-pointed at the last one
      defaults       LeakyRelu / Elu / HardSigmoid without attributes, and with them
      unnamed        nodes without names, an unknown op, an empty optional input
      inputs_inits   an initializer also listed as a graph input; dims written unpacked
      dtypes         FLOAT16 / DOUBLE / INT64 raw, INT64 / FLOAT typed, an empty tensor
      dtypes_extra   FLOAT16 in int32_data, DOUBLE in double_data, INT32 / UINT8 / INT8 raw: forms
                     the reference reads as zeros, so they are checked against their values
      const_attrs    Constant tensors with dims (float and int64), scalar attributes of each kind
      value_info     value_info shape hints on node outputs, symbolic and fixed dims"""
    r = _rng(11)
    x = [value_info("x", [1, 4, 5, 5])]
    if case == "ssa":
        nodes = [node("Relu", ["x"], ["t"], name="r1"), node("Sigmoid", ["t"], ["t"], name="s1"),
                 node("Add", ["t", "x"], ["t"], name="a1"), node("Relu", ["t"], ["y"], name="r2"),
                 node("Sigmoid", ["y"], ["y"], name="s2")]
        g = graph(nodes, x, [value_info("y", [1, 4, 5, 5])])
    elif case == "defaults":
        nodes = [node("LeakyRelu", ["x"], ["a"]), node("Elu", ["a"], ["b"]), node("HardSigmoid", ["b"], ["c"]),
                 node("LeakyRelu", ["c"], ["d"], alpha=0.25), node("Elu", ["d"], ["e"], alpha=0.5),
                 node("HardSigmoid", ["e"], ["y"], alpha=0.125, beta=0.25)]
        g = graph(nodes, x, [value_info("y")])
    elif case == "unnamed":
        nodes = [node("Relu", ["x"], ["a"]), node("FancyOp", ["a", ""], ["b", ""], name=""), node("Tanh", ["b"], ["y"]),
                 node("ReduceSum", ["y"], ["z"]), node("Pow", ["z", "z"], ["w"])]
        g = graph(nodes, x, [value_info("w")])
    elif case == "inputs_inits":
        w = r.standard_normal((6, 4, 1, 1)).astype(np.float32)
        nodes = [node("Conv", ["x", "w"], ["y"], name="c")]
        g = graph(nodes, x + [value_info("w", [6, 4, 1, 1])], [value_info("y")], [tensor("w", w, packed=False)])
    elif case == "dtypes":
        inits = [tensor("hr", r.standard_normal((2, 3)), FLOAT16),
                 tensor("dr", r.standard_normal((3,)), DOUBLE),
                 tensor("lr", np.array([1, -2, 3 << 40], np.int64), INT64),
                 tensor("lt", np.array([4, -5], np.int64), INT64, store="typed"),
                 tensor("ft", r.standard_normal((2, 2)), FLOAT, store="typed"),
                 tensor("e", np.zeros((0, 3), np.float32))]
        nodes = [node("Concat", ["x"] + [t for t in ("hr", "dr", "lr", "lt", "ft", "e")], ["y"], name="cat", axis=0)]
        g = graph(nodes, x, [value_info("y")], inits)
    elif case == "dtypes_extra":
        inits = [tensor(n, a, dt, store=st) for n, a, dt, st in DTYPES_EXTRA]
        nodes = [node("Concat", ["x"] + [t[0] for t in DTYPES_EXTRA], ["y"], name="cat", axis=0)]
        g = graph(nodes, x, [value_info("y")], inits)
    elif case == "const_attrs":
        nodes = [node("Constant", [], ["k1"], name="k1", value=("tensor", tensor("", r.standard_normal((2, 3)).astype(np.float32)))),
                 node("Constant", [], ["k2"], name="k2", value=("tensor", tensor("", np.array([[1, 2], [3, -4]], np.int64), INT64))),
                 node("Constant", [], ["k3"], name="k3", value=("tensor", tensor("", np.array([5], np.int64), INT64, store="typed"))),
                 node("Constant", [], ["k4"], name="k4", value=("tensor", tensor("", np.array(2.5, np.float32), store="typed"))),
                 node("Custom", ["x", "k1", "k2", "k3", "k4"], ["y"], name="c", f=0.75, i=-3, s="text", fs=[0.5, -1.0], iz=[3, -1, 0])]
        g = graph(nodes, x, [value_info("y")])
    elif case == "value_info":
        nodes = [node("Relu", ["x"], ["a"], name="r"), node("Sigmoid", ["a"], ["y"], name="s")]
        g = graph(nodes, [value_info("x", ["batch", 4, 5, 5])], [value_info("y", ["batch", 4, 5, 5])],
                  value_infos=[value_info("a", [1, 4, 5, 5]), value_info("zzz", [9])])
    else:
        raise ValueError(case)
    with open(path, "wb") as f:
        f.write(model(g))
    return path


# (name, values, dtype, storage) of the dtypes_extra initializers
DTYPES_EXTRA = [("h16", np.array([0.5, -1.25, 3.0e-5, 65504.0]), FLOAT16, "typed"),
                ("f64", np.array([1.0 / 3.0, -2.5e10, 7.0]), DOUBLE, "typed"),
                ("i32", np.array([7, -8, 1 << 20], np.int32), INT32, "raw"),
                ("u8", np.array([1, 2, 255], np.uint8), UINT8, "raw"),
                ("i8", np.array([-128, 5], np.int8), INT8, "raw")]

IMPORT_CASES = ["ssa", "defaults", "unnamed", "inputs_inits", "dtypes", "const_attrs", "value_info"]


def mixed_model(path, seed=5):
    """A network whose graph alternates between ops the HIP backend runs (Conv, Add, global pool)
    and ops it does not (LeakyRelu, Tanh, Elu), so a session with a host backend splits it into
    HIP -> CPU -> HIP -> CPU -> HIP -> CPU -> HIP segments. x [2,8,10,10] -> y [2,8,1,1]."""
    r = _rng(seed)
    wa = (r.standard_normal((12, 8, 3, 3)) * 0.2).astype(np.float32)
    ba = (r.standard_normal(12) * 0.1).astype(np.float32)
    wb = (r.standard_normal((12, 12, 1, 1)) * 0.3).astype(np.float32)
    bb = (r.standard_normal(12) * 0.1).astype(np.float32)
    wc = (r.standard_normal((8, 12, 1, 1)) * 0.3).astype(np.float32)
    inits = [tensor("wa", wa), tensor("ba", ba), tensor("wb", wb), tensor("bb", bb), tensor("wc", wc)]
    nodes = [
        node("Conv", ["x", "wa", "ba"], ["a"], name="conv_a", kernel_shape=[3, 3], pads=[1, 1, 1, 1]),
        node("LeakyRelu", ["a"], ["l"], name="leaky", alpha=0.1),
        node("Conv", ["l", "wb", "bb"], ["b"], name="conv_b", kernel_shape=[1, 1]),
        node("Tanh", ["b"], ["t"], name="tanh"),
        node("Add", ["t", "a"], ["s"], name="add"),
        node("Elu", ["s"], ["e"], name="elu", alpha=0.7),
        node("Conv", ["e", "wc"], ["c"], name="conv_c", kernel_shape=[1, 1]),
        node("GlobalAveragePool", ["c"], ["y"], name="gap"),
    ]
    g = graph(nodes, [value_info("x", [2, 8, 10, 10])], [value_info("y", [2, 8, 1, 1])], inits)
    with open(path, "wb") as f:
        f.write(model(g))
    return path


def host_only_model(path):
    """Ops the test host backend runs alone: x [2,3,4,5] -> LeakyRelu -> Tanh -> Add x -> Elu -> GAP."""
    nodes = [node("LeakyRelu", ["x"], ["l"], name="leaky", alpha=0.2), node("Tanh", ["l"], ["t"], name="tanh"),
             node("Add", ["t", "x"], ["s"], name="add"), node("Elu", ["s"], ["e"], name="elu"),
             node("GlobalAveragePool", ["e"], ["y"], name="gap")]
    g = graph(nodes, [value_info("x", [2, 3, 4, 5])], [value_info("y", [2, 3, 1, 1])])
    with open(path, "wb") as f:
        f.write(model(g))
    return path
