"""Test-side ONNX protobuf codec, written independently of the C++ reader.

`decode_model(bytes, base_dir)` walks the wire format of a ModelProto into
plain Python data (the checker for the reader in
fast-arm-tbcnn_amd/runtime/onnx.cpp); `encode_*` builds ModelProto bytes for
synthetic models, including encodings the reference's model files never use
(unpacked repeated fields, int32_data for 8-bit tensors, attributes without a
type, external data at an offset).  Field numbers follow onnx/onnx.proto.
Nothing here executes content from a model file: it only reads bytes.
"""
import os
import struct

import numpy as np

# TensorProto.DataType -> numpy dtype
DTYPES = {1: np.float32, 2: np.uint8, 3: np.int8, 4: np.uint16, 5: np.int16, 6: np.int32, 7: np.int64,
          9: np.bool_, 10: np.float16, 12: np.uint32, 13: np.uint64}
ONNX_DTYPE = {np.dtype(v): k for k, v in DTYPES.items()}


# ---- decoding ------------------------------------------------------------------------

def _varint(b, i):
    r = shift = 0
    while True:
        c = b[i]
        i += 1
        r |= (c & 0x7F) << shift
        shift += 7
        if c < 0x80:
            return r, i


def fields(b):
    """Yields (field number, wire type, value) of one message."""
    i = 0
    while i < len(b):
        key, i = _varint(b, i)
        num, wt = key >> 3, key & 7
        if wt == 0:
            v, i = _varint(b, i)
        elif wt == 1:
            v = b[i:i + 8]
            i += 8
        elif wt == 2:
            n, i = _varint(b, i)
            v = b[i:i + n]
            i += n
        elif wt == 5:
            v = b[i:i + 4]
            i += 4
        else:
            raise ValueError("wire type %d" % wt)
        if i > len(b):
            raise ValueError("truncated")
        yield num, wt, v


def _signed(v):
    return v - (1 << 64) if v >= 1 << 63 else v


def _varints(wt, v):
    if wt == 0:
        return [_signed(v)]
    out, i = [], 0
    while i < len(v):
        x, i = _varint(v, i)
        out.append(_signed(x))
    return out


def _floats(wt, v):
    return list(struct.unpack("<%df" % (len(v) // 4), bytes(v)))


def _tensor(b, base_dir):
    t = {"dims": [], "float": [], "int32": [], "int64": [], "uint64": [], "external": {}, "raw": None, "dt": 0,
         "name": "", "location": 0}
    for num, wt, v in fields(b):
        if num == 1:
            t["dims"] += _varints(wt, v)
        elif num == 2:
            t["dt"] = v
        elif num == 4:
            t["float"] += _floats(wt, v) if wt == 2 else [struct.unpack("<f", bytes(v))[0]]
        elif num == 5:
            t["int32"] += _varints(wt, v)
        elif num == 7:
            t["int64"] += _varints(wt, v)
        elif num == 8:
            t["name"] = bytes(v).decode()
        elif num == 9:
            t["raw"] = bytes(v)
        elif num == 11:
            t["uint64"] += [x & ((1 << 64) - 1) for x in _varints(wt, v)]
        elif num == 13:
            kv = {k: bytes(x).decode() for k, _, x in fields(v)}
            t["external"][kv.get(1, "")] = kv.get(2, "")
        elif num == 14:
            t["location"] = v
    dt = np.dtype(DTYPES[t["dt"]])
    shape = tuple(t["dims"])
    if t["external"]:
        ext = t["external"]
        with open(os.path.join(base_dir, ext["location"]), "rb") as f:
            f.seek(int(ext.get("offset", "0")))
            data = f.read(int(ext["length"])) if "length" in ext else f.read()
        arr = np.frombuffer(data, dt)
    elif t["raw"] is not None:
        arr = np.frombuffer(t["raw"], dt)
    elif dt == np.float32:
        arr = np.array(t["float"], np.float32)
    elif dt == np.int64:
        arr = np.array(t["int64"], np.int64)
    elif dt in (np.dtype(np.uint32), np.dtype(np.uint64)):
        arr = np.array(t["uint64"], np.uint64).astype(dt)
    else:
        arr = np.array([x & 0xFFFFFFFF for x in t["int32"]], np.uint32).astype(
            {1: np.uint8, 2: np.uint16, 4: np.uint32}[dt.itemsize]).view(dt)
    return t["name"], arr.reshape(shape).copy()


def _value_info(b):
    name, dims = "", []
    for num, wt, v in fields(b):
        if num == 1:
            name = bytes(v).decode()
        elif num == 2:
            for tn, _, tv in fields(v):
                if tn != 1:
                    continue
                for sn, _, sv in fields(tv):
                    if sn != 2:
                        continue
                    for dn, _, dv in fields(sv):
                        if dn == 1:
                            val = 1
                            for en, _, ev in fields(dv):
                                if en == 1:
                                    val = _signed(ev)
                            dims.append(val)
    return name, dims


def _attribute(b, base_dir):
    a = {"type": 0}
    for num, wt, v in fields(b):
        if num == 1:
            a["name"] = bytes(v).decode()
        elif num == 2:
            a["f"] = struct.unpack("<f", bytes(v))[0]
        elif num == 3:
            a["i"] = _signed(v)
        elif num == 4:
            a["s"] = bytes(v).decode()
        elif num == 5:
            a["t"] = _tensor(v, base_dir)[1]
        elif num == 7:
            a.setdefault("floats", []).extend(_floats(wt, v) if wt == 2 else [struct.unpack("<f", bytes(v))[0]])
        elif num == 8:
            a.setdefault("ints", []).extend(_varints(wt, v))
        elif num == 9:
            a.setdefault("strings", []).append(bytes(v).decode())
        elif num == 20:
            a["type"] = v
    key = {1: "f", 2: "i", 3: "s", 4: "t", 6: "floats", 7: "ints", 8: "strings"}.get(a["type"])
    if key is None:
        key = next((k for k in ("f", "i", "s", "t", "floats", "ints", "strings") if k in a), None)
    return a.get("name", ""), (a.get(key, [] if key in ("floats", "ints", "strings") else None) if key else None)


def decode_model(b, base_dir="."):
    """ModelProto bytes -> dict(producer, ir_version, opsets, inputs, outputs,
    value_info, inits, nodes), shapes as lists, initializers as numpy arrays."""
    m = {"producer": ("", ""), "ir_version": 0, "opsets": {}, "inputs": [], "outputs": [], "value_info": {},
         "inits": {}, "nodes": []}
    prod = ["", ""]
    for num, wt, v in fields(b):
        if num == 1:
            m["ir_version"] = v
        elif num in (2, 3):
            prod[num - 2] = bytes(v).decode()
        elif num == 8:
            d = {n: x for n, _, x in fields(v)}
            m["opsets"][bytes(d.get(1, b"")).decode()] = d.get(2, 0)
        elif num == 7:
            gi, go, gv, gn = [], [], [], []
            for gnum, _, gvv in fields(v):
                if gnum == 5:
                    name, arr = _tensor(gvv, base_dir)
                    m["inits"][name] = arr
                elif gnum == 11:
                    gi.append(_value_info(gvv))
                elif gnum == 12:
                    go.append(_value_info(gvv))
                elif gnum == 13:
                    gv.append(_value_info(gvv))
                elif gnum == 1:
                    gn.append(gvv)
            for name, dims in gi:
                if name not in m["inits"]:
                    m["inputs"].append(name)
                    m["value_info"][name] = dims
            for name, dims in go:
                m["outputs"].append(name)
                m["value_info"][name] = dims
            for name, dims in gv:
                m["value_info"][name] = dims
            for nb in gn:
                node = {"inputs": [], "outputs": [], "name": "", "op_type": "", "attributes": {}}
                for nn, _, nv in fields(nb):
                    if nn == 1:
                        node["inputs"].append(bytes(nv).decode())
                    elif nn == 2:
                        node["outputs"].append(bytes(nv).decode())
                    elif nn == 3:
                        node["name"] = bytes(nv).decode()
                    elif nn == 4:
                        node["op_type"] = bytes(nv).decode()
                    elif nn == 5:
                        k, val = _attribute(nv, base_dir)
                        if val is not None:
                            node["attributes"][k] = val
                if not node["name"]:
                    node["name"] = node["op_type"] + "_" + (node["outputs"][0] if node["outputs"] else "")
                m["nodes"].append(node)
    m["producer"] = tuple(prod)
    return m


def load(path):
    with open(path, "rb") as f:
        return decode_model(f.read(), os.path.dirname(os.path.abspath(path)))


# ---- encoding ------------------------------------------------------------------------

def _enc_varint(v):
    v &= (1 << 64) - 1
    out = bytearray()
    while True:
        c = v & 0x7F
        v >>= 7
        if v:
            out.append(c | 0x80)
        else:
            out.append(c)
            return bytes(out)


def key(num, wt):
    return _enc_varint(num << 3 | wt)


def f_varint(num, v):
    return key(num, 0) + _enc_varint(v)


def f_bytes(num, b):
    if isinstance(b, str):
        b = b.encode()
    return key(num, 2) + _enc_varint(len(b)) + bytes(b)


def f_fixed32(num, x):
    return key(num, 5) + struct.pack("<f", x)


def f_packed_varints(num, vals):
    return f_bytes(num, b"".join(_enc_varint(v) for v in vals))


def encode_tensor(name, arr, mode="raw", external=None):
    """mode: 'raw' (raw_data), 'typed' (float_data / int32_data / int64_data,
    packed), 'unpacked' (typed, one record per value), 'external' (external
    = (location, offset, length or None))."""
    arr = np.require(np.asarray(arr), requirements="C")  # keeps 0-d arrays 0-d
    dt = ONNX_DTYPE[arr.dtype]
    out = b""
    if mode == "unpacked":
        out += b"".join(f_varint(1, d) for d in arr.shape)
    else:
        out += f_packed_varints(1, arr.shape) if arr.ndim else b""
    out += f_varint(2, dt) + f_bytes(8, name)
    flat = arr.reshape(-1)
    if mode == "raw":
        out += f_bytes(9, flat.tobytes())
    elif mode == "external":
        loc, off, length = external
        out += f_bytes(13, f_bytes(1, "location") + f_bytes(2, loc))
        out += f_bytes(13, f_bytes(1, "offset") + f_bytes(2, str(off)))
        if length is not None:
            out += f_bytes(13, f_bytes(1, "length") + f_bytes(2, str(length)))
        out += f_varint(14, 1)
    elif arr.dtype == np.float32:
        out += (b"".join(f_fixed32(4, float(x)) for x in flat) if mode == "unpacked"
                else f_bytes(4, flat.astype("<f4").tobytes()))
    elif arr.dtype == np.int64:
        out += (b"".join(f_varint(7, int(x)) for x in flat) if mode == "unpacked"
                else f_packed_varints(7, [int(x) for x in flat]))
    elif arr.dtype in (np.uint32, np.uint64):
        out += f_packed_varints(11, [int(x) for x in flat])
    else:
        bits = flat.view({1: np.uint8, 2: np.uint16, 4: np.uint32}[arr.itemsize]) if arr.dtype != np.int32 else flat
        vals = [int(x) for x in (flat if arr.dtype.kind == "i" else bits)]
        out += (b"".join(f_varint(5, v) for v in vals) if mode == "unpacked" else f_packed_varints(5, vals))
    return out


def encode_value_info(name, dims, symbolic=()):
    dim_msgs = b"".join(
        f_bytes(1, f_bytes(2, "N") if i in symbolic else f_varint(1, d)) for i, d in enumerate(dims))
    tensor_type = f_varint(1, 1) + f_bytes(2, dim_msgs)
    return f_bytes(1, name) + f_bytes(2, f_bytes(1, tensor_type))


def encode_attribute(name, value, typed=True):
    out = f_bytes(1, name)
    if isinstance(value, bool) or isinstance(value, (int, np.integer)):
        out += f_varint(3, int(value)) + (f_varint(20, 2) if typed else b"")
    elif isinstance(value, float):
        out += f_fixed32(2, value) + (f_varint(20, 1) if typed else b"")
    elif isinstance(value, str):
        out += f_bytes(4, value) + (f_varint(20, 3) if typed else b"")
    elif isinstance(value, np.ndarray):
        out += f_bytes(5, encode_tensor("", value)) + (f_varint(20, 4) if typed else b"")
    elif isinstance(value, (list, tuple)) and value and isinstance(value[0], float):
        out += b"".join(f_fixed32(7, v) for v in value) + (f_varint(20, 6) if typed else b"")
    elif isinstance(value, (list, tuple)) and value and isinstance(value[0], str):
        out += b"".join(f_bytes(9, v) for v in value) + (f_varint(20, 8) if typed else b"")
    else:
        out += f_packed_varints(8, [int(v) for v in value]) + (f_varint(20, 7) if typed else b"")
    return out


def encode_node(op, inputs, outputs, name="", attrs=None, typed=True):
    out = b"".join(f_bytes(1, i) for i in inputs) + b"".join(f_bytes(2, o) for o in outputs)
    if name:
        out += f_bytes(3, name)
    out += f_bytes(4, op)
    for k, v in (attrs or {}).items():
        out += f_bytes(5, encode_attribute(k, v, typed))
    return out


def encode_model(nodes, inits, inputs, outputs, value_info=(), producer=("tests", "1"), opset=18,
                 ir_version=8, extra_graph=b""):
    """nodes: encoded NodeProtos; inits: encoded TensorProtos; inputs/outputs/
    value_info: encoded ValueInfoProtos."""
    g = b"".join(f_bytes(1, n) for n in nodes) + f_bytes(2, "g")
    g += b"".join(f_bytes(5, t) for t in inits)
    g += b"".join(f_bytes(11, v) for v in inputs) + b"".join(f_bytes(12, v) for v in outputs)
    g += b"".join(f_bytes(13, v) for v in value_info) + extra_graph
    m = f_varint(1, ir_version) + f_bytes(2, producer[0]) + f_bytes(3, producer[1])
    m += f_bytes(8, f_bytes(1, "") + f_varint(2, opset))
    return m + f_bytes(7, g)
