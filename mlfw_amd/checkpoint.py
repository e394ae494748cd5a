"""mlfw checkpoint container and the packed-weight record of the int8 path.

The container is the reference's `mlfw-ckpt-v1` format
(src/lightning/io/checkpoint_format.ts:82-179): an 8-byte little-endian
header length, a JSON header {format, tree, buffers}, then the raw bytes of
every tensor / typed array back to back.  Tree nodes are JSON values, with
{"$buf": i} for buffer i and {"$map": [[key, node], ...]} for a JS Map.
Files written here are byte-identical to what serializeCheckpoint writes for
the same tree (JSON numbers are formatted the way JS prints them), so the
reference's deserializeCheckpoint / loadCheckpoint read them, and this module
reads the reference's files.

Python stand-ins for the JS values:
  Tensor(dtype, shape, data)  -- an mlfw Tensor (dtype names of
                                 src/util/dtype_map.ts: 'f32', 'i8', ...)
  numpy.ndarray (1-D)         -- a typed array (Int8Array, Float64Array, ...)
  JSMap([(key, value), ...])  -- a JS Map
  dict / list / str / int / float / bool / None -- plain JSON values

A packed linear weight is one record (packed_linear_record) under
modelState[name]:
  {"kind": "q8_packed_linear", "layout": "NK", "shape": [N, K],
   "weight": Tensor('i8', [N, K]) or, for 4-bit weights,
             Tensor('ui8', [N, ceil(K / 2)]) with element 2j in the low
             nibble and 2j + 1 in the high nibble (two's complement),
   "params": QuantizationParams.serialize() fields
             (src/compiler/ir/graph/quantization_types.ts:231-246):
             scheme, scale, zeroPoint, axis, groupSize, dtype, numBits --
             scale a Float64Array and zeroPoint an Int32Array (both accepted
             by QuantizationParams' config), so
             QuantizationParams.deserialize(record.params) rebuilds the
             reference object and the f64 scales round-trip exactly}
"""
from __future__ import annotations

import json
import math
import struct

import numpy as np

MAGIC = "mlfw-ckpt-v1"
HEADER_PREFIX_BYTES = 8

# typed-array constructors of checkpoint_format.ts:57-61 -> numpy dtypes
TYPED_ARRAYS = {
    "Int8Array": np.int8, "Uint8Array": np.uint8, "Uint8ClampedArray": np.uint8,
    "Int16Array": np.int16, "Uint16Array": np.uint16, "Int32Array": np.int32,
    "Uint32Array": np.uint32, "Float32Array": np.float32, "Float64Array": np.float64,
    "BigInt64Array": np.int64, "BigUint64Array": np.uint64,
}
_ARRAY_NAME = {np.dtype(np.int8): "Int8Array", np.dtype(np.uint8): "Uint8Array",
               np.dtype(np.int16): "Int16Array", np.dtype(np.uint16): "Uint16Array",
               np.dtype(np.int32): "Int32Array", np.dtype(np.uint32): "Uint32Array",
               np.dtype(np.float32): "Float32Array", np.dtype(np.float64): "Float64Array",
               np.dtype(np.int64): "BigInt64Array", np.dtype(np.uint64): "BigUint64Array"}
# mlfw tensor dtypes -> storage (DTYPE_TABLE, src/util/dtype_map.ts:53-65)
TENSOR_DTYPES = {"f16": np.uint16, "bf16": np.uint16, "f32": np.float32, "f64": np.float64,
                 "i8": np.int8, "i16": np.int16, "i32": np.int32, "i64": np.int64,
                 "ui8": np.uint8, "bool": np.uint8, "index": np.int32}


class Tensor:
    """An mlfw Tensor in a checkpoint: dtype name, shape and flat data."""

    __slots__ = ("dtype", "shape", "data")

    def __init__(self, dtype: str, shape, data):
        if dtype not in TENSOR_DTYPES:
            raise ValueError(f"unknown mlfw dtype {dtype!r}")
        self.dtype = dtype
        self.shape = [int(d) for d in shape]
        self.data = np.ascontiguousarray(data, dtype=TENSOR_DTYPES[dtype]).reshape(-1)
        if self.data.size != math.prod(self.shape):
            raise ValueError(f"tensor data has {self.data.size} elements, shape {self.shape}")

    def numpy(self) -> np.ndarray:
        return self.data.reshape(self.shape)

    def __repr__(self):
        return f"Tensor({self.dtype!r}, {self.shape})"


class JSMap(list):
    """A JS Map: an ordered list of (key, value) pairs."""

    def get(self, key, default=None):
        for k, v in self:
            if k == key:
                return v
        return default

    def keys(self):
        return [k for k, _ in self]


# ---------------------------------------------------------------- JSON as JS prints it
def _js_number(x) -> str:
    """Number::toString (ECMA-262 6.1.6.1.20) of a double, as JSON.stringify
    writes it: with s the shortest round-trip digit string (k digits) and
    value = s * 10^(n-k), positional when -6 < n <= 21, else exponential
    (d.ddde+N / e-N); null for NaN and +-inf."""
    if isinstance(x, bool):
        return "true" if x else "false"
    if isinstance(x, int) and abs(x) < 2 ** 53:
        return str(x)
    x = float(x)
    if x != x or x in (float("inf"), float("-inf")):
        return "null"
    if x == 0:
        return "0"
    sign = "-" if x < 0 else ""
    r = repr(abs(x))                       # shortest round-trip digits
    mant, _, exp = r.partition("e")
    ip, _, fp = mant.partition(".")
    digits = (ip + fp).lstrip("0")
    trail = len(digits) - len(digits.rstrip("0"))
    digits = digits.rstrip("0")
    k = len(digits)
    n = k + (int(exp) if exp else 0) - len(fp) + trail
    if k <= n <= 21:
        return sign + digits + "0" * (n - k)
    if 0 < n <= 21:
        return sign + digits[:n] + "." + digits[n:]
    if -6 < n <= 0:
        return sign + "0." + "0" * (-n) + digits
    e = n - 1
    return (sign + digits[0] + ("." + digits[1:] if k > 1 else "") + "e" +
            ("+" if e >= 0 else "-") + str(abs(e)))


def _is_array_index(k: str) -> bool:
    """A canonical array index (ECMA-262 6.1.7): the decimal form of an
    integer 0 <= n < 2^32 - 1 with no leading zeros."""
    return (k.isascii() and k.isdigit() and (k == "0" or k[0] != "0")
            and int(k) < 2 ** 32 - 1)


def _js_items(d: dict):
    """A plain object's own keys in the order JS enumerates them
    (OrdinaryOwnPropertyKeys, ECMA-262 10.1.11.1; Object.keys and
    JSON.stringify follow it): array-index keys ascending, then the other
    string keys in insertion order."""
    items = [(str(k), v) for k, v in d.items()]
    index = sorted((int(k), k, v) for k, v in items if _is_array_index(k))
    return [(k, v) for _, k, v in index] + [(k, v) for k, v in items if not _is_array_index(k)]


def _js_json(v) -> str:
    if v is None:
        return "null"
    if isinstance(v, (bool, int, float, np.integer, np.floating)):
        return _js_number(v.item() if hasattr(v, "item") else v)
    if isinstance(v, str):
        return json.dumps(v, ensure_ascii=False)
    if isinstance(v, list):
        return "[" + ",".join(_js_json(e) for e in v) + "]"
    if isinstance(v, dict):
        return "{" + ",".join(json.dumps(k, ensure_ascii=False) + ":" + _js_json(e)
                              for k, e in _js_items(v)) + "}"
    raise TypeError(f"not JSON-encodable: {type(v)}")


# ---------------------------------------------------------------- encode / decode
def _encode(value, buffers):
    if isinstance(value, Tensor):
        buffers.append(({"kind": "tensor", "dtype": value.dtype, "shape": list(value.shape)},
                        value.data.tobytes()))
        return {"$buf": len(buffers) - 1}
    if isinstance(value, np.ndarray):
        arr = np.ascontiguousarray(value).reshape(-1)
        name = _ARRAY_NAME.get(arr.dtype)
        if name is None:
            raise TypeError(f"no typed array for dtype {arr.dtype}")
        buffers.append(({"kind": "array", "arrayType": name}, arr.tobytes()))
        return {"$buf": len(buffers) - 1}
    if isinstance(value, JSMap):
        return {"$map": [[k, _encode(v, buffers)] for k, v in value]}
    if isinstance(value, (list, tuple)):
        return [_encode(v, buffers) for v in value]
    if isinstance(value, dict):
        return {k: _encode(v, buffers) for k, v in _js_items(value)}
    return value


def serialize_checkpoint(tree) -> bytes:
    """serializeCheckpoint (checkpoint_format.ts:82-107)."""
    buffers = []
    enc = _encode(tree, buffers)
    metas, offset = [], 0
    for meta, data in buffers:
        meta = dict(meta)
        meta["offset"] = offset
        meta["length"] = len(data)
        offset += len(data)
        metas.append(meta)
    header = _js_json({"format": MAGIC, "tree": enc, "buffers": metas}).encode("utf-8")
    return b"".join([struct.pack("<Q", len(header)), header] + [d for _, d in buffers])


def _decode_buffer(meta, raw, start):
    chunk = raw[start + meta["offset"]:start + meta["offset"] + meta["length"]]
    if meta["kind"] == "tensor":
        dt = np.dtype(TENSOR_DTYPES[meta["dtype"]])
        return Tensor(meta["dtype"], meta["shape"], np.frombuffer(chunk, dtype=dt).copy())
    dt = TYPED_ARRAYS.get(meta["arrayType"])
    if dt is None:
        raise ValueError("mlfw: unknown typed array in checkpoint: " + str(meta["arrayType"]))
    return np.frombuffer(chunk, dtype=dt).copy()


def _decode(node, decoded):
    if node is None or not isinstance(node, (dict, list)):
        return node
    if isinstance(node, list):
        return [_decode(n, decoded) for n in node]
    if "$buf" in node and isinstance(node["$buf"], int):
        return decoded[node["$buf"]]
    if "$map" in node and isinstance(node["$map"], list):
        return JSMap((k, _decode(v, decoded)) for k, v in node["$map"])
    return {k: _decode(v, decoded) for k, v in node.items()}


def deserialize_checkpoint(raw: bytes):
    """deserializeCheckpoint (checkpoint_format.ts:109-127)."""
    raw = bytes(raw)
    (hlen,) = struct.unpack_from("<Q", raw, 0)
    start = HEADER_PREFIX_BYTES + hlen
    header = json.loads(raw[HEADER_PREFIX_BYTES:start].decode("utf-8"))
    if header.get("format") != MAGIC:
        raise ValueError("mlfw: unrecognized checkpoint format: " + str(header.get("format")))
    decoded = [_decode_buffer(m, raw, start) for m in header["buffers"]]
    return _decode(header["tree"], decoded)


# ---------------------------------------------------------------- packed weights
def pack_int4(q: np.ndarray) -> np.ndarray:
    """[N, K] int8 codes in [-8, 7] -> [N, ceil(K/2)] bytes, element 2j in
    the low nibble, 2j + 1 in the high nibble."""
    q = np.asarray(q, dtype=np.int8)
    N, K = q.shape
    if q.min(initial=0) < -8 or q.max(initial=0) > 7:
        raise ValueError("int4 codes must lie in [-8, 7]")
    qp = np.zeros((N, K + (K & 1)), np.uint8)
    qp[:, :K] = (q.astype(np.int16) & 0xF).astype(np.uint8)
    return np.ascontiguousarray(qp[:, 0::2] | (qp[:, 1::2] << 4))


def unpack_int4(p: np.ndarray, K: int) -> np.ndarray:
    p = np.asarray(p, dtype=np.uint8)
    lo = (p & 0xF).astype(np.int8)
    hi = (p >> 4).astype(np.int8)
    q = np.empty((p.shape[0], 2 * p.shape[1]), np.int8)
    q[:, 0::2] = np.where(lo > 7, lo - 16, lo)
    q[:, 1::2] = np.where(hi > 7, hi - 16, hi)
    return np.ascontiguousarray(q[:, :K])


SCHEMES = ("per_tensor_symmetric", "per_tensor_asymmetric", "per_channel", "per_group")


def packed_linear_record(weight_codes: np.ndarray, scales, scheme: str, num_bits: int = 8,
                         group_size: int | None = None) -> dict:
    """The checkpoint record of one packed [N, K] weight (see the module
    docstring).  weight_codes: int8 [N, K] codes (4-bit ones are packed
    here); scales: f64 per channel [N], per group [N*K/group_size] or a
    scalar for per_tensor_symmetric."""
    codes = np.asarray(weight_codes, dtype=np.int8)
    if codes.ndim != 2:
        raise ValueError("weight codes must be [N, K]")
    if scheme not in SCHEMES:
        raise ValueError(f"unknown scheme {scheme!r}")
    if num_bits not in (4, 8):
        raise ValueError("num_bits must be 4 or 8")
    N, K = codes.shape
    weight = (Tensor("ui8", [N, (K + 1) // 2], pack_int4(codes)) if num_bits == 4
              else Tensor("i8", [N, K], codes))
    if scheme == "per_tensor_symmetric":
        scale, zp = float(np.asarray(scales).reshape(-1)[0]), 0
    else:
        scale = np.ascontiguousarray(scales, dtype=np.float64).reshape(-1)
        zp = np.zeros(scale.size, np.int32)
        want = N if scheme == "per_channel" else (N * K) // (group_size or 1)
        if scheme == "per_group" and (not group_size or (N * K) % group_size):
            raise ValueError("per_group needs a group_size dividing N*K")
        if scale.size != want:
            raise ValueError(f"{scheme} needs {want} scales, got {scale.size}")
    params = {"scheme": scheme, "scale": scale, "zeroPoint": zp,
              "axis": 0 if scheme == "per_channel" else None,
              "groupSize": group_size if scheme == "per_group" else None,
              "dtype": "i8", "numBits": num_bits}
    return {"kind": "q8_packed_linear", "layout": "NK", "shape": [N, K], "weight": weight,
            "params": params}


def record_codes(rec: dict) -> np.ndarray:
    """int8 [N, K] codes of a packed record (4-bit ones unpacked)."""
    N, K = rec["shape"]
    w = rec["weight"].numpy()
    return unpack_int4(w, K) if rec["params"]["numBits"] == 4 else np.ascontiguousarray(w)


def save_packed(path: str, records: dict) -> None:
    """Write {name: record} as a checkpoint whose modelState is a Map, the
    layout ModelCheckpoint / loadCheckpoint use for module state."""
    with open(path, "wb") as f:
        f.write(serialize_checkpoint({"modelState": JSMap(records.items())}))


def load_packed(path: str) -> dict:
    with open(path, "rb") as f:
        tree = deserialize_checkpoint(f.read())
    state = tree["modelState"]
    return {k: v for k, v in state if isinstance(v, dict) and v.get("kind") == "q8_packed_linear"}
