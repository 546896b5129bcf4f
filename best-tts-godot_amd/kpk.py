"""KPK1 packed-model files: the reader the product loads a graph with, and a
writer for packing a graph description with its weights.

Layout (little-endian), as tools/pack_model.py:11-19 writes it:

    "KPK1"          magic
    u32 version     (1)
    u32 json_len
    u32 blob_len
    json_len bytes  graph description, utf-8 JSON, zero-padded to 4 bytes
    blob_len bytes  weight data, each tensor 4-byte aligned

The description holds "ops" (op names), "tensors" (tensor names), "nodes"
([op id, input ids, output ids, attributes or null, placement], id -1 for an
absent input), "weights" ({tensor id: {"o": offset, "n": bytes, "d": dtype
code, "s": shape}}), "inputs" ({"input_ids", "style", "speed"}), "output",
"sample_rate" and "samples_per_frame" (tools/pack_model.py:208-219).

Reading follows the reference loaders -- tools/kpk_runtime.py:27-50 (numpy
views of the blob) and runtime/kpk_model.gd:67-139 (the checks: magic,
version 1, a whole blob, a JSON object, every weight inside the blob) -- and
executes nothing from the file: struct, json and numpy.frombuffer only.
"""
import json
import struct

import numpy as np

MAGIC = b"KPK1"
VERSION = 1
HEADER = 16

# dtype codes shared by the packer and both loaders (tools/pack_model.py:38-44,
# tools/kpk_runtime.py:21-24)
CODE_TO_NP = {0: np.float32, 1: np.int8, 2: np.uint8, 3: np.int32, 4: np.int64, 5: np.bool_,
              6: np.float16}
NP_TO_CODE = {np.dtype(v): k for k, v in CODE_TO_NP.items()}


class KpkError(ValueError):
    """A file that is not a well-formed KPK1 model."""


def parse_kpk(data):
    """(description dict, {tensor id: read-only ndarray view of the blob})
    from the bytes of a KPK1 file."""
    data = memoryview(data)
    if len(data) < HEADER or bytes(data[:4]) != MAGIC:
        raise KpkError("not a .kpk file")
    version, json_len, blob_len = struct.unpack_from("<III", data, 4)
    if version != VERSION:
        raise KpkError(f"unsupported version {version}")
    if HEADER + json_len > len(data):
        raise KpkError("truncated graph description")
    if HEADER + json_len + blob_len > len(data):
        raise KpkError("truncated weight blob")
    try:
        desc = json.loads(bytes(data[HEADER:HEADER + json_len]).rstrip(b"\0").decode("utf-8"))
    except (UnicodeDecodeError, json.JSONDecodeError) as exc:
        raise KpkError(f"malformed graph description ({exc})") from None
    if not isinstance(desc, dict):
        raise KpkError("malformed graph description (not a JSON object)")
    for key in ("ops", "tensors", "nodes", "weights", "inputs", "output"):
        if key not in desc:
            raise KpkError(f"graph description lacks '{key}'")
    blob = data[HEADER + json_len:HEADER + json_len + blob_len]
    weights = {}
    for key, w in desc["weights"].items():
        tid = int(key)
        off, nbytes, code, shape = int(w["o"]), int(w["n"]), int(w["d"]), [int(s) for s in w["s"]]
        if code not in CODE_TO_NP:
            raise KpkError(f"weight {tid} has unknown dtype code {code}")
        if off < 0 or nbytes < 0 or off + nbytes > blob_len:
            raise KpkError(f"weight {tid} runs past the blob")
        dt = np.dtype(CODE_TO_NP[code])
        count = int(np.prod(shape, dtype=np.int64))
        if nbytes != count * dt.itemsize:
            raise KpkError(f"weight {tid}: {nbytes} bytes for shape {shape} of {dt}")
        weights[tid] = np.frombuffer(blob, dtype=dt, count=count, offset=off).reshape(shape)
    return desc, weights


def read_kpk(path):
    """parse_kpk of the file at `path`."""
    with open(path, "rb") as f:
        return parse_kpk(f.read())


def pack_kpk(desc, weights):
    """The bytes of a KPK1 file: `desc` without its "weights" entry (it is
    rebuilt from `weights`, {tensor id: ndarray}, in ascending id order, each
    tensor 4-byte aligned in the blob)."""
    blob = bytearray()
    table = {}
    for tid in sorted(int(t) for t in weights):
        arr = np.asarray(weights[tid])  # (np.ascontiguousarray would make a 0-d tensor 1-d)
        if not arr.flags.c_contiguous:
            arr = arr.copy(order="C")
        if arr.dtype not in NP_TO_CODE:
            raise KpkError(f"weight {tid}: dtype {arr.dtype} has no KPK code")
        blob += b"\0" * (-len(blob) % 4)
        table[str(tid)] = {"o": len(blob), "n": arr.nbytes, "d": NP_TO_CODE[arr.dtype],
                           "s": list(arr.shape)}
        blob += arr.tobytes()
    out = {k: v for k, v in desc.items() if k != "weights"}
    out["version"] = VERSION
    out["weights"] = table
    payload = json.dumps(out, separators=(",", ":")).encode("utf-8")
    payload += b"\0" * (-len(payload) % 4)
    return MAGIC + struct.pack("<III", VERSION, len(payload), len(blob)) + payload + bytes(blob)


def write_kpk(path, desc, weights):
    with open(path, "wb") as f:
        f.write(pack_kpk(desc, weights))


__all__ = ["KpkError", "parse_kpk", "read_kpk", "pack_kpk", "write_kpk", "CODE_TO_NP",
           "NP_TO_CODE"]
