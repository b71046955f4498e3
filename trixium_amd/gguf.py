"""GGUF (v2/v3) files: a zero-copy reader and a writer.

The reader has model/gguf_reader.py's interface (`GGUFReader(path)` with `.metadata`, `.tensors`
of `GGUFTensor` (numpy-order shape, type id, file offset, bytes) and `tensor_bytes(name)`,
model/gguf_reader.py:60-205). A tensor of a block type listed in BLOCK_BYTES has its exact
payload size; any other (the PrismML fork's type 42, which is one of two block sizes, or a type
this table does not know) takes the gap to the next tensor's offset, as the reference does for
every type, so the fork's files load either way. The writer
makes the same layout (header, key/values, tensor infos, aligned data section) and is what the
tests use to build synthetic Bonsai files; no real model file is needed.

`python -m trixium_amd.gguf FILE...` prints a file's metadata and tensor table.
"""

import struct
import sys

import numpy as np

MAGIC = 0x46554747          # "GGUF"
# Metadata value types of the GGUF specification.
(T_U8, T_I8, T_U16, T_I16, T_U32, T_I32, T_F32, T_BOOL, T_STR, T_ARR, T_U64, T_I64,
 T_F64) = range(13)
_NP = {T_U8: np.uint8, T_I8: np.int8, T_U16: np.uint16, T_I16: np.int16, T_U32: np.uint32,
       T_I32: np.int32, T_F32: np.float32, T_U64: np.uint64, T_I64: np.int64, T_F64: np.float64}

TYPE_NAMES = {0: "F32", 1: "F16", 2: "Q4_0", 3: "Q4_1", 6: "Q5_0", 7: "Q5_1", 8: "Q8_0",
              9: "Q8_1", 10: "Q2_K", 11: "Q3_K", 12: "Q4_K", 13: "Q5_K", 14: "Q6_K", 15: "Q8_K",
              24: "I8", 25: "I16", 26: "I32", 27: "I64", 28: "F64", 30: "BF16", 34: "TQ1_0",
              35: "TQ2_0", 41: "Q1_0", 42: "Q2_0", 142: "PQ2_0", 143: "PTQ1_0"}


# (weights, bytes) per block of the types whose size is known; type 42 is either of two blocks.
BLOCK_BYTES = {0: (1, 4), 1: (1, 2), 30: (1, 2), 8: (32, 34), 41: (128, 18), 142: (128, 34),
               143: (128, 28)}


class GGUFTensor:
    """A tensor's entry: numpy-order shape (the last axis contiguous), type id, absolute file
    offset and payload bytes."""

    def __init__(self, name, shape, type_id, file_offset, nbytes):
        self.name, self.shape, self.type_id = name, tuple(shape), type_id
        self.file_offset, self.nbytes = file_offset, nbytes
        self.type_name = TYPE_NAMES.get(type_id, f"UNK{type_id}")

    @property
    def n_elements(self):
        return int(np.prod(self.shape, dtype=np.int64))

    @property
    def bits_per_weight(self):
        return 8.0 * self.nbytes / self.n_elements

    def __repr__(self):
        return f"<GGUFTensor {self.name} {self.type_name} {self.shape} {self.nbytes}B>"


class GGUFReader:
    def __init__(self, path):
        self.path = path
        self._data = np.memmap(path, dtype=np.uint8, mode="r")
        self.metadata, self.tensors = {}, {}
        self._at = 0
        self._parse()

    def _take(self, n):
        if self._at + n > self._data.size:
            raise ValueError(f"{self.path}: truncated GGUF header at byte {self._at}")
        b = self._data[self._at:self._at + n]
        self._at += n
        return b

    def _num(self, t):
        dt = np.dtype(_NP[t])
        v = np.frombuffer(self._take(dt.itemsize).tobytes(), dt)[0]
        return float(v) if dt.kind == "f" else int(v)

    def _str(self):
        return bytes(self._take(self._num(T_U64))).decode("utf-8")

    def _val(self, t):
        if t == T_STR:
            return self._str()
        if t == T_BOOL:
            return bool(self._take(1)[0])
        if t == T_ARR:
            et, n = self._num(T_U32), self._num(T_U64)
            if et in _NP:
                dt = np.dtype(_NP[et])
                return np.frombuffer(self._take(n * dt.itemsize).tobytes(), dt)
            return [self._val(et) for _ in range(n)]
        if t not in _NP:
            raise ValueError(f"{self.path}: unknown metadata type {t}")
        return self._num(t)

    def _parse(self):
        magic, version = self._num(T_U32), self._num(T_U32)
        if magic != MAGIC:
            raise ValueError(f"{self.path}: not a GGUF file (magic {magic:#x})")
        if version < 2:
            raise ValueError(f"{self.path}: GGUF version {version} is not supported")
        n_tensors, n_kv = self._num(T_U64), self._num(T_U64)
        for _ in range(n_kv):
            key = self._str()
            t = self._num(T_U32)
            if key in self.metadata:
                raise ValueError(f"duplicate GGUF metadata key: {key}")
            self.metadata[key] = self._val(t)
        infos = []
        for _ in range(n_tensors):
            name = self._str()
            dims = [self._num(T_U64) for _ in range(self._num(T_U32))]
            infos.append((name, tuple(reversed(dims)), self._num(T_U32), self._num(T_U64)))
        align = int(self.metadata.get("general.alignment", 32))
        self.data_start = -(-self._at // align) * align
        order = sorted(infos, key=lambda i: i[3])
        for k, (name, shape, tid, off) in enumerate(order):
            end = self.data_start + order[k + 1][3] if k + 1 < len(order) else self._data.size
            if name in self.tensors:
                raise ValueError(f"duplicate GGUF tensor name: {name}")
            gap = end - self.data_start - off
            n = int(np.prod(shape, dtype=np.int64))
            nbytes = gap
            if tid in BLOCK_BYTES and n % BLOCK_BYTES[tid][0] == 0:
                nbytes = n // BLOCK_BYTES[tid][0] * BLOCK_BYTES[tid][1]
                if nbytes > gap:
                    raise ValueError(f"{self.path}: tensor {name} needs {nbytes} bytes, has {gap}")
            self.tensors[name] = GGUFTensor(name, shape, tid, self.data_start + off, nbytes)

    def tensor_bytes(self, name):
        """The payload as a uint8 view of the mapped file."""
        t = self.tensors[name]
        return self._data[t.file_offset:t.file_offset + t.nbytes]


# Writer ---------------------------------------------------------------------------------------

class Typed:
    """A metadata value with its GGUF type pinned (and an array's element type)."""

    def __init__(self, t, value, elem=None):
        self.t, self.value, self.elem = t, value, elem


def _pack_str(s):
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _infer(v):
    if isinstance(v, bool):
        return T_BOOL
    if isinstance(v, (int, np.integer)):
        return T_U32 if 0 <= int(v) < 1 << 32 else T_I64
    if isinstance(v, (float, np.floating)):
        return T_F32
    if isinstance(v, str):
        return T_STR
    if isinstance(v, (list, tuple, np.ndarray)):
        return T_ARR
    raise TypeError(f"no GGUF type for {type(v)}")


def _pack_val(t, v, elem=None):
    if t == T_STR:
        return _pack_str(v)
    if t == T_BOOL:
        return struct.pack("<B", int(bool(v)))
    if t == T_ARR:
        if isinstance(v, np.ndarray):
            et = elem if elem is not None else {np.dtype(d): k for k, d in _NP.items()}[v.dtype]
            return struct.pack("<IQ", et, v.size) + np.ascontiguousarray(v, _NP[et]).tobytes()
        v = list(v)
        et = elem if elem is not None else (_infer(v[0]) if v else T_U32)
        return struct.pack("<IQ", et, len(v)) + b"".join(_pack_val(et, x) for x in v)
    return np.array(v, _NP[t]).tobytes()


def write_gguf(path, metadata, tensors, alignment=32, version=3):
    """metadata: {key: value} with the type inferred (int -> uint32, float -> float32, str,
    bool, list/array -> array) or given by a `Typed`. tensors: [(name, numpy-order shape, type id,
    payload bytes)] in file order."""
    md = dict(metadata)
    if alignment != 32:
        md["general.alignment"] = Typed(T_U32, alignment)
    out = [struct.pack("<IIQQ", MAGIC, version, len(tensors), len(md))]
    for k, v in md.items():
        t, val, elem = (v.t, v.value, v.elem) if isinstance(v, Typed) else (_infer(v), v, None)
        out.append(_pack_str(k) + struct.pack("<I", t) + _pack_val(t, val, elem))
    offs, at = [], 0
    for name, shape, tid, payload in tensors:
        at = -(-at // alignment) * alignment
        offs.append(at)
        at += len(payload)
        dims = list(reversed([int(d) for d in shape]))
        out.append(_pack_str(name) + struct.pack("<I", len(dims)) +
                   struct.pack(f"<{len(dims)}Q", *dims) + struct.pack("<IQ", tid, offs[-1]))
    head = b"".join(out)
    start = -(-len(head) // alignment) * alignment
    with open(path, "wb") as f:
        f.write(head + b"\0" * (start - len(head)))
        for (name, shape, tid, payload), off in zip(tensors, offs):
            f.write(b"\0" * (start + off - f.tell()))
            f.write(bytes(payload) if not isinstance(payload, np.ndarray) else payload.tobytes())


def inspect(path):
    r = GGUFReader(path)
    print(f"== {path}")
    for k, v in r.metadata.items():
        if isinstance(v, (np.ndarray, list)) and len(v) > 4:
            v = f"[{len(v)}] {list(v[:4])}..."
        print(f"  {k:56s} {v}")
    for t in r.tensors.values():
        print(f"  {t.name:44s} {t.type_name:8s} {str(t.shape):20s} {t.nbytes:12d} {t.bits_per_weight:6.3f}")
    return r


if __name__ == "__main__":
    for f in sys.argv[1:]:
        inspect(f)
