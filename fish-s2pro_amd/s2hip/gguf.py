"""Read-only GGUF v3 access for host tools: metadata and raw tensor bytes.

The file is memory-mapped; tensors come back as zero-copy byte views.  Same
layout rules as GgufFile::open / tensor / tensor_bytes
(crates/fish_s2_core/src/gguf.rs:35-120,233-258): little-endian header
(magic, version, tensor count, metadata count), metadata key / typed value
pairs, tensor infos {name, dims ne0-first, ggml type, offset}, and the data
section at the next multiple of `general.alignment` (default 32).
"""

import mmap
import struct

import numpy as np

GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q8_0 = 0, 1, 2, 8
_BLOCK = {GGML_F32: (1, 4), GGML_F16: (1, 2), GGML_Q4_0: (32, 18), GGML_Q8_0: (32, 34)}
# metadata value types: fixed-size scalars (struct code), 8 = string, 9 = array
_SCALAR = {0: "B", 1: "b", 2: "H", 3: "h", 4: "I", 5: "i", 6: "f", 7: "?", 10: "Q", 11: "q", 12: "d"}


def row_bytes(ggml_type: int, n: int) -> int:
    """Bytes of one row of n elements (GgmlType::byte_len, gguf.rs:233-258)."""
    if ggml_type not in _BLOCK:
        raise ValueError(f"unsupported ggml type {ggml_type}")
    per, size = _BLOCK[ggml_type]
    if n % per:
        raise ValueError(f"row of {n} elements is not a whole number of {per}-element blocks")
    return n // per * size


class GgufTensor:
    def __init__(self, name, dims, ggml_type, data):
        self.name = name
        self.dims = dims          # ne0 first (ne0 = row length)
        self.ggml_type = ggml_type
        self.data = data          # np.uint8 view of the tensor's bytes

    @property
    def row_len(self) -> int:
        return int(self.dims[0])

    @property
    def rows(self) -> int:
        return int(np.prod(self.dims[1:], dtype=np.int64)) if len(self.dims) > 1 else 1

    def f32(self) -> np.ndarray:
        """F32 / F16 tensors as float32 (norm gains and other small vectors)."""
        if self.ggml_type == GGML_F32:
            return np.frombuffer(self.data, np.float32).copy()
        if self.ggml_type == GGML_F16:
            return np.frombuffer(self.data, np.float16).astype(np.float32)
        raise ValueError(f"{self.name}: type {self.ggml_type} is not F32/F16")


class GgufFile:
    def __init__(self, path: str):
        self.path = path
        with open(path, "rb") as f:
            self._map = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
        buf = self._map
        self._pos = 0
        if bytes(buf[:4]) != b"GGUF":
            raise ValueError(f"{path}: not a GGUF file")
        self._pos = 4
        version, n_tensors, n_kv = self._unpack("<IQQ")
        if version != 3:
            raise ValueError(f"{path}: GGUF version {version} (3 expected)")
        self.metadata = {}
        for _ in range(n_kv):
            key = self._string()
            (vtype,) = self._unpack("<I")
            self.metadata[key] = self._value(vtype)
        infos = []
        for _ in range(n_tensors):
            name = self._string()
            (nd,) = self._unpack("<I")
            dims = list(self._unpack(f"<{nd}Q"))
            gtype, offset = self._unpack("<IQ")
            infos.append((name, dims, gtype, offset))
        align = int(self.metadata.get("general.alignment", 32))
        data_start = (self._pos + align - 1) // align * align
        self.tensors = {}
        for name, dims, gtype, offset in infos:
            nbytes = row_bytes(gtype, int(dims[0])) * (int(np.prod(dims[1:], dtype=np.int64)) if len(dims) > 1 else 1)
            start = data_start + offset
            if start + nbytes > len(buf):
                raise ValueError(f"{path}: tensor {name} extends past the end of the file")
            view = np.frombuffer(buf, np.uint8, count=nbytes, offset=start)
            self.tensors[name] = GgufTensor(name, dims, gtype, view)

    def _unpack(self, fmt):
        vals = struct.unpack_from(fmt, self._map, self._pos)
        self._pos += struct.calcsize(fmt)
        return vals

    def _string(self) -> str:
        (n,) = self._unpack("<Q")
        s = bytes(self._map[self._pos:self._pos + n]).decode("utf-8", errors="replace")
        self._pos += n
        return s

    def _value(self, vtype):
        if vtype in _SCALAR:
            return self._unpack("<" + _SCALAR[vtype])[0]
        if vtype == 8:
            return self._string()
        if vtype == 9:
            etype, n = self._unpack("<IQ")
            return [self._value(etype) for _ in range(n)]
        raise ValueError(f"{self.path}: unknown metadata value type {vtype}")

    def tensor(self, name: str) -> GgufTensor:
        if name not in self.tensors:
            raise KeyError(f"tensor {name} not found in {self.path}")
        return self.tensors[name]

    def close(self):
        """Drops this file's tensor views; the mapping closes once no view
        handed out earlier is alive."""
        self.tensors = {}
        try:
            self._map.close()
        except BufferError:
            pass
