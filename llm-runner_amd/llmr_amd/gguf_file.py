"""GGUF checkpoints: a writer and a reader that uploads tensors to the device.

* `write_gguf` lays a file out as the reference's tool does
  (tools/gguf_writer.py:176-240): header (magic, version 3, tensor and
  key/value counts), the key/values, the tensor infos with ne = the reversed
  row-major shape and offsets padded to 32 bytes, zero padding to a 32-byte
  data section, then each tensor's bytes padded to 32. It also writes Q4_K
  (the reference's tool stops at Q8_0) and every GGUF metadata type.
* `GGUFFile` reads through the library's native parser (llmr_gguf_*,
  gguf_parse, lib/gguf/parser.c3:164-208) and uploads tensor bytes unchanged
  (llmr_gguf_upload_tensor, upload_weight, lib/model/tensor.c3:48-66): the
  quantized blocks land in the layout the GEMM kernels read.
"""
from __future__ import annotations

import ctypes
import dataclasses
import os
import struct

import numpy as np

from . import capi, gguf

GGUF_MAGIC = 0x46554747   # lib/gguf/types.c3:6
GGUF_VERSION = 3
GGUF_ALIGNMENT = 32       # lib/gguf/types.c3:8 (the reference hard-codes it)

# Metadata value types (GGUFType, lib/gguf/types.c3:11-25).
(T_UINT8, T_INT8, T_UINT16, T_INT16, T_UINT32, T_INT32, T_FLOAT32, T_BOOL, T_STRING, T_ARRAY,
 T_UINT64, T_INT64, T_FLOAT64) = range(13)
_FMT = {T_UINT8: "<B", T_INT8: "<b", T_UINT16: "<H", T_INT16: "<h", T_UINT32: "<I", T_INT32: "<i",
        T_FLOAT32: "<f", T_BOOL: "<?", T_UINT64: "<Q", T_INT64: "<q", T_FLOAT64: "<d"}
_NP = {T_UINT8: "<u1", T_INT8: "<i1", T_UINT16: "<u2", T_INT16: "<i2", T_UINT32: "<u4", T_INT32: "<i4",
       T_FLOAT32: "<f4", T_BOOL: "<u1", T_UINT64: "<u8", T_INT64: "<i8", T_FLOAT64: "<f8"}

# Every GGML type whose size the parser knows (GGMLType.block_size/type_size,
# lib/gguf/types.c3:50-98): (elements per block, bytes per block).
GGML_SIZES = {0: (1, 4), 1: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34),
              9: (32, 36), 10: (256, 84), 11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210),
              24: (1, 1), 25: (1, 2), 26: (1, 4), 27: (1, 8), 28: (1, 8), 30: (1, 2)}


def tensor_bytes(ggml_type: int, n_elements: int) -> int:
    bs, ts = GGML_SIZES[ggml_type]
    return (n_elements + bs - 1) // bs * ts


def _pad(n: int) -> int:
    return (-n) % GGUF_ALIGNMENT


def _string(s: str) -> bytes:
    raw = s.encode("utf-8")
    return struct.pack("<Q", len(raw)) + raw


def _infer(v) -> int:
    if isinstance(v, bool):
        return T_BOOL
    if isinstance(v, int):
        return T_UINT32 if 0 <= v < 2 ** 32 else (T_INT64 if v < 0 else T_UINT64)
    if isinstance(v, float):
        return T_FLOAT32
    if isinstance(v, str):
        return T_STRING
    if isinstance(v, (list, tuple)):
        return T_ARRAY
    raise TypeError(f"no GGUF type for {type(v).__name__}")


def _value(t: int, v) -> bytes:
    if t == T_STRING:
        return _string(v)
    if t == T_ARRAY:
        # v = (element type, items) from Typed, or a list of one inferred type
        at, items = v if isinstance(v, tuple) else (_infer(v[0]) if v else T_UINT32, v)
        return struct.pack("<IQ", at, len(items)) + b"".join(_value(at, x) for x in items)
    return struct.pack(_FMT[t], v)


def encode_kv(key: str, value, vtype: int | None = None) -> bytes:
    """One metadata key/value; the type is inferred unless given (arrays:
    value = (element_type, items) or a list)."""
    t = _infer(value) if vtype is None else vtype
    return _string(key) + struct.pack("<I", t) + _value(t, value)


def encode_tensor(x: np.ndarray, ggml_type: int) -> bytes:
    """Row-major float data as GGUF tensor bytes of `ggml_type`."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    if ggml_type == gguf.GGML_F32:
        return x.astype("<f4").tobytes()
    if ggml_type == gguf.GGML_F16:
        return x.astype("<f2").tobytes()
    if ggml_type == gguf.GGML_BF16:
        u = x.view(np.uint32).astype(np.uint64)
        r = ((u + 0x7fff + ((u >> 16) & 1)) >> 16).astype(np.uint16)  # round to nearest even
        nan = (u & 0x7fffffff) > 0x7f800000  # NaN stays a (quiet) NaN, as the rounding would carry it to Inf or 0
        r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
        return r.astype("<u2").tobytes()
    if ggml_type in (gguf.GGML_Q8_0, gguf.GGML_Q4_K):
        return gguf.quantize(x.reshape(-1, x.shape[-1]), ggml_type).tobytes()
    raise ValueError(f"no encoder for GGML type {ggml_type}")


@dataclasses.dataclass
class Typed:
    """A metadata value with an explicit GGUF type (for an array: vtype
    T_ARRAY and value = (element_type, items))."""
    vtype: int
    value: object


@dataclasses.dataclass
class TensorEntry:
    """A tensor to write: `shape` is row-major ([out, in] for a weight); `data`
    its GGUF bytes (see encode_tensor)."""
    name: str
    ggml_type: int
    shape: tuple
    data: bytes


def write_gguf(path: str, tensors: list[TensorEntry], metadata: dict | None = None) -> int:
    """Writes a GGUF v3 file; returns its size in bytes. Metadata values are
    encoded by type inference (bool, int -> UINT32 / INT64 / UINT64, float ->
    FLOAT32, str, list) or given as Typed(vtype, value)."""
    metadata = metadata or {}
    kvs = [encode_kv(k, v.value, v.vtype) if isinstance(v, Typed) else encode_kv(k, v) for k, v in metadata.items()]
    header = struct.pack("<IIQQ", GGUF_MAGIC, GGUF_VERSION, len(tensors), len(kvs)) + b"".join(kvs)
    infos = bytearray()
    offset = 0
    for t in tensors:
        n = int(np.prod(t.shape)) if len(t.shape) else 1
        size = tensor_bytes(t.ggml_type, n)
        if len(t.data) != size:
            raise ValueError(f"{t.name}: {len(t.data)} bytes, expected {size} for {t.shape} of type {t.ggml_type}")
        dims = list(reversed(t.shape)) or [1]  # ne: fastest-varying first
        infos += _string(t.name) + struct.pack("<I", len(dims))
        for d in dims:
            infos += struct.pack("<Q", d)
        infos += struct.pack("<IQ", t.ggml_type, offset)
        offset += size + _pad(size)
    body = len(header) + len(infos)
    tmp = path + ".partial"
    with open(tmp, "wb") as f:
        f.write(header)
        f.write(infos)
        f.write(b"\0" * _pad(body))
        for t in tensors:
            f.write(t.data)
            f.write(b"\0" * _pad(len(t.data)))
    os.replace(tmp, path)
    return body + _pad(body) + offset


@dataclasses.dataclass
class GGUFTensor:
    """GGUFTensorInfo: shape is row-major (ne reversed), ne as stored."""
    index: int
    name: str
    ggml_type: int
    shape: tuple
    ne: tuple
    offset: int
    data_size: int


class GGUFFile:
    """A GGUF file opened by the library's native parser."""

    def __init__(self, path: str):
        self._lib = capi.lib()
        self._h = ctypes.c_void_p()
        capi.check(self._lib.llmr_gguf_open(os.fsencode(path), ctypes.byref(self._h)))
        ver, nt, nk = ctypes.c_uint32(), ctypes.c_uint64(), ctypes.c_uint64()
        capi.check(self._lib.llmr_gguf_info(self._h, ctypes.byref(ver), ctypes.byref(nt), ctypes.byref(nk)))
        self.version = ver.value
        self.tensors: list[GGUFTensor] = []
        for i in range(nt.value):
            ti = capi.GgufTensorInfo()
            capi.check(self._lib.llmr_gguf_tensor(self._h, i, ctypes.byref(ti)))
            ne = tuple(int(x) for x in ti.ne[:ti.n_dims])
            self.tensors.append(GGUFTensor(i, ti.name.decode("utf-8"), ti.type, tuple(reversed(ne)), ne,
                                           ti.offset, ti.data_size))
        self.by_name = {t.name: t for t in self.tensors}
        self.metadata = {}
        for i in range(nk.value):
            kv = capi.GgufKvInfo()
            capi.check(self._lib.llmr_gguf_kv(self._h, i, ctypes.byref(kv)))
            self.metadata[kv.key.decode("utf-8")] = self._decode(kv)

    @staticmethod
    def _decode(kv):
        raw = ctypes.string_at(kv.data, kv.data_len) if kv.data_len else b""
        if kv.type == T_STRING:
            return raw.decode("utf-8")
        if kv.type in _FMT:
            v = struct.unpack(_FMT[kv.type], raw)[0]
            return bool(v) if kv.type == T_BOOL else v
        if kv.type == T_ARRAY:
            if kv.array_type in _NP:
                a = np.frombuffer(raw, dtype=_NP[kv.array_type], count=kv.array_len)
                return [bool(x) for x in a] if kv.array_type == T_BOOL else a.tolist()
            if kv.array_type == T_STRING:
                out, pos = [], 0
                for _ in range(kv.array_len):
                    n = struct.unpack_from("<Q", raw, pos)[0]
                    out.append(raw[pos + 8:pos + 8 + n].decode("utf-8"))
                    pos += 8 + n
                return out
            return raw  # nested arrays: the raw bytes
        raise ValueError(f"unknown GGUF value type {kv.type}")

    def close(self) -> None:
        if self._h:
            self._lib.llmr_gguf_close(self._h)
            self._h = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def host_bytes(self, name: str) -> np.ndarray:
        """A copy of the tensor's bytes as stored in the file."""
        t = self.by_name[name]
        ti = capi.GgufTensorInfo()
        capi.check(self._lib.llmr_gguf_tensor(self._h, t.index, ctypes.byref(ti)))
        return np.frombuffer(ctypes.string_at(ti.data, ti.data_size), dtype=np.uint8).copy()

    def upload(self, name: str, device="cuda", ctx: capi.Context | None = None):
        """The tensor's bytes, unchanged, in a new uint8 device tensor
        (upload_weight)."""
        import torch
        from .ops import default_graph
        t = self.by_name[name]
        out = torch.empty(t.data_size, dtype=torch.uint8, device=device)
        g = default_graph()
        g.bind_stream()
        capi.check(self._lib.llmr_gguf_upload_tensor((ctx or g.ctx)._h, self._h, t.index, out.data_ptr(),
                                                     t.data_size))
        return out

    def upload_f32(self, name: str, device="cuda"):
        """A small F32/F16/BF16 tensor widened to f32 on the device
        (upload_weight_as_f32, the path of norm weights)."""
        import torch
        t = self.by_name[name]
        b = self.host_bytes(name)
        if t.ggml_type == gguf.GGML_F32:
            a = b.view("<f4")
        elif t.ggml_type == gguf.GGML_F16:
            a = b.view("<f2").astype(np.float32)
        elif t.ggml_type == gguf.GGML_BF16:
            a = (b.view("<u2").astype(np.uint32) << 16).view(np.float32)
        else:
            raise ValueError(f"{name}: type {t.ggml_type} is not a float type")
        return torch.from_numpy(a.reshape(t.shape).copy()).to(device)
