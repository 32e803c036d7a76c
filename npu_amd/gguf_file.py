"""GGUF files: a reader that maps tensors straight out of the file, a writer, and the
``TensorStore`` surface the MoE drop-in reads.

The reference opens its model with gguf-py's ``GGUFReader`` (``qwen/model.py:80-157``,
``qwen/inspect_gguf.py:94-122``; gguf-py 0.18.0 pinned at ``uv.lock:132-134``, not
available here) and wraps it in ``TensorStore`` (``qwen/model.py:164-277``).  This module
parses the container itself (GGUF v2/v3, little-endian):

    header      magic "GGUF", uint32 version, uint64 n_tensors, uint64 n_kv
    n_kv x      key (uint64 length + UTF-8), uint32 value type, value
    n_tensors x name, uint32 n_dims, uint64 dims[n_dims] (ggml order: dims[0] fastest),
                uint32 ggml type, uint64 offset (from the start of the data section)
    padding     to ``general.alignment`` (default 32); then the tensor data

Tensor data is a read-only ``numpy.memmap`` view shaped as gguf-py shapes it: F32 / F16 /
F64 / integer tensors as their element type with the dims reversed, every other type as
uint8 rows of ``dims[0] / block * type_size`` bytes (``(n_expert, out, bytes_per_row)``
for a stacked expert tensor), so the raw superblocks go to HBM without repacking.
Nothing from a file is executed: values are decoded field by field.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field
from pathlib import Path
from typing import Any, Iterable

import numpy as np

from npu_amd.gguf_types import GGMLQuantizationType as QT

GGUF_MAGIC = b"GGUF"
DEFAULT_ALIGNMENT = 32

# ggml type id -> (elements per block, bytes per block): the type traits of the ggml
# library that GGUF files are written with.
GGML_TYPE_SIZES: dict[int, tuple[int, int]] = {
    0: (1, 4),        # F32
    1: (1, 2),        # F16
    2: (32, 18),      # Q4_0
    3: (32, 20),      # Q4_1
    6: (32, 22),      # Q5_0
    7: (32, 24),      # Q5_1
    8: (32, 34),      # Q8_0
    9: (32, 36),      # Q8_1
    10: (256, 84),    # Q2_K
    11: (256, 110),   # Q3_K
    12: (256, 144),   # Q4_K
    13: (256, 176),   # Q5_K
    14: (256, 210),   # Q6_K
    15: (256, 292),   # Q8_K
    16: (256, 66),    # IQ2_XXS
    17: (256, 74),    # IQ2_XS
    18: (256, 98),    # IQ3_XXS
    19: (256, 50),    # IQ1_S
    20: (32, 18),     # IQ4_NL
    21: (256, 110),   # IQ3_S
    22: (256, 82),    # IQ2_S
    23: (256, 136),   # IQ4_XS
    24: (1, 1),       # I8
    25: (1, 2),       # I16
    26: (1, 4),       # I32
    27: (1, 8),       # I64
    28: (1, 8),       # F64
    29: (256, 56),    # IQ1_M
    30: (1, 2),       # BF16
    34: (256, 54),    # TQ1_0
    35: (256, 66),    # TQ2_0
}
_ELEMENT_DTYPES = {0: np.float32, 1: np.float16, 24: np.int8, 25: np.int16, 26: np.int32, 27: np.int64,
                   28: np.float64}

# GGUF metadata value types.
UINT8, INT8, UINT16, INT16, UINT32, INT32, FLOAT32, BOOL, STRING, ARRAY, UINT64, INT64, FLOAT64 = range(13)
_SCALAR = {UINT8: "<B", INT8: "<b", UINT16: "<H", INT16: "<h", UINT32: "<I", INT32: "<i", FLOAT32: "<f",
           BOOL: "<?", UINT64: "<Q", INT64: "<q", FLOAT64: "<d"}
_SCALAR_NP = {UINT8: np.uint8, INT8: np.int8, UINT16: np.uint16, INT16: np.int16, UINT32: np.uint32,
              INT32: np.int32, FLOAT32: np.float32, BOOL: np.bool_, UINT64: np.uint64, INT64: np.int64,
              FLOAT64: np.float64}


class GGUFError(ValueError):
    """A malformed or unsupported GGUF file."""


def tensor_nbytes(ggml_type: int, dims: Iterable[int]) -> int:
    """Bytes of a tensor of `dims` (ggml order) in `ggml_type`."""
    dims = [int(d) for d in dims]
    try:
        blk, tsz = GGML_TYPE_SIZES[int(ggml_type)]
    except KeyError:
        raise GGUFError(f"unknown ggml type {ggml_type}") from None
    if dims and dims[0] % blk:
        raise GGUFError(f"dims[0]={dims[0]} is not a multiple of the block size {blk} of type {ggml_type}")
    n = int(np.prod(dims, dtype=np.int64)) if dims else 1
    return n // blk * tsz


@dataclass
class ReaderField:
    """One metadata entry: ``contents()`` is the decoded value (str, int, float, bool, or a
    list / numpy array for arrays), as gguf-py's ``ReaderField.contents()`` returns it."""

    name: str
    types: list[int]
    value: Any

    def contents(self) -> Any:
        return self.value


@dataclass
class ReaderTensor:
    """One tensor: ggml-order ``shape``, ``tensor_type``, and ``data`` mapped from the file."""

    name: str
    tensor_type: QT | int
    shape: tuple[int, ...]
    n_elements: int
    n_bytes: int
    data_offset: int
    data: np.ndarray = field(repr=False)


class _Cursor:
    def __init__(self, buf: np.ndarray):
        self.buf, self.pos = buf, 0

    def take(self, n: int) -> bytes:
        if self.pos + n > len(self.buf):
            raise GGUFError("unexpected end of file")
        b = self.buf[self.pos:self.pos + n].tobytes()
        self.pos += n
        return b

    def scalar(self, t: int):
        fmt = _SCALAR[t]
        return struct.unpack(fmt, self.take(struct.calcsize(fmt)))[0]

    def string(self) -> str:
        n = self.scalar(UINT64)
        return self.take(n).decode("utf-8", errors="replace")

    def value(self, t: int) -> tuple[Any, list[int]]:
        if t == STRING:
            return self.string(), [t]
        if t in _SCALAR:
            return self.scalar(t), [t]
        if t == ARRAY:
            et = self.scalar(UINT32)
            n = self.scalar(UINT64)
            if et in _SCALAR_NP:
                size = np.dtype(_SCALAR_NP[et]).itemsize
                arr = np.frombuffer(self.take(n * size), dtype=np.dtype(_SCALAR_NP[et]).newbyteorder("<"))
                return arr.astype(_SCALAR_NP[et]), [t, et]
            if n > len(self.buf) - self.pos:                  # every element takes at least a byte
                raise GGUFError("metadata array longer than the file")
            items, sub = [], [et]
            for _ in range(n):
                v, sub = self.value(et)
                items.append(v)
            return items, [t] + sub
        raise GGUFError(f"unknown metadata value type {t}")


class GGUFReader:
    """Parses a GGUF file; tensors stay in the file (memory-mapped, read-only)."""

    def __init__(self, path: str | Path):
        self.path = Path(path)
        self._mm = np.memmap(self.path, dtype=np.uint8, mode="r")
        c = _Cursor(self._mm)
        if c.take(4) != GGUF_MAGIC:
            raise GGUFError(f"{self.path}: not a GGUF file")
        self.version = c.scalar(UINT32)
        if self.version not in (2, 3):
            raise GGUFError(f"{self.path}: GGUF version {self.version} not supported (2 or 3; "
                            "big-endian files read as a huge version)")
        n_tensors, n_kv = c.scalar(UINT64), c.scalar(UINT64)
        self.fields: dict[str, ReaderField] = {}
        for _ in range(n_kv):
            key = c.string()
            vt = c.scalar(UINT32)
            v, types = c.value(vt)
            self.fields[key] = ReaderField(key, types, v)
        infos = []
        for _ in range(n_tensors):
            name = c.string()
            nd = c.scalar(UINT32)
            dims = tuple(int(c.scalar(UINT64)) for _ in range(nd))
            tt = c.scalar(UINT32)
            off = c.scalar(UINT64)
            infos.append((name, dims, tt, off))
        al = self.fields.get("general.alignment")
        self.alignment = int(al.value) if al is not None else DEFAULT_ALIGNMENT
        if self.alignment <= 0 or self.alignment & (self.alignment - 1):
            raise GGUFError(f"general.alignment {self.alignment} is not a power of two")
        self.data_offset = (c.pos + self.alignment - 1) // self.alignment * self.alignment
        self.tensors: list[ReaderTensor] = []
        for name, dims, tt, off in infos:
            nbytes = tensor_nbytes(tt, dims)
            start = self.data_offset + off
            if off % self.alignment or start + nbytes > len(self._mm):
                raise GGUFError(f"{name}: data [{start}, {start + nbytes}) misaligned or past the end")
            raw = self._mm[start:start + nbytes]
            np_dims = tuple(reversed(dims))
            if tt in _ELEMENT_DTYPES:
                data = raw.view(_ELEMENT_DTYPES[tt]).reshape(np_dims)
            else:
                blk, tsz = GGML_TYPE_SIZES[tt]
                data = raw.reshape(np_dims[:-1] + (np_dims[-1] // blk * tsz,))
            try:
                ttype: QT | int = QT(tt)
            except ValueError:
                ttype = tt
            self.tensors.append(ReaderTensor(name, ttype, dims, int(np.prod(dims, dtype=np.int64)) if dims else 1,
                                             nbytes, start, data))

    def get_field(self, key: str) -> ReaderField | None:
        return self.fields.get(key)

    def get_tensor(self, i: int) -> ReaderTensor:
        return self.tensors[i]


# ------------------------------------------------------------------ writer
@dataclass
class Typed:
    """A metadata value with an explicit GGUF value type (for ``write_gguf``)."""

    value: Any
    vtype: int


def _pack_string(s: str) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _pack_value(v: Any, vtype: int | None = None) -> tuple[int, bytes]:
    if vtype is None:
        if isinstance(v, bool):
            vtype = BOOL
        elif isinstance(v, int):
            vtype = INT64 if v < 0 else (UINT32 if v < 2 ** 32 else UINT64)
        elif isinstance(v, float):
            vtype = FLOAT32
        elif isinstance(v, str):
            vtype = STRING
        elif isinstance(v, (list, tuple, np.ndarray)):
            vtype = ARRAY
        else:
            raise TypeError(f"cannot store {type(v).__name__} in GGUF metadata")
    if vtype == STRING:
        return vtype, _pack_string(v)
    if vtype == ARRAY:
        if isinstance(v, np.ndarray):
            inv = {np.dtype(d): t for t, d in _SCALAR_NP.items()}
            et = inv[v.dtype]
            return vtype, struct.pack("<IQ", et, v.size) + np.ascontiguousarray(v).astype(v.dtype.newbyteorder("<")).tobytes()
        items = list(v)
        et = _pack_value(items[0])[0] if items else UINT32
        body = b"".join(_pack_value(x, et)[1] for x in items)
        return vtype, struct.pack("<IQ", et, len(items)) + body
    return vtype, struct.pack(_SCALAR[vtype], v)


def write_gguf(path: str | Path, kv: dict[str, Any], tensors: Iterable[tuple[str, int, tuple[int, ...], np.ndarray]],
               alignment: int = DEFAULT_ALIGNMENT) -> None:
    """Write a GGUF v3 file.  ``kv`` values: str, int, float, bool, lists or numpy arrays
    (or ``Typed(value, gguf_type)`` to force a type).  ``tensors``: ``(name, ggml_type, dims
    in ggml order, data)`` with ``data`` holding exactly ``tensor_nbytes(type, dims)`` bytes."""
    tensors = list(tensors)
    kv = dict(kv)
    if alignment != DEFAULT_ALIGNMENT:
        kv["general.alignment"] = Typed(alignment, UINT32)
    head = [GGUF_MAGIC, struct.pack("<IQQ", 3, len(tensors), len(kv))]
    for k, v in kv.items():
        vt, body = _pack_value(v.value, v.vtype) if isinstance(v, Typed) else _pack_value(v)
        head += [_pack_string(k), struct.pack("<I", vt), body]
    blobs, off = [], 0
    for name, tt, dims, data in tensors:
        raw = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
        n = tensor_nbytes(tt, dims)
        if raw.size != n:
            raise GGUFError(f"{name}: {raw.size} bytes given, {n} expected for type {tt} dims {dims}")
        head += [_pack_string(name), struct.pack("<I", len(dims)), struct.pack(f"<{len(dims)}Q", *dims),
                 struct.pack("<IQ", int(tt), off)]
        blobs.append((off, raw))
        off = (off + n + alignment - 1) // alignment * alignment
    header = b"".join(head)
    pad = (-len(header)) % alignment
    with open(path, "wb") as f:
        f.write(header + b"\0" * pad)
        pos = 0
        for o, raw in blobs:
            f.write(b"\0" * (o - pos))
            f.write(raw.tobytes())
            pos = o + raw.size
        f.write(b"\0" * ((-pos) % alignment))


# ------------------------------------------------------------ tensor store
def _get(r: GGUFReader, key: str):
    f = r.fields.get(key)
    return None if f is None else f.contents()


def build_config(r: GGUFReader):
    """The MoE fields of ``qwen/model.py:build_config`` (95-157) from a file's metadata."""
    from npu_amd.qwen_moe import Config
    arch = _get(r, "general.architecture")
    if arch is None:
        raise GGUFError("missing general.architecture")
    p = f"{arch}."

    def need(key, cast):
        v = _get(r, p + key)
        if v is None:
            raise GGUFError(f"missing {p + key}")
        return cast(v)

    return Config(d_model=need("embedding_length", int), n_expert=need("expert_count", int),
                  n_expert_used=need("expert_used_count", int), d_expert_ff=need("expert_feed_forward_length", int),
                  rms_eps=need("attention.layer_norm_rms_epsilon", float), n_layer=need("block_count", int))


class TensorStore:
    """``qwen/model.py:TensorStore`` (164-277) over a GGUF file read by ``GGUFReader``.

    ``raw(name)`` is the mapped tensor (what the device block uploads: quantised bytes are
    never converted on the host); ``get`` / ``get_expert`` return dequantised fp32 numpy
    arrays in (out, in) order, through the device dequant kernels for IQ3_XXS / IQ4_XS /
    Q8_0 / Q4_K / Q5_K / Q6_K and by element conversion for F32 / F16 / BF16.  Other
    quant types raise ``NotImplementedError``.
    """

    def __init__(self, path: str | Path):
        self.path = Path(path)
        self.reader = GGUFReader(self.path)
        self.cfg = build_config(self.reader)
        self._by_name = {t.name: t for t in self.reader.tensors}
        self._cache: dict[tuple[str, str], np.ndarray] = {}

    def names(self) -> list[str]:
        return list(self._by_name)

    def has(self, name: str) -> bool:
        return name in self._by_name

    def raw(self, name: str) -> ReaderTensor:
        t = self._by_name.get(name)
        if t is None:
            raise KeyError(name)
        return t

    @staticmethod
    def _dequant(tt: int, data: np.ndarray, np_shape: tuple[int, ...]) -> np.ndarray:
        tt = int(tt)
        if tt == QT.F32:
            return np.asarray(data, dtype=np.float32).reshape(np_shape)
        if tt == QT.F16:
            return np.asarray(data).astype(np.float32).reshape(np_shape)
        if tt == QT.BF16:
            u = np.ascontiguousarray(data).view(np.uint16).astype(np.uint32) << 16
            return u.view(np.float32).reshape(np_shape)
        if tt in (QT.IQ3_XXS, QT.IQ4_XS, QT.Q8_0, QT.Q4_K, QT.Q5_K, QT.Q6_K):
            import torch
            from npu_amd import ops
            from npu_amd._dropin import device
            flat = np.ascontiguousarray(data).reshape(-1)
            if not flat.flags.writeable:                   # a read-only map of the file
                flat = flat.copy()
            flat = torch.from_numpy(flat).to(device())
            return ops.dequant(tt, flat).cpu().numpy().reshape(np_shape)
        raise NotImplementedError(f"dequantisation of ggml type {tt} is not implemented")

    @staticmethod
    def _convert(arr: np.ndarray, dtype: str) -> np.ndarray:
        if dtype == "fp16":
            return arr.astype(np.float16)
        if dtype == "bf16":
            from npu_amd.synth import to_bf16
            return to_bf16(arr)
        return arr

    def get(self, name: str, dtype: str = "fp32", keep: bool = True) -> np.ndarray:
        """Dequantised tensor with numpy shape = reversed(ggml shape), as ``qwen/model.py:185-223``."""
        if dtype not in ("fp32", "fp16", "bf16"):
            raise ValueError(dtype)
        key = (name, dtype)
        if key in self._cache:
            return self._cache[key]
        t = self.raw(name)
        arr = self._convert(self._dequant(t.tensor_type, t.data, tuple(reversed(t.shape))), dtype)
        if keep:
            self._cache[key] = arr
        return arr

    def drop(self, name: str, dtype: str = "fp32") -> None:
        self._cache.pop((name, dtype), None)

    def cache_bytes(self) -> int:
        return sum(a.nbytes for a in self._cache.values())

    def get_expert(self, name: str, expert_idx: int, dtype: str = "fp32") -> np.ndarray:
        """One expert of a stacked (in, out, n_expert) tensor as (out, in), as ``qwen/model.py:232-277``."""
        if dtype not in ("fp32", "fp16", "bf16"):
            raise ValueError(dtype)
        t = self.raw(name)
        if len(t.shape) != 3:
            raise ValueError(f"{name} is not a stacked expert tensor (got shape {list(t.shape)})")
        if not 0 <= expert_idx < t.shape[2]:
            raise IndexError(expert_idx)
        arr = self._dequant(t.tensor_type, t.data[expert_idx], (t.shape[1], t.shape[0]))
        return self._convert(arr, dtype)
