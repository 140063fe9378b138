"""GGUF checkpoints for the verify path: a memory-mapped reader and a small writer.

Public surface as the reference's reader exposes it to its loaders
(snowllm/checkpoint/gguf/__init__.py:177-346): `GGUF(path)` with `.kv`, `.tensors`, `.arch`,
`get("{arch}.key")`, `need(...)`, `g[name]` (shape outermost first, `.quant.name`, `.nbytes`),
`read(name)`; split checkpoints named NAME-0000i-of-0000n.gguf. This module adds `payload(name)`,
a zero-copy uint8 tensor over the mapping, which is what the repack entry points read from.

File format (GGUF v2/v3, little-endian), as published with ggml:
  "GGUF" | u32 version | u64 n_tensors | u64 n_kv
  n_kv x (string key | u32 value type | value)
  n_tensors x (string name | u32 n_dims | u64 dims[n_dims], innermost first | u32 ggml type |
               u64 offset from the data section)
  zero padding to general.alignment (32 unless the key says otherwise) | data section
A string is a u64 byte count and UTF-8 bytes; an array is a u32 element type, a u64 count and
the elements.
"""
import dataclasses
import mmap
import pathlib
import re
import struct
import warnings

import numpy as np
import torch

from .errors import SnowLLMError

MAGIC = b"GGUF"
VERSIONS = (2, 3)
DEFAULT_ALIGNMENT = 32

# value types of the key/value section
KV_U8, KV_I8, KV_U16, KV_I16, KV_U32, KV_I32, KV_F32, KV_BOOL, KV_STRING, KV_ARRAY, \
    KV_U64, KV_I64, KV_F64 = range(13)
_KV_NUMPY = {KV_U8: "<u1", KV_I8: "<i1", KV_U16: "<u2", KV_I16: "<i2", KV_U32: "<u4",
             KV_I32: "<i4", KV_F32: "<f4", KV_BOOL: "<u1", KV_U64: "<u8", KV_I64: "<i8",
             KV_F64: "<f8"}


@dataclasses.dataclass(frozen=True)
class Quant:
    """A ggml storage type: `block` elements are stored in `size` bytes."""
    name: str
    type_id: int
    block: int
    size: int
    dtype: torch.dtype = None

    def nbytes(self, numel: int) -> int:
        blocks, rest = divmod(numel, self.block)
        if rest:
            raise SnowLLMError(f"{self.name} stores {self.block} elements per block; {numel} "
                               f"elements do not fill whole blocks")
        return blocks * self.size


# The ggml type ids with their block geometry (values fixed by the GGUF format). The verify
# path computes on Q4_K, Q5_K, Q6_K and Q8_0 weights and F32/F16/BF16 norms, embeddings and
# heads; the other entries let a checkpoint that also holds them be opened.
_QUANTS = [
    ("F32", 0, 1, 4, torch.float32), ("F16", 1, 1, 2, torch.float16),
    ("BF16", 30, 1, 2, torch.bfloat16), ("F64", 28, 1, 8, torch.float64),
    ("I8", 24, 1, 1, torch.int8), ("I16", 25, 1, 2, torch.int16),
    ("I32", 26, 1, 4, torch.int32), ("I64", 27, 1, 8, torch.int64),
    ("Q4_0", 2, 32, 18, None), ("Q4_1", 3, 32, 20, None), ("Q5_0", 6, 32, 22, None),
    ("Q5_1", 7, 32, 24, None), ("Q8_0", 8, 32, 34, None), ("Q8_1", 9, 32, 40, None),
    ("Q2_K", 10, 256, 84, None), ("Q3_K", 11, 256, 110, None), ("Q4_K", 12, 256, 144, None),
    ("Q5_K", 13, 256, 176, None), ("Q6_K", 14, 256, 210, None), ("Q8_K", 15, 256, 292, None),
]
QUANTS = {name: Quant(name, tid, blk, size, dt) for name, tid, blk, size, dt in _QUANTS}
_BY_ID = {q.type_id: q for q in QUANTS.values()}
# this library's k-quant format ids (the reference's snowllm/ops/moe.py:189-190)
KQUANT_FORMAT = {"Q4_K": 4, "Q5_K": 5, "Q6_K": 6, "Q8_0": 8}


@dataclasses.dataclass
class TensorInfo:
    name: str
    dims: tuple          # innermost first, as stored
    quant: Quant
    offset: int          # from the start of its file's data section
    part: int = 0        # which file of a split checkpoint holds it

    @property
    def shape(self):     # outermost first, as torch
        return tuple(reversed(self.dims))

    @property
    def numel(self):
        return int(np.prod(self.dims, dtype=np.int64)) if self.dims else 1

    @property
    def nbytes(self):
        return self.quant.nbytes(self.numel)

    def __repr__(self):
        return f"TensorInfo({self.name}, {self.shape}, {self.quant.name})"


class _Header:
    """Sequential little-endian decoding of a GGUF header held in a numpy byte array."""

    def __init__(self, data: np.ndarray, where: str):
        self.data, self.pos, self.where = data, 0, where

    def _bytes(self, n: int) -> np.ndarray:
        end = self.pos + n
        if n < 0 or end > self.data.size:
            raise SnowLLMError(f"{self.where}: truncated GGUF header (a field at byte {self.pos} "
                               f"needs {n} bytes)")
        out = self.data[self.pos:end]
        self.pos = end
        return out

    def num(self, dtype: str):
        return self._bytes(np.dtype(dtype).itemsize).view(dtype)[0].item()

    def text(self) -> str:
        return self._bytes(self.num("<u8")).tobytes().decode("utf-8", "replace")

    def value(self, kind: int):
        if kind == KV_STRING:
            return self.text()
        if kind == KV_ARRAY:
            elem, count = self.num("<u4"), self.num("<u8")
            if elem in (KV_STRING, KV_ARRAY):
                return [self.value(elem) for _ in range(count)]
            if elem not in _KV_NUMPY:
                raise SnowLLMError(f"{self.where}: array element type {elem} is not a GGUF type")
            dt = np.dtype(_KV_NUMPY[elem])
            vals = self._bytes(dt.itemsize * count).view(dt)
            return [bool(v) for v in vals] if elem == KV_BOOL else vals.tolist()
        if kind not in _KV_NUMPY:
            raise SnowLLMError(f"{self.where}: value type {kind} is not a GGUF type")
        v = self.num(_KV_NUMPY[kind])
        return bool(v) if kind == KV_BOOL else v


_PART_NAME = re.compile(r"(?P<stem>.+)-(?P<index>\d{5})-of-(?P<count>\d{5})\.gguf")


def split_parts(path: pathlib.Path) -> list:
    """Every file of the checkpoint `path` belongs to, first part first."""
    m = _PART_NAME.fullmatch(path.name)
    if m is None:
        return [path]
    count = int(m["count"])
    files = [path.parent / f"{m['stem']}-{i:05d}-of-{count:05d}.gguf"
             for i in range(1, count + 1)]
    absent = [f.name for f in files if not f.is_file()]
    if absent:
        raise SnowLLMError(f"split checkpoint {path.name}: {len(absent)} of {count} parts are "
                           f"absent ({', '.join(absent[:3])})")
    return files


class GGUF:
    """A GGUF checkpoint, one file or the parts of a split one, mapped read-only."""

    def __init__(self, path):
        self.path = pathlib.Path(path)
        self.parts = split_parts(self.path)
        self.kv, self.tensors = {}, {}
        self._maps, self._data_at = [], []
        try:
            for index, file in enumerate(self.parts):
                self._open(file, index)
        except Exception:
            self.close()
            raise
        if len(self.parts) > 1:
            said = int(self.kv.get("split.count", len(self.parts)))
            if said != len(self.parts):
                raise SnowLLMError(f"{self.path.name}: split.count {said} disagrees with the "
                                   f"{len(self.parts)} parts its name gives")
            said = self.kv.get("split.tensors.count")
            if said is not None and int(said) != len(self.tensors):
                raise SnowLLMError(f"{self.path.name}: split.tensors.count {said}, the parts "
                                   f"hold {len(self.tensors)}")

    def _open(self, file: pathlib.Path, index: int):
        with open(file, "rb") as f:
            size = f.seek(0, 2)
            if size < 24:
                raise SnowLLMError(f"{file}: {size} bytes is too short for a GGUF header")
            mapping = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
        self._maps.append(mapping)
        data = np.frombuffer(mapping, dtype=np.uint8)
        h = _Header(data, str(file))
        if h._bytes(4).tobytes() != MAGIC:
            raise SnowLLMError(f"{file}: no GGUF magic at the start; not a GGUF file")
        version = h.num("<u4")
        if version not in VERSIONS:
            raise SnowLLMError(f"{file}: GGUF version {version} (versions 2 and 3 are read)")
        n_tensors, n_kv = h.num("<u8"), h.num("<u8")
        kv = {}
        for _ in range(n_kv):
            key = h.text()
            kv[key] = h.value(h.num("<u4"))
        align = int(kv.get("general.alignment", DEFAULT_ALIGNMENT))
        if align < 1 or align & (align - 1):
            raise SnowLLMError(f"{file}: general.alignment must be a power of two, not {align}")
        infos = []
        for _ in range(n_tensors):
            name = h.text()
            dims = tuple(h.num("<u8") for _ in range(h.num("<u4")))
            type_id = h.num("<u4")
            offset = h.num("<u8")
            if type_id not in _BY_ID:
                raise SnowLLMError(f"{file}: {name!r} is stored as ggml type {type_id}, which "
                                   f"this reader does not know")
            if name in self.tensors or any(t.name == name for t in infos):
                raise SnowLLMError(f"{file}: a second tensor named {name!r}")
            if offset % align:
                raise SnowLLMError(f"{file}: {name!r} starts at {offset}, off the {align}-byte "
                                   f"alignment")
            infos.append(TensorInfo(name, dims, _BY_ID[type_id], offset, index))
        data_at = h.pos + (-h.pos % align)
        for t in infos:
            if data_at + t.offset + t.nbytes > data.size:
                raise SnowLLMError(f"{file}: {t.name!r} ends past the end of the file "
                                   f"(truncated?)")
            self.tensors[t.name] = t
        self._data_at.append(data_at)
        if index == 0:
            self.version, self.alignment, self.kv = version, align, kv

    def close(self):
        """Unmap the files. Views handed out by payload() keep their mapping alive."""
        for mapping in self._maps:
            try:
                mapping.close()
            except BufferError:
                pass
        self._maps = []

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # -- metadata ---------------------------------------------------------------------------
    @property
    def arch(self) -> str:
        return self.kv.get("general.architecture", "")

    def get(self, key: str, default=None):
        """A metadata value; "{arch}" in the key stands for general.architecture."""
        return self.kv.get(key.replace("{arch}", self.arch), default)

    def need(self, key: str):
        value = self.get(key)
        if value is None:
            raise SnowLLMError(f"{self.path.name}: required metadata "
                               f"{key.replace('{arch}', self.arch)!r} is missing")
        return value

    # -- tensors ----------------------------------------------------------------------------
    def __contains__(self, name: str) -> bool:
        return name in self.tensors

    def __getitem__(self, name: str) -> TensorInfo:
        t = self.tensors.get(name)
        if t is None:
            raise SnowLLMError(f"{self.path.name}: no tensor {name!r}")
        return t

    def payload(self, name: str) -> torch.Tensor:
        """The stored bytes of a tensor: a uint8 CPU tensor viewing the read-only mapping (no
        copy; never write to it -- copy it first, e.g. with .to("cuda") or .clone())."""
        t = self[name]
        if not self._maps:
            raise SnowLLMError(f"{self.path.name} is closed")
        with warnings.catch_warnings():   # torch warns that the mapping is not writable
            warnings.simplefilter("ignore", UserWarning)
            return torch.frombuffer(self._maps[t.part], dtype=torch.uint8, count=t.nbytes,
                                    offset=self._data_at[t.part] + t.offset)

    def read(self, name: str) -> bytes:
        return self.payload(name).numpy().tobytes()

    def tensor(self, name: str) -> torch.Tensor:
        """An element-typed tensor (F32/F16/BF16/I*) in its torch shape, viewing the mapping."""
        t = self[name]
        if t.quant.dtype is None:
            raise SnowLLMError(f"{name} is block-quantised {t.quant.name}; use payload()")
        return self.payload(name).view(t.quant.dtype).view(t.shape)

    def __repr__(self):
        return (f"GGUF({self.path.name}, v{self.version}, arch={self.arch!r}, "
                f"{len(self.tensors)} tensors, {len(self.parts)} file(s))")


# ---------------------------------------------------------------------------------------------
# writer (checkpoints of synthetic weights for the tests and the benchmark)
# ---------------------------------------------------------------------------------------------
def _encode_text(s: str) -> bytes:
    raw = s.encode("utf-8")
    return struct.pack("<Q", len(raw)) + raw


def _encode_value(v):
    """(GGUF value type, bytes) for a Python bool / int / float / str / list."""
    if isinstance(v, bool):
        return KV_BOOL, bytes([int(v)])
    if isinstance(v, int):
        if v < 0:
            return KV_I64, struct.pack("<q", v)
        return (KV_U32, struct.pack("<I", v)) if v < 1 << 32 else (KV_U64, struct.pack("<Q", v))
    if isinstance(v, float):
        return KV_F32, struct.pack("<f", v)
    if isinstance(v, str):
        return KV_STRING, _encode_text(v)
    if isinstance(v, (list, tuple)):
        items = [_encode_value(x) for x in v]
        kinds = {k for k, _ in items} or {KV_U32}
        if len(kinds) > 1:
            raise SnowLLMError("GGUF arrays hold a single value type")
        return KV_ARRAY, struct.pack("<IQ", kinds.pop(), len(items)) + b"".join(b for _, b in items)
    raise SnowLLMError(f"no GGUF encoding for a {type(v).__name__}")


def _as_bytes(data) -> bytes:
    if isinstance(data, (bytes, bytearray, memoryview)):
        return bytes(data)
    if isinstance(data, torch.Tensor):
        data = data.detach().cpu().contiguous().view(-1).view(torch.uint8).numpy()
    return np.ascontiguousarray(data).reshape(-1).view(np.uint8).tobytes()


def write_gguf(path, kv: dict, tensors, *, alignment: int = DEFAULT_ALIGNMENT,
               version: int = 3) -> pathlib.Path:
    """Write a GGUF file. `tensors`: (name, torch-order shape, quant name, payload) tuples,
    the payload as bytes, a numpy array or a torch tensor of exactly the stored bytes."""
    kv = dict(kv)
    if alignment != DEFAULT_ALIGNMENT:
        kv["general.alignment"] = alignment
    head = bytearray(MAGIC + struct.pack("<IQQ", version, len(tensors), len(kv)))
    for key, value in kv.items():
        kind, enc = _encode_value(value)
        head += _encode_text(key) + struct.pack("<I", kind) + enc
    blobs, at = [], 0
    for name, shape, qname, data in tensors:
        info = TensorInfo(name, tuple(int(d) for d in reversed(tuple(shape))), QUANTS[qname], at)
        blob = _as_bytes(data)
        if len(blob) != info.nbytes:
            raise SnowLLMError(f"{name}: {qname}{tuple(shape)} is {info.nbytes} bytes, the "
                               f"payload {len(blob)}")
        head += _encode_text(name) + struct.pack("<I", len(info.dims))
        head += struct.pack(f"<{len(info.dims)}Q", *info.dims)
        head += struct.pack("<IQ", info.quant.type_id, at)
        blobs.append(blob)
        at += len(blob) + (-len(blob) % alignment)
    head += bytes(-len(head) % alignment)
    path = pathlib.Path(path)
    with open(path, "wb") as f:
        f.write(head)
        for blob in blobs:
            f.write(blob)
            f.write(bytes(-len(blob) % alignment))
    return path
