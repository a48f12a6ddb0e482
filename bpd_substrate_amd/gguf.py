"""GGUF tensor locator: header / key-value / tensor-info walk, data alignment,
tensor byte ranges, pre-load validation, and hand-off of a tensor's bytes to
the GPU ABI unchanged.

Reference behaviour followed:
  * the header and KV walk of bench/verify_quant_gpu.py:56-102 (magic, version,
    u64 counts, length-prefixed strings, typed values and arrays) and
    lib/gguf_native_reader.pl:82-260 (same, value types 0..12);
  * the data section starts at the end of the tensor infos rounded up to
    `general.alignment` (32 when absent): lib/gguf_native_reader.pl:54-70,
    bench/verify_quant_gpu.py:94;
  * byte ownership (lib/safe_read.pl:1-40): every byte of the file belongs to at
    most one structure, so a "crossword" file whose strings, tensor infos or
    tensor data share bytes is rejected instead of being read two ways;
  * the five pre-load checks of lib/gguf_validate.pl:74-256: tensor_overlap,
    quant_version, type_consistency, rope_params, known_types.

One deliberate difference: tensor sizes use the exact GGUF block sizes
(Q4_K 144 B per 256 elements, Q6_K 210 B, Q8_0 34 B per 32, ...).  The Prolog
validator sizes quantized tensors as one byte per element
(lib/gguf_validate.pl:262-270), which is only an approximation; a locator that
hands bytes to a kernel needs the exact range.

Everything here is host-side parsing of untrusted bytes: no value read from a
file is used as a size or offset before it has been checked against the file.
"""
import mmap
import os
import struct
from dataclasses import dataclass, field

MAGIC = 0x46554747  # "GGUF" read as little-endian u32

# value types (lib/gguf_native_reader.pl:110-185)
T_U8, T_I8, T_U16, T_I16, T_U32, T_I32, T_F32, T_BOOL, T_STR, T_ARR, T_U64, T_I64, T_F64 = range(13)
_SCALAR = {T_U8: "<B", T_I8: "<b", T_U16: "<H", T_I16: "<h", T_U32: "<I", T_I32: "<i", T_F32: "<f",
           T_BOOL: "<?", T_U64: "<Q", T_I64: "<q", T_F64: "<d"}

# tensor types: code -> (name, elements per block, bytes per block)
TYPES = {
    0: ("F32", 1, 4), 1: ("F16", 1, 2), 2: ("Q4_0", 32, 18), 3: ("Q4_1", 32, 20), 6: ("Q5_0", 32, 22),
    7: ("Q5_1", 32, 24), 8: ("Q8_0", 32, 34), 9: ("Q8_1", 32, 36), 10: ("Q2_K", 256, 84), 11: ("Q3_K", 256, 110),
    12: ("Q4_K", 256, 144), 13: ("Q5_K", 256, 176), 14: ("Q6_K", 256, 210), 15: ("Q8_K", 256, 292),
    24: ("I8", 1, 1), 25: ("I16", 1, 2), 26: ("I32", 1, 4), 27: ("I64", 1, 8), 28: ("F64", 1, 8), 30: ("BF16", 1, 2),
}
Q8_0, Q4_K, Q6_K = 8, 12, 14
KQUANT = {12, 13, 14, 15}  # Q4_K, Q5_K, Q6_K, Q8_K: the reference's kquant_type (lib/gguf_validate.pl:148-152)
MAX_DIMS = 4
# architectures whose blocks use rotary embeddings (lib/gguf_validate.pl:204-213)
ROPE_ARCHS = {"llama", "falcon", "mistral", "qwen", "qwen2", "phi", "phi3", "gemma", "gemma2", "starcoder2"}
ROPE_KEYS = ("llama.rope.freq_base", "rope.freq_base", "llama.rope.dimension_count", "rope.dimension_count")


class GGUFError(Exception):
    """A file that cannot be read as GGUF, or whose structures share bytes."""

    def __init__(self, what, offset=None):
        super().__init__(what if offset is None else f"{what} (at byte {offset})")
        self.what, self.offset = what, offset


@dataclass
class Tensor:
    name: str
    dims: tuple          # ne[0] first: ne[0] is the contiguous (row) length
    type: int
    offset: int          # relative to the data section, as stored
    abs_offset: int      # in the file
    nbytes: int

    @property
    def type_name(self):
        return TYPES[self.type][0]

    @property
    def n_elements(self):
        n = 1
        for d in self.dims:
            n *= d
        return n

    @property
    def row_len(self):
        return self.dims[0] if self.dims else 1

    @property
    def n_rows(self):
        return self.n_elements // self.row_len if self.row_len else 0


@dataclass
class GGUF:
    path: str
    file_size: int
    version: int
    metadata: dict
    kv_types: dict
    tensors: list
    alignment: int
    data_start: int
    unclaimed: list = field(default_factory=list)   # byte ranges no structure owns
    issues: list = field(default_factory=list)      # (check, detail) found by a lenient parse

    def __post_init__(self):
        self.by_name = {t.name: t for t in self.tensors}

    def tensor(self, name):
        if name not in self.by_name:
            raise KeyError(f"no tensor named {name!r}")
        return self.by_name[name]

    def tensor_bytes(self, name):
        """The tensor's bytes, exactly as stored (a read-only memory map slice)."""
        t = self.tensor(name)
        with open(self.path, "rb") as f:
            mm = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
        return memoryview(mm)[t.abs_offset:t.abs_offset + t.nbytes]

    def to_device(self, name, device):
        """A uint8 device tensor holding the tensor's bytes unchanged (GGUF row-major, ne[0]
        contiguous), ready for the library's entry points."""
        import numpy as np
        import torch

        host = np.frombuffer(self.tensor_bytes(name), dtype=np.uint8)
        return torch.from_numpy(host.copy()).to(device)


class _Ledger:
    """Claims byte ranges of a file; a byte may be claimed once (lib/safe_read.pl:1-20)."""

    def __init__(self, size):
        self.size = size
        self.ranges = []  # sorted, disjoint [start, end)

    def claim(self, start, end, what):
        if start < 0 or end > self.size or start > end:
            raise GGUFError(f"{what} runs past the end of the file ({end} > {self.size} bytes)", start)
        if start == end:
            return
        import bisect
        i = bisect.bisect_left(self.ranges, (start, end))
        for j in (i - 1, i):
            if 0 <= j < len(self.ranges):
                s, e = self.ranges[j]
                if s < end and start < e:
                    raise GGUFError(f"{what} shares bytes [{max(s, start)}, {min(e, end)}) with another structure",
                                    start)
        self.ranges.insert(i, (start, end))

    def unclaimed(self):
        out, pos = [], 0
        for s, e in self.ranges:
            if s > pos:
                out.append((pos, s))
            pos = max(pos, e)
        if pos < self.size:
            out.append((pos, self.size))
        return out


class _Reader:
    def __init__(self, buf, ledger):
        self.buf, self.pos, self.ledger = buf, 0, ledger

    def take(self, n, what):
        if n < 0 or self.pos + n > len(self.buf):
            raise GGUFError(f"{what}: {n} bytes needed, {len(self.buf) - self.pos} left", self.pos)
        self.ledger.claim(self.pos, self.pos + n, what)
        b = self.buf[self.pos:self.pos + n]
        self.pos += n
        return b

    def scalar(self, fmt, what):
        return struct.unpack(fmt, self.take(struct.calcsize(fmt), what))[0]

    def string(self, what):
        n = self.scalar("<Q", what + " length")
        raw = self.take(n, what)
        try:
            return bytes(raw).decode("utf-8")
        except UnicodeDecodeError:
            raise GGUFError(f"{what} is not UTF-8", self.pos - n)

    def value(self, vtype, what, depth=0):
        if vtype in _SCALAR:
            return self.scalar(_SCALAR[vtype], what)
        if vtype == T_STR:
            return self.string(what)
        if vtype == T_ARR:
            if depth > 0:
                raise GGUFError(f"{what}: nested arrays are not supported", self.pos)
            etype = self.scalar("<I", what + " element type")
            count = self.scalar("<Q", what + " element count")
            if etype not in _SCALAR and etype != T_STR:
                raise GGUFError(f"{what}: unknown array element type {etype}", self.pos)
            # every element needs at least one byte (strings: 8): bound the count by the file
            least = 8 if etype == T_STR else struct.calcsize(_SCALAR[etype])
            if count * least > len(self.buf) - self.pos:
                raise GGUFError(f"{what}: {count} elements cannot fit in the file", self.pos)
            if etype in _SCALAR and etype != T_BOOL:
                size = struct.calcsize(_SCALAR[etype])
                raw = self.take(count * size, what)
                import numpy as np
                return np.frombuffer(bytes(raw), dtype=np.dtype(_SCALAR[etype])).tolist()
            return [self.value(etype, f"{what}[{i}]", depth + 1) for i in range(count)]
        raise GGUFError(f"{what}: unknown value type {vtype}", self.pos)


def tensor_nbytes(dims, ttype, name="tensor"):
    """Exact byte size of a tensor of GGUF type `ttype` (ne[0] a multiple of the block)."""
    if ttype not in TYPES:
        raise GGUFError(f"{name}: unknown tensor type {ttype}")
    tname, blk, bb = TYPES[ttype]
    if dims and dims[0] % blk:
        raise GGUFError(f"{name}: row length {dims[0]} is not a multiple of the {tname} block ({blk})")
    n = 1
    for d in dims:
        n *= d
    return n // blk * bb


def parse(buf, path="<bytes>", strict=True):
    """Parse GGUF bytes (bytes, bytearray, memoryview or mmap).

    strict=True (loading): any tensor that cannot be located exactly is an
    error.  strict=False (reporting): a row length that is not a whole number of
    blocks, or a data offset off the alignment, is recorded in `issues` and the
    walk goes on; such a tensor is sized as one byte per element, as the
    reference's validator sizes every quantized tensor
    (lib/gguf_validate.pl:262-270), so overlaps are still found.
    """
    size = len(buf)
    ledger = _Ledger(size)
    r = _Reader(buf, ledger)
    magic = r.scalar("<I", "magic")
    if magic != MAGIC:
        raise GGUFError(f"bad magic 0x{magic:08x}", 0)
    version = r.scalar("<I", "version")
    if version not in (2, 3):
        raise GGUFError(f"unsupported GGUF version {version}", 4)
    n_tensors = r.scalar("<Q", "tensor count")
    n_kv = r.scalar("<Q", "metadata count")
    # a KV pair takes >= 8+4+1 bytes, a tensor info >= 8+4+4+8: bound both by the file
    if n_kv * 13 + n_tensors * 24 > size - r.pos:
        raise GGUFError(f"{n_kv} KV pairs and {n_tensors} tensor infos cannot fit in {size} bytes", 8)

    metadata, kv_types = {}, {}
    for i in range(n_kv):
        key = r.string(f"key {i}")
        vtype = r.scalar("<I", f"type of {key!r}")
        if key in metadata:
            raise GGUFError(f"duplicate key {key!r}", r.pos)
        metadata[key] = r.value(vtype, f"value of {key!r}")
        kv_types[key] = vtype

    align = metadata.get("general.alignment", 32)
    if not isinstance(align, int) or align <= 0 or align & (align - 1):
        raise GGUFError(f"general.alignment {align!r} is not a power of two")

    infos = []
    for i in range(n_tensors):
        name = r.string(f"name of tensor {i}")
        nd = r.scalar("<I", f"ndims of {name!r}")
        if nd > MAX_DIMS:
            raise GGUFError(f"{name!r} has {nd} dimensions (at most {MAX_DIMS})", r.pos)
        dims = tuple(r.scalar("<Q", f"dim {k} of {name!r}") for k in range(nd))
        ttype = r.scalar("<I", f"type of {name!r}")
        off = r.scalar("<Q", f"offset of {name!r}")
        infos.append((name, dims, ttype, off))

    meta_end = r.pos
    data_start = (meta_end + align - 1) // align * align
    ledger.claim(meta_end, min(data_start, size), "alignment padding")
    tensors, names, issues = [], set(), []
    for name, dims, ttype, off in infos:
        if name in names:
            raise GGUFError(f"duplicate tensor name {name!r}")
        names.add(name)
        try:
            nbytes = tensor_nbytes(dims, ttype, repr(name))
        except GGUFError as e:
            if strict or ttype not in TYPES:
                raise
            issues.append(("block_shape", str(e)))
            nbytes = 1
            for d in dims:
                nbytes *= d
        if off % align:
            what = f"{name!r}: data offset {off} is not a multiple of the alignment {align}"
            if strict:
                raise GGUFError(what)
            issues.append(("alignment", what))
        start = data_start + off
        ledger.claim(start, start + nbytes, f"data of {name!r}")
        tensors.append(Tensor(name, dims, ttype, off, start, nbytes))
    return GGUF(path, size, version, metadata, kv_types, tensors, align, data_start, ledger.unclaimed(), issues)


def _mapped(path, fn):
    size = os.path.getsize(path)
    if size == 0:
        raise GGUFError("empty file")
    with open(path, "rb") as f:
        mm = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
    try:
        return fn(mm)
    finally:
        mm.close()


def open_gguf(path):
    """Parse a GGUF file for loading (memory-mapped; the tensor data is not read)."""
    return _mapped(path, lambda mm: parse(mm, path))


def report(path):
    """Pre-load report of a file, as (check, ok, detail) in the order of
    lib/gguf_validate.pl:74-95 plus this locator's own structural checks.
    A file that cannot be walked at all gives [("parse", False, why)]
    (the reference's error(parse_failure, _))."""
    try:
        g = _mapped(path, lambda mm: parse(mm, path, strict=False))
    except GGUFError as e:
        return [("parse", False, str(e))]
    out = validate(g)
    for check in ("block_shape", "alignment"):
        found = [d for c, d in g.issues if c == check]
        out.append((check, not found, "; ".join(found)))
    return out


def validate(g):
    """The five pre-load checks of lib/gguf_validate.pl:74-256, as (check, ok, detail).

    tensor_overlap is enforced while parsing (a file with overlapping tensor
    data does not parse); it is reported here for the files that do.
    """
    out = [("tensor_overlap", True, "")]
    kq = sorted({t.type_name for t in g.tensors if t.type in KQUANT})
    qv = g.metadata.get("general.quantization_version")
    if kq and qv is None:
        out.append(("quant_version", False, f"K-quant tensors ({', '.join(kq)}) but no general.quantization_version"))
    elif kq and (isinstance(qv, bool) or not isinstance(qv, (int, float))):
        out.append(("quant_version", False, f"general.quantization_version={qv!r} is not a number"))
    elif kq and qv < 3:
        out.append(("quant_version", False, f"general.quantization_version={qv}; K-quant tensors require >= 3"))
    else:
        out.append(("quant_version", True, ""))
    mixed = []
    for t in g.tensors:
        for suffix in (".weight", ".bias"):
            if suffix in t.name:
                layer = t.name[:t.name.index(suffix)]
                types = sorted({u.type_name for u in g.tensors if u.name.startswith(layer)})
                if len(types) > 1 and (layer, types) not in mixed:
                    mixed.append((layer, types))
                break
    out.append(("type_consistency", not mixed, "; ".join(f"{l}: {'/'.join(ts)}" for l, ts in mixed)))
    arch = g.metadata.get("general.architecture")
    if arch in ROPE_ARCHS and not any(k in g.metadata for k in ROPE_KEYS):
        out.append(("rope_params", False, f"architecture {arch} needs rope parameters, none in the metadata"))
    else:
        out.append(("rope_params", True, ""))
    out.append(("known_types", True, ""))  # an unknown type already fails to parse (its size is unknown)
    return out


def _pack_value(vtype, value):
    if vtype in _SCALAR:
        return struct.pack(_SCALAR[vtype], value)
    if vtype == T_STR:
        raw = value.encode("utf-8")
        return struct.pack("<Q", len(raw)) + raw
    if vtype == T_ARR:
        etype, items = value
        return struct.pack("<IQ", etype, len(items)) + b"".join(_pack_value(etype, v) for v in items)
    raise ValueError(f"unknown value type {vtype}")


def write_gguf(path, metadata, tensors, alignment=32, version=3):
    """Write a GGUF file.  metadata: [(key, vtype, value)] (arrays as
    (T_ARR, (elem_type, [values]))); tensors: [(name, dims, type, bytes)] with
    dims ne[0] first.  Tensor data is laid out in order, each at the next
    multiple of `alignment` of the data section."""
    kv = [(k, t, v) for k, t, v in metadata]
    if alignment != 32 and not any(k == "general.alignment" for k, _, _ in kv):
        kv.append(("general.alignment", T_U32, alignment))
    head = bytearray(struct.pack("<IIQQ", MAGIC, version, len(tensors), len(kv)))
    for k, t, v in kv:
        head += _pack_value(T_STR, k) + struct.pack("<I", t) + _pack_value(t, v)
    off, offsets = 0, []
    for name, dims, ttype, data in tensors:
        if len(data) != tensor_nbytes(tuple(dims), ttype, name):
            raise ValueError(f"{name}: {len(data)} bytes for dims {dims} of type {ttype}")
        offsets.append(off)
        off = (off + len(data) + alignment - 1) // alignment * alignment
    for (name, dims, ttype, _), o in zip(tensors, offsets):
        head += _pack_value(T_STR, name) + struct.pack("<I", len(dims))
        head += b"".join(struct.pack("<Q", d) for d in dims) + struct.pack("<IQ", ttype, o)
    pad = (-len(head)) % alignment
    with open(path, "wb") as f:
        f.write(head + b"\0" * pad)
        for (name, dims, ttype, data), o in zip(tensors, offsets):
            f.write(bytes(data))
            nxt = (o + len(data) + alignment - 1) // alignment * alignment
            f.write(b"\0" * (nxt - o - len(data)))
