"""The `.sam3` weight container on the host: writer and mmap reader.

Format (docs/weight-format.md; src/core/weight.h:26-72, header :44-56,
descriptor :62-70): a 52-byte little-endian header (48 bytes in version
3), `n_tensors` descriptors of 176 bytes, zero padding to a 4096-byte
boundary, then the data blob with every tensor at a 64-byte aligned
offset. Lookup by name goes through an
open-addressing table of FNV-1a hashes (weight.c:51-62, 238-301).

This mirrors `sam3_weight_write` / `sam3_weight_open` / `sam3_weight_find`
/ `sam3_weight_to_tensor` (weight.c:64-236, 303-558) so tests and the
bench can build files and hand their data blob to
`sam3_hip_backend_map_weights`. Errors raise `WeightError` with the
reference's codes (EINVAL, EIO, EMODEL).
"""
import mmap
import os

import numpy as np

from . import abi

MAGIC = 0x334D4153
VERSION = 4
NAME_MAX = 128
DATA_ALIGN = 64
PAGE_ALIGN = 4096
HASH_EMPTY = 0xFFFFFFFF

HEADER = np.dtype([("magic", "<u4"), ("version", "<u4"), ("flags", "<u4"),
                   ("n_tensors", "<u4"), ("image_size", "<i4"), ("encoder_dim", "<i4"),
                   ("decoder_dim", "<i4"), ("n_encoder_layers", "<i4"),
                   ("n_decoder_layers", "<i4"), ("reserved", "<u4", 3),
                   ("text_backbone", "<u4")])
DESC = np.dtype([("name", "S128"), ("dtype", "<u4"), ("n_dims", "<u4"), ("dims", "<i4", 4),
                 ("data_offset", "<u8"), ("data_size", "<u8"), ("reserved", "<u8")])
assert HEADER.itemsize == 52 and DESC.itemsize == 176

# header field <- sam3_model_config field (weight.c:84-99)
CONFIG_KEYS = ("image_size", "encoder_dim", "decoder_dim", "n_encoder_layers",
               "n_decoder_layers", "backbone_type", "n_fpn_scales", "variant", "text_backbone")


class WeightError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"{abi.ERROR_NAMES.get(code, code)}: {msg}")
        self.code = code


def fnv1a(name):
    """32-bit FNV-1a over the name's bytes (weight.c:51-62)."""
    h = 0x811C9DC5
    for b in name.encode() if isinstance(name, str) else name:
        h = ((h ^ b) * 0x01000193) & 0xFFFFFFFF
    return h


def _align(v, a):
    return (v + a - 1) & ~(a - 1)


def tensor_nbytes(dtype, dims):
    n = int(np.prod(dims)) if len(dims) else 1
    if dtype == abi.Q8_0:
        return abi.q8_nbytes(n)
    return n * {abi.F32: 4, abi.F16: 2, abi.BF16: 2, abi.I32: 4, abi.I8: 1}[dtype]


def write(path, tensors, config=None):
    """sam3_weight_write (weight.c:64-236) over a list of
    (name, dtype, dims, data) with data any buffer of the tensor's bytes.
    The file is removed again when writing fails."""
    if not tensors:
        raise WeightError(abi.EINVAL, "weight_write: no tensors")
    cfg = dict.fromkeys(CONFIG_KEYS, 0)
    cfg.update(config or {})
    hdr = np.zeros((), HEADER)
    hdr["magic"], hdr["version"], hdr["flags"], hdr["n_tensors"] = MAGIC, VERSION, 0, len(tensors)
    for k in ("image_size", "encoder_dim", "decoder_dim", "n_encoder_layers", "n_decoder_layers",
              "text_backbone"):
        hdr[k] = cfg[k]
    hdr["reserved"] = (cfg["backbone_type"], cfg["variant"], cfg["n_fpn_scales"])
    descs = np.zeros(len(tensors), DESC)
    blobs = []
    off = 0
    for i, (name, dtype, dims, data) in enumerate(tensors):
        arr = (np.ascontiguousarray(data) if isinstance(data, np.ndarray)
               else np.frombuffer(data, np.uint8))
        raw = memoryview(arr.reshape(-1).view(np.uint8))
        nb = raw.nbytes
        enc = name.encode()[:NAME_MAX - 1]
        descs[i]["name"] = enc
        descs[i]["dtype"] = dtype
        descs[i]["n_dims"] = len(dims)
        descs[i]["dims"] = list(dims) + [0] * (4 - len(dims))
        descs[i]["data_offset"] = off
        descs[i]["data_size"] = nb
        descs[i]["reserved"] = fnv1a(enc)
        blobs.append(raw)
        off = _align(off + nb, DATA_ALIGN)
    table_end = HEADER.itemsize + len(tensors) * DESC.itemsize
    data_start = _align(table_end, PAGE_ALIGN)
    try:
        with open(path, "wb") as f:
            f.write(hdr.tobytes())
            f.write(descs.tobytes())
            f.write(b"\0" * (data_start - table_end))
            for i, raw in enumerate(blobs):
                f.write(raw)
                if i < len(blobs) - 1:
                    f.write(b"\0" * (_align(raw.nbytes, DATA_ALIGN) - raw.nbytes))
    except OSError as e:
        try:
            os.remove(path)
        except OSError:
            pass
        raise WeightError(abi.EIO, f"weight_write: {e}") from e


class WeightFile:
    """sam3_weight_open (weight.c:303-474): the file mapped read-only, the
    descriptor table and data ranges checked, a hash table built for
    lookup by name."""

    def __init__(self, path):
        try:
            fd = os.open(path, os.O_RDONLY)
        except OSError as e:
            raise WeightError(abi.EIO, f"weight_open: cannot open {path}") from e
        try:
            size = os.fstat(fd).st_size
            if size < HEADER.itemsize:
                raise WeightError(abi.EMODEL, f"weight_open: file too small: {path}")
            self.mm = mmap.mmap(fd, size, prot=mmap.PROT_READ)
        finally:
            os.close(fd)
        self.size = size
        self.buf = np.frombuffer(self.mm, np.uint8)
        hdr = self.buf[:HEADER.itemsize].view(HEADER)[0]
        if int(hdr["magic"]) != MAGIC:
            self.close()
            raise WeightError(abi.EMODEL, f"weight_open: bad magic 0x{int(hdr['magic']):08x}")
        ver = int(hdr["version"])
        if ver == 3:
            hsize, self.text_backbone = 48, 0
        elif ver == 4:
            hsize, self.text_backbone = HEADER.itemsize, int(hdr["text_backbone"])
        else:
            self.close()
            raise WeightError(abi.EMODEL, f"weight_open: unsupported version {ver}")
        self.header = hdr
        n = int(hdr["n_tensors"])
        table_end = hsize + n * DESC.itemsize
        if table_end > size:
            self.close()
            raise WeightError(abi.EMODEL, "weight_open: tensor table exceeds file")
        self.data_start = _align(table_end, PAGE_ALIGN)
        if self.data_start > size:
            self.close()
            raise WeightError(abi.EMODEL, "weight_open: data section starts past the end")
        self.descs = self.buf[hsize:table_end].view(DESC)
        ends = self.descs["data_offset"].astype(object) + self.descs["data_size"].astype(object)
        if n and max(ends) > size - self.data_start:
            self.close()
            raise WeightError(abi.EMODEL, "weight_open: tensor data extends past file end")
        self._build_hash()

    def _build_hash(self):
        """build_hash_table (weight.c:250-301): 4x the tensor count rounded
        up to a power of two, at least 8; the stored hash is used when the
        descriptor's reserved field holds one."""
        n = len(self.descs)
        cap = 1
        while cap < max(8, 4 * n):
            cap <<= 1
        self.table = [HASH_EMPTY] * cap
        mask = cap - 1
        for i in range(n):
            r = int(self.descs[i]["reserved"])
            h = r & 0xFFFFFFFF if r else fnv1a(self.descs[i]["name"])
            slot = h & mask
            while self.table[slot] != HASH_EMPTY:
                slot = (slot + 1) & mask
            self.table[slot] = i

    @property
    def n_tensors(self):
        return len(self.descs)

    def find(self, name):
        """sam3_weight_find (weight.c:505-522): index of the descriptor, or None."""
        enc = name.encode() if isinstance(name, str) else name
        mask = len(self.table) - 1
        slot = fnv1a(enc) & mask
        while self.table[slot] != HASH_EMPTY:
            i = self.table[slot]
            if self.descs[i]["name"] == enc:
                return i
            slot = (slot + 1) & mask
        return None

    @property
    def data_base(self):
        """Host address of the data blob."""
        return self.buf.ctypes.data + self.data_start

    @property
    def data_size(self):
        return self.size - self.data_start

    def array(self, i):
        """The tensor's bytes in the mapping (read-only uint8 view)."""
        d = self.descs[i]
        o = self.data_start + int(d["data_offset"])
        return self.buf[o:o + int(d["data_size"])]

    def to_tensor(self, i):
        """sam3_weight_to_tensor (weight.c:534-558): a tensor header whose
        data points into the mapping; Q8_0 strides zero."""
        d = self.descs[i]
        nd = int(d["n_dims"])
        dims = [int(x) for x in d["dims"][:nd]]
        t = abi.make_tensor(int(d["dtype"]), dims, self.data_base + int(d["data_offset"]),
                            int(d["data_size"]))
        return t

    def close(self):
        self.descs = None
        self.buf = None
        if getattr(self, "mm", None) is not None:
            try:
                self.mm.close()
            except BufferError:
                pass  # views still alive; the mapping goes with them
            self.mm = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()
