"""The `.fni8` checkpoint container: quantized weights stored in the layout the
kernels consume, so loading is a memory map plus one copy per tensor.

Mirrors the interface the reference reaches in its closed `fni8.format` module:
`save_fni8(path, tensors, shards=..., meta=...)` (tests/test_smoke.py:40, :61;
tests/test_convert.py:132), the streaming `FQWriter(path)` with `.add(name, qt)`
and `.finalize(meta=...)` (fni8serve/convert.py:318-361), and `FQReader(path)`
with `.header`, `.names`, `.shards`, `.load_many(names, device)` and `.close()`
(fni8serve/loader.py:32-45, :59-69; tools/fine_tune.py:57-58).  The reference's
byte layout is not available, so this one is its own, versioned design:

    [0, 16)       b"FNI8AMD\\0", u32 format version, u32 flags (0)
    [4096, ...)   tensor blobs, each at a 4096-byte aligned offset, in the
                  resident layout: per_row_i8 int8 [N, K] + fp32 [N];
                  per_group_i4 packed uint8 [N, K/2] + fp32 [N, K/g];
                  raw tensors as stored
    [h, h + n)    the header: UTF-8 JSON (tensor table, shard index, meta)
    last 24 bytes u64 h, u64 n, b"FNI8AMD\\0"

The header sits at the end so the writer can stream tensors to disk as they are
produced (the converter quantizes one source shard at a time).  Header fields
follow what the reference's callers read: "arch" (the hardware target, the
reference's is "sm70" -- tests/test_convert.py:361-362), "quant", "version",
"__meta__" (the model description, convert.py:351-359) and the shard index
{"experts": {id: [names]}, "pp_stages": [[names], ...]} (loader.py:33-40).
All integers are little-endian.
"""
from __future__ import annotations

import json
import mmap
import os
import struct
import threading
import warnings
from concurrent.futures import ThreadPoolExecutor

import torch

from .qtensor import QTensor

MAGIC = b"FNI8AMD\0"
FORMAT_VERSION = 1
ARCH = "gfx950"
ALIGN = 4096
_TRAILER = struct.Struct("<QQ8s")
_CHUNK = 8 << 20  # bytes per read / host-to-device copy of a device load
_THREADS = 8      # reader threads of a device load, two pinned staging buffers each

# Pinned staging buffers of device loads, allocated on first use and kept for
# reuse (pinning memory costs more than a warm read of the same size); at most
# 2 * _THREADS * _CHUNK bytes (128 MiB).
_STAGING_LOCK = threading.Lock()
_STAGING: list[torch.Tensor] = []


def _staging(count: int, size: int) -> list[torch.Tensor]:
    global _STAGING
    if len(_STAGING) < count or _STAGING[0].numel() < size:
        _STAGING = []  # drop the old set before pinning the new one
        _STAGING = [torch.empty(size, dtype=torch.uint8, pin_memory=True) for _ in range(count)]
    return _STAGING[:count]


def release_staging() -> None:
    """Free the pinned staging buffers kept by device loads."""
    global _STAGING
    with _STAGING_LOCK:
        _STAGING = []


_DTYPES = {
    "int8": torch.int8, "uint8": torch.uint8, "int16": torch.int16, "int32": torch.int32,
    "int64": torch.int64, "float16": torch.float16, "bfloat16": torch.bfloat16,
    "float32": torch.float32, "float64": torch.float64, "bool": torch.bool,
}
_NAMES = {v: k for k, v in _DTYPES.items()}


def _as_qtensor(obj) -> QTensor:
    if isinstance(obj, QTensor):
        return obj
    if isinstance(obj, torch.Tensor):  # norms, embeddings, router gates: stored unquantized
        return QTensor(obj, None, scheme="raw")
    raise TypeError(f"cannot store {type(obj).__name__}: expected a QTensor or a tensor")


class FQWriter:
    """Streaming writer: `add` appends a tensor's blobs, `finalize` writes the
    header and trailer.  Use as a context manager; leaving the block without
    `finalize` (an exception) removes the partial file."""

    def __init__(self, path: str, *, arch: str = ARCH):
        self.path = path
        self.arch = arch
        self._f = open(path, "wb")
        self._f.write(MAGIC + struct.pack("<II", FORMAT_VERSION, 0))
        self._pos = 16
        self._tensors: dict[str, dict] = {}
        self._schemes: set[str] = set()
        self._done = False

    def _blob(self, t: torch.Tensor) -> dict:
        t = t.detach().to("cpu").contiguous()
        if t.dtype not in _NAMES:
            raise TypeError(f"unsupported dtype {t.dtype}")
        pad = (-self._pos) % ALIGN
        if pad:
            self._f.write(b"\0" * pad)
            self._pos += pad
        raw = t.reshape(-1).view(torch.uint8).numpy() if t.numel() else b""
        self._f.write(memoryview(raw))
        entry = {"dtype": _NAMES[t.dtype], "shape": list(t.shape), "offset": self._pos,
                 "nbytes": t.numel() * t.element_size()}
        self._pos += entry["nbytes"]
        return entry

    def add(self, name: str, obj) -> None:
        if self._done:
            raise RuntimeError("writer already finalized")
        if name in self._tensors:
            raise ValueError(f"duplicate tensor name {name!r}")
        qt = _as_qtensor(obj)
        self._tensors[name] = {
            "scheme": qt.scheme, "group_size": qt.group_size, "codebook": qt.codebook,
            "data": self._blob(qt.data),
            "scale": None if qt.scale is None else self._blob(qt.scale),
        }
        self._schemes.add(qt.scheme)

    def finalize(self, meta: dict | None = None, shards: dict | None = None) -> None:
        if self._done:
            return
        shards = {} if shards is None else shards
        for key, groups in shards.items():
            lists = groups.values() if isinstance(groups, dict) else groups
            for names in lists:
                missing = [n for n in names if n not in self._tensors]
                if missing:
                    raise KeyError(f"shard {key!r} names unknown tensors {missing[:3]}")
        quant = sorted(self._schemes - {"raw"})
        header = {
            "version": FORMAT_VERSION, "arch": self.arch,
            "quant": quant[0] if len(quant) == 1 else ("mixed" if quant else "raw"),
            "tensors": self._tensors, "shards": shards, "__meta__": meta or {},
        }
        blob = json.dumps(header, separators=(",", ":")).encode()
        self._f.write(blob)
        self._f.write(_TRAILER.pack(self._pos, len(blob), MAGIC))
        self._f.close()
        self._done = True

    def close(self) -> None:
        if not self._done:
            self._f.close()
            os.remove(self.path)
            self._done = True

    def __enter__(self):
        return self

    def __exit__(self, exc_type, exc, tb):
        if exc_type is None:
            self.finalize()
        else:
            self.close()
        return False


class FQReader:
    """Memory-mapped reader.  `load`/`load_many` copy only the requested tensors'
    pages, which is what makes per-shard (pipeline stage, expert) loads cheap."""

    def __init__(self, path: str):
        self.path = path
        self._f = open(path, "rb")
        size = os.fstat(self._f.fileno()).st_size
        if size < 16 + _TRAILER.size:
            self._f.close()
            raise ValueError(f"{path}: too short to be a .fni8 container")
        self._mm = mmap.mmap(self._f.fileno(), 0, access=mmap.ACCESS_READ)
        try:
            if self._mm[:8] != MAGIC:
                raise ValueError(f"{path}: not a .fni8 container (bad magic)")
            version = struct.unpack_from("<I", self._mm, 8)[0]
            if version != FORMAT_VERSION:
                raise ValueError(f"{path}: container version {version}, this library reads "
                                 f"{FORMAT_VERSION}")
            hoff, hlen, tail = _TRAILER.unpack_from(self._mm, size - _TRAILER.size)
            if tail != MAGIC or hoff + hlen != size - _TRAILER.size or hoff < 16:
                raise ValueError(f"{path}: truncated or corrupt container trailer")
            self.header = json.loads(bytes(self._mm[hoff:hoff + hlen]))
            for name, t in self.header["tensors"].items():
                for part in ("data", "scale"):
                    b = t[part]
                    if b is None:
                        continue
                    if b["dtype"] not in _DTYPES:
                        raise ValueError(f"{path}: tensor {name!r} has unknown dtype {b['dtype']!r}")
                    n = torch.empty((), dtype=_DTYPES[b["dtype"]]).element_size()
                    for d in b["shape"]:
                        n *= d
                    if n != b["nbytes"]:
                        raise ValueError(f"{path}: tensor {name!r} {part} size disagrees with "
                                         f"its shape")
                    if b["offset"] < 16 or b["offset"] + b["nbytes"] > hoff:
                        raise ValueError(f"{path}: tensor {name!r} lies outside the data region")
        except Exception:
            self.close()
            raise
        self.names = list(self.header["tensors"])
        self.shards = self.header.get("shards", {})

    def _entry(self, name: str) -> dict:
        try:
            return self.header["tensors"][name]
        except KeyError:
            raise KeyError(f"no tensor {name!r} in {self.path}") from None

    def _cpu_tensor(self, b: dict) -> torch.Tensor:
        dtype = _DTYPES[b["dtype"]]
        n = b["nbytes"] // torch.empty((), dtype=dtype).element_size()
        if n == 0:
            return torch.empty(b["shape"], dtype=dtype)
        with warnings.catch_warnings():  # the map is read-only; the view is copied at once
            warnings.simplefilter("ignore", UserWarning)
            view = torch.frombuffer(self._mm, dtype=dtype, count=n, offset=b["offset"])
        return view.reshape(b["shape"]).clone()

    def _device_tensors(self, blobs: list[dict], device) -> list[torch.Tensor]:
        """Allocate the blobs on `device` and fill them from the file.  The byte
        ranges are cut into chunks, in file order, and dealt round-robin to
        `_THREADS` workers; each worker `preadv`s a chunk into one of its two
        pinned buffers and copies it to the device on its own stream, so reads
        (page cache -> pinned memory, a CPU copy) overlap one another and the
        host-to-device copies."""
        outs, pieces = [], []
        for b in blobs:
            t = torch.empty(b["shape"], dtype=_DTYPES[b["dtype"]], device=device)
            outs.append(t)
            if b["nbytes"]:
                flat = t.view(-1).view(torch.uint8)
                for s in range(0, b["nbytes"], _CHUNK):
                    pieces.append((b["offset"] + s, min(_CHUNK, b["nbytes"] - s), flat, s))
        if not pieces:
            return outs
        pieces.sort(key=lambda p: p[0])
        nthreads = min(_THREADS, len(pieces))
        fd = self._f.fileno()
        producer = torch.cuda.current_stream(device)

        def work(w, bufs):
            views = [memoryview(b.numpy()) for b in bufs]
            stream = torch.cuda.Stream(device)
            stream.wait_stream(producer)  # the outputs were allocated on `producer`
            freed = [None, None]
            for k, i in enumerate(range(w, len(pieces), nthreads)):
                j = k & 1
                if freed[j] is not None:
                    freed[j].synchronize()  # the copy that last read this buffer is done
                off, n, dst, s = pieces[i]
                got = 0
                while got < n:
                    r = os.preadv(fd, [views[j][got:n]], off + got)
                    if r <= 0:
                        raise OSError(f"{self.path}: short read at offset {off + got}")
                    got += r
                with torch.cuda.stream(stream):
                    dst[s:s + n].copy_(bufs[j][:n], non_blocking=True)
                    freed[j] = torch.cuda.Event()
                    freed[j].record(stream)
            stream.synchronize()

        with _STAGING_LOCK:
            bufs = _staging(2 * nthreads, max(p[1] for p in pieces))
            with ThreadPoolExecutor(nthreads) as pool:
                jobs = [pool.submit(work, w, bufs[2 * w:2 * w + 2]) for w in range(nthreads)]
                for job in jobs:
                    job.result()
        return outs

    def load(self, name: str, device="cpu") -> QTensor:
        return self.load_many([name], device)[name]

    def load_many(self, names, device="cpu") -> dict[str, QTensor]:
        entries = {n: self._entry(n) for n in names}
        blobs = [t[p] for t in entries.values() for p in ("data", "scale") if t[p] is not None]
        if torch.device(device).type == "cpu":
            tensors = [self._cpu_tensor(b) for b in blobs]
        else:
            tensors = self._device_tensors(blobs, device)
        out, it = {}, iter(tensors)
        for n, t in entries.items():
            data = next(it)
            scale = None if t["scale"] is None else next(it)
            out[n] = QTensor(data, scale, scheme=t["scheme"], group_size=t["group_size"],
                             codebook=t["codebook"])
        return out

    def close(self) -> None:
        mm, self._mm = getattr(self, "_mm", None), None
        if mm is not None:
            mm.close()
        if not self._f.closed:
            self._f.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
        return False


def save_fni8(path: str, tensors: dict, *, shards: dict | None = None, meta: dict | None = None,
              arch: str = ARCH) -> None:
    """Write {name: QTensor or tensor} in one call."""
    with FQWriter(path, arch=arch) as w:
        for name, obj in tensors.items():
            w.add(name, obj)
        w.finalize(meta=meta, shards=shards)
