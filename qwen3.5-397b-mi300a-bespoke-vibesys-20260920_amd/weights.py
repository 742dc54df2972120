"""Checkpoint reader for the on-disk format: safetensors shards and the stacked expert layout.

`Checkpoint` maps every tensor name of a directory of `*.safetensors` shards to its shard,
dtype, shape and byte range by reading the shard headers (an 8-byte little-endian header
length, then a JSON table of `dtype`, `shape` and `data_offsets` relative to the end of the
header), and reads tensors on demand with `os.preadv`, which releases the GIL and shares no
file offset, so many threads read at once (`weights.py:30-79`). `load_experts` stacks one
layer's per-expert tensors into the `[E, ...]` layout the MoE kernels read (`model.py:758-804`):
`gate_up = cat(gate_proj, up_proj)` per expert, MXFP4 payloads and e8m0 scales kept as uint8.

For a device target the bytes go from the file straight into a pinned host buffer and from
there by DMA into the slice of the stacked device tensor they belong to: no pageable copy and
no stacked host copy. One MI355X holds a whole checkpoint's experts (205 GB of MXFP4 for the
397B model in 288 GB of HBM), so `Shard` is normally the whole expert axis; a slice of it is
what an expert-parallel rank would read.
"""

from __future__ import annotations

import json
import os
import threading
from concurrent.futures import ThreadPoolExecutor
from dataclasses import dataclass
from pathlib import Path

import torch

LOAD_THREADS = int(os.environ.get("SEED_LOAD_THREADS", "32"))
"""Reader threads of `load_experts` (`model.py:146`)."""

_DTYPES = {
    "BF16": torch.bfloat16,
    "F16": torch.float16,
    "F32": torch.float32,
    "U8": torch.uint8,
    "I8": torch.int8,
    "I32": torch.int32,
    "I64": torch.int64,
    "BOOL": torch.bool,
}


@dataclass(frozen=True)
class Shard:
    """`count` consecutive items of an axis, the first at index `start` (`tp.py:131-143`)."""

    start: int
    count: int

    @property
    def stop(self) -> int:
        return self.start + self.count

    def rows(self, width: int) -> slice:
        """The rows of a weight laid out as `width` output rows per item of this axis."""
        return slice(self.start * width, self.stop * width)


@dataclass(frozen=True)
class TensorInfo:
    path: Path
    dtype: torch.dtype
    shape: tuple[int, ...]
    offset: int  # absolute byte offset in the shard
    nbytes: int


def _parse_shard(path: Path) -> dict[str, TensorInfo]:
    """The tensor table of one safetensors file, from the format itself: a little-endian u64
    header size N, N bytes of UTF-8 JSON mapping each tensor name to its `dtype`, `shape` and
    `data_offsets` [begin, end) within the data section that follows the header (plus an
    optional `__metadata__` entry), then the data section. Every entry is checked: a known
    dtype, a byte range inside the data section, and a size equal to shape x item size."""
    size = path.stat().st_size
    with open(path, "rb") as fh:
        prefix = fh.read(8)
        if len(prefix) < 8:
            raise OSError(f"{path}: shorter than a safetensors header")
        header_len = int.from_bytes(prefix, "little")
        if header_len > size - 8:
            raise OSError(f"{path}: header of {header_len} bytes overruns the file")
        table = json.loads(fh.read(header_len).decode("utf-8"))
    data_start, data_len = 8 + header_len, size - 8 - header_len
    out: dict[str, TensorInfo] = {}
    for key, entry in table.items():
        if key == "__metadata__":
            continue
        dtype = _DTYPES.get(entry.get("dtype"))
        if dtype is None:
            raise ValueError(f"{path}: tensor {key} has unsupported dtype {entry.get('dtype')!r}")
        shape = tuple(int(d) for d in entry["shape"])
        begin, stop = (int(o) for o in entry["data_offsets"])
        want = dtype.itemsize
        for d in shape:
            want *= d
        if not 0 <= begin <= stop <= data_len or stop - begin != want:
            raise ValueError(f"{path}: tensor {key} has byte range [{begin}, {stop}) for "
                             f"{want} bytes in a {data_len}-byte data section")
        out[key] = TensorInfo(path, dtype, shape, data_start + begin, stop - begin)
    return out


class Checkpoint:
    """Every tensor of a directory of `*.safetensors` shards, indexed by name from the shard
    headers (`weights.py:30-59` is the interface: `files`, `has`, `load`); the bytes are read on
    demand with `os.preadv` through one read-only descriptor per shard, opened on first use."""

    def __init__(self, path: str | Path) -> None:
        root = Path(path)
        self.files = sorted(root.glob("*.safetensors"))
        if not self.files:
            raise FileNotFoundError(f"{root} holds no *.safetensors shard")
        self._index: dict[str, TensorInfo] = {}
        for shard in self.files:
            for key, meta in _parse_shard(shard).items():
                if key in self._index:
                    raise ValueError(f"tensor {key} appears in {self._index[key].path.name} "
                                     f"and {shard.name}")
                self._index[key] = meta
        self._open: dict[Path, int] = {}
        self._open_lock = threading.Lock()

    def _fd(self, shard: Path) -> int:
        fd = self._open.get(shard)
        if fd is None:
            with self._open_lock:
                fd = self._open.get(shard)
                if fd is None:
                    fd = self._open[shard] = os.open(shard, os.O_RDONLY)
        return fd

    def close(self) -> None:
        with self._open_lock:
            for fd in self._open.values():
                os.close(fd)
            self._open.clear()

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass

    def has(self, name: str) -> bool:
        return name in self._index

    def names(self) -> list[str]:
        return sorted(self._index)

    def info(self, name: str) -> TensorInfo:
        return self._index[name]

    def read_into(self, name: str, buf: torch.Tensor) -> torch.Tensor:
        """Read the raw bytes of `name` into the front of the uint8 CPU tensor `buf` (pinned or
        not); returns the filled `[nbytes]` view. Safe from many threads."""
        meta = self._index[name]
        if buf.dtype != torch.uint8 or buf.device.type != "cpu" or not buf.is_contiguous():
            raise ValueError("buf must be a contiguous uint8 CPU tensor")
        if buf.numel() < meta.nbytes:
            raise ValueError(f"buf holds {buf.numel()} bytes, {name} needs {meta.nbytes}")
        view = memoryview(buf.numpy()).cast("B")
        got = 0
        while got < meta.nbytes:
            n = os.preadv(self._fd(meta.path), [view[got:meta.nbytes]], meta.offset + got)
            if n <= 0:
                raise OSError(f"short read for {name}")
            got += n
        return buf[: meta.nbytes]

    def load(self, name: str, device: str | torch.device,
             dtype: torch.dtype | None = None) -> torch.Tensor:
        """Read one tensor onto `device`, cast to `dtype` unless None. Safe from many threads."""
        meta = self._index[name]
        device = torch.device(device)
        pin = device.type == "cuda"
        raw = torch.empty(meta.nbytes, dtype=torch.uint8, pin_memory=pin)
        if meta.nbytes:
            self.read_into(name, raw)
        host = raw.view(meta.dtype).reshape(meta.shape) if meta.nbytes else \
            torch.empty(meta.shape, dtype=meta.dtype)
        return host.to(device=device, dtype=dtype or meta.dtype)


class _Staging(threading.local):
    """One pinned (or plain, for a CPU target) byte buffer per reader thread, grown on demand."""

    def get(self, nbytes: int, pin: bool) -> torch.Tensor:
        buf = getattr(self, "buf", None)
        if buf is None or buf.numel() < nbytes:
            buf = torch.empty(nbytes, dtype=torch.uint8, pin_memory=pin)
            self.buf = buf
        return buf


def load_experts(ck: Checkpoint, p: str, sh: Shard, dev: torch.device | str,
                 dtype: torch.dtype) -> dict[str, torch.Tensor]:
    """Stack experts `[sh.start, sh.stop)` of layer prefix `p` (e.g. `mtp.layers.0.mlp`) into
    `gate_up` `[count, 2I, ...]` (gate rows, then up rows), `down` `[count, H, ...]` and, for an
    MXFP4 checkpoint, `gate_up_scale` / `down_scale` (`model.py:758-804`). MXFP4 payloads stay
    uint8; dense checkpoints are cast to `dtype`. Local expert i is global expert
    `sh.start + i`.

    An MXFP4 shard loaded onto a device that runs the fused kernels (`mxfp4_gemv.available`)
    is checked there and then (`mxfp4_gemv.require_supported`, the reference's boot check
    `model.py:1568-1575`): a block the kernels cannot decode exactly raises `ValueError` here."""
    dev = torch.device(dev)
    quant = ck.has(f"{p}.experts.{sh.start}.gate_proj.weight_scale")
    if sh.count <= 0:
        raise ValueError("empty expert shard")

    def name(e: int, proj: str, suffix: str) -> str:
        return f"{p}.experts.{e}.{proj}.{suffix}"

    def stacked(parts: tuple[str, ...], suffix: str, keep: torch.dtype | None) -> torch.Tensor:
        first = [ck.info(name(sh.start, proj, suffix)) for proj in parts]
        src = first[0].dtype
        for m in first[1:]:
            if m.dtype != src or m.shape[1:] != first[0].shape[1:]:
                raise ValueError(f"{p}: {parts} of expert {sh.start} do not concatenate")
        shape = (sum(m.shape[0] for m in first), *first[0].shape[1:])
        nbytes = sum(m.nbytes for m in first)
        out = torch.empty((sh.count, *shape), dtype=keep or src, device=dev)
        staging = _Staging()

        def fill(i: int) -> None:
            e = sh.start + i
            buf = staging.get(nbytes, dev.type == "cuda")
            at = 0
            for proj, ref in zip(parts, first):
                meta = ck.info(name(e, proj, suffix))
                if meta.dtype != ref.dtype or meta.shape != ref.shape:
                    raise ValueError(f"{name(e, proj, suffix)}: {meta.dtype} {meta.shape}, "
                                     f"expert {sh.start} has {ref.dtype} {ref.shape}")
                ck.read_into(name(e, proj, suffix), buf[at:])
                at += meta.nbytes
            # the concatenation along rows is the concatenation of the row-major bytes
            host = buf[:nbytes].view(src).reshape(shape)
            out[i].copy_(host)  # synchronous: the staging buffer is reused by this thread

        with ThreadPoolExecutor(max(1, min(LOAD_THREADS, sh.count))) as pool:
            list(pool.map(fill, range(sh.count)))
        return out

    keep = None if quant else dtype  # uint8 payloads stay uint8; dense checkpoints take `dtype`
    ex = {
        "gate_up": stacked(("gate_proj", "up_proj"), "weight", keep),
        "down": stacked(("down_proj",), "weight", keep),
    }
    if quant:
        ex["gate_up_scale"] = stacked(("gate_proj", "up_proj"), "weight_scale", None)
        ex["down_scale"] = stacked(("down_proj",), "weight_scale", None)
        if dev.type == "cuda":
            import mxfp4_gemv

            if mxfp4_gemv.available(dev):
                mxfp4_gemv.require_supported(ex, f"{p} experts [{sh.start}, {sh.start + sh.count})")
    return ex
