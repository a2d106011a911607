"""Safetensors shard streaming for EXL3 checkpoints.

Keeps the reference loader's surface (src/sglang_exl3/loader.py:121-229):
``iter_safetensors_pread`` yields one ``(name, cpu tensor)`` at a time, read
with ``pread`` into a buffer of its own (no mmap), and asks the kernel to drop
the file range from the page cache once it is read, so host memory holds about
one copy of the weights while they move to the GPU; ``exl3_mmap_weights_iterator``
chains the shards in load order.  ``EXL3MMapModelLoader`` plugs the iterator
into SGLang's model loader when SGLang is importable, and lists the
``*.safetensors`` shards of a local folder itself when it is not.

The file format (safetensors): an 8-byte little-endian header length, a JSON
header mapping each tensor name to ``dtype``, ``shape`` and ``data_offsets``
(relative to the end of the header), an optional ``__metadata__`` entry, then
the raw little-endian tensor bytes.
"""

from __future__ import annotations

import glob
import json
import logging
import math
import os
import struct
import time
from typing import Any, Dict, Generator, List, Optional, Tuple, Union

import torch

logger = logging.getLogger("sglang.exl3.loader")

LOAD_FORMAT_EXL3_MMAP = "exl3_mmap"


class LoadFormatEXL3:
    EXL3_MMAP = LOAD_FORMAT_EXL3_MMAP


# safetensors dtype name -> torch dtype (the names are the file format's)
_DTYPES: Dict[str, torch.dtype] = {
    "BOOL": torch.bool,
    "U8": torch.uint8,
    "I8": torch.int8,
    "I16": torch.int16,
    "I32": torch.int32,
    "I64": torch.int64,
    "F16": torch.float16,
    "BF16": torch.bfloat16,
    "F32": torch.float32,
    "F64": torch.float64,
}
for _name, _attr in (("F8_E4M3", "float8_e4m3fn"), ("F8_E5M2", "float8_e5m2")):
    if hasattr(torch, _attr):
        _DTYPES[_name] = getattr(torch, _attr)

_MAX_HEADER_BYTES = 100 << 20  # a header larger than this is not a safetensors file


def is_unified_memory_platform() -> bool:
    """Whether the GPU shares one coherent memory with the host.  An MI355X is a
    discrete accelerator with its own HBM, so this is False on the target; the
    function stays for callers of the reference API."""
    return False


def madvise_file_preload(file_path: str) -> bool:
    """Ask the kernel to start reading a whole file ahead (POSIX_FADV_WILLNEED)."""
    advise = getattr(os, "posix_fadvise", None)
    if advise is None:
        return False
    try:
        fd = os.open(file_path, os.O_RDONLY)
    except OSError:
        return False
    try:
        advise(fd, 0, 0, getattr(os, "POSIX_FADV_WILLNEED", 3))
        return True
    except OSError:
        return False
    finally:
        os.close(fd)


def _drop_pages(fd: int, offset: int, length: int) -> None:
    """Best effort: release the clean page-cache pages of a file range (length 0: to the end)."""
    advise = getattr(os, "posix_fadvise", None)
    if advise is None:
        return
    try:
        advise(fd, offset, length, getattr(os, "POSIX_FADV_DONTNEED", 4))
    except OSError:
        pass


def host_memory_summary(device: Union[str, torch.device, None] = None) -> str:
    """One line of host and device memory figures for load-time logging."""
    avail = swap = float("nan")
    try:
        info: Dict[str, int] = {}
        with open("/proc/meminfo") as fh:
            for line in fh:
                key, _, rest = line.partition(":")
                info[key] = int(rest.split()[0])
        avail = info["MemAvailable"] / (1 << 20)
        swap = (info.get("SwapTotal", 0) - info.get("SwapFree", 0)) / 1024
    except (OSError, KeyError, ValueError, IndexError):
        pass
    dev_gib = float("nan")
    try:
        if torch.cuda.is_available():
            dev_gib = torch.cuda.memory_allocated(device) / (1 << 30)
    except Exception:  # noqa: BLE001 - a logging helper never raises
        pass
    return f"MemAvailable={avail:.2f}GiB swap_used={swap:.0f}MiB device_allocated={dev_gib:.2f}GiB"


def _pread_exact(fd: int, size: int, offset: int, path: str, what: str) -> bytearray:
    buf = bytearray(size)
    view = memoryview(buf)
    done = 0
    try:
        while done < size:
            n = os.preadv(fd, [view[done:]], offset + done)
            if n <= 0:
                raise IOError(f"[EXL3 loader] short read in {path} at {what}: {done}/{size} bytes")
            done += n
    finally:
        view.release()
    return buf


def read_safetensors_header(fd: int, path: str) -> Tuple[Dict[str, Any], int]:
    """The tensor entries of a safetensors file (``__metadata__`` removed) and
    the file offset of its data section."""
    size = os.fstat(fd).st_size
    if size < 8:
        raise ValueError(f"[EXL3 loader] {path} is too short to be a safetensors file")
    (hlen,) = struct.unpack("<Q", bytes(_pread_exact(fd, 8, 0, path, "header length")))
    if hlen > min(size - 8, _MAX_HEADER_BYTES):
        raise ValueError(f"[EXL3 loader] {path}: header length {hlen} does not fit the file ({size} bytes)")
    header = json.loads(bytes(_pread_exact(fd, hlen, 8, path, "header")))
    if not isinstance(header, dict):
        raise ValueError(f"[EXL3 loader] {path}: header is not a JSON object")
    header.pop("__metadata__", None)
    return header, 8 + hlen


def iter_safetensors_pread(path: str) -> Generator[Tuple[str, torch.Tensor], None, None]:
    """Yield the tensors of one safetensors shard in file order, each read with
    pread into a buffer of its own (so it is freed when the consumer drops
    it), then drop the file range from the page cache.

    Raises RuntimeError for a dtype the table above does not know, ValueError
    for an entry whose byte range does not match its shape or lies outside the
    file, IOError on a short read (reference: src/sglang_exl3/loader.py:121-168).
    """
    fd = os.open(path, os.O_RDONLY)
    try:
        header, base = read_safetensors_header(fd, path)
        fsize = os.fstat(fd).st_size
        entries = sorted(header.items(), key=lambda kv: int(kv[1]["data_offsets"][0]))
        for name, info in entries:
            dname = info.get("dtype")
            if dname not in _DTYPES:
                raise RuntimeError(f"[EXL3 loader] unsupported safetensors dtype {dname} for {name} in {path}")
            dtype = _DTYPES[dname]
            shape = tuple(int(d) for d in info["shape"])
            start, end = (int(v) for v in info["data_offsets"])
            nbytes = end - start
            itemsize = torch.empty((), dtype=dtype).element_size()
            if nbytes != math.prod(shape) * itemsize or start < 0 or base + end > fsize:
                raise ValueError(f"[EXL3 loader] {path}: {name} has byte range [{start}, {end}) for shape {shape} "
                                 f"{dname} in a file of {fsize} bytes")
            if nbytes == 0:
                yield name, torch.empty(shape, dtype=dtype)
                continue
            buf = _pread_exact(fd, nbytes, base + start, path, name)
            _drop_pages(fd, base + start, nbytes)
            tensor = torch.frombuffer(buf, dtype=dtype).reshape(shape)
            del buf
            yield name, tensor
            del tensor
    finally:
        _drop_pages(fd, 0, 0)
        os.close(fd)


def exl3_mmap_weights_iterator(hf_weights_files: List[str], device: Union[str, torch.device] = "cpu",
                               num_threads: int = 8, prefetch_shards: int = 2,
                               drop_cache_after_load: bool = False) -> Generator[Tuple[str, torch.Tensor], None, None]:
    """The tensors of every shard, shard after shard (reference:
    src/sglang_exl3/loader.py:171-229).  Shards are read one at a time;
    ``num_threads``, ``prefetch_shards`` and ``drop_cache_after_load`` are
    accepted for the reference's signature (the page cache is always dropped)."""
    del num_threads, prefetch_shards, drop_cache_after_load
    if not hf_weights_files:
        return
    t0 = time.perf_counter()
    total_bytes = total = 0
    try:
        for index, path in enumerate(hf_weights_files, start=1):
            count = 0
            for name, tensor in iter_safetensors_pread(path):
                total_bytes += tensor.numel() * tensor.element_size()
                total += 1
                count += 1
                yield name, tensor
            logger.info("[EXL3 loader] shard %d/%d %s tensors=%d %s", index, len(hf_weights_files),
                        os.path.basename(path), count, host_memory_summary(device))
    finally:
        dt = time.perf_counter() - t0
        logger.info("[EXL3 loader] read %d tensors (%.2f GiB) from %d shards in %.2fs", total,
                    total_bytes / (1 << 30), len(hf_weights_files), dt)


try:  # pragma: no cover - depends on SGLang being installed
    from sglang.srt.model_loader.loader import DefaultModelLoader  # type: ignore

    _HAVE_SGLANG_LOADER = True
except Exception:  # noqa: BLE001
    DefaultModelLoader = object  # type: ignore[assignment,misc]
    _HAVE_SGLANG_LOADER = False


def list_safetensors_shards(folder: str) -> List[str]:
    """The ``*.safetensors`` files of a local checkpoint folder, in name order."""
    return sorted(glob.glob(os.path.join(folder, "*.safetensors")))


class EXL3MMapModelLoader(DefaultModelLoader):  # type: ignore[misc,valid-type]
    """Model loader whose weights iterator is ``exl3_mmap_weights_iterator``
    (reference: src/sglang_exl3/loader.py:245-315)."""

    def __init__(self, load_config: Any):
        if _HAVE_SGLANG_LOADER:  # pragma: no cover
            super().__init__(load_config)
        else:
            self.load_config = load_config
        self.load_format = LOAD_FORMAT_EXL3_MMAP

    def _prepare_weights(self, model_name_or_path: str, revision: Optional[str],
                         fall_back_to_pt: bool) -> Tuple[str, List[str], bool]:
        if _HAVE_SGLANG_LOADER:  # pragma: no cover
            # SGLang's shard discovery knows only its own formats: present the
            # custom format as safetensors for the lookup, then restore it
            from sglang.srt.configs.load_config import LoadFormat  # type: ignore

            saved = self.load_config.load_format
            self.load_config.load_format = LoadFormat.SAFETENSORS
            try:
                return super()._prepare_weights(model_name_or_path, revision, fall_back_to_pt)
            finally:
                self.load_config.load_format = saved
        files = list_safetensors_shards(model_name_or_path)
        if not files:
            raise FileNotFoundError(f"[EXL3 loader] no *.safetensors shards in {model_name_or_path}")
        return model_name_or_path, files, True

    def _get_weights_iterator(self, source: Any, *, resolved_source: Optional[Any] = None,
                              startup_prefetch_started: bool = False, startup_prefetch_active: bool = False):
        extra = getattr(self.load_config, "model_loader_extra_config", None) or {}
        if resolved_source is None:
            _, files, use_safetensors = self._prepare_weights(source.model_or_path, getattr(source, "revision", None),
                                                              getattr(source, "fall_back_to_pt", False))
        else:
            files = list(resolved_source.weight_files)
            use_safetensors = resolved_source.use_safetensors
        if not use_safetensors:
            if not _HAVE_SGLANG_LOADER:
                raise RuntimeError("[EXL3 loader] only safetensors checkpoints are supported without SGLang")
            return super()._get_weights_iterator(  # pragma: no cover
                source, resolved_source=resolved_source, startup_prefetch_started=startup_prefetch_started,
                startup_prefetch_active=startup_prefetch_active)
        device = "cuda:0" if torch.cuda.is_available() else "cpu"
        it = exl3_mmap_weights_iterator(files, device=device, num_threads=extra.get("num_threads", 8),
                                        prefetch_shards=extra.get("prefetch_shards", 2),
                                        drop_cache_after_load=extra.get("drop_cache_after_load", False))
        prefix = getattr(source, "prefix", "") or ""
        return ((prefix + name, tensor) for name, tensor in it)
