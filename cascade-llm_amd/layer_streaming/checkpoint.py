"""Safetensors checkpoint -> packed host arena, read straight into place.

The reference loads each tensor through the safetensors library into a
temporary tensor and copies it into the arena (layer_streaming/
weight_store.py:20-38, :109-171).  Here the checkpoint is described first and
read second:

1. ``describe_checkpoint(path)`` resolves the shard files (a directory with
   ``model.safetensors.index.json`` and its ``weight_map``, a directory with
   ``model.safetensors``, or one ``.safetensors`` file) and parses each
   shard's header itself: an 8-byte little-endian length, then a JSON object
   of ``name -> {dtype, shape, data_offsets}`` whose offsets are relative to
   the end of the header (the published safetensors format).
2. ``load_into(store, path)`` checks the plan against that description
   before any data moves -- every non-alias tensor present, shapes equal,
   dtypes readable, byte ranges the right size and inside the file -- then
   reads every tensor with positional reads (``os.preadv``) from a few
   threads.  bf16 tensors land directly in their arena bytes (no temporary);
   f16 / f32 ones are read in pieces and rounded to bf16 into place.

Errors keep the reference's types: FileNotFoundError (no checkpoint),
KeyError (tensors missing), ValueError (shape, dtype, malformed file).
"""

from concurrent.futures import ThreadPoolExecutor
from dataclasses import dataclass
import json
import os
from pathlib import Path
import struct

import torch

__all__ = ["TensorRecord", "describe_checkpoint", "load_into"]

INDEX_NAME = "model.safetensors.index.json"
SINGLE_NAME = "model.safetensors"

# safetensors dtype tag -> (torch dtype, bytes per element)
_DTYPES = {
    "BF16": (torch.bfloat16, 2),
    "F16": (torch.float16, 2),
    "F32": (torch.float32, 4),
}
_CONVERT_PIECE_BYTES = 64 << 20


@dataclass(frozen=True)
class TensorRecord:
    """Where one tensor's bytes sit in a shard file."""

    path: Path
    dtype: str
    shape: tuple
    begin: int  # absolute file offset of the first byte
    end: int    # absolute file offset past the last byte


def _read_header(path):
    size = path.stat().st_size
    with path.open("rb") as handle:
        prefix = handle.read(8)
        if len(prefix) != 8:
            raise ValueError("{}: shorter than a safetensors header".format(path))
        (length,) = struct.unpack("<Q", prefix)
        if length > size - 8:
            raise ValueError("{}: header length {} runs past the file".format(
                path, length))
        try:
            header = json.loads(handle.read(length).decode("utf-8"))
        except (UnicodeDecodeError, json.JSONDecodeError) as error:
            raise ValueError("{}: malformed safetensors header".format(path)) from error
    if not isinstance(header, dict):
        raise ValueError("{}: malformed safetensors header".format(path))
    base = 8 + length
    records = {}
    for name, entry in header.items():
        if name == "__metadata__":
            continue
        try:
            begin, end = (int(v) for v in entry["data_offsets"])
            dtype = str(entry["dtype"])
            shape = tuple(int(d) for d in entry["shape"])
        except (KeyError, TypeError, ValueError) as error:
            raise ValueError("{}: malformed entry for {}".format(path, name)) from error
        if not 0 <= begin <= end or base + end > size:
            raise ValueError("{}: byte range of {} lies outside the file".format(
                path, name))
        records[name] = TensorRecord(path, dtype, shape, base + begin, base + end)
    return records


def _shard_files(checkpoint):
    """(shard files, index key -> file or None) of a checkpoint path."""

    root = Path(checkpoint)
    if root.is_file():
        return [root], None
    index = root / INDEX_NAME
    if index.is_file():
        with index.open("r", encoding="utf-8") as handle:
            weight_map = json.load(handle).get("weight_map")
        if not isinstance(weight_map, dict):
            raise ValueError("{}: weight_map missing or not an object".format(index))
        mapping = {key: root / name for key, name in weight_map.items()}
        return sorted(set(mapping.values())), mapping
    single = root / SINGLE_NAME
    if single.is_file():
        return [single], None
    raise FileNotFoundError(
        "no safetensors checkpoint at {}: expected {}, {} or a .safetensors "
        "file".format(root, SINGLE_NAME, INDEX_NAME))


def describe_checkpoint(checkpoint):
    """name -> TensorRecord over every shard of ``checkpoint``."""

    files, mapping = _shard_files(checkpoint)
    records = {}
    for path in files:
        for name, record in _read_header(path).items():
            # an index names the shard that owns each tensor
            if mapping is None or mapping.get(name) == path:
                records[name] = record
    return records


def _plan_reads(store, records):
    """Validate the checkpoint against the plan; (record, arena view) pairs."""

    plan = store.plan
    required = store.required_keys()
    missing = [key for key in required if key not in records]
    if missing:
        raise KeyError("checkpoint lacks {} tensor(s) the plan needs, e.g. "
                       "{}".format(len(missing), ", ".join(missing[:8])))
    reads = []
    for key in required:
        record = records[key]
        spec = plan.tensors[key]
        if record.shape != tuple(spec.shape):
            raise ValueError("{}: checkpoint shape {} does not match the plan's "
                             "{}".format(key, record.shape, tuple(spec.shape)))
        if record.dtype not in _DTYPES:
            raise ValueError("{}: checkpoint dtype {} cannot be read (BF16, F16 or "
                             "F32)".format(key, record.dtype))
        width = _DTYPES[record.dtype][1]
        if record.end - record.begin != spec.numel * width:
            raise ValueError("{}: {} bytes stored for {} {} elements".format(
                key, record.end - record.begin, spec.numel, record.dtype))
        reads.append((record, store.tensor(key)))
    return reads


def _pread_into(fd, buffer, offset):
    view = memoryview(buffer).cast("B")
    done = 0
    while done < len(view):
        got = os.preadv(fd, [view[done:]], offset + done)
        if got <= 0:
            raise ValueError("unexpected end of checkpoint data at byte {}".format(
                offset + done))
        done += got


def _read_one(record, target):
    fd = os.open(record.path, os.O_RDONLY)
    try:
        flat = target.reshape(-1)
        if record.dtype == "BF16":
            _pread_into(fd, flat.view(torch.uint8).numpy(), record.begin)
            return
        dtype, width = _DTYPES[record.dtype]
        step = max(1, _CONVERT_PIECE_BYTES // width)
        piece = torch.empty(min(step, flat.numel()), dtype=dtype)
        for first in range(0, flat.numel(), step):
            count = min(step, flat.numel() - first)
            part = piece[:count]
            _pread_into(fd, part.view(torch.uint8).numpy(), record.begin + first * width)
            flat[first:first + count].copy_(part)
    finally:
        os.close(fd)


def load_into(store, checkpoint, threads=None):
    """Fill ``store``'s allocated arena from ``checkpoint``; every check runs
    before the first byte is read."""

    reads = _plan_reads(store, describe_checkpoint(checkpoint))
    # largest first, so the threads finish together
    reads.sort(key=lambda item: item[0].begin - item[0].end)
    workers = threads or min(8, len(os.sched_getaffinity(0)))
    with ThreadPoolExecutor(max_workers=max(1, workers),
                            thread_name_prefix="checkpoint-read") as pool:
        for result in [pool.submit(_read_one, record, target)
                       for record, target in reads]:
            result.result()
    return len(reads)
