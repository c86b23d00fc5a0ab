"""Versioned binary index files: the on-disk form of the tables EngineI8, EngineS and SpaceX search.

The reference keeps its built index as torch.save dicts (throughput/cache.py:9-21), which unpickle on load.
This format stores only data and is read without executing anything from the file:

    bytes 0-7    magic b"FVSINDEX"
    bytes 8-11   format version (u32, little endian) = 1
    bytes 12-15  manifest length n (u32)
    bytes 16..   manifest: UTF-8 JSON {"format": 1, "tree": <tree>, "arrays": {key: {"dtype", "shape",
                 "offset", "nbytes", "crc32"}}}
    then         every array's bytes at a 4096-byte aligned offset (C order, little endian)

<tree> restates the nested objects the engines use (the index tables `s1`, the refinement `code`, int8
codes ...): dicts, lists and tuples are kept as such (a dict with keys other than plain strings as
{"__dict__": [[key, value], ...]}, a tuple as {"__tuple__": [...]}), numbers, strings, booleans and None
inline, and each array as {"__array__": key, "torch": bool, "gpu": bool, "pinned": bool} pointing into
"arrays". Arrays are memory-mapped on load and checked against their CRC-32.
"""
import json
import os
import struct
import zlib

import numpy as np
import torch

MAGIC = b"FVSINDEX"
VERSION = 1
ALIGN = 4096

_TORCH_TO_NP = {torch.float32: np.float32, torch.float16: np.float16, torch.float64: np.float64,
                torch.int8: np.int8, torch.uint8: np.uint8, torch.int16: np.int16, torch.int32: np.int32,
                torch.int64: np.int64, torch.bool: np.bool_}
_NP_NAMES = {np.dtype(v).name: v for v in _TORCH_TO_NP.values()}
_NP_TO_TORCH = {np.dtype(v).name: k for k, v in _TORCH_TO_NP.items()}


def _raw(a):
    """The bytes of a C-contiguous array as a flat uint8 view (empty arrays included)."""
    return a.reshape(-1).view(np.uint8)


class IndexFormatError(ValueError):
    """The file is not an index file of a version this build reads, or it is damaged."""


def _put(arrays, path, a):
    """Register an array under its path; two objects flattened to one path would overwrite each other."""
    if path in arrays:
        raise ValueError(f"{path}: two arrays map to the same key")
    arrays[path] = a


def _flatten(obj, arrays, path):
    if isinstance(obj, torch.Tensor):
        if obj.dtype not in _TORCH_TO_NP:
            raise TypeError(f"{path}: unsupported tensor dtype {obj.dtype}")
        _put(arrays, path, obj.detach().to("cpu").contiguous().numpy())
        return {"__array__": path, "torch": True, "gpu": obj.device.type == "cuda",
                "pinned": obj.device.type == "cpu" and obj.is_pinned()}
    if isinstance(obj, np.ndarray):
        if obj.dtype.name not in _NP_NAMES:
            raise TypeError(f"{path}: unsupported array dtype {obj.dtype}")
        _put(arrays, path, np.ascontiguousarray(obj))
        return {"__array__": path, "torch": False}
    if isinstance(obj, dict):
        for k in obj:
            if not (k is None or isinstance(k, (bool, int, float, str, np.integer, np.floating, np.bool_))):
                raise TypeError(f"{path}: dict keys must be scalars, not {type(k).__name__}")
            if isinstance(k, str) and "." in k:
                raise ValueError(f"{path}: dict key {k!r} contains '.', the path separator")
        if all(isinstance(k, str) and not k.startswith("__") for k in obj):
            return {k: _flatten(v, arrays, f"{path}.{k}") for k, v in obj.items()}
        # other keys (the per-bit-width tables use int keys) as a list of [key, value] pairs
        return {"__dict__": [[_flatten(k, arrays, path), _flatten(v, arrays, f"{path}.{i}")]
                             for i, (k, v) in enumerate(obj.items())]}
    if isinstance(obj, (list, tuple)):
        items = [_flatten(v, arrays, f"{path}.{i}") for i, v in enumerate(obj)]
        return {"__tuple__": items} if isinstance(obj, tuple) else items
    if isinstance(obj, (np.integer, np.floating, np.bool_)):
        return obj.item()
    if obj is None or isinstance(obj, (bool, int, float, str)):
        return obj
    raise TypeError(f"{path}: cannot store a {type(obj).__name__}")


def save(path, **objects):
    """Write the named objects (e.g. s1=..., code=..., Z=..., zs=..., Vr=...) to an index file."""
    arrays = {}
    tree = {name: _flatten(obj, arrays, name) for name, obj in objects.items()}
    entries, offset = {}, 0
    for key, a in arrays.items():
        entries[key] = {"dtype": a.dtype.name, "shape": list(a.shape), "offset": offset, "nbytes": int(a.nbytes),
                        "crc32": zlib.crc32(_raw(a)) & 0xFFFFFFFF}
        offset += (a.nbytes + ALIGN - 1) // ALIGN * ALIGN
    manifest = json.dumps({"format": VERSION, "tree": tree, "arrays": entries}).encode()
    head = MAGIC + struct.pack("<II", VERSION, len(manifest)) + manifest
    base = (len(head) + ALIGN - 1) // ALIGN * ALIGN
    tmp = path + ".tmp"
    with open(tmp, "wb") as f:
        f.write(head)
        f.write(b"\0" * (base - len(head)))
        for key, a in arrays.items():
            f.seek(base + entries[key]["offset"])
            f.write(_raw(a))
        f.truncate(base + offset)
    os.replace(tmp, path)
    return path


def _manifest(f, size):
    head = f.read(16)
    if len(head) < 16 or head[:8] != MAGIC:
        raise IndexFormatError("not an index file (bad magic)")
    version, n = struct.unpack("<II", head[8:16])
    if version != VERSION:
        raise IndexFormatError(f"index format version {version}; this build reads version {VERSION}")
    if 16 + n > size:
        raise IndexFormatError("truncated manifest")
    try:
        man = json.loads(f.read(n).decode())
    except (UnicodeDecodeError, json.JSONDecodeError) as e:
        raise IndexFormatError(f"damaged manifest: {e}") from None
    return man, (16 + n + ALIGN - 1) // ALIGN * ALIGN


def load(path, device=None, verify=True):
    """The objects saved in `path`, as a dict name -> object, placed where they were when saved: tensors
    saved from the GPU go to `device` (default: "cuda" when a GPU is present, else the CPU), tensors saved
    from pinned host memory come back pinned when a GPU is present, other CPU tensors and numpy arrays stay
    on the host. verify: check every array's CRC-32 before use."""
    if device is None:
        device = "cuda" if torch.cuda.is_available() else "cpu"
    size = os.path.getsize(path)
    with open(path, "rb") as f:
        man, base = _manifest(f, size)
    arrays = {}
    for key, e in man["arrays"].items():
        if e["dtype"] not in _NP_NAMES:
            raise IndexFormatError(f"{key}: unknown dtype {e['dtype']}")
        dt = np.dtype(_NP_NAMES[e["dtype"]])
        shape = tuple(e["shape"])
        nbytes = int(np.prod(shape, dtype=np.int64)) * dt.itemsize
        if nbytes != e["nbytes"] or base + e["offset"] + nbytes > size:
            raise IndexFormatError(f"{key}: truncated or inconsistent array")
        a = np.memmap(path, dtype=dt, mode="r", offset=base + e["offset"], shape=shape) if nbytes else \
            np.empty(shape, dt)
        if verify and (zlib.crc32(_raw(np.ascontiguousarray(a))) & 0xFFFFFFFF) != e["crc32"]:
            raise IndexFormatError(f"{key}: checksum mismatch")
        arrays[key] = a
    gpu_host = torch.cuda.is_available()

    def build(node):
        if isinstance(node, dict):
            if "__array__" in node:
                a = np.array(arrays[node["__array__"]])
                if not node["torch"]:
                    return a
                t = torch.from_numpy(a)
                if node["gpu"]:
                    return t.to(device)
                return t.pin_memory() if node["pinned"] and gpu_host else t
            if "__tuple__" in node:
                return tuple(build(v) for v in node["__tuple__"])
            if "__dict__" in node:
                return {build(k): build(v) for k, v in node["__dict__"]}
            return {k: build(v) for k, v in node.items()}
        if isinstance(node, list):
            return [build(v) for v in node]
        return node

    return {name: build(node) for name, node in man["tree"].items()}
