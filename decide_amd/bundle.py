"""Model bundle IO for the device engine (internal/bundle/bundle.go,
internal/safetensors/safetensors.go).

A bundle is a directory with model.safetensors, config.json, tokenizer.json
and decide.json. Weights may be stored as F32, BF16, F16 or F64 (the
reference's reader widens F16/BF16/F64 to float32, safetensors.go:86-140).
BF16 entries go to the device as bf16 bits (``dn_upload_tensor_bf16``): in
bf16 mode the projection matrices are used exactly as stored, with no
float32 round trip.
"""
from __future__ import annotations

import json
import os
import struct
from typing import Callable, Dict, Optional, Sequence, Tuple

import numpy as np

from . import nn
from .local import Calibration, Local

FORMAT_VERSION = 1  # bundle.FormatVersion (bundle.go:22)

_DTYPES = {"F32": np.dtype("<f4"), "BF16": np.dtype("<u2"), "F16": np.dtype("<f2"), "F64": np.dtype("<f8")}


def read_safetensors(path: str) -> Tuple[Dict[str, Tuple[str, tuple, np.ndarray]], Dict[str, str]]:
    """Open (safetensors.go:45-84): {name: (dtype, shape, raw values)} and the
    metadata. Raw values are a read-only memory map in the stored dtype (BF16
    as uint16 bit patterns)."""
    with open(path, "rb") as fh:
        head = fh.read(8)
        if len(head) != 8:
            raise ValueError("safetensors: short file")
        (hlen,) = struct.unpack("<Q", head)
        if hlen > 1 << 28:
            raise ValueError("safetensors: implausible header size")
        header = json.loads(fh.read(hlen))
    base = 8 + hlen
    meta = header.pop("__metadata__", {}) or {}
    mm = np.memmap(path, dtype=np.uint8, mode="r")
    out = {}
    for name, info in header.items():
        dt = info["dtype"]
        if dt not in _DTYPES:
            raise ValueError(f"safetensors: {name} has unsupported dtype {dt}")
        shape = tuple(int(d) for d in info["shape"])
        n = int(np.prod(shape, dtype=np.int64)) if shape else 1
        b, e = (int(x) for x in info["data_offsets"])
        if e - b != n * _DTYPES[dt].itemsize:
            raise ValueError(f"safetensors: {name} has {e - b} bytes for {n} values of {dt}")
        out[name] = (dt, shape, mm[base + b:base + e].view(_DTYPES[dt]))
    return out, meta


def to_float32(dtype: str, raw: np.ndarray) -> np.ndarray:
    """Float32 (safetensors.go:86-140): exact widening of BF16/F16, rounding of F64."""
    if dtype == "BF16":
        return (raw.astype(np.uint32) << 16).view(np.float32)
    return raw.astype(np.float32)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round float32 values to bfloat16 (nearest even), as uint16 bit patterns."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(np.asarray(x, np.float32))
    return np.where(nan, (u >> 16).astype(np.uint16) | 0x40, r)


def write_safetensors(path: str, tensors: Dict[str, np.ndarray], dtype: str = "F32",
                      metadata: Optional[Dict[str, str]] = None) -> None:
    """Write (safetensors.go:176-240) with names sorted and the header padded
    with spaces to 8 bytes; dtype "BF16" stores round-to-nearest-even bf16."""
    names = sorted(tensors)
    header, blobs, off = {}, [], 0
    if metadata:
        header["__metadata__"] = dict(metadata)
    for name in names:
        a = np.asarray(tensors[name], np.float32)
        raw = bf16_bits(a.reshape(-1)) if dtype == "BF16" else np.ascontiguousarray(a.reshape(-1), "<f4")
        header[name] = {"dtype": dtype, "shape": list(a.shape), "data_offsets": [off, off + raw.nbytes]}
        off += raw.nbytes
        blobs.append(raw)
    hb = json.dumps(header, separators=(",", ":")).encode()
    hb += b" " * ((8 - (8 + len(hb)) % 8) % 8)
    tmp = path + ".tmp"
    with open(tmp, "wb") as fh:
        fh.write(struct.pack("<Q", len(hb)))
        fh.write(hb)
        for raw in blobs:
            fh.write(raw.tobytes())
    os.replace(tmp, path)


def upload_weights(engine: "nn.Engine", path: str) -> None:
    """Model.LoadWeights (internal/nn/model.go:217-234) into a device engine."""
    tensors, _ = read_safetensors(path)
    for name, shape in nn.tensor_shapes(engine.cfg).items():
        if name not in tensors:
            raise KeyError(f"safetensors: tensor {name!r} not found")
        dt, got, raw = tensors[name]
        if int(np.prod(got, dtype=np.int64)) != int(np.prod(shape, dtype=np.int64)):
            raise ValueError(f"nn: {name} has shape {list(got)}, model expects {list(shape)}")
        if dt == "BF16":
            engine.upload_bf16(name, raw)
        else:
            engine.upload(name, to_float32(dt, raw))


def read_meta(bundle_dir: str) -> dict:
    """decide.json with the format check of bundle.Load (bundle.go:96-107)."""
    with open(os.path.join(bundle_dir, "decide.json")) as fh:
        meta = json.load(fh)
    if meta.get("format", 0) != FORMAT_VERSION:
        raise ValueError(f"bundle: {bundle_dir} has format {meta.get('format', 0)}, "
                         f"this build reads format {FORMAT_VERSION}")
    return meta


def bundle_encoder(tokenizer_json: str) -> Tuple[Callable[[str], Sequence[int]], int]:
    """Encode(text, addSpecial=True) and the [MASK] id of a bundle's
    tokenizer.json, through the library's host tokenizer (dn_tokenizer_*)."""
    from .tokenizer import Tokenizer

    tok = Tokenizer.load(tokenizer_json)
    return tok.encode, tok.mask_id


def load_bundle(bundle_dir: str, precision: str = "bf16", device: int = 0,
                encoder: Optional[Tuple[Callable[[str], Sequence[int]], int]] = None, certify: float = 0.0) -> Local:
    """bundle.Load (bundle.go:95-125) onto the device: a Local whose weights are
    resident and whose tokenizer is the bundle's tokenizer.json.
    ``encoder`` = (encode, mask_id) replaces that tokenizer; ``certify`` > 0
    turns on dn_set_certify with that margin (16-bit precisions)."""
    meta = read_meta(bundle_dir)
    cfg = nn.load_config(os.path.join(bundle_dir, "config.json"))
    engine = nn.Engine(cfg, precision=precision, device=device, certify=certify)
    upload_weights(engine, os.path.join(bundle_dir, "model.safetensors"))
    encode, mask_id = encoder if encoder is not None else bundle_encoder(os.path.join(bundle_dir, "tokenizer.json"))
    cal = meta.get("calibration") or {}
    return Local(engine, encode, mask_id, model_id=meta.get("model_id") or "decide-0.2.0",
                 independent_options=bool(meta.get("independent_options", False)),
                 calibration=Calibration(dict(cal.get("temperature") or {}), float(cal.get("default") or 0)))
