"""Host-side pieces of the engine's model format: the experts-pack index
reader that hands wh_store_expert_pack its entries, and the in-memory
ZCBLK01 block builder.

Mirrors load_optional_expert_pack (engine/zc_infer_core/src/model_format.rs:458-504):
`<model>.experts_pack.index.json` beside the model file (the model path with
its extension replaced), a JSON object {format, pack_file, entries: [{layer_id,
expert_id, offset, disk_bytes, payload_bytes}]}.  Missing `format`,
`pack_file` or `entries` read as empty (serde defaults); the format must be
"wohper-experts-pack" or the legacy "zeroclaw-experts-pack"; the pack file is
resolved against the index's directory and must exist; every offset and
disk_bytes must be a multiple of 2 MiB.  A later entry with the same
(layer_id, expert_id) replaces an earlier one.
"""
from __future__ import annotations

import json
import struct
from dataclasses import dataclass
from pathlib import Path
from typing import Dict, Optional, Sequence, Tuple

ALIGN_2MB = 2 * 1024 * 1024  # engine/zc_infer_core/src/lib.rs:10
PACK_FORMATS = ("wohper-experts-pack", "zeroclaw-experts-pack")


class ModelFormatError(RuntimeError):
    """ModelFormatError (model_format.rs:32-56): `kind` is the variant name
    ("ShardMap", "Unaligned", "Io")."""

    def __init__(self, kind: str, message: str):
        self.kind = kind
        super().__init__(message)


@dataclass(frozen=True)
class ExpertPackEntry:
    """model_format.rs:180-184"""
    offset: int
    disk_bytes: int
    payload_bytes: int


@dataclass
class ExpertPackInfo:
    """model_format.rs:187-190"""
    file: Path
    entries: Dict[Tuple[int, int], ExpertPackEntry]


def expert_pack_index_path(model_path) -> Path:
    """Path::with_extension("experts_pack.index.json")."""
    return Path(model_path).with_suffix(".experts_pack.index.json")


def _uint(entry: dict, key: str, bits: int) -> int:
    if key not in entry:
        raise ModelFormatError("ShardMap", f"missing field `{key}`")
    v = entry[key]
    if isinstance(v, bool) or not isinstance(v, int) or not 0 <= v < (1 << bits):
        raise ModelFormatError("ShardMap", f"invalid value for `{key}`: {v!r}, expected u{bits}")
    return v


def load_optional_expert_pack(model_path) -> Optional[ExpertPackInfo]:
    """None when the model has no experts pack; raises ModelFormatError on a
    malformed index, in the reference's order of checks."""
    index_path = expert_pack_index_path(model_path)
    if not index_path.exists():
        return None
    try:
        text = index_path.read_text(encoding="utf-8")
    except OSError as e:
        raise ModelFormatError("Io", str(e)) from e
    try:
        disk = json.loads(text)
    except json.JSONDecodeError as e:
        raise ModelFormatError("ShardMap", str(e)) from e
    if not isinstance(disk, dict):
        raise ModelFormatError("ShardMap", "invalid type: expected struct ExpertPackDisk")
    fmt = disk.get("format", "")
    pack_file = disk.get("pack_file", "")
    raw_entries = disk.get("entries", [])
    if not isinstance(fmt, str) or not isinstance(pack_file, str) or not isinstance(raw_entries, list):
        raise ModelFormatError("ShardMap", "invalid type in experts pack index")
    if fmt not in PACK_FORMATS:
        raise ModelFormatError("ShardMap", f"unsupported experts pack format in {index_path}: {fmt}")
    pack = index_path.parent / pack_file
    if not pack.exists():
        raise ModelFormatError("ShardMap", f"experts pack file missing: {pack}")
    parsed = []
    for entry in raw_entries:
        if not isinstance(entry, dict):
            raise ModelFormatError("ShardMap", "invalid type: expected struct ExpertPackEntryDisk")
        parsed.append((_uint(entry, "layer_id", 32), _uint(entry, "expert_id", 32), _uint(entry, "offset", 64),
                       _uint(entry, "disk_bytes", 64), _uint(entry, "payload_bytes", 64)))
    entries: Dict[Tuple[int, int], ExpertPackEntry] = {}
    for layer_id, expert_id, offset, disk_bytes, payload_bytes in parsed:
        for field, value in (("expert_pack.offset", offset), ("expert_pack.disk_bytes", disk_bytes)):
            if value % ALIGN_2MB:
                raise ModelFormatError("Unaligned",
                                       f"unaligned field {field}: value={value}, required={ALIGN_2MB}")
        entries[(layer_id, expert_id)] = ExpertPackEntry(offset, disk_bytes, payload_bytes)
    return ExpertPackInfo(pack, entries)


@dataclass
class SyntheticTensor:
    """SyntheticTensor (engine/zc_infer_core/src/compute.rs:3255-3264)."""
    name: str
    role_code: int
    shape: Sequence[int]
    data: bytes
    dtype_original: int
    quant_format: int
    scale: float = 1.0
    zero_point: float = 0.0


def build_synthetic_quant_block(tensors: Sequence[SyntheticTensor]) -> bytes:
    """A ZCBLK01 block in memory from loose tensors, laid out as
    build_synthetic_quant_block does (compute.rs:3272-3320): the 40-byte
    header (quant_format 4, flags 0), one 52-byte record per tensor, the
    names blob ({u16 len, bytes} each), then each tensor's data followed by
    its shape blob ({u32 rank, u64 dims})."""
    names = bytearray()
    name_offsets = []
    for t in tensors:
        raw = t.name.encode()
        name_offsets.append(len(names))
        names += struct.pack("<H", len(raw)) + raw
    names_offset = 40 + 52 * len(tensors)
    cursor = names_offset + len(names)
    body = bytearray()
    places = []
    for t in tensors:
        data_off = cursor + len(body)
        body += bytes(t.data)
        shape_off = cursor + len(body)
        body += struct.pack("<I", len(t.shape)) + b"".join(struct.pack("<Q", int(d)) for d in t.shape)
        places.append((data_off, shape_off))
    out = bytearray(struct.pack("<8sIIIIQQ", b"ZCBLK01\0", 1, len(tensors), 4, 0, 40, names_offset))
    for t, off, (data_off, shape_off) in zip(tensors, name_offsets, places):
        out += struct.pack("<HHIIQQQQff", t.dtype_original, t.quant_format, len(t.shape), t.role_code, off,
                           shape_off, data_off, len(t.data), t.scale, t.zero_point)
    return bytes(out + names + body)
