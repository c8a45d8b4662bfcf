"""Test-side writers of the engine's expert storage formats, to feed the
product's readers.

* ZCBLK01 blocks in the layout of the reference's block builders
  (build_synthetic_quant_block, engine/zc_infer_core/src/compute.rs:3272-3320,
  and its test twin make_multi_tensor_zcblk01_with_formats,
  compute.rs:9141-9195): header, records, names blob, then each tensor's data
  followed by its shape blob.  `shapes_last=True` gives the converter's order
  instead (tools/stream_convert_deepseek_v4.py:286-338: all data, then the
  shape blobs).
* Experts packs: 2 MiB-aligned blocks in one file plus the
  `<model>.experts_pack.index.json` index (tools/build_experts_pack.py).
"""
from __future__ import annotations

import json
import struct
from pathlib import Path

import numpy as np

MAGIC = b"ZCBLK01\0"
HEADER = struct.Struct("<8sIIIIQQ")          # 40 bytes
RECORD = struct.Struct("<HHIIQQQQff")        # 52 bytes
QUANT_FP4 = 2402
QUANT_UE8M0 = 2403
ROLE_GATE, ROLE_UP, ROLE_DOWN = 6, 7, 8
ALIGN = 2 * 1024 * 1024


def tensor(name, shape, data, quant_format, role=0, dtype_original=0, scale=1.0, zero_point=0.0):
    data = bytes(np.ascontiguousarray(data, dtype=np.uint8).reshape(-1)) if not isinstance(data, bytes) else data
    return {"name": name.encode() if isinstance(name, str) else name, "shape": [int(d) for d in shape],
            "data": data, "quant_format": quant_format, "role": role, "dtype_original": dtype_original,
            "scale": scale, "zero_point": zero_point}


def build_block(tensors, header_quant_format=4, shapes_last=False, version=1, magic=MAGIC) -> bytes:
    names = bytearray()
    name_offsets = []
    for t in tensors:
        name_offsets.append(len(names))
        names += struct.pack("<H", len(t["name"])) + t["name"]
    names_offset = HEADER.size + len(tensors) * RECORD.size
    cursor = names_offset + len(names)
    data_offsets, shape_offsets, tail = [], [], bytearray()
    shape_blob = lambda t: struct.pack("<I", len(t["shape"])) + b"".join(struct.pack("<Q", d) for d in t["shape"])
    if shapes_last:
        for t in tensors:
            data_offsets.append(cursor + len(tail))
            tail += t["data"]
        for t in tensors:
            shape_offsets.append(cursor + len(tail))
            tail += shape_blob(t)
    else:
        for t in tensors:
            data_offsets.append(cursor + len(tail))
            tail += t["data"]
            shape_offsets.append(cursor + len(tail))
            tail += shape_blob(t)
    out = bytearray(HEADER.pack(magic, version, len(tensors), header_quant_format, 0, HEADER.size, names_offset))
    for i, t in enumerate(tensors):
        out += RECORD.pack(t["dtype_original"], t["quant_format"], len(t["shape"]), t["role"], name_offsets[i],
                           shape_offsets[i], data_offsets[i], len(t["data"]), t["scale"], t["zero_point"])
    return bytes(out + names + tail)


def kat_block(kat) -> bytes:
    """A block of the golden known-answer entries (tensors as JSON)."""
    ts = [tensor(t["name"], t["shape"], t["data"], t["quant_format"], t["role"], t["dtype_original"], t["scale"],
                 t["zero_point"]) for t in kat["tensors"]]
    return build_block(ts, kat["header_quant_format"])


def expert_block(w1, w3, w2, prefix="layers.0.ffn.experts.0", order=(0, 1, 2), shapes_last=False,
                 extra=()) -> bytes:
    """An FP4 expert block from host (packed [rows, cols/2], scales [rows,
    cols/32]) pairs for w1 (gate), w3 (up), w2 (down)."""
    mats = {"w1": (w1, ROLE_GATE), "w3": (w3, ROLE_UP), "w2": (w2, ROLE_DOWN)}
    keys = ["w1", "w3", "w2"]
    ts = []
    for i in order:
        k = keys[i]
        (packed, scales), role = mats[k]
        ts.append(tensor(f"{prefix}.{k}.weight", packed.shape, packed, QUANT_FP4, role, 12))
        ts.append(tensor(f"{prefix}.{k}.scale", scales.shape, scales, QUANT_UE8M0, role, 1))
    ts.extend(extra)
    return build_block(ts, 2400, shapes_last)


def write_pack(directory, model_name, blocks, fmt="wohper-experts-pack"):
    """blocks: {(layer_id, expert_id): bytes}.  Writes <model_name>.experts_pack.bin
    (each block at a 2 MiB-aligned offset, disk_bytes rounded up to 2 MiB) and
    <model_name>.experts_pack.index.json; returns the model path."""
    directory = Path(directory)
    pack = directory / f"{model_name}.experts_pack.bin"
    entries, offset = [], 0
    with pack.open("wb") as f:
        for (layer_id, expert_id), block in blocks.items():
            disk = (len(block) + ALIGN - 1) // ALIGN * ALIGN
            f.seek(offset)
            f.write(block)
            entries.append({"layer_id": layer_id, "expert_id": expert_id, "offset": offset, "disk_bytes": disk,
                            "payload_bytes": len(block)})
            offset += disk
        f.truncate(offset)
    index = {"format": fmt, "pack_file": pack.name, "entries": entries}
    (directory / f"{model_name}.experts_pack.index.json").write_text(json.dumps(index))
    return directory / f"{model_name}.zcinf"
