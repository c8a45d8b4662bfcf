"""CPU checks of the ZCBLK01 expert-block reader (host code of the C ABI:
wh_quant_block_header / _tensor / _fp4_expert) and of the experts-pack
index reader.

Pinned by the reference's own block tests (compute.rs:7552-7568 and
8599-8621, their blocks rebuilt byte for byte from the builders' layout), by
the error texts of ComputeError's Display (compute.rs:346-372) for every
check of parse_quant_block / QuantBlockLayout::tensor /
deepseek_fp4_matvec_from_tensors, in the reference's order, and by a
sanitizer run of the same parser over mutated blocks."""
import json
import shutil
import struct
import subprocess
from pathlib import Path

import numpy as np
import pytest

import wohper_amd
import zcblk
from wohper_amd import model_format as mf

ROOT = Path(__file__).resolve().parents[1]
KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())
U64 = (1 << 64) - 1


def _err(block, fn=wohper_amd.deepseek_v4_fp4_expert_from_quant_block):
    with pytest.raises(wohper_amd.DeepSeekV4KernelError) as e:
        fn(block)
    return e.value.name, e.value.detail


def _patch(block, off, fmt, value):
    b = bytearray(block)
    struct.pack_into(fmt, b, off, value)
    return bytes(b)


def _rec(i):
    return zcblk.HEADER.size + i * zcblk.RECORD.size


def _small_expert(rows=4, cols=64, seed=0):
    """Host (packed, scales) for w1, w3 [rows, cols] and w2 [cols, rows]."""
    rng = np.random.default_rng(seed)
    mk = lambda r, c: (rng.integers(0, 256, (r, c // 2), dtype=np.uint8),
                       rng.integers(110, 130, (r, max(1, c // 32)), dtype=np.uint8))
    return mk(rows, cols), mk(rows, cols), mk(cols, rows)


# ------------------------------------------------------------ known answers
def test_single_tensor_block_known_answer():
    k = KATS["zcblk_single_tensor"]
    block = zcblk.kat_block(k)
    assert len(block) == 40 + 52 + 2 + 21 + 4 + 4 + 8 * 2
    e = k["expect"]
    assert wohper_amd.quant_block_header(block) == (e["tensor_count"], e["quant_format"], 0)
    t = wohper_amd.quant_block_tensor(block, 0)
    assert t.quant_format == e["quant_format"] and t.name == e["name"].encode() and t.role == e["role"]
    assert t.rank == 2 and t.shape == tuple(e["shape"]) and list(t.data) == e["data"]
    assert abs(t.scale - e["scale"]) < 1e-5 and abs(t.zero_point - e["zero_point"]) < 1e-5
    assert _err(block, lambda b: wohper_amd.quant_block_tensor(b, 1)) == (
        "TensorIndexOutOfRange", "tensor index out of range: index=1, count=1")


def test_fp4_expert_block_known_answer(oracle):
    """The reference's bridge test: the expert read out of the block computes
    [h, 2h] for x = [2, 3], h = act_quant(silu(2) * 3)."""
    k = KATS["zcblk_fp4_expert"]
    ex = wohper_amd.deepseek_v4_fp4_expert_from_quant_block(zcblk.kat_block(k))
    dims = [(m.rows, m.cols, m.scale_cols) for m in (ex.w1, ex.w3, ex.w2)]
    assert dims == [(2, 2, 1)] * 3
    assert [list(m.packed_weight) for m in (ex.w1, ex.w3, ex.w2)] == [[2, 0], [32, 0], [2, 4]]
    assert all(list(m.ue8m0_scales) == [127, 127] for m in (ex.w1, ex.w3, ex.w2))
    spec = lambda m: (m.packed_weight, m.ue8m0_scales, m.rows, m.cols, m.scale_cols)
    out = oracle.fp4_expert_forward(spec(ex.w1), spec(ex.w3), spec(ex.w2), np.array(k["input"], np.float32))
    h = oracle.act_quant([np.float32(2.0) / (1 + np.exp(np.float32(-2.0))) * np.float32(3.0)], 64)[0]
    assert abs(out[0] - h) < k["tol"] and abs(out[1] - 2 * h) < k["tol"]


@pytest.mark.parametrize("shapes_last", [False, True])
@pytest.mark.parametrize("order", [(0, 1, 2), (2, 0, 1)])
def test_expert_views_any_layout(shapes_last, order):
    """Tensors are found by suffix wherever the writer put them, next to
    unrelated tensors of other formats."""
    w1, w3, w2 = _small_expert(4, 64)
    extra = [zcblk.tensor("layers.0.ffn.gate.weight", (8, 64), np.arange(512) % 251, 2401, 9, 12),
             zcblk.tensor("layers.0.attn_norm.weight", (64,), np.zeros(128, np.uint8), 2404, 10, 5)]
    block = zcblk.expert_block(w1, w3, w2, order=order, shapes_last=shapes_last, extra=extra)
    assert wohper_amd.quant_block_header(block) == (8, 2400, 0)
    ex = wohper_amd.deepseek_v4_fp4_expert_from_quant_block(block)
    for m, (packed, scales) in zip((ex.w1, ex.w3, ex.w2), (w1, w3, w2)):
        assert (m.rows, m.cols, m.scale_cols) == (packed.shape[0], 2 * packed.shape[1], scales.shape[1])
        assert np.array_equal(m.packed_weight, packed.reshape(-1))
        assert np.array_equal(m.ue8m0_scales, scales.reshape(-1))


def test_expert_views_take_the_required_prefix_of_longer_data():
    """data_bytes beyond rows * packed_cols is ignored (E/compute.rs:1240-1246)."""
    w1, w3, w2 = _small_expert(4, 64)
    ts = []
    for k, (p, s) in (("w1", w1), ("w3", w3), ("w2", w2)):
        ts.append(zcblk.tensor(f"e.{k}.weight", p.shape, np.concatenate([p.reshape(-1), [7, 7, 7]]), 2402))
        ts.append(zcblk.tensor(f"e.{k}.scale", s.shape, np.concatenate([s.reshape(-1), [9]]), 2403))
    ex = wohper_amd.deepseek_v4_fp4_expert_from_quant_block(zcblk.build_block(ts))
    assert ex.w1.packed_weight.size == w1[0].size and ex.w2.ue8m0_scales.size == w2[1].size


# ------------------------------------------------------------------ errors
def _good():
    w1, w3, w2 = _small_expert(4, 64)
    return zcblk.expert_block(w1, w3, w2)


def test_header_errors():
    good = _good()
    assert _err(good[:39]) == ("TruncatedQuantBlock", "truncated ZCBLK field: block header")
    assert _err(b"") == ("TruncatedQuantBlock", "truncated ZCBLK field: block header")
    bad = b"ZCBLK02\0" + good[8:]
    assert _err(bad) == ("InvalidQuantBlockMagic", "invalid ZCBLK magic: [90, 67, 66, 76, 75, 48, 50, 0]")
    assert _err(_patch(good, 8, "<I", 2)) == ("UnsupportedQuantBlockVersion", "unsupported ZCBLK version: 2")
    assert _err(_patch(good, 12, "<I", 10 ** 6)) == ("TruncatedQuantBlock", "truncated ZCBLK field: record table")
    assert _err(_patch(good, 24, "<Q", 39)) == ("TruncatedQuantBlock", "truncated ZCBLK field: record table")
    assert _err(_patch(good, 24, "<Q", U64 - 10)) == ("InvalidQuantBlock", "invalid ZCBLK: record table range overflow")
    assert _err(_patch(good, 32, "<Q", len(good) + 1)) == ("TruncatedQuantBlock", "truncated ZCBLK field: names blob")
    # names_offset == len is allowed by the header check; the first name read fails
    assert _err(_patch(good, 32, "<Q", len(good))) == ("TruncatedQuantBlock", "truncated ZCBLK field: name.len")


def test_record_errors():
    good = _good()
    r0 = _rec(0)
    cases = [
        ((r0 + 12, "<Q", U64 - 1), ("InvalidQuantBlock", "invalid ZCBLK: name offset overflow")),
        ((r0 + 12, "<Q", len(good)), ("TruncatedQuantBlock", "truncated ZCBLK field: name.len")),
        ((r0 + 4, "<I", 3), ("InvalidQuantBlock", "invalid ZCBLK: shape rank mismatch")),
        ((r0 + 20, "<Q", len(good) - 2), ("TruncatedQuantBlock", "truncated ZCBLK field: shape.rank")),
        ((r0 + 20, "<Q", U64 - 1), ("InvalidQuantBlock", "invalid ZCBLK: read range overflow")),
        ((r0 + 28, "<Q", len(good)), ("TruncatedQuantBlock", "truncated ZCBLK field: tensor data")),
        ((r0 + 36, "<Q", U64), ("InvalidQuantBlock", "invalid ZCBLK: tensor data range overflow")),
        ((r0 + 36, "<Q", len(good)), ("TruncatedQuantBlock", "truncated ZCBLK field: tensor data")),
    ]
    for (off, fmt, v), want in cases:
        assert _err(_patch(good, off, fmt, v)) == want, (off, v)
    # a name running past the end of the block
    names_offset = struct.unpack_from("<Q", good, 32)[0]
    assert _err(_patch(good, names_offset, "<H", 0xFFFF)) == ("TruncatedQuantBlock", "truncated ZCBLK field: name blob")
    # a shape blob whose dims run past the end: point tensor 0's shape at the last 12 bytes, rank 2
    b = _patch(good, r0 + 20, "<Q", len(good) - 12)
    b = _patch(b, len(good) - 12, "<I", 2)
    assert _err(b) == ("TruncatedQuantBlock", "truncated ZCBLK field: shape blob")


def _expert_ts(w1, w3, w2, **over):
    ts = {}
    for k, (p, s) in (("w1", w1), ("w3", w3), ("w2", w2)):
        ts[f"{k}.weight"] = zcblk.tensor(f"e.{k}.weight", p.shape, p, 2402, 0, 12)
        ts[f"{k}.scale"] = zcblk.tensor(f"e.{k}.scale", s.shape, s, 2403, 0, 1)
    ts.update(over)
    return [t for t in ts.values() if t is not None]


def test_expert_errors_in_reference_order():
    w1, w3, w2 = _small_expert(4, 64)
    inv = lambda s: ("InvalidQuantBlock", "invalid ZCBLK: " + s)
    shp = lambda s: ("InvalidShape", "invalid compute shape: " + s)
    trunc = lambda s: ("TruncatedQuantBlock", "truncated ZCBLK field: " + s)
    T = zcblk.tensor
    cases = [
        ({"w3.scale": None}, inv("missing DeepSeek expert tensor suffix")),
        ({"x": T("f.w1.weight", w1[0].shape, w1[0], 2402)}, inv("duplicate DeepSeek expert tensor suffix")),
        ({"w1.weight": T("e.w1.weight", w1[0].shape, w1[0], 2401)}, inv("DeepSeek expert weight is not FP4 E2M1 packed")),
        ({"w2.scale": T("e.w2.scale", w2[1].shape, w2[1], 2404)}, inv("DeepSeek expert scale is not UE8M0")),
        ({"w1.weight": T("e.w1.weight", (4, 32, 1), w1[0], 2402)}, shp("DeepSeek FP4 expert rank")),
        ({"w3.scale": T("e.w3.scale", (8,), w3[1], 2403)}, shp("DeepSeek FP4 expert rank")),
        ({"w1.weight": T("e.w1.weight", (0, 32), w1[0], 2402)}, shp("DeepSeek FP4 expert shape")),
        ({"w1.weight": T("e.w1.weight", (4, 0), w1[0], 2402)}, shp("DeepSeek FP4 expert shape")),
        ({"w1.scale": T("e.w1.scale", (4, 0), w1[1], 2403)}, shp("DeepSeek FP4 expert shape")),
        ({"w1.scale": T("e.w1.scale", (5, 2), w1[1], 2403)}, shp("DeepSeek FP4 expert shape")),
        ({"w1.weight": T("e.w1.weight", (4, 1 << 63), w1[0], 2402)}, shp("DeepSeek FP4 expert cols overflow")),
        ({"w1.weight": T("e.w1.weight", (1 << 33, 1 << 31), w1[0], 2402),
          "w1.scale": T("e.w1.scale", (1 << 33, 1), w1[1], 2403)}, shp("DeepSeek FP4 expert weight overflow")),
        ({"w2.weight": T("e.w2.weight", w2[0].shape, w2[0][:-1], 2402)}, trunc("DeepSeek FP4 expert weight")),
        ({"w2.scale": T("e.w2.scale", w2[1].shape, w2[1][:-1], 2403)}, trunc("DeepSeek FP4 expert scale")),
        ({"w3.weight": T("e.w3.weight", (4, 16), w3[0][:, :16], 2402),
          "w3.scale": T("e.w3.scale", (4, 1), w3[1][:, :1], 2403)}, shp("DeepSeek FP4 expert projection")),
        ({"w2.weight": T("e.w2.weight", (64, 4), np.zeros((64, 4), np.uint8), 2402),
          "w2.scale": T("e.w2.scale", (64, 1), np.zeros((64, 1), np.uint8), 2403)}, shp("DeepSeek FP4 expert projection")),
    ]
    for over, want in cases:
        assert _err(zcblk.build_block(_expert_ts(w1, w3, w2, **over))) == want, want
    # order: w1's format error is reported although w3 is missing ...
    both = _expert_ts(w1, w3, w2, **{"w1.weight": T("e.w1.weight", w1[0].shape, w1[0], 2401), "w3.scale": None})
    assert _err(zcblk.build_block(both)) == inv("DeepSeek expert weight is not FP4 E2M1 packed")
    # ... but every record is resolved while w1.weight is searched for
    blk = zcblk.build_block(both)
    last = _rec(len(both) - 1)
    assert _err(_patch(blk, last + 36, "<Q", len(blk))) == trunc("tensor data")


def test_empty_block_has_no_expert():
    assert _err(zcblk.build_block([])) == ("InvalidQuantBlock", "invalid ZCBLK: missing DeepSeek expert tensor suffix")
    assert wohper_amd.quant_block_header(zcblk.build_block([])) == (0, 4, 0)


def test_mutated_blocks_stay_in_bounds():
    """Random byte flips and truncations: every call returns a status, and an
    accepted block's views lie inside it."""
    w1, w3, w2 = _small_expert(4, 64)
    good = zcblk.expert_block(w1, w3, w2)
    rng = np.random.default_rng(7)
    statuses = set()
    for it in range(3000):
        b = bytearray(good)
        if it % 3 == 0:
            b = b[:rng.integers(0, len(good))]
        else:
            for _ in range(rng.integers(1, 4)):
                i = int(rng.integers(0, min(len(b), 40 + 6 * 52 + 120)))  # header, records, names
                b[i] = int(rng.integers(0, 256))
        try:
            ex = wohper_amd.deepseek_v4_fp4_expert_from_quant_block(bytes(b))
            statuses.add("ok")
            for m in (ex.w1, ex.w3, ex.w2):
                assert m.packed_weight.size == m.rows * m.cols // 2 and m.ue8m0_scales.size == m.rows * m.scale_cols
        except wohper_amd.DeepSeekV4KernelError as e:
            statuses.add(e.name)
    assert {"ok", "TruncatedQuantBlock", "InvalidQuantBlock"} <= statuses


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_parser_under_address_sanitizer(tmp_path):
    """The same header, built for the host with ASan/UBSan, over the mutated
    blocks of a small driver (tests/quant_block_asan.cpp)."""
    w1, w3, w2 = _small_expert(4, 64)
    seed = tmp_path / "seed.bin"
    seed.write_bytes(zcblk.expert_block(w1, w3, w2))
    exe = tmp_path / "qb_asan"
    subprocess.run(["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
                    "-I", str(ROOT / "wohper_amd" / "csrc"), str(ROOT / "tests" / "quant_block_asan.cpp"),
                    "-o", str(exe)], check=True)
    res = subprocess.run([str(exe), str(seed), "20000"], capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stderr[-2000:]
    assert "accepted" in res.stdout


# ---------------------------------------------------------- experts pack
def test_expert_pack_index_reader(tmp_path):
    assert mf.load_optional_expert_pack(tmp_path / "m.zcinf") is None
    model = zcblk.write_pack(tmp_path, "m", {(3, 1): b"a" * 10, (3, 2): b"b" * (3 << 20), (4, 1): b"c"})
    assert mf.expert_pack_index_path(model) == tmp_path / "m.experts_pack.index.json"
    info = mf.load_optional_expert_pack(model)
    assert info.file == tmp_path / "m.experts_pack.bin"
    assert info.entries[(3, 2)] == mf.ExpertPackEntry(2 << 20, 4 << 20, 3 << 20)
    assert info.entries[(4, 1)].offset == 6 << 20 and len(info.entries) == 3


def _index(tmp_path, **over):
    model = zcblk.write_pack(tmp_path, "m", {(0, 0): b"x" * 100, (0, 1): b"y" * 100})
    p = tmp_path / "m.experts_pack.index.json"
    d = json.loads(p.read_text())
    for k, v in over.items():
        if v is None:
            d.pop(k, None)
        else:
            d[k] = v
    p.write_text(json.dumps(d))
    return model


def test_expert_pack_index_errors(tmp_path):
    def err(model):
        with pytest.raises(mf.ModelFormatError) as e:
            mf.load_optional_expert_pack(model)
        return e.value.kind, str(e.value)

    kind, text = err(_index(tmp_path, format="other"))
    assert kind == "ShardMap" and text.startswith("unsupported experts pack format in ") and text.endswith(": other")
    assert err(_index(tmp_path, format=None))[0] == "ShardMap"  # serde default "" is not a known format
    assert mf.load_optional_expert_pack(_index(tmp_path, format="zeroclaw-experts-pack")) is not None
    kind, text = err(_index(tmp_path, pack_file="gone.bin"))
    assert kind == "ShardMap" and text == f"experts pack file missing: {tmp_path / 'gone.bin'}"
    e0 = {"layer_id": 0, "expert_id": 0, "offset": 0, "disk_bytes": 2 << 20, "payload_bytes": 5}
    assert err(_index(tmp_path, entries=[dict(e0, offset=4096)])) == (
        "Unaligned", "unaligned field expert_pack.offset: value=4096, required=2097152")
    assert err(_index(tmp_path, entries=[dict(e0, disk_bytes=100)])) == (
        "Unaligned", "unaligned field expert_pack.disk_bytes: value=100, required=2097152")
    assert err(_index(tmp_path, entries=[{k: v for k, v in e0.items() if k != "payload_bytes"}]))[0] == "ShardMap"
    assert err(_index(tmp_path, entries=[dict(e0, layer_id=-1)]))[0] == "ShardMap"
    info = mf.load_optional_expert_pack(_index(tmp_path, entries=[e0, dict(e0, offset=2 << 20)]))
    assert info.entries[(0, 0)].offset == 2 << 20  # a later duplicate replaces the earlier one
    assert mf.load_optional_expert_pack(_index(tmp_path, entries=None)).entries == {}


def test_package_block_builder_matches_the_test_writer():
    """model_format.build_synthetic_quant_block (the product's builder) lays
    out bytes exactly as the test writer does for the reference's layout."""
    w1, w3, w2 = _small_expert(4, 64)
    ts = [zcblk.tensor("e.w1.weight", w1[0].shape, w1[0], 2402, 6, 12),
          zcblk.tensor("e.w1.scale", w1[1].shape, w1[1], 2403, 6, 1, 0.5, 0.25)]
    want = zcblk.build_block(ts, 4)
    got = mf.build_synthetic_quant_block([mf.SyntheticTensor(t["name"].decode(), t["role"], t["shape"], t["data"],
                                                             t["dtype_original"], t["quant_format"], t["scale"],
                                                             t["zero_point"]) for t in ts])
    assert got == want
