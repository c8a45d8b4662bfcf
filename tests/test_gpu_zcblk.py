"""GPU parity of experts made resident from the engine's storage formats:
ZCBLK01 expert blocks (wh_store_expert_block) and the consolidated experts
pack (wh_store_expert_pack), against the oracle and against the same
weights stored directly - bit-exact.  Also the raw -> resident FP4 relayout
that every FP4 store now runs on the device (k_fp4_relayout)."""
import json
from pathlib import Path

import numpy as np
import pytest

import wohper_amd
import zcblk
from parity_util import bits
from wohper_amd import model_format as mf
from wohper_amd import workloads as wl

pytestmark = pytest.mark.gpu

KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())


@pytest.fixture(autouse=True)
def exact_numerics(ctx):
    ctx.set_exact_numerics(True)
    yield


def _pairs(host):
    """(packed, scales, rows, cols, scale_cols) -> (packed 2-D, scales 2-D)."""
    p, s, rows, cols, scols = host
    return p.reshape(rows, cols // 2), s.reshape(rows, scols)


def _block(seed, layer, expert, **kw):
    host = wl.synth_expert_host(wohper_amd.load_library(), seed, layer, expert)
    return host, zcblk.expert_block(*[_pairs(m) for m in host], prefix=f"layers.{layer}.ffn.experts.{expert}", **kw)


def _oracle_routed(oracle, experts, weights, x):
    outs = np.stack([oracle.fp4_expert_forward(*m, x) for m in experts])
    return oracle.routed_combine(outs, weights)


def test_kat_block_forward(ctx, oracle):
    """The reference's bridge test through the store: [h, 2h]."""
    k = KATS["zcblk_fp4_expert"]
    ctx.store_expert_block(40, 0, zcblk.kat_block(k))
    x = np.array(k["input"], np.float32)
    got = ctx.fp4_expert_forward(40, 0, x, 2, 4)
    ex = wohper_amd.deepseek_v4_fp4_expert_from_quant_block(zcblk.kat_block(k))
    spec = lambda m: (m.packed_weight, m.ue8m0_scales, m.rows, m.cols, m.scale_cols)
    want = oracle.fp4_expert_forward(spec(ex.w1), spec(ex.w3), spec(ex.w2), x)
    assert np.array_equal(bits(got), bits(want))
    h = oracle.act_quant([np.float32(2.0) / (1 + np.exp(np.float32(-2.0))) * np.float32(3.0)], 64)[0]
    assert abs(got[0] - h) < k["tol"] and abs(got[1] - 2 * h) < k["tol"]


@pytest.mark.parametrize("shapes_last,order", [(False, (0, 1, 2)), (True, (2, 1, 0))])
def test_model_shape_blocks_bit_exact(ctx, oracle, shapes_last, order):
    """Six experts of the model's shapes stored from blocks route exactly as
    the same bytes stored directly and as the oracle."""
    seed, layer = 31, 41
    idx, w, x = wl.moe_token_case(seed)
    hosts = []
    for e in idx:
        host, block = _block(seed, layer, int(e), shapes_last=shapes_last, order=order)
        ctx.store_expert_block(layer, int(e), block)
        hosts.append(host)
    got = ctx.routed_experts([(layer, int(e), float(wt)) for e, wt in zip(idx, w)], x)
    assert np.array_equal(bits(got), bits(_oracle_routed(oracle, hosts, w, x)))


def test_block_and_direct_store_agree(ctx):
    """A block and wh_store_fp4 of the same bytes route identically."""
    seed, layer, e = 33, 43, 5
    host, block = _block(seed, layer, e)
    ctx.store_expert_block(layer, e, block)
    hs = [ctx.store_fp4(p, s, r, c, sc) for p, s, r, c, sc in host]
    ctx.store_expert(layer + 1, e, *hs)
    x = np.random.default_rng(seed).standard_normal(wl.HIDDEN).astype(np.float32)
    a = ctx.routed_experts([(layer, e, 1.0)], x)
    b = ctx.routed_experts([(layer + 1, e, 1.0)], x)
    assert np.array_equal(bits(a), bits(b))


def test_bad_block_keeps_the_resident_expert(ctx, oracle):
    seed, layer, e = 35, 44, 9
    host, block = _block(seed, layer, e)
    ctx.store_expert_block(layer, e, block)
    x = np.random.default_rng(seed).standard_normal(wl.HIDDEN).astype(np.float32)
    before = ctx.routed_experts([(layer, e, 1.0)], x)
    bad = bytearray(block)
    bad[8] = 2  # version
    with pytest.raises(wohper_amd.DeepSeekV4KernelError) as err:
        ctx.store_expert_block(layer, e, bytes(bad))
    assert err.value.name == "UnsupportedQuantBlockVersion"
    assert err.value.detail == "unsupported ZCBLK version: 2"
    with pytest.raises(wohper_amd.DeepSeekV4KernelError) as err:
        ctx.store_expert_block(layer, e, block[:-1])  # the last shape blob is cut
    assert err.value.name == "TruncatedQuantBlock"
    assert np.array_equal(bits(ctx.routed_experts([(layer, e, 1.0)], x)), bits(before))
    # replacing the expert with another block releases the tensors it owned
    _, before_tensors, _ = ctx.usage()
    host2, block2 = _block(seed + 1, layer, e)
    ctx.store_expert_block(layer, e, block2)
    _, after_tensors, _ = ctx.usage()
    assert after_tensors == before_tensors
    want = oracle.fp4_expert_forward(*host2, x)
    assert np.array_equal(bits(ctx.routed_experts([(layer, e, 1.0)], x)), bits(want))


def test_expert_pack_load_bit_exact(ctx, oracle, tmp_path):
    seed = 37
    keys = [(45, 3), (45, 200), (46, 3), (46, 17)]
    blocks, hosts = {}, {}
    for layer, e in keys:
        hosts[(layer, e)], blocks[(layer, e)] = _block(seed, layer, e)
    model = zcblk.write_pack(tmp_path, "dense_core", blocks)
    info = mf.load_optional_expert_pack(model)
    assert ctx.store_expert_pack(info, keys=[(46, 3), (45, 200)]) == 2
    assert ctx.store_expert_pack(info) == 4
    x = np.random.default_rng(seed).standard_normal(wl.HIDDEN).astype(np.float32)
    for layer in (45, 46):
        es = [e for l, e in keys if l == layer]
        wts = [0.6, 0.4]
        got = ctx.routed_experts([(layer, e, wt) for e, wt in zip(es, wts)], x)
        want = _oracle_routed(oracle, [hosts[(layer, e)] for e in es], wts, x)
        assert np.array_equal(bits(got), bits(want)), layer


def test_expert_pack_errors(ctx, tmp_path):
    seed = 39
    _, block = _block(seed, 47, 1)
    model = zcblk.write_pack(tmp_path, "m", {(47, 1): block, (47, 2): block})
    info = mf.load_optional_expert_pack(model)
    e = info.entries[(47, 2)]

    def load(entries):
        with pytest.raises(wohper_amd.DeepSeekV4KernelError) as err:
            ctx.store_expert_pack(mf.ExpertPackInfo(info.file, entries))
        return err.value

    # the index checks run before any read
    v = load({(47, 1): info.entries[(47, 1)], (47, 2): mf.ExpertPackEntry(e.offset + 4096, e.disk_bytes,
                                                                           e.payload_bytes)})
    assert v.name == "Unaligned" and v.detail.startswith("unaligned field expert_pack.offset: value=")
    v = load({(47, 2): mf.ExpertPackEntry(e.offset, e.disk_bytes, e.disk_bytes + 1)})
    assert v.name == "InvalidArgument"
    # a block past the end of the file
    v = load({(47, 3): mf.ExpertPackEntry(e.offset + e.disk_bytes, e.disk_bytes, e.payload_bytes)})
    assert v.name == "Io" and "unexpected end of file" in v.detail
    # a corrupt block names its (layer, expert)
    bad = tmp_path / "bad.bin"
    raw = bytearray(info.file.read_bytes())
    raw[e.offset:e.offset + 8] = b"XXXXXXXX"
    bad.write_bytes(bytes(raw))
    with pytest.raises(wohper_amd.DeepSeekV4KernelError) as err:
        ctx.store_expert_pack(mf.ExpertPackInfo(bad, dict(info.entries)))
    assert err.value.name == "InvalidQuantBlockMagic" and err.value.detail.startswith("layer 47 expert 2: invalid ZCBLK magic")
    missing = mf.ExpertPackInfo(tmp_path / "nope.bin", dict(info.entries))
    with pytest.raises(wohper_amd.DeepSeekV4KernelError) as err:
        ctx.store_expert_pack(missing)
    assert err.value.name == "Io"


def test_relayout_across_upload_pieces(ctx, oracle):
    """A 160 MB FP4 tensor goes up in 64 MB pieces; rows of the last piece
    match the same rows stored on their own, and both match the oracle."""
    rows, cols = 40960, 8192
    rng = np.random.default_rng(5)
    packed = rng.integers(0, 256, (rows, cols // 2), dtype=np.uint8)
    scales = rng.integers(118, 128, (rows, cols // 32), dtype=np.uint8)
    big = ctx.store_fp4(packed, scales, rows, cols, cols // 32)
    tail = 512
    small = ctx.store_fp4(packed[-tail:], scales[-tail:], tail, cols, cols // 32)
    x = rng.standard_normal(cols).astype(np.float32)
    y_big = ctx.fp4_matvec(big, x, rows)
    y_small = ctx.fp4_matvec(small, x, tail)
    assert np.array_equal(bits(y_big[-tail:]), bits(y_small))
    want = oracle.fp4_matvec(packed[-tail:], scales[-tail:], tail, cols, cols // 32, x)
    assert np.array_equal(bits(y_small), bits(want))
    piece = (64 << 20) // (cols // 2)  # rows per upload piece
    for r0 in (0, piece - 1, piece, 2 * piece + 3):
        want = oracle.fp4_matvec(packed[r0:r0 + 1], scales[r0:r0 + 1], 1, cols, cols // 32, x)
        assert np.array_equal(bits(y_big[r0:r0 + 1]), bits(want)), r0
    ctx.release(big)
    ctx.release(small)
