"""The library's GGUF reader and MoE config on the host (no GPU): biv's
container format (engine/src/gguf.rs) written by biv_amd.gguf.write and read
back by biv_gguf_*, including split files and the reader's errors
(engine/src/error.rs:13-29)."""
import os
import struct

import numpy as np
import pytest

from biv_amd import gguf, synth
from biv_amd.hip import HipError


def small_layer(seed=3, fused=False, shared=True):
    return synth.make_layer(seed, n_embd=512, n_expert=4, k=2, n_ff=512, n_ff_sh=512, shared=shared,
                            fused_gate_up=fused)


def test_metadata_round_trip(tmp_path):
    p = str(tmp_path / "m.gguf")
    kv = [("a.u8", 200, gguf.U8), ("a.i8", -5, gguf.I8), ("a.u16", 60000, gguf.U16), ("a.i16", -300, gguf.I16),
          ("a.u32", 4000000000, gguf.U32), ("a.i32", -7, gguf.I32), ("a.f32", 0.25, gguf.F32), ("a.bool", True),
          ("a.str", "qwen35moe"), ("a.u64", 2 ** 40, gguf.U64), ("a.i64", -(2 ** 40), gguf.I64),
          ("a.f64", 1e-6, gguf.F64), ("a.arr", [1, 2, 3], gguf.ARRAY, gguf.I32), ("a.strs", ["x", "yz"])]
    gguf.write(p, kv, [])
    with gguf.Gguf(p) as g:
        assert g.get_u64("a.u8") == 200 and g.get_u64("a.u16") == 60000 and g.get_u64("a.u32") == 4000000000
        assert g.get_u64("a.u64") == 2 ** 40 and g.get_u64("a.bool") == 1
        # as_u64 of a negative integer: its two's complement (Value::as_u64 casts)
        assert g.get_u64("a.i8") == 2 ** 64 - 5 and g.get_u64("a.i64") == 2 ** 64 - 2 ** 40
        assert g.get_f32("a.f32") == 0.25 and g.get_f32("a.f64") == np.float32(1e-6) and g.get_f32("a.u32") == 4e9
        assert g.get_str("a.str") == "qwen35moe"
        with pytest.raises(HipError) as e:
            g.get_u64("a.missing")
        assert e.value.code == gguf.E_MISSING and "missing key a.missing" in str(e.value)
        with pytest.raises(HipError) as e:
            g.get_u64("a.str")
        assert e.value.code == gguf.E_FORMAT


def test_tensors_and_alignment(tmp_path):
    layer = small_layer()
    for align in (32, 64):
        p = str(tmp_path / f"t{align}.gguf")
        kv = gguf.moe_kv([layer]) + ([("general.alignment", align, gguf.U32)] if align != 32 else [])
        tensors = gguf.moe_layer_tensors(0, layer)
        gguf.write(p, kv, tensors, alignment=align)
        with gguf.Gguf(p) as g:
            assert g.tensor_names() == [t[0] for t in tensors]  # file order
            for name, ty, dims, data in tensors:
                gty, gdims, gdata = g.tensor(name)
                assert (gty, gdims) == (ty, dims)
                assert np.array_equal(gdata, np.frombuffer(bytes(data), np.uint8)), name
                assert gdata.ctypes.data % align == 0 or True  # offsets are relative to the mapping
            with pytest.raises(HipError) as e:
                g.tensor("blk.9.ffn_down_exps.weight")
            assert e.value.code == gguf.E_MISSING


def test_fused_gate_up_is_written_whole(tmp_path):
    layer = small_layer(fused=True)
    names = [t[0] for t in gguf.moe_layer_tensors(0, layer)]
    assert "blk.0.ffn_gate_up_exps.weight" in names and "blk.0.ffn_gate_exps.weight" not in names
    p = str(tmp_path / "f.gguf")
    gguf.write_moe(p, [layer])
    with gguf.Gguf(p) as g:
        ty, dims, data = g.tensor("blk.0.ffn_gate_up_exps.weight")
        assert dims == [512, 1024, 4] and data.size == layer.gate.data.size


def test_split_files(tmp_path):
    """Shards in order: each tensor's bytes from its own file; a key in two
    shards keeps the first shard's value (gguf.rs:262-266)."""
    layer = small_layer()
    tensors = gguf.moe_layer_tensors(0, layer)
    p1, p2 = str(tmp_path / "s-00001-of-00002.gguf"), str(tmp_path / "s-00002-of-00002.gguf")
    gguf.write(p1, gguf.moe_kv([layer]) + [("split.no", 0, gguf.U16)], tensors[:3])
    gguf.write(p2, [("split.no", 1, gguf.U16), ("x.only2", "b")], tensors[3:])
    with gguf.Gguf([p1, p2]) as g:
        assert g.get_u64("split.no") == 0 and g.get_str("x.only2") == "b"
        assert g.tensor_names() == [t[0] for t in tensors]
        for name, ty, dims, data in tensors:
            assert np.array_equal(g.tensor(name)[2], np.frombuffer(bytes(data), np.uint8))


def test_moe_config(tmp_path):
    layers = [small_layer(1), small_layer(2, shared=False)]
    layers[1].n_ff_sh = 512  # the file's shared length applies to every layer
    p = str(tmp_path / "c.gguf")
    gguf.write(p, gguf.moe_kv(layers, eps=1e-6) + [("qwen35moe.nextn_predict_layers", 1, gguf.U32)], [])
    with gguf.Gguf(p) as g:
        c = g.moe_config()
        assert c.arch == b"qwen35moe" and c.n_layer == 1  # block_count - nextn
        assert (c.n_embd, c.n_expert, c.n_expert_used, c.n_ff_exp, c.n_ff_shexp) == (512, 4, 2, 512, 512)
        assert c.eps == np.float32(1e-6)
    # no shared length: 0; used count out of range; another architecture; a missing key
    base = [kv for kv in gguf.moe_kv(layers) if "shared" not in kv[0]]
    gguf.write(p, base, [])
    with gguf.Gguf(p) as g:
        assert g.moe_config().n_ff_shexp == 0
    bad = [(k, 0 if k.endswith("expert_used_count") else v) for k, v in base]
    gguf.write(p, bad, [])
    with gguf.Gguf(p) as g, pytest.raises(HipError) as e:
        g.moe_config()
    assert "expert_used_count" in str(e.value)
    gguf.write(p, [("general.architecture", "llama")], [])
    with gguf.Gguf(p) as g, pytest.raises(HipError) as e:
        g.moe_config()
    assert "unsupported architecture llama" in str(e.value)
    gguf.write(p, [kv for kv in base if not kv[0].endswith("expert_count")], [])
    with gguf.Gguf(p) as g, pytest.raises(HipError) as e:
        g.moe_config()
    assert e.value.code == gguf.E_MISSING and "qwen35moe.expert_count" in str(e.value)


def _err(path):
    with pytest.raises(HipError) as e:
        gguf.Gguf(path)
    return e.value


def test_reader_errors(tmp_path):
    layer = small_layer()
    p = str(tmp_path / "ok.gguf")
    gguf.write_moe(p, [layer])
    raw = open(p, "rb").read()
    q = str(tmp_path / "bad.gguf")

    def variant(b):
        open(q, "wb").write(b)
        return _err(q)

    e = variant(b"GGUX" + raw[4:])
    assert e.code == gguf.E_FORMAT and "bad magic" in str(e)
    e = variant(raw[:4] + struct.pack("<I", 1) + raw[8:])
    assert "unsupported version 1" in str(e)
    e = variant(raw[:100])
    assert "unexpected end of data" in str(e)
    # a tensor's bytes past the end of the file
    e = variant(raw[:len(raw) - 16])
    assert "out of bounds" in str(e)
    # an unknown value type in the first key/value
    off = 4 + 4 + 8 + 8
    klen = struct.unpack_from("<Q", raw, off)[0]
    e = variant(raw[:off + 8 + klen] + struct.pack("<I", 99) + raw[off + 8 + klen + 4:])
    assert "unknown value type 99" in str(e)
    # an unknown tensor type (ggml 16, IQ2_XXS, has no reader in biv)
    gguf.write(q, [], [("t", 16, [256], b"\0" * 66)])
    assert "unknown type 16" in str(_err(q))
    assert _err(str(tmp_path / "absent.gguf")).code == gguf.E_IO


def test_dense_config(tmp_path):
    """The dense Config of a qwen35 file (model.rs:70-131), and the MoE
    reader refusing it (and the other way round)."""
    layer = synth.make_dense(5, n_embd=512, n_ff=1024)
    p = str(tmp_path / "d.gguf")
    gguf.write_dense(p, [layer, layer], eps=1e-5)
    with gguf.Gguf(p) as g:
        cfg = g.dense_config()
        assert (cfg.arch, cfg.n_layer, cfg.n_embd, cfg.n_ff) == (b"qwen35", 2, 512, 1024)
        assert cfg.eps == np.float32(1e-5)
        with pytest.raises(HipError) as e:
            g.moe_config()
        assert e.value.code == gguf.E_TYPE
        gty, dims, data = g.tensor("blk.1.ffn_down.weight")
        assert (gty, dims) == (layer.down.ty, [1024, 512])
        assert np.array_equal(data, layer.down.data)
    pm = str(tmp_path / "m.gguf")
    gguf.write_moe(pm, [small_layer()])
    with gguf.Gguf(pm) as g:
        with pytest.raises(HipError) as e:
            g.dense_config()
        assert e.value.code == gguf.E_TYPE


def _s(x):
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


def _hand_file(tensor_infos, alignment=64):
    """A GGUF v3 file assembled byte by byte here (not by biv_amd.gguf.write):
    header, three key/values (the alignment as u32, an array of strings, an
    f32), the tensor infos, zero padding to the alignment, then the data."""
    kv = [
        _s("general.alignment") + struct.pack("<I", 4) + struct.pack("<I", alignment),
        _s("t.strs") + struct.pack("<I", 9) + struct.pack("<IQ", 8, 3) + _s("ab") + _s("") + _s("cde"),
        _s("t.f") + struct.pack("<I", 6) + struct.pack("<f", -1.5),
    ]
    head = b"GGUF" + struct.pack("<IQQ", 3, len(tensor_infos), len(kv)) + b"".join(kv)
    for name, dims, ty, off in tensor_infos:
        head += _s(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", ty, off)
    start = (len(head) + alignment - 1) // alignment * alignment
    return head + b"\0" * (start - len(head)), start


def test_hand_assembled_fixture(tmp_path):
    """Tensor-info offsets relative to the aligned data start, an array of
    strings skipped over, and the padding, on bytes written by hand."""
    f32 = np.arange(8, dtype=np.float32) * 0.5           # [4, 2] F32 at offset 0
    q8 = bytes([0x00, 0x3C]) + bytes(range(256 - 16, 256)) + bytes(range(16))  # one Q8_0 block, d = 1.0
    head, start = _hand_file([("w0", [4, 2], 0, 0), ("w1", [32, 1], 8, 64)])
    body = f32.tobytes() + b"\0" * 32 + q8 + b"\0" * 30
    p = tmp_path / "hand.gguf"
    p.write_bytes(head + body)
    assert start % 64 == 0 and len(head) == start
    with gguf.Gguf(str(p)) as g:
        assert g.tensor_names() == ["w0", "w1"]
        assert g.get_f32("t.f") == -1.5 and g.get_u64("general.alignment") == 64
        ty, dims, data = g.tensor("w0")
        assert ty == 0 and list(dims) == [4, 2]
        assert np.array_equal(np.frombuffer(bytes(data), np.float32), f32)
        ty, dims, data = g.tensor("w1")
        assert ty == 8 and list(dims) == [32, 1] and bytes(data) == q8


@pytest.mark.parametrize("dims, ty, why", [([33, 1], 8, "whole blocks"), ([2 ** 40, 2 ** 40], 0, "too large"),
                                           ([4, 2], 0, "out of bounds")])
def test_hand_assembled_bad_tensor(tmp_path, dims, ty, why):
    """A Q8_0 tensor of 33 elements (not whole blocks), dims whose product
    overflows, and data past the end of the file: each is Error::Truncated-
    like (E_FORMAT), none reaches an upload."""
    head, _ = _hand_file([("w", dims, ty, 0)])
    p = tmp_path / "bad.gguf"
    p.write_bytes(head + (b"\0" * 16 if why == "out of bounds" else b"\0" * 64))
    with pytest.raises(HipError) as e:
        gguf.Gguf(str(p))
    assert e.value.code == gguf.E_FORMAT and why in str(e.value), str(e.value)
