"""The GGUF reader (gx_gguf_*, golem's tensors/gguf.go + gguf_meta.go) and the
Qwen3 binding on top of it (qwen/config.go LoadConfig, qwen/weights.go
LoadWeights), on files written by tests/gguf_writer.py.  Host code only: no
GPU is needed.

golem's own GGUF tests read a real checkpoint named by GOLEM_MODEL and skip
without one (tensors/gguf_test.go:9-21); none exists here, so these files are
synthetic, built field by field from the format, and each refusal golem's
reader makes (tensors/gguf.go:177-301) is provoked once.
"""
import struct

import numpy as np
import pytest

from golem_amd import capi, gguf, synth
from tests import gguf_writer as gw


def test_metadata_types_and_accessors(tmp_path):
    meta = [("u8", gw.U8, 200), ("i8", gw.I8, -3), ("u16", gw.U16, 65000), ("i16", gw.I16, -30000),
            ("u32", gw.U32, 4000000000), ("i32", gw.I32, -5), ("f32", gw.F32, 1.5), ("b", gw.BOOL, True),
            ("s", gw.STRING, "qwen3"), ("u64", gw.U64, 2 ** 40 + 7), ("i64", gw.I64, -(2 ** 40)),
            ("f64", gw.F64, 0.1), ("arr", gw.ARRAY, (gw.U16, [1, 2, 3])),
            ("bools", gw.ARRAY, (gw.BOOL, [True, False, True])), ("strs", gw.ARRAY, (gw.STRING, ["<bos>", "", "é"])),
            ("nested", gw.ARRAY, (gw.ARRAY, [(gw.U8, [1]), (gw.U8, [2, 3])])), ("u8", gw.U8, 9)]
    path = gw.write(tmp_path / "m.gguf", meta, [])
    with gguf.GGUF(path) as g:
        # a repeated key keeps its last value; the keys keep file order
        assert g.keys() == [k for k, _, _ in meta[:-1]]
        assert g.uint32("u8") == 9
        # Uint32 widens any integer as Go converts it (tensors/gguf_meta.go:56-77)
        assert g.uint32("i8") == (-3) & 0xFFFFFFFF
        assert g.uint32("u16") == 65000 and g.uint32("i16") == (-30000) & 0xFFFFFFFF
        assert g.uint32("u32") == 4000000000 and g.uint32("u64") == 7 and g.uint32("i64") == 0
        assert g.float32("f32") == np.float32(1.5)
        assert g.float32("f64") == np.float32(0.1)  # float64 narrowed
        assert g.bool("b") is True and g.string("s") == "qwen3"
        assert g.uint32_slice("arr") == [1, 2, 3] and g.uint32_slice("u32") == [4000000000]  # scalar as one
        assert g.bool_slice("bools") == [True, False, True] and g.bool_slice("b") == [True]
        assert g.strings("strs") == ["<bos>", "", "é"]
        for call, key, msg in ((g.uint32, "f32", 'metadata "f32" is float32, not an integer'),
                               (g.string, "u8", 'metadata "u8" is uint8, not a string'),
                               (g.float32, "s", 'metadata "s" is string, not a float'),
                               (g.bool, "i8", 'metadata "i8" is int8, not a bool'),
                               (g.strings, "s", 'metadata "s" is string, not an array'),
                               (g.strings, "arr", 'metadata "arr" holds a uint16, not a string'),
                               (g.uint32_slice, "strs", 'metadata "strs" is string, not an integer'),
                               (g.uint32, "missing", 'metadata "missing" is absent')):
            with pytest.raises(capi.GxError) as e:
                call(key)
            assert e.value.message == msg


def test_tensor_table_views_and_alignment(tmp_path):
    g0 = synth.rng(11)
    q4 = synth.q4_0_weights(g0, 3, 64)
    q6 = synth.q6_k_weights(g0, 2, 256)
    f = g0.standard_normal(5).astype(np.float32)
    f16 = np.arange(6, dtype=np.float16)
    tensors = [("a.q4", 2, [64, 3], q4.tobytes()), ("b.q6", 14, [256, 2], q6.tobytes()),
               ("c.f32", 0, [5], f.tobytes()), ("d.f16", 1, [3, 2], f16.tobytes()),
               ("e.4d", 0, [1, 1, 2, 2], np.ones(4, np.float32).tobytes())]
    for alignment, meta in ((32, []), (64, [("general.alignment", gw.U32, 64)]),
                            (32, [("general.alignment", gw.STRING, "x")])):  # not an integer: the default
        path = gw.write(tmp_path / f"t{alignment}.gguf", meta, tensors, alignment=alignment)
        with gguf.GGUF(path) as g:
            assert list(g.tensors) == [t[0] for t in tensors]
            a = g.get("a.q4")
            assert (a.dtype, a.shape, a.nbytes) == ("Q4_0", [64, 3], 3 * 2 * 18)
            np.testing.assert_array_equal(a.raw, q4)
            assert a.ptr % alignment == 0
            b = g.get("b.q6")
            assert (b.dtype, b.shape, b.nbytes) == ("Q6_K", [256, 2], 2 * 210)
            np.testing.assert_array_equal(b.raw, q6)
            np.testing.assert_array_equal(g.get("c.f32").floats(), f)
            assert g.get("d.f16").nbytes == 12 and g.get("e.4d").shape == [1, 1, 2, 2]
            with pytest.raises(capi.GxError, match='tensor "no.such.tensor" is absent'):
                g.get("no.such.tensor")
            with pytest.raises(capi.GxError, match='tensor "d.f16" is F16, not F32'):
                g.get("d.f16").floats()


def _refusal(tmp_path, data, name="bad.gguf"):
    path = tmp_path / name
    path.write_bytes(data)
    with pytest.raises(capi.GxError) as e:
        gguf.GGUF(path)
    assert e.value.code == capi.GX_ERR_INVALID
    assert e.value.message.startswith(str(path) + ": ") or "empty" in e.value.message
    return e.value.message[len(str(path)) + 2:]


def test_refusals(tmp_path):
    good = gw.gguf_bytes([("k", gw.U32, 1)], [("w", 2, [32, 2], bytes(36))])
    with pytest.raises(capi.GxError, match="is empty"):
        (tmp_path / "empty.gguf").write_bytes(b"")
        gguf.GGUF(tmp_path / "empty.gguf")
    assert _refusal(tmp_path, b"GGML" + good[4:]) == "not a GGUF file"
    assert _refusal(tmp_path, b"GG") == "not a GGUF file"
    assert _refusal(tmp_path, b"GGUF") == "GGUF version 0, only 2 and 3 are read"
    assert _refusal(tmp_path, gw.gguf_bytes([], [], version=1)) == "GGUF version 1, only 2 and 3 are read"
    assert _refusal(tmp_path, good[:20]) == "truncated at byte 16"
    # the metadata value cut short
    cut = len(struct.pack("<IIQQ", 0, 0, 0, 0)) + 8 + 1 + 4 + 2
    assert _refusal(tmp_path, good[:cut]) == 'metadata 0 ("k"): truncated at byte 37'
    bad_type = struct.pack("<IIQQ", 0x46554747, 3, 0, 1) + struct.pack("<Q", 1) + b"k" + struct.pack("<I", 13)
    assert _refusal(tmp_path, bad_type) == 'metadata 0 ("k"): unknown metadata type 13 at byte 37'
    huge = struct.pack("<IIQQ", 0x46554747, 3, 0, 1) + struct.pack("<Q", 1) + b"k" + struct.pack("<IQ", 8, 10 ** 9)
    assert _refusal(tmp_path, huge) == 'metadata 0 ("k"): string of 1000000000 bytes at 45'
    arr = struct.pack("<IIQQ", 0x46554747, 3, 0, 1) + struct.pack("<Q", 1) + b"k" + struct.pack("<IIQ", 9, 0, 10 ** 9)
    assert _refusal(tmp_path, arr) == 'metadata 0 ("k"): array of 1000000000 values at 49'
    for dims in (0, 5):
        data = gw.gguf_bytes([], [("w", 0, [4] * max(dims, 1), bytes(16))])
        hdr = 24 + 8 + 1
        data = data[:hdr] + struct.pack("<I", dims) + data[hdr + 4:]
        assert _refusal(tmp_path, data) == f'tensor "w" has {dims} dimensions'
    assert _refusal(tmp_path, gw.gguf_bytes([], [("w", 3, [32, 1], bytes(20))])) == \
        'tensor "w": unsupported ggml type 3'
    assert _refusal(tmp_path, gw.gguf_bytes([], [("w", 2, [48, 1], bytes(36))])) == \
        'tensor "w": a row of 48 does not divide into blocks of 32 (Q4_0)'
    assert _refusal(tmp_path, gw.gguf_bytes([], [("w", 14, [128, 1], bytes(210))])) == \
        'tensor "w": a row of 128 does not divide into blocks of 256 (Q6_K)'
    assert _refusal(tmp_path, gw.gguf_bytes([("general.alignment", gw.U32, 48)], [], alignment=32)) == \
        "alignment 48 is not a power of two"
    assert _refusal(tmp_path, gw.gguf_bytes([("general.alignment", gw.U32, 0)], [], alignment=32)) == \
        "alignment 0 is not a power of two"
    short = gw.gguf_bytes([], [("w", 2, [32, 2], bytes(36))])[:-10]
    msg = _refusal(tmp_path, short)
    assert msg.startswith('tensor "w" runs from ') and msg.endswith(", past the end of the file")
    far = gw.gguf_bytes([], [("w", 0, [1], bytes(4))], offsets=[2 ** 63])
    assert "past the end of the file" in _refusal(tmp_path, far)
    # a truncated tensor record
    t = gw.gguf_bytes([], [("w", 0, [1], bytes(4))])
    assert _refusal(tmp_path, t[:24 + 8 + 1 + 4 + 3]) == 'tensor "w": truncated at byte 37'


def _tiny_cfg(**kw):
    return synth.QwenConfig(256, 512, 2, 4, 2, 64, 1024, 32, **kw)


def test_qwen_binding_matches_the_weights(tmp_path):
    cfg = _tiny_cfg()
    w = synth.qwen_weights(cfg, 21)
    path = gw.qwen_file(tmp_path / "q.gguf", cfg, w)
    g, got_cfg, got = gguf.load_qwen(path, 32)
    try:
        # eps and the RoPE base are float32 in the file, as in golem's Config
        want = dict(vars(cfg), eps=float(np.float32(cfg.eps)), rope_base=float(np.float32(cfg.rope_base)))
        assert vars(got_cfg) == want
        assert got["token_embd_quant"] == capi.Q6_K
        np.testing.assert_array_equal(got["token_embd"], w["token_embd"])
        np.testing.assert_array_equal(got["output_norm"], w["output_norm"])
        for a, b in zip(got["blocks"], w["blocks"]):
            assert set(a) == set(b)
            for k in b:
                np.testing.assert_array_equal(np.asarray(a[k]).view(np.uint8), np.asarray(b[k]).view(np.uint8))
    finally:
        g.close()


def test_qwen_binding_refusals(tmp_path):
    cfg = _tiny_cfg()
    w = synth.qwen_weights(cfg, 22)

    def refused(name, **kw):
        path = gw.qwen_file(tmp_path / name, cfg, w, **kw)
        with pytest.raises(capi.GxError) as e:
            gguf.load_qwen(path, 32)
        return e.value.message

    assert refused("arch.gguf", extra_meta=[("general.architecture", gw.STRING, "gemma4")]) == \
        'architecture "gemma4" is not qwen3'
    assert refused("heads.gguf", extra_meta=[("qwen3.attention.head_count_kv", gw.U32, 3)]) == \
        "block 0: 4 query heads do not divide into 3 key-value heads"
    assert refused("vlen.gguf", extra_meta=[("qwen3.attention.value_length", gw.U32, 32)]) == \
        "keys are 64 wide and values 32, which this engine does not do"
    assert refused("nok.gguf", drop=("blk.1.attn_k.weight",)) == 'tensor "blk.1.attn_k.weight" is absent'
    qd = cfg.heads * cfg.head_dim
    assert refused("shape.gguf", replace={"blk.0.attn_q.weight": (2, [cfg.dim, qd - 32],
                                                                  bytes((qd - 32) * cfg.dim // 32 * 18))}) == \
        f"blk.0.attn_q.weight is {qd - 32} by {cfg.dim}, not {qd} by {cfg.dim}"
    assert refused("norm.gguf", replace={"blk.0.attn_q_norm.weight": (0, [32], bytes(128))}) == \
        "blk.0.attn_q_norm.weight is 32 wide, not 64"
    assert refused("f16norm.gguf", replace={"output_norm.weight": (1, [cfg.dim], bytes(2 * cfg.dim))}) == \
        'tensor "output_norm.weight" is F16, not F32'
    assert refused("q8.gguf", replace={"blk.0.ffn_up.weight": (8, [cfg.dim, cfg.ffn],
                                                               bytes(cfg.ffn * cfg.dim // 32 * 34))}) == \
        'tensor "blk.0.ffn_up.weight" is Q8_0, which is not a weight format'


def test_qwen_binding_refuses_an_own_head(tmp_path):
    cfg = _tiny_cfg()
    w = synth.qwen_weights(cfg, 23)
    base = gw.qwen_file(tmp_path / "base.gguf", cfg, w)
    with gguf.GGUF(base) as g:
        tensors = [(t.name, t.ggml_type, t.shape, t.raw.tobytes()) for t in g.tensors.values()]
        meta = [("general.architecture", gw.STRING, "qwen3"), ("qwen3.block_count", gw.U32, cfg.layers),
                ("qwen3.embedding_length", gw.U32, cfg.dim),
                ("qwen3.attention.layer_norm_rms_epsilon", gw.F32, cfg.eps),
                ("qwen3.attention.head_count", gw.U32, cfg.heads),
                ("qwen3.attention.head_count_kv", gw.ARRAY, (gw.U32, [cfg.kv_heads] * cfg.layers)),
                ("qwen3.feed_forward_length", gw.U32, cfg.ffn), ("qwen3.attention.key_length", gw.U32, cfg.head_dim),
                ("qwen3.rope.freq_base", gw.F32, cfg.rope_base)]
    # per-block arrays read like scalars (perBlock, qwen/config.go:50-55)
    ok = gw.write(tmp_path / "arrays.gguf", meta, tensors)
    g, got_cfg, _ = gguf.load_qwen(ok, 32)
    g.close()
    assert got_cfg.kv_heads == cfg.kv_heads
    own = gw.write(tmp_path / "own.gguf", meta, tensors + [("output.weight", 14, [cfg.dim, cfg.vocab],
                                                            bytes(cfg.vocab * cfg.dim // 256 * 210))])
    with pytest.raises(capi.GxError) as e:
        gguf.load_qwen(own, 32)
    assert e.value.message == "this checkpoint has an output.weight; the engine assumes a tied head"
