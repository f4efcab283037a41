"""Writes GGUF files for the tests (the format as tensors/gguf.go reads it:
version 3 header, typed metadata, tensor table, data at the alignment).

Metadata values are (type, value) pairs with GGUF's type numbers; an array is
(ARRAY, (element type, [values])).  Tensors are (name, ggml type, shape with
the row length first, bytes).  `corrupt` hooks let a test damage one field.
"""
import struct

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?", U64: "<Q",
        I64: "<q", F64: "<d"}


def _string(s):
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _value(kind, v):
    if kind == STRING:
        return _string(v)
    if kind == ARRAY:
        elem, items = v
        return struct.pack("<IQ", elem, len(items)) + b"".join(_value(elem, x) for x in items)
    return struct.pack(_FMT[kind], v)


def gguf_bytes(meta, tensors, alignment=32, version=3, magic=0x46554747, offsets=None):
    """The file as bytes.  meta: list of (key, type, value); tensors: list of
    (name, ggml_type, shape, data).  offsets overrides tensor offsets."""
    out = struct.pack("<IIQQ", magic, version, len(tensors), len(meta))
    for key, kind, v in meta:
        out += _string(key) + struct.pack("<I", kind) + _value(kind, v)
    pos, offs = 0, []
    for _, _, _, data in tensors:
        offs.append(pos)
        pos += (len(data) + alignment - 1) // alignment * alignment
    if offsets is not None:
        offs = offsets
    for (name, kind, shape, _), off in zip(tensors, offs):
        out += _string(name) + struct.pack("<I", len(shape)) + b"".join(struct.pack("<Q", d) for d in shape)
        out += struct.pack("<IQ", kind, off)
    out += b"\0" * ((-len(out)) % alignment)
    base = len(out)
    for (_, _, _, data), off in zip(tensors, offs):
        if off > 1 << 32:  # an offset meant to point past any file: no data placed
            continue
        if base + off > len(out):
            out += b"\0" * (base + off - len(out))
        out = out[:base + off] + bytes(data) + out[base + off + len(data):]
    return out


def write(path, meta, tensors, **kw):
    with open(path, "wb") as f:
        f.write(gguf_bytes(meta, tensors, **kw))
    return path


def qwen_file(path, cfg, weights, extra_meta=(), drop=(), replace=None):
    """A Qwen3 checkpoint of config `cfg` holding `weights` (synth.qwen_weights
    layout) under llama.cpp's names and keys (qwen/config.go, qwen/weights.go).
    drop: tensor names left out; replace: {name: (ggml_type, shape, data)}."""
    import numpy as np
    qd, kvd = cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
    head_type = 14 if weights.get("token_embd_quant", 3) == 3 else 2
    meta = [("general.architecture", STRING, "qwen3"),
            ("qwen3.block_count", U32, cfg.layers),
            ("qwen3.embedding_length", U32, cfg.dim),
            ("qwen3.attention.layer_norm_rms_epsilon", F32, cfg.eps),
            ("qwen3.attention.head_count", U32, cfg.heads),
            ("qwen3.attention.head_count_kv", U32, cfg.kv_heads),
            ("qwen3.feed_forward_length", U32, cfg.ffn),
            ("qwen3.attention.key_length", U32, cfg.head_dim),
            ("qwen3.attention.value_length", U32, cfg.head_dim),
            ("qwen3.rope.freq_base", F32, cfg.rope_base),
            ("qwen3.context_length", U32, 40960)] + list(extra_meta)
    t = [("token_embd.weight", head_type, [cfg.dim, cfg.vocab], weights["token_embd"]),
         ("output_norm.weight", 0, [cfg.dim], np.asarray(weights["output_norm"], np.float32).tobytes())]
    for i, b in enumerate(weights["blocks"]):
        p = f"blk.{i}."
        t += [(p + "attn_norm.weight", 0, [cfg.dim], b["attn_norm"].tobytes()),
              (p + "attn_q.weight", 2, [cfg.dim, qd], b["q"]),
              (p + "attn_k.weight", 2, [cfg.dim, kvd], b["k"]),
              (p + "attn_v.weight", 2, [cfg.dim, kvd], b["v"]),
              (p + "attn_output.weight", 2, [qd, cfg.dim], b["o"]),
              (p + "attn_q_norm.weight", 0, [cfg.head_dim], b["q_norm"].tobytes()),
              (p + "attn_k_norm.weight", 0, [cfg.head_dim], b["k_norm"].tobytes()),
              (p + "ffn_norm.weight", 0, [cfg.dim], b["ffn_norm"].tobytes()),
              (p + "ffn_gate.weight", 2, [cfg.dim, cfg.ffn], b["gate"]),
              (p + "ffn_up.weight", 2, [cfg.dim, cfg.ffn], b["up"]),
              (p + "ffn_down.weight", 2, [cfg.ffn, cfg.dim], b["down"])]
    t = [x for x in t if x[0] not in drop]
    if replace:
        t = [(n, *replace[n]) if n in replace else (n, k, s, d) for n, k, s, d in t]
    return write(path, meta, t)
