"""GGUF checkpoints: golem's tensors.GGUF over the library's reader, and the
Qwen3 binding of its tensors.

`GGUF` wraps gx_gguf_open (tensors/gguf.go:164 OpenGGUF): the file is mapped
whole and every tensor is a numpy view into the mapping, valid until close().
The metadata accessors are golem's (tensors/gguf_meta.go): string, bool,
float32, uint32, uint32_slice (a scalar reads as a list of one), bool_slice,
strings; an absent key or a value of the wrong type raises GxError with
golem's message.

`load_qwen(path, max_context)` is qwen.LoadConfig (qwen/config.go:60-163)
followed by qwen.LoadWeights (qwen/weights.go:104-177): the same keys, the
same tensor names, the same shape checks and refusals.  It returns a
synth.QwenConfig and the weights dict QwenModel takes, whose arrays are views
into the file; QwenModel uploads them (one pass over the mapping, no host
copy of a matrix beyond the Q|K|V and Gate|Up concatenations).
"""
import ctypes

import numpy as np

from . import capi, synth

# ggml tensor types golem reads (tensors/gguf.go:200-207)
GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q8_0, GGML_Q6_K, GGML_BF16 = 0, 1, 2, 8, 14, 30
GGML_NAMES = {GGML_F32: "F32", GGML_F16: "F16", GGML_Q4_0: "Q4_0", GGML_Q8_0: "Q8_0", GGML_Q6_K: "Q6_K",
              GGML_BF16: "BF16"}
# nn.QuantOf (nn/quant.go:35-47): the tensor types that are weight formats
QUANT_OF = {GGML_F32: capi.F32, GGML_BF16: capi.BF16, GGML_Q4_0: capi.Q4_0, GGML_Q6_K: capi.Q6_K}


class Tensor:
    """One entry of the tensor table: name, ggml type, shape (row length
    first, as the file stores it), and the bytes as a uint8 view."""

    def __init__(self, name, ggml_type, shape, ptr, nbytes):
        self.name, self.ggml_type, self.shape = name, ggml_type, shape
        self.ptr, self.nbytes = ptr, nbytes
        self.raw = np.ctypeslib.as_array((ctypes.c_uint8 * nbytes).from_address(ptr)) if nbytes else \
            np.zeros(0, np.uint8)

    @property
    def dtype(self):
        return GGML_NAMES[self.ggml_type]

    def floats(self):
        """The F32 tensor's values (golem's floats, qwen/weights.go:88-102)."""
        if self.ggml_type != GGML_F32:
            raise capi.GxError("gguf", capi.GX_ERR_INVALID, f'tensor "{self.name}" is {self.dtype}, not F32')
        return self.raw.view(np.float32)


class GGUF:
    def __init__(self, path):
        self.ptr = ctypes.c_void_p()
        capi.call("gx_gguf_open", str(path).encode(), ctypes.byref(self.ptr))
        self.path = str(path)
        n = ctypes.c_int()
        capi.call("gx_gguf_tensor_count", self.ptr, ctypes.byref(n))
        self.tensors = {}
        for i in range(n.value):
            name = ctypes.c_char_p()
            capi.call("gx_gguf_tensor_name", self.ptr, i, ctypes.byref(name))
            t = self._get(name.value)
            self.tensors[t.name] = t

    def _get(self, name_bytes):
        kind, nd = ctypes.c_int(), ctypes.c_int()
        shape = (ctypes.c_int64 * 4)()
        data, nbytes = ctypes.c_void_p(), ctypes.c_size_t()
        capi.call("gx_gguf_tensor", self.ptr, name_bytes, ctypes.byref(kind), ctypes.byref(nd), shape,
                  ctypes.byref(data), ctypes.byref(nbytes))
        return Tensor(name_bytes.decode(), kind.value, [int(shape[d]) for d in range(nd.value)], data.value or 0,
                      nbytes.value)

    def get(self, name):
        """Get (tensors/gguf.go:305): raises when the tensor is absent."""
        t = self.tensors.get(name)
        if t is None:
            raise capi.GxError("gx_gguf_tensor", capi.GX_ERR_INVALID, f'tensor "{name}" is absent')
        return t

    def keys(self):
        n = ctypes.c_int()
        capi.call("gx_gguf_meta_count", self.ptr, ctypes.byref(n))
        out = []
        for i in range(n.value):
            key, kind = ctypes.c_char_p(), ctypes.c_int()
            capi.call("gx_gguf_meta_key", self.ptr, i, ctypes.byref(key), ctypes.byref(kind))
            out.append(key.value.decode())
        return out

    def string(self, key):
        s, n = ctypes.c_void_p(), ctypes.c_size_t()
        capi.call("gx_gguf_meta_string", self.ptr, key.encode(), ctypes.byref(s), ctypes.byref(n))
        return ctypes.string_at(s.value, n.value).decode() if n.value else ""

    def bool(self, key):
        v = ctypes.c_int()
        capi.call("gx_gguf_meta_bool", self.ptr, key.encode(), ctypes.byref(v))
        return bool(v.value)

    def float32(self, key):
        v = ctypes.c_float()
        capi.call("gx_gguf_meta_f32", self.ptr, key.encode(), ctypes.byref(v))
        return np.float32(v.value)

    def uint32(self, key):
        v = ctypes.c_uint32()
        capi.call("gx_gguf_meta_u32", self.ptr, key.encode(), ctypes.byref(v))
        return v.value

    def uint32_slice(self, key):
        n = ctypes.c_size_t()
        capi.call("gx_gguf_meta_u32s", self.ptr, key.encode(), None, 0, ctypes.byref(n))
        buf = (ctypes.c_uint32 * max(n.value, 1))()
        capi.call("gx_gguf_meta_u32s", self.ptr, key.encode(), buf, n.value, ctypes.byref(n))
        return [int(buf[i]) for i in range(n.value)]

    def bool_slice(self, key):
        n = ctypes.c_size_t()
        capi.call("gx_gguf_meta_bools", self.ptr, key.encode(), None, 0, ctypes.byref(n))
        buf = (ctypes.c_uint8 * max(n.value, 1))()
        capi.call("gx_gguf_meta_bools", self.ptr, key.encode(), buf, n.value, ctypes.byref(n))
        return [bool(buf[i]) for i in range(n.value)]

    def strings(self, key):
        n = ctypes.c_size_t()
        capi.call("gx_gguf_meta_strings", self.ptr, key.encode(), 0, None, None, ctypes.byref(n))
        out = []
        for i in range(n.value):
            s, ln = ctypes.c_void_p(), ctypes.c_size_t()
            capi.call("gx_gguf_meta_strings", self.ptr, key.encode(), i, ctypes.byref(s), ctypes.byref(ln),
                      ctypes.byref(n))
            out.append(ctypes.string_at(s.value, ln.value).decode() if ln.value else "")
        return out

    def has(self, key):
        return key in self.keys()

    def close(self):
        if self.ptr:
            capi.call("gx_gguf_close", self.ptr)
            self.ptr = ctypes.c_void_p()
            self.tensors = {}

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


def _refuse(message):
    raise capi.GxError("gguf", capi.GX_ERR_INVALID, message)


def _optional(fn, key):
    try:
        return fn(key)
    except capi.GxError:
        return None


def qwen_config(g, max_context):
    """qwen.LoadConfig (qwen/config.go:60-163) for the device model: the
    geometry read from the file, every block alike (this engine's model has
    one geometry for all blocks; a file whose blocks differ is refused)."""
    arch = g.string("general.architecture")
    if arch != "qwen3":
        _refuse(f'architecture "{arch}" is not qwen3')

    def key(suffix):
        return f"{arch}.{suffix}"

    blocks = g.uint32(key("block_count"))
    dim = g.uint32(key("embedding_length"))
    eps = g.float32(key("attention.layer_norm_rms_epsilon"))
    heads = g.uint32_slice(key("attention.head_count"))
    kv_heads = g.uint32_slice(key("attention.head_count_kv"))
    ffn = g.uint32_slice(key("feed_forward_length"))
    head_dim = g.uint32(key("attention.key_length"))
    value_dim = _optional(g.uint32, key("attention.value_length"))
    if value_dim is not None and value_dim != head_dim:
        _refuse(f"keys are {head_dim} wide and values {value_dim}, which this engine does not do")
    rope_base = g.float32(key("rope.freq_base"))
    rope_dims = _optional(g.uint32, key("rope.dimension_count"))
    if rope_dims is None:
        rope_dims = head_dim
    embd = g.tensors.get("token_embd.weight")
    if embd is None or len(embd.shape) != 2:
        _refuse("token_embd.weight is absent or not two-dimensional")
    vocab = embd.shape[1]  # GGUF stores the row length first

    def per_block(values, i):
        return values[0] if len(values) == 1 else values[i]

    geo = set()
    for i in range(blocks):
        h, kv, f = per_block(heads, i), per_block(kv_heads, i), per_block(ffn, i)
        if head_dim % 2 != 0 or rope_dims > head_dim:
            _refuse(f"block {i}: head {head_dim}, rotated {rope_dims}")
        if kv == 0 or h % kv != 0:
            _refuse(f"block {i}: {h} query heads do not divide into {kv} key-value heads")
        geo.add((h, kv, f))
    if len(geo) > 1:
        _refuse("qwen: blocks of different geometry are not supported on the device")
    if rope_dims != head_dim:
        _refuse(f"qwen: a partial rotation ({rope_dims} of {head_dim}) is not supported on the device")
    (h, kv, f), = geo
    return synth.QwenConfig(dim, f, blocks, h, kv, head_dim, vocab, max_context, rope_base=float(rope_base),
                            eps=float(eps))


def qwen_weights(g, cfg):
    """qwen.LoadWeights (qwen/weights.go:104-177): every tensor the geometry
    names, checked against the shape it must have, as the dict QwenModel
    takes (matrices as GGUF bytes, norms as float32) plus the head's format
    under "token_embd_quant"."""
    def matrix(name, rows, cols, formats=(GGML_Q4_0,)):
        t = g.get(name)
        if len(t.shape) != 2:
            _refuse(f'tensor "{name}" has {len(t.shape)} dimensions')
        if t.ggml_type not in QUANT_OF:
            _refuse(f'tensor "{name}" is {t.dtype}, which is not a weight format')
        if t.shape[1] != rows or t.shape[0] != cols:
            _refuse(f"{name} is {t.shape[1]} by {t.shape[0]}, not {rows} by {cols}")
        if t.ggml_type not in formats:
            _refuse(f"qwen: {name} is {t.dtype}; the device model takes "
                    f"{' or '.join(GGML_NAMES[f] for f in formats)} here")
        return t

    def floats(name, want):
        t = g.get(name)
        v = t.floats()
        if len(v) != want:
            _refuse(f"{name} is {len(v)} wide, not {want}")
        return v

    embd = matrix("token_embd.weight", cfg.vocab, cfg.dim, formats=(GGML_Q4_0, GGML_Q6_K))
    out = {"token_embd": embd.raw, "token_embd_quant": QUANT_OF[embd.ggml_type],
           "output_norm": floats("output_norm.weight", cfg.dim), "blocks": []}
    if "output.weight" in g.tensors:
        _refuse("this checkpoint has an output.weight; the engine assumes a tied head")
    qd, kvd = cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
    for i in range(cfg.layers):
        def name(suffix):
            return f"blk.{i}.{suffix}"
        b = {
            "attn_norm": floats(name("attn_norm.weight"), cfg.dim),
            "ffn_norm": floats(name("ffn_norm.weight"), cfg.dim),
            "q_norm": floats(name("attn_q_norm.weight"), cfg.head_dim),
            "k_norm": floats(name("attn_k_norm.weight"), cfg.head_dim),
        }
        for key, tname, rows, cols in (("q", "attn_q.weight", qd, cfg.dim), ("k", "attn_k.weight", kvd, cfg.dim),
                                       ("v", "attn_v.weight", kvd, cfg.dim), ("o", "attn_output.weight", cfg.dim, qd),
                                       ("gate", "ffn_gate.weight", cfg.ffn, cfg.dim),
                                       ("up", "ffn_up.weight", cfg.ffn, cfg.dim),
                                       ("down", "ffn_down.weight", cfg.dim, cfg.ffn)):
            b[key] = matrix(name(tname), rows, cols).raw
        out["blocks"].append(b)
    return out


def load_qwen(path, max_context):
    """Opens a Qwen3 GGUF and binds it: (GGUF, QwenConfig, weights).  The
    weights are views into the GGUF; close it once the model is built."""
    g = GGUF(path)
    try:
        cfg = qwen_config(g, max_context)
        return g, cfg, qwen_weights(g, cfg)
    except Exception:
        g.close()
        raise
