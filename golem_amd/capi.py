"""ctypes binding of the C ABI in include/golem_hip.h.

This is how Python (the tests, bench.py, smoke) reaches the HIP library; a Go
caller reaches the same entry points through a cgo shim over the same
header.  Device pointers are passed as integers (for instance a torch
tensor's data_ptr()); the library itself never sees a torch type.

Loading fails loudly when libgolem_hip.so is missing: there is no CPU
fallback behind this module.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libgolem_hip.so")

GX_OK = 0
GX_ERR_INVALID = 1
GX_ERR_HIP = 2
GX_ERR_UNSUPPORTED = 3
GX_ERR_NOMEM = 4

# golem's nn.Quant values (nn/quant.go:12-17)
F32, BF16, Q4_0, Q6_K = 0, 1, 2, 3

_c_int = ctypes.c_int
_c_size = ctypes.c_size_t
_vp = ctypes.c_void_p
_pp = ctypes.POINTER(ctypes.c_void_p)

# name -> (argtypes); every function returns int unless listed in _RESTYPE
_SIGNATURES = {
    "gx_last_error": [],
    "gx_init": [_c_int, _pp],
    "gx_free": [_vp],
    "gx_set_stream": [_vp, _vp],
    "gx_sync": [_vp],
    "gx_alloc": [_vp, _c_size, _pp],
    "gx_dealloc": [_vp, _vp],
    "gx_upload": [_vp, _vp, _vp, _c_size],
    "gx_download": [_vp, _vp, _vp, _c_size],
    "gx_timer_start": [_vp],
    "gx_timer_stop": [_vp, ctypes.POINTER(ctypes.c_float)],
    "gx_weight_upload": [_vp, _vp, _c_size, _c_int, _c_int, _c_int, _c_int, _pp],
    "gx_weight_upload_stack": [_vp, _vp, _c_size, _c_int, _c_int, _c_int, _c_int, _c_int, _pp],
    "gx_weight_free": [_vp],
    "gx_weight_info": [_vp, ctypes.POINTER(_c_int), ctypes.POINTER(_c_int), ctypes.POINTER(_c_int),
                       ctypes.POINTER(_c_int), ctypes.POINTER(_c_size)],
    "gx_weight_rows": [_vp, _vp, _c_int, _vp, _c_int, _vp],
    "gx_quantize_q8_0": [_vp, _vp, _c_int, _c_int, _c_int, _vp, _vp, _vp, _vp, _vp],
    "gx_calib_empty": [_vp, _c_int],
    "gx_calib_read": [_vp, _vp, _c_size, _c_int, _vp],
    "gx_calib_valu": [_vp, _c_int, _c_int, _vp],
    "gx_quantize_q8_k": [_vp, _vp, _c_int, _c_int, _c_int, _vp, _vp, _vp],
    "gx_matmul_q4_0": [_vp, _vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _vp, _vp, _c_int],
    "gx_matmul_q4_0_expert": [_vp, _vp, _c_int, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _vp, _c_int],
    "gx_matmul_q6_k": [_vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _vp, _vp, _c_int],
    "gx_matmul_f32": [_vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _vp, _c_int],
    "gx_matvec_rows_q4_0": [_vp, _vp, _vp, _vp, _vp, _c_int, ctypes.c_uint64, _c_int, _c_int, _vp, _c_int],
    "gx_matvec_rows_q6_k": [_vp, _vp, _vp, _vp, _vp, _c_int, ctypes.c_uint64, _c_int, _c_int, _vp, _c_int],
    "gx_matvec_rows_stats": [_vp, ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64)],
    "gx_q4_0_block_dots": [_vp, _vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _vp],
    "gx_q4_0_fused_block_dots": [_vp, _vp, _c_int, _vp, _vp, _vp, ctypes.c_float, _c_int, _c_int, _vp, _vp, _vp,
                                 _vp],
    "gx_q6_k_block_dots": [_vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _vp],
    "gx_moe_block_dots": [_vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _vp, _vp, _vp, _vp, _vp, ctypes.c_size_t,
                          _vp, _vp],
    "gx_gelu_table": [_vp, _vp],
    "gx_moe_workspace_bytes": [_c_int, _c_int, _c_int, _c_int, _c_int, ctypes.POINTER(_c_size)],
    "gx_moe_route": [_vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, ctypes.c_float, _vp, _vp, _vp],
    "gx_moe_experts": [_vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _vp, _vp, _vp, _c_int, _vp, _c_size],
    "gx_moe_experts_noalloc": [_vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _vp, _vp, _vp, _c_int],
    "gx_norm_quant": [_vp, _vp, _c_int, _vp, _c_int, _vp, _c_int, _c_int, ctypes.c_float, _vp, _c_int, _vp, _vp, _vp],
    "gx_qwen_qkv_rope": [_vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _vp, _vp, _vp, _vp, _vp,
                         ctypes.c_float, _vp, _vp, _vp, _c_int, _vp, _c_int, _vp],
    "gx_qwen_qk_rope": [_vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_int, _vp, _vp, _vp, _vp, _vp, ctypes.c_float,
                        _vp, _vp, _vp, _c_int, _vp, _c_int],
    "gx_qwen_attention_workspace_bytes": [_c_int, _c_int, _c_int, ctypes.POINTER(_c_size)],
    "gx_qwen_rope_attention": [_vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_int, _vp, _vp, _vp, _vp, _vp,
                               ctypes.c_float, _vp, _vp, _c_int, _vp, _vp, _vp, _vp, _c_int],
    "gx_qwen_attention": [_vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_int, _vp, _vp, _vp, _c_int, _vp, _vp, _vp,
                          _vp, _c_size, _vp, _c_int],
    "gx_qwen_attention_parallel": [_vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_int, _vp, _vp, _vp, _c_int, _vp, _vp,
                                   _vp, _vp, _c_size, _vp, _c_int],
    "gx_qwen_rope_attention_parallel": [_vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_int, _vp, _vp, _vp, _vp, _vp,
                                        ctypes.c_float, _vp, _vp, _c_int, _vp, _vp, _vp, _vp, _c_int],
    "gx_qwen_rope_attention_slots": [_vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _vp, _vp, _vp, _vp,
                                     _vp, ctypes.c_float, _vp, _vp, _c_int, _vp, _vp, _vp, _vp, _c_int, _c_int],
    "gx_qwen_attention_heads": [_vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_int, _vp, _vp, _vp, _c_int, _vp],
    "gx_swiglu_quant": [_vp, _vp, _c_int, _c_int, _c_int, _c_int, _vp, _vp, _vp],
    "gx_matmul_swiglu_q4_0": [_vp, _vp, _vp, _vp, _vp, _c_int, _vp, _vp, _vp],
    "gx_norm_matmul_q4_0": [_vp, _vp, _vp, _vp, _vp, ctypes.c_float, _vp, _c_int, _c_int, _vp],
    "gx_norm_swiglu_q4_0": [_vp, _vp, _vp, _vp, _vp, ctypes.c_float, _vp, _vp, _vp, _vp],
    "gx_argmax_step": [_vp, _vp, _c_int, _vp, _vp, _c_int, _vp, _vp],
    "gx_argmax_slots_step": [_vp, _vp, _c_int, _c_int, _c_int, _vp, _vp, _vp],
    "gx_argmax": [_vp, _vp, _c_int, _c_int, _c_int, _vp],
    "gx_geglu_quant": [_vp, _vp, _c_int, _c_int, _c_int, _vp, _vp, _vp],
    "gx_moe_join": [_vp, _vp, _c_int, _vp, _c_int, _vp, _c_int, _vp, _vp, _vp, _c_int, _c_int, ctypes.c_float, _vp,
                    _c_int],
    "gx_gguf_open": [ctypes.c_char_p, _pp],
    "gx_gguf_close": [_vp],
    "gx_gguf_tensor_count": [_vp, ctypes.POINTER(_c_int)],
    "gx_gguf_tensor_name": [_vp, _c_int, ctypes.POINTER(ctypes.c_char_p)],
    "gx_gguf_tensor": [_vp, ctypes.c_char_p, ctypes.POINTER(_c_int), ctypes.POINTER(_c_int),
                       ctypes.POINTER(ctypes.c_int64), _pp, ctypes.POINTER(_c_size)],
    "gx_gguf_meta_count": [_vp, ctypes.POINTER(_c_int)],
    "gx_gguf_meta_key": [_vp, _c_int, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(_c_int)],
    "gx_gguf_meta_string": [_vp, ctypes.c_char_p, _pp, ctypes.POINTER(_c_size)],
    "gx_gguf_meta_bool": [_vp, ctypes.c_char_p, ctypes.POINTER(_c_int)],
    "gx_gguf_meta_f32": [_vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_float)],
    "gx_gguf_meta_u32": [_vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint32)],
    "gx_gguf_meta_u32s": [_vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint32), _c_size, ctypes.POINTER(_c_size)],
    "gx_gguf_meta_bools": [_vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint8), _c_size, ctypes.POINTER(_c_size)],
    "gx_gguf_meta_strings": [_vp, ctypes.c_char_p, _c_size, _pp, ctypes.POINTER(_c_size), ctypes.POINTER(_c_size)],
}
_RESTYPE = {"gx_last_error": ctypes.c_char_p}

_lib = None


class GxError(RuntimeError):
    def __init__(self, fn, code, message):
        super().__init__(f"{fn}: status {code}: {message}")
        self.code = code
        self.message = message


def load():
    """Loads libgolem_hip.so and declares every entry point; raises when the
    library has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: build it with golem_amd/build.py "
                           "(there is no CPU fallback for the GPU path)")
    lib = ctypes.CDLL(LIB_PATH)
    for name, args in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = _RESTYPE.get(name, _c_int)
    _lib = lib
    return lib


def exported_names():
    return list(_SIGNATURES)


def call(name, *args):
    """Calls an entry point and raises GxError on a non-zero status."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != GX_OK:
        raise GxError(name, rc, lib.gx_last_error().decode())
    return rc


def last_error():
    return load().gx_last_error().decode()


class Context:
    """One gx_ctx on a device.  stream: a hipStream_t as an int, or None for
    the null stream."""

    def __init__(self, device=0, stream=None):
        self.ptr = ctypes.c_void_p()
        call("gx_init", device, ctypes.byref(self.ptr))
        if stream is not None:
            call("gx_set_stream", self.ptr, ctypes.c_void_p(stream))

    def sync(self):
        call("gx_sync", self.ptr)

    def close(self):
        if self.ptr:
            call("gx_free", self.ptr)
            self.ptr = ctypes.c_void_p()

    def timer_start(self):
        call("gx_timer_start", self.ptr)

    def timer_stop(self):
        ms = ctypes.c_float()
        call("gx_timer_stop", self.ptr, ctypes.byref(ms))
        return ms.value


class Weight:
    """A resident matrix (or stack of `count` matrices) uploaded from GGUF
    bytes: a numpy uint8 array on the host, or (device_ptr, nbytes)."""

    def __init__(self, ctx, data, quant, rows, cols, count=1):
        self.ctx = ctx
        self.ptr = ctypes.c_void_p()
        self.quant, self.rows, self.cols, self.count = quant, rows, cols, count
        if isinstance(data, tuple):
            addr, nbytes = data
            on_device = 1
        else:
            addr, nbytes = data.ctypes.data, data.nbytes
            on_device = 0
        if count == 1:
            call("gx_weight_upload", ctx.ptr, ctypes.c_void_p(addr), nbytes, on_device, quant, rows, cols,
                 ctypes.byref(self.ptr))
        else:
            call("gx_weight_upload_stack", ctx.ptr, ctypes.c_void_p(addr), nbytes, on_device, quant, rows, cols,
                 count, ctypes.byref(self.ptr))

    def device_bytes(self):
        n = ctypes.c_size_t()
        call("gx_weight_info", self.ptr, None, None, None, None, ctypes.byref(n))
        return n.value

    def free(self):
        if self.ptr:
            call("gx_weight_free", self.ptr)
            self.ptr = ctypes.c_void_p()


def vp(x):
    """A device pointer argument from an int, a torch tensor or None.  Only the
    address is kept: the caller must hold the tensor until the work that uses
    it has run."""
    if x is None:
        return None
    if hasattr(x, "data_ptr"):
        return ctypes.c_void_p(x.data_ptr())
    return ctypes.c_void_p(int(x))


def q16_elems(M, K):
    """Values in the fp16 copy of a Q8_0 batch (gx_quantize_q8_0's q16):
    tokens padded to a multiple of 32."""
    return (M + 31) // 32 * 32 * K


def size_out(name, *args):
    """Calls an entry point whose last argument is a size_t out-parameter and
    returns that size."""
    n = _c_size(0)
    call(name, *args, ctypes.byref(n))
    return int(n.value)
