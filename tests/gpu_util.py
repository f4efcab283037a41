"""Helpers of the GPU tests: device buffers (torch as the allocator), and
thin calls of the C ABI that take and return numpy arrays."""
import ctypes
import sys

import numpy as np

from golem_amd import capi


def log(*args):
    print(*args, flush=True)
    sys.stdout.flush()


class Device:
    def __init__(self):
        import torch
        self.torch = torch
        assert torch.cuda.is_available(), "GPU tests need a GPU"
        torch.cuda.init()
        self.ctx = capi.Context(0, stream=torch.cuda.current_stream().cuda_stream)

    def close(self):
        self.ctx.close()

    # ---- buffers ----
    def put(self, a):
        t = self.torch
        a = np.ascontiguousarray(a)
        return t.from_numpy(a.copy()).to("cuda")

    def empty(self, shape, dtype):
        t = self.torch
        tdt = {np.float32: t.float32, np.int8: t.int8, np.int32: t.int32, np.int16: t.int16,
               np.uint8: t.uint8}[np.dtype(dtype).type]
        return t.empty(shape, dtype=tdt, device="cuda")

    def full(self, shape, value, dtype=np.float32):
        x = self.empty(shape, dtype)
        x.fill_(value)
        return x

    def get(self, x):
        self.ctx.sync()
        return x.cpu().numpy()

    # ---- calls ----
    def weight(self, data, quant, rows, cols, count=1):
        return capi.Weight(self.ctx, np.ascontiguousarray(data), quant, rows, cols, count)

    def quantize_q8_0(self, x, with_corr=True, with_q16=True):
        """The Q8_0 form on the device: (q, scales, qsum, q16, corr)."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        M, K = x.shape
        xd = self.put(x)
        q = self.empty((M, K), np.int8)
        sc = self.empty((M, K // 32), np.float32)
        qs = self.empty((M, K // 32), np.int32)
        co = self.empty((M, K // 32), np.float32) if with_corr else None
        q16 = self.empty((capi.q16_elems(M, K),), np.int16) if with_q16 else None
        capi.call("gx_quantize_q8_0", self.ctx.ptr, capi.vp(xd), K, M, K, capi.vp(q), capi.vp(sc), capi.vp(qs),
                  capi.vp(co), capi.vp(q16))
        return q, sc, qs, q16, co

    def quantize_q8_k(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        M, K = x.shape
        xd = self.put(x)
        q = self.empty((M, K), np.int8)
        ks = self.empty((M, K // 256), np.float32)
        bs = self.empty((M, K // 16), np.int16)
        capi.call("gx_quantize_q8_k", self.ctx.ptr, capi.vp(xd), K, M, K, capi.vp(q), capi.vp(ks), capi.vp(bs))
        return q, ks, bs

    def matmul_q4_0(self, w, act, M, start=0, end=None, bias=None, y=None, f16=True):
        """act is quantize_q8_0's tuple (or its first four entries, sliced);
        f16=False withholds q16 (the product runs on int8 MFMA either way)."""
        q, sc, qs, q16 = act[:4]
        end = w.rows if end is None else end
        if y is None:
            y = self.full((M, w.rows), float("nan"))
        b = None if bias is None else self.put(np.asarray(bias, dtype=np.float32))
        capi.call("gx_matmul_q4_0", self.ctx.ptr, w.ptr, capi.vp(q), capi.vp(sc), capi.vp(qs),
                  capi.vp(q16 if f16 else None), M, start, end, capi.vp(b), capi.vp(y), y.shape[1])
        return y

    def matmul_q6_k(self, w, act, M, start=0, end=None, bias=None, y=None):
        q, ks, bs = act
        end = w.rows if end is None else end
        if y is None:
            y = self.full((M, w.rows), float("nan"))
        b = None if bias is None else self.put(np.asarray(bias, dtype=np.float32))
        capi.call("gx_matmul_q6_k", self.ctx.ptr, w.ptr, capi.vp(q), capi.vp(ks), capi.vp(bs), M, start, end,
                  capi.vp(b), capi.vp(y), y.shape[1])
        return y

    def q4_0_block_dots(self, w, act, M, start, end, path):
        q, sc, qs, q16 = act[:4]
        out = self.empty((M, end - start, w.cols // 32), np.int32)
        capi.call("gx_q4_0_block_dots", self.ctx.ptr, w.ptr, capi.vp(q), capi.vp(sc), capi.vp(qs), capi.vp(q16), M,
                  start, end, path, capi.vp(out))
        return self.get(out)

    def q6_k_block_dots(self, w, act, M, start, end):
        q, ks, bs = act
        out = self.empty((M, end - start, w.cols // 256), np.int32)
        capi.call("gx_q6_k_block_dots", self.ctx.ptr, w.ptr, capi.vp(q), capi.vp(bs), M, start, end, capi.vp(out))
        return self.get(out)

    def rows(self, w, ids, expert=0):
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        idd = self.put(ids)
        out = self.empty((len(ids), w.cols), np.float32)
        capi.call("gx_weight_rows", self.ctx.ptr, w.ptr, expert, capi.vp(idd), len(ids), capi.vp(out))
        return self.get(out)


def q16_rows(q16, M, K):
    """The panel-ordered fp16 copy (gx_quantize_q8_0's q16) back to token rows
    [ceil(M/32)*32][K], as float32."""
    Mp = (M + 31) // 32 * 32
    # [G][b][h][g][li][e] -> token 32G + li, input 32b + 16h + 8g + e
    a = np.asarray(q16).view(np.float16).astype(np.float32).reshape(Mp // 32, K // 32, 2, 2, 32, 8)
    return a.transpose(0, 4, 1, 2, 3, 5).reshape(Mp, K)
