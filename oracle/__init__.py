"""Python handle on the oracle: golem's generic Go arithmetic restated in C
(oracle/oracle.c), for checking the GPU path.

TEST INFRASTRUCTURE ONLY: tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg are the only importers.  The product (golem_amd/) never
imports it.

Arrays are numpy; layouts are golem's nn.Batch (nn/batch.go:17-45):
Q int8 [block][column][32], Scales/Corr [block][column], QK [column][width],
KScales [column][width/256], BSums [column][width/16]; outputs [column][rows].
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

F32, BF16, Q4_0, Q6_K = 0, 1, 2, 3

_lib = None


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        from . import build
        build.build(verbose=False)
    lib = ctypes.CDLL(LIB_PATH)
    I, F, V, S = ctypes.c_int, ctypes.c_float, ctypes.c_void_p, ctypes.c_size_t
    sig = {
        "orc_half_to_float": (F, [ctypes.c_uint16]),
        "orc_float_to_half": (ctypes.c_uint16, [F]),
        "orc_round_half": (F, [F]),
        "orc_round_half_n": (None, [V, I]),
        "orc_nearest_int": (ctypes.c_int32, [F]),
        "orc_quantize_range": (I, [V, I, I, I, V, V, V, I, I]),
        "orc_quantize_column_range": (None, [V, I, I, V, V, V, I, I, I]),
        "orc_quantize_k": (I, [V, I, I, V, V, V]),
        "orc_dot_q4_0_go": (None, [V, V, V, V, I, I, I, I, V]),
        "orc_fold": (F, [V, F]),
        "orc_mat_vec_q4_0_rows": (None, [V, V, V, V, I, I, I, V, I, I, I]),
        "orc_dequantize_q4_0_row": (None, [V, I, V]),
        "orc_packed_q4_0_bytes": (S, [I, I]),
        "orc_pack_q4_0": (I, [V, I, I, V]),
        "orc_dot_packed_q4_0_go": (None, [V, V, V, V, I, I, I, I, V]),
        "orc_mat_vec_packed_q4_0_rows": (None, [V, V, V, V, I, I, I, V, I, I, I]),
        "orc_q6_k_block_isum": (ctypes.c_int32, [V, V, V]),
        "orc_q4_0_acc": (ctypes.c_int32, [V, V]),
        "orc_dot_q6_k_go": (F, [V, V, V, V, I]),
        "orc_mat_vec_q6_k_rows": (None, [V, V, V, V, I, I, I, V, I, I, I]),
        "orc_dequantize_q6_k": (None, [V, I, V]),
        "orc_dot_f32": (F, [V, V, I]),
        "orc_dot_f32_avx2": (F, [V, V, I]),
        "orc_rope_prepare": (None, [I, I, ctypes.c_double, V, V]),
        "orc_rope_apply": (None, [V, I, V, V]),
        "orc_attend": (None, [V, V, V, I, I, I, I, F, V, V]),
        "orc_attend_parallel": (None, [V, V, V, I, I, I, I, F, V, V]),
        "orc_exp_neg": (F, [F]),
        "orc_exp_neg_check": (ctypes.c_long, [V, ctypes.c_long, V]),
        "orc_matrix_rows": (I, [I, V, V, I, I, V, I, V, V, V, V, V, V, V, I, I, V, I, I, I]),
        "orc_rms_norm_plain": (None, [V, I, V, F]),
        "orc_gelu_table_build": (None, [V]),
        "orc_gelu_table": (None, [V, I]),
        "orc_expf": (F, [F]),
        "orc_swiglu_range": (None, [V, V, I, I]),
        "orc_softmax_in_place": (None, [V, I]),
        "orc_axpy": (None, [V, V, I, F]),
        "orc_choose_experts": (None, [V, I, I, V, V]),
        "orc_route_one": (None, [V, I, V, V, I, I, F, V, V, V, V]),
        "orc_expert_unit": (None, [I, V, V, V, I, I, V]),
        "orc_expert_reduce": (None, [V, V, V, V, I, I, V]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


# ---- scalars --------------------------------------------------------------

def half_to_float(h):
    return load().orc_half_to_float(int(h))


def float_to_half(f):
    return load().orc_float_to_half(float(f))


def nearest_int(f):
    return load().orc_nearest_int(float(f))


def expf(x):
    return load().orc_expf(float(x))


# ---- batches (nn.Batch) ---------------------------------------------------

class Batch:
    """golem's nn.Batch (nn/batch.go:17-66): F [size][width] float32 and the
    Q8_0 form interleaved by column; QuantizeK adds the Q8_K form."""

    def __init__(self, F):
        F = np.ascontiguousarray(F, dtype=np.float32)
        self.size, self.width = F.shape
        if self.width % 32:
            raise ValueError("nn: activation length must be a multiple of the block size")
        self.stride = self.size
        self.F = F
        blocks = self.width // 32
        self.Q = np.zeros(blocks * self.size * 32, dtype=np.int8)
        self.Scales = np.zeros(blocks * self.size, dtype=np.float32)
        self.Corr = np.zeros(blocks * self.size, dtype=np.float32)
        self.QK = self.KScales = self.BSums = None

    def quantize(self):
        rc = load().orc_quantize_range(_p(self.F), self.width, self.size, self.stride, _p(self.Q),
                                       _p(self.Scales), _p(self.Corr), 0, self.width)
        assert rc == 0
        return self

    def quantize_k(self):
        if self.width % 256:
            raise ValueError("nn: the Q8_K form needs a multiple of the superblock size")
        self.QK = np.zeros(self.size * self.width, dtype=np.int8)
        self.KScales = np.zeros(self.size * self.width // 256, dtype=np.float32)
        self.BSums = np.zeros(self.size * self.width // 16, dtype=np.int16)
        rc = load().orc_quantize_k(_p(self.F), self.width, self.size, _p(self.QK), _p(self.KScales),
                                   _p(self.BSums))
        assert rc == 0
        return self

    # Views in the GPU's token-major layout.
    def q_rows(self):
        """Q as [size][width] (token-major)."""
        b = self.width // 32
        return self.Q.reshape(b, self.size, 32).transpose(1, 0, 2).reshape(self.size, self.width).copy()

    def scales_rows(self):
        b = self.width // 32
        return self.Scales.reshape(b, self.size).T.copy()

    def corr_rows(self):
        b = self.width // 32
        return self.Corr.reshape(b, self.size).T.copy()

    def qsum_rows(self):
        return self.q_rows().reshape(self.size, -1, 32).astype(np.int32).sum(axis=2).astype(np.int32)


# ---- products -------------------------------------------------------------

def mat_vec_q4_0_rows(w, batch, rows, start=0, end=None, ys=None):
    """matVecQ4_0Rows with golem's generic kernels (row layout)."""
    end = rows if end is None else end
    if ys is None:
        ys = np.full((batch.size, rows), np.nan, dtype=np.float32)
    load().orc_mat_vec_q4_0_rows(_p(w), _p(batch.Q), _p(batch.Scales), _p(batch.Corr), batch.stride,
                                 batch.size, batch.width, _p(ys), ys.shape[1], start, end)
    return ys


def pack_q4_0(w, rows, cols):
    out = np.zeros(load().orc_packed_q4_0_bytes(rows, cols), dtype=np.uint8)
    assert load().orc_pack_q4_0(_p(w), rows, cols, _p(out)) == 0
    return out


def mat_vec_packed_q4_0_rows(packed, batch, rows, start=0, end=None, ys=None):
    end = rows if end is None else end
    if ys is None:
        ys = np.full((batch.size, rows), np.nan, dtype=np.float32)
    load().orc_mat_vec_packed_q4_0_rows(_p(packed), _p(batch.Q), _p(batch.Scales), _p(batch.Corr),
                                        batch.stride, batch.size, batch.width, _p(ys), ys.shape[1], start, end)
    return ys


def matrix_rows(quant, data, rows, cols, batch, start=0, end=None, packed=None, bias=None, ys=None):
    """Matrix.rows (nn/matrix.go:94-131)."""
    end = rows if end is None else end
    if ys is None:
        ys = np.full((batch.size, rows), np.nan, dtype=np.float32)
    rc = load().orc_matrix_rows(quant, _p(data), _p(packed), rows, cols, _p(bias),
                                0 if bias is None else len(bias), _p(batch.F), _p(batch.Q), _p(batch.Scales),
                                _p(batch.Corr), _p(batch.QK), _p(batch.KScales), _p(batch.BSums), batch.stride,
                                batch.size, _p(ys), ys.shape[1], start, end)
    if rc != 0:
        raise ValueError(f"nn: matrix_rows refused (status {rc})")
    return ys


def mat_vec_q6_k_rows(w, batch, rows, start=0, end=None, ys=None):
    end = rows if end is None else end
    if ys is None:
        ys = np.full((batch.size, rows), np.nan, dtype=np.float32)
    load().orc_mat_vec_q6_k_rows(_p(w), _p(batch.QK), _p(batch.KScales), _p(batch.BSums), batch.width,
                                 batch.size, batch.width, _p(ys), ys.shape[1], start, end)
    return ys


def dequantize_q4_0_row(w_row, n):
    out = np.zeros(n, dtype=np.float32)
    load().orc_dequantize_q4_0_row(_p(np.ascontiguousarray(w_row)), n, _p(out))
    return out


def dequantize_q6_k(w_row, n):
    out = np.zeros(n, dtype=np.float32)
    load().orc_dequantize_q6_k(_p(np.ascontiguousarray(w_row)), n, _p(out))
    return out


def q4_0_block_acc(w, batch, rows):
    """golem's per-block integer accumulator (unsigned nibbles) for every
    (column, row, block): [size][rows][blocks] int32, computed in numpy from
    the same bytes (the oracle's C loop states the same sum)."""
    blocks = batch.width // 32
    wb = w.reshape(rows, blocks, 18)
    nib = wb[:, :, 2:]
    lo = (nib & 0x0F).astype(np.int32)
    hi = (nib >> 4).astype(np.int32)
    wv = np.concatenate([lo, hi], axis=2)  # [rows][blocks][32]: weight j at index j
    q = batch.q_rows().reshape(batch.size, blocks, 32).astype(np.int32)
    return np.einsum("rbj,cbj->crb", wv, q, optimize=True).astype(np.int32)


def q6_k_block_isum(w, batch, rows):
    """dotQ6_KGo's per-superblock integer for every (column, row, superblock)
    via the oracle's C restatement."""
    nsb = batch.width // 256
    lib = load()
    out = np.zeros((batch.size, rows, nsb), dtype=np.int32)
    wb = w.reshape(rows, nsb, 210)
    for c in range(batch.size):
        qk = batch.QK[c * batch.width:(c + 1) * batch.width]
        bs = batch.BSums[c * batch.width // 16:(c + 1) * batch.width // 16]
        for r in range(rows):
            for b in range(nsb):
                out[c, r, b] = lib.orc_q6_k_block_isum(_p(np.ascontiguousarray(wb[r, b])),
                                                       _p(qk[b * 256:(b + 1) * 256]), _p(bs[b * 16:(b + 1) * 16]))
    return out


def dot_f32(a, b):
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    return load().orc_dot_f32(_p(a), _p(b), min(len(a), len(b)))


def dot_f32_avx2(a, b):
    """DotF32 in dotF32AVX2's order (the form golem runs on amd64)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    return load().orc_dot_f32_avx2(_p(a), _p(b), min(len(a), len(b)))


def rms_norm_plain(x, gain=None, eps=1e-6):
    x = np.array(x, dtype=np.float32)
    g = None if gain is None else np.ascontiguousarray(gain, dtype=np.float32)
    load().orc_rms_norm_plain(_p(x), len(x), _p(g), eps)
    return x


def gelu_table(x):
    x = np.array(x, dtype=np.float32)
    load().orc_gelu_table(_p(x), len(x))
    return x


def gelu_table_build():
    t = np.zeros(1 << 16, dtype=np.float32)
    load().orc_gelu_table_build(_p(t))
    return t


def softmax_in_place(x):
    x = np.array(x, dtype=np.float32)
    load().orc_softmax_in_place(_p(x), len(x))
    return x


def choose_experts(logits, used):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    ids = np.zeros(used, dtype=np.int32)
    weights = np.zeros(used, dtype=np.float32)
    load().orc_choose_experts(_p(logits), len(logits), used, _p(ids), _p(weights))
    return ids, weights


def route_one(resid, router, used, eps=1e-6, router_scale=None):
    resid = np.ascontiguousarray(resid, dtype=np.float32)
    router = np.ascontiguousarray(router, dtype=np.float32)
    experts, dim = router.shape
    scratch = np.zeros(dim, dtype=np.float32)
    logits = np.zeros(experts, dtype=np.float32)
    ids = np.zeros(used, dtype=np.int32)
    weights = np.zeros(used, dtype=np.float32)
    rs = None if router_scale is None else np.ascontiguousarray(router_scale, dtype=np.float32)
    load().orc_route_one(_p(resid), dim, _p(router), _p(rs), experts, used, eps, _p(scratch), _p(logits),
                         _p(ids), _p(weights))
    return logits, ids, weights


def expert_unit(gate_up_w, down_w, x, dim, ffn, quant=None):
    """One (position, expert) unit of ExpertFFN; quant Q4_0 (default) or F32
    stacks."""
    partial = np.zeros(dim, dtype=np.float32)
    load().orc_expert_unit(Q4_0 if quant is None else quant, _p(np.ascontiguousarray(gate_up_w)),
                           _p(np.ascontiguousarray(down_w)), _p(np.ascontiguousarray(x, dtype=np.float32)), dim, ffn,
                           _p(partial))
    return partial


def expert_reduce(partials, ids, weights, dim, down_scale=None):
    out = np.zeros(dim, dtype=np.float32)
    ds = None if down_scale is None else np.ascontiguousarray(down_scale, dtype=np.float32)
    load().orc_expert_reduce(_p(np.ascontiguousarray(partials, dtype=np.float32)),
                             _p(np.ascontiguousarray(ids, dtype=np.int32)),
                             _p(np.ascontiguousarray(weights, dtype=np.float32)), _p(ds), len(ids), dim, _p(out))
    return out


def compare_floats(got, want):
    """golem's compareFloats (nn/quants_reference_test.go:96-120): the worst
    absolute gap over RMS(want) + 1e-6.  Returns (relative, index)."""
    got = np.asarray(got, dtype=np.float32).reshape(-1)
    want = np.asarray(want, dtype=np.float32).reshape(-1)
    assert got.shape == want.shape
    scale = np.float32(np.sqrt(np.sum(want.astype(np.float64) ** 2) / len(want))) + np.float32(1e-6)
    gaps = np.abs(got - want)
    at = int(np.argmax(gaps))
    return float(gaps[at] / scale), at


# ---- the CPU baseline: golem's AVX2 kernels and worker pool ----------------

CPU_LIB_PATH = os.path.join(HERE, "libcpu_avx2.so")
_cpu = None


def host_has_avx2():
    try:
        flags = open("/proc/cpuinfo").read()
    except OSError:
        return False
    return all(f" {f}" in flags for f in ("avx2", "fma", "f16c"))


def host_threads():
    """The threads the CPU baseline may use: OMP_NUM_THREADS when set (the GPU
    host sets it to its per-GPU share of cores), else this process's CPUs."""
    env = os.environ.get("OMP_NUM_THREADS", "")
    n = len(os.sched_getaffinity(0))
    return min(int(env), n) if env.isdigit() and int(env) > 0 else n


def cpu_lib(threads=None):
    """libcpu_avx2.so with its pool started (once per process)."""
    global _cpu
    if _cpu is not None:
        return _cpu
    if not host_has_avx2():
        raise RuntimeError("the CPU baseline needs AVX2, FMA and F16C")
    if not os.path.exists(CPU_LIB_PATH):
        from . import build
        build.build(verbose=False)
    lib = ctypes.CDLL(CPU_LIB_PATH)
    I, F, V = ctypes.c_int, ctypes.c_float, ctypes.c_void_p
    for name, (res, args) in {
        "cpu_pool_init": (I, [I]),
        "cpu_pool_threads": (I, []),
        "cpu_mat_vec_q6_k": (I, [V, V, V, V, I, I, I, V, I, I]),
        "cpu_mat_vec_q4_0": (I, [V, V, V, V, I, I, I, V, I, I]),
        "cpu_mat_vec_packed_q4_0": (I, [V, V, V, V, I, I, I, V, I, I]),
        "cpu_moe_ffn": (I, [V, V, V, V, I, I, I, I, I, V, V, V, V, V, V, V, V, V, V, V, V, V, V, I]),
        "cpu_qwen_token": (I, [V, I, I, I, I, I, I, I, I, F, V, V, V, V, I, V, V, I]),
        "cpu_dot_q4_0": (None, [V, V, V, V, I, I, I, I, V, I, I]),
        "cpu_dot_q6_k": (F, [V, V, V, V, I]),
        "cpu_dot_f32": (F, [V, V, I]),
    }.items():
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = res, args
    if lib.cpu_pool_init(threads or host_threads()) != 0:
        raise RuntimeError("cpu_pool_init refused")
    _cpu = lib
    return lib


def cpu_mat_vec_q6_k(w, batch, rows, threads, ys=None):
    """MatVecQ6_K through golem's AVX2 kernel on at most `threads` threads."""
    if ys is None:
        ys = np.full((batch.size, rows), np.nan, dtype=np.float32)
    rc = cpu_lib().cpu_mat_vec_q6_k(_p(w), _p(batch.QK), _p(batch.BSums), _p(batch.KScales), rows, batch.width,
                                    batch.size, _p(ys), ys.shape[1], threads)
    assert rc == 0
    return ys


def cpu_mat_vec_q4_0(w, batch, rows, threads, ys=None):
    """MatVecQ4_0 (row layout) through golem's AVX2 x8/x4/x1 kernels."""
    if ys is None:
        ys = np.full((batch.size, rows), np.nan, dtype=np.float32)
    rc = cpu_lib().cpu_mat_vec_q4_0(_p(w), _p(batch.Q), _p(batch.Scales), _p(batch.Corr), rows, batch.width,
                                    batch.size, _p(ys), ys.shape[1], threads)
    assert rc == 0
    return ys


def cpu_mat_vec_packed_q4_0(packed, batch, rows, threads, ys=None):
    """matVecPackedQ4_0Rows (whole groups of eight rows) through golem's AVX2
    x4/x1 packed kernels, from pack_q4_0's layout."""
    if ys is None:
        ys = np.full((batch.size, rows), np.nan, dtype=np.float32)
    rc = cpu_lib().cpu_mat_vec_packed_q4_0(_p(packed), _p(batch.Q), _p(batch.Scales), _p(batch.Corr), rows,
                                           batch.width, batch.size, _p(ys), ys.shape[1], threads)
    assert rc == 0
    return ys


class CpuMoE:
    """gemma's Route + ExpertFFN (gemma/moe.go:34-180) through golem's x86
    kernels (cpu_avx2.c: dotF32AVX2, matVecQ4_0Rows over the row-layout
    expert stacks, the worker pool's sections), with its scratch for `batch`
    positions.  run() returns (out [batch][D], ids [batch][k], weights)."""

    def __init__(self, router, gate_up, down, D, F, E, k, batch):
        self.router = np.ascontiguousarray(router, np.float32)
        self.gate_up, self.down = np.ascontiguousarray(gate_up), np.ascontiguousarray(down)
        self.D, self.F, self.E, self.k, self.batch = D, F, E, k, batch
        self.gelu = gelu_table_build()
        u = batch * k
        z = lambda shape, dt=np.float32: np.zeros(shape, dt)
        self.rin, self.logits = z((batch, D)), z((batch, E))
        self.ids, self.weights = z((batch, k), np.int32), z((batch, k))
        self.xq, self.xs, self.xc = z((batch, D), np.int8), z((batch, D // 32)), z((batch, D // 32))
        self.gu = z((u, 2 * F))
        self.mq, self.ms, self.mc = z((u, F), np.int8), z((u, F // 32)), z((u, F // 32))
        self.partial, self.out = z((u, D)), z((batch, D))

    def run(self, resid, threads):
        resid = np.ascontiguousarray(resid, np.float32)
        assert resid.shape == (self.batch, self.D)
        rc = cpu_lib().cpu_moe_ffn(_p(self.router), _p(self.gate_up), _p(self.down), _p(self.gelu), self.D, self.F,
                                   self.E, self.k, self.batch, _p(resid), _p(self.rin), _p(self.logits), _p(self.ids),
                                   _p(self.weights), _p(self.xq), _p(self.xs), _p(self.xc), _p(self.gu), _p(self.mq),
                                   _p(self.ms), _p(self.mc), _p(self.partial), _p(self.out), threads)
        assert rc == 0
        return self.out, self.ids, self.weights


class CpuQwen:
    """golem's Qwen3 decode token (qwen/block.go:32-102, attention.go:34-127,
    model.go:181-194) through its x86 kernels (cpu_avx2.c): the dense
    matrices in PackQ4_0's layout (golem's loader repacks them), the fp32
    caches of golem's LayerCache, the Q6_K tied head.  `layers` is a list of
    weight dicts as synth.qwen_weights builds them."""

    KEYS = ("q", "k", "v", "o", "gate", "up", "down")

    def __init__(self, cfg, weights, layers=None):
        self.cfg = cfg
        blocks = weights["blocks"] if layers is None else layers
        shapes = {"q": (cfg.heads * cfg.head_dim, cfg.dim), "k": (cfg.kv_heads * cfg.head_dim, cfg.dim),
                  "v": (cfg.kv_heads * cfg.head_dim, cfg.dim), "o": (cfg.dim, cfg.heads * cfg.head_dim),
                  "gate": (cfg.ffn, cfg.dim), "up": (cfg.ffn, cfg.dim), "down": (cfg.dim, cfg.ffn)}
        self.keep = []
        ptrs = []
        for b in blocks:
            mats = [pack_q4_0(b[n], *shapes[n]) for n in self.KEYS]
            norms = [np.ascontiguousarray(b[n], np.float32) for n in ("attn_norm", "ffn_norm", "q_norm", "k_norm")]
            caches = [np.zeros((cfg.max_context, cfg.kv_heads, cfg.head_dim), np.float32) for _ in range(2)]
            self.keep += mats + norms + caches
            ptrs += [a.ctypes.data for a in mats + norms + caches]
        self.ptrs = np.array(ptrs, dtype=np.uint64)
        self.caches = [(self.keep[i + 11], self.keep[i + 12]) for i in range(0, len(self.keep), 13)]
        self.output_norm = np.ascontiguousarray(weights["output_norm"], np.float32)
        self.head = np.ascontiguousarray(weights["token_embd"])
        self.logits = np.zeros(cfg.vocab, np.float32)

    def token(self, x, pos, cos, sin, threads):
        """x: the embedding row (float32 [dim], updated to the final-normed
        hidden state); cos / sin: RoPETable's row for pos.  Returns the
        logits."""
        cfg = self.cfg
        rc = cpu_lib().cpu_qwen_token(ctypes.c_void_p(self.ptrs.ctypes.data), len(self.caches), cfg.dim, cfg.ffn,
                                      cfg.heads, cfg.kv_heads, cfg.head_dim, cfg.max_context, pos, cfg.eps,
                                      _p(np.ascontiguousarray(cos, np.float32)),
                                      _p(np.ascontiguousarray(sin, np.float32)), _p(self.output_norm),
                                      _p(self.head), cfg.vocab, _p(x), _p(self.logits), threads)
        assert rc == 0
        return self.logits


def cpu_dot_q4_0(w_row, batch, block, column, n, state, mode, cols):
    cpu_lib().cpu_dot_q4_0(_p(w_row), _p(batch.Q), _p(batch.Scales), _p(batch.Corr), batch.stride, block, column, n,
                           _p(state), mode, cols)
    return state
