"""ctypes binding of the CPU oracle (liboracle.so).

Test infrastructure: imported by tests/, __graft_entry__.smoke() (as the
checker) and bench.py's cpu_baseline leg only.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

_lib = None

f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
u8p = np.ctypeslib.ndpointer(dtype=np.uint8, flags="C_CONTIGUOUS")
i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")

MAX_ROUNDS = 20


class CutoffTrace(C.Structure):
    _fields_ = [("rounds", C.c_int), ("converged", C.c_int),
                ("init_min", C.c_float), ("init_max", C.c_float),
                ("bounds", C.c_float * MAX_ROUNDS), ("counts", C.c_int * MAX_ROUNDS),
                ("final_min", C.c_float), ("final_max", C.c_float),
                ("final_min_count", C.c_int), ("final_max_count", C.c_int)]


class ModelConfig(C.Structure):
    _fields_ = [("n_layers", C.c_int), ("dim", C.c_int), ("ffn_dim", C.c_int),
                ("n_heads", C.c_int), ("n_kv_heads", C.c_int), ("head_dim", C.c_int),
                ("vocab", C.c_int), ("max_ctx", C.c_int), ("rope_theta", C.c_double),
                ("norm_eps", C.c_float)]


class Matrix(C.Structure):
    _fields_ = [("buckets", C.c_void_p), ("stats", C.c_void_p), ("probes", C.c_void_p),
                ("in_dim", C.c_int), ("out_dim", C.c_int)]


class Layer(C.Structure):
    _fields_ = [("wq", Matrix), ("wk", Matrix), ("wv", Matrix), ("wo", Matrix),
                ("w1", Matrix), ("w3", Matrix), ("w2", Matrix),
                ("attn_gain", C.c_void_p), ("ffn_gain", C.c_void_p)]


class Model(C.Structure):
    _fields_ = [("cfg", ModelConfig), ("layers", C.c_void_p), ("embed", C.c_void_p),
                ("final_gain", C.c_void_p), ("lm_head", Matrix), ("kcache", C.c_void_p),
                ("vcache", C.c_void_p), ("rope", C.c_void_p), ("lm_dense", C.c_void_p)]


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"oracle library missing: {LIB_PATH} (run `make -C oracle`)")
    L = C.CDLL(LIB_PATH)
    L.orc_f16_to_f32.restype = C.c_float
    L.orc_f16_to_f32.argtypes = [C.c_uint16]
    L.orc_f32_to_f16.restype = C.c_uint16
    L.orc_f32_to_f16.argtypes = [C.c_float]
    L.orc_f32_to_f16_n.argtypes = [f32p, u16p, C.c_size_t]
    L.orc_f64_to_f16.restype = C.c_uint16
    L.orc_f64_to_f16.argtypes = [C.c_double]
    L.orc_f64_to_f16_n.argtypes = [np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS"),
                                   u16p, C.c_size_t]
    L.orc_f16_to_f32_n.argtypes = [u16p, f32p, C.c_size_t]
    L.orc_pack_fp16.restype = C.c_uint16
    L.orc_pack_fp16.argtypes = [C.c_float, C.c_int]
    L.orc_unpack_fp16.argtypes = [C.c_uint16, C.POINTER(C.c_float), C.POINTER(C.c_int)]
    L.orc_gen_normal.restype = C.c_double
    L.orc_gen_normal.argtypes = [C.c_uint64, C.c_uint64, C.c_uint64]
    L.orc_gen_u32.restype = C.c_uint32
    L.orc_gen_u32.argtypes = [C.c_uint64, C.c_uint64, C.c_uint64]
    L.orc_gen_f16.argtypes = [C.c_uint64, C.c_uint64, C.c_size_t, C.c_double, C.c_double, u16p]
    L.orc_gen_f32.argtypes = [C.c_uint64, C.c_uint64, C.c_size_t, C.c_double, C.c_double, f32p]
    L.orc_gen_tokens.argtypes = [C.c_uint64, C.c_uint64, C.c_size_t, C.c_uint32, i32p]
    L.orc_bucketize.restype = C.c_int
    L.orc_bucketize.argtypes = [u16p, C.c_int, C.c_int, u16p, u16p, u16p]
    L.orc_np_pairwise_sum_f32.restype = C.c_float
    L.orc_np_pairwise_sum_f32.argtypes = [f32p, C.c_ssize_t]
    L.orc_effort_quantile.restype = C.c_int
    L.orc_effort_quantile.argtypes = [C.c_float]
    L.orc_importance.argtypes = [f32p, u16p, C.c_int, f32p]
    L.orc_find_cutoff.restype = C.c_float
    L.orc_find_cutoff.argtypes = [f32p, u16p, C.c_int, C.c_int, C.POINTER(CutoffTrace)]
    L.orc_find_cutoff_imp.restype = C.c_float
    L.orc_find_cutoff_imp.argtypes = [f32p, C.c_int, C.POINTER(CutoffTrace)]
    L.orc_select_rows.restype = C.c_int64
    L.orc_select_rows.argtypes = [f32p, u16p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float, u8p]
    L.orc_select_rows_block.restype = C.c_int64
    L.orc_select_rows_block.argtypes = [f32p, u16p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float, C.c_int,
                                        u8p]
    L.orc_bucket_walk.argtypes = [u16p, C.c_int, C.c_int, C.c_int, u8p, f32p, f32p, C.c_int]
    L.orc_bucketmul.restype = C.c_int64
    L.orc_bucketmul.argtypes = [f32p, u16p, u16p, u16p, C.c_int, C.c_int, C.c_int, C.c_int,
                                C.c_float, f32p, C.POINTER(C.c_float), u8p, C.c_int]
    L.orc_rmsnorm_gain.argtypes = [f32p, u16p, C.c_int, C.c_float, f32p]
    L.orc_silu_mul.argtypes = [f32p, f32p, C.c_int, f32p]
    L.orc_rope_table.argtypes = [C.c_double, C.c_int, C.c_int, f32p]
    L.orc_rope.argtypes = [f32p, f32p, C.c_int, C.c_int, f32p]
    L.orc_embed.argtypes = [u16p, C.c_int, C.c_int, f32p]
    L.orc_add.argtypes = [f32p, f32p, C.c_int, f32p]
    L.orc_attention_f16kv.argtypes = [f32p, u16p, u16p, C.c_int, C.c_int, C.c_int, C.c_int, f32p]
    L.orc_attention_f32rep.argtypes = [f32p, f32p, f32p, C.c_int, C.c_int, C.c_int, f32p]
    L.orc_rope_kv_rep32.argtypes = [f32p, f32p, f32p, f32p, C.c_int, C.c_int, C.c_int, f32p, f32p, f32p]
    L.orc_matmul_f16_dense.argtypes = [u16p, f32p, C.c_int, C.c_int, f32p]
    L.orc_argmax.restype = C.c_int
    L.orc_argmax.argtypes = [f32p, C.c_int]
    L.orc_set_selection_block.argtypes = [C.c_int, C.c_float]
    L.orc_threads.restype = C.c_int
    L.orc_threads.argtypes = []
    L.orc_layer_forward.argtypes = [C.POINTER(Model), C.c_int, C.c_int, C.c_float, f32p]
    L.orc_model_forward.argtypes = [C.POINTER(Model), C.c_int, C.c_int, C.c_float,
                                    C.c_void_p, f32p]
    _lib = L
    return L


# ---------------------------------------------------------------- helpers ---

def f32_to_f16(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, dtype=np.uint16)
    lib().orc_f32_to_f16_n(a.ravel(), out.ravel(), a.size)
    return out


def f64_to_f16(a):
    a = np.ascontiguousarray(a, dtype=np.float64)
    out = np.empty(a.shape, dtype=np.uint16)
    lib().orc_f64_to_f16_n(a.ravel(), out.ravel(), a.size)
    return out


def f16_to_f32(a):
    a = np.ascontiguousarray(a, dtype=np.uint16)
    out = np.empty(a.shape, dtype=np.float32)
    lib().orc_f16_to_f32_n(a.ravel(), out.ravel(), a.size)
    return out


def gen_f16(seed, tid, n, mean, sigma):
    out = np.empty(n, dtype=np.uint16)
    lib().orc_gen_f16(seed, tid, n, mean, sigma, out)
    return out


def gen_f32(seed, tid, n, mean, sigma):
    out = np.empty(n, dtype=np.float32)
    lib().orc_gen_f32(seed, tid, n, mean, sigma, out)
    return out


def gen_tokens(seed, tid, n, vocab):
    out = np.empty(n, dtype=np.int32)
    lib().orc_gen_tokens(seed, tid, n, vocab, out)
    return out


def bucketize(W):
    """W: uint16 (fp16 bits) [out_dim][in_dim] -> (buckets [16in][out/16], stats [16in][4], probes [in])"""
    W = np.ascontiguousarray(W, dtype=np.uint16)
    out_dim, in_dim = W.shape
    b = np.empty((in_dim * 16, out_dim // 16), dtype=np.uint16)
    s = np.empty((in_dim * 16, 4), dtype=np.uint16)
    p = np.empty(in_dim, dtype=np.uint16)
    rc = lib().orc_bucketize(W, out_dim, in_dim, b, s, p)
    if rc != 0:
        raise ValueError("bucketize: out_dim must be a multiple of 16")
    return b, s, p


def effort_quantile(effort):
    return lib().orc_effort_quantile(effort)


def find_cutoff(x, probes, quantile, exp_no=0, trace=False):
    tr = CutoffTrace()
    c = lib().orc_find_cutoff(np.ascontiguousarray(x, np.float32),
                              np.ascontiguousarray(probes, np.uint16), exp_no, quantile,
                              C.byref(tr))
    return (c, tr) if trace else c


def find_cutoff_imp(imp, quantile, trace=False):
    tr = CutoffTrace()
    c = lib().orc_find_cutoff_imp(np.ascontiguousarray(imp, np.float32), quantile, C.byref(tr))
    return (c, tr) if trace else c


def importance(x, probes, exp_no=0):
    out = np.empty(4096, dtype=np.float32)
    lib().orc_importance(np.ascontiguousarray(x, np.float32),
                         np.ascontiguousarray(probes, np.uint16), exp_no, out)
    return out


def select_rows(x, stats, cutoff, expert_rows, in_size, exp_no=0, channels=4):
    mask = np.empty(expert_rows, dtype=np.uint8)
    s = lib().orc_select_rows(np.ascontiguousarray(x, np.float32),
                              np.ascontiguousarray(stats, np.uint16).ravel(), channels,
                              exp_no, expert_rows, in_size, cutoff, mask)
    return mask, s


def select_rows_block(x, stats, cutoff, expert_rows, in_size, block, exp_no=0, channels=4):
    """Block-structured selection: blocks of `block` consecutive inputs share
    each rank's selection (block 1: select_rows)."""
    mask = np.empty(expert_rows, dtype=np.uint8)
    s = lib().orc_select_rows_block(np.ascontiguousarray(x, np.float32),
                                    np.ascontiguousarray(stats, np.uint16).ravel(), channels,
                                    exp_no, expert_rows, in_size, cutoff, block, mask)
    return mask, s


def bucket_walk(buckets, mask, x, expert_rows, exp_no=0, acc64=True):
    C_ = buckets.shape[-1]
    y = np.empty(16 * C_, dtype=np.float32)
    lib().orc_bucket_walk(np.ascontiguousarray(buckets, np.uint16).ravel(), C_, exp_no,
                          expert_rows, np.ascontiguousarray(mask, np.uint8),
                          np.ascontiguousarray(x, np.float32), y, 1 if acc64 else 0)
    return y


def bucketmul(x, stats, probes, buckets, effort, in_size=None, exp_no=0, acc64=True):
    buckets = np.ascontiguousarray(buckets, np.uint16)
    C_ = buckets.shape[-1]
    R = buckets.shape[-2]
    if in_size is None:
        in_size = R // 16
    y = np.empty(16 * C_, dtype=np.float32)
    mask = np.empty(R, dtype=np.uint8)
    cut = C.c_float()
    s = lib().orc_bucketmul(np.ascontiguousarray(x, np.float32),
                            np.ascontiguousarray(stats, np.uint16).ravel(),
                            np.ascontiguousarray(probes, np.uint16).ravel(), buckets.ravel(),
                            exp_no, in_size, C_, R, effort, y, C.byref(cut), mask,
                            1 if acc64 else 0)
    return y, cut.value, mask, s


def rmsnorm_gain(x, gain, eps=1e-5):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    lib().orc_rmsnorm_gain(x, np.ascontiguousarray(gain, np.uint16), x.size, eps, out)
    return out


def silu_mul(g, u):
    g = np.ascontiguousarray(g, np.float32)
    out = np.empty_like(g)
    lib().orc_silu_mul(g, np.ascontiguousarray(u, np.float32), g.size, out)
    return out


def rope_table(theta, head_dim, max_pos):
    t = np.empty((max_pos, head_dim // 2, 2), dtype=np.float32)
    lib().orc_rope_table(theta, head_dim, max_pos, t.ravel())
    return t


def rope(x, table_row, n_heads, head_dim):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    lib().orc_rope(x, np.ascontiguousarray(table_row, np.float32).ravel(), n_heads, head_dim, out)
    return out


def attention_f16kv(q, kcache, vcache, n_tok, n_heads, n_kv, head_dim):
    out = np.empty(n_heads * head_dim, dtype=np.float32)
    lib().orc_attention_f16kv(np.ascontiguousarray(q, np.float32),
                              np.ascontiguousarray(kcache, np.uint16).ravel(),
                              np.ascontiguousarray(vcache, np.uint16).ravel(), n_tok, n_heads,
                              n_kv, head_dim, out)
    return out


def attention_f32rep(q, kcache, vcache, n_tok, n_heads, head_dim):
    """The reference's fp32 attention over K, V [ctx][n_heads][head_dim] fp32
    (every query head's own copy of its KV head's rows)."""
    out = np.empty(n_heads * head_dim, dtype=np.float32)
    lib().orc_attention_f32rep(np.ascontiguousarray(q, np.float32),
                               np.ascontiguousarray(kcache, np.float32).ravel(),
                               np.ascontiguousarray(vcache, np.float32).ravel(), n_tok, n_heads, head_dim, out)
    return out


def rope_kv_rep32(q, k, v, table_row, n_heads, n_kv, head_dim):
    """(q after RoPE, the K row and the V row of one position repeated to
    n_heads heads), all fp32."""
    qo = np.empty(n_heads * head_dim, np.float32)
    kr = np.empty(n_heads * head_dim, np.float32)
    vr = np.empty(n_heads * head_dim, np.float32)
    lib().orc_rope_kv_rep32(np.ascontiguousarray(q, np.float32), np.ascontiguousarray(k, np.float32),
                            np.ascontiguousarray(v, np.float32),
                            np.ascontiguousarray(table_row, np.float32).ravel(), n_heads, n_kv, head_dim,
                            qo, kr, vr)
    return qo, kr, vr


def matmul_f16_dense(W, x):
    """matmul16x32: W uint16 (fp16 bits) [rows][cols] times x fp32 [cols]."""
    W = np.ascontiguousarray(W, np.uint16)
    rows, cols = W.shape
    out = np.empty(rows, np.float32)
    lib().orc_matmul_f16_dense(W.ravel(), np.ascontiguousarray(x, np.float32), rows, cols, out)
    return out


def argmax(v):
    return lib().orc_argmax(np.ascontiguousarray(v, np.float32), len(v))


class OracleModel:
    """An orc_model over host copies of a model's tensors.

    read(name, dtype) returns the named tensor (e.g. "layer0.wq.buckets") as a
    numpy array; cfg is a dict of ModelConfig fields.  The arrays are kept
    alive by this object."""

    MATS = ["wq", "wk", "wv", "wo", "w1", "w3", "w2"]

    def __init__(self, cfg, read, lm_dense=None):
        """lm_dense: the dense fp16 LM head [vocab][dim] (uint16), used by the
        forward instead of the bucket layout (matmul16x32)."""
        self.keep = []
        self.cfg = dict(cfg)
        c = self.cfg
        layers = (Layer * c["n_layers"])()
        for L in range(c["n_layers"]):
            for w in self.MATS:
                mat = getattr(layers[L], w)
                b = read(f"layer{L}.{w}.buckets", np.uint16)
                s = read(f"layer{L}.{w}.stats", np.uint16)
                p = read(f"layer{L}.{w}.probes", np.uint16)
                in_dim = s.size // 64
                mat.buckets, mat.stats, mat.probes = self._p(b), self._p(s), self._p(p)
                mat.in_dim, mat.out_dim = in_dim, b.size // in_dim
            layers[L].attn_gain = self._p(read(f"layer{L}.attn_gain", np.uint16))
            layers[L].ffn_gain = self._p(read(f"layer{L}.ffn_gain", np.uint16))
        self.layers = layers
        mod = Model()
        mod.cfg = ModelConfig(**c)
        mod.layers = C.cast(layers, C.c_void_p)
        mod.embed = self._p(read("embed", np.uint16))
        mod.final_gain = self._p(read("final_gain", np.uint16))
        if lm_dense is None:
            mod.lm_head.buckets = self._p(read("lm_head.buckets", np.uint16))
            mod.lm_head.stats = self._p(read("lm_head.stats", np.uint16))
            mod.lm_head.probes = self._p(read("lm_head.probes", np.uint16))
        mod.lm_head.in_dim, mod.lm_head.out_dim = c["dim"], c["vocab"]
        kv = c["n_layers"] * c["max_ctx"] * c["n_kv_heads"] * c["head_dim"]
        self.kc = np.zeros(kv, np.uint16)
        self.vc = np.zeros(kv, np.uint16)
        mod.kcache, mod.vcache = self._p(self.kc), self._p(self.vc)
        mod.rope = self._p(rope_table(c["rope_theta"], c["head_dim"], c["max_ctx"]))
        mod.lm_dense = None if lm_dense is None else self._p(np.ascontiguousarray(lm_dense, np.uint16))
        self.mod = mod

    def _p(self, a):
        a = np.ascontiguousarray(a)
        self.keep.append(a)
        return a.ctypes.data

    def forward(self, token, pos, effort, hidden_in=None):
        logits = np.empty(self.cfg["vocab"], np.float32)
        h = None
        if hidden_in is not None:
            hh = np.ascontiguousarray(hidden_in, np.float32)
            self.keep.append(hh)
            h = hh.ctypes.data
        lib().orc_model_forward(C.byref(self.mod), token, pos, effort, h, logits)
        return logits

    def layer_forward(self, layer, pos, effort, h):
        """orc_layer_forward on a copy of h; returns the layer output."""
        out = np.ascontiguousarray(h, np.float32).copy()
        lib().orc_layer_forward(C.byref(self.mod), layer, pos, effort, out)
        return out


def threads():
    """Threads of the oracle's parallel loops (OpenMP's maximum)."""
    return lib().orc_threads()


def set_selection_block(block, below_effort=2.0):
    """The selection of bucketmul and the layer/model forwards: blocks of
    `block` inputs for efforts below `below_effort` (1: per row)."""
    lib().orc_set_selection_block(int(block), float(below_effort))
