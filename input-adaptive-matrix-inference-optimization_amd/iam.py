"""ctypes binding of libiam.so (the C ABI declared in include/iam.h).

Used by the tests, __graft_entry__ and bench.py.  It loads the in-tree
library only and raises if it is missing: there is no fallback path.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libiam.so")
# a different build of the same library (e.g. another launch shape) may be
# named with IAM_LIBRARY
LIB_PATH = os.environ.get("IAM_LIBRARY", LIB_PATH)
HEADER = os.path.join(os.path.dirname(HERE), "include", "iam.h")

IAM_OK = 0
IAM_E_INVALID = -1
IAM_E_HIP = -2
IAM_E_NOMEM = -3
IAM_E_STATE = -4
IAM_E_IO = -5

_lib = None


class IamError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"iam error {code}: {msg}")
        self.code = code


class BucketMatrix(C.Structure):
    _fields_ = [("buckets", C.c_void_p), ("stats", C.c_void_p), ("probes", C.c_void_p),
                ("expert_rows", C.c_int), ("bucket_cols", C.c_int),
                ("stats_stride", C.c_int), ("stats_channel", C.c_int)]


class ModelConfig(C.Structure):
    _fields_ = [("n_layers", C.c_int), ("dim", C.c_int), ("ffn_dim", C.c_int),
                ("n_heads", C.c_int), ("n_kv_heads", C.c_int), ("head_dim", C.c_int),
                ("vocab", C.c_int), ("max_ctx", C.c_int), ("rope_theta", C.c_double),
                ("norm_eps", C.c_float)]


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"libiam.so not built: {LIB_PATH} (run __graft_entry__.build())")
        L = C.CDLL(LIB_PATH)
        L.iam_last_error.restype = C.c_char_p
        L.iam_effort_quantile.restype = C.c_int
        L.iam_effort_quantile.argtypes = [C.c_float]
        _lib = L
    return _lib


def last_error():
    return lib().iam_last_error().decode(errors="replace")


def check(rc):
    if rc != IAM_OK:
        raise IamError(rc, last_error())
    return rc


def header_symbols(path=HEADER):
    """Names of the functions declared in include/iam.h."""
    import re
    txt = open(path).read()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(iam_\w+)\s*\(", txt, re.M)))


def _vp(x):
    return C.c_void_p(x if isinstance(x, int) else x.ptr)


class DevBuf:
    """A device allocation owned by a Ctx."""

    def __init__(self, ctx, nbytes, dtype=np.uint8, shape=None):
        self.ctx = ctx
        self.nbytes = int(nbytes)
        self.dtype = np.dtype(dtype)
        self.shape = shape if shape is not None else (self.nbytes // self.dtype.itemsize,)
        p = C.c_void_p()
        check(lib().iam_alloc(ctx.h, C.c_size_t(self.nbytes), C.byref(p)))
        self.ptr = p.value

    def write(self, arr, offset=0):
        a = np.ascontiguousarray(arr)
        check(lib().iam_write(self.ctx.h, C.c_void_p(self.ptr), C.c_size_t(offset),
                              a.ctypes.data_as(C.c_void_p), C.c_size_t(a.nbytes)))
        return self

    def read(self, dtype=None, count=None, offset=0):
        dt = np.dtype(dtype) if dtype is not None else self.dtype
        n = count if count is not None else (self.nbytes - offset) // dt.itemsize
        out = np.empty(n, dtype=dt)
        check(lib().iam_read(self.ctx.h, out.ctypes.data_as(C.c_void_p), C.c_void_p(self.ptr),
                             C.c_size_t(offset), C.c_size_t(out.nbytes)))
        return out

    def zero(self):
        check(lib().iam_zero(self.ctx.h, C.c_void_p(self.ptr), C.c_size_t(0), C.c_size_t(self.nbytes)))
        return self

    def free(self):
        if self.ptr:
            check(lib().iam_free(self.ctx.h, C.c_void_p(self.ptr)))
            self.ptr = None


class Ctx:
    def __init__(self, device=0):
        h = C.c_void_p()
        check(lib().iam_ctx_create(device, C.byref(h)))
        self.h = h

    def close(self):
        if self.h:
            lib().iam_ctx_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    # ---- memory
    def copy(self, dst, src, nbytes, dst_offset=0, src_offset=0):
        """Device-to-device copy on the context's stream (asynchronous)."""
        check(lib().iam_copy(self.h, _vp(dst), C.c_size_t(dst_offset), _vp(src), C.c_size_t(src_offset),
                             C.c_size_t(nbytes)))

    def alloc(self, nbytes, dtype=np.uint8):
        return DevBuf(self, nbytes, dtype)

    def upload(self, arr):
        a = np.ascontiguousarray(arr)
        b = DevBuf(self, max(a.nbytes, 1), a.dtype, a.shape)
        if a.nbytes:
            b.write(a)
        return b

    def empty(self, n, dtype):
        dt = np.dtype(dtype)
        return DevBuf(self, max(n * dt.itemsize, 1), dt, (n,))

    def mem_status(self):
        """(bytes allocated through this context, usable bytes)."""
        a, u = C.c_size_t(), C.c_size_t()
        check(lib().iam_mem_status(self.h, C.byref(a), C.byref(u)))
        return a.value, u.value

    def sync(self):
        check(lib().iam_sync(self.h))

    def device_info(self):
        name = C.create_string_buffer(256)
        cus = C.c_int()
        mem = C.c_size_t()
        check(lib().iam_device_info(self.h, name, 256, C.byref(cus), C.byref(mem)))
        return name.value.decode(), cus.value, mem.value

    def profiling(self, on=True):
        check(lib().iam_profiling(self.h, 1 if on else 0))

    def kernel_stats(self):
        buf = C.create_string_buffer(1 << 16)
        check(lib().iam_kernel_stats(self.h, buf, len(buf)))
        return buf.value.decode()

    def kernel_stats_reset(self):
        check(lib().iam_kernel_stats_reset(self.h))

    def kernel_stat(self, name):
        t = C.c_double()
        n = C.c_int()
        check(lib().iam_kernel_stat(self.h, name.encode(), C.byref(t), C.byref(n)))
        return t.value, n.value

    # ---- bucketMul
    def calc_dispatch(self, x, stats, probes, expert_no, in_size, bucket_cols, expert_size, effort):
        check(lib().iam_bucketmul_calc_dispatch(self.h, _vp(x), _vp(stats), _vp(probes), expert_no,
                                                in_size, bucket_cols, expert_size, C.c_float(effort)))

    def mul(self, buckets, bucket_cols, y):
        check(lib().iam_bucketmul_mul(self.h, _vp(buckets), bucket_cols, _vp(y)))

    def full_mul(self, x, stats, probes, buckets, expert_no, in_size, bucket_cols, expert_size,
                 effort, y):
        check(lib().iam_bucketmul_full(self.h, _vp(x), _vp(stats), _vp(probes), _vp(buckets),
                                       expert_no, in_size, bucket_cols, expert_size,
                                       C.c_float(effort), _vp(y)))

    def multi(self, mats, xs, in_sizes, ys, effort, expert_no=0):
        n = len(mats)
        M = (BucketMatrix * n)(*mats)
        X = (C.c_void_p * n)(*[x.ptr if not isinstance(x, int) else x for x in xs])
        I = (C.c_int * n)(*in_sizes)
        Y = (C.c_void_p * n)(*[y.ptr if not isinstance(y, int) else y for y in ys])
        check(lib().iam_bucketmul_multi(self.h, n, M, X, I, Y, expert_no, C.c_float(effort)))

    def fused(self, mats, x, in_size, ys, effort, h=None, gain=None, eps=1e-5, expert_no=0):
        """One matrix group with the input (or RMSNorm(h) * gain, written to x)
        and the cutoff computed inside the walk."""
        n = len(mats)
        M = (BucketMatrix * n)(*mats)
        Y = (C.c_void_p * n)(*[y.ptr if not isinstance(y, int) else y for y in ys])
        check(lib().iam_bucketmul_fused(self.h, n, M, _vp(x), in_size, Y, expert_no, C.c_float(effort),
                                        _vp(h) if h is not None else None,
                                        _vp(gain) if gain is not None else None, C.c_float(eps)))

    def fused_noalloc(self, mats, x, in_size, ys, effort, h=None, gain=None, eps=1e-5, expert_no=0):
        """fused() with the scratch in the library's fixed per-GPU array: no
        device allocation during the call."""
        n = len(mats)
        M = (BucketMatrix * n)(*mats)
        Y = (C.c_void_p * n)(*[y.ptr if not isinstance(y, int) else y for y in ys])
        check(lib().iam_bucketmul_fused_noalloc(self.h, n, M, _vp(x), in_size, Y, expert_no, C.c_float(effort),
                                                _vp(h) if h is not None else None,
                                                _vp(gain) if gain is not None else None, C.c_float(eps)))

    def dispatch_info(self, slot=0):
        cut = C.c_float()
        cnt = C.c_uint32()
        check(lib().iam_bucketmul_dispatch_info(self.h, slot, C.byref(cut), C.byref(cnt)))
        return cut.value, cnt.value

    def dispatch_rows(self, slot=0, cap=None):
        cnt = C.c_uint32()
        check(lib().iam_bucketmul_dispatch_rows(self.h, slot, None, C.c_size_t(0), C.byref(cnt)))
        n = cnt.value if cap is None else min(cap, cnt.value)
        out = np.empty(max(n, 1), dtype=np.uint32)
        check(lib().iam_bucketmul_dispatch_rows(self.h, slot, out.ctypes.data_as(C.c_void_p),
                                                C.c_size_t(n), C.byref(cnt)))
        return out[:n]

    def set_accumulation(self, mode):
        """"fp64" (default) or "fp32"."""
        check(lib().iam_set_accumulation(self.h, {"fp32": 0, "fp64": 1}[mode]))

    def read_bandwidth(self, nbytes=2 << 30, reps=10):
        """Measured streaming-read bandwidth in GB/s."""
        g = C.c_double()
        check(lib().iam_read_bandwidth(self.h, C.c_size_t(nbytes), reps, C.byref(g)))
        return g.value

    def set_walk_counting(self, on):
        """Count the walk's selected rows (default on; off shortens each reduce)."""
        check(lib().iam_set_walk_counting(self.h, 1 if on else 0))

    def walk_group_hints(self, group):
        """(hinted cutoff searches, hits) of a walk group ('qkv', 'o', ...)
        since the counters' reset."""
        t, k = C.c_uint64(), C.c_uint64()
        check(lib().iam_walk_group_hints(self.h, self.WALK_GROUPS[group], C.byref(t), C.byref(k)))
        return t.value, k.value

    def set_search_hints(self, on):
        """Start each fused call's cutoff search from the slot's previous
        cutoff (same results; default off)."""
        check(lib().iam_set_search_hints(self.h, 1 if on else 0))

    def set_search_hint(self, slot, value):
        """Set matrix slot `slot`'s search hint (any float; unusable ones mean none)."""
        check(lib().iam_set_search_hint(self.h, int(slot), C.c_float(value)))

    def set_selection_block(self, block_inputs, below_effort=2.0):
        """Block-structured selection: blocks of `block_inputs` consecutive
        inputs share each rank's selection, for efforts below `below_effort`
        (1: the reference's per-row selection)."""
        check(lib().iam_set_selection_block(self.h, int(block_inputs), C.c_float(below_effort)))

    def get_selection_block(self):
        b, e = C.c_int(), C.c_float()
        check(lib().iam_get_selection_block(self.h, C.byref(b), C.byref(e)))
        return b.value, e.value

    def get_accumulation(self):
        m = C.c_int()
        check(lib().iam_get_accumulation(self.h, C.byref(m)))
        return "fp64" if m.value == 1 else "fp32"

    def walk_count(self, slot=0):
        """Rows selected by the last walk of the slot (counted in the kernel)."""
        n = C.c_uint32()
        check(lib().iam_bucketmul_walk_count(self.h, slot, C.byref(n)))
        return n.value

    def walk_counters(self, reset=False):
        b, r, m = C.c_uint64(), C.c_uint64(), C.c_uint64()
        check(lib().iam_walk_counters(self.h, C.byref(b), C.byref(r), C.byref(m), 1 if reset else 0))
        return b.value, r.value, m.value

    WALK_GROUPS = {"none": 0, "qkv": 1, "o": 2, "ffn13": 3, "ffn2": 4, "lm": 5}

    def walk_group_counters(self, group):
        """(weight bytes, rows, matrices) the model's walks of one matrix group
        ('qkv', 'o', 'ffn13', 'ffn2', 'lm'; 'none': standalone calls) added."""
        b, r, m = C.c_uint64(), C.c_uint64(), C.c_uint64()
        check(lib().iam_walk_group_counters(self.h, self.WALK_GROUPS[group], C.byref(b), C.byref(r),
                                            C.byref(m)))
        return b.value, r.value, m.value

    def stats_compact(self, stats, rows, stride=4, channel=3, out=None):
        if out is None:
            out = self.empty(rows, np.uint16)
        check(lib().iam_stats_compact(self.h, _vp(stats), C.c_size_t(rows), stride, channel, _vp(out)))
        return out

    # ---- layer ops
    def rmsnorm_gain(self, x, gain, n, eps, out):
        check(lib().iam_rmsnorm_gain(self.h, _vp(x), _vp(gain), n, C.c_float(eps), _vp(out)))

    def add_rmsnorm_gain(self, h, delta, gain, n, eps, out):
        check(lib().iam_add_rmsnorm_gain(self.h, _vp(h), _vp(delta), _vp(gain), n, C.c_float(eps), _vp(out)))

    def add(self, a, b, n, out):
        check(lib().iam_add(self.h, _vp(a), _vp(b), n, _vp(out)))

    def silu_mul(self, g, u, n, out):
        check(lib().iam_silu_mul(self.h, _vp(g), _vp(u), n, _vp(out)))

    def rope(self, x, table, pos_dev, n_heads, head_dim, out):
        check(lib().iam_rope(self.h, _vp(x), _vp(table), _vp(pos_dev), n_heads, head_dim, _vp(out)))

    def rope_kv_append(self, q, k, v, table, pos_dev, n_heads, n_kv, head_dim, max_ctx, q_out, kc, vc):
        check(lib().iam_rope_kv_append(self.h, _vp(q), _vp(k), _vp(v), _vp(table), _vp(pos_dev),
                                       n_heads, n_kv, head_dim, max_ctx, _vp(q_out), _vp(kc), _vp(vc)))

    def attention(self, q, kc, vc, pos_dev, n_heads, n_kv, head_dim, max_ctx, out):
        check(lib().iam_attention_decode(self.h, _vp(q), _vp(kc), _vp(vc), _vp(pos_dev), n_heads,
                                         n_kv, head_dim, max_ctx, _vp(out)))

    def rope_kv_append_f32(self, q, k, v, table, pos_dev, n_heads, n_kv, head_dim, max_ctx, q_out, kc, vc):
        """RoPE + append into the reference's fp32 cache layout (K and V
        repeated to every query head)."""
        check(lib().iam_rope_kv_append_f32(self.h, _vp(q), _vp(k), _vp(v), _vp(table), _vp(pos_dev),
                                           n_heads, n_kv, head_dim, max_ctx, _vp(q_out), _vp(kc), _vp(vc)))

    def attention_f32(self, q, kc, vc, pos_dev, n_heads, head_dim, max_ctx, out):
        """The reference's fp32 attention over its repeated-head fp32 caches."""
        check(lib().iam_attention_decode_f32(self.h, _vp(q), _vp(kc), _vp(vc), _vp(pos_dev), n_heads,
                                             head_dim, max_ctx, _vp(out)))

    def matmul_f16_dense(self, w, x, rows, cols, out):
        """matmul16x32: the reference's dense fp16 GEMV."""
        check(lib().iam_matmul_f16_dense(self.h, _vp(w), _vp(x), rows, cols, _vp(out)))

    def embed(self, table, cols, vocab, token_dev, out):
        check(lib().iam_embed_gather(self.h, _vp(table), cols, vocab, _vp(token_dev), _vp(out)))

    def argmax(self, v, n, out_dev):
        check(lib().iam_argmax(self.h, _vp(v), n, _vp(out_dev)))

    # ---- synthetic data
    def gen_f16(self, seed, tid, count, mean, sigma, out):
        check(lib().iam_gen_f16(self.h, C.c_uint64(seed), C.c_uint64(tid), C.c_size_t(count),
                                C.c_double(mean), C.c_double(sigma), _vp(out)))

    def gen_f32(self, seed, tid, count, mean, sigma, out):
        check(lib().iam_gen_f32(self.h, C.c_uint64(seed), C.c_uint64(tid), C.c_size_t(count),
                                C.c_double(mean), C.c_double(sigma), _vp(out)))

    def bucketize(self, w, out_dim, in_dim, buckets, stats, probes):
        check(lib().iam_bucketize(self.h, _vp(w), out_dim, in_dim, _vp(buckets), _vp(stats), _vp(probes)))


def rope_table(theta, head_dim, max_pos):
    t = np.empty((max_pos, head_dim // 2, 2), dtype=np.float32)
    check(lib().iam_rope_table(C.c_double(theta), head_dim, max_pos, t.ctypes.data_as(C.c_void_p)))
    return t


def effort_quantile(effort):
    return lib().iam_effort_quantile(C.c_float(effort))


class Model:
    """iam_model_* wrapper."""

    def __init__(self, ctx, cfg: ModelConfig):
        self.ctx = ctx
        self.cfg = cfg
        h = C.c_void_p()
        check(lib().iam_model_create(ctx.h, C.byref(cfg), C.byref(h)))
        self.h = h

    def close(self):
        if self.h:
            check(lib().iam_model_destroy(self.h))
            self.h = None

    def synthesize(self, seed):
        check(lib().iam_model_synthesize(self.h, C.c_uint64(seed)))

    def forward(self, token, pos, effort, logits_dev):
        check(lib().iam_model_forward(self.h, token, pos, C.c_float(effort), _vp(logits_dev)))

    def step_device(self, effort, hidden_override=None):
        check(lib().iam_model_step_device(self.h, C.c_float(effort),
                                          None if hidden_override is None else _vp(hidden_override)))

    def generate(self, prompt, n_new, effort, use_graph=True):
        p = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.empty(max(n_new, 1), dtype=np.int32)
        check(lib().iam_model_generate(self.h, p.ctypes.data_as(C.c_void_p), len(p), n_new,
                                       C.c_float(effort), 1 if use_graph else 0,
                                       out.ctypes.data_as(C.c_void_p)))
        return out[:n_new]

    def decode(self, n_steps, effort, use_graph=True):
        check(lib().iam_model_decode(self.h, n_steps, C.c_float(effort), 1 if use_graph else 0))

    def set_position(self, pos):
        check(lib().iam_model_set_position(self.h, int(pos)))

    def set_lm_dense(self, w_dev):
        """The LM head as the reference's dense fp16 product over w_dev
        ([vocab][dim] fp16 on the device); None: the bucket layout."""
        check(lib().iam_model_set_lm_dense(self.h, None if w_dev is None else _vp(w_dev)))

    def set_embed_scale(self, scale):
        if scale is None:
            check(lib().iam_model_set_embed_scale(self.h, None))
        else:
            a = np.ascontiguousarray(scale, np.float32)
            check(lib().iam_model_set_embed_scale(self.h, a.ctypes.data_as(C.c_void_p)))

    def reset_caches(self):
        check(lib().iam_model_reset_caches(self.h))

    def tensor(self, name):
        p = C.c_void_p()
        n = C.c_size_t()
        check(lib().iam_model_tensor(self.h, name.encode(), C.byref(p), C.byref(n)))
        return p.value, n.value

    def read_tensor(self, name, dtype):
        p, n = self.tensor(name)
        dt = np.dtype(dtype)
        out = np.empty(n // dt.itemsize, dtype=dt)
        check(lib().iam_read(self.ctx.h, out.ctypes.data_as(C.c_void_p), C.c_void_p(p),
                             C.c_size_t(0), C.c_size_t(out.nbytes)))
        return out

    def write_tensor(self, name, arr):
        p, n = self.tensor(name)
        a = np.ascontiguousarray(arr)
        assert a.nbytes <= n, (name, a.nbytes, n)
        check(lib().iam_write(self.ctx.h, C.c_void_p(p), C.c_size_t(0), a.ctypes.data_as(C.c_void_p),
                              C.c_size_t(a.nbytes)))

    def matrix(self, name):
        m = BucketMatrix()
        check(lib().iam_model_matrix(self.h, name.encode(), C.byref(m)))
        return m
