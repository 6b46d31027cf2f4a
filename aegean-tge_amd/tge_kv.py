"""Python binding of libtge_kv.so (include/tge_kv.h) over ctypes.

The library is the product: gfx950 kernels for the paged-KV append, decode
attention and chunked-prefill attention of the reference engine's Qwen2
KV path, its C ABI and the C++20 Qwen2-shaped driver. This module only binds
it. Device memory, copies and timing go through the system HIP runtime
(libamdhip64, loaded by the library itself); there is no CPU fallback: if the
library is missing or the GPU is unavailable, calls raise.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtge_kv.so")

PAGE_TOKENS = 16
OK, ERR_INVALID, ERR_RUNTIME, ERR_UNAVAILABLE, ERR_DEVICE, ERR_CAPACITY = 0, -1, -2, -3, -4, -5
KV_F16, KV_I8 = 1, 2
SCALE_F16, SCALE_F32 = 0, 1

_lib = None
_hip = None


class TgeError(RuntimeError):
    def __init__(self, status, message):
        super().__init__(f"{message} (status {status})")
        self.status = status


class PoolDesc(C.Structure):
    _fields_ = [("layers", C.c_int), ("pages", C.c_int), ("kv_heads", C.c_int),
                ("head_dim", C.c_int), ("format", C.c_int), ("scale_format", C.c_int)]


class LayerView(C.Structure):
    _fields_ = [("k", C.c_void_p), ("v", C.c_void_p), ("k_scales", C.c_void_p),
                ("v_scales", C.c_void_p), ("kv_block_bytes", C.c_size_t),
                ("scale_block_bytes", C.c_size_t), ("block_bytes", C.c_size_t),
                ("block_dims", C.c_int)]


class BatchDesc(C.Structure):
    _fields_ = [("n_sessions", C.c_int), ("ctx", C.POINTER(C.c_int)),
                ("n_new", C.POINTER(C.c_int)), ("table_offsets", C.POINTER(C.c_int)),
                ("page_ids", C.POINTER(C.c_int)), ("q_heads", C.c_int)]


class Qwen2Config(C.Structure):
    _fields_ = [("layers", C.c_int), ("q_heads", C.c_int), ("kv_heads", C.c_int),
                ("head_dim", C.c_int), ("context", C.c_int), ("sequences", C.c_int),
                ("pages", C.c_int), ("format", C.c_int), ("scale_format", C.c_int)]


# (name, restype, argtypes) of every symbol include/tge_kv.h declares.
_VP, _I, _PI = C.c_void_p, C.c_int, C.POINTER(C.c_int)
class AttentionGroupArgs(C.Structure):
    """tge_attention_group_args (AttentionGroupArgs over pages)."""
    _fields_ = [("pool", C.c_void_p), ("layer", C.c_int), ("kv_head", C.c_int),
                ("page_ids", C.c_void_p), ("first", C.c_int), ("count", C.c_int),
                ("queries", C.c_void_p), ("group_heads", C.c_int), ("scale", C.c_float),
                ("maxima", C.c_void_p), ("sums", C.c_void_p), ("accumulators", C.c_void_p)]


class RopeAppendArgs(C.Structure):
    _fields_ = [("q", C.c_void_p), ("q_out", C.c_void_p), ("k", C.c_void_p), ("v", C.c_void_p),
                ("q_bias", C.c_void_p), ("k_bias", C.c_void_p), ("v_bias", C.c_void_p),
                ("rope_cos", C.c_void_p), ("rope_sin", C.c_void_p),
                ("rope_positions", C.c_int), ("rope_fma", C.c_int)]


def rope_args(k, v, rope_cos, rope_sin, positions, q=None, q_out=None, q_bias=None, k_bias=None,
              v_bias=None, fma=True):
    """tge_rope_append_args from DeviceArrays (or raw addresses / None)."""
    def ptr(a):
        return None if a is None else (a if isinstance(a, int) else a.ptr)
    return RopeAppendArgs(ptr(q), ptr(q_out), ptr(k), ptr(v), ptr(q_bias), ptr(k_bias),
                          ptr(v_bias), ptr(rope_cos), ptr(rope_sin), int(positions), int(bool(fma)))


def rope_tables(head_dim, positions, theta=10000.0, attn_factor=1.0, factors=None):
    """Host rotary tables (tge_rope_tables): cos, sin as [positions][head_dim/2]."""
    half = head_dim // 2
    c = np.empty((positions, half), np.float32)
    s = np.empty((positions, half), np.float32)
    f = None if factors is None else np.ascontiguousarray(factors, dtype=np.float32)
    check(lib().tge_rope_tables(head_dim, positions, theta, attn_factor,
                                None if f is None else f.ctypes.data_as(C.c_void_p),
                                c.ctypes.data_as(C.c_void_p), s.ctypes.data_as(C.c_void_p)),
          "rope_tables")
    return c, s


SIGNATURES = [
    ("tge_status_string", C.c_char_p, [_I]),
    ("tge_last_error", C.c_char_p, []),
    ("tge_backend_init", _I, []),
    ("tge_backend_arch", C.c_char_p, []),
    ("tge_kv_pool_create", _I, [C.POINTER(PoolDesc), C.POINTER(_VP)]),
    ("tge_kv_pool_destroy", None, [_VP]),
    ("tge_kv_pool_layer", _I, [_VP, _I, C.POINTER(LayerView)]),
    ("tge_kv_pool_bytes", C.c_size_t, [_VP]),
    ("tge_kv_copy_page", _I, [_VP, _I, _I, _VP]),
    ("tge_kv_append_rope", _I, [_VP, _VP, _I, C.POINTER(RopeAppendArgs), _VP]),
    ("tge_eligible_gqa", _I, [_I, _I, _I, _I, _I]),
    ("tge_attention_group", _I, [C.POINTER(AttentionGroupArgs), _VP]),
    ("tge_batch_attention", _I, [_VP, _VP, _I, _VP, _VP, _VP]),
    ("tge_batch_set_sparse", _I, [_VP, _I, _I, _I, _I]),
    ("tge_rope_tables", _I, [_I, _I, C.c_float, C.c_float, _VP, _VP, _VP]),
    ("tge_qwen2_kv_layer_rope", _I, [_VP, _I, C.POINTER(RopeAppendArgs), _VP, _VP]),
    ("tge_kv_k_index", _I, [_I, _I, _I]),
    ("tge_kv_v_index", _I, [_I, _I, _I]),
    ("tge_kv_scale_index", _I, [_I, _I, _I]),
    ("tge_batch_create", _I, [C.POINTER(_VP)]),
    ("tge_batch_destroy", None, [_VP]),
    ("tge_batch_plan", _I, [_VP, _VP, C.POINTER(BatchDesc), _VP]),
    ("tge_batch_info", _I, [_VP, _PI, _PI, _PI]),
    ("tge_batch_set_profiling", _I, [_VP, _I]),
    ("tge_batch_kernel_times", _I, [_VP, _PI, C.POINTER(C.c_float), C.POINTER(C.c_float)]),
    ("tge_kv_append", _I, [_VP, _VP, _I, _VP, _VP, _VP]),
    ("tge_decode_attention", _I, [_VP, _VP, _I, _VP, _VP, _VP]),
    ("tge_decode_step", _I, [_VP, _VP, _I, _VP, _VP, _VP, _VP, _VP]),
    ("tge_batch_step_info", _I, [_VP, _PI, _PI]),
    ("tge_decode_attention_static", _I, [C.POINTER(BatchDesc), _VP, _I, _VP, _VP, _VP]),
    ("tge_prefill_attention", _I, [_VP, _VP, _I, _VP, _VP, _VP]),
    ("tge_kv_gather", _I, [_VP, _VP, _I, _I, _I, _VP, _VP, _VP, _VP, _VP]),
    ("tge_block_table_create", _I, [_I, _I, C.POINTER(_VP)]),
    ("tge_block_table_destroy", None, [_VP]),
    ("tge_block_table_allocate", _I, [_VP, _PI]),
    ("tge_block_table_share", _I, [_VP, _I]),
    ("tge_block_table_release", _I, [_VP, _I]),
    ("tge_block_table_refcount", _I, [_VP, _I, _PI]),
    ("tge_block_table_free_count", _I, [_VP]),
    ("tge_block_table_capacity", _I, [_VP]),
    ("tge_block_table_remember_prefix", _I, [_VP, C.c_uint64, _I]),
    ("tge_block_table_find_prefix", _I, [_VP, C.c_uint64]),
    ("tge_slot_for", _I, [_I, _I, _PI, _PI]),
    ("tge_hash_tokens", _I, [_PI, _I, C.POINTER(C.c_uint64)]),
    ("tge_qwen2_kv_create", _I, [C.POINTER(Qwen2Config), C.POINTER(_VP)]),
    ("tge_qwen2_kv_destroy", None, [_VP]),
    ("tge_qwen2_kv_begin_forward", _I, [_VP, _I, _I, _VP]),
    ("tge_qwen2_kv_begin_forward_batch", _I, [_VP, _PI, _I, _PI, _VP]),
    ("tge_qwen2_kv_begin_prefill", _I, [_VP, _I, _I, _I, _VP]),
    ("tge_qwen2_kv_begin_verify", _I, [_VP, _I, _I, _I, _VP]),
    ("tge_qwen2_kv_layer", _I, [_VP, _I, _VP, _VP, _VP, _VP, _VP]),
    ("tge_qwen2_kv_store", _I, [_VP, _I, _VP, _VP, _VP]),
    ("tge_qwen2_kv_reset", _I, [_VP, _I]),
    ("tge_qwen2_kv_length", _I, [_VP, _I]),
    ("tge_qwen2_kv_pages", _I, [_VP, _I, _PI, _I]),
    ("tge_qwen2_kv_pool", _VP, [_VP]),
    ("tge_qwen2_kv_batch", _VP, [_VP]),
    ("tge_qwen2_kv_free_pages", _I, [_VP]),
    ("tge_qwen2_kv_table", _VP, [_VP]),
    ("tge_qwen2_kv_set_sparse", _I, [_VP, _I, _I, _I, _I]),
    ("tge_qwen2_kv_remember_prefix", _I, [_VP, _I, _PI, _I]),
    ("tge_qwen2_kv_shared_prefix_len", _I, [_VP, _PI, _I]),
    ("tge_qwen2_kv_attach_prefix", _I, [_VP, _I, _PI, _I]),
    ("tge_read_ceiling", _I, [_VP, C.c_size_t, _I, _I, _I, _VP]),
    ("tge_batch_decode_stores_rows", _I, [_VP, C.POINTER(C.c_int)]),
    ("tge_wait_expiries", _I, [C.POINTER(C.c_uint)]),
]


def lib():
    """Loads libtge_kv.so (built in-tree by __graft_entry__.build())."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it (make -C aegean-tge_amd)")
        L = C.CDLL(LIB_PATH)
        for name, res, args in SIGNATURES:
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def attention_group(pool, layer, kv_head, page_ids, first, count, queries, scale=None,
                    stream=None):
    """tge_attention_group for one KV head's query group over positions
    [first, first + count): page_ids (host ints) and queries ([group][head_dim]
    fp32, host) are copied to the device; returns (maxima, sums,
    accumulators) as numpy arrays after synchronising."""
    q = np.ascontiguousarray(queries, np.float32)
    g = q.shape[0]
    ids = DeviceArray.from_numpy(np.ascontiguousarray(page_ids, np.int32))
    dq = DeviceArray.from_numpy(q)
    m = DeviceArray((g,), np.float32)
    sm = DeviceArray((g,), np.float32)
    acc = DeviceArray((g, pool.head_dim), np.float32)
    a = AttentionGroupArgs(pool.h, layer, kv_head, ids.ptr, first, count, dq.ptr, g,
                           float(1.0 / np.sqrt(pool.head_dim)) if scale is None else float(scale),
                           m.ptr, sm.ptr, acc.ptr)
    try:
        check(lib().tge_attention_group(C.byref(a), stream), "attention_group")
        hip().sync()
        return m.numpy(), sm.numpy(), acc.numpy()
    finally:
        for x in (ids, dq, m, sm, acc):
            x.close()


def check(status, what=""):
    if status != OK:
        msg = lib().tge_last_error().decode(errors="replace")
        raise TgeError(status, f"{what}: {msg}" if what else msg)
    return status


def backend_ready():
    return lib().tge_backend_init() == OK


def require_gpu():
    check(lib().tge_backend_init(), "tge_backend_init")


# ---------------------------------------------------------------------------
# Minimal HIP runtime access (device memory, copies, events, streams).
# ---------------------------------------------------------------------------
class Hip:
    H2D, D2H, D2D = 1, 2, 3

    def __init__(self):
        lib()  # libtge_kv.so pulls in the system libamdhip64 first
        h = C.CDLL("libamdhip64.so.7")
        h.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
        h.hipFree.argtypes = [C.c_void_p]
        h.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        h.hipMemcpyAsync.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int, C.c_void_p]
        h.hipMemset.argtypes = [C.c_void_p, C.c_int, C.c_size_t]
        h.hipDeviceSynchronize.argtypes = []
        h.hipStreamSynchronize.argtypes = [C.c_void_p]
        h.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
        h.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
        h.hipEventSynchronize.argtypes = [C.c_void_p]
        h.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
        h.hipEventDestroy.argtypes = [C.c_void_p]
        h.hipStreamCreate.argtypes = [C.POINTER(C.c_void_p)]
        h.hipStreamDestroy.argtypes = [C.c_void_p]
        h.hipGetErrorString.restype = C.c_char_p
        h.hipGetErrorString.argtypes = [C.c_int]
        h.hipMemGetInfo.argtypes = [C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]
        self.h = h

    def ok(self, e, what):
        if e != 0:
            raise TgeError(ERR_DEVICE, f"{what}: {self.h.hipGetErrorString(e).decode()}")

    def malloc(self, nbytes):
        p = C.c_void_p()
        self.ok(self.h.hipMalloc(C.byref(p), max(int(nbytes), 1)), "hipMalloc")
        return p.value

    def free(self, p):
        if p:
            self.ok(self.h.hipFree(C.c_void_p(p)), "hipFree")

    def upload(self, dst, arr):
        arr = np.ascontiguousarray(arr)
        self.ok(self.h.hipMemcpy(C.c_void_p(dst), arr.ctypes.data_as(C.c_void_p), arr.nbytes,
                                 self.H2D), "hipMemcpy H2D")

    def download(self, src, arr):
        assert arr.flags["C_CONTIGUOUS"]
        self.ok(self.h.hipMemcpy(arr.ctypes.data_as(C.c_void_p), C.c_void_p(src), arr.nbytes,
                                 self.D2H), "hipMemcpy D2H")
        return arr

    def memset(self, p, value, nbytes):
        self.ok(self.h.hipMemset(C.c_void_p(p), value, nbytes), "hipMemset")

    def sync(self):
        self.ok(self.h.hipDeviceSynchronize(), "hipDeviceSynchronize")

    def event(self):
        e = C.c_void_p()
        self.ok(self.h.hipEventCreate(C.byref(e)), "hipEventCreate")
        return e.value

    def record(self, ev, stream=None):
        self.ok(self.h.hipEventRecord(C.c_void_p(ev), C.c_void_p(stream)), "hipEventRecord")

    def elapsed_ms(self, a, b):
        self.ok(self.h.hipEventSynchronize(C.c_void_p(b)), "hipEventSynchronize")
        ms = C.c_float()
        self.ok(self.h.hipEventElapsedTime(C.byref(ms), C.c_void_p(a), C.c_void_p(b)),
                "hipEventElapsedTime")
        return ms.value

    def mem_info(self):
        free, total = C.c_size_t(), C.c_size_t()
        self.ok(self.h.hipMemGetInfo(C.byref(free), C.byref(total)), "hipMemGetInfo")
        return free.value, total.value


_hip_inst = None


def hip():
    global _hip_inst
    if _hip_inst is None:
        _hip_inst = Hip()
    return _hip_inst


class DeviceArray:
    """A device allocation with a numpy shape/dtype, freed on close()."""

    def __init__(self, shape, dtype):
        self.shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        self.ptr = hip().malloc(self.nbytes)

    @classmethod
    def from_numpy(cls, arr):
        arr = np.ascontiguousarray(arr)
        d = cls(arr.shape, arr.dtype)
        hip().upload(d.ptr, arr)
        return d

    def numpy(self):
        return hip().download(self.ptr, np.empty(self.shape, self.dtype))

    def zero(self):
        hip().memset(self.ptr, 0, self.nbytes)
        return self

    def close(self):
        if self.ptr:
            hip().free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _ints(values):
    arr = (C.c_int * max(len(values), 1))(*[int(v) for v in values])
    return arr


# ---------------------------------------------------------------------------
# Object wrappers
# ---------------------------------------------------------------------------
class BlockTable:
    """tge_block_table_*: the reference BlockTable's behaviour (host side)."""

    def __init__(self, blocks, block_tokens=PAGE_TOKENS, view=None):
        self.owned = view is None
        if view is not None:
            self.h = C.c_void_p(view)
            return
        h = C.c_void_p()
        check(lib().tge_block_table_create(blocks, block_tokens, C.byref(h)), "BlockTable")
        self.h = h

    def allocate(self):
        out = C.c_int()
        check(lib().tge_block_table_allocate(self.h, C.byref(out)), "allocate")
        return out.value

    def share(self, block):
        check(lib().tge_block_table_share(self.h, block), "share")

    def release(self, block):
        check(lib().tge_block_table_release(self.h, block), "release")

    def refcount(self, block):
        out = C.c_int()
        check(lib().tge_block_table_refcount(self.h, block, C.byref(out)), "refcount")
        return out.value

    def free_count(self):
        return lib().tge_block_table_free_count(self.h)

    def capacity(self):
        return lib().tge_block_table_capacity(self.h)

    def remember_prefix(self, hash_value, block):
        check(lib().tge_block_table_remember_prefix(self.h, C.c_uint64(hash_value), block),
              "remember_prefix")

    def find_prefix(self, hash_value):
        return lib().tge_block_table_find_prefix(self.h, C.c_uint64(hash_value))

    @staticmethod
    def slot_for(pos, block_tokens=PAGE_TOKENS):
        b, o = C.c_int(), C.c_int()
        check(lib().tge_slot_for(pos, block_tokens, C.byref(b), C.byref(o)), "slot_for")
        return b.value, o.value

    @staticmethod
    def hash_tokens(tokens):
        out = C.c_uint64()
        arr = _ints(tokens) if len(tokens) else None
        check(lib().tge_hash_tokens(arr, len(tokens), C.byref(out)), "hash_tokens")
        return out.value

    def fragment(self, seed):
        """Allocate every free page, then release them in a seeded random
        order: later allocations pop scattered ids (LIFO)."""
        ids = [self.allocate() for _ in range(self.free_count())]
        for i in np.random.default_rng(seed).permutation(len(ids)):
            self.release(ids[int(i)])
        return self

    def close(self):
        if self.h and self.owned:
            lib().tge_block_table_destroy(self.h)
        self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class KvPool:
    def __init__(self, layers, pages, kv_heads, head_dim, fmt=KV_F16, scale_format=SCALE_F16):
        self.desc = PoolDesc(layers, pages, kv_heads, head_dim, fmt, scale_format)
        h = C.c_void_p()
        check(lib().tge_kv_pool_create(C.byref(self.desc), C.byref(h)), "kv_pool_create")
        self.h = h
        self.layers, self.pages, self.kv_heads, self.head_dim = layers, pages, kv_heads, head_dim
        self.format, self.scale_format = fmt, scale_format

    def layer(self, layer):
        v = LayerView()
        check(lib().tge_kv_pool_layer(self.h, layer, C.byref(v)), "kv_pool_layer")
        return v

    def bytes(self):
        return lib().tge_kv_pool_bytes(self.h)

    def copy_page(self, src, dst, stream=None):
        check(lib().tge_kv_copy_page(self.h, src, dst, stream), "kv_copy_page")

    def close(self):
        if self.h:
            lib().tge_kv_pool_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


@dataclass
class Session:
    ctx: int
    n_new: int
    pages: list


def batch_info(handle):
    """(rows, decode work items, max splits) of a planned tge_batch handle."""
    r, w, s = C.c_int(), C.c_int(), C.c_int()
    check(lib().tge_batch_info(handle, C.byref(r), C.byref(w), C.byref(s)), "batch_info")
    return r.value, w.value, s.value


def batch_desc(sessions, q_heads):
    """A tge_batch_desc over `sessions` (Session records) and the int arrays
    it points to (keep them alive while the descriptor is used)."""
    ctx = [s.ctx for s in sessions]
    n_new = [s.n_new for s in sessions]
    offs = [0]
    ids = []
    for s in sessions:
        ids.extend(int(p) for p in s.pages)
        offs.append(len(ids))
    keep = (_ints(ctx), _ints(n_new), _ints(offs), _ints(ids))
    return BatchDesc(len(sessions), keep[0], keep[1], keep[2], keep[3], q_heads), keep


def wait_expiries():
    """tge_wait_expiries: bounded in-kernel waits that ran out so far."""
    n = C.c_uint()
    check(lib().tge_wait_expiries(C.byref(n)), "wait_expiries")
    return n.value


def decode_attention_static(pool, sessions, q_heads, layer, q, out, stream=None):
    """tge_decode_attention_static: plan and decode one step with no
    allocation (plan and partials in the library's static device array)."""
    d, keep = batch_desc(sessions, q_heads)
    check(lib().tge_decode_attention_static(C.byref(d), pool.h, layer, q.ptr, out.ptr, stream),
          "decode_attention_static")
    del keep


class Batch:
    def __init__(self):
        h = C.c_void_p()
        check(lib().tge_batch_create(C.byref(h)), "batch_create")
        self.h = h
        self.sessions = []

    def plan(self, pool, sessions, q_heads, stream=None):
        ctx = [s.ctx for s in sessions]
        n_new = [s.n_new for s in sessions]
        offs = [0]
        ids = []
        for s in sessions:
            ids.extend(int(p) for p in s.pages)
            offs.append(len(ids))
        self._keep = (_ints(ctx), _ints(n_new), _ints(offs), _ints(ids))
        d = BatchDesc(len(sessions), self._keep[0], self._keep[1], self._keep[2], self._keep[3],
                      q_heads)
        check(lib().tge_batch_plan(self.h, pool.h, C.byref(d), stream), "batch_plan")
        self.sessions = list(sessions)
        self.rows = sum(n_new)
        return self

    def info(self):
        return batch_info(self.h)

    def set_sparse(self, sink=4, window=512, stride=4, enabled=True):
        """Static sparse attention (tge_batch_set_sparse); enabled=False: dense."""
        check(lib().tge_batch_set_sparse(self.h, int(bool(enabled)), sink, window, stride),
              "batch_set_sparse")
        return self

    def set_profiling(self, enable):
        check(lib().tge_batch_set_profiling(self.h, int(bool(enable))), "batch_set_profiling")

    def kernel_times(self):
        """(calls, attention kernel us, merge kernel us) summed over the
        attention calls since profiling was enabled."""
        n, a, m = C.c_int(), C.c_float(), C.c_float()
        check(lib().tge_batch_kernel_times(self.h, C.byref(n), C.byref(a), C.byref(m)),
              "batch_kernel_times")
        return n.value, a.value, m.value

    def append(self, pool, layer, k, v, stream=None):
        check(lib().tge_kv_append(self.h, pool.h, layer, k.ptr, v.ptr, stream), "kv_append")

    def append_rope(self, pool, layer, args, stream=None):
        """tge_kv_append_rope with a RopeAppendArgs (see rope_args)."""
        check(lib().tge_kv_append_rope(self.h, pool.h, layer, C.byref(args), stream),
              "kv_append_rope")

    def decode(self, pool, layer, q, out, stream=None):
        check(lib().tge_decode_attention(self.h, pool.h, layer, q.ptr, out.ptr, stream),
              "decode_attention")

    def step_info(self):
        """tge_batch_step_info: (workgroups, max pieces) of the one-kernel
        step, (0, 0) when the step runs the append and decode kernels."""
        w, m = C.c_int(), C.c_int()
        check(lib().tge_batch_step_info(self.h, C.byref(w), C.byref(m)), "batch_step_info")
        return w.value, m.value

    def decode_stores_rows(self):
        """tge_batch_decode_stores_rows: True when tge_decode_step runs the
        current plan as one decode launch that also stores the new rows."""
        x = C.c_int()
        check(lib().tge_batch_decode_stores_rows(self.h, C.byref(x)), "batch_decode_stores_rows")
        return bool(x.value)

    def decode_step(self, pool, layer, q, k, v, out, stream=None):
        """tge_decode_step: append the step's K/V rows, then decode attention
        (one kernel for a small step)."""
        check(lib().tge_decode_step(self.h, pool.h, layer, q.ptr, k.ptr, v.ptr, out.ptr, stream),
              "decode_step")

    def attention(self, pool, layer, q, out, stream=None):
        """tge_batch_attention: decode kernel for short sessions, prefill kernel for the rest."""
        check(lib().tge_batch_attention(self.h, pool.h, layer, q.ptr, out.ptr, stream),
              "batch_attention")

    def prefill(self, pool, layer, q, out, stream=None):
        check(lib().tge_prefill_attention(self.h, pool.h, layer, q.ptr, out.ptr, stream),
              "prefill_attention")

    def gather(self, pool, layer, session, count):
        """Positions [0, count) of a session as flat rows (codes/bits, scales)."""
        kv_dim = pool.kv_heads * pool.head_dim
        et = np.uint16 if pool.format == KV_F16 else np.int8
        k = DeviceArray((count, kv_dim), et)
        v = DeviceArray((count, kv_dim), et)
        ks = vs = None
        if pool.format == KV_I8:
            st = np.float32 if pool.scale_format == SCALE_F32 else np.uint16
            ks = DeviceArray((count, kv_dim // 32), st)
            vs = DeviceArray((count, kv_dim // 32), st)
        check(lib().tge_kv_gather(self.h, pool.h, layer, session, count, k.ptr, v.ptr,
                                  ks.ptr if ks else None, vs.ptr if vs else None, None),
              "kv_gather")
        hip().sync()
        res = (k.numpy(), v.numpy(), ks.numpy() if ks else None, vs.numpy() if vs else None)
        for a in (k, v, ks, vs):
            if a is not None:
                a.close()
        return res

    def close(self):
        if self.h:
            lib().tge_batch_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Qwen2KvPath:
    """tge_qwen2_kv_*: the Qwen2-shaped store-then-attend driver."""

    def __init__(self, layers, q_heads, kv_heads, head_dim, context=4096, sequences=1, pages=0,
                 fmt=KV_F16, scale_format=SCALE_F16):
        self.cfg = Qwen2Config(layers, q_heads, kv_heads, head_dim, context, sequences, pages,
                               fmt, scale_format)
        h = C.c_void_p()
        check(lib().tge_qwen2_kv_create(C.byref(self.cfg), C.byref(h)), "qwen2_kv_create")
        self.h = h

    def begin_forward(self, sequence, position):
        check(lib().tge_qwen2_kv_begin_forward(self.h, sequence, position, None), "forward")

    def begin_forward_batch(self, positions, sequences):
        check(lib().tge_qwen2_kv_begin_forward_batch(self.h, _ints(positions), len(positions),
                                                     _ints(sequences), None), "forward_batch")

    def begin_prefill(self, sequence, start, count):
        check(lib().tge_qwen2_kv_begin_prefill(self.h, sequence, start, count, None), "prefill")

    def begin_verify(self, sequence, start, count):
        check(lib().tge_qwen2_kv_begin_verify(self.h, sequence, start, count, None), "verify")

    def layer(self, layer, q, k, v, out):
        check(lib().tge_qwen2_kv_layer(self.h, layer, q.ptr, k.ptr, v.ptr, out.ptr, None), "layer")

    def layer_rope(self, layer, args, out):
        """layer() with bias + RoPE fused into the append; attention reads args.q_out."""
        check(lib().tge_qwen2_kv_layer_rope(self.h, layer, C.byref(args), out.ptr, None), "layer")

    def store(self, layer, k, v):
        """Append-only (cache priming); k/v are DeviceArrays or raw device addresses."""
        kp = k if isinstance(k, int) else k.ptr
        vp = v if isinstance(v, int) else v.ptr
        check(lib().tge_qwen2_kv_store(self.h, layer, kp, vp, None), "store")

    def layer_ptrs(self, layer, q, k, v, out):
        check(lib().tge_qwen2_kv_layer(self.h, layer, q, k, v, out, None), "layer")

    def pool_handle(self):
        return lib().tge_qwen2_kv_pool(self.h)

    def batch_handle(self):
        return lib().tge_qwen2_kv_batch(self.h)

    def reset(self, sequence):
        check(lib().tge_qwen2_kv_reset(self.h, sequence), "reset_cache")

    def length(self, sequence):
        n = lib().tge_qwen2_kv_length(self.h, sequence)
        if n < 0:
            check(n, "length")
        return n

    def pages(self, sequence):
        buf = (C.c_int * 65536)()
        n = lib().tge_qwen2_kv_pages(self.h, sequence, buf, 65536)
        if n < 0:
            check(n, "pages")
        return list(buf[:n])

    def free_pages(self):
        return lib().tge_qwen2_kv_free_pages(self.h)

    def _count(self, n, what):
        if n < 0:
            check(n, what)
        return n

    def set_sparse(self, sink=4, window=512, stride=4, enabled=True):
        """set_sparse_config: static sparse attention (f16 caches; i8 stays dense)."""
        check(lib().tge_qwen2_kv_set_sparse(self.h, int(bool(enabled)), sink, window, stride),
              "set_sparse_config")

    def remember_prefix(self, sequence, tokens):
        """Keys the sequence's full cached pages among `tokens`; returns the pages keyed."""
        arr = _ints(tokens) if len(tokens) else None
        return self._count(lib().tge_qwen2_kv_remember_prefix(self.h, sequence, arr, len(tokens)),
                           "remember_prefix")

    def shared_prefix_len(self, tokens):
        arr = _ints(tokens) if len(tokens) else None
        return self._count(lib().tge_qwen2_kv_shared_prefix_len(self.h, arr, len(tokens)),
                           "shared_prefix_len")

    def attach_prefix(self, sequence, tokens):
        """Shares the longest remembered page chain of `tokens`; returns the cached length."""
        arr = _ints(tokens) if len(tokens) else None
        return self._count(lib().tge_qwen2_kv_attach_prefix(self.h, sequence, arr, len(tokens)),
                           "attach_prefix")

    def table(self):
        """A view of the driver's BlockTable (not owned)."""
        return BlockTable(0, view=lib().tge_qwen2_kv_table(self.h))

    def close(self):
        if self.h:
            lib().tge_qwen2_kv_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
