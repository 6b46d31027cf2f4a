"""Python access to the CPU oracle — TEST INFRASTRUCTURE ONLY.

Binds oracle/liboracle.so (the C restatement, oracle.c) and, when it was
built, oracle/_ref/libtge_ref.so (the reference's own attention kernels and
header-only BlockTable/layout code, compiled from /root/reference by
oracle/Makefile). Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg import this module. The product never does.

Also holds OracleBlockTable, a pure-Python restatement of the reference
BlockTable (block_table.hpp:21-130), used to cross-check the product's C++
table and the reference build on random operation sequences.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libtge_ref.so")

F32, F16, I8 = 0, 1, 2

_orc = None
_ref = None
_VP, _I, _F = C.c_void_p, C.c_int, C.c_float


def _fp(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def orc():
    global _orc
    if _orc is None:
        if not os.path.exists(ORACLE_PATH):
            raise RuntimeError(f"{ORACLE_PATH} missing: run make -C oracle")
        L = C.CDLL(ORACLE_PATH)
        L.orc_half_to_float.restype = _F
        L.orc_half_to_float.argtypes = [C.c_uint16]
        L.orc_float_to_half.restype = C.c_uint16
        L.orc_float_to_half.argtypes = [_F]
        L.orc_float_to_half_n.argtypes = [_VP, _VP, C.c_size_t]
        L.orc_half_to_float_n.argtypes = [_VP, _VP, C.c_size_t]
        L.orc_quantize_kv_block.restype = _F
        L.orc_quantize_kv_block.argtypes = [_VP, _VP]
        L.orc_quantize_rows.argtypes = [_VP, _I, _I, _VP, _VP]
        L.orc_kv_layer_offset.restype = C.c_size_t
        L.orc_kv_layer_offset.argtypes = [_I, _I, _I, _I, _I]
        L.orc_attention_head.restype = _I
        L.orc_attention_head.argtypes = [_I, _VP, _VP, _VP, _VP, _VP, _I, _I, _I, _F, _VP, _VP]
        L.orc_attention_head_f64.restype = _I
        L.orc_attention_head_f64.argtypes = [_I, _VP, _VP, _VP, _VP, _VP, _I, _I, _I,
                                             C.c_double, _VP]
        L.orc_attention_group.argtypes = [_I, _VP, _VP, _VP, _VP, _VP, _I, _I, _I, _I, _F,
                                          _VP, _VP, _VP]
        L.orc_merge_chunks.argtypes = [_VP, _VP, _VP, C.c_size_t, _I, _I, _I, _I, _VP]
        L.orc_attention_gqa.argtypes = [_I, _VP, _VP, _VP, _VP, _VP, _I, _I, _I, _I, _I, _VP]
        L.orc_gqa_chunks.restype = _I
        L.orc_gqa_chunks.argtypes = [_I, _I, _I, C.POINTER(_I)]
        L.orc_rope_neox.argtypes = [_VP, _I, _I, _VP, _VP, _I]
        L.orc_sparse_index.restype = _I
        L.orc_sparse_index.argtypes = [_I, _I, _I, _I, _VP]
        L.orc_attention_head_sparse.restype = _I
        L.orc_attention_head_sparse.argtypes = [_I, _VP, _VP, _VP, _VP, _VP, _I, _I, _I, _F, _I, _I,
                                                _I, _VP, _VP]
        L.orc_bias_rope_row.argtypes = [_VP, _VP, _VP, _VP, _VP, _VP, _I, _I, _I, _VP, _VP, _I]
        L.orc_rope_tables.argtypes = [_I, _I, _F, _F, _VP, _VP, _VP]
        L.orc_attention_block_head.restype = _I
        L.orc_attention_block_head.argtypes = [_I, _VP, _VP, _VP, _I, _I, _I, _I, _I, _I, _I,
                                               _F, _VP, _VP]
        _orc = L
    return _orc


def ref_available():
    return os.path.exists(REF_PATH)


def ref():
    """The reference build (oracle/_ref), or None when it was not built."""
    global _ref
    if _ref is None and ref_available():
        L = C.CDLL(REF_PATH)
        L.ref_float_to_half.restype = C.c_uint16
        L.ref_float_to_half.argtypes = [_F]
        L.ref_half_to_float.restype = _F
        L.ref_half_to_float.argtypes = [C.c_uint16]
        L.ref_float_to_half_n.argtypes = [_VP, _VP, C.c_size_t]
        L.ref_attention_head.restype = _I
        L.ref_attention_head.argtypes = [_I, _I, _VP, _VP, _VP, _VP, _VP, _I, _I, _I, _F, _VP, _VP]
        L.ref_attention_group.argtypes = [_I, _I, _VP, _VP, _VP, _VP, _VP, _I, _I, _I, _I, _F,
                                          _VP, _VP, _VP]
        L.ref_attention_block_head.argtypes = [_I, _VP, _VP, _VP, _I, _I, _I, _I, _I, _I, _I, _I,
                                               _F, _I, _VP, _VP]
        L.ref_bt_create.restype = _VP
        L.ref_bt_create.argtypes = [_I, _I]
        L.ref_bt_destroy.argtypes = [_VP]
        for n in ("ref_bt_allocate", "ref_bt_free_count"):
            getattr(L, n).restype = _I
            getattr(L, n).argtypes = [_VP]
        for n in ("ref_bt_release", "ref_bt_share", "ref_bt_refcount"):
            getattr(L, n).restype = _I
            getattr(L, n).argtypes = [_VP, _I]
        L.ref_bt_slot_for.restype = _I
        L.ref_bt_slot_for.argtypes = [_I, _I, C.POINTER(_I), C.POINTER(_I)]
        L.ref_bt_hash_tokens.restype = _I
        L.ref_bt_hash_tokens.argtypes = [_VP, _I, C.POINTER(C.c_uint64)]
        L.ref_bt_remember_prefix.restype = _I
        L.ref_bt_remember_prefix.argtypes = [_VP, C.c_uint64, _I]
        L.ref_bt_find_prefix.restype = _I
        L.ref_bt_find_prefix.argtypes = [_VP, C.c_uint64]
        L.ref_gather_blocks.restype = _I
        L.ref_gather_blocks.argtypes = [_VP, _I, _I, _VP, _I, _I, _VP]
        L.ref_team_create.restype = _VP
        L.ref_team_create.argtypes = [_I]
        L.ref_team_destroy.argtypes = [_VP]
        L.ref_hw_threads.restype = _I
        L.ref_baseline_decode.argtypes = [_VP, _I, _VP, _VP, _VP, _VP, _VP, _I, _I, _I, _I, _VP, _VP]
        L.ref_baseline_batch_heads.argtypes = [_VP, _I, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _I, _I,
                                               _I, _I, _I, _VP, _VP]
        L.ref_baseline_block_prefill.argtypes = [_VP, _I, _VP, _VP, _VP, _I, _I, _I, _I, _I, _I,
                                                 _VP, _VP]
        L.ref_baseline_append_f16.argtypes = [_VP, _VP, _I, _I, _VP, _VP]
        L.ref_apply_rope.argtypes = [_I, _VP, _I, _I, _I, _VP, _VP]
        L.ref_attention_head_sparse.restype = _I
        L.ref_attention_head_sparse.argtypes = [_I, _VP, _VP, _VP, _I, _I, _I, _F, _I, _I, _I, _VP,
                                                _VP]
        _ref = L
    return _ref


# ---------------------------------------------------------------------------
# Array-level helpers over the C oracle
# ---------------------------------------------------------------------------
def float_to_half(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    orc().orc_float_to_half_n(_fp(x), _fp(out), x.size)
    return out


def half_to_float(h):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    orc().orc_half_to_float_n(_fp(h), _fp(out), h.size)
    return out


def rope_neox(values, heads, head_dim, cos_t, sin_t, fma=True):
    """apply_rope (NeoX halves) of every row of `values` ([rows][heads*head_dim])
    with per-row tables cos_t/sin_t ([rows][head_dim/2]); returns a copy."""
    v = np.ascontiguousarray(values, dtype=np.float32).copy()
    c = np.ascontiguousarray(cos_t, dtype=np.float32)
    s = np.ascontiguousarray(sin_t, dtype=np.float32)
    L = orc()
    half = head_dim // 2
    for r in range(v.shape[0]):
        L.orc_rope_neox(v[r].ctypes.data_as(C.c_void_p), heads, head_dim,
                        c[r].ctypes.data_as(C.c_void_p), s[r].ctypes.data_as(C.c_void_p), int(fma))
    assert c.shape[1] == half
    return v


def bias_rope_rows(q, k, v, q_bias, k_bias, v_bias, q_heads, kv_heads, head_dim, cos_t, sin_t,
                   fma=True):
    """The per-token sequence before the store (bias adds, then RoPE of q and
    k) for every row; per-row tables. Returns new (q, k, v) arrays."""
    q = None if q is None else np.ascontiguousarray(q, dtype=np.float32).copy()
    k = np.ascontiguousarray(k, dtype=np.float32).copy()
    v = np.ascontiguousarray(v, dtype=np.float32).copy()
    c = np.ascontiguousarray(cos_t, dtype=np.float32)
    s = np.ascontiguousarray(sin_t, dtype=np.float32)
    qb, kb, vb = (None if b is None else np.ascontiguousarray(b, dtype=np.float32)
                  for b in (q_bias, k_bias, v_bias))
    L = orc()
    for r in range(k.shape[0]):
        L.orc_bias_rope_row(None if q is None else q[r].ctypes.data_as(C.c_void_p),
                            k[r].ctypes.data_as(C.c_void_p), v[r].ctypes.data_as(C.c_void_p),
                            _fp(qb), _fp(kb), _fp(vb), q_heads, kv_heads, head_dim,
                            c[r].ctypes.data_as(C.c_void_p), s[r].ctypes.data_as(C.c_void_p),
                            int(fma))
    return q, k, v


def rope_tables(head_dim, positions, theta=10000.0, attn_factor=1.0, factors=None):
    half = head_dim // 2
    c = np.empty((positions, half), np.float32)
    s = np.empty((positions, half), np.float32)
    f = None if factors is None else np.ascontiguousarray(factors, dtype=np.float32)
    orc().orc_rope_tables(head_dim, positions, theta, attn_factor, _fp(f), _fp(c), _fp(s))
    return c, s


def ref_rope(values, heads, head_dim, cos_t, sin_t, avx2=True):
    """The reference's own apply_rope_avx2 / apply_rope_scalar (oracle/_ref)
    over every row; per-row tables. Returns a copy."""
    v = np.ascontiguousarray(values, dtype=np.float32).copy()
    c = np.ascontiguousarray(cos_t, dtype=np.float32)
    s = np.ascontiguousarray(sin_t, dtype=np.float32)
    R = ref()
    for r in range(v.shape[0]):
        R.ref_apply_rope(int(avx2), v[r].ctypes.data_as(C.c_void_p), heads, head_dim, 0,
                         c[r].ctypes.data_as(C.c_void_p), s[r].ctypes.data_as(C.c_void_p))
    return v


def quantize_rows(x):
    """x [rows][kv_dim] fp32 -> (codes int8 [rows][kv_dim], scales fp32 [rows][kv_dim/32])."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, kv_dim = x.shape
    codes = np.empty((rows, kv_dim), np.int8)
    scales = np.empty((rows, kv_dim // 32), np.float32)
    orc().orc_quantize_rows(_fp(x), rows, kv_dim, _fp(codes), _fp(scales))
    return codes, scales


def attention_head(fmt, q, keys, values, k_scales, v_scales, kv_stride, span, head_dim, scale):
    """Per-head oracle over flat head-sliced rows (arrays already offset)."""
    scores = np.empty(span, np.float32)
    out = np.empty(head_dim, np.float32)
    rc = orc().orc_attention_head(fmt, _fp(q), _fp(keys), _fp(values), _fp(k_scales),
                                  _fp(v_scales), kv_stride, span, head_dim, C.c_float(scale),
                                  _fp(scores), _fp(out))
    if rc != 0:
        raise ValueError("orc_attention_head rejected its arguments")
    return out


def attention_head_sparse(fmt, q, keys, values, k_scales, v_scales, kv_stride, span, head_dim,
                          scale, sink, window, stride):
    scores = np.empty(span, np.float32)
    out = np.empty(head_dim, np.float32)
    rc = orc().orc_attention_head_sparse(fmt, _fp(q), _fp(keys), _fp(values), _fp(k_scales),
                                         _fp(v_scales), kv_stride, span, head_dim,
                                         C.c_float(scale), sink, window, stride, _fp(scores),
                                         _fp(out))
    if rc != 0:
        raise ValueError("orc_attention_head_sparse rejected its arguments")
    return out


def sparse_index(span, sink, window, stride):
    kept = np.empty(max(span, 1), np.int32)
    n = orc().orc_sparse_index(span, sink, window, stride, _fp(kept))
    return kept[:n]


def ref_attention_head_sparse(fmt, q, keys, values, kv_stride, span, head_dim, scale, sink,
                              window, stride):
    scores = np.empty(span, np.float32)
    out = np.empty(head_dim, np.float32)
    rc = ref().ref_attention_head_sparse(fmt, _fp(q), _fp(keys), _fp(values), kv_stride, span,
                                         head_dim, C.c_float(scale), sink, window, stride,
                                         _fp(scores), _fp(out))
    if rc != 0:
        raise ValueError("reference sparse kernel rejected its arguments")
    return out


class FlatCache:
    """The reference's flat KV cache for one (sequence, layer):
    rows [position][kv_dim] as f16 bits, int8 codes (+fp32 scales) or fp32."""

    def __init__(self, fmt, k, v):
        self.fmt = fmt
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        self.rows, self.kv_dim = k.shape
        self.ks = self.vs = None
        self.sparse = None  # (sink, window, stride): the static sparse subset
        if fmt == F16:
            self.k, self.v = float_to_half(k), float_to_half(v)
        elif fmt == I8:
            self.k, self.ks = quantize_rows(k)
            self.v, self.vs = quantize_rows(v)
        else:
            self.k, self.v = k, v

    def with_sparse(self, sink, window, stride):
        """Attend over the static sparse subset (orc_attention_head_sparse)."""
        self.sparse = (sink, window, stride)
        return self

    def with_scales(self, ks, vs):
        """Replace the fp32 scales (e.g. by f16-rounded ones)."""
        self.ks = np.ascontiguousarray(ks, np.float32)
        self.vs = np.ascontiguousarray(vs, np.float32)
        return self

    def head(self, q, kv_head, head_dim, span, f64=False):
        """attention_head_scalar over positions [0, span) of one KV head."""
        o = kv_head * head_dim
        kv = self.kv_dim
        kb = self.k.reshape(-1)[o:]
        vb = self.v.reshape(-1)[o:]
        ks = self.ks.reshape(-1)[o // 32:] if self.ks is not None else None
        vs = self.vs.reshape(-1)[o // 32:] if self.vs is not None else None
        q = np.ascontiguousarray(q, np.float32)
        scale = 1.0 / np.sqrt(np.float32(head_dim))
        if f64:
            out = np.empty(head_dim, np.float64)
            rc = orc().orc_attention_head_f64(self.fmt, _fp(q), _fp(kb), _fp(vb), _fp(ks),
                                              _fp(vs), kv, span, head_dim,
                                              C.c_double(1.0 / np.sqrt(head_dim)), _fp(out))
            if rc != 0:
                raise ValueError("orc_attention_head_f64 rejected its arguments")
            return out
        if self.sparse is not None:
            return attention_head_sparse(self.fmt, q, kb, vb, ks, vs, kv, span, head_dim,
                                         float(np.float32(scale)), *self.sparse)
        return attention_head(self.fmt, q, kb, vb, ks, vs, kv, span, head_dim,
                              float(np.float32(scale)))

    def attend(self, q_rows, q_heads, kv_heads, head_dim, ctx, f64=False):
        """Store-then-attend outputs for new rows at positions ctx, ctx+1, ..."""
        group = q_heads // kv_heads
        n = q_rows.shape[0]
        out = np.empty((n, q_heads * head_dim), np.float64 if f64 else np.float32)
        for i in range(n):
            for h in range(q_heads):
                q = q_rows[i, h * head_dim:(h + 1) * head_dim]
                out[i, h * head_dim:(h + 1) * head_dim] = self.head(q, h // group, head_dim,
                                                                    ctx + i + 1, f64)
        return out


# ---------------------------------------------------------------------------
# BlockTable restatement (block_table.hpp:21-130), pure Python
# ---------------------------------------------------------------------------
class OracleBlockTable:
    class Error(RuntimeError):
        pass

    NO_HASH = 0xFFFFFFFFFFFFFFFF

    def __init__(self, blocks, block_tokens=16):
        if blocks <= 0 or block_tokens <= 0:
            raise self.Error("bad size")
        self.block_tokens = block_tokens
        self.ref = [0] * blocks
        self.free = list(range(blocks - 1, -1, -1))  # top of stack = lowest id
        self.owner = {}
        self.hash_of = {}

    def capacity(self):
        return len(self.ref)

    def free_count(self):
        return len(self.free)

    def _live(self, b):
        if b < 0 or b >= len(self.ref):
            raise self.Error("out of range")
        if self.ref[b] <= 0:
            raise self.Error("not live")

    def allocate(self):
        if not self.free:
            raise self.Error("full")
        b = self.free.pop()
        self.ref[b] = 1
        return b

    def share(self, b):
        self._live(b)
        self.ref[b] += 1

    def release(self, b):
        self._live(b)
        self.ref[b] -= 1
        if self.ref[b] == 0:
            self.free.append(b)
            self.owner.pop(self.hash_of.get(b, self.NO_HASH), None)

    def refcount(self, b):
        self._live(b)
        return self.ref[b]

    @staticmethod
    def slot_for(pos, block_tokens=16):
        if pos < 0 or block_tokens <= 0:
            raise OracleBlockTable.Error("bad slot_for")
        return pos // block_tokens, pos % block_tokens

    @staticmethod
    def hash_tokens(tokens):
        h = 1469598103934665603
        for t in tokens:
            w = int(t) & 0xFFFFFFFF
            for s in (0, 8, 16, 24):
                h ^= (w >> s) & 0xFF
                h = (h * 1099511628211) & 0xFFFFFFFFFFFFFFFF
        return h

    def remember_prefix(self, hsh, b):
        self._live(b)
        self.owner[hsh] = b
        self.hash_of[b] = hsh

    def find_prefix(self, hsh):
        return self.owner.get(hsh, -1)
