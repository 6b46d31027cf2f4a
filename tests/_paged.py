"""Builds paged-KV cases for the GPU tests: a fragmented page pool, sessions
with seeded K/V/Q rows, the product's store and attention calls, and the
oracle's flat-cache view of the same rows."""
import math

import numpy as np

import oracle as O
import synth
import tge_kv as tk


class PagedCase:
    def __init__(self, q_heads, kv_heads, head_dim, fmt, contexts, n_new, scale_format=0,
                 seed=0, layers=1, pool_pages=None, outlier_frac=0.0, table=None, q_scale=1.0):
        self.qh, self.kvh, self.hd = q_heads, kv_heads, head_dim
        self.fmt, self.sf = fmt, scale_format
        self.contexts = list(contexts)
        self.n_new = list(n_new) if isinstance(n_new, (list, tuple)) else [n_new] * len(contexts)
        self.kv_dim = kv_heads * head_dim
        self.layers = layers
        rng = np.random.default_rng(seed)
        totals = [c + n for c, n in zip(self.contexts, self.n_new)]
        need = sum(math.ceil(t / 16) for t in totals)
        pages = pool_pages or need + 8
        self.table = table or synth.fragmented_table(pages, seed + 100)
        self.pool = tk.KvPool(layers, pages, kv_heads, head_dim, fmt, scale_format)
        self.pages = [[self.table.allocate() for _ in range(math.ceil(t / 16))] for t in totals]
        self.k, self.v = [], []
        for t in totals:
            k = rng.standard_normal((t, self.kv_dim), dtype=np.float32)
            v = rng.standard_normal((t, self.kv_dim), dtype=np.float32)
            if outlier_frac:
                ch = synth.outlier_channels(self.kv_dim, outlier_frac, seed)
                k[:, ch] *= np.float32(8)
            self.k.append(k)
            self.v.append(v)
        rows = sum(self.n_new)
        self.q = (rng.standard_normal((rows, q_heads * head_dim), dtype=np.float32)
                  * np.float32(q_scale))

    # ---- product calls -------------------------------------------------
    def sessions(self, step):
        if step:
            return [tk.Session(c, n, p) for c, n, p in zip(self.contexts, self.n_new, self.pages)]
        return [tk.Session(0, c, p) for c, p in zip(self.contexts, self.pages) if c > 0]

    def fill(self, layer=0):
        """Append every session's context rows (one batch, ctx 0)."""
        ss = self.sessions(False)
        if not ss:
            return
        b = tk.Batch().plan(self.pool, ss, self.qh)
        kk = np.concatenate([k[:c] for k, c in zip(self.k, self.contexts) if c > 0])
        vv = np.concatenate([v[:c] for v, c in zip(self.v, self.contexts) if c > 0])
        dk, dv = tk.DeviceArray.from_numpy(kk), tk.DeviceArray.from_numpy(vv)
        b.append(self.pool, layer, dk, dv)
        tk.hip().sync()
        b.close()

    def step(self, layer=0, kind="decode"):
        """Append the new rows, attend; returns (out rows, batch)."""
        b = tk.Batch().plan(self.pool, self.sessions(True), self.qh)
        if getattr(self, "sparse", None):
            b.set_sparse(*self.sparse)
        kk = np.concatenate([k[c:] for k, c in zip(self.k, self.contexts)])
        vv = np.concatenate([v[c:] for v, c in zip(self.v, self.contexts)])
        dk, dv = tk.DeviceArray.from_numpy(kk), tk.DeviceArray.from_numpy(vv)
        dq = tk.DeviceArray.from_numpy(self.q)
        dout = tk.DeviceArray((self.q.shape[0], self.qh * self.hd), np.float32).zero()
        if kind == "step":  # append + attention in one call
            b.decode_step(self.pool, layer, dq, dk, dv, dout)
            tk.hip().sync()
            return dout.numpy(), b
        b.append(self.pool, layer, dk, dv)
        if kind == "decode":
            b.decode(self.pool, layer, dq, dout)
        elif kind == "mixed":
            b.attention(self.pool, layer, dq, dout)
        else:
            b.prefill(self.pool, layer, dq, dout)
        tk.hip().sync()
        return dout.numpy(), b

    # ---- oracle view ------------------------------------------------------
    def flat(self, s):
        """The reference flat cache of session s (scales as the pool stores
        them: f16-rounded for SCALE_F16)."""
        fc = O.FlatCache({tk.KV_F16: O.F16, tk.KV_I8: O.I8}[self.fmt], self.k[s], self.v[s])
        if getattr(self, "sparse", None):
            fc.with_sparse(*self.sparse)
        if self.fmt == tk.KV_I8 and self.sf == tk.SCALE_F16:
            fc.with_scales(O.half_to_float(O.float_to_half(fc.ks)),
                           O.half_to_float(O.float_to_half(fc.vs)))
        return fc

    def oracle_out(self, f64=False):
        outs, row = [], 0
        for s, (c, n) in enumerate(zip(self.contexts, self.n_new)):
            outs.append(self.flat(s).attend(self.q[row:row + n], self.qh, self.kvh, self.hd, c,
                                            f64=f64))
            row += n
        return np.concatenate(outs)

    def close(self):
        self.pool.close()
