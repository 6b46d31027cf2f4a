"""GPU tests of the Qwen2-shaped KV driver (tge_qwen2_kv_*): the
store-then-attend flows of Qwen2::forward / forward_batch / prefill_run /
verify_draft / reset_cache (qwen2.cpp:2032-2095, 1613-1747, 2130-2335,
2502-2577) over paged device memory, checked against the CPU oracle's flat
cache, plus the driver's validation rules and page reuse order."""
import math
import sys

import numpy as np
import pytest

import oracle as O
import tge_kv as tk
from _util import assert_attention_close

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


class Model:
    """A driver plus the host copy of every row it was given, per layer and
    sequence, so the oracle can replay the same cache."""

    def __init__(self, layers, qh, kvh, hd, fmt, sequences, pages, context=4096, seed=0,
                 fragment=None):
        self.layers, self.qh, self.kvh, self.hd, self.fmt = layers, qh, kvh, hd, fmt
        self.m = tk.Qwen2KvPath(layers, qh, kvh, hd, context=context, sequences=sequences,
                                pages=pages, fmt=fmt, scale_format=tk.SCALE_F16)
        if fragment is not None:
            self.m.table().fragment(fragment)
        self.rng = np.random.default_rng(seed)
        self.k = {}  # (layer, seq) -> rows in position order
        self.v = {}

    def rows(self, n):
        kv_dim = self.kvh * self.hd
        k = [self.rng.standard_normal((n, kv_dim), dtype=np.float32) for _ in range(self.layers)]
        v = [self.rng.standard_normal((n, kv_dim), dtype=np.float32) for _ in range(self.layers)]
        q = [self.rng.standard_normal((n, self.qh * self.hd), dtype=np.float32)
             for _ in range(self.layers)]
        return q, k, v

    def keep(self, seq, start, k, v):
        for l in range(self.layers):
            old_k = self.k.get((l, seq), np.zeros((0, k[l].shape[1]), np.float32))
            old_v = self.v.get((l, seq), np.zeros((0, v[l].shape[1]), np.float32))
            assert old_k.shape[0] >= start
            self.k[(l, seq)] = np.concatenate([old_k[:start], k[l]])
            self.v[(l, seq)] = np.concatenate([old_v[:start], v[l]])

    def run_layers(self, q, k, v, attend=True):
        """Run every layer of the begun step; returns the outputs per layer."""
        outs = []
        for l in range(self.layers):
            dk, dv = tk.DeviceArray.from_numpy(k[l]), tk.DeviceArray.from_numpy(v[l])
            if attend:
                dq = tk.DeviceArray.from_numpy(q[l])
                dout = tk.DeviceArray(q[l].shape, np.float32).zero()
                self.m.layer(l, dq, dk, dv, dout)
                tk.hip().sync()
                outs.append(dout.numpy())
                dq.close()
                dout.close()
            else:
                self.m.store(l, dk, dv)
                tk.hip().sync()
            dk.close()
            dv.close()
        return outs

    def oracle(self, l, seq, q_rows, ctx):
        fc = O.FlatCache({tk.KV_F16: O.F16, tk.KV_I8: O.I8}[self.fmt], self.k[(l, seq)],
                         self.v[(l, seq)])
        if self.fmt == tk.KV_I8:
            fc.with_scales(O.half_to_float(O.float_to_half(fc.ks)),
                           O.half_to_float(O.float_to_half(fc.vs)))
        return fc.attend(q_rows, self.qh, self.kvh, self.hd, ctx)

    def close(self):
        self.m.close()


@pytest.mark.parametrize("fmt", [tk.KV_F16, tk.KV_I8])
def test_prefill_then_forward_matches_oracle(gpu, fmt):
    """prefill_run of 100 tokens (block-prefill kernel), then forward of one
    token (decode kernel), two layers, fragmented pool."""
    say(f"driver prefill+forward fmt={fmt}")
    md = Model(2, 14, 2, 64, fmt, sequences=2, pages=40, context=512, seed=1, fragment=5)
    q, k, v = md.rows(100)
    md.m.begin_prefill(0, 0, 100)
    md.keep(0, 0, k, v)
    outs = md.run_layers(q, k, v)
    for l in range(2):
        assert_attention_close(outs[l], md.oracle(l, 0, q[l], 0), f"prefill layer {l}")
    assert md.m.length(0) == 100 and len(md.m.pages(0)) == 7
    q, k, v = md.rows(1)
    md.m.begin_forward(0, 100)
    md.keep(0, 100, k, v)
    outs = md.run_layers(q, k, v)
    for l in range(2):
        assert_attention_close(outs[l], md.oracle(l, 0, q[l], 100), f"forward layer {l}")
    assert md.m.length(0) == 101 and len(md.m.pages(0)) == 7
    md.close()


def test_forward_batch_and_verify_match_oracle(gpu):
    """forward_batch over two sequences (two rows for one, one for the
    other), then verify_draft of 4 tokens (7B-like group of 7)."""
    md = Model(1, 28, 4, 128, tk.KV_I8, sequences=3, pages=200, seed=2, fragment=9)
    fills = {0: 300, 1: 47}
    for s, n in fills.items():
        _, k, v = md.rows(n)
        md.m.begin_prefill(s, 0, n)
        md.keep(s, 0, k, v)
        md.run_layers(None, k, v, attend=False)
    q, k, v = md.rows(3)
    md.m.begin_forward_batch([300, 301, 47], [0, 0, 1])
    md.keep(0, 300, [k[0][:2]], [v[0][:2]])
    md.keep(1, 47, [k[0][2:]], [v[0][2:]])
    out = md.run_layers(q, k, v)[0]
    want = np.concatenate([md.oracle(0, 0, q[0][:2], 300), md.oracle(0, 1, q[0][2:], 47)])
    assert_attention_close(out, want, "forward_batch")
    assert md.m.length(0) == 302 and md.m.length(1) == 48
    q, k, v = md.rows(4)
    md.m.begin_verify(1, 48, 4)
    md.keep(1, 48, k, v)
    out = md.run_layers(q, k, v)[0]
    assert_attention_close(out, md.oracle(0, 1, q[0], 48), "verify_draft")
    # a verified draft can be rolled back: verifying again from 49 rewrites
    # positions 49..52 (the store-then-attend order of verify_draft)
    q, k, v = md.rows(4)
    md.m.begin_verify(1, 49, 4)
    md.keep(1, 49, k, v)
    out = md.run_layers(q, k, v)[0]
    assert_attention_close(out, md.oracle(0, 1, q[0], 49), "verify_draft again")
    md.close()


def test_reset_releases_pages_in_logical_order(gpu):
    """reset_cache returns a sequence's pages in logical order, so the free
    list hands them out again LIFO (last page first), exactly as the
    reference BlockTable does (block_table.hpp:59-71)."""
    md = Model(1, 14, 2, 64, tk.KV_F16, sequences=2, pages=16, seed=3)
    orc = O.OracleBlockTable(16)
    _, k, v = md.rows(40)
    md.m.begin_prefill(0, 0, 40)
    md.run_layers(None, k, v, attend=False)
    want0 = [orc.allocate() for _ in range(3)]
    assert md.m.pages(0) == want0
    _, k, v = md.rows(20)
    md.m.begin_prefill(1, 0, 20)
    md.run_layers(None, k, v, attend=False)
    want1 = [orc.allocate() for _ in range(2)]
    assert md.m.pages(1) == want1
    md.m.reset(0)
    for p in want0:
        orc.release(p)
    assert md.m.length(0) == 0 and md.m.pages(0) == []
    assert md.m.free_pages() == orc.free_count()
    _, k, v = md.rows(30)
    md.m.begin_prefill(1, 20, 30)
    md.run_layers(None, k, v, attend=False)
    want1 += [orc.allocate() for _ in range(2)]
    assert md.m.pages(1) == want1
    assert want1[2:] == [want0[2], want0[1]]
    md.close()


def test_driver_validation(gpu):
    """Misuse is rejected with the reference's error class and leaves the
    model unchanged."""
    md = Model(2, 14, 2, 64, tk.KV_F16, sequences=2, pages=8, context=100, seed=4)
    L = tk.lib()
    h = md.m.h

    def status(f):
        with pytest.raises(tk.TgeError) as e:
            f()
        return e.value.status

    assert status(lambda: md.m.begin_forward(0, 100)) == tk.ERR_RUNTIME     # beyond context
    assert status(lambda: md.m.begin_forward(2, 0)) == tk.ERR_RUNTIME       # no such sequence
    assert status(lambda: md.m.begin_forward(0, 5)) == tk.ERR_RUNTIME       # leaves a gap
    assert status(lambda: md.m.begin_verify(0, 0, 7)) == tk.ERR_RUNTIME     # > 6 drafts
    assert status(lambda: md.m.begin_forward_batch([0, 2], [0, 0])) == tk.ERR_RUNTIME
    assert status(lambda: md.m.begin_prefill(0, 90, 20)) == tk.ERR_RUNTIME  # past context
    assert L.tge_qwen2_kv_layer(h, 0, None, None, None, None, None) == tk.ERR_RUNTIME
    # the pool has 8 pages = 128 positions: 2 x 70 does not fit
    _, k, v = md.rows(70)
    md.m.begin_prefill(0, 0, 70)
    md.run_layers(None, k, v, attend=False)
    assert status(lambda: md.m.begin_prefill(1, 0, 70)) == tk.ERR_RUNTIME   # table full
    assert md.m.length(1) == 0 and md.m.length(0) == 70 and md.m.free_pages() == 3
    md.m.begin_forward(0, 70)
    assert L.tge_qwen2_kv_layer(h, 5, None, None, None, None, None) == tk.ERR_INVALID
    md.close()


def pool_rows(md, layer, seq, count):
    """Positions [0, count) of a driver sequence as stored (f16 bits), read
    through a throwaway plan over the driver's pool (nothing is written)."""
    from types import SimpleNamespace
    pool = SimpleNamespace(h=md.m.pool_handle(), kv_heads=md.kvh, head_dim=md.hd,
                           format=md.fmt, scale_format=tk.SCALE_F16)
    sess = SimpleNamespace(ctx=count - 1, n_new=1, pages=md.m.pages(seq))
    b = tk.Batch().plan(pool, [sess], md.qh)
    k, v, _, _ = b.gather(pool, layer, 0, count)
    b.close()
    return k, v


def test_prefix_sharing_and_copy_on_write(gpu):
    """Shared prefixes matched token by token (shared_prefix_len,
    qwen2.cpp:1948-1971): recorded pages are attached to a new sequence by
    reference count (BlockTable share, block_table.hpp:52-111), the last
    one possibly in part, replacing the reference's copied prefix rows
    (qwen2.cpp:1973-2026). The attached sequence appends after them (its
    first write copies the partly matched page); attention over the shared
    pages equals attention over a privately filled copy bit for bit; a write
    into a shared page copies it first, so the other holder's rows never
    change."""
    say("driver prefix sharing")
    md = Model(2, 14, 2, 64, tk.KV_F16, sequences=4, pages=64, context=512, seed=6)
    tab = md.m.table()
    toks = list(range(1000, 1050))
    _, k0, v0 = md.rows(50)
    md.m.begin_prefill(0, 0, 50)
    md.keep(0, 0, k0, v0)
    md.run_layers(None, k0, v0, attend=False)
    assert md.m.remember_prefix(0, toks) == 50  # every cached token, page 3 in part
    assert md.m.shared_prefix_len(toks + [1, 2]) == 50
    assert md.m.shared_prefix_len(toks[:40] + [7] * 10) == 40
    assert md.m.shared_prefix_len(toks[:47]) == 47  # inside page 2
    assert md.m.shared_prefix_len([999] + toks) == 0
    p0 = md.m.pages(0)

    # sequence 1 takes a 47-token run (page 2 in part), then prefills 20 of its own
    assert md.m.attach_prefix(1, toks[:47] + [5] * 20) == 47
    assert md.m.pages(1) == p0[:3] and md.m.length(1) == 47
    assert [tab.refcount(p) for p in p0] == [2, 2, 2, 1]
    _, k1, v1 = md.rows(20)
    md.m.begin_prefill(1, 47, 20)
    for l in range(md.layers):
        md.k[(l, 1)] = np.concatenate([md.k[(l, 0)][:47], k1[l]])
        md.v[(l, 1)] = np.concatenate([md.v[(l, 0)][:47], v1[l]])
    md.run_layers(None, k1, v1, attend=False)
    p1 = md.m.pages(1)
    assert p1[:2] == p0[:2] and p1[2] not in p0 and len(p1) == 5
    assert [tab.refcount(p) for p in p0] == [2, 2, 1, 1]
    # sequence 2 holds the same 67 rows in private pages
    k2 = [md.k[(l, 1)].copy() for l in range(md.layers)]
    v2 = [md.v[(l, 1)].copy() for l in range(md.layers)]
    md.m.begin_prefill(2, 0, 67)
    md.keep(2, 0, k2, v2)
    md.run_layers(None, k2, v2, attend=False)
    assert not set(md.m.pages(2)) & set(p0)

    q, k, v = md.rows(1)
    md.m.begin_forward(1, 67)
    md.keep(1, 67, k, v)
    out1 = md.run_layers(q, k, v)
    md.m.begin_forward(2, 67)
    md.keep(2, 67, k, v)
    out2 = md.run_layers(q, k, v)
    for l in range(md.layers):
        assert np.array_equal(out1[l], out2[l]), f"shared vs private pages differ, layer {l}"
        assert_attention_close(out1[l], md.oracle(l, 1, q[l], 67), f"shared prefix layer {l}")

    # copy-on-write: sequence 1 verifies drafts at 20..21, inside shared page 1
    q, k, v = md.rows(2)
    md.m.begin_verify(1, 20, 2)
    md.keep(1, 20, k, v)
    out = md.run_layers(q, k, v)
    for l in range(md.layers):
        assert_attention_close(out[l], md.oracle(l, 1, q[l], 20), f"after copy layer {l}")
    p1 = md.m.pages(1)
    assert p1[0] == p0[0] and p1[1] not in p0
    assert [tab.refcount(p) for p in p0] == [2, 1, 1, 1]
    for l in range(md.layers):
        gk, gv = pool_rows(md, l, 0, 50)
        assert np.array_equal(gk, O.float_to_half(md.k[(l, 0)])), f"sequence 0 K changed, layer {l}"
        assert np.array_equal(gv, O.float_to_half(md.v[(l, 0)])), f"sequence 0 V changed, layer {l}"
        gk, gv = pool_rows(md, l, 1, 22)
        assert np.array_equal(gk, O.float_to_half(md.k[(l, 1)]))
        assert np.array_equal(gv, O.float_to_half(md.v[(l, 1)]))

    # an attach needs an empty sequence
    with pytest.raises(tk.TgeError) as e:
        md.m.attach_prefix(1, toks)
    assert e.value.status == tk.ERR_RUNTIME
    # releases: recorded pages stay found while some sequence holds them
    md.m.reset(0)
    assert tab.refcount(p0[0]) == 1
    assert md.m.shared_prefix_len(toks) == 16  # page 1's record went with its last holder
    md.m.reset(1)
    assert md.m.shared_prefix_len(toks) == 0
    md.close()


def test_layer_rope_flow_matches_oracle(gpu):
    """The driver's fused layer (bias + RoPE + append, then attention on the
    rotated q) over a prefill and a decode step equals the oracle running
    the reference's per-token sequence on the same raw rows."""
    say("driver layer_rope")
    md = Model(2, 14, 2, 64, tk.KV_I8, sequences=1, pages=20, context=256, seed=8)
    cos_t, sin_t = tk.rope_tables(64, 256)
    dc, ds = tk.DeviceArray.from_numpy(cos_t), tk.DeviceArray.from_numpy(sin_t)
    rng = np.random.default_rng(4)
    biases = [[rng.standard_normal(n).astype(np.float32) for n in (14 * 64, 128, 128)]
              for _ in range(md.layers)]
    for start, count in ((0, 70), (70, 1)):
        if count > 1:
            md.m.begin_prefill(0, start, count)
        else:
            md.m.begin_forward(0, start)
        q, k, v = md.rows(count)
        pos = np.arange(start, start + count)
        for l in range(md.layers):
            qb, kb, vb = biases[l]
            q_o, k_o, v_o = O.bias_rope_rows(q[l], k[l], v[l], qb, kb, vb, 14, 2, 64,
                                             cos_t[pos], sin_t[pos], True)
            empty = np.zeros((0, 128), np.float32)
            md.k[(l, 0)] = np.concatenate([md.k.get((l, 0), empty)[:start], k_o])
            md.v[(l, 0)] = np.concatenate([md.v.get((l, 0), empty)[:start], v_o])
            a = {n: tk.DeviceArray.from_numpy(x) for n, x in
                 (("q", q[l]), ("k", k[l]), ("v", v[l]), ("qb", qb), ("kb", kb), ("vb", vb))}
            out = tk.DeviceArray(q[l].shape, np.float32).zero()
            args = tk.rope_args(a["k"], a["v"], dc, ds, 256, q=a["q"], q_out=a["q"],
                                q_bias=a["qb"], k_bias=a["kb"], v_bias=a["vb"])
            md.m.layer_rope(l, args, out)
            tk.hip().sync()
            assert np.array_equal(a["q"].numpy(), q_o)
            assert_attention_close(out.numpy(), md.oracle(l, 0, q_o, start),
                                   f"layer_rope start {start} layer {l}")
    md.close()


def test_forward_batch_mixing_prefill_and_decode(gpu):
    """forward_batch rows of one sequence prefilling a 90-token chunk next
    to two sequences decoding one token each: one plan, one layer call, the
    decode kernel for the short sessions and the prefill kernel for the
    chunk, against the oracle."""
    say("driver mixed forward_batch")
    md = Model(1, 14, 2, 64, tk.KV_F16, sequences=3, pages=60, seed=9, fragment=3)
    for s, n in ((0, 130), (1, 40)):
        _, k, v = md.rows(n)
        md.m.begin_prefill(s, 0, n)
        md.keep(s, 0, k, v)
        md.run_layers(None, k, v, attend=False)
    positions = [130] + [40] + list(range(0, 90))
    seqs = [0, 1] + [2] * 90
    q, k, v = md.rows(len(positions))
    md.m.begin_forward_batch(positions, seqs)
    md.keep(0, 130, [k[0][:1]], [v[0][:1]])
    md.keep(1, 40, [k[0][1:2]], [v[0][1:2]])
    md.keep(2, 0, [k[0][2:]], [v[0][2:]])
    out = md.run_layers(q, k, v)[0]
    want = np.concatenate([md.oracle(0, 0, q[0][:1], 130), md.oracle(0, 1, q[0][1:2], 40),
                           md.oracle(0, 2, q[0][2:], 0)])
    assert_attention_close(out, want, "mixed forward_batch")
    md.close()


def test_driver_sparse_config(gpu):
    """set_sparse_config on the driver: f16 caches attend over the static
    sparse subset, i8 caches stay dense (uses_sparse, qwen2.cpp:1313-1317),
    bad strides are a runtime error (qwen2.cpp:182-189)."""
    say("driver sparse")
    for fmt in (tk.KV_F16, tk.KV_I8):
        md = Model(1, 14, 2, 64, fmt, sequences=1, pages=40, context=600, seed=12)
        _, k, v = md.rows(400)
        md.m.begin_prefill(0, 0, 400)
        md.keep(0, 0, k, v)
        md.run_layers(None, k, v, attend=False)
        md.m.set_sparse(4, 100, 7)
        q, k, v = md.rows(2)
        md.m.begin_verify(0, 400, 2)
        md.keep(0, 400, k, v)
        out = md.run_layers(q, k, v)[0]
        fc = O.FlatCache({tk.KV_F16: O.F16, tk.KV_I8: O.I8}[fmt], md.k[(0, 0)], md.v[(0, 0)])
        if fmt == tk.KV_I8:
            fc.with_scales(O.half_to_float(O.float_to_half(fc.ks)),
                           O.half_to_float(O.float_to_half(fc.vs)))
        else:
            fc.with_sparse(4, 100, 7)
        assert_attention_close(out, fc.attend(q[0], 14, 2, 64, 400), f"driver sparse fmt={fmt}")
        with pytest.raises(tk.TgeError) as e:
            md.m.set_sparse(4, 100, 1)
        assert e.value.status == tk.ERR_RUNTIME
        md.close()


@pytest.mark.parametrize("fmt", [tk.KV_F16, tk.KV_I8])
def test_native_cpp_driver(gpu, tmp_path, fmt):
    """The C++20 driver used natively (tests/native/driver_check.cpp, built
    by the package Makefile): hipMalloc'd buffers, a second sequence's pages
    interleaved, a 37-token prefill chunk and three decode steps per layer
    through tge::models::Qwen2KvPath, then its misuse exceptions
    (qwen2.cpp:2036-2044). Outputs match the oracle's flat cache."""
    import os
    import subprocess
    exe = os.path.join(os.path.dirname(tk.LIB_PATH), "bin", "driver_check")
    if not os.path.exists(exe):
        pytest.fail(f"{exe} is missing: build the package (make -C aegean-tge_amd)")
    layers, qh, kvh, hd, n_pre, n_dec, context = 2, 14, 2, 64, 37, 3, 256
    n = n_pre + n_dec
    rng = np.random.default_rng(90 + fmt)
    data = [[rng.standard_normal((n, d)).astype(np.float32) for d in (kvh * hd, kvh * hd, qh * hd)]
            for _ in range(layers)]
    src = tmp_path / "in.bin"
    with open(src, "wb") as f:
        f.write(np.array([layers, qh, kvh, hd, n_pre, n_dec, context, fmt], np.int32).tobytes())
        for k, v, q in data:
            f.write(k.tobytes() + v.tobytes() + q.tobytes())
    dst = tmp_path / "out.bin"
    say(f"native driver_check fmt={fmt}")
    r = subprocess.run([exe, str(src), str(dst)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    assert "exceptions ok" in r.stdout
    got = np.fromfile(dst, np.float32).reshape(layers, n, qh * hd)
    for layer, (k, v, q) in enumerate(data):
        fc = O.FlatCache(O.F16 if fmt == tk.KV_F16 else O.I8, k, v)
        if fmt == tk.KV_I8:
            fc.with_scales(O.half_to_float(O.float_to_half(fc.ks)),
                           O.half_to_float(O.float_to_half(fc.vs)))
        want = fc.attend(q, qh, kvh, hd, 0)
        err = assert_attention_close(got[layer], want, f"native driver layer {layer}")
        say(f"  layer {layer}: max abs err {err:.2e}")


@pytest.mark.parametrize("fmt", [tk.KV_F16, tk.KV_I8])
def test_random_serving_flow(gpu, fmt):
    """A seeded serving run through the driver (c5's pattern at small size,
    7B-like group of 7): twelve forward_batch steps over a random subset of
    six sequences with 1-4 new tokens each, and every fourth step one
    sequence reset and refilled with a random-length prompt (its pages go
    back to the table and are reused). Every step's rows match the oracle
    and the lengths follow."""
    say(f"random serving flow fmt={fmt}")
    md = Model(1, 28, 4, 128, fmt, sequences=6, pages=600, context=2048, seed=70, fragment=71)
    r = np.random.default_rng(72)
    length = [0] * 6

    def refill(s):
        n = int(r.integers(1, 700))
        md.m.reset(s)
        _, k, v = md.rows(n)
        md.m.begin_prefill(s, 0, n)
        md.k.pop((0, s), None)
        md.v.pop((0, s), None)
        md.keep(s, 0, k, v)
        md.run_layers(None, k, v, attend=False)
        length[s] = n

    for s in range(6):
        refill(s)
    for step in range(12):
        if step % 4 == 3:
            refill(int(r.integers(0, 6)))
        seqs = sorted(int(x) for x in r.choice(6, int(r.integers(1, 7)), replace=False))
        counts = [int(r.integers(1, 5)) for _ in seqs]
        positions = [length[s] + i for s, n in zip(seqs, counts) for i in range(n)]
        owners = [s for s, n in zip(seqs, counts) for _ in range(n)]
        q, k, v = md.rows(len(positions))
        md.m.begin_forward_batch(positions, owners)
        row = 0
        for s, n in zip(seqs, counts):
            md.keep(s, length[s], [k[0][row:row + n]], [v[0][row:row + n]])
            row += n
        out = md.run_layers(q, k, v)[0]
        want, row = [], 0
        for s, n in zip(seqs, counts):
            want.append(md.oracle(0, s, q[0][row:row + n], length[s]))
            row += n
            length[s] += n
        assert_attention_close(out, np.concatenate(want), f"serving step {step}")
        assert [md.m.length(s) for s in range(6)] == length
    md.close()
