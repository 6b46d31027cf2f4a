"""GPU parity at every BASELINE configuration's full stated size.

Each test runs one configuration's workload through the C ABI at the sizes
the configuration names (layers are independent on this path, so one layer
stands for all) and checks every attention output against the CPU oracle
(attention_head_scalar, attention_scalar.cpp:48-115, restated in oracle.c)
within max-abs 2e-3 + rel 1e-3, and the appended pool contents bit for bit
where the configuration appends. Each prints its worst error and its worst
ratio of error to the bound (the margin left by the kernels' f16 rounding of
Q and of the softmax weights).

  C1  Qwen2-0.5B, f16, 1024 cached + 64 decode steps, 128-page permuted pool
  C2  Qwen2-0.5B, int8 + f16 scales, 1 % outlier K channels x8,
      4096 cached + 128 decode steps
  C3  Qwen2-1.5B, f16, sessions 512/2048/4096/8192 on a fragmented pool,
      32 batched decode steps
  C4  Qwen2-7B, f16, 2048-token prompt in four causal chunks of 512
  C5  Qwen2-7B, int8 + f16 scales, 1 % outlier K channels x8, the 64
      sessions of the bench (log-uniform 1k-32k), 4-query verify; then
      8 sessions released and 8 new 2048-token sessions on their pages
"""
import math
import sys
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

import oracle as O
import synth
import tge_kv as tk
from _util import ATOL, MARGINS, RTOL, bits

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


class Margin:
    """Worst absolute error and worst error / bound over many checks."""

    def __init__(self, name):
        self.name, self.err, self.ratio, self.checked = name, 0.0, 0.0, 0

    def check(self, got, want, what):
        got = np.asarray(got, np.float64)
        want = np.asarray(want, np.float64)
        assert got.shape == want.shape
        assert np.all(np.isfinite(got)), f"{self.name} {what}: non-finite output"
        err = np.abs(got - want)
        bound = ATOL + RTOL * np.abs(want)
        ratio = err / bound
        worst = np.unravel_index(np.argmax(ratio), ratio.shape)
        assert np.all(err <= bound), (
            f"{self.name} {what}: err {err[worst]:.3e} > bound {bound[worst]:.3e} at {worst}")
        self.err = max(self.err, float(err.max()))
        self.ratio = max(self.ratio, float(ratio.max()))
        self.checked += got.size

    def report(self):
        say(f"  {self.name}: {self.checked} outputs, max abs err {self.err:.3e}, "
            f"max err/bound {self.ratio:.3f}")
        MARGINS[self.name] = (self.checked, self.err, self.ratio)


def flat_cache(fmt, k, v):
    """The oracle's flat cache holding the scales as the pool stores them
    (f16-rounded for SCALE_F16 int8 pools)."""
    fc = O.FlatCache(O.F16 if fmt == tk.KV_F16 else O.I8, k, v)
    if fmt == tk.KV_I8:
        fc.with_scales(O.half_to_float(O.float_to_half(fc.ks)),
                       O.half_to_float(O.float_to_half(fc.vs)))
    return fc


def check_pool(pool, batch, s, fmt, fc, count):
    """Session s's positions [0, count) in the pool equal the oracle's store."""
    gk, gv, gks, gvs = batch.gather(pool, 0, s, count)
    assert np.array_equal(gk, fc.k[:count].view(gk.dtype)), f"K bits differ, session {s}"
    assert np.array_equal(gv, fc.v[:count].view(gv.dtype)), f"V bits differ, session {s}"
    if fmt == tk.KV_I8:
        assert np.array_equal(gks, O.float_to_half(fc.ks[:count]))
        assert np.array_equal(gvs, O.float_to_half(fc.vs[:count]))


def oracle_outputs(fcs, q, contexts, n, sh, f64=False):
    """The oracle's outputs of every session (threads: the C oracle runs
    outside the interpreter lock)."""
    def one(s):
        return fcs[s].attend(q[s * n:(s + 1) * n], sh.q_heads, sh.kv_heads, sh.head_dim,
                             contexts[s], f64=f64)
    with ThreadPoolExecutor(max_workers=8) as ex:
        return list(ex.map(one, range(len(contexts))))


class Serving:
    """Sessions of one configuration on one layer's pool: every session's
    K/V rows for its whole run, pages from a BlockTable, store + attend
    steps through the C ABI, the oracle's flat cache per session."""

    def __init__(self, cfg, contexts, steps, n_new, pool_pages, table_seed, seed):
        sh = cfg.shape
        self.cfg, self.sh, self.n_new = cfg, sh, n_new
        self.rng = np.random.default_rng(seed)
        self.pool = tk.KvPool(1, pool_pages, sh.kv_heads, sh.head_dim, cfg.fmt, tk.SCALE_F16)
        self.table = (synth.fragmented_table(pool_pages, table_seed) if table_seed is not None
                      else tk.BlockTable(pool_pages))
        self.ctx, self.k, self.v, self.pages, self.fc = [], [], [], [], []
        for c in contexts:
            self.add_session(c, steps)

    def add_session(self, ctx, steps, slot=None):
        total = ctx + steps * self.n_new
        k, v = synth.make_kv(self.rng, total, self.sh.kv_dim, self.cfg)
        pages = [self.table.allocate() for _ in range(math.ceil(total / 16))]
        entry = (ctx, k, v, pages, flat_cache(self.cfg.fmt, k, v))
        if slot is None:
            for lst, x in zip((self.ctx, self.k, self.v, self.pages, self.fc), entry):
                lst.append(x)
        else:
            for lst, x in zip((self.ctx, self.k, self.v, self.pages, self.fc), entry):
                lst[slot] = x

    def release(self, s):
        for p in self.pages[s]:  # logical order, as reset_cache releases them
            self.table.release(p)

    def fill(self, only=None):
        """Store the cached context rows of the sessions (all, or `only`)."""
        idx = [s for s in range(len(self.ctx)) if self.ctx[s] > 0 and (only is None or s in only)]
        if not idx:
            return
        b = tk.Batch().plan(self.pool, [tk.Session(0, self.ctx[s], self.pages[s]) for s in idx],
                            self.sh.q_heads)
        dk = tk.DeviceArray.from_numpy(np.concatenate([self.k[s][:self.ctx[s]] for s in idx]))
        dv = tk.DeviceArray.from_numpy(np.concatenate([self.v[s][:self.ctx[s]] for s in idx]))
        b.append(self.pool, 0, dk, dv)
        tk.hip().sync()
        for a in (dk, dv):
            a.close()
        b.close()

    def step(self, margin, kind="decode", check_store=False):
        """Append n_new rows per session, attend, check every output row
        against the oracle; the contexts advance."""
        n = self.n_new
        sess = [tk.Session(c, n, p) for c, p in zip(self.ctx, self.pages)]
        b = tk.Batch().plan(self.pool, sess, self.sh.q_heads)
        q = synth.make_q(self.rng, n * len(self.ctx), self.sh.q_dim, self.cfg)
        dk = tk.DeviceArray.from_numpy(np.concatenate([k[c:c + n] for k, c in zip(self.k, self.ctx)]))
        dv = tk.DeviceArray.from_numpy(np.concatenate([v[c:c + n] for v, c in zip(self.v, self.ctx)]))
        dq = tk.DeviceArray.from_numpy(q)
        out = tk.DeviceArray(q.shape, np.float32).zero()
        if kind == "step":  # tge_decode_step: append + attention in one call
            b.decode_step(self.pool, 0, dq, dk, dv, out)
        else:
            b.append(self.pool, 0, dk, dv)
            getattr(b, kind)(self.pool, 0, dq, out)
        tk.hip().sync()
        self.last_step_info = b.step_info()
        self.last_stores_rows = b.decode_stores_rows()
        got = out.numpy()
        sh = self.sh
        wants = oracle_outputs(self.fc, q, self.ctx, n, sh)
        for s, c in enumerate(self.ctx):
            margin.check(got[s * n:(s + 1) * n], wants[s], f"session {s} ctx {c}")
            if check_store:
                check_pool(self.pool, b, s, self.cfg.fmt, self.fc[s], c + n)
        info = b.info()
        for a in (dk, dv, dq, out):
            a.close()
        b.close()
        self.ctx = [c + n for c in self.ctx]
        return info

    def close(self):
        self.pool.close()
        self.table.close()


def test_c1_full_size(gpu):
    """C1: 1024 cached positions, then 64 decode steps (append one token,
    attend over 1025..1088 positions), every step checked; the pool's 68
    live pages are a seeded permutation of 128."""
    cfg = synth.configs()["c1"]
    say("C1 full size")
    sv = Serving(cfg, cfg.contexts, cfg.steps, 1, 128, table_seed=cfg.seed, seed=101)
    assert sorted(sv.pages[0]) != sv.pages[0]
    sv.fill()
    m = Margin("c1")
    for i in range(cfg.steps):
        sv.step(m, check_store=(i in (0, cfg.steps - 1)))
    m.report()
    sv.close()


def test_c2_full_size(gpu):
    """C2: int8 KV with f16 scales and 1 % outlier K channels x8, 4096
    cached positions, 128 decode steps, every step checked; the pool
    contents after the last step are bit-exact."""
    cfg = synth.configs()["c2"]
    say("C2 full size")
    sv = Serving(cfg, cfg.contexts, cfg.steps, 1, cfg.pool_pages, table_seed=None, seed=102)
    sv.fill()
    m = Margin("c2")
    for i in range(cfg.steps):
        sv.step(m, check_store=(i == cfg.steps - 1))
    m.report()
    sv.close()


def test_c3_full_size(gpu):
    """C3: four sessions of 512/2048/4096/8192 cached positions on a
    fragmented shared pool, 32 decode steps batched into one attention
    launch per step, every step checked."""
    cfg = synth.configs()["c3"]
    say("C3 full size")
    sv = Serving(cfg, cfg.contexts, cfg.steps, 1, cfg.pool_pages, table_seed=cfg.seed, seed=103)
    sv.fill()
    m = Margin("c3")
    for i in range(cfg.steps):
        rows, items, splits = sv.step(m, check_store=(i == cfg.steps - 1))
        if i == 0:
            say(f"  plan: {rows} rows, {items} work items, up to {splits} splits")
    m.report()
    sv.close()


@pytest.mark.parametrize("name", ["c1", "c2", "c3"])
def test_small_step_kernel_full_run(gpu, name):
    """C1-C3 through tge_decode_step, the path the driver's layer call and
    the bench time for these configurations: one kernel per layer-step
    (paged_step_kernel) that stores the step's rows, attends and merges its
    split contexts in the launch, re-arming its arrival counters for the
    next step. Every step of the configuration's whole run is checked
    against the oracle and the pool holds every stored row bit for bit at
    the end."""
    cfg = synth.configs()[name]
    say(f"{name} full run through the one-kernel step")
    seed = {"c1": 111, "c2": 112, "c3": 113}[name]
    pool_pages = 128 if name == "c1" else cfg.pool_pages
    table_seed = None if name == "c2" else cfg.seed
    sv = Serving(cfg, cfg.contexts, cfg.steps, 1, pool_pages, table_seed=table_seed, seed=seed)
    sv.fill()
    m = Margin(f"{name}_step")
    for i in range(cfg.steps):
        sv.step(m, kind="step", check_store=(i == cfg.steps - 1))
        assert sv.last_step_info[0] > 0, f"step {i} did not run as one kernel: {sv.last_step_info}"
    m.report()
    sv.close()


def test_c4_full_size(gpu):
    """C4: a 2048-token prompt (bf16-representable inputs) in four causal
    chunks of 512; each chunk is appended, then block-attended over every
    prior page on the MFMA path; all 2048 x 28 outputs checked, and the
    pool holds the prompt bit for bit."""
    cfg = synth.configs()["c4"]
    say("C4 full size")
    sh = cfg.shape
    rng = np.random.default_rng(104)
    total, chunk = cfg.prompt, cfg.prefill_chunk
    k, v = synth.make_kv(rng, total, sh.kv_dim, cfg)
    q = synth.make_q(rng, total, sh.q_dim, cfg)
    table = synth.fragmented_table(cfg.pool_pages, cfg.seed)
    pages = [table.allocate() for _ in range(total // 16)]
    pool = tk.KvPool(1, cfg.pool_pages, sh.kv_heads, sh.head_dim, tk.KV_F16)
    fc = flat_cache(tk.KV_F16, k, v)
    m = Margin("c4")
    for c0 in range(0, total, chunk):
        b = tk.Batch().plan(pool, [tk.Session(c0, chunk, pages)], sh.q_heads)
        dk = tk.DeviceArray.from_numpy(k[c0:c0 + chunk])
        dv = tk.DeviceArray.from_numpy(v[c0:c0 + chunk])
        dq = tk.DeviceArray.from_numpy(q[c0:c0 + chunk])
        out = tk.DeviceArray((chunk, sh.q_dim), np.float32).zero()
        b.append(pool, 0, dk, dv)
        b.prefill(pool, 0, dq, out)
        tk.hip().sync()
        m.check(out.numpy(), fc.attend(q[c0:c0 + chunk], sh.q_heads, sh.kv_heads, sh.head_dim, c0),
                f"chunk at {c0}")
        if c0 + chunk == total:
            check_pool(pool, b, 0, tk.KV_F16, fc, total)
        for a in (dk, dv, dq, out):
            a.close()
        b.close()
    m.report()
    assert tk.wait_expiries() == 0, "a bounded in-kernel wait ran out"
    pool.close()
    table.close()


def test_c5_full_size(gpu):
    """C5: the bench's 64 sessions (contexts log-uniform in [1k, 32k],
    seeded), int8 KV with f16 scales and 1 % outlier K channels x8, one
    4-query verify step over all of them; then the churn of the workload:
    8 sessions release their pages (logical order) and 8 new 2048-token
    sessions take them (LIFO reuse), and a second step runs over the
    changed batch through tge_decode_step (the decode launch attends to and
    stores the new rows, as in the bench's layer call). Every output row is checked, and
    the pool contents of the new sessions are bit-exact."""
    cfg = synth.configs()["c5"]
    say("C5 full size")
    sh = cfg.shape
    contexts = cfg.contexts
    say(f"  contexts min {min(contexts)} max {max(contexts)} total {sum(contexts)}")
    need = sum(math.ceil((c + 2 * cfg.n_new) / 16) for c in contexts)
    pool_pages = need + 8 * math.ceil((cfg.churn_context + cfg.n_new) / 16) + 64
    sv = Serving(cfg, contexts, 2, cfg.n_new, pool_pages, table_seed=None, seed=105)
    sv.fill()
    m = Margin("c5")
    rows, items, splits = sv.step(m)
    say(f"  step 1 plan: {rows} rows, {items} work items, up to {splits} splits")
    churn = sorted(np.random.default_rng(205).choice(len(contexts), cfg.churn_sessions,
                                                     replace=False).tolist())
    freed = []
    for s in churn:
        freed += sv.pages[s]
        sv.release(s)
    for s in churn:
        sv.add_session(cfg.churn_context, 1, slot=s)
    reused = sum(p in set(freed) for s in churn for p in sv.pages[s])
    assert reused == sum(len(sv.pages[s]) for s in churn), "new sessions should reuse freed pages"
    sv.fill(only=set(churn))
    rows, items, splits = sv.step(m, kind="step")
    assert sv.last_step_info == (0, 0) and sv.last_stores_rows, "the decode launch stores the rows"
    say(f"  step 2 plan: {rows} rows, {items} work items, up to {splits} splits")
    b = tk.Batch().plan(sv.pool, [tk.Session(c - cfg.n_new, cfg.n_new, p)
                                  for c, p in zip(sv.ctx, sv.pages)], sh.q_heads)
    for s in churn:
        check_pool(sv.pool, b, s, cfg.fmt, sv.fc[s], sv.ctx[s])
    b.close()
    m.report()
    sv.close()


def test_c5_span_extremes_f32_oracle_margin(gpu):
    """The f16 rounding of Q and of the softmax weights at C5's longest
    spans: sessions at 1024, 8192 and 32768 positions (int8, f16 scales,
    outlier K channels), 4-query verify, checked against the fp32 oracle
    and against float64 truth (attention_head in double), both within the
    bound."""
    cfg = synth.configs()["c5"]
    sh = cfg.shape
    say("C5 span extremes")
    sv = Serving(cfg, [1024, 8192, 32768], 1, cfg.n_new, 4200, table_seed=7, seed=106)
    sv.fill()
    n = cfg.n_new
    sess = [tk.Session(c, n, p) for c, p in zip(sv.ctx, sv.pages)]
    b = tk.Batch().plan(sv.pool, sess, sh.q_heads)
    q = synth.make_q(sv.rng, n * 3, sh.q_dim, cfg)
    dk = tk.DeviceArray.from_numpy(np.concatenate([k[c:c + n] for k, c in zip(sv.k, sv.ctx)]))
    dv = tk.DeviceArray.from_numpy(np.concatenate([v[c:c + n] for v, c in zip(sv.v, sv.ctx)]))
    dq = tk.DeviceArray.from_numpy(q)
    out = tk.DeviceArray(q.shape, np.float32).zero()
    b.append(sv.pool, 0, dk, dv)
    b.decode(sv.pool, 0, dq, out)
    tk.hip().sync()
    got = out.numpy()
    m32, m64 = Margin("c5 extremes vs fp32 oracle"), Margin("c5 extremes vs float64")
    w32 = oracle_outputs(sv.fc, q, sv.ctx, n, sh)
    w64 = oracle_outputs(sv.fc, q, sv.ctx, n, sh, f64=True)
    for s, c in enumerate(sv.ctx):
        m32.check(got[s * n:(s + 1) * n], w32[s], f"ctx {c}")
        m64.check(got[s * n:(s + 1) * n], w64[s], f"ctx {c}")
    m32.report()
    m64.report()
    # the decode output does not depend on the launch: a replay is bit-identical
    out2 = tk.DeviceArray(q.shape, np.float32).zero()
    b.decode(sv.pool, 0, dq, out2)
    tk.hip().sync()
    assert np.array_equal(bits(out2.numpy()), bits(got))
    for a in (dk, dv, dq, out, out2):
        a.close()
    b.close()
    sv.close()
