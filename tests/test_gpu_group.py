"""GPU parity of the kernel-level group call (tge_attention_group, the
reference's attention_group plugin over pages) against the oracle's
attention_group (attention_scalar.cpp:117-199, pinned bit-exact against the
reference's own scalar kernel), through the C ABI."""
import ctypes as C
import sys

import numpy as np
import pytest

import oracle as O
import tge_kv as tk
from _paged import PagedCase

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _fp(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def oracle_group(case, kv_head, first, count, queries):
    """orc_attention_group over the flat cache of session 0, positions
    [first, first + count) of KV head kv_head."""
    fc = case.flat(0)
    hd, kv = case.hd, case.kv_dim
    g = queries.shape[0]
    off = first * kv + kv_head * hd
    fmt = {tk.KV_F16: O.F16, tk.KV_I8: O.I8}[case.fmt]
    k = fc.k.reshape(-1)[off:]
    v = fc.v.reshape(-1)[off:]
    ks = fc.ks.reshape(-1)[off // 32:] if fc.ks is not None else None
    vs = fc.vs.reshape(-1)[off // 32:] if fc.vs is not None else None
    mx, sm = np.empty(g, np.float32), np.empty(g, np.float32)
    ac = np.empty(g * hd, np.float32)
    q = np.ascontiguousarray(queries, np.float32)
    O.orc().orc_attention_group(fmt, _fp(q), _fp(np.ascontiguousarray(k)), _fp(np.ascontiguousarray(v)),
                                _fp(None if ks is None else np.ascontiguousarray(ks)),
                                _fp(None if vs is None else np.ascontiguousarray(vs)),
                                kv, count, hd, g, np.float32(1.0 / np.sqrt(np.float32(hd))),
                                _fp(mx), _fp(sm), _fp(ac))
    return mx, sm, ac.reshape(g, hd)


CASES = {
    # name: (q_heads, kv_heads, head_dim, format, scale format, context, chunks)
    "f16_d64_g7": (14, 2, 64, tk.KV_F16, 0, 1100, [(0, 1100), (37, 300), (256, 512), (1099, 1)]),
    "i8_d128_g7_f16scales": (28, 4, 128, tk.KV_I8, tk.SCALE_F16, 900,
                             [(0, 900), (5, 16), (100, 611), (16, 16)]),
    "i8_d64_g1_f32scales": (2, 2, 64, tk.KV_I8, tk.SCALE_F32, 300, [(0, 300), (17, 2)]),
    "f16_d128_g16": (32, 2, 128, tk.KV_F16, 0, 700, [(0, 700), (333, 64)]),
    # head sizes the pool pads to the block width
    "f16_d80_g7": (14, 2, 80, tk.KV_F16, 0, 500, [(0, 500), (33, 100)]),
    "i8_d96_g4_f32scales": (16, 4, 96, tk.KV_I8, tk.SCALE_F32, 400, [(0, 400), (7, 64)]),
    "f16_d256_g8": (16, 2, 256, tk.KV_F16, 0, 300, [(0, 300), (40, 90)]),
    "i8_d256_g4": (8, 2, 256, tk.KV_I8, tk.SCALE_F16, 300, [(0, 300), (5, 70)]),
}


@pytest.mark.parametrize("name", list(CASES))
def test_attention_group_matches_oracle(gpu, name):
    qh, kvh, hd, fmt, sf, ctx, chunks = CASES[name]
    say(f"attention_group case {name}")
    case = PagedCase(qh, kvh, hd, fmt, [ctx], 1, scale_format=sf, seed=61, outlier_frac=0.01)
    case.fill()
    g = qh // kvh
    rng = np.random.default_rng(62)
    for kv_head in range(kvh):
        q = rng.standard_normal((g, hd)).astype(np.float32)
        for first, count in chunks:
            m, s, a = tk.attention_group(case.pool, 0, kv_head, case.pages[0], first, count, q)
            rm, rs, ra = oracle_group(case, kv_head, first, count, q)
            # the same running state up to fp32 summation order and exp
            assert np.all(np.abs(m - rm) <= 1e-5 * (1 + np.abs(rm))), (first, count, m, rm)
            assert np.all(np.abs(s - rs) <= 1e-4 * rs), (first, count, s, rs)
            assert np.all(np.abs(a - ra) <= 1e-4 * rs[:, None]), (first, count)
            # the normalised output: the product's attention tolerance
            np.testing.assert_allclose(a / s[:, None], ra / rs[:, None], atol=2e-3, rtol=1e-3)
    case.close()


def test_attention_group_empty_chunk_and_bad_page(gpu):
    case = PagedCase(14, 2, 64, tk.KV_F16, [40], 1, seed=63)
    case.fill()
    q = np.ones((7, 64), np.float32)
    m, s, a = tk.attention_group(case.pool, 0, 1, case.pages[0], 3, 0, q)
    assert np.all(m == -np.inf) and np.all(s == 0) and np.all(a == 0)
    bad = list(case.pages[0])
    bad[1] = case.pool.pages  # outside the pool: not read, outputs NaN
    m, s, a = tk.attention_group(case.pool, 0, 0, bad, 0, 40, q)
    assert np.all(np.isnan(m)) and np.all(np.isnan(s)) and np.all(np.isnan(a))
    with pytest.raises(tk.TgeError) as e:
        tk.attention_group(case.pool, 0, 2, case.pages[0], 0, 40, q)  # kv_head 2 of 2
    assert e.value.status == tk.ERR_INVALID
    with pytest.raises(tk.TgeError) as e:  # first + count past INT_MAX
        tk.attention_group(case.pool, 0, 0, case.pages[0], 2**31 - 10, 20, q)
    assert e.value.status == tk.ERR_INVALID
    assert "overflow" in tk.lib().tge_last_error().decode()
    case.close()
