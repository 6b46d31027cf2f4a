"""GPU parity of tge_decode_step (append + decode attention in one call; a
small step is one kernel that stores the new rows, attends and merges its
split contexts in-kernel) against the oracle: pool contents bit for bit,
attention within max-abs 2e-3 / rel 1e-3."""
import sys

import numpy as np
import pytest

import synth
import tge_kv as tk
from _paged import PagedCase
from _util import assert_attention_close, bits
from test_gpu_kv import check_contents

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


STEP_CASES = {
    # name: (q_heads, kv_heads, hd, fmt, sf, contexts, n_new, outliers)
    "c1_shape": (14, 2, 64, tk.KV_F16, 0, [1024], 1, 0),
    "c2_shape_i8": (14, 2, 64, tk.KV_I8, 0, [4096], 1, 0.01),
    "c3_shape": (12, 2, 128, tk.KV_F16, 0, [512, 2048, 4096, 8192], 1, 0),
    "verify_i8_f32_scales": (28, 4, 128, tk.KV_I8, 1, [700, 35, 1500], 4, 0.01),
    "span_edges": (8, 2, 64, tk.KV_F16, 0, [0, 15, 16, 17, 31, 32, 255, 256, 257], 1, 0),
    "verify_six_page_cross": (14, 2, 64, tk.KV_I8, 0, [13, 510, 1000], 6, 0),
}


@pytest.mark.parametrize("name", list(STEP_CASES))
def test_step_matches_oracle(gpu, name):
    qh, kvh, hd, fmt, sf, ctx, nn, out = STEP_CASES[name]
    say(f"step case {name}")
    case = PagedCase(qh, kvh, hd, fmt, ctx, nn, scale_format=sf, seed=31, outlier_frac=out)
    case.fill()
    got, b = case.step(kind="step")
    assert b.step_info()[0] > 0, "the step ran the append + decode kernels"
    err = assert_attention_close(got, case.oracle_out(), name)
    say(f"  max abs err {err:.2e}")
    b.close()
    check_contents(case)
    case.close()


SPARSE_STEP_CASES = {
    # name: (q_heads, kv_heads, hd, fmt, sf, contexts, n_new, (sink, window, stride), one kernel)
    "c1_shape_stride4": (14, 2, 64, tk.KV_F16, 0, [1024], 1, (4, 512, 4), True),
    "c2_shape_i8_stride37": (14, 2, 64, tk.KV_I8, 0, [4096], 1, (4, 512, 37), True),
    "c3_shape_stride5": (12, 2, 128, tk.KV_F16, 0, [512, 2048, 4096, 8192], 1, (4, 512, 5), True),
    "verify_i8_sink_straddles": (28, 4, 128, tk.KV_I8, 0, [700, 35, 1500, 3000], 4, (20, 40, 17), True),
    "verify_i8_f32_scales": (28, 4, 128, tk.KV_I8, 1, [700, 35, 1500], 4, (4, 64, 3), False),
}


@pytest.mark.parametrize("name", list(SPARSE_STEP_CASES))
def test_sparse_step_matches_oracle(gpu, name):
    """A static sparse subset (sink + strided middle + window, the kept set
    of build_sparse_index, qwen2.cpp:192-220) on tge_decode_step: small
    steps stay one kernel (the sparse variant of the step kernel; int8
    pages with fp32 scales at 32 rows and more take the append and sparse
    decode kernels instead), against the oracle's sparse head, pool
    contents bit for bit."""
    qh, kvh, hd, fmt, sf, ctx, nn, sparse, one = SPARSE_STEP_CASES[name]
    say(f"sparse step case {name}")
    case = PagedCase(qh, kvh, hd, fmt, ctx, nn, scale_format=sf, seed=33, outlier_frac=0.01)
    case.fill()
    case.sparse = sparse
    got, b = case.step(kind="step")
    assert (b.step_info()[0] > 0) == one, b.step_info()
    err = assert_attention_close(got, case.oracle_out(), name)
    say(f"  max abs err {err:.2e}")
    b.close()
    case.sparse = None
    check_contents(case)
    case.close()


def test_step_split_counters_across_layers(gpu):
    """A context cut into the most pieces, run on three layers in a row and
    twice on one layer: every launch's last piece merges and resets its
    segment counter, so each launch matches the oracle and a repeat is
    bit-identical."""
    case = PagedCase(12, 2, 128, tk.KV_F16, [8000, 300], 2, seed=44, layers=3)
    for layer in range(3):
        case.fill(layer)
    outs = []
    for layer in (0, 1, 2, 2):
        got, b = case.step(layer=layer, kind="step")
        # 500 context pages in pieces of 16, then the page of the new rows
        assert b.step_info()[1] == 33
        assert_attention_close(got, case.oracle_out(), f"layer {layer}")
        outs.append(got)
        b.close()
    assert np.array_equal(bits(outs[2]), bits(outs[3]))
    case.close()


def test_step_pieces_of_several_batches(gpu):
    """A context long enough that one batch per wave would need more than 64
    pieces: pieces of two batches, every wave loading twice."""
    case = PagedCase(8, 1, 64, tk.KV_F16, [48000], 1, seed=46)
    case.fill()
    got, b = case.step(kind="step")
    wg, pieces = b.step_info()
    assert wg == pieces and 32 < pieces <= 64, (wg, pieces)
    assert_attention_close(got, case.oracle_out(), "two-batch pieces")
    b.close()
    check_contents(case)
    case.close()


def _random_step_case(i):
    r = np.random.default_rng(7000 + i)
    kvh = int(r.choice([1, 2, 4, 8]))
    hd = int(r.choice([64, 128]))
    group = int(r.integers(1, 9))
    fmt = int(r.choice([tk.KV_F16, tk.KV_I8]))
    sf = int(r.choice([tk.SCALE_F16, tk.SCALE_F32])) if fmt == tk.KV_I8 else tk.SCALE_F16
    n_s = int(r.integers(1, 6))
    # rows per unit the one-kernel step holds (step_fits)
    cap = 64 if hd == 64 else (32 if fmt == tk.KV_I8 and sf == tk.SCALE_F32 else 48)
    max_q = max(1, cap // group)
    contexts = [int(r.choice([0, int(r.integers(1, 400)), int(r.integers(400, 3000))]))
                for _ in range(n_s)]
    n_new = [int(r.integers(1, min(6, max_q) + 1)) for _ in range(n_s)]
    return dict(qh=kvh * group, kvh=kvh, hd=hd, fmt=fmt, sf=sf, contexts=contexts, n_new=n_new)


@pytest.mark.parametrize("i", range(16))
def test_random_steps(gpu, i):
    """Sixteen seeded random small steps (heads, head_dim, formats, empty and
    ragged contexts, 1-6 new rows per session) through tge_decode_step:
    pool contents bit-exact, attention against the oracle."""
    c = _random_step_case(i)
    say(f"random step {i}: {c}")
    case = PagedCase(c["qh"], c["kvh"], c["hd"], c["fmt"], c["contexts"], c["n_new"],
                     scale_format=c["sf"], seed=8000 + i,
                     outlier_frac=0.01 if c["fmt"] == tk.KV_I8 else 0)
    case.fill()
    got, b = case.step(kind="step")
    assert b.step_info()[0] > 0
    err = assert_attention_close(got, case.oracle_out(), f"random step {i}")
    say(f"  max abs err {err:.2e}")
    b.close()
    check_contents(case)
    case.close()


def test_step_large_falls_back(gpu):
    """A step above the one-launch size (more than 4096 page blocks) runs the
    append, the persistent decode kernel and its merge: same results."""
    case = PagedCase(28, 4, 128, tk.KV_I8, [9000, 9000], 4, seed=45, outlier_frac=0.01)
    case.fill()
    got, b = case.step(kind="step")
    assert b.step_info() == (0, 0)
    assert_attention_close(got, case.oracle_out(), "large step")
    b.close()
    check_contents(case)
    case.close()


def test_batch_planned_for_another_format_is_refused(gpu):
    """A batch planned on an int8 pool and used on an f16 pool of the same
    shape (or with the other scale format) is refused: the one-launch step's
    page batches depend on the storage format."""
    say("step: batch planned for another format")
    qh, kvh, hd = 14, 2, 64
    p_i8 = tk.KvPool(1, 8, kvh, hd, tk.KV_I8, tk.SCALE_F16)
    p_i8f32 = tk.KvPool(1, 8, kvh, hd, tk.KV_I8, tk.SCALE_F32)
    p_f16 = tk.KvPool(1, 8, kvh, hd, tk.KV_F16)
    q = tk.DeviceArray((1, qh * hd), np.float32).zero()
    k = tk.DeviceArray((1, kvh * hd), np.float32).zero()
    v = tk.DeviceArray((1, kvh * hd), np.float32).zero()
    out = tk.DeviceArray((1, qh * hd), np.float32).zero()
    b = tk.Batch().plan(p_i8, [tk.Session(40, 1, [0, 1, 2])], qh)
    L = tk.lib()
    for other in (p_f16, p_i8f32):
        st = L.tge_decode_step(b.h, other.h, 0, q.ptr, k.ptr, v.ptr, out.ptr, None)
        assert st == tk.ERR_INVALID, st
        assert "another pool" in L.tge_last_error().decode()
        assert L.tge_kv_append(b.h, other.h, 0, k.ptr, v.ptr, None) == tk.ERR_INVALID
    # the pool it was planned for still works
    assert L.tge_decode_step(b.h, p_i8.h, 0, q.ptr, k.ptr, v.ptr, out.ptr, None) == tk.OK
    tk.hip().sync()
    assert np.all(np.isfinite(out.numpy()))
    b.close()
    for a in (q, k, v, out):
        a.close()
    for pl in (p_i8, p_i8f32, p_f16):
        pl.close()


LARGE_STEP_CASES = {
    # name: (q_heads, kv_heads, hd, fmt, sf, contexts, n_new, the decode
    # launch stores the rows); each above 4096 page blocks, so
    # tge_decode_step runs the persistent decode kernel: it writes the new
    # rows of the pages each wave reads into the wave's copy of the page and
    # stores them into the pool, or (head_dim 256, more than 32 rows per
    # unit, too many rows on one wave's pages) the append runs first.
    "verify_i8": (28, 4, 128, tk.KV_I8, 0, [9000, 37, 5000, 15, 3000, 300], 4, True),
    "f16_d64_ragged": (6, 2, 64, tk.KV_F16, 0, [20000, 12000, 31, 16, 17, 2047], [9, 1, 2, 9, 3, 5],
                       True),
    # 63 rows per unit (four row groups): the append runs first
    "f16_d64_wide_group": (14, 2, 64, tk.KV_F16, 0, [20000, 12000, 31, 16, 17, 2047], [9, 1, 2, 9, 3, 5],
                           False),
    "i8_f32_group1": (8, 8, 128, tk.KV_I8, 1, [9000, 1, 255, 40, 600], 8, True),
    "short_sessions_first_pages": (28, 4, 128, tk.KV_I8, 0, [17000, 20, 3, 45, 0, 16], 4, True),
    "d256_append_first": (12, 2, 256, tk.KV_F16, 0, [30000, 5000, 8, 100], 8, False),
    # a head off the 16-dim grid (100 dims in 128-dim blocks): the decode
    # launch reads and stores the rows' own dims in runs of 4
    "f16_d100_verify": (28, 4, 100, tk.KV_F16, 0, [9000, 37, 5000, 15, 3000, 300], 4, True),
    # many short sessions: shares of many units; more rows on one wave's
    # pages than it holds, so the append runs first
    "many_short": (28, 4, 128, tk.KV_I8, 0, [int(x) for x in np.random.default_rng(5).integers(0, 60, 160)]
                   + [12000], 4, None),
}


@pytest.mark.parametrize("name", list(LARGE_STEP_CASES))
def test_large_step_stores_rows_in_decode(gpu, name):
    """A large step through tge_decode_step: pool contents bit-exact against
    the oracle, attention against the oracle, and outputs bit-identical to
    the separate append followed by tge_decode_attention on a second pool of
    the same case; the path taken is the one the case names."""
    qh, kvh, hd, fmt, sf, ctx, nn, folds = LARGE_STEP_CASES[name]
    say(f"large step case {name}")
    out = {}
    for kind in ("step", "decode"):
        case = PagedCase(qh, kvh, hd, fmt, ctx, nn, scale_format=sf, seed=61,
                         outlier_frac=0.01 if fmt == tk.KV_I8 else 0)
        case.fill()
        got, b = case.step(kind=kind)
        assert b.step_info() == (0, 0), "a large step"
        if kind == "step":
            stores = b.decode_stores_rows()
            say(f"  decode launch stores the rows: {stores}")
            if folds is not None:
                assert stores == folds
        out[kind] = got
        b.close()
        if kind == "step":
            err = assert_attention_close(got, case.oracle_out(), name)
            say(f"  max abs err {err:.2e}")
            check_contents(case)
        case.close()
    assert np.array_equal(bits(out["step"]), bits(out["decode"])), "fused and separate append differ"
