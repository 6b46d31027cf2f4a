"""GPU parity of the KV append (bit-exact) and attention (tolerance) against
the CPU oracle, through the C ABI. Runs on a gfx950 device."""
import math
import sys

import numpy as np
import pytest

import oracle as O
import synth
import tge_kv as tk
from _paged import PagedCase
from _util import assert_attention_close, bits

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def raw_pool_rows(case, layer, s, count):
    """Decode positions [0, count) of session s straight from the pool bytes
    with the documented layout formulas (independent of tge_kv_gather); the
    dims of a block past the head's own must hold zeros (codes, bits and
    the scales of whole padding blocks)."""
    view = case.pool.layer(layer)
    pages = case.pool.pages
    W = view.block_dims
    assert W == (64 if case.hd <= 64 else 128 if case.hd <= 128 else 256)
    elem = np.uint16 if case.fmt == tk.KV_F16 else np.int8
    esz = np.dtype(elem).itemsize
    bb = view.block_bytes
    assert view.v - view.k == 16 * W * esz == view.kv_block_bytes
    sbytes = 0
    if case.fmt == tk.KV_I8:
        sbytes = 16 * (W // 32) * (4 if case.sf == tk.SCALE_F32 else 2)
        assert view.scale_block_bytes == sbytes and bb == 2 * view.kv_block_bytes + 2 * sbytes
        assert view.k_scales - view.k == 2 * view.kv_block_bytes
        assert view.v_scales - view.k_scales == sbytes
    else:
        assert bb == 2 * view.kv_block_bytes and not view.k_scales
    raw = tk.hip().download(view.k, np.empty(pages * case.kvh * bb, np.uint8))
    t = np.arange(16)[:, None]
    d = np.arange(W)[None, :]
    n = W // 32
    pe = 16 // esz  # elements per 16-byte piece; piece i of lane l at (64 i + l) pe
    kl, kj = ((d >> 2) & 3) * 16 + t, (d >> 5) * 8 + (((d >> 4) & 1) << 2) + (d & 3)
    vl, vj = (t >> 2) * 16 + (d & 15), (d >> 5) * 8 + (((d >> 4) & 1) << 2) + (t & 3)
    kidx = ((kj // pe) * 64 + kl) * pe + kj % pe
    vidx = ((vj // pe) * 64 + vl) * pe + vj % pe
    sidx = ((t >> 2) * n + np.arange(n)[None, :]) * 4 + (t & 3)
    k = np.empty((count, case.kv_dim), elem)
    v = np.empty((count, case.kv_dim), elem)
    for pos0 in range(0, count, 16):
        page = case.pages[s][pos0 // 16]
        n_t = min(16, count - pos0)
        for h in range(case.kvh):
            blk = raw[(page * case.kvh + h) * bb:(page * case.kvh + h + 1) * bb]
            kpart = blk[:view.kv_block_bytes].view(elem)[kidx][:n_t]
            vpart = blk[view.kv_block_bytes:2 * view.kv_block_bytes].view(elem)[vidx][:n_t]
            k[pos0:pos0 + n_t, h * case.hd:(h + 1) * case.hd] = kpart[:, :case.hd]
            v[pos0:pos0 + n_t, h * case.hd:(h + 1) * case.hd] = vpart[:, :case.hd]
            assert not kpart[:, case.hd:].any() and not vpart[:, case.hd:].any(), "padding dims"
            if sbytes and case.hd < W:
                sc = blk[2 * view.kv_block_bytes:].view(np.uint8)
                ks = sc[:sbytes].view(np.uint16 if case.sf != tk.SCALE_F32 else np.uint32)
                vs = sc[sbytes:2 * sbytes].view(ks.dtype)
                pad = sidx[:n_t, case.hd // 32:]
                assert not ks[pad].any() and not vs[pad].any(), "padding scales"
    return k, v


def check_contents(case, layer=0):
    b = tk.Batch().plan(case.pool, case.sessions(True), case.qh)
    for s in range(len(case.contexts)):
        total = case.contexts[s] + case.n_new[s]
        fc = O.FlatCache({tk.KV_F16: O.F16, tk.KV_I8: O.I8}[case.fmt], case.k[s], case.v[s])
        gk, gv, gks, gvs = b.gather(case.pool, layer, s, total)
        assert np.array_equal(gk, fc.k.view(gk.dtype)), f"K bits differ, session {s}"
        assert np.array_equal(gv, fc.v.view(gv.dtype)), f"V bits differ, session {s}"
        if case.fmt == tk.KV_I8:
            if case.sf == tk.SCALE_F32:
                assert np.array_equal(bits(gks), bits(fc.ks)) and np.array_equal(bits(gvs), bits(fc.vs))
            else:
                assert np.array_equal(gks, O.float_to_half(fc.ks))
                assert np.array_equal(gvs, O.float_to_half(fc.vs))
        rk, rv = raw_pool_rows(case, layer, s, total)
        assert np.array_equal(rk, gk) and np.array_equal(rv, gv)
    b.close()


# ---------------------------------------------------------------------------
# append
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("fmt,sf,kvh,hd", [(tk.KV_F16, 0, 2, 64), (tk.KV_F16, 0, 4, 128),
                                           (tk.KV_I8, 0, 2, 64), (tk.KV_I8, 1, 4, 128),
                                           (tk.KV_I8, 0, 4, 128)])
def test_append_bitexact(gpu, fmt, sf, kvh, hd):
    say(f"append fmt={fmt} sf={sf} kvh={kvh} hd={hd}")
    case = PagedCase(kvh * 7, kvh, hd, fmt, [37, 0, 100], [3, 5, 1], scale_format=sf, seed=11,
                     outlier_frac=0.01 if fmt == tk.KV_I8 else 0)
    case.fill()
    case.step()
    check_contents(case)
    case.close()


def edge_values(n, rng):
    f = lambda u: np.array(u, np.uint32).view(np.float32)
    special = np.concatenate([
        f([0x00000000, 0x80000000, 0x7F800000, 0xFF800000, 0x7FC00000, 0xFFC00001, 0x7F800001,
           0x33000000, 0x33000001, 0x337FFFFF, 0x33800000, 0x33C00000, 0x387FE000, 0x38800000,
           0x477FEFFF, 0x477FF000, 0x477FE000, 0x3F801000, 0x3F803000, 0x3F800FFF, 0x00000001]),
        np.array([65504, 65519, 65520, 1e-8, -1e-8, 6e-5, 6.1e-5, 3.0e38, -3e38], np.float32)])
    x = rng.standard_normal(n).astype(np.float32)
    x[:special.size] = special
    return x


def test_append_f16_edge_and_structured_values(gpu):
    """Rounding-critical inputs through the real append kernel: every sign,
    exponent and top-10 mantissa bit pattern combined with dropped-bit
    patterns {0, 0x0FFF, 0x1000, 0x1001, 0x1FFF}, plus NaN/inf/subnormal
    specials; must equal the oracle's bits (which are pinned exhaustively
    against the reference build)."""
    hi = (np.arange(1 << 19, dtype=np.uint32) << 13)
    low = np.array([0, 0x0FFF, 0x1000, 0x1001, 0x1FFF], np.uint32)
    xs = (hi[:, None] | low[None, :]).reshape(-1).view(np.float32)
    rng = np.random.default_rng(3)
    xs = np.concatenate([edge_values(4096, rng), xs,
                         rng.integers(0, 2 ** 32, 1 << 20, dtype=np.uint64).astype(np.uint32).view(np.float32)])
    kv_dim = 128
    rows = math.ceil(xs.size / kv_dim)
    xs = np.resize(xs, rows * kv_dim).reshape(rows, kv_dim)
    pages = math.ceil(rows / 16)
    pool = tk.KvPool(1, pages, 1, 128, tk.KV_F16)
    sess = [tk.Session(0, rows, list(range(pages)))]
    b = tk.Batch().plan(pool, sess, 1)
    dk = tk.DeviceArray.from_numpy(xs)
    dv = tk.DeviceArray.from_numpy(-xs)
    b.append(pool, 0, dk, dv)
    tk.hip().sync()
    gk, gv, _, _ = b.gather(pool, 0, 0, rows)
    assert np.array_equal(gk, O.float_to_half(xs))
    assert np.array_equal(gv, O.float_to_half(-xs))
    pool.close()


def test_append_i8_edge_blocks(gpu):
    rng = np.random.default_rng(5)
    rows, kv_dim = 64, 64
    x = rng.standard_normal((rows, kv_dim)).astype(np.float32)
    x[0] = 0.0
    x[1] = 0.0
    x[1, 31] = -0.0
    x[1, 63] = -0.0
    below = np.nextafter(np.float32(0.5), np.float32(0))
    x[2, :] = 0
    x[2, 0], x[2, 1], x[2, 2], x[2, 3], x[2, 4] = 127, below, -below, 2.5, -2.5
    x[3] *= np.float32(1e-38)
    x[4] *= np.float32(1e35)
    x[5, 5] = np.inf
    x[6, 40] = np.nan
    x[7] = np.arange(64, dtype=np.float32) - 32
    for sf in (tk.SCALE_F32, tk.SCALE_F16):
        pool = tk.KvPool(1, 4, 1, 64, tk.KV_I8, sf)
        b = tk.Batch().plan(pool, [tk.Session(0, rows, [3, 0, 2, 1])], 1)
        dk, dv = tk.DeviceArray.from_numpy(x), tk.DeviceArray.from_numpy(x[::-1].copy())
        b.append(pool, 0, dk, dv)
        tk.hip().sync()
        gk, gv, gks, gvs = b.gather(pool, 0, 0, rows)
        ck, sk = O.quantize_rows(x)
        cv, sv = O.quantize_rows(x[::-1].copy())
        assert np.array_equal(gk, ck) and np.array_equal(gv, cv)
        if sf == tk.SCALE_F32:
            assert np.array_equal(bits(gks), bits(sk)) and np.array_equal(bits(gvs), bits(sv))
        else:
            assert np.array_equal(gks, O.float_to_half(sk)) and np.array_equal(gvs, O.float_to_half(sv))
        pool.close()


def test_append_i8_rounding_closed_forms(gpu):
    # Blocks whose codes change if the quantizer fuses x*inv +- 0.5 into one
    # multiply-add, and blocks whose codes change if they are derived from
    # the f16-rounded scale (expected codes from exact arithmetic,
    # tests/_quant_cases.py); K gets one kind, V the other.
    from _quant_cases import contraction_blocks, f16_scale_blocks
    kb, kc = contraction_blocks(32, seed=11)
    vb, vc, vs16 = f16_scale_blocks(32, seed=12)
    rows, kv_dim = 8, 128
    k = kb.reshape(rows, kv_dim)
    v = vb.reshape(rows, kv_dim)
    for sf in (tk.SCALE_F16, tk.SCALE_F32):
        say(f"append rounding closed forms, scale format {sf}")
        pool = tk.KvPool(1, 2, 1, kv_dim, tk.KV_I8, sf)
        b = tk.Batch().plan(pool, [tk.Session(0, rows, [1])], 1)
        b.append(pool, 0, tk.DeviceArray.from_numpy(k), tk.DeviceArray.from_numpy(v))
        tk.hip().sync()
        gk, gv, _, gvs = b.gather(pool, 0, 0, rows)
        assert np.array_equal(gk.reshape(-1, 32), kc)
        assert np.array_equal(gv.reshape(-1, 32), vc)
        if sf == tk.SCALE_F16:
            assert np.array_equal(gvs.reshape(-1), vs16)
        pool.close()


# ---------------------------------------------------------------------------
# attention
# ---------------------------------------------------------------------------
ATTN_CASES = {
    # name: (q_heads, kv_heads, hd, fmt, sf, contexts, n_new, outliers)
    "c1_shape_f16": (14, 2, 64, tk.KV_F16, 0, [1024], 1, 0),
    "c2_shape_i8": (14, 2, 64, tk.KV_I8, 0, [700], 1, 0.01),
    "c3_shape_multi": (12, 2, 128, tk.KV_F16, 0, [31, 512, 1200, 16], 1, 0),
    "c5_shape_verify": (28, 4, 128, tk.KV_I8, 0, [40, 1000, 17, 300], 4, 0.01),
    "i8_f32_scales": (14, 2, 64, tk.KV_I8, 1, [257, 64], 2, 0),
    "verify_six": (14, 2, 64, tk.KV_F16, 0, [90, 13], 6, 0),
    "span_edges": (8, 2, 64, tk.KV_F16, 0, [0, 15, 16, 17, 31, 32], 1, 0),
}


@pytest.mark.parametrize("name", list(ATTN_CASES))
def test_decode_matches_oracle(gpu, name):
    qh, kvh, hd, fmt, sf, ctx, nn, out = ATTN_CASES[name]
    say(f"decode case {name}")
    case = PagedCase(qh, kvh, hd, fmt, ctx, nn, scale_format=sf, seed=21, outlier_frac=out)
    case.fill()
    got, b = case.step()
    want = case.oracle_out()
    err = assert_attention_close(got, want, name)
    say(f"  max abs err {err:.2e}, plan {b.info()}")
    case.close()


def test_decode_span_one_is_exact(gpu):
    case = PagedCase(14, 2, 64, tk.KV_F16, [0, 0], 1, seed=3)
    got, _ = case.step()
    want = case.oracle_out()
    assert np.array_equal(got, want)
    case.close()


def test_decode_split_k_long_context(gpu):
    """A long context is split over many workgroups and merged by the
    reduction pass; the result still matches the oracle."""
    case = PagedCase(28, 4, 128, tk.KV_F16, [20000], 1, seed=9)
    case.fill()
    got, b = case.step()
    rows, items, splits = b.info()
    assert splits > 1, b.info()
    assert_attention_close(got, case.oracle_out(), "split-k")
    case.close()


def test_decode_many_splits_merge(gpu):
    """Contexts from one page to 30k tokens in one batch: the merge runs
    over hundreds of splits per unit (eight slots per row) next to unsplit
    sessions."""
    case = PagedCase(14, 2, 64, tk.KV_F16, [30000, 5, 700, 3000], 1, seed=12)
    case.fill()
    got, b = case.step()
    rows, items, splits = b.info()
    assert splits >= 32, b.info()
    assert_attention_close(got, case.oracle_out(), "many splits")
    case.close()


def test_kernel_timing_record(gpu):
    """tge_batch_set_profiling / tge_batch_kernel_times: calls issued back
    to back are all recorded; enabling again clears the record."""
    case = PagedCase(14, 2, 64, tk.KV_I8, [2000, 300], 2, seed=13)
    case.fill()
    got, b = case.step()
    dq = tk.DeviceArray.from_numpy(case.q)
    dout = tk.DeviceArray((case.q.shape[0], case.qh * case.hd), np.float32).zero()
    b.set_profiling(True)
    for _ in range(3):
        b.decode(case.pool, 0, dq, dout)
    n, att_us, merge_us = b.kernel_times()
    assert n == 3 and att_us > 0.0 and merge_us >= 0.0, (n, att_us, merge_us)
    assert np.array_equal(bits(dout.numpy()), bits(got))
    b.set_profiling(True)
    assert b.kernel_times() == (0, 0.0, 0.0)
    b.set_profiling(False)
    dq.close()
    dout.close()
    case.close()


def test_decode_64_rows(gpu):
    """n_new * group = 64 rows (four 16-row groups per unit)."""
    case = PagedCase(16, 2, 128, tk.KV_I8, [333, 50], 8, seed=4)
    case.fill()
    got, _ = case.step()
    assert_attention_close(got, case.oracle_out(), "64 rows")
    case.close()


def test_decode_rejects_more_than_64_rows(gpu):
    case = PagedCase(16, 2, 64, tk.KV_F16, [10], 9, seed=4)
    with pytest.raises(tk.TgeError) as e:
        case.step()
    assert e.value.status == tk.ERR_INVALID
    case.close()


def test_page_permutation_invariance(gpu):
    """The same logical rows stored in two different page assignments give
    bit-identical attention outputs (the work split depends on logical
    positions only)."""
    outs = []
    for tseed in (1, 2):
        case = PagedCase(14, 2, 64, tk.KV_I8, [500, 77], 2, seed=30, pool_pages=64,
                         table=synth.fragmented_table(64, tseed))
        case.fill()
        got, _ = case.step()
        outs.append((got, case.pages))
        case.close()
    assert outs[0][1] != outs[1][1], "the two tables should place pages differently"
    assert np.array_equal(bits(outs[0][0]), bits(outs[1][0]))


def test_decode_many_units_per_workgroup(gpu):
    """Sixty sessions of a few pages each give every workgroup more units
    than its LDS table of Q operands holds, so the table is reloaded
    mid-share; results match the oracle and are bit-reproducible."""
    ctx = [17 + 23 * i for i in range(60)]
    case = PagedCase(28, 4, 128, tk.KV_I8, ctx, 4, seed=41, outlier_frac=0.01)
    case.fill()
    want = case.oracle_out()
    outs = []
    for _ in range(2):
        out, b = case.step()
        say(f"  plan {b.info()}")
        assert b.info()[1] > 4 * 64, "expected several units per workgroup"
        assert_attention_close(out, want, "many units")
        outs.append(out)
        b.close()
    assert np.array_equal(bits(outs[0]), bits(outs[1]))
    case.close()


def test_decode_short_units_mixed_rows(gpu):
    """Units shorter than a wave's page ring with mixed row counts: eighty
    sessions of 0-50 cached positions with 1-6 new tokens (7-42 rows, one to
    three 16-row groups), so a workgroup's share holds many one- to
    four-page units whose pages cross unit boundaries in the ring, and the
    Q table is reloaded mid-share. Matches the oracle and is
    bit-reproducible."""
    r = np.random.default_rng(77)
    ctx = [int(x) for x in r.integers(0, 51, 80)]
    nn = [int(x) for x in r.integers(1, 7, 80)]
    nn[0] = 6  # at least one unit of three row groups
    case = PagedCase(28, 4, 128, tk.KV_I8, ctx, nn, seed=43, outlier_frac=0.01)
    case.fill()
    want = case.oracle_out()
    outs = []
    for _ in range(2):
        out, b = case.step()
        say(f"  plan {b.info()}")
        assert_attention_close(out, want, "row-split short units")
        outs.append(out)
        b.close()
    assert np.array_equal(bits(outs[0]), bits(outs[1]))
    case.close()


def test_prefill_chunks_match_oracle(gpu):
    """Chunked prefill (7B shapes, reduced length): 3 causal chunks of 96
    appended then block-attended over all prior pages."""
    qh, kvh, hd = 28, 4, 128
    rng = np.random.default_rng(8)
    total, chunk = 288, 96
    k = synth.to_bf16_representable(rng.standard_normal((total, kvh * hd)).astype(np.float32))
    v = synth.to_bf16_representable(rng.standard_normal((total, kvh * hd)).astype(np.float32))
    q = synth.to_bf16_representable(rng.standard_normal((total, qh * hd)).astype(np.float32))
    table = synth.fragmented_table(32, 5)
    pages = [table.allocate() for _ in range(total // 16)]
    pool = tk.KvPool(1, 32, kvh, hd, tk.KV_F16)
    fc = O.FlatCache(O.F16, k, v)
    for c0 in range(0, total, chunk):
        b = tk.Batch().plan(pool, [tk.Session(c0, chunk, pages)], qh)
        dk = tk.DeviceArray.from_numpy(k[c0:c0 + chunk])
        dv = tk.DeviceArray.from_numpy(v[c0:c0 + chunk])
        dq = tk.DeviceArray.from_numpy(q[c0:c0 + chunk])
        dout = tk.DeviceArray((chunk, qh * hd), np.float32).zero()
        b.append(pool, 0, dk, dv)
        b.prefill(pool, 0, dq, dout)
        tk.hip().sync()
        want = fc.attend(q[c0:c0 + chunk], qh, kvh, hd, c0)
        err = assert_attention_close(dout.numpy(), want, f"prefill chunk at {c0}")
        say(f"  prefill chunk {c0}: max abs err {err:.2e}")
    pool.close()


# Block prefill at head_dim 128 in both tile widths: (q_heads, kv_heads,
# format, contexts, n_new). On 256 compute units the planner takes 128-row
# tiles for the "wide" cases (144 items; 280 as 64-row tiles), unsplit
# 64-row tiles where the 128-row ones would be split and merged (136
# pieces of 68 tiles; 136 narrow items; f16 only: int8 keeps the split
# 128-row tiles) and 64-row tiles for a small step (56 items).
TILE_CASES = {
    "wide_f16": (16, 8, tk.KV_F16, [0], [1100]),
    "wide_i8": (16, 8, tk.KV_I8, [0], [1100]),
    "narrow_unsplit_f16": (28, 4, tk.KV_F16, [1500], [300]),
    "wide_split_i8": (28, 4, tk.KV_I8, [1500], [300]),
    "narrow_small_i8": (28, 4, tk.KV_I8, [200, 0], [150, 90]),
}


@pytest.mark.parametrize("name", list(TILE_CASES))
def test_prefill_tile_widths(gpu, name):
    """128-row and 64-row block-prefill tiles (the planner's choice by step
    size) against the oracle, stored rows bit-exact."""
    qh, kvh, fmt, contexts, n_new = TILE_CASES[name]
    say(f"prefill tiles {name}: contexts {contexts} n_new {n_new}")
    case = PagedCase(qh, kvh, 128, fmt, contexts, n_new, seed=7400 + len(name),
                     outlier_frac=0.01 if fmt == tk.KV_I8 else 0)
    case.fill()
    got, b = case.step(kind="prefill")
    err = assert_attention_close(got, case.oracle_out(), f"prefill tiles {name}")
    say(f"  max abs err {err:.2e}")
    assert tk.wait_expiries() == 0, "a bounded in-kernel wait ran out"
    b.close()
    check_contents(case)
    case.close()


@pytest.mark.parametrize("fmt", [tk.KV_F16, tk.KV_I8])
def test_pool_layer_beyond_4gib(gpu, fmt):
    """One layer's block array past 4 GiB: the kernels address each page
    block by its 64-bit address, so a session whose pages alternate between
    the array's last 20,000 pages (byte offsets above 4 GiB) and its first
    1,000 appends, block-prefills and decodes like any other."""
    qh, kvh, hd = 14, 2, 128
    n_pages = 300_000 if fmt == tk.KV_F16 else 600_000  # 8192 or 4352 B blocks
    pool = tk.KvPool(1, n_pages, kvh, hd, fmt, tk.SCALE_F16)
    block_bytes = 8192 if fmt == tk.KV_F16 else 4352
    assert pool.bytes() > (1 << 32) + 20_000 * kvh * block_bytes
    rng = np.random.default_rng(41)
    hi = rng.choice(np.arange(n_pages - 20_000, n_pages), 6, replace=False)
    lo = rng.choice(np.arange(0, 1_000), 6, replace=False)
    pages = [int(x) for pair in zip(hi, lo) for x in pair]
    assert min(hi) * kvh * block_bytes >= 1 << 32
    n_fill, n_dec = 150, 1
    total = n_fill + n_dec
    k = rng.standard_normal((total, kvh * hd)).astype(np.float32)
    v = rng.standard_normal((total, kvh * hd)).astype(np.float32)
    q = rng.standard_normal((total, qh * hd)).astype(np.float32)
    say(f"beyond-4GiB fmt={fmt} pages {pages}")
    fc = O.FlatCache(O.F16 if fmt == tk.KV_F16 else O.I8, k, v)
    if fmt == tk.KV_I8:
        fc.with_scales(O.half_to_float(O.float_to_half(fc.ks)),
                       O.half_to_float(O.float_to_half(fc.vs)))
    for start, n, kind in ((0, n_fill, "prefill"), (n_fill, n_dec, "decode")):
        b = tk.Batch().plan(pool, [tk.Session(start, n, pages)], qh)
        dk = tk.DeviceArray.from_numpy(k[start:start + n])
        dv = tk.DeviceArray.from_numpy(v[start:start + n])
        dq = tk.DeviceArray.from_numpy(q[start:start + n])
        dout = tk.DeviceArray((n, qh * hd), np.float32).zero()
        b.append(pool, 0, dk, dv)
        getattr(b, kind)(pool, 0, dq, dout)
        tk.hip().sync()
        want = fc.attend(q[start:start + n], qh, kvh, hd, start)
        err = assert_attention_close(dout.numpy(), want, f"{kind} beyond 4 GiB")
        say(f"  {kind}: max abs err {err:.2e}")
        for a in (dk, dv, dq, dout):
            a.close()
        b.close()
    pool.close()


def test_prefill_i8_matches_oracle(gpu):
    case = PagedCase(14, 2, 64, tk.KV_I8, [40], 70, seed=12)
    case.fill()
    got, _ = case.step(kind="prefill")
    assert_attention_close(got, case.oracle_out(), "i8 prefill")
    case.close()


@pytest.mark.parametrize("fmt,sf,kvh,hd,fma", [
    (tk.KV_F16, tk.SCALE_F16, 4, 128, True),
    (tk.KV_I8, tk.SCALE_F16, 4, 128, True),
    (tk.KV_I8, tk.SCALE_F32, 2, 64, False),
    (tk.KV_F16, tk.SCALE_F16, 2, 64, False),
    # head sizes padded to the block width (the NeoX halves are the head's:
    # pairs (i, i + head_dim/2))
    (tk.KV_F16, tk.SCALE_F16, 2, 80, True),
    (tk.KV_I8, tk.SCALE_F16, 2, 96, False),
    (tk.KV_F16, tk.SCALE_F16, 1, 48, False),
    # 7 q heads x 6 lanes: Q lanes that end a row off a 4-lane boundary
    (tk.KV_I8, tk.SCALE_F16, 1, 96, True),
    # 256-dim blocks
    (tk.KV_F16, tk.SCALE_F16, 2, 256, True),
    (tk.KV_I8, tk.SCALE_F32, 1, 160, False),
])
def test_append_rope_bitexact(gpu, fmt, sf, kvh, hd, fma):
    """Fused bias + RoPE + append (tge_kv_append_rope): the pool contents and
    the rotated q equal the oracle's per-token sequence (fp32 bias adds,
    apply_rope of q and k, then the store; qwen2.cpp:2062-2093) bit for bit,
    in either rounding of apply_rope; q may be rotated in place; decode over
    the result matches the oracle within tolerance."""
    say(f"append_rope fmt={fmt} sf={sf} kvh={kvh} hd={hd} fma={fma}")
    qh = kvh * 7
    case = PagedCase(qh, kvh, hd, fmt, [37, 0, 100], [3, 5, 1], scale_format=sf, seed=31,
                     outlier_frac=0.01 if fmt == tk.KV_I8 else 0)
    case.fill()
    rng = np.random.default_rng(77)
    rows = sum(case.n_new)
    kv_dim = kvh * hd
    pos = np.concatenate([np.arange(c, c + n) for c, n in zip(case.contexts, case.n_new)])
    raw_q = rng.standard_normal((rows, qh * hd)).astype(np.float32)
    raw_k = rng.standard_normal((rows, kv_dim)).astype(np.float32)
    raw_v = rng.standard_normal((rows, kv_dim)).astype(np.float32)
    raw_k[:, :3] *= np.float32(6)  # rotation mixes large and small halves into a block
    qb = rng.standard_normal(qh * hd).astype(np.float32)
    kb = rng.standard_normal(kv_dim).astype(np.float32)
    vb = rng.standard_normal(kv_dim).astype(np.float32)
    cos_t, sin_t = tk.rope_tables(hd, 512)
    q_o, k_o, v_o = O.bias_rope_rows(raw_q, raw_k, raw_v, qb, kb, vb, qh, kvh, hd,
                                     cos_t[pos], sin_t[pos], fma)
    row = 0
    for s, (c, n) in enumerate(zip(case.contexts, case.n_new)):
        case.k[s][c:c + n] = k_o[row:row + n]
        case.v[s][c:c + n] = v_o[row:row + n]
        row += n
    b = tk.Batch().plan(case.pool, case.sessions(True), qh)
    d = {name: tk.DeviceArray.from_numpy(a) for name, a in
         (("q", raw_q), ("k", raw_k), ("v", raw_v), ("qb", qb), ("kb", kb), ("vb", vb),
          ("c", cos_t), ("s", sin_t))}
    q_out = tk.DeviceArray(raw_q.shape, np.float32).zero()
    args = tk.rope_args(d["k"], d["v"], d["c"], d["s"], 512, q=d["q"], q_out=q_out, q_bias=d["qb"],
                        k_bias=d["kb"], v_bias=d["vb"], fma=fma)
    b.append_rope(case.pool, 0, args)
    tk.hip().sync()
    assert np.array_equal(q_out.numpy().view(np.uint32), q_o.view(np.uint32)), "rotated q differs"
    b.close()
    check_contents(case)
    # in place: q_out is q
    b = tk.Batch().plan(case.pool, case.sessions(True), qh)
    args = tk.rope_args(d["k"], d["v"], d["c"], d["s"], 512, q=d["q"], q_out=d["q"],
                        q_bias=d["qb"], k_bias=d["kb"], v_bias=d["vb"], fma=fma)
    b.append_rope(case.pool, 0, args)
    out = tk.DeviceArray(raw_q.shape, np.float32).zero()
    b.decode(case.pool, 0, d["q"], out)
    tk.hip().sync()
    assert np.array_equal(d["q"].numpy().view(np.uint32), q_o.view(np.uint32)), "in-place q differs"
    case.q = q_o
    assert_attention_close(out.numpy(), case.oracle_out(), "decode after append_rope")
    b.close()
    check_contents(case)
    case.close()


def test_append_rope_checks(gpu):
    """Argument checks of the fused append: tables must cover every position
    of the plan; q needs q_out; no bias and no q are allowed (K/V only); a
    head size off the 16-dim grid is refused."""
    case = PagedCase(14, 2, 64, tk.KV_F16, [20], [2], seed=3)
    b = tk.Batch().plan(case.pool, case.sessions(True), 14)
    k = tk.DeviceArray.from_numpy(np.ones((2, 128), np.float32))
    c = tk.DeviceArray.from_numpy(np.ones((22, 32), np.float32))
    s = tk.DeviceArray.from_numpy(np.zeros((22, 32), np.float32))
    with pytest.raises(tk.TgeError) as e:
        b.append_rope(case.pool, 0, tk.rope_args(k, k, c, s, 21))  # position 21 not covered
    assert e.value.status == tk.ERR_INVALID
    with pytest.raises(tk.TgeError) as e:
        b.append_rope(case.pool, 0, tk.rope_args(k, k, c, s, 22, q=k))
    assert e.value.status == tk.ERR_INVALID
    b.append_rope(case.pool, 0, tk.rope_args(k, k, c, s, 22))
    tk.hip().sync()
    gk, gv, _, _ = b.gather(case.pool, 0, 0, 22)
    assert np.array_equal(gk[20:], O.float_to_half(np.ones((2, 128), np.float32)))
    b.close()
    case.close()
    # a head off the 16-dim grid (a pool takes multiples of 4): the NeoX
    # halves are not whole runs of 8, so the fused append refuses it
    case = PagedCase(14, 2, 72, tk.KV_F16, [20], [2], seed=3)
    b = tk.Batch().plan(case.pool, case.sessions(True), 14)
    k = tk.DeviceArray.from_numpy(np.ones((2, 144), np.float32))
    c = tk.DeviceArray.from_numpy(np.ones((22, 36), np.float32))
    s = tk.DeviceArray.from_numpy(np.zeros((22, 36), np.float32))
    with pytest.raises(tk.TgeError) as e:
        b.append_rope(case.pool, 0, tk.rope_args(k, k, c, s, 22))
    assert e.value.status == tk.ERR_INVALID
    b.close()
    case.close()


@pytest.mark.parametrize("fmt", [tk.KV_F16, tk.KV_I8])
def test_mixed_step_attention(gpu, fmt):
    """One step mixing decoding sessions (1-4 new rows, the decode kernel)
    and prefilling ones (long chunks, the block-prefill kernel) through
    tge_batch_attention, against the oracle; a step of one kind runs exactly
    the single-kind entry point (bit-identical)."""
    say(f"mixed step fmt={fmt}")
    case = PagedCase(28, 4, 128, fmt, [300, 0, 5000, 64, 1000], [4, 150, 1, 40, 9], seed=41,
                     outlier_frac=0.01 if fmt == tk.KV_I8 else 0)
    case.fill()
    b = tk.Batch().plan(case.pool, case.sessions(True), case.qh)
    kk = np.concatenate([k[c:] for k, c in zip(case.k, case.contexts)])
    vv = np.concatenate([v[c:] for v, c in zip(case.v, case.contexts)])
    dk, dv = tk.DeviceArray.from_numpy(kk), tk.DeviceArray.from_numpy(vv)
    dq = tk.DeviceArray.from_numpy(case.q)
    out = tk.DeviceArray(case.q.shape, np.float32).zero()
    b.append(case.pool, 0, dk, dv)
    b.attention(case.pool, 0, dq, out)
    tk.hip().sync()
    assert_attention_close(out.numpy(), case.oracle_out(), "mixed step")
    b.close()
    case.close()
    # decode-only step: tge_batch_attention == tge_decode_attention, bit for bit
    case = PagedCase(28, 4, 128, fmt, [300, 700], [4, 1], seed=42)
    case.fill()
    got, b = case.step()
    dq = tk.DeviceArray.from_numpy(case.q)
    out = tk.DeviceArray(case.q.shape, np.float32).zero()
    b.attention(case.pool, 0, dq, out)
    tk.hip().sync()
    assert np.array_equal(out.numpy(), got)
    b.close()
    case.close()


@pytest.mark.parametrize("fmt", [tk.KV_F16, tk.KV_I8])
def test_mixed_one_launch_split_merges_repeat(gpu, fmt):
    """A dense mixed step is one launch whose split decode contexts and split
    prefill tiles are merged in the launch by their last piece (arrival
    counters that each merge re-arms): long decode contexts and a prefill
    chunk over a long prefix, called four times on two layers; every call
    matches the oracle and repeats bit for bit."""
    say(f"mixed one launch fmt={fmt}")
    case = PagedCase(28, 4, 128, fmt, [20000, 9000, 2000, 300, 0], [4, 4, 300, 2, 200], seed=44,
                     layers=2, outlier_frac=0.01 if fmt == tk.KV_I8 else 0)
    for layer in range(2):
        case.fill(layer)
    b = tk.Batch().plan(case.pool, case.sessions(True), case.qh)
    kk = np.concatenate([k[c:] for k, c in zip(case.k, case.contexts)])
    vv = np.concatenate([v[c:] for v, c in zip(case.v, case.contexts)])
    dk, dv = tk.DeviceArray.from_numpy(kk), tk.DeviceArray.from_numpy(vv)
    dq = tk.DeviceArray.from_numpy(case.q)
    want = case.oracle_out()
    first = None
    for call in range(4):
        layer = call % 2
        if call < 2:
            b.append(case.pool, layer, dk, dv)
        out = tk.DeviceArray(case.q.shape, np.float32).zero()
        b.attention(case.pool, layer, dq, out)
        tk.hip().sync()
        got = out.numpy()
        out.close()
        assert_attention_close(got, want, f"mixed one launch call {call}")
        if first is None:
            first = got
        else:
            assert np.array_equal(bits(got), bits(first)), f"call {call} differs from call 0"
    say(f"  plan {b.info()}")
    for a in (dk, dv, dq):
        a.close()
    b.close()
    case.close()


@pytest.mark.parametrize("fmt,sparse,kind", [
    (tk.KV_F16, (4, 64, 4), "decode"),
    (tk.KV_F16, (4, 100, 37), "decode"),   # stride > 16: pages with nothing kept are skipped
    (tk.KV_I8, (20, 40, 17), "decode"),    # sink straddles a page; most middle pages kept
    (tk.KV_I8, (0, 48, 3), "decode"),
    (tk.KV_F16, (4, 64, 5), "prefill"),
    (tk.KV_F16, (2, 80, 24), "mixed"),     # one launch: the sparse mixed kernel
    (tk.KV_I8, (4, 64, 4), "mixed"),
    (tk.KV_F16, (4, 100, 37), "mixed"),
])
def test_static_sparse_attention(gpu, fmt, sparse, kind):
    """Static sparse attention (sink + strided middle + window, the kept set
    of build_sparse_index) on the decode, block-prefill and mixed paths,
    against the oracle's sparse head (pinned against the reference's
    attention_head_static_sparse kernels); spans on both sides of
    sink + window, multi-query rows whose windows differ by one."""
    say(f"sparse fmt={fmt} {sparse} {kind}")
    contexts = {"decode": [30, 700, 3000, 150], "prefill": [300, 0],
                "mixed": [2000, 500]}[kind]
    n_new = {"decode": [1, 4, 2, 3], "prefill": [120, 200], "mixed": [3, 160]}[kind]
    case = PagedCase(28, 4, 128, fmt, contexts, n_new, seed=51)
    case.fill()
    case.sparse = sparse
    b = tk.Batch().plan(case.pool, case.sessions(True), case.qh).set_sparse(*sparse)
    kk = np.concatenate([k[c:] for k, c in zip(case.k, case.contexts)])
    vv = np.concatenate([v[c:] for v, c in zip(case.v, case.contexts)])
    dk, dv = tk.DeviceArray.from_numpy(kk), tk.DeviceArray.from_numpy(vv)
    dq = tk.DeviceArray.from_numpy(case.q)
    out = tk.DeviceArray(case.q.shape, np.float32).zero()
    b.append(case.pool, 0, dk, dv)
    {"decode": b.decode, "prefill": b.prefill, "mixed": b.attention}[kind](case.pool, 0, dq, out)
    tk.hip().sync()
    assert_attention_close(out.numpy(), case.oracle_out(), f"sparse {sparse} {kind}")
    # turning it off gives dense attention again
    b.set_sparse(enabled=False)
    out2 = tk.DeviceArray(case.q.shape, np.float32).zero()
    {"decode": b.decode, "prefill": b.prefill, "mixed": b.attention}[kind](case.pool, 0, dq, out2)
    tk.hip().sync()
    case.sparse = None
    assert_attention_close(out2.numpy(), case.oracle_out(), "dense again")
    with pytest.raises(tk.TgeError) as e:
        b.set_sparse(4, 64, 1)
    assert e.value.status == tk.ERR_RUNTIME
    b.close()
    case.close()


def _random_case(i, kind=None):
    """Seeded random shape for test_random_cases: GQA group 1-8, 1-8 KV
    heads, head_dim 64/128, f16 or int8 (f16 or f32 scales), 1-6 sessions
    with empty, ragged and page-aligned contexts; decode, block prefill or
    a mixed step."""
    r = np.random.default_rng(1000 + i)
    kvh = int(r.choice([1, 2, 4, 8]))
    group = int(r.integers(1, 9))
    hd = int(r.choice([64, 128]))
    fmt = int(r.choice([tk.KV_F16, tk.KV_I8]))
    sf = int(r.choice([tk.SCALE_F16, tk.SCALE_F32])) if fmt == tk.KV_I8 else tk.SCALE_F16
    if kind is None:
        kind = "mixed" if i >= 16 else "decode" if i % 3 else "prefill"
    n_s = int(r.integers(1, 7))
    ctx_max = 6000 if kind == "decode" else 1500
    contexts = []
    for _ in range(n_s):
        pick = r.integers(0, 4)
        contexts.append(0 if pick == 0 else int(16 * r.integers(1, 40)) if pick == 1
                        else int(r.integers(1, ctx_max)))
    if kind == "decode":
        n_new = [int(r.integers(1, 64 // group + 1)) for _ in range(n_s)]
    elif kind == "mixed":  # each session decodes (rows fit a unit) or prefills
        n_new = [int(r.integers(1, 64 // group + 1)) if r.integers(0, 2) else
                 int(r.integers(64 // group + 1, 121)) for _ in range(n_s)]
    else:
        n_new = [int(r.integers(1, 81)) for _ in range(n_s)]
    return dict(qh=kvh * group, kvh=kvh, hd=hd, fmt=fmt, sf=sf, kind=kind, contexts=contexts,
                n_new=n_new)


@pytest.mark.parametrize("i", range(24))
def test_random_cases(gpu, i):
    """Twenty-four seeded random configurations (shapes, formats, ragged
    spans including empty contexts; decode, block prefill, and steps mixing
    both through tge_batch_attention) against the oracle."""
    c = _random_case(i)
    say(f"random case {i}: {c}")
    case = PagedCase(c["qh"], c["kvh"], c["hd"], c["fmt"], c["contexts"], c["n_new"],
                     scale_format=c["sf"], seed=2000 + i)
    case.fill()
    got, b = case.step(kind=c["kind"])
    err = assert_attention_close(got, case.oracle_out(), f"random case {i}")
    say(f"  max abs err {err:.2e}")
    b.close()
    case.close()


# Head sizes between the block widths: (q_heads, kv_heads, head_dim, format,
# scale format); dims past the head's own are stored as zeros and every
# path reads and writes only the head's own dims of q, k, v and out.
HEAD_SIZES = {
    "f16_d80": (14, 2, 80, tk.KV_F16, 0),
    "f16_d112_g4": (16, 4, 112, tk.KV_F16, 0),
    "f16_d48_g8": (8, 1, 48, tk.KV_F16, 0),
    "f16_d16": (4, 2, 16, tk.KV_F16, 0),
    # off the 16-dim grid (f16 heads are multiples of 4; 16-byte runs of q,
    # k, v and out rows past the head's end are never read or written)
    "f16_d72": (14, 2, 72, tk.KV_F16, 0),
    "f16_d100": (14, 2, 100, tk.KV_F16, 0),
    "f16_d120_g4": (16, 4, 120, tk.KV_F16, 0),
    "f16_d4": (4, 2, 4, tk.KV_F16, 0),
    "i8_d96_f16scales": (12, 2, 96, tk.KV_I8, tk.SCALE_F16),
    "i8_d32_f32scales": (8, 4, 32, tk.KV_I8, tk.SCALE_F32),
    # 256-dim blocks (one wave per SIMD in decode and prefill)
    "f16_d256_g8": (16, 2, 256, tk.KV_F16, 0),
    "f16_d192_g4": (8, 2, 192, tk.KV_F16, 0),
    "f16_d252": (8, 2, 252, tk.KV_F16, 0),
    "i8_d256_f16scales": (8, 2, 256, tk.KV_I8, tk.SCALE_F16),
    "i8_d160_f32scales_g8": (8, 1, 160, tk.KV_I8, tk.SCALE_F32),
}


@pytest.mark.parametrize("name", list(HEAD_SIZES))
@pytest.mark.parametrize("kind", ["decode", "step", "prefill", "mixed"])
def test_head_sizes_between_block_widths(gpu, name, kind):
    """Decode (the decode kernel and the one-launch step), block prefill and
    a mixed step at head sizes the pool pads to 64, 128 or 256 dims: attention
    against the oracle at the model's head_dim, the stored rows bit-exact
    (gather and raw layout, padding zero)."""
    qh, kvh, hd, fmt, sf = HEAD_SIZES[name]
    group = qh // kvh
    contexts = [700, 0, 33, 1600] if kind != "prefill" else [0, 160, 517]
    if kind in ("decode", "step"):
        n_new = [max(1, min(3, 64 // group))] * len(contexts)
    elif kind == "mixed":
        n_new = [2, 90, 1, 40]
    else:
        n_new = [70, 33, 129]
    say(f"head size case {name} {kind}: contexts {contexts} n_new {n_new}")
    case = PagedCase(qh, kvh, hd, fmt, contexts, n_new, scale_format=sf, seed=7100 + hd,
                     outlier_frac=0.01 if fmt == tk.KV_I8 else 0)
    case.fill()
    got, b = case.step(kind=kind)
    err = assert_attention_close(got, case.oracle_out(), f"head size {name} {kind}")
    say(f"  max abs err {err:.2e}")
    b.close()
    check_contents(case)
    case.close()


def _random_head_case(i):
    """Seeded random head size for test_random_head_sizes: f16 any multiple
    of 16 up to 256, int8 any multiple of 32; GQA group 1-8, 1-4 KV heads,
    1-4 sessions; decode, the one-launch step, block prefill or a mixed
    step, within the row limits of the head size's block width."""
    r = np.random.default_rng(5000 + i)
    fmt = int(r.choice([tk.KV_F16, tk.KV_I8]))
    hd = int(16 * r.integers(1, 17)) if fmt == tk.KV_F16 else int(32 * r.integers(1, 9))
    sf = int(r.choice([tk.SCALE_F16, tk.SCALE_F32])) if fmt == tk.KV_I8 else tk.SCALE_F16
    kvh = int(r.choice([1, 2, 4]))
    group = int(r.integers(1, 9))
    unit = 48 if hd > 128 else 64  # rows of a decode unit
    kind = ("decode", "step", "prefill", "mixed")[i % 4]
    n_s = int(r.integers(1, 5))
    contexts = [0 if r.integers(0, 4) == 0 else int(r.integers(1, 1800)) for _ in range(n_s)]
    if kind in ("decode", "step"):
        n_new = [int(r.integers(1, unit // group + 1)) for _ in range(n_s)]
    elif kind == "mixed":
        n_new = [int(r.integers(1, unit // group + 1)) if k % 2 == 0 else
                 int(r.integers(unit // group + 1, 100)) for k in range(n_s)]
    else:
        n_new = [int(r.integers(1, 90)) for _ in range(n_s)]
    return dict(qh=kvh * group, kvh=kvh, hd=hd, fmt=fmt, sf=sf, kind=kind, contexts=contexts,
                n_new=n_new)


@pytest.mark.parametrize("i", range(16))
def test_random_head_sizes(gpu, i):
    """Sixteen seeded random head sizes (16-256 dims, padded to 64-, 128-
    or 256-dim blocks) over random shapes and step kinds against the
    oracle, stored rows bit-exact."""
    c = _random_head_case(i)
    say(f"random head size case {i}: {c}")
    case = PagedCase(c["qh"], c["kvh"], c["hd"], c["fmt"], c["contexts"], c["n_new"],
                     scale_format=c["sf"], seed=6000 + i,
                     outlier_frac=0.01 if c["fmt"] == tk.KV_I8 else 0)
    case.fill()
    got, b = case.step(kind=c["kind"])
    err = assert_attention_close(got, case.oracle_out(), f"random head size case {i}")
    say(f"  max abs err {err:.2e}")
    b.close()
    check_contents(case)
    case.close()


@pytest.mark.parametrize("kind", ["decode", "prefill", "mixed"])
def test_head_size_96_int8_sparse(gpu, kind):
    """The static sparse subset at a padded head size (int8, 96 dims in
    128-dim blocks): decode, block prefill and mixed steps against the
    oracle's sparse head."""
    contexts, n_new = [3000, 150, 900], ([2, 2, 2] if kind == "decode" else
                                        [40, 2, 70] if kind == "mixed" else [60, 20, 33])
    case = PagedCase(12, 2, 96, tk.KV_I8, contexts, n_new, scale_format=tk.SCALE_F16, seed=7300,
                     outlier_frac=0.01)
    case.fill()
    case.sparse = (4, 300, 24)
    b = tk.Batch().plan(case.pool, case.sessions(True), case.qh).set_sparse(*case.sparse)
    kk = np.concatenate([k[c:] for k, c in zip(case.k, case.contexts)])
    vv = np.concatenate([v[c:] for v, c in zip(case.v, case.contexts)])
    dk, dv = tk.DeviceArray.from_numpy(kk), tk.DeviceArray.from_numpy(vv)
    dq = tk.DeviceArray.from_numpy(case.q)
    out = tk.DeviceArray(case.q.shape, np.float32).zero()
    b.append(case.pool, 0, dk, dv)
    {"decode": b.decode, "prefill": b.prefill, "mixed": b.attention}[kind](case.pool, 0, dq, out)
    tk.hip().sync()
    err = assert_attention_close(out.numpy(), case.oracle_out(), f"sparse head 96 {kind}")
    say(f"sparse head 96 {kind}: max abs err {err:.2e}")
    for a in (dk, dv, dq, out):
        a.close()
    b.close()
    case.close()


@pytest.mark.parametrize("i", range(12))
def test_random_sparse_cases(gpu, i):
    """Twelve seeded random static sparse subsets (sink 0-40, window 1-600,
    stride 2-70, so both the masking-only and the page-skipping decode paths
    run) over random shapes and kinds, against the oracle's sparse head."""
    c = _random_case(100 + i, ("decode", "decode", "prefill", "mixed")[i % 4])
    r = np.random.default_rng(3000 + i)
    sparse = (int(r.integers(0, 41)), int(r.integers(1, 601)),
              int(r.choice([int(r.integers(2, 17)), int(r.integers(17, 71))])))
    say(f"random sparse case {i}: {c} sparse {sparse}")
    case = PagedCase(c["qh"], c["kvh"], c["hd"], c["fmt"], c["contexts"], c["n_new"],
                     scale_format=c["sf"], seed=4000 + i)
    case.fill()
    case.sparse = sparse
    b = tk.Batch().plan(case.pool, case.sessions(True), case.qh).set_sparse(*sparse)
    kk = np.concatenate([k[cc:] for k, cc in zip(case.k, case.contexts)])
    vv = np.concatenate([v[cc:] for v, cc in zip(case.v, case.contexts)])
    dk, dv = tk.DeviceArray.from_numpy(kk), tk.DeviceArray.from_numpy(vv)
    dq = tk.DeviceArray.from_numpy(case.q)
    out = tk.DeviceArray(case.q.shape, np.float32).zero()
    b.append(case.pool, 0, dk, dv)
    {"decode": b.decode, "prefill": b.prefill, "mixed": b.attention}[c["kind"]](
        case.pool, 0, dq, out)
    tk.hip().sync()
    err = assert_attention_close(out.numpy(), case.oracle_out(), f"random sparse case {i}")
    say(f"  max abs err {err:.2e}")
    for a in (dk, dv, dq, out):
        a.close()
    b.close()
    case.close()


@pytest.mark.parametrize("i", range(10))
def test_random_append_bitexact(gpu, i):
    """Ten seeded random shapes (the random-case generator's heads, head_dim,
    formats, scale formats, empty and ragged contexts, 1-120 new rows per
    session crossing page boundaries): after the fill and one appended step,
    every session's pool contents (codes, f16 bits, scales) equal the
    oracle's store bit for bit, read both through the gather and by the
    layout formula."""
    c = _random_case(200 + i, "prefill")
    r = np.random.default_rng(5000 + i)
    c["contexts"] = [min(x, 1200) for x in c["contexts"]]
    c["n_new"] = [int(r.integers(1, 121)) for _ in c["n_new"]]
    say(f"random append case {i}: {c}")
    case = PagedCase(c["qh"], c["kvh"], c["hd"], c["fmt"], c["contexts"], c["n_new"],
                     scale_format=c["sf"], seed=6000 + i,
                     outlier_frac=0.01 if c["fmt"] == tk.KV_I8 else 0)
    case.fill()
    _, b = case.step(kind="prefill")
    b.close()
    check_contents(case)
    case.close()
