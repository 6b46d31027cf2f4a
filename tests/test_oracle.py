"""Pins the CPU oracle (oracle/) before it is trusted as the checker.

Each oracle function is checked against something that is not its own
formula: the reference engine's code built from /root/reference
(oracle/_ref), the reference tests' known-answer values, hardware IEEE
conversions with an exactly characterised difference set, closed forms and
float64 truth. CPU only.
"""
import ctypes as C
import json
import math
import os
import shutil
import subprocess
import tempfile

import numpy as np
import pytest

import oracle as O
from _util import bits, make_values

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
needs_ref = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built here")


def f2h(x):
    return O.orc().orc_float_to_half(C.c_float(x))


def _fp(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


# ---------------------------------------------------------------------------
# float <-> half
# ---------------------------------------------------------------------------
def test_half_round_trip_kats():
    # test_attention.cpp:107-115
    for v in [0.0, 1.0, -1.0, 0.5, 2.0, 1024.0, 65504.0]:
        back = O.orc().orc_half_to_float(f2h(v))
        assert abs(back - v) <= max(abs(v) * 0.001, 1e-6)
    assert f2h(math.inf) == 0x7C00


def test_float_to_half_bit_kats():
    f32 = lambda u: float(np.uint32(u).view(np.float32))
    assert f2h(1.0) == 0x3C00
    assert f2h(-2.0) == 0xC000
    assert f2h(65504.0) == 0x7BFF
    assert f2h(65519.0) == 0x7BFF
    assert f2h(65520.0) == 0x7C00          # guard-bit carry into the exponent
    assert f2h(-math.inf) == 0xFC00
    assert f2h(math.nan) == 0x7E00
    assert f2h(f32(0xFFC00001)) == 0xFE00  # any payload -> sign|0x7E00
    assert f2h(2.0 ** -24) == 0x0001
    assert f2h(1.5 * 2.0 ** -24) == 0x0002  # subnormal guard rounding
    assert f2h(2.0 ** -25) == 0x0000        # below 2^-24 flushes
    assert f2h(-(2.0 ** -25) * 1.9) == 0x8000
    assert f2h(2.0 ** -14) == 0x0400
    # an exact tie with an even truncated result rounds up (RNE would not)
    assert f2h(1.0 + 2.0 ** -11) == 0x3C01
    assert np.float16(1.0 + 2.0 ** -11).view(np.uint16) == 0x3C00
    assert f2h(1.0 + 3 * 2.0 ** -11) == 0x3C02


def test_half_to_float_exhaustive():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = O.half_to_float(h)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(bits(got)[~nan], bits(want)[~nan])
    assert np.all(np.isnan(got[nan]))
    assert np.array_equal(np.signbit(got[nan]), np.signbit(want[nan]))
    if O.ref_available():
        r = np.array([O.ref().ref_half_to_float(int(x)) for x in h[::97]], np.float32)
        assert np.array_equal(bits(r)[~np.isnan(r)], bits(got[::97])[~np.isnan(r)])


@pytest.fixture(scope="module")
def sweep_tool():
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    d = tempfile.mkdtemp(prefix="tge_f16_")
    exe = os.path.join(d, "f16_sweep")
    subprocess.run([gcc, "-O2", "-mf16c", "-fopenmp", "-o", exe,
                    os.path.join(HERE, "native", "f16_sweep.c"), "-ldl"], check=True)
    yield exe
    shutil.rmtree(d, ignore_errors=True)


def test_float_to_half_exhaustive(sweep_tool):
    """All 2^32 inputs: the oracle equals the reference build bit for bit and
    differs from hardware RNE exactly on the predicted set, whose sizes are
    closed forms (ties with an even truncation: 2*(30*512 + 511) = 31742;
    flushed (2^-25, 2^-24): 2*(2^23-1); NaN payloads: 2*(2^23-1))."""
    args = [sweep_tool, O.ORACLE_PATH, "orc_float_to_half"]
    if O.ref_available():
        args += [O.REF_PATH, "ref_float_to_half"]
    res = json.loads(subprocess.run(args, check=True, capture_output=True, text=True).stdout)
    assert res["violations"] == 0, res
    assert res["ties_up"] == 31742
    assert res["tiny_flush"] == 2 * (2 ** 23 - 1)
    assert res["nan"] == 2 * (2 ** 23 - 1)
    if O.ref_available():
        assert res["vs_other"] == 0, res


# ---------------------------------------------------------------------------
# int8 block quantizer (qwen2.cpp:88-104)
# ---------------------------------------------------------------------------
def quant(block):
    x = np.ascontiguousarray(block, np.float32)
    codes = np.empty(32, np.int8)
    s = O.orc().orc_quantize_kv_block(_fp(x), _fp(codes))
    return codes, np.float32(s)


def test_quantize_exact_multiples():
    ks = np.array([127, -127, 0, 1, -1, 64, -63, 100] * 4, np.int32)
    for step in (0.125, 2.0, 2.0 ** -10):
        codes, s = quant(ks.astype(np.float32) * np.float32(step))
        assert s == np.float32(step)
        assert np.array_equal(codes.astype(np.int32), ks)


def test_quantize_all_zero_block_takes_sign_of_last():
    z = np.zeros(32, np.float32)
    codes, s = quant(z)
    assert np.all(codes == 0) and s == 0 and not np.signbit(s)
    z[31] = -0.0
    codes, s = quant(z)
    assert np.all(codes == 0) and s == 0 and np.signbit(s)
    z[:] = -0.0
    z[31] = 0.0
    _, s = quant(z)
    assert not np.signbit(s)


def test_quantize_half_rounding_is_add_then_truncate():
    # scale 1 (max 127): codes are trunc(x +- 0.5) in fp32, so the float just
    # below 0.5 becomes 1 (0.49999997 + 0.5 rounds to 1.0f), unlike
    # rintf/roundf which give 0.
    below_half = np.float32(np.nextafter(np.float32(0.5), np.float32(0)))
    x = np.zeros(32, np.float32)
    x[0] = 127
    x[1], x[2] = below_half, -below_half
    x[3], x[4], x[5], x[6] = 0.5, 1.5, 2.5, -2.5
    x[7] = np.nextafter(np.float32(0.25), np.float32(0))
    codes, s = quant(x)
    assert s == 1.0
    assert list(codes[:8]) == [127, 1, -1, 1, 2, 3, -3, 0]
    assert round(float(below_half)) == 0


def test_quantize_multiply_then_add_is_not_fused():
    # Values whose exact product x*inv lies just below 0.5 - 2^-25: the
    # reference rounds the product (to 0.5 - 2^-25), then the add ties to
    # 1.0 (code +-1); one fused multiply-add rounds once to 1 - 2^-24 (code
    # 0). A contracted oracle fails every block.
    from _quant_cases import contraction_blocks
    blocks, want = contraction_blocks(24, seed=3)
    for b, w in zip(blocks, want):
        codes, _ = quant(b)
        assert np.array_equal(codes, w), (b[:3], codes[:9], w[:9])
    # the row quantizer (the store path) agrees block for block
    rows = blocks.reshape(6, 128)
    codes, _ = O.quantize_rows(rows)
    assert np.array_equal(codes.reshape(-1, 32), want)


def test_quantize_codes_use_the_fp32_scale():
    # The f16-scale format stores float_to_half(scale) but its codes come
    # from the fp32 scale (quantize_kv_block / store_kv_q8, qwen2.cpp:88-120). Each value sits a margin above a
    # half-integer multiple of the fp32 scale and below it for the (larger)
    # f16-rounded scale, so codes derived from the stored f16 scale would be
    # one smaller in magnitude on every non-maximum slot.
    from _quant_cases import f16_scale_blocks
    blocks, want, s16 = f16_scale_blocks(24, seed=4)
    for b, w, h in zip(blocks, want, s16):
        codes, s = quant(b)
        assert np.array_equal(codes, w), (codes[:6], w[:6])
        assert O.float_to_half(np.array([s], np.float32))[0] == h
        inv16 = np.float32(1) / O.half_to_float(np.array([h], np.uint16))[0]
        alt = np.trunc(b[1:] * inv16 + np.where(b[1:] >= 0, 0.5, -0.5).astype(np.float32))
        assert np.all(np.abs(alt) == np.abs(w[1:].astype(np.float32)) - 1)


def test_quantize_properties_random():
    rng = np.random.default_rng(7)
    for trial in range(400):
        kind = trial % 4
        x = rng.standard_normal(32).astype(np.float32)
        if kind == 1:
            x[rng.integers(0, 32)] *= 8
        elif kind == 2:
            x *= np.float32(1e-30)
        elif kind == 3:
            x *= np.float32(1e30)
        codes, s = quant(x)
        m = np.max(np.abs(x))
        assert s == np.float32(m) / np.float32(127)
        c = codes.astype(np.float64)
        assert np.all(np.abs(c) <= 127)
        assert np.abs(c[np.argmax(np.abs(x))]) == 127
        # each code is the nearest integer to x/scale (within fp32 slack)
        err = np.abs(c * float(s) - x.astype(np.float64))
        assert np.all(err <= 0.5 * float(s) * (1 + 1e-5) + 1e-45)
        assert np.all((np.sign(c) == np.sign(x)) | (c == 0))


# ---------------------------------------------------------------------------
# attention oracle against the reference build
# ---------------------------------------------------------------------------
def flat_inputs(fmt, span, head_dim, seed=2):
    keys = make_values(span * head_dim, seed)
    vals = make_values(span * head_dim, seed + 1)
    if fmt == O.F16:
        return O.float_to_half(keys), O.float_to_half(vals), None, None
    if fmt == O.I8:
        kc, ks = O.quantize_rows(keys.reshape(span, head_dim))
        vc, vs = O.quantize_rows(vals.reshape(span, head_dim))
        return kc.reshape(-1), vc.reshape(-1), ks.reshape(-1), vs.reshape(-1)
    return keys, vals, None, None


@needs_ref
@pytest.mark.parametrize("fmt", [O.F32, O.F16, O.I8])
def test_head_matches_reference_scalar_bitexact(fmt):
    for span in (1, 7, 64, 257):
        for hd in (64, 128):
            q = make_values(hd, 1)
            k, v, ks, vs = flat_inputs(fmt, span, hd)
            scale = np.float32(1.0) / np.sqrt(np.float32(hd))
            so, oo = np.empty(span, np.float32), np.empty(hd, np.float32)
            sr, orr = np.empty(span, np.float32), np.empty(hd, np.float32)
            assert O.orc().orc_attention_head(fmt, _fp(q), _fp(k), _fp(v), _fp(ks), _fp(vs), hd,
                                              span, hd, C.c_float(scale), _fp(so), _fp(oo)) == 0
            assert O.ref().ref_attention_head(0, fmt, _fp(q), _fp(k), _fp(v), _fp(ks), _fp(vs), hd,
                                              span, hd, C.c_float(scale), _fp(sr), _fp(orr)) == 0
            assert np.array_equal(bits(oo), bits(orr)), (fmt, span, hd)
            assert np.array_equal(bits(so), bits(sr))
            # and the shipped AVX2 kernel is within the reference's own 1e-4
            sa, oa = np.empty(span, np.float32), np.empty(hd, np.float32)
            O.ref().ref_attention_head(1, fmt, _fp(q), _fp(k), _fp(v), _fp(ks), _fp(vs), hd, span,
                                       hd, C.c_float(scale), _fp(sa), _fp(oa))
            assert np.max(np.abs(oa - oo)) <= 1e-4


@needs_ref
@pytest.mark.parametrize("fmt", [O.F32, O.F16, O.I8])
def test_group_matches_reference_scalar_bitexact(fmt):
    for count in (1, 9, 130):
        for g in (1, 7):
            hd = 64
            qs = make_values(g * hd, 11)
            k, v, ks, vs = flat_inputs(fmt, count, hd, seed=5)
            scale = C.c_float(0.125)
            outs = []
            for which in ("orc", "ref"):
                mx, sm = np.empty(g, np.float32), np.empty(g, np.float32)
                ac = np.empty(g * hd, np.float32)
                if which == "orc":
                    O.orc().orc_attention_group(fmt, _fp(qs), _fp(k), _fp(v), _fp(ks), _fp(vs), hd,
                                                count, hd, g, scale, _fp(mx), _fp(sm), _fp(ac))
                else:
                    O.ref().ref_attention_group(0, fmt, _fp(qs), _fp(k), _fp(v), _fp(ks), _fp(vs),
                                                hd, count, hd, g, scale, _fp(mx), _fp(sm), _fp(ac))
                outs.append((mx, sm, ac))
            for a, b in zip(*outs):
                assert np.array_equal(bits(a), bits(b)), (fmt, count, g)


def test_head_rejects_bad_arguments():
    # attention_scalar.cpp:11-44: span 0, stride < head_dim, ragged q8
    q = make_values(64, 1)
    k, v, ks, vs = flat_inputs(O.I8, 4, 64)
    sc, out = np.empty(4, np.float32), np.empty(64, np.float32)
    f = O.orc().orc_attention_head
    assert f(O.I8, _fp(q), _fp(k), _fp(v), _fp(ks), _fp(vs), 64, 0, 64, C.c_float(1), _fp(sc), _fp(out)) == -1
    assert f(O.I8, _fp(q), _fp(k), _fp(v), _fp(ks), _fp(vs), 32, 4, 64, C.c_float(1), _fp(sc), _fp(out)) == -1
    assert f(O.I8, _fp(q), _fp(k), _fp(v), _fp(ks), _fp(vs), 48, 1, 48, C.c_float(1), _fp(sc), _fp(out)) == -1
    assert f(O.I8, _fp(q), _fp(k), _fp(v), None, _fp(vs), 64, 4, 64, C.c_float(1), _fp(sc), _fp(out)) == -1


# ---------------------------------------------------------------------------
# closed forms
# ---------------------------------------------------------------------------
def test_span_one_returns_first_value_row():
    for fmt in (O.F32, O.F16, O.I8):
        k, v, ks, vs = flat_inputs(fmt, 1, 64)
        q = make_values(64, 3) * 50
        out = O.attention_head(fmt, q, k, v, ks, vs, 64, 1, 64, 0.125)
        if fmt == O.F16:
            want = O.half_to_float(v)
        elif fmt == O.I8:
            want = v.astype(np.float32) * np.repeat(vs, 32)
        else:
            want = v
        assert np.array_equal(out, want.astype(np.float32))


def test_equal_keys_give_mean_of_values():
    span, hd = 37, 64
    key = make_values(hd, 9)
    keys = np.tile(key, span)
    vals = make_values(span * hd, 10)
    out = O.attention_head(O.F32, make_values(hd, 4), keys, vals, None, None, hd, span, hd, 0.125)
    want = vals.reshape(span, hd).astype(np.float64).mean(axis=0)
    assert np.max(np.abs(out - want)) < 1e-6


def test_dominant_key_selects_its_value():
    span, hd = 50, 64
    q = np.ones(hd, np.float32)
    keys = np.zeros((span, hd), np.float32)
    keys[23] = 10.0  # score 10*64*scale = 80 above the rest
    vals = make_values(span * hd, 12).reshape(span, hd)
    out = O.attention_head(O.F32, q, keys.reshape(-1), vals.reshape(-1), None, None, hd, span,
                           hd, 0.125)
    assert np.max(np.abs(out - vals[23])) < 1e-6


def test_fp32_oracle_close_to_float64_truth():
    rng = np.random.default_rng(3)
    for fmt in (O.F32, O.F16, O.I8):
        span, hd = 700, 128
        kf = rng.standard_normal((span, hd)).astype(np.float32)
        vf = rng.standard_normal((span, hd)).astype(np.float32)
        cache = O.FlatCache(fmt, kf, vf)
        q = rng.standard_normal(hd).astype(np.float32)
        o32 = cache.head(q, 0, hd, span)
        o64 = cache.head(q, 0, hd, span, f64=True)
        assert np.max(np.abs(o32 - o64)) < 2e-6


def test_gqa_split_invariance():
    """qwen2.cpp attention_gqa (split-K + merge_gqa_chunks) equals the per-head
    oracle for every chunk count the thread rule produces."""
    rng = np.random.default_rng(4)
    heads, kvh, hd = 14, 2, 64
    for span in (256, 1024, 1500):
        kf = rng.standard_normal((span, kvh * hd)).astype(np.float32)
        vf = rng.standard_normal((span, kvh * hd)).astype(np.float32)
        cache = O.FlatCache(O.F16, kf, vf)
        q = rng.standard_normal(heads * hd).astype(np.float32)
        want = np.concatenate([cache.head(q[h * hd:(h + 1) * hd], h // 7, hd, span)
                               for h in range(heads)])
        for threads in (1, 2, 6, 16):
            out = np.empty(heads * hd, np.float32)
            O.orc().orc_attention_gqa(O.F16, _fp(q), _fp(cache.k), _fp(cache.v), None, None, heads,
                                      kvh, hd, span, threads, _fp(out))
            assert np.max(np.abs(out - want)) < 1e-5, (span, threads)


def test_gqa_chunk_rule():
    cs = C.c_int()
    assert O.orc().orc_gqa_chunks(300, 2, 6, C.byref(cs)) == 6 and cs.value == 50
    assert O.orc().orc_gqa_chunks(2048, 2, 1, C.byref(cs)) == 4 and cs.value == 512
    assert O.orc().orc_gqa_chunks(100000, 1, 64, C.byref(cs)) == 16


def test_merge_skips_empty_chunks_and_zeroes_when_none():
    hd = 4
    mx = np.array([1.0, 5.0, 2.0], np.float32)
    sm = np.array([2.0, 0.0, 3.0], np.float32)
    ac = np.arange(12, dtype=np.float32)
    out = np.empty(hd, np.float32)
    O.orc().orc_merge_chunks(_fp(mx), _fp(sm), _fp(ac), 0, 3, 1, 0, hd, _fp(out))
    a, b = math.exp(1 - 2), 1.0
    want = (ac[0:4] * a + ac[8:12] * b) / (2 * a + 3 * b)
    assert np.max(np.abs(out - want)) < 1e-6
    sm[:] = 0
    O.orc().orc_merge_chunks(_fp(mx), _fp(sm), _fp(ac), 0, 3, 1, 0, hd, _fp(out))
    assert np.all(out == 0)


def test_block_prefill_matches_per_head_oracle():
    rng = np.random.default_rng(5)
    heads, kvh, hd, start, tokens = 4, 2, 64, 40, 24
    kv_dim, qd = kvh * hd, heads * hd
    kf = rng.standard_normal((start + tokens, kv_dim)).astype(np.float32)
    vf = rng.standard_normal((start + tokens, kv_dim)).astype(np.float32)
    cache = O.FlatCache(O.F16, kf, vf)
    q = rng.standard_normal((tokens, qd)).astype(np.float32)
    out = np.zeros((tokens, qd), np.float32)
    scores = np.empty(tokens * (start + tokens), np.float32)
    for h in range(heads):
        assert O.orc().orc_attention_block_head(O.F16, _fp(q), _fp(cache.k), _fp(cache.v), tokens,
                                                start, hd, kv_dim, (h // 2) * hd, qd, h,
                                                C.c_float(0.125), _fp(scores), _fp(out)) == 0
    want = cache.attend(q, heads, kvh, hd, start)
    assert np.max(np.abs(out - want)) < 1e-5
    if O.ref_available():
        ref_out = np.zeros((tokens, qd), np.float32)
        ctx = start + tokens
        sc = np.empty(tokens * heads * ctx, np.float32)
        for h in range(heads):
            O.ref().ref_attention_block_head(O.F16, _fp(q), _fp(cache.k), _fp(cache.v), tokens,
                                             start, hd, kv_dim, (h // 2) * hd, qd, heads * ctx, ctx,
                                             C.c_float(0.125), h,
                                             _fp(sc[h * ctx:]), _fp(ref_out))
        assert np.max(np.abs(ref_out - out)) < 1e-4


# ---------------------------------------------------------------------------
# flat layout and gather KATs
# ---------------------------------------------------------------------------
def test_kv_layer_offset_kats():
    # test_gguf.cpp:842-846
    f = O.orc().orc_kv_layer_offset
    assert f(0, 0, 2, 16, 8) == 0
    assert f(1, 0, 2, 16, 8) == 256
    assert f(1, 1, 2, 16, 8) == 384


@needs_ref
def test_reference_gather_order_kat():
    # test_block_table.cpp:121-136: table {2, 0} over {1,2},{3,4},{5,6}
    pool = np.array([1, 2, 3, 4, 5, 6], np.float32)
    out = np.empty(4, np.float32)
    table = (C.c_int * 2)(2, 0)
    assert O.ref().ref_gather_blocks(_fp(pool), 3, 2, table, 2, 2, _fp(out)) == 4
    assert list(out) == [5, 6, 1, 2]
    bad = (C.c_int * 1)(9)
    assert O.ref().ref_gather_blocks(_fp(pool), 3, 2, bad, 1, 2, _fp(out)) == -1


def test_split_absmax_fold_matches_sequential():
    """The append kernel folds each 32-value block's absmax as four runs of
    eight joined in order (FoldRun in csrc/tge_common.h); the reference folds
    sequentially from +0 (qwen2.cpp:88-93). Two million blocks mixing NaNs of
    both signs, zeros of both signs, infinities, subnormals, ties and raw bit
    patterns must give the same maximum bit for bit (a join in the wrong
    order fails on ~40 % of them)."""
    hipcc = "/opt/rocm/bin/hipcc"
    if not os.path.exists(hipcc):
        pytest.skip("hipcc not available")
    d = tempfile.mkdtemp(prefix="tge_fold_")
    exe = os.path.join(d, "fold_check")
    try:
        subprocess.run([hipcc, "-O2", "-std=c++20", "-ffp-contract=off",
                        "-I", os.path.join(ROOT, "aegean-tge_amd", "csrc"), "-I", os.path.join(ROOT, "include"),
                        "-o", exe, os.path.join(HERE, "native", "fold_check.cpp")],
                       check=True, capture_output=True)
        r = subprocess.run([exe, "2000000", "7"], capture_output=True, text=True)
        out = json.loads(r.stdout)
        assert r.returncode == 0 and out["mismatches"] == 0, (out, r.stderr)
        assert out["blocks_with_nan"] > 100000 and out["zero_max_blocks"] > 100000, out
    finally:
        shutil.rmtree(d, ignore_errors=True)


def _rope_inputs(rows, heads, hd, seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((rows, heads * hd)) * rng.choice([1e-3, 1, 30, 3e4], (rows, 1))
         ).astype(np.float32)
    x[0, :4] = [0.0, -0.0, 1e-40, -3e-41]  # signed zeros and subnormals
    c, s = O.rope_tables(hd, 4096)
    pos = rng.integers(0, 4096, rows)
    return x, c[pos], s[pos]


@pytest.mark.parametrize("hd", [64, 128])
@pytest.mark.parametrize("fma", [True, False])
def test_rope_matches_reference_bitexact(hd, fma):
    """orc_rope_neox against the reference's own apply_rope_avx2 (FMA
    rounding) and apply_rope_scalar, built from norm_rope_*.cpp."""
    if not O.ref_available():
        pytest.skip("oracle/_ref not built (reference tree absent)")
    x, c, s = _rope_inputs(300, 7, hd, 21 + hd)
    a = O.rope_neox(x, 7, hd, c, s, fma)
    b = O.ref_rope(x, 7, hd, c, s, avx2=fma)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    # the two roundings really differ, so a swapped recipe cannot pass
    other = O.rope_neox(x, 7, hd, c, s, not fma)
    assert (other.view(np.uint32) != a.view(np.uint32)).mean() > 0.05


def test_rope_closed_forms():
    """Position 0 (cos 1, sin 0) is the identity (a zero may change sign:
    -0 - (h*0) is +0 when h*0 is -0); a rotation keeps each pair's norm;
    rotating by +a then -a returns the input (float64 model bounds)."""
    x, _, _ = _rope_inputs(64, 4, 128, 5)
    c, s = O.rope_tables(128, 1)
    c0, s0 = np.repeat(c, 64, 0), np.repeat(s, 64, 0)
    for fma in (True, False):
        y = O.rope_neox(x, 4, 128, c0, s0, fma)
        assert np.array_equal(y, x)
        nz = x != 0
        assert np.array_equal(y.view(np.uint32)[nz], x.view(np.uint32)[nz])
    rng = np.random.default_rng(9)
    ang = rng.uniform(-3, 3, (64, 64)).astype(np.float32)
    ca, sa = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    y = O.rope_neox(x, 4, 128, ca, sa, True).astype(np.float64).reshape(64, 4, 2, 64)
    x64 = x.astype(np.float64).reshape(64, 4, 2, 64)
    n0 = np.hypot(x64[:, :, 0], x64[:, :, 1])
    n1 = np.hypot(y[:, :, 0], y[:, :, 1])
    assert np.all(np.abs(n1 - n0) <= 1e-5 * n0 + 1e-30)
    back = O.rope_neox(y.reshape(64, -1).astype(np.float32), 4, 128, ca, -sa, True)
    assert np.allclose(back, x, rtol=1e-5, atol=1e-6 * np.abs(x).max())


def test_bias_rope_row_order():
    """orc_bias_rope_row is: fp32 bias adds, then RoPE of q and k, v only
    biased — composed here from numpy float32 adds and orc_rope_neox."""
    rng = np.random.default_rng(13)
    rows, qh, kvh, hd = 20, 14, 2, 64
    q = rng.standard_normal((rows, qh * hd)).astype(np.float32)
    k = rng.standard_normal((rows, kvh * hd)).astype(np.float32)
    v = rng.standard_normal((rows, kvh * hd)).astype(np.float32)
    qb, kb, vb = (rng.standard_normal(n).astype(np.float32) for n in (qh * hd, kvh * hd, kvh * hd))
    c, s = O.rope_tables(hd, 100)
    pos = rng.integers(0, 100, rows)
    q2, k2, v2 = O.bias_rope_rows(q, k, v, qb, kb, vb, qh, kvh, hd, c[pos], s[pos])
    assert np.array_equal(q2, O.rope_neox(q + qb, qh, hd, c[pos], s[pos], True))
    assert np.array_equal(k2, O.rope_neox(k + kb, kvh, hd, c[pos], s[pos], True))
    assert np.array_equal(v2, v + vb)


def test_rope_tables_against_float64_and_product(tk):
    """Tables within 2 ulp of float64 truth of the same float angles, the
    YaRN factor and attn_factor terms applied, and the product's host builder
    (tge_rope_tables) bit-identical to the oracle (same C library calls)."""
    hd, n = 128, 2048
    c, s = O.rope_tables(hd, n)
    i = np.arange(hd // 2, dtype=np.float32)
    freq = np.array([np.float32(10000.0) ** np.float32(-2.0 * j / hd) for j in i], np.float32)
    ang = np.arange(n, dtype=np.float32)[:, None] * freq[None, :]
    ulp = np.spacing(np.abs(np.cos(ang.astype(np.float64))).astype(np.float32))
    assert np.all(np.abs(c - np.cos(ang.astype(np.float64))) <= 2 * ulp + 1e-12)
    ulp = np.spacing(np.abs(np.sin(ang.astype(np.float64))).astype(np.float32))
    assert np.all(np.abs(s - np.sin(ang.astype(np.float64))) <= 2 * ulp + 1e-12)
    pc, ps = tk.rope_tables(hd, n)
    assert np.array_equal(pc.view(np.uint32), c.view(np.uint32))
    assert np.array_equal(ps.view(np.uint32), s.view(np.uint32))
    f = np.linspace(1, 8, hd // 2).astype(np.float32)
    c2, s2 = O.rope_tables(hd, 64, 1e6, 1.19024, f)
    p2, q2 = tk.rope_tables(hd, 64, 1e6, 1.19024, f)
    assert np.array_equal(p2, c2) and np.array_equal(q2, s2)
    assert np.isclose(c2[0, 0], 1.19024) and s2[0, 5] == 0


def test_sparse_index_closed_forms():
    """build_sparse_index (qwen2.cpp:192-220): dense when the span fits
    sink + window; else sink, every stride-th from sink below span - window,
    then the window; stride < 2 acts as 2."""
    assert list(O.sparse_index(10, 4, 8, 4)) == list(range(10))
    k = O.sparse_index(100, 4, 8, 5)
    assert list(k) == [0, 1, 2, 3] + list(range(4, 92, 5)) + list(range(92, 100))
    assert list(O.sparse_index(50, 0, 10, 1)) == list(range(0, 40, 2)) + list(range(40, 50))
    k = O.sparse_index(1000, 4, 512, 4)
    assert k.size == 4 + (488 - 4 + 3) // 4 + 512 and np.all(np.diff(k) > 0)


@pytest.mark.parametrize("fmt", [O.F32, O.F16])
def test_sparse_head_against_reference_and_dense(fmt):
    """orc_attention_head_sparse against the reference's own static sparse
    kernels (attention_head_static_sparse_avx2 / _fp16_avx2, whose exp is a
    vectorised approximation: 1e-5), equal to the dense oracle when the span
    fits sink + window, and equal to the dense oracle over a cache holding
    only the kept rows (same arithmetic on the same rows)."""
    rng = np.random.default_rng(17)
    hd, span = 64, 700
    k = rng.standard_normal((span, hd)).astype(np.float32)
    v = rng.standard_normal((span, hd)).astype(np.float32)
    q = (rng.standard_normal(hd) * 2).astype(np.float32)
    fc = O.FlatCache(fmt, k, v)
    scale = float(np.float32(1.0 / np.sqrt(np.float32(hd))))
    for sink, window, stride in ((4, 512, 4), (0, 64, 3), (7, 100, 33), (4, 512, 1)):
        got = O.attention_head_sparse(fmt, q, fc.k, fc.v, None, None, hd, span, hd, scale, sink,
                                      window, stride)
        if O.ref_available():
            want = O.ref_attention_head_sparse(fmt, q, fc.k, fc.v, hd, span, hd, scale, sink,
                                               window, stride)
            assert np.allclose(got, want, rtol=1e-5, atol=1e-5)
        kept = O.sparse_index(span, sink, window, stride)
        sub = O.attention_head(fmt, q, fc.k[kept], fc.v[kept], None, None, hd, kept.size, hd, scale)
        assert np.array_equal(got, sub)
    dense = O.attention_head(fmt, q, fc.k, fc.v, None, None, hd, 300, hd, scale)
    assert np.array_equal(O.attention_head_sparse(fmt, q, fc.k, fc.v, None, None, hd, 300, hd,
                                                  scale, 4, 296, 4), dense)
