"""tge_decode_attention_static (the entry point that allocates nothing)
against tge_batch_plan + tge_decode_attention, through the C ABI, on the GPU.

Two calls in a row, the second on a smaller step, must each equal the
allocating entry point bit for bit (same plan, same kernels), and match the
oracle within the attention tolerance. A step whose plan exceeds the static
array is refused with TGE_ERR_CAPACITY before anything runs, and a later
call still works. A call on a stream that is capturing a graph is refused
with TGE_ERR_INVALID (its plan is uploaded from host memory at each call,
which a captured graph would replay stale), with nothing captured.
"""
import ctypes as C
import sys

import numpy as np
import pytest

import tge_kv as tk
from _paged import PagedCase
from _util import assert_attention_close, bits

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def run_both(case):
    """(static output, allocating output) of the case's decode step."""
    got_alloc, b = case.step()  # appends the step's rows, then decodes
    dq = tk.DeviceArray.from_numpy(case.q)
    out = tk.DeviceArray(case.q.shape, np.float32)
    tk.hip().memset(out.ptr, 0xFF, out.nbytes)  # NaN bits: every row must be written
    tk.decode_attention_static(case.pool, case.sessions(True), case.qh, 0, dq, out)
    tk.hip().sync()
    got_static = out.numpy()
    info = b.info()
    for a in (dq, out):
        a.close()
    b.close()
    return got_static, got_alloc, info


def test_static_decode_equals_allocating_decode(gpu):
    # first call: c5-shaped (int8, f16 scales, 4-query verify) with split-K
    say("static decode: first call (c5 shape, 6 sessions up to 9000 positions)")
    big = PagedCase(28, 4, 128, tk.KV_I8, [9000, 40, 3000, 1, 1500, 700], 4, seed=71,
                    outlier_frac=0.01)
    big.fill()
    s1, a1, info1 = run_both(big)
    assert info1[2] > 1, f"expected split-K partials in the first call: {info1}"
    assert np.array_equal(bits(s1), bits(a1)), "static and allocating decode differ (call 1)"
    assert_attention_close(s1, big.oracle_out(), "static decode call 1")
    # second call, smaller: the array keeps the first call's contents
    say("static decode: second, smaller call (c1 shape)")
    small = PagedCase(14, 2, 64, tk.KV_F16, [300, 17], 1, seed=72)
    small.fill()
    s2, a2, _ = run_both(small)
    assert np.array_equal(bits(s2), bits(a2)), "static and allocating decode differ (call 2)"
    assert_attention_close(s2, small.oracle_out(), "static decode call 2")
    # third call: a head size the pool pads (80 dims in 128-dim blocks)
    say("static decode: third call (head_dim 80)")
    pad = PagedCase(14, 2, 80, tk.KV_F16, [2500, 33], 2, seed=73)
    pad.fill()
    s3, a3, _ = run_both(pad)
    assert np.array_equal(bits(s3), bits(a3)), "static and allocating decode differ (call 3)"
    assert_attention_close(s3, pad.oracle_out(), "static decode call 3")
    # fourth call: 256-dim blocks (int8, split contexts)
    say("static decode: fourth call (head_dim 256, int8)")
    wide = PagedCase(16, 2, 256, tk.KV_I8, [3000, 20], 2, seed=74, outlier_frac=0.01)
    wide.fill()
    s4, a4, _ = run_both(wide)
    assert np.array_equal(bits(s4), bits(a4)), "static and allocating decode differ (call 4)"
    assert_attention_close(s4, wide.oracle_out(), "static decode call 4")
    wide.close()
    pad.close()
    small.close()
    big.close()


def test_static_decode_rejects_oversized_plans(gpu):
    say("static decode: oversized plan")
    pool = tk.KvPool(1, 4, 2, 64, tk.KV_F16)
    q = tk.DeviceArray((1, 14 * 64), np.float32).zero()
    out = tk.DeviceArray((1, 14 * 64), np.float32).zero()
    # a 17.6M-position session: its block table alone (4.4 MB) exceeds the
    # 4 MiB plan area (page ids may repeat; nothing is launched)
    ctx = 1_100_000 * 16 - 1
    with pytest.raises(tk.TgeError) as e:
        tk.decode_attention_static(pool, [tk.Session(ctx, 1, [0] * 1_100_000)], 14, 0, q, out)
    assert e.value.status == tk.ERR_CAPACITY, e.value
    assert "static limit" in tk.lib().tge_last_error().decode()
    # still usable afterwards
    tk.decode_attention_static(pool, [tk.Session(20, 1, [1, 2])], 14, 0, q, out)
    tk.hip().sync()
    assert np.all(np.isfinite(out.numpy()))
    for a in (q, out):
        a.close()
    pool.close()


def test_static_decode_refuses_a_capturing_stream(gpu):
    say("static decode: call on a capturing stream")
    hip = tk.hip()
    h = hip.h
    h.hipStreamBeginCapture.argtypes = [C.c_void_p, C.c_int]
    h.hipStreamEndCapture.argtypes = [C.c_void_p, C.POINTER(C.c_void_p)]
    h.hipGraphDestroy.argtypes = [C.c_void_p]
    h.hipStreamSynchronize.argtypes = [C.c_void_p]
    st = C.c_void_p()
    hip.ok(h.hipStreamCreate(C.byref(st)), "hipStreamCreate")
    pool = tk.KvPool(1, 4, 2, 64, tk.KV_F16)
    q = tk.DeviceArray((1, 14 * 64), np.float32).zero()
    out = tk.DeviceArray((1, 14 * 64), np.float32).zero()
    hip.sync()
    hip.ok(h.hipStreamBeginCapture(st, 2), "hipStreamBeginCapture")  # relaxed mode
    err = None
    try:
        tk.decode_attention_static(pool, [tk.Session(20, 1, [1, 2])], 14, 0, q, out, stream=st.value)
    except tk.TgeError as e:
        err = e
    finally:
        graph = C.c_void_p()
        hip.ok(h.hipStreamEndCapture(st, C.byref(graph)), "hipStreamEndCapture")
        if graph.value:
            h.hipGraphDestroy(graph)
    assert err is not None and err.status == tk.ERR_INVALID, err
    assert "capturing" in tk.lib().tge_last_error().decode()
    # the same stream decodes normally once the capture has ended
    tk.decode_attention_static(pool, [tk.Session(20, 1, [1, 2])], 14, 0, q, out, stream=st.value)
    hip.ok(h.hipStreamSynchronize(st), "hipStreamSynchronize")
    assert np.all(np.isfinite(out.numpy()))
    h.hipStreamDestroy(st)
    for a in (q, out):
        a.close()
    pool.close()
