"""Closed-form int8 block cases for the reference quantizer (qwen2.cpp:88-104).

The reference computes, per 32-value block with absolute maximum m,
    scale = m / 127.0f,  inv = 1.0f / scale   (fp32, correctly rounded)
    code  = trunc(fl(fl(x * inv) +- 0.5f))      (product rounded, then the add)
and a format with f16 scales stores float_to_half(scale) but keeps these
codes. The two generators below build blocks whose expected codes follow from
exact arithmetic (float64 holds every product of two fp32 values exactly), so
that a quantizer that fuses the multiply-add, or that derives its codes from
the f16-rounded scale, returns a different code on every block.
"""
import numpy as np


def _f32(x):
    return np.float32(x)


def _scale_inv(m):
    scale = _f32(_f32(m) / _f32(127.0))
    inv = _f32(_f32(1.0) / scale)
    return scale, inv


def contraction_blocks(n, seed=0):
    """n blocks of 32 values with, at slot 0, the block maximum m and at
    slots 1..8 values +-x whose exact product x*inv lies in
    (0.5 - 1.5 * 2^-25, 0.5 - 2^-25): rounded first it is 0.5 - 2^-25, and
    adding 0.5 gives 1 - 2^-25, a tie that rounds to 1.0 (code +-1); fused
    into one multiply-add, x*inv + 0.5 lies below 1 - 2^-25 and rounds to
    1 - 2^-24 (code 0). Returns (blocks [n, 32] float32, expected codes
    [n, 32] int8)."""
    rng = np.random.default_rng(seed)
    lo, hi = 0.5 - 1.5 * 2.0 ** -25, 0.5 - 2.0 ** -25
    blocks, codes = [], []
    while len(blocks) < n:
        m = _f32(np.ldexp(1.0 + rng.random(), int(rng.integers(-40, 40))))
        _, inv = _scale_inv(m)
        center = _f32(0.5 / float(inv))
        hit = None
        for d in range(-64, 65):
            x = _f32(center + _f32(d) * np.spacing(center))
            p = float(x) * float(inv)  # exact
            if lo < p < hi:
                hit = x
                break
        if hit is None:
            continue
        # the two roundings really differ on this value
        un = _f32(_f32(p) + _f32(0.5))
        fu = _f32(p + 0.5)
        assert int(un) == 1 and int(fu) == 0, (m, hit)
        b = np.zeros(32, np.float32)
        c = np.zeros(32, np.int8)
        b[0], c[0] = m, 127
        for j in range(1, 9):
            s = 1 if j % 2 else -1
            b[j], c[j] = s * hit, s
        blocks.append(b)  # the other slots stay 0 (code 0 for any scale)
        codes.append(c)
    return np.stack(blocks), np.stack(codes)


def f16_scale_blocks(n, seed=0):
    """n blocks whose fp32 scale s rounds to an f16 value s16 > s with
    relative gap rho >= 2^-13. Slot 0 holds the maximum m = 127 s-ish; slots
    1..31 hold x = (k + 0.5) * s * (1 + rho / 2) for k = 4..123: x/s sits
    (k + 0.5) * rho / 2 >= 2e-4 above k + 0.5, so the reference's code is
    k + 1, while x/s16 sits below k + 0.5 and a quantizer using the f16
    scale gives k. Returns (blocks [n, 32] float32, expected codes, the f16
    scale bits)."""
    import oracle as O

    rng = np.random.default_rng(seed)
    blocks, codes, scales = [], [], []
    while len(blocks) < n:
        m = _f32(np.ldexp(1.0 + rng.random(), int(rng.integers(-8, 12))))
        scale, _ = _scale_inv(m)
        s16 = float(O.half_to_float(O.float_to_half(np.array([scale], np.float32)))[0])
        rho = s16 / float(scale) - 1.0
        if rho < 2.0 ** -13:
            continue
        ks = rng.choice(np.arange(4, 124), size=31, replace=False)
        x = np.array([(k + 0.5) * float(scale) * (1 + rho / 2) for k in ks])
        xs = x.astype(np.float32)
        # keep x below m so the maximum stays slot 0, and check the margins
        # in exact arithmetic with the float32 values actually stored
        if np.any(np.abs(xs) >= m):
            continue
        r = xs.astype(np.float64) / float(scale)
        assert np.all(r - (ks + 0.5) > 1e-4)
        assert np.all(xs.astype(np.float64) / s16 < ks + 0.5)
        sign = np.where(rng.random(31) < 0.5, -1, 1)
        b = np.empty(32, np.float32)
        c = np.empty(32, np.int8)
        b[0], c[0] = m, 127
        b[1:], c[1:] = sign * xs, sign * (ks + 1)
        blocks.append(b)
        codes.append(c)
        scales.append(O.float_to_half(np.array([scale], np.float32))[0])
    return np.stack(blocks), np.stack(codes), np.array(scales)
