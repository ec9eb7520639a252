"""The KV-cache writer's quotient x / scale (csrc/cache_kernels.hpp, div_rn).

The writer divides every bf16 element by the per-tensor scale and rounds to
e4m3, as torch's ``(x / scale).to(torch.float8_e4m3fn)`` does (run_poc.py:96-103
quantises the cache; torch divides with IEEE single division).  For scales in
[2^-80, 2^126] it computes the quotient from y = RN(1 / scale) by Markstein's
correction, q0 = RN(x y), r = x - scale q0 (exact, one FMA), q = RN(q0 + r y),
and the host enables that path only in this range.  This test checks, on the
CPU with exact float32 FMA emulation, that q equals the correctly rounded
quotient RN(x / scale) for every finite bf16 x (the operands and quotients
below 2^-100, which round to an e4m3 zero either way, excepted) at scales
spread over the whole range and at its two ends.  The device code itself is
compared with torch's cast in tests/test_gpu_cache.py.
"""

import numpy as np

F32, F64 = np.float32, np.float64
LO, HI = F32(2.0 ** -80), F32(2.0 ** 126)  # the writer's fast-division range


def _fma32(a, b, c):
    """RN32(a * b + c) exactly for float32 arrays: a * b is exact in float64,
    the sum's float64 rounding error is recovered by TwoSum and decides the
    float32 rounding when the float64 sum lies on a float32 midpoint."""
    p = a.astype(F64) * b.astype(F64)
    cc = c.astype(F64)
    s = p + cc
    bb = s - p
    err = (p - (s - bb)) + (cc - bb)
    f = s.astype(F32)
    back = f.astype(F64)
    diff = s - back
    half = np.abs(np.spacing(f).astype(F64)) / 2
    mid = (np.abs(diff) == half) & (err != 0)
    away = np.nextafter(f, np.where(s > back, F32(np.inf), F32(-np.inf)).astype(F32))
    # on a midpoint s was rounded to f; the exact value lies beyond s (away
    # from f) when err has the sign of s - f
    return np.where(mid & (np.sign(err) == np.sign(diff)), away, f)


def _finite_bf16():
    x = (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)
    return x[np.isfinite(x)]


def _check(scales):
    x = _finite_bf16()
    x64 = x.astype(F64)
    checked = 0
    for d in scales:
        d = F32(d)
        assert LO <= d <= HI
        y = F32(F64(1.0) / F64(d))
        q0 = (x64 * F64(y)).astype(F32)
        r = _fma32(np.full_like(x, -d), q0, x)
        q = _fma32(r, np.full_like(x, y), q0)
        # RN32 of the exact quotient: float64 division then float32 rounding
        # is innocuous (53 >= 2 * 24 + 2 bits)
        exact = (x64 / F64(d)).astype(F32)
        ok = np.isfinite(exact) & (np.abs(exact) >= F32(2.0 ** -100)) & (np.abs(x) >= F32(2.0 ** -100))
        bad = ok & (q.view(np.uint32) != exact.view(np.uint32))
        assert not bad.any(), (float(d), float(x[bad][0]), float(q[bad][0]), float(exact[bad][0]))
        checked += int(ok.sum())
    return checked


def test_quotient_is_correctly_rounded_over_the_scale_range():
    # every third exponent from 2^-80 up with a random significand, per-tensor
    # scales amax / 448 of typical amaxes, the range's two ends and 48 random
    # scales below 1
    rng = np.random.default_rng(7)
    scales = [F32(2.0 ** e) * F32(1 + rng.integers(0, 1 << 23) / (1 << 23)) for e in range(-80, 126, 3)]
    scales += [F32(a) / F32(448.0) for a in (0.5, 1.0, 3.0, 4.5, 17.25, 300.0, 65504.0)]
    scales += [LO, np.nextafter(LO, F32(1)), HI, np.nextafter(HI, F32(0))]
    scales += list(rng.uniform(1e-4, 1.0, 48).astype(F32))
    with np.errstate(over="ignore", invalid="ignore"):
        assert _check([s for s in scales if LO <= s <= HI]) > 6_000_000


def test_the_check_finds_a_dropped_correction():
    """The uncorrected q0 = RN(x RN(1/d)) is off by an ulp for some x: the
    comparison above would see a missing FMA step."""
    x = _finite_bf16()
    x64 = x.astype(F64)
    d = F32(3.0) / F32(448.0)
    y = F32(F64(1.0) / F64(d))
    with np.errstate(over="ignore", invalid="ignore"):
        q0 = (x64 * F64(y)).astype(F32)
        exact = (x64 / F64(d)).astype(F32)
    assert (q0.view(np.uint32) != exact.view(np.uint32)).any()
