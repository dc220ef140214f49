# SPDX-License-Identifier: Apache-2.0
"""The pack kernels' division-free KIVI quantization rule, checked on the CPU.

The device quantizes with d = x - mn, k = floor(d * rcp(scale)) and code
k + [y >= 0], y = fma(scale * 2^-24, 2^e(t), fma(-scale, t, d)), where
t = k + pred(0.5) and 2^e(t) is t with its mantissa cleared; it takes the
code as t + 0.25 (y >= 0) or t - 0.25 rounded to nearest even, with the sign
moved from y (kivi_pack_word in csrc/kvq_common.h).  This test replays that
rule in fp32
with both fmas emulated exactly (one rounding each) and the reciprocal off by
up to one ulp either way (v_rcp_f32's bound), and requires codes identical to
the exact rule of the reference (pkg/ops/triton/kivi_pack.py:98-104, 195-204)
on random groups, on groups on the bf16 grid (where exact ties are common), on
groups built so the quotients sit on the x.5 boundaries, and on groups whose
elements step ulp by ulp across the thresholds, including the k = 0 one where
RN(q + 0.5) reaches 1 at q = pred(0.5).  Two planted mistakes in the rule
(threshold 0.5 for k = 0; no half-ulp term) must fail on that data.
"""

from __future__ import annotations

from fractions import Fraction

import numpy as np

F = np.float32
PRED_HALF = np.nextafter(F(0.5), F(0))


def _exact(x, mn, sc):
    t = np.floor(((x - mn) / sc).astype(F) + F(0.5)).astype(F)
    return np.clip(t, 0, 15)


def _fma32(a, b, c):
    """fl32(a * b + c) with a single rounding, for fp32 arrays."""
    a, b, c = (np.asarray(v, dtype=np.float64) for v in (a, b, c))
    p = a * b  # exact: 48 significant bits
    s = p + c
    bb = s - p
    err = (p - (s - bb)) + (c - bb)  # p + c == s + err exactly
    r = s.astype(F)
    # s exactly halfway between two floats while err != 0: round by err's sign
    other = np.where(r.astype(np.float64) < s, np.nextafter(r, F(np.inf)),
                     np.nextafter(r, F(-np.inf)))
    mid = (r.astype(np.float64) + other.astype(np.float64)) / 2
    at_mid = (s == mid) & (err != 0)
    toward_other = np.sign(err) == np.sign(other.astype(np.float64) - s)
    return np.where(at_mid & toward_other, other, r).astype(F)


def _rule(x, mn, sc, rcp, t_of=None, half_ulp=True):
    d = (x - mn).astype(F)
    k = np.floor((d * rcp).astype(F))
    t = (k + PRED_HALF).astype(F) if t_of is None else t_of(k)
    e = (t.view(np.uint32) & np.uint32(0x7F800000)).view(F)
    s24 = (sc * F(2.0**-24)).astype(F)
    inner = _fma32(-sc, t, d)
    y = _fma32(s24, e, inner) if half_ulp else inner
    # the sign of y picks +-0.25; a -0 would pick the wrong side, and cannot occur
    assert not (np.signbit(y) & (y == 0)).any()
    step = np.where(np.signbit(y), F(-0.25), F(0.25)).astype(F)
    r = np.rint((t + step).astype(F)).astype(F)  # v_cvt_pk_u8_f32: nearest even
    assert (r == np.where(y >= 0, k + 1, k)).all()
    assert (r >= 0).all() and (r <= 15).all()  # codes with no clamp
    return r


def _boundary_groups(rng, rows, g):
    out = np.empty((rows, g), dtype=F)
    for row in out:
        mn = F(rng.normal())
        s = F(np.exp(rng.normal()) * 0.1)
        k = rng.integers(0, 15, g).astype(F)
        v = (mn + (k + F(0.5)) * s).astype(F)
        nudge = rng.integers(-1, 2, g)
        v = np.where(nudge < 0, np.nextafter(v, F(-np.inf)), v)
        v = np.where(nudge > 0, np.nextafter(v, F(np.inf)), v).astype(F)
        v[0], v[-1] = mn, F(mn + F(15) * s)
        row[:] = v
    return out


def _tie_groups(rng, rows, g):
    # mn = 0 so d = x exactly; elements step -4..4 ulps around scale * T for
    # T = k + 0.5 and around the k = 0 threshold just below scale / 2
    out = np.empty((rows, g), dtype=F)
    for row in out:
        mx = F(np.exp(rng.uniform(-6, 6)))
        sc = max(F(mx / F(15)), F(1e-6))
        k = rng.integers(0, 15, g)
        c = np.where(k == 0, (sc * PRED_HALF).astype(F), (sc * (k + F(0.5))).astype(F))
        v = c.astype(F)
        for step in range(4):
            up = rng.integers(-1, 2, g)
            v = np.where(up < 0, np.nextafter(v, F(-np.inf)), v)
            v = np.where(up > 0, np.nextafter(v, F(np.inf)), v).astype(F)
        v = np.clip(v, F(0), mx).astype(F)
        v[0], v[-1] = F(0), mx
        row[:] = v
    return out


def _check(x):
    mn = x.min(axis=1, keepdims=True)
    mx = x.max(axis=1, keepdims=True)
    sc = np.maximum(((mx - mn) / F(15)).astype(F), F(1e-6)).astype(F)
    r = (F(1) / sc).astype(F)
    want = _exact(x, mn, sc)
    for rcp in (r, np.nextafter(r, F(np.inf)), np.nextafter(r, F(0))):
        assert (_rule(x, mn, sc, rcp) == want).all()
    return mn, sc, r, want


def test_rule_matches_exact_on_random_groups():
    rng = np.random.default_rng(0)
    for g in (8, 32, 128):
        _check(rng.normal(size=(512, g)).astype(F))
        _check((rng.normal(size=(256, g)) * np.exp(rng.normal(size=(256, 1)) * 3)).astype(F))


def test_rule_matches_exact_on_the_bf16_grid():
    import torch

    rng = np.random.default_rng(2)
    for g in (64, 128):
        x = torch.from_numpy(rng.normal(size=(1024, g)).astype(F))
        x = x * torch.exp(torch.from_numpy(rng.normal(size=(1, g)).astype(F)))
        x = x.to(torch.bfloat16).float().numpy()
        mn, sc, _, want = _check(x)
        q = ((x - mn) / sc).astype(F)
        assert (q == np.floor(q) + F(0.5)).mean() > 1e-4  # exact ties are frequent


def test_rule_matches_exact_on_boundary_quotients():
    rng = np.random.default_rng(1)
    _check(_boundary_groups(rng, 256, 128))


def test_rule_matches_exact_stepping_across_thresholds():
    rng = np.random.default_rng(3)
    x = _tie_groups(rng, 512, 128)
    mn, sc, rcp, want = _check(x)
    q = (x / sc).astype(F)
    # the data reaches the k = 0 quirk: code 1 with q = pred(0.5) < 0.5
    assert ((want == 1) & (q < F(0.5))).any()
    # and the quotients straddle every k + 0.5 both ways
    for k in range(1, 15):
        assert ((q >= F(k + 0.5)) & (q < F(k + 0.5) + 1e-5) & (want == k + 1)).any()
        assert ((q < F(k + 0.5)) & (q > F(k + 0.5) - 1e-5) & (want == k)).any()
    # planted mistakes fail on it: threshold 0.5 for k = 0, and no half-ulp term
    wrong_t = _rule(x, mn, sc, rcp, t_of=lambda k: (k + F(0.5)).astype(F))
    assert (wrong_t != want).any()
    assert (_rule(x, mn, sc, rcp, half_ulp=False) != want).any()


def test_rule_tiny_ranges_use_the_scale_floor():
    # mx - mn below 15e-6: scale floors to 1e-6, quotients stay in range
    rng = np.random.default_rng(2)
    base = rng.normal(size=(64, 1)).astype(F)
    x = (base + rng.uniform(0, 1e-5, size=(64, 32))).astype(F)
    _check(x)


def _round32_exact(v):
    """Nearest float32 to the rational v, ties to even (brute force)."""
    f = np.float32(float(v))
    best = None
    for c in (np.nextafter(f, F(-np.inf)), f, np.nextafter(f, F(np.inf))):
        key = (abs(Fraction(float(c)) - v), int(c.view(np.uint32)) & 1)
        if best is None or key < best[0]:
            best = (key, c)
    return best[1]


def test_fma32_emulation_rounds_once():
    # products that nearly cancel the addend, as in the threshold test
    rng = np.random.default_rng(4)
    n = 3000
    a = (np.exp(rng.uniform(-10, 10, n)) * rng.choice([-1, 1], n)).astype(F)
    b = rng.uniform(0.25, 16, n).astype(F)
    c = (-(a.astype(np.float64) * b) * (1 + rng.uniform(-1e-6, 1e-6, n))).astype(F)
    c[::3] = (-(a * b)).astype(F)[::3]  # rounded product: the residue is the rounding error
    got = _fma32(a, b, c)
    for i in range(n):
        want = _round32_exact(Fraction(float(a[i])) * Fraction(float(b[i])) + Fraction(float(c[i])))
        assert got[i] == want, (a[i], b[i], c[i])


def test_group_scale_division_by_15_is_exact_for_every_mantissa():
    # kivi_group_scale: q0 = x * RN(1/15); q = fma(fma(-q0, 15, x), RN(1/15), q0)
    # must equal IEEE x / 15 (the reference's (mx - mn) / 15) for all of a
    # binade's 2^23 mantissas; powers of two scale every step exactly
    x = ((np.uint32(127) << 23) | np.arange(2**23, dtype=np.uint32)).view(F)
    rcp15 = F(1) / F(15)
    for shift in (0, 1, 3):
        xs = (x * F(2.0**shift)).astype(F)
        q0 = (xs * rcp15).astype(F)
        q = _fma32(_fma32(-q0, F(15), xs), rcp15, q0)
        assert (q == (xs / F(15)).astype(F)).all()
    # a planted mistake (no remainder step) does not pass
    assert ((x * rcp15).astype(F) != (x / F(15)).astype(F)).any()
