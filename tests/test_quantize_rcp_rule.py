# SPDX-License-Identifier: Apache-2.0
"""The pack kernels' division-free KIVI quantization rule, checked on the CPU.

The device quantizes with v = (x - mn) * rcp(scale), code rndne(v) with no
clamp (v stays inside [0, 15 + 4e-6]), and redoes an element with the exact
(x - mn) / scale + 0.5 when its v lies within 1e-5 of a tie k + 0.5
(kivi_pack_word in csrc/kvq_common.h).  This test replays that rule in numpy
fp32 with the reciprocal off by up to one ulp either way (v_rcp_f32's bound)
and requires codes identical to the exact rule of the reference
(pkg/ops/triton/kivi_pack.py:98-104, 195-204) on random groups, on groups on
the bf16 grid (where exact ties are common) and on groups built so the
quotients sit on the x.5 boundaries.
"""

from __future__ import annotations

import numpy as np

F = np.float32


def _exact(x, mn, sc):
    t = np.floor(((x - mn) / sc).astype(F) + F(0.5)).astype(F)
    return np.clip(t, 0, 15)


def _rule(x, mn, sc, rcp):
    d = (x - mn).astype(F)
    v = (d * rcp).astype(F)
    r = np.rint(v)  # round half to even, as v_rndne_f32
    near = ~(np.abs((v - r).astype(F)) <= F(0.49999))
    # without a clamp the fast codes must already be codes
    assert (r[~near] >= 0).all() and (r[~near] <= 15).all()
    # the fallback redoes the near-tie elements alone
    return np.where(near, _exact(x, mn, sc), r), near.mean()


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


def _check(x):
    mn = x.min(axis=1, keepdims=True)
    mx = x.max(axis=1, keepdims=True)
    sc = np.maximum(((mx - mn) / F(15)).astype(F), F(1e-6)).astype(F)
    r = (F(1) / sc).astype(F)
    want = _exact(x, mn, sc)
    rates = []
    for rcp in (r, np.nextafter(r, F(np.inf)), np.nextafter(r, F(0))):
        got, rate = _rule(x, mn, sc, rcp)
        assert (got == want).all()
        rates.append(rate)
    return float(np.mean(rates))


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
        rate = _check(x.to(torch.bfloat16).float().numpy())
        assert rate > 1e-4  # ties are frequent on a 16-bit grid


def test_rule_matches_exact_on_boundary_quotients():
    rng = np.random.default_rng(1)
    rate = _check(_boundary_groups(rng, 256, 128))
    assert rate > 0.5  # the data does drive the exact fallback


def test_rule_tiny_ranges_use_the_scale_floor():
    # mx - mn below 15e-6: scale floors to 1e-6, quotients stay in range
    rng = np.random.default_rng(2)
    base = rng.normal(size=(64, 1)).astype(F)
    x = (base + rng.uniform(0, 1e-5, size=(64, 32))).astype(F)
    _check(x)
