"""Pins of the iterative weight quantizers by what their mathematics fixes.

The oracle restates make_qkx1_quants (utils.rs:205-254), make_qx_quants
(utils.rs:65-202) and make_q3_quants (utils.rs:257-322) and the from_float
functions built on them (k_quants.rs:951-1011 Q2_K, 1170-1236 Q3_K,
1418-1473 Q4_K, 1608-1679 Q5_K, 1801-1871 Q6_K).  No Rust-produced GGUF
bytes exist to compare with, so each property below is one the algorithm
guarantees and one a plausible slip (a wrong weight, clamp bound, rounding
mode, pass count chaining, scale grid or field) breaks:

make_qkx1_quants (affine levels l in 0..nmax for x ~ scale * l + min):
  * the first pass starts from iscale = nmax / (max - min(min_x, 0));
  * every pass assigns each element its nearest level under that pass's
    (iscale, min), clamped to 0..nmax;
  * the returned scale is the least-squares scale of those levels at the
    pass's offset: sum((x - min) l) / sum(l^2);
  * the returned min is min(0, mean(x - scale l));
  * pass p+1 starts from 1/scale and the min pass p returned; the loop stops
    after the first pass that changes no level, or after ntry passes.
make_qx_quants / make_q3_quants (symmetric levels l in -nmax..nmax-1, x ~ scale l):
  * the returned scale is the x^2-weighted least-squares scale of the
    returned levels, sum(w x l) / sum(w l^2) with w = x^2 (rmse_type 1);
  * when the per-element loop stopped because a pass changed nothing, no
    single-element move of the kind that loop tries raises sum(w x l)^2 /
    sum(w l^2) (the quantity it maximises).
from_float (block level, decoded with the independent decoders of
tests/_formats.py): super-block scales on the 6-bit (4-bit for Q2_K,
8-bit for Q6_K/Q3_K) grid of the sub-block scales, and every quant the
nearest level under its decoded sub-block scale and min.
"""
import numpy as np
import pytest

from tests import _formats as F

Q2K, Q3K, Q4K, Q5K, Q6K = 10, 11, 12, 13, 14
EPS = 1e-4  # slack on f64 recomputations of f32 arithmetic (rounding ties)


def _round_away(v):
    """Rust f32::round (half away from zero), utils.rs:3-5 nearest_int."""
    return np.sign(v) * np.floor(np.abs(v) + 0.5)


def _blocks(rng, nblk, n):
    """Sub-blocks of realistic and awkward shapes: N(0, 0.02) weights, all
    positive (min clamps to 0), one outlier, a constant block, few distinct
    values, and tiny magnitudes."""
    out = [rng.normal(0, 0.02, n) for _ in range(nblk)]
    out += [np.abs(rng.normal(0.05, 0.02, n)) + 0.01 for _ in range(nblk // 8)]
    for _ in range(nblk // 8):
        v = rng.normal(0, 0.02, n)
        v[rng.integers(n)] = rng.choice([-1, 1]) * 0.5
        out.append(v)
    for _ in range(nblk // 4):  # opposite extremes: the top level (nmax - 1) is reachable
        v = rng.normal(0, 0.02, n)
        a, b = rng.choice(n, 2, replace=False)
        v[a] = 0.1
        v[b] = -rng.uniform(0.090, 0.0999)
        out.append(v)
    out.append(np.full(n, 0.3))
    out += [rng.choice([-0.1, 0.0, 0.05, 0.2], n) for _ in range(nblk // 16)]
    out += [rng.normal(0, 1e-6, n) for _ in range(4)]
    return [np.asarray(v, np.float32) for v in out]


def _nearest_level_ok(t, l, lo, hi):
    """l is t rounded to the nearest integer and clamped to [lo, hi]."""
    t = np.asarray(t, np.float64)
    inner = (l > lo) & (l < hi)
    ok = np.ones(t.shape, bool)
    ok &= ~inner | (np.abs(t - l) <= 0.5 + EPS)
    ok &= ~(l == lo) | (t <= lo + 0.5 + EPS)
    ok &= ~(l == hi) | (t >= hi - 0.5 - EPS)
    return ok.all()


# ------------------------------------------------------------ make_qkx1_quants
@pytest.mark.parametrize("nmax,n", [(15, 32), (31, 32), (3, 16)])  # Q4_K, Q5_K, Q2_K
def test_make_qkx1_quants_properties(orc, nmax, n):
    rng = np.random.default_rng(100 + nmax)
    passes_seen = []
    for x in _blocks(rng, 400, n):
        s, nm, lv, passes, isu, mu = orc.make_qkx1_quants(nmax, 5, x)
        x64 = x.astype(np.float64)
        if x.max() == x.min():
            assert s == 0 and nm == 0 and passes == 0
            continue
        passes_seen.append(passes)
        assert 1 <= passes <= 5
        assert lv.max() <= nmax
        # levels: nearest under the last pass's affine map, clamped
        assert _nearest_level_ok(np.float64(isu) * (x64 - mu), lv.astype(np.int64), 0, nmax)
        # least-squares scale at the pass's offset
        l64 = lv.astype(np.float64)
        want = ((x64 - mu) * l64).sum() / (l64 * l64).sum()
        assert abs(s - want) <= 1e-5 * abs(want)
        # min = min(0, mean(x - scale l))
        want_min = min(0.0, float((x64 - np.float64(s) * l64).mean()))
        assert abs(-nm - want_min) <= 1e-5 * np.abs(x64).max()
        # chaining of passes and the stop rule
        if passes == 1:
            m0 = np.float32(min(x.min(), np.float32(0)))
            assert mu == m0
            assert isu == np.float32(nmax) / (x.max() - m0)
        else:
            s1, nm1, lv1, p1, _, _ = orc.make_qkx1_quants(nmax, passes - 1, x)
            assert p1 == passes - 1
            assert isu == np.float32(1) / s1 and mu == -nm1
            if passes < 5:
                assert np.array_equal(lv, lv1), "stopped although the last pass changed levels"
            prev = np.zeros(n, np.uint8)
            for p in range(1, passes):
                lp = orc.make_qkx1_quants(nmax, p, x)[2]
                assert not np.array_equal(lp, prev), f"pass {p} changed nothing but the loop went on"
                prev = lp
    # all pass counts occur, including blocks that still change at pass 5
    assert max(passes_seen) == 5 and min(passes_seen) <= 2


def test_make_qkx1_quants_ntry_bounds_passes(orc):
    rng = np.random.default_rng(7)
    x = rng.normal(0, 0.02, 32).astype(np.float32)
    for ntry in range(1, 6):
        assert orc.make_qkx1_quants(15, ntry, x)[3] <= ntry


# ------------------------------------------------------------ make_qx_quants
def _weighted_optimal(x, l, lo, hi):
    """Per block (rows of x, l): no single-element move of the per-element
    loop raises slx^2 / sl2."""
    x = np.atleast_2d(x).astype(np.float64)
    l = np.atleast_2d(l).astype(np.float64)
    w = x * x
    S_lx = (w * x * l).sum(axis=1, keepdims=True)
    S_l2 = (w * l * l).sum(axis=1, keepdims=True)
    slx = S_lx - w * x * l
    sl2 = S_l2 - w * l * l
    with np.errstate(divide="ignore", invalid="ignore"):
        t = x * sl2 / slx
    tie = np.abs(np.abs(t - np.trunc(t)) - 0.5) < EPS  # the f32 loop may round either way
    new = np.clip(_round_away(np.nan_to_num(t)), lo, hi)
    slx2 = slx + w * x * new
    sl22 = sl2 + w * new * new
    better = (slx > 0) & ~tie & (new != l) & (sl22 > 0) & (slx2 * slx2 * S_l2 > S_lx * S_lx * sl22 * (1 + EPS))
    return ~better.any(axis=1)


def _symmetric_quantizer_case(fn, nmax, seed, rmse_passes_idx, changed_idx):
    rng = np.random.default_rng(seed)
    blocks = _blocks(rng, 600, 16)
    for _ in range(20000):  # opposite extremes: moves onto the top level nmax - 1 occur
        v = rng.normal(0, 0.02, 16)
        a, b = rng.choice(16, 2, replace=False)
        v[a] = 0.1
        v[b] = -rng.uniform(0.08, 0.0999)
        blocks.append(v.astype(np.float32))
    xs, ls = [], []
    for x in blocks:
        s, lv, info = fn(x)
        if np.abs(x).max() == 0:
            assert s == 0
            continue
        l = lv.astype(np.int64) - nmax
        assert l.min() >= -nmax and l.max() <= nmax - 1
        x64 = x.astype(np.float64)
        w = x64 * x64
        want = (w * x64 * l).sum() / (w * l * l).sum()
        assert abs(s - want) <= 1e-4 * abs(want), (s, want)
        if info[changed_idx] == 0:
            xs.append(x)
            ls.append(l)
        else:
            assert info[rmse_passes_idx] == 5
    ok = _weighted_optimal(np.stack(xs), np.stack(ls), -nmax, nmax - 1)
    assert ok.all(), f"{(~ok).sum()} blocks not locally optimal"
    assert len(xs) > 0.9 * len(blocks)


def test_make_qx_quants_properties(orc):
    """Q6_K's make_qx_quants(16, 32, ., ., 1)."""
    _symmetric_quantizer_case(lambda x: orc.make_qx_quants(32, x, 1), 32, 200, 1, 2)


def test_make_q3_quants_properties(orc):
    """Q3_K's make_q3_quants(., 4, true)."""
    _symmetric_quantizer_case(lambda x: orc.make_q3_quants(4, x, True), 4, 300, 0, 1)


def _wlsq_objective(x, l):
    """sum(w x l)^2 / sum(w l^2) with w = x^2, in f64 (the quantity the
    refinement loops of make_qx_quants / make_q3_quants maximise)."""
    x = x.astype(np.float64)
    l = l.astype(np.float64)
    w = x * x
    den = (w * l * l).sum()
    return ((w * x * l).sum()) ** 2 / den if den > 0 else 0.0


def _near_half(v):
    """Elements whose nearest-integer rounding an f32 / f64 difference may flip."""
    return np.abs(np.abs(v - np.trunc(v)) - 0.5) < EPS * np.maximum(1.0, np.abs(v))


def test_make_qx_quants_whole_block_loop(orc):
    """The first (whole-block) refinement loop of make_qx_quants
    (utils.rs:113-139), from the levels it leaves and its pass counts:
      * it starts from l0 = nearest(-nmax / max * x) (clamped) and runs at
        most 3 passes; a pass whose levels are kept strictly raises the
        objective, so kept passes end above l0 and differ from it;
      * its first pass decides on the candidate nearest(x / scale0), scale0
        the least-squares scale of l0: a candidate equal to l0 ends the loop
        after one pass, a clearly better one (objective up by more than
        1e-5 relative, well above f32 rounding) is kept;
      * when it stopped before 3 kept passes, it stopped at the first pass
        whose candidate levels nearest(x / scale) under the levels' own
        least-squares scale either change nothing or do not raise the
        objective (slx^2 <= best * sl2).
    A flipped stop test or a dropped pass (clearly better candidates not
    kept), an extra pass, or a candidate built from a stale scale breaks one
    of these."""
    nmax = 32
    rng = np.random.default_rng(410)
    blocks = _blocks(rng, 800, 16)
    kept = np.zeros(4, int)
    checked = clearly_better = 0
    for x in blocks:
        s, lv, info, mid = orc.make_qx_quants(nmax, x, 1, mid=True)
        passes, kept_passes = int(info[0]), int(info[3])
        if np.abs(x).max() == 0:
            assert passes == 0
            continue
        assert 1 <= passes <= 3 and 0 <= kept_passes <= passes
        assert kept_passes == 3 or passes == kept_passes + 1, info
        kept[kept_passes] += 1
        x64 = x.astype(np.float64)
        amax_i = int(np.argmax(np.abs(x)))
        t0 = -nmax / x64[amax_i] * x64
        l0 = np.clip(_round_away(t0), -nmax, nmax - 1)
        l = mid.astype(np.int64) - nmax
        assert l.min() >= -nmax and l.max() <= nmax - 1
        if _near_half(t0).any():
            continue
        f0, f = _wlsq_objective(x64, l0), _wlsq_objective(x64, l)
        w = x64 * x64
        t1 = x64 / ((w * x64 * l0).sum() / (w * l0 * l0).sum())
        if not _near_half(t1).any():
            cand1 = np.clip(_round_away(t1), -nmax, nmax - 1)
            if np.array_equal(cand1, l0):
                assert passes == 1 and kept_passes == 0, info
            elif _wlsq_objective(x64, cand1) > f0 * (1 + 1e-5):
                assert kept_passes >= 1, (x.tolist(), info)
                clearly_better += 1
        if kept_passes == 0:
            assert np.array_equal(l, l0)
        else:
            assert not np.array_equal(l, l0) and f > f0 * (1 - EPS), (f, f0)
        if kept_passes < 3:
            w = x64 * x64
            scale = (w * x64 * l).sum() / (w * l * l).sum()
            t = x64 / scale
            if _near_half(t).any():
                continue
            cand = np.clip(_round_away(t), -nmax, nmax - 1)
            assert np.array_equal(cand, l) or _wlsq_objective(x64, cand) <= f * (1 + EPS), \
                (x.tolist(), l.tolist(), cand.tolist())
        checked += 1
    # the distribution is not degenerate: blocks stop after 0, 1 and 2 kept passes
    assert checked > 0.8 * len(blocks)
    assert kept[0] > 0 and kept[1] > 0 and clearly_better > 20, (kept, clearly_better)


def test_make_q3_quants_initial_levels(orc):
    """make_q3_quants' counterpart of the whole-block start (utils.rs:275-284):
    its per-element loop starts from l0 = round(-nmax / max * x) clamped to
    -nmax..nmax-1 (max the signed element of largest magnitude).  When that
    loop's first pass changes nothing, the returned levels are exactly l0 and
    the returned scale is their weighted least-squares scale; the
    non-rmse path returns l0 and 1 / iscale."""
    nmax = 4
    rng = np.random.default_rng(420)
    blocks = _blocks(rng, 800, 16)
    untouched = 0
    for x in blocks:
        if np.abs(x).max() == 0:
            continue
        x64 = x.astype(np.float64)
        amax_i = int(np.argmax(np.abs(x)))
        t0 = -nmax / x64[amax_i] * x64
        if _near_half(t0).any():
            continue
        l0 = np.clip(_round_away(t0), -nmax, nmax - 1)
        s, lv, info = orc.make_q3_quants(nmax, x, False)
        assert np.array_equal(lv.astype(np.int64) - nmax, l0)
        assert abs(s - x64[amax_i] / -nmax) <= 1e-6 * abs(s)
        s, lv, info = orc.make_q3_quants(nmax, x, True)
        if info[0] == 1 and info[1] == 0:
            untouched += 1
            assert np.array_equal(lv.astype(np.int64) - nmax, l0)
            w = x64 * x64
            want = (w * x64 * l0).sum() / (w * l0 * l0).sum()
            assert abs(s - want) <= 1e-4 * abs(want)
    assert untouched > 10


# ------------------------------------------------------------ from_float, block level
def _f16(v):
    return np.float32(np.float16(np.float32(v)))


def _weights(rng, nblk):
    x = rng.normal(0, 0.02, (nblk, 256)).astype(np.float32)
    x[1] = 0.0
    x[2, :32] = 0.0  # one all-zero sub-block
    x[3] = np.abs(x[3]) + 0.01  # all positive
    x[4, 7] = 0.9  # outlier
    return x


@pytest.mark.parametrize("dt,nmax,sub,grid", [(Q4K, 15, 32, 63), (Q5K, 31, 32, 63), (Q2K, 3, 16, 15)])
def test_affine_kquant_from_float_block(orc, dt, nmax, sub, grid):
    rng = np.random.default_rng(400 + dt)
    x = _weights(rng, 48)
    b = orc.from_float(dt, x)
    dec = {Q4K: F.decode_q4k, Q5K: F.decode_q5k, Q2K: F.decode_q2k}[dt](b)
    d, dmin, sc, mn, q = dec
    nsub = 256 // sub
    for i in range(x.shape[0]):
        res = [orc.make_qkx1_quants(nmax, 5, x[i, j * sub:(j + 1) * sub]) for j in range(nsub)]
        scales = np.array([r[0] for r in res], np.float32)
        mins = np.array([r[1] for r in res], np.float32)
        max_scale = max(np.float32(0), scales.max())
        max_min = max(np.float32(0), mins.max())
        assert d[i] == _f16(max_scale / np.float32(grid))
        assert dmin[i] == _f16(max_min / np.float32(grid))
        for j in range(nsub):
            # the scale grid: sc_j = round(grid * s_j / max_s) (6-bit fields clamp at 63)
            ws = _round_away(np.float32(np.float32(grid) / max_scale) * scales[j]) if max_scale > 0 else 0
            wm = _round_away(np.float32(np.float32(grid) / max_min) * mins[j]) if max_min > 0 else 0
            if dt != Q2K:
                ws, wm = min(ws, 63), min(wm, 63)
            assert sc[i, j] == ws and mn[i, j] == wm
            qs = q[i, j * sub:(j + 1) * sub]
            step = np.float64(d[i]) * sc[i, j]
            if np.float32(d[i]) * np.float32(sc[i, j]) == 0:
                assert not qs.any()
                continue
            t = (x[i, j * sub:(j + 1) * sub].astype(np.float64) + np.float64(dmin[i]) * mn[i, j]) / step
            assert _nearest_level_ok(t, qs, 0, nmax)


def test_q6k_from_float_block(orc):
    rng = np.random.default_rng(500)
    x = _weights(rng, 48)
    b = orc.from_float(Q6K, x)
    d, sc, q = F.decode_q6k(b)
    for i in range(x.shape[0]):
        res = [orc.make_qx_quants(32, x[i, 16 * j:16 * j + 16], 1) for j in range(16)]
        scales = np.array([r[0] for r in res], np.float32)
        jmax = int(np.argmax(np.abs(scales)))  # first of the largest |scale|
        max_scale = scales[jmax] if np.abs(scales).max() > 0 else np.float32(0)
        with np.errstate(divide="ignore", invalid="ignore"):
            iscale = np.float32(-128) / max_scale
            assert d[i] == _f16(np.float32(1) / iscale) or (max_scale == 0 and d[i] == 0)
            for j in range(16):
                v = np.float32(iscale * scales[j])
                want = 0 if np.isnan(v) else min(int(_round_away(np.float64(v))), 127)
                assert sc[i, j] == want
        for j in range(16):
            qs = q[i, 16 * j:16 * j + 16]
            if np.float32(d[i]) * np.float32(sc[i, j]) == 0:
                # the sub-block keeps make_qx_quants' own levels
                assert np.array_equal(qs, res[j][1].astype(np.int64) - 32)
                continue
            t = x[i, 16 * j:16 * j + 16].astype(np.float64) / (np.float64(d[i]) * sc[i, j])
            assert _nearest_level_ok(t, qs, -32, 31)


def test_q3k_from_float_block(orc):
    rng = np.random.default_rng(600)
    x = _weights(rng, 48)
    b = orc.from_float(Q3K, x)
    d, sc, q = F.decode_q3k(b)
    for i in range(x.shape[0]):
        scales = np.array([orc.make_q3_quants(4, x[i, 16 * j:16 * j + 16], True)[0] for j in range(16)], np.float32)
        jmax = int(np.argmax(np.abs(scales)))
        max_scale = scales[jmax]
        if max_scale == 0:  # every scale field 0 (decoded -32), d = 0, every level stored 0
            assert d[i] == 0 and np.all(sc[i] == -32) and np.all(q[i] == -4)
            continue
        iscale = np.float32(-32) / max_scale
        assert d[i] == _f16(np.float32(1) / iscale)
        for j in range(16):
            want = min(max(int(_round_away(np.float64(np.float32(iscale * scales[j])))), -32), 31)
            assert sc[i, j] == want
            qs = q[i, 16 * j:16 * j + 16]
            if np.float32(d[i]) * np.float32(sc[i, j]) == 0:
                assert np.all(qs == -4)  # levels left at stored 0
                continue
            t = x[i, 16 * j:16 * j + 16].astype(np.float64) / (np.float64(d[i]) * sc[i, j])
            assert _nearest_level_ok(t, qs, -4, 3)
