"""Independent pins of the oracle's density-control plan and L1 loss gradient (CPU).

adc_plan (maybe_densify_and_prune!, training.jl:313-444) on hand-built Gaussians whose
values sit exactly on, and one float32 step past, every threshold:

- prune: opacity logit < logit(pruning_min_opacity), strict (:340-341, :344-345);
- the max-scale prune: max log-scale > log(pruning_3d_max_scale), strict (:346-347), and
  only once iteration_nb > opacity_reset_interval (:337-349);
- the average 2D-mean gradient norm: accumulated / count for count >= 1, 0 for count 0
  (:327-334), against the threshold with >= (:351-354); a pruned Gaussian is not densified;
- clone where max log-scale <= log(densification_size_threshold), split otherwise (:355-359);
- the new counts, their inclusive scan and the ngidx_to_gidx map (:361-395).

l1_loss_grad (training.jl:206-215): +w where rendered > gt, -w where rendered < gt and for
ties (the reference's ifelse), w = (1 - weight) / length in float32, the D-SSIM term added as
a rounded product and a sum; the L1 sum on dyadic values whose sum is exact.
"""
import numpy as np

from tdgs_amd import host, training

f32 = np.float32


def _up(x):
    return np.nextafter(f32(x), f32(np.inf))


def _down(x):
    return np.nextafter(f32(x), f32(-np.inf))


PRUNE_LOGIT = f32(host.logit32(0.005))
LOG_MAX_SCALE = f32(np.log(f32(0.1 * 4.0)))
GRAD_T = f32(2e-4)
LOG_SIZE = f32(np.log(f32(0.01 * 4.0)))


def _gaussians(rows):
    """rows: (opacity logit, max log-scale, accumulated norm, count)."""
    n = len(rows)
    mo = np.zeros((n, 4), f32)
    sc = np.full((n, 3), f32(-6.0), f32)
    for i, (op, smax, _, _) in enumerate(rows):
        mo[i, 3] = op
        sc[i, i % 3] = smax   # the maximum sits on a different axis per Gaussian
    rot = np.tile(np.array([1, 0, 0, 0], f32), (n, 1))
    g = host.HostGaussians(mo, sc, rot, np.zeros((n, 3, 1), f32))
    return g


def _plan(oracle, rows, use_max_scale):
    g = _gaussians(rows)
    adc = oracle.AdcHost(len(rows))
    adc.accum[:] = [r[2] for r in rows]
    adc.counts[:] = [r[3] for r in rows]
    n_new = oracle.adc_plan(adc, g, float(PRUNE_LOGIT), use_max_scale, float(LOG_MAX_SCALE), float(GRAD_T),
                            float(LOG_SIZE))
    return n_new, adc


OK_OP = f32(1.0)     # an opacity logit far above the prune threshold
SMALL = f32(-8.0)    # a max log-scale far below both scale thresholds
# (opacity logit, max log-scale, accumulated norm, count), expected (prune, densify, clone)
CASES = [
    ((PRUNE_LOGIT, SMALL, 0.0, 1), (0, 0, 0)),                   # 0: logit exactly at the bound: kept
    ((_down(PRUNE_LOGIT), SMALL, 0.0, 1), (1, 0, 0)),            # 1: one step below: pruned
    ((OK_OP, LOG_MAX_SCALE, 0.0, 1), (0, 0, 0)),                 # 2: max scale exactly at the bound: kept
    ((OK_OP, _up(LOG_MAX_SCALE), 0.0, 1), (1, 0, 0)),            # 3: one step above: pruned (if active)
    ((OK_OP, SMALL, f32(5.0), 0), (0, 0, 0)),                    # 4: count 0: average 0, not densified
    ((OK_OP, SMALL, f32(2) * GRAD_T, 2), (0, 1, 1)),             # 5: average exactly the threshold: densified
    ((OK_OP, SMALL, _down(f32(4) * GRAD_T), 4), (0, 0, 0)),      # 6: just below: not densified
    ((OK_OP, LOG_SIZE, f32(1.0), 1), (0, 1, 1)),                 # 7: size exactly at the bound: clone
    ((OK_OP, _up(LOG_SIZE), f32(1.0), 1), (0, 1, 0)),            # 8: one step above: split
    ((_down(PRUNE_LOGIT), SMALL, f32(1.0), 1), (1, 0, 0)),       # 9: pruned wins over densify
    ((OK_OP, _up(LOG_MAX_SCALE), f32(1.0), 1), (1, 0, 0)),       # 10: scale-pruned wins over densify
]


def test_adc_plan_thresholds_and_average(oracle):
    rows = [c[0] for c in CASES]
    for use_max_scale in (True, False):
        n_new, adc = _plan(oracle, rows, use_max_scale)
        exp = np.array([c[1] for c in CASES], np.uint8)
        if not use_max_scale:
            # the scale-pruned ones are kept: 3 carried, 10 densified (split: its scale is
            # above the size threshold too)
            exp[3] = (0, 0, 0)
            exp[10] = (0, 1, 0)
        np.testing.assert_array_equal(adc.prune, exp[:, 0], err_msg=f"prune, max scale {use_max_scale}")
        np.testing.assert_array_equal(adc.densify, exp[:, 1], err_msg=f"densify, max scale {use_max_scale}")
        np.testing.assert_array_equal(adc.clone & adc.densify, exp[:, 2], err_msg=f"clone, max scale {use_max_scale}")
        counts = (1 - exp[:, 0]).astype(np.int32) + exp[:, 1]
        np.testing.assert_array_equal(adc.cs, np.cumsum(counts))
        assert n_new == int(counts.sum())
        parents = np.repeat(np.arange(1, len(rows) + 1), counts)
        np.testing.assert_array_equal(adc.ngidx[:n_new], parents)


def test_adc_plan_count_zero_never_divides(oracle):
    """count 0 with any accumulated value (also inf and a huge one) gives average 0."""
    rows = [(OK_OP, SMALL, f32(np.inf), 0), (OK_OP, SMALL, f32(3e38), 0), (OK_OP, SMALL, f32(0.0), 0)]
    n_new, adc = _plan(oracle, rows, True)
    assert n_new == 3 and not adc.densify.any() and not adc.prune.any()


def test_max_scale_prune_gate():
    o = training.TrainingOptions.for_scene(4.0)
    assert o.opacity_reset_interval == 3000
    for it, active in [(600, False), (2999, False), (3000, False), (3001, True), (3100, True)]:
        th = training.adc_plan_thresholds(it, o)
        assert th[1] is active, it
    th = training.adc_plan_thresholds(3100, o)
    assert th[0] == float(PRUNE_LOGIT)
    # pruning_3d_max_scale = 0.1 R and densification_size_threshold = 0.01 R (scene radius 4)
    assert th[2] == float(LOG_MAX_SCALE) and th[4] == float(LOG_SIZE)
    assert th[3] == o.densification_mean2d_grad_norm_threshold_ndc == 2e-4


def test_l1_gradient_sign_ties_and_weight(oracle):
    r = np.array([0.25, 0.5, 0.75, 0.5, 0.0, 1.0, 0.125, 0.625], f32)
    g = np.array([0.5, 0.5, 0.5, 0.25, 0.0, 1.0, 0.5, 0.625], f32)
    n = r.size
    l1_w = f32(1) - f32(0.2)
    s, out = oracle.l1_loss_grad(r, g, float(l1_w))
    w = f32(l1_w / f32(n))
    #           <   tie   >   >  tie  tie  <  tie
    sign = np.array([-1, -1, 1, 1, -1, -1, -1, -1], f32)
    np.testing.assert_array_equal(out, sign * w)
    assert s == 0.25 + 0 + 0.25 + 0.25 + 0 + 0 + 0.375 + 0   # dyadic: exact in double


def test_l1_gradient_dssim_term_rounds_product_then_sum(oracle):
    rng = np.random.default_rng(3)
    n = 4096
    r = rng.random(n, dtype=f32)
    g = np.where(rng.random(n) < 0.25, r, rng.random(n, dtype=f32)).astype(f32)   # a quarter ties
    dg = (rng.standard_normal(n) * 1e-3).astype(f32)
    weight = f32(0.2)
    l1_w = f32(1) - weight
    _, out = oracle.l1_loss_grad(r, g, float(l1_w), float(weight), dg)
    w = f32(l1_w / f32(n))
    base = np.where(r > g, w, -w).astype(f32)
    prod = (weight * dg).astype(f32)            # rounded to float32
    np.testing.assert_array_equal(out, (base + prod).astype(f32))
    fused = (base.astype(np.float64) + weight.astype(np.float64) * dg.astype(np.float64)).astype(f32)
    assert np.any(fused != out), "values chosen so that a fused multiply-add would differ"
    ties = r == g
    assert ties.sum() > 500
    np.testing.assert_array_equal(out[ties], (-w + prod[ties]).astype(f32))
