"""Host-side trainer logic without a GPU: the learning-rate annealing of
update_learning_rates! (training.jl:287-302) against its closed form
lr(it) = lr0^(1 - x) lr1^x, x = clamp((it - 1) / (steps - 1), 0, 1), evaluated in float64."""
import math

import numpy as np
import pytest

from tdgs_amd import training


def _closed_form(it, lr0, lr1, steps):
    x = min(max((it - 1) / (steps - 1), 0.0), 1.0)
    return lr0 ** (1.0 - x) * lr1 ** x


@pytest.mark.parametrize("radius", [1.0, 6.6, 0.37])
def test_annealed_means_lr_closed_form(radius):
    steps = 3001   # odd: iteration 1501 sits at x = 1/2 exactly
    to = training.TrainingOptions.for_scene(radius, nb_iterations=steps)
    lr0, lr1 = to.initial_means_lr, to.final_means_lr
    assert lr0 == pytest.approx(0.00016 * radius, rel=1e-6) and lr1 == pytest.approx(lr0 / 100, rel=1e-6)
    its = [1, 2, 3, 750, 1501, 2999, 3000, 3001, 3002, 10_000]
    got = [training.annealed_means_lr(it, to) for it in its]
    for it, v in zip(its, got):
        assert v == pytest.approx(_closed_form(it, lr0, lr1, steps), rel=2e-6), it
    # first iteration: the initial rate; the midpoint: the geometric mean; from the last
    # annealing step on: the final rate
    assert got[0] == pytest.approx(lr0, rel=1e-6)
    assert got[its.index(1501)] == pytest.approx(math.sqrt(lr0 * lr1), rel=2e-6)
    assert all(v == pytest.approx(lr1, rel=1e-6) for v in got[its.index(3001):])
    assert all(a > b for a, b in zip(got[:its.index(3001)], got[1:its.index(3001) + 1]))
    # float32 values, as the reference's F = Float32 arithmetic produces them
    assert all(float(np.float32(v)) == v for v in got)


def test_annealed_means_lr_two_steps():
    """nb_lr_annealing_steps == 2: the initial rate at iteration 1, the final one from 2 on
    (training.jl:293-295)."""
    to = training.TrainingOptions(nb_lr_annealing_steps=2, initial_means_lr=1e-3, final_means_lr=1e-5)
    assert training.annealed_means_lr(1, to) == pytest.approx(1e-3, rel=1e-6)
    assert training.annealed_means_lr(2, to) == pytest.approx(1e-5, rel=1e-6)
    assert training.annealed_means_lr(7, to) == pytest.approx(1e-5, rel=1e-6)
