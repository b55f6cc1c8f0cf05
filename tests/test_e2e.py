"""The end-to-end training step's pieces (``ace_kernels.e2e``) on the CPU:
network shapes, Dice closed forms, deep-supervision weights, deterministic
synthetic batches, and two training steps with the CPU reference loss."""

from __future__ import annotations

import math

import torch

from ace_kernels import e2e


def test_network_outputs_four_levels_full_resolution_first() -> None:
    torch.manual_seed(0)
    net = e2e.SegResNetDS(1, 4, init_filters=4)
    outs = net(torch.randn(1, 1, 32, 32, 32))
    assert [tuple(o.shape) for o in outs] == [(1, 4, 32, 32, 32), (1, 4, 16, 16, 16),
                                              (1, 4, 8, 8, 8), (1, 4, 4, 4, 4)]


def test_dice_closed_forms() -> None:
    labels = torch.zeros(1, 1, 4, 4, 4)
    labels[..., :2] = 1.0
    perfect = torch.nn.functional.one_hot(labels[:, 0].long(), 2).movedim(-1, 1).float() * 40.0
    assert float(e2e.dice_loss(perfect, labels)) < 1e-6
    # every voxel class 0, predicted perfectly: class 1 is absent, and with
    # smooth_nr = 0 its term is 1 - 0 / (sum p^2 + 1e-5) = 1
    zeros = torch.zeros(1, 1, 4, 4, 4)
    only0 = torch.stack((torch.full((1, 4, 4, 4), 40.0), torch.full((1, 4, 4, 4), -40.0)), 1)
    assert math.isclose(float(e2e.dice_loss(only0, zeros)), 0.5, rel_tol=1e-5)
    # uniform prediction over C classes, one class everywhere:
    # present class 1 - 2 (N/C) / (N + N/C^2); the others 1
    c, n = 4, 64
    uniform = torch.zeros(1, c, 4, 4, 4)
    want = ((1 - 2 * (n / c) / (n + n / c ** 2)) + (c - 1)) / c
    assert math.isclose(float(e2e.dice_loss(uniform, zeros)), want, rel_tol=1e-5)


def test_deep_supervision_weights_and_targets() -> None:
    assert e2e.ds_weights(4) == [1.0, 0.5, 0.25, 0.125]
    assert e2e.ds_weights(6)[-2:] == [0.0625, 0.0625]
    labels = torch.arange(64, dtype=torch.float32).reshape(1, 1, 4, 4, 4) % 3
    outs = [torch.zeros(1, 3, 4, 4, 4), torch.zeros(1, 3, 2, 2, 2)]
    t = e2e.level_targets(labels, outs)
    assert t[0] is labels
    assert torch.equal(t[1], labels[..., ::2, ::2, ::2])


def test_synthetic_batches_are_deterministic_per_step() -> None:
    a = e2e.synthetic_batch(3, 0, 2, 4, (16, 16, 16), "cpu")
    b = e2e.synthetic_batch(3, 0, 2, 4, (16, 16, 16), "cpu")
    c = e2e.synthetic_batch(4, 0, 2, 4, (16, 16, 16), "cpu")
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    assert not torch.equal(a[1], c[1])
    assert a[1].dtype == torch.float32 and set(a[1].unique().tolist()) <= {0.0, 1.0, 2.0, 3.0}


def test_two_cpu_steps_with_the_reference_loss() -> None:
    from oracle.reference import register_reference

    register_reference()
    for ace in ("reference", "none"):
        cfg = e2e.E2EConfig(binning="hard", ace=ace, batch=1, patch=(32, 32, 32),
                            init_filters=4, steps=2, skip_steps=0, device="cpu")
        res = e2e.train(cfg)
        assert len(res.losses) == 2 and all(math.isfinite(v) for v in res.losses)
        if ace == "none":
            assert res.aces == [0.0, 0.0]
        else:
            assert all(v > 0 for v in res.aces)
