"""train_impl's per-epoch lr / entropy-coefficient schedule (host logic,
pufferlib.cu:1828-1833, 1912-1948), pinned by closed forms: the cosine's end
points and midpoint, the anchor epoch, the warmup ramp composed with the
anneal, and the unchanged values when no schedule is on."""
import numpy as np

from ptcg_amd.trainer import TRAIN_DEFAULTS, epoch_schedule, cosine_annealing


def cfg(**kw):
    c = dict(TRAIN_DEFAULTS)
    c.update(kw)
    return c


def test_no_schedule_keeps_values():
    c = cfg(learning_rate=3e-4, ent_coef=0.01, total_epochs=10)
    for e in range(12):
        assert epoch_schedule(c, e) == (3e-4, 0.01)


def test_cosine_end_points_and_midpoint():
    base, lo = 1e-3, 1e-4
    assert cosine_annealing(base, lo, 0, 10) == np.float32(base)
    assert cosine_annealing(base, lo, 10, 10) == np.float32(lo)
    assert cosine_annealing(base, lo, 15, 10) == np.float32(lo)   # ratio clamps to 1
    assert abs(cosine_annealing(base, lo, 5, 10) - 0.5 * (base + lo)) < 1e-9
    assert cosine_annealing(base, lo, 3, 0) == np.float32(base)


def test_anneal_anchor_and_warmup():
    c = cfg(learning_rate=1e-3, anneal_lr=1, min_lr_ratio=0.1, total_epochs=20, lr_anneal_from_epoch=10)
    lr0, _ = epoch_schedule(c, 4)               # before the anchor: t clamps to 0
    assert lr0 == np.float32(1e-3)
    lr_end, _ = epoch_schedule(c, 20)
    assert abs(lr_end - 1e-4) < 1e-10
    lr_mid, _ = epoch_schedule(c, 15)
    assert abs(lr_mid - 0.5 * (1e-3 + 1e-4)) < 1e-9
    w = cfg(learning_rate=1e-3, lr_warmup_epochs=4, start_epoch=2, total_epochs=20)
    got = [epoch_schedule(w, e)[0] for e in (2, 3, 4, 5, 6)]
    want = [np.float32(np.float32(1e-3) * np.float32(k / 4)) for k in (1, 2, 3, 4, 4)]
    assert got == [float(x) for x in want]


def test_entropy_anneal():
    c = cfg(ent_coef=0.02, anneal_ent_coef=1, min_ent_coef_ratio=0.1, total_epochs=8)
    assert epoch_schedule(c, 0)[1] == np.float32(0.02)
    assert abs(epoch_schedule(c, 8)[1] - 0.002) < 1e-9
    assert abs(epoch_schedule(c, 4)[1] - 0.011) < 1e-9
