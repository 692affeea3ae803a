"""Seeded training state built with this package (host tensors), for the
checkpoint fixture whose file this package writes and the reference reads
(``make_golden.py``'s ``package_checkpoint_case``) and for the host test that
checks that fixture (``tests/test_checkpoint.py``)."""

from __future__ import annotations

import numpy as np

# save_checkpoint's keyword arguments for the fixture.
SAVE = dict(step=7, epoch=1, config={"case": "package-writer", "layers": [2, 3]}, cumulative_tokens=12345)


def build(nt):
    """(named parameters, AdamW, WarmupCosine, GradScaler) in this package:
    a 40 x 48 weight (decay 0.1) and a 40-element bias (no decay), moments
    and step counts set through load_state_dict, the schedule advanced four
    times, the scaler halfway to its next growth."""
    from namitorch_amd.optim.lr_scheduler import WarmupCosine

    rng = np.random.Generator(np.random.PCG64(6161))

    def normal(shape, sigma):
        return (rng.standard_normal(shape, dtype=np.float32) * np.float32(sigma)).astype(np.float32)

    named = {"weight": nt.Parameter(normal((40, 48), 0.02)), "bias": nt.Parameter(normal(40, 0.02))}
    optimizer = nt.optim.AdamW([{"params": [named["weight"]], "weight_decay": 0.1},
                                {"params": [named["bias"]], "weight_decay": 0.0}],
                               lr=2e-3, betas=(0.9, 0.95), eps=1e-8)
    state = optimizer.state_dict()
    state["state"] = {
        index: {"step": 7,
                "exp_avg": nt.Tensor(normal(parameter.shape, 1e-4)),
                "exp_avg_sq": nt.Tensor(np.abs(normal(parameter.shape, 1e-7)))}
        for index, parameter in enumerate((named["weight"], named["bias"]))
    }
    optimizer.load_state_dict(state)
    scheduler = WarmupCosine(optimizer, 3, 12, min_lr=1e-4)
    for _ in range(4):
        scheduler.step()
    scaler = nt.GradScaler(init_scale=4096.0, growth_interval=3)
    scaler.load_state_dict(dict(scaler.state_dict(), scale=2048.0, growth_tracker=2))
    return named, optimizer, scheduler, scaler

