"""The perf model's prediction (cairn_amd/perf.py, predict) against launches measured on this GPU: the kernel the
selector picks, priced at the rate the machine card records for it (bench.py --only calibrate), on the share of the
machine its tiling keeps busy; the skinny kernels at their recorded share of HBM. The reference's own pricing test
(tests/soundness/test_tensor.py:132-148) checks its roofline's arithmetic only; this one runs the launches.

A launch's time is the average of a burst of 20 back to back (one event pair around them) after 300 warm-up launches
(a GPU out of idle takes about that many to reach its clock): the steady state the card's rates were calibrated in, where the launch cost the card adds to a lone call (its
`launch_ns`) is hidden, so the prediction's device time (its `ns` less `launch_ns`) is what is compared. The model
leaves out what it cannot know before a launch: the per-tile fixed cost (the prologue's first loads and the epilogue,
about 10 us a round of tiles, more with GELU), and the clock, which rises on a partly idle chip (power sets it: a
round of 48 tiles on 256 CUs runs at about 2.4 GHz, a full one at about 1.6). So each case is held to a band around
the measured time: a full machine within about 15%; a partial round, where the model charges the idle CUs at the
full-load clock, as an upper bound."""

from __future__ import annotations

import sys

import numpy as np
import pytest

from cairn_amd import hip
from cairn_amd import lib as L
from cairn_amd import perf

pytestmark = pytest.mark.gpu


def say(*what):
    print("[gpu]", *what, flush=True)
    sys.stdout.flush()


def burst_us(descs: list, stream: hip.Stream, warmup: int = 300, reps: int = 20) -> float:
    """Launches cycle through `descs` (the decode shapes rotate copies of b past the 256 MB MALL, as the card's
    calibration did)."""
    for i in range(warmup):
        L.run(descs[i % len(descs)], stream.handle)
    stream.synchronize()
    a, b = hip.Event(), hip.Event()
    a.record(stream)
    for i in range(reps):
        L.run(descs[i % len(descs)], stream.handle)
    b.record(stream)
    b.synchronize()
    us = a.elapsed_ms(b) * 1e3 / reps
    a.close()
    b.close()
    return us


def operand(ab: int, shape, rng) -> np.ndarray:
    if ab == L.I8:
        return rng.integers(-127, 128, shape, dtype=np.int8)
    x = rng.standard_normal(shape, dtype=np.float32) / np.float32(64.0)
    u = x.view(np.uint32)
    return ((u + np.uint32(0x7FFF) + ((u >> 16) & np.uint32(1))) >> 16).astype(np.uint16)


# (name, ab type, c type, m, n, k, layout, extra, band): measured / predicted device time must lie inside band.
CASES = [
    ("C2 bf16 4096^3", L.BF16, L.BF16, 4096, 4096, 4096, "nn", {}, (0.85, 1.2)),
    ("C4 int8 W8A8 4096^3", L.I8, L.BF16, 4096, 4096, 4096, "nn", {"scales": True}, (0.85, 1.3)),
    ("C3 forward + bias + GELU", L.BF16, L.BF16, 8192, 11008, 4096, "nn", {"bias": True, "gelu": True}, (0.85, 1.35)),
    ("C3 dX (NT)", L.BF16, L.BF16, 8192, 4096, 11008, "nt", {}, (0.85, 1.3)),
    # 688 tiles: 2.69 rounds, the last a partial one the model charges as a full round at the full-load clock.
    ("C3 dW (TN)", L.BF16, L.BF16, 4096, 11008, 8192, "tn", {}, (0.75, 1.3)),
    ("2048^3 (64 tiles)", L.BF16, L.BF16, 2048, 2048, 2048, "nn", {}, (0.55, 1.05)),
    ("520 x 4096 x 4096 (48 tiles)", L.BF16, L.BF16, 520, 4096, 4096, "nn", {}, (0.55, 1.05)),
    ("C5 decode m=1", L.BF16, L.BF16, 1, 14336, 4096, "nt", {}, (0.8, 1.2)),
    ("C5 decode m=4", L.BF16, L.BF16, 4, 14336, 4096, "nt", {}, (0.8, 1.2)),
    ("C5 decode m=16", L.BF16, L.BF16, 16, 14336, 4096, "nt", {}, (0.8, 1.2)),
]


def test_the_prediction_tracks_the_measured_launch():
    rng = np.random.default_rng(77)
    stream = hip.Stream()
    rows, outside = [], []
    for name, ab, out, m, n, k, layout, extra, (lo, hi) in CASES:
        ta, tb = layout[0] == "t", layout[1] == "t"
        a = hip.Buffer.of(operand(ab, (k, m) if ta else (m, k), rng))
        copies = 4 if m <= 16 else 1  # 4 x 117 MB of b for the decode shapes
        bs = [hip.Buffer.of(operand(ab, (n, k) if tb else (k, n), rng)) for _ in range(copies)]
        c = hip.Buffer(m * n * 2)
        keep = [a, *bs, c]
        kw = {}
        if extra.get("scales"):
            rs = hip.Buffer.of(rng.uniform(1e-3, 1e-2, m).astype(np.float32))
            cs = hip.Buffer.of(rng.uniform(1e-3, 1e-2, n).astype(np.float32))
            keep += [rs, cs]
            kw.update(row_scale=rs.ptr, col_scale=cs.ptr)
        if extra.get("bias"):
            bias = hip.Buffer.of(operand(L.BF16, (n,), rng))
            keep.append(bias)
            kw.update(bias=bias.ptr, bias_type=L.BF16)
        if extra.get("gelu"):
            kw.update(act=L.ACT_GELU)
        descs = [L.desc(ab, out, m, n, k, a.ptr, b.ptr, c.ptr, trans_a=ta, trans_b=tb, **kw) for b in bs]
        d = descs[0]
        predicted = (perf.predict(d)["ns"] - perf.card()["device"]["launch_ns"]) / 1e3
        measured = burst_us(descs, stream)
        ratio = measured / predicted
        rows.append((name, L.select(d)["name"], predicted, measured, ratio))
        say(f"{name}: predicted {predicted:.1f} us, measured {measured:.1f} us (x {ratio:.2f}) on {rows[-1][1]}")
        if not lo <= ratio <= hi:
            outside.append((name, ratio, (lo, hi)))
        for x in keep:
            x.close()
    stream.close()
    assert not outside, outside
