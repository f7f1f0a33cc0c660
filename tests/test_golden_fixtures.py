"""The oracle reproduces the fixtures recorded from the compiled reference
(tests/golden/make_goldens.py) bit for bit, so the oracle stays pinned where
the reference itself is absent (the GPU box)."""
import os

import numpy as np

from snapjudge_amd import synth


def test_cfg1_fixture(orc, golden_dir):
    g = np.load(os.path.join(golden_dir, "cfg1_forward.npz"))
    rl, enc, w = synth.make_model(**synth.PRESETS["cfg1"], seed=int(g["seed"]))
    om = orc.model(w, synth.flat_cfg(rl, enc))
    assert np.array_equal(om.encode(g["ids"], g["mask"]), g["hidden"])
    lg, act = om.forward(g["ids"], g["mask"], g["marker_pos"], g["marker_mask"], g["qtype"])
    assert np.array_equal(lg, g["logits"]) and np.array_equal(act, g["act"])


def test_cfg2_fixture(orc, golden_dir):
    g = np.load(os.path.join(golden_dir, "cfg2_b1s128.npz"))
    rl, enc, w = synth.make_model(**synth.PRESETS["cfg2"], seed=int(g["seed"]))
    om = orc.model(w, synth.flat_cfg(rl, enc))
    assert np.array_equal(om.encode(g["ids"], g["mask"]), g["hidden"])
