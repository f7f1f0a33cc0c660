"""Writes the golden fixtures in this directory from the compiled reference.

Run in the build container (where /root/reference exists and oracle/_ref is
built): ``python tests/golden/make_goldens.py``.  Each fixture records the
reference's own CPU forward (DecisionModel::encode / ::forward via
oracle/_ref/libsjref.so) on a synthetic checkpoint that snapjudge_amd.synth
regenerates bit-identically from the stored seed, so only inputs and outputs
are committed, never weights.

  cfg1_forward.npz   BASELINE config 1 (tiny fp32): 8 forward rows (4 examples x
                     {choice K=4, noul K=2}), hidden/logits/act
  cfg2_b1s128.npz    BASELINE config 2 (22 layers, D=768, bf16 weights), B=1,
                     S=128: encoder hidden states
"""
import os
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import RefModel  # noqa: E402
from snapjudge_amd import synth  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))


def cfg1():
    seed = 11
    p = dict(synth.PRESETS["cfg1"])
    store = p["store"]
    rl, enc, w = synth.make_model(**p, seed=seed)
    ids4, mask4, lens4 = synth.make_batch(4, 32, 8, 32, enc["vocab_size"], seed=3)
    # each example carries a choice question (K=4) and a noul question (K=2):
    # two forward rows with identical ids, one qtype each (src/model.cpp:410-416)
    ids = np.repeat(ids4, 2, axis=0)
    mask = np.repeat(mask4, 2, axis=0)
    lens = np.repeat(lens4, 2)
    mp, mm, qt = synth.make_markers(lens, 4, [(0, 4), (2, 2)] * 4, seed=3)
    with tempfile.TemporaryDirectory() as d:
        synth.write_checkpoint(d, rl, enc, w, store=store)
        ref = RefModel(d)
        hidden = ref.encode(ids, mask)
        logits, act = ref.forward(ids, mask, mp, mm, qt)
    np.savez(os.path.join(HERE, "cfg1_forward.npz"), seed=seed, ids=ids, mask=mask,
             marker_pos=mp, marker_mask=mm, qtype=qt, hidden=hidden, logits=logits, act=act)


def cfg2():
    seed = 0
    p = dict(synth.PRESETS["cfg2"])
    rl, enc, w = synth.make_model(**p, seed=seed)
    rng = np.random.default_rng(7)
    ids = rng.integers(0, enc["vocab_size"], size=(1, 128)).astype(np.int64)
    mask = np.ones((1, 128), np.int64)
    with tempfile.TemporaryDirectory() as d:
        synth.write_checkpoint(d, rl, enc, w, store=p["store"])
        del w
        ref = RefModel(d)
        t0 = time.time()
        hidden = ref.encode(ids, mask)
        print(f"cfg2 reference encode: {time.time() - t0:.1f} s")
    np.savez(os.path.join(HERE, "cfg2_b1s128.npz"), seed=seed, ids=ids, mask=mask, hidden=hidden)


if __name__ == "__main__":
    which = sys.argv[1:] or ["cfg1", "cfg2"]
    for name in which:
        globals()[name]()
        print("wrote", name)
