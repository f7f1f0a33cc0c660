"""GPU parity of the reference-API hook: the reference's own DecisionModel
(loaded by the compiled reference, oracle/_ref) is handed to
snapjudge::FastSnapjudge (libsnapjudge_fast_hip.so) exactly as
Agent::accelerate does (src/agent.cpp:363-386); its forward/encode must match
the reference's DecisionModel::forward/encode on the same model object
(tolerances of BASELINE.json's north_star: hidden 1e-4 fp32 / 2e-2 bf16 on
valid positions, calibrated probabilities 5e-3, argmax labels equal)."""
import os

import numpy as np
import pytest

from hook_util import HOOK_LIB, Fast
from snapjudge_amd import synth

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not os.path.exists(HOOK_LIB), reason="hook not built")]

TOL = {0: 1e-4, 1: 2e-2}


def _ref():
    from oracle import RefModel

    if not RefModel.available():
        pytest.skip("compiled reference (oracle/_ref) not built")
    return RefModel


def _cases(golden_dir, tmp_path):
    rl, enc, w = synth.read_checkpoint(os.path.join(golden_dir, "tiny-ckpt"))
    yield "tiny-ckpt", os.path.join(golden_dir, "tiny-ckpt"), synth.flat_cfg(rl, enc)
    rl, enc, w = synth.make_model(hidden_size=128, num_hidden_layers=3, num_attention_heads=2,
                                  intermediate_size=192, vocab_size=1000, store="BF16",
                                  max_position_embeddings=256, head_layers=2, n_act=3,
                                  layer_types=["full_attention", "sliding_attention",
                                               "full_attention"],
                                  local_attention=16, theta_sliding=7000.0, lora_r=8, seed=5)
    d = os.path.join(str(tmp_path), "sliding-lora")
    synth.write_checkpoint(d, rl, enc, w, store="BF16")
    yield "sliding-lora", d, synth.flat_cfg(rl, enc)


@pytest.mark.parametrize("prec", [0, 1])
def test_hook_matches_reference_forward_and_encode(orc, golden_dir, tmp_path, prec):
    RefModel = _ref()
    for name, ckpt, cfg in _cases(golden_dir, tmp_path):
        print(f"hook {name} precision={prec}", flush=True)
        ref = RefModel(ckpt)
        B, L = 6, min(48, cfg["max_position_embeddings"])
        ids, mask, lens = synth.make_batch(B, L, 2, L, cfg["vocab_size"], seed=9)
        kinds = [(0, 4), (2, 2), (1, 5), (0, 3), (2, 2), (1, 5)]
        mp, mm, qt = synth.make_markers(lens, 5, kinds, seed=9)
        f = Fast(ref.h, max_len=L, graphs=True, precision=prec)
        try:
            lg, act = f.forward(ids, mask, mp, mm, qt, ref.n_act)
            h = f.encode(ids, mask, ref.D)
        finally:
            f.close()
        rlg, ract = ref.forward(ids, mask, mp, mm, qt)
        rh = ref.encode(ids, mask)
        valid = mask.astype(bool)
        assert float(np.abs(h[valid] - rh[valid]).max()) <= TOL[prec], name
        assert np.all(lg[mm == 0] == -1e4)
        for b in range(B):
            k = int(mm[b].sum())
            p, rp = orc.calibrated_probs(lg[b, :k], 1.0), orc.calibrated_probs(rlg[b, :k], 1.0)
            assert float(np.abs(p - rp).max()) <= 5e-3, name
            assert int(np.argmax(p)) == int(np.argmax(rp)), name
        assert float(np.abs(act - ract).max()) <= 5e-3, name


def test_hook_pad_rows_reproduces_padded_positions(golden_dir):
    RefModel = _ref()
    ckpt = os.path.join(golden_dir, "tiny-ckpt")
    ref = RefModel(ckpt)
    rl, enc, _ = synth.read_checkpoint(ckpt)
    cfg = synth.flat_cfg(rl, enc)
    ids, mask, _ = synth.make_batch(3, 30, 5, 30, cfg["vocab_size"], seed=2)
    f = Fast(ref.h, max_len=30, precision=0, pad_rows=True)
    try:
        h = f.encode(ids, mask, ref.D)
    finally:
        f.close()
    assert float(np.abs(h - ref.encode(ids, mask)).max()) <= 1e-4
