"""SjModel (snapjudge's own BERT-style model, src/sj_model.cpp:206-368) on the
GPU against the oracle's restatement, which tests/test_oracle_vs_ref.py pins
bit for bit to the compiled reference.  Tolerances as for the DecisionModel:
hidden states max-abs 1e-4 (fp32) and 2e-2 (bf16) on valid positions,
probabilities and the act head's {top1, 1 - top1} 5e-3, masked logits -1e4
exactly."""
import numpy as np
import pytest

import snapjudge_amd as sj
from snapjudge_amd import synth

pytestmark = pytest.mark.gpu

FP32, BF16 = sj.SJH_PREC_FP32, sj.SJH_PREC_BF16
TOL = {FP32: 1e-4, BF16: 2e-2}


def check(orc, tmp_path, cfg, w, store, prec, B, L, lo, hi, kinds, K, seed, pad_rows=False):
    synth.write_sj_checkpoint(str(tmp_path), cfg, w, store=store)
    om = orc.sj_model(w, cfg)
    ids, mask, lens = synth.make_batch(B, L, lo, hi, cfg["vocab_size"], seed=seed)
    mp, mm, qt = synth.make_markers(lens, K, kinds, seed=seed)
    m = sj.Model.load(str(tmp_path), precision=prec, pad_rows=pad_rows)
    assert m.n_act == 2
    h = m.encode(ids, mask)
    ref = om.encode(ids, mask)
    sel = np.ones_like(mask, bool) if pad_rows else mask.astype(bool)
    err = float(np.abs(h[sel] - ref[sel]).max())
    lg, act = m.forward(ids, mask, mp, mm, qt)
    rlg, ract = om.forward(ids, mask, mp, mm, qt)
    perr = 0.0
    for b in range(B):
        k = int(mm[b].sum())
        for t in (0.5, 1.0, 5.0):
            perr = max(perr, float(np.abs(orc.calibrated_probs(lg[b, :k], t) -
                                          orc.calibrated_probs(rlg[b, :k], t)).max()))
    aerr = float(np.abs(act - ract).max())
    print(f"D={cfg['hidden_size']} prec={prec} hidden {err:.3g} probs {perr:.3g} act {aerr:.3g}",
          flush=True)
    assert err <= TOL[prec]
    assert perr <= 5e-3 and aerr <= 5e-3
    assert np.all(lg[mm == 0] == np.float32(-1e4))
    assert np.allclose(act.sum(1), 1.0, atol=1e-6)
    m.close()


@pytest.mark.parametrize("prec", [FP32, BF16])
def test_small_sj_model(orc, tmp_path, prec):
    # rows longer than max_positions (positions clamp to the last row), two
    # head layers, every bias random
    cfg, w = synth.make_sj_model(hidden_size=64, num_layers=2, num_heads=4, vocab_size=500,
                                 intermediate_size=160, max_positions=48, head_layers=2,
                                 head_intermediate=96, store="BF16", seed=101)
    check(orc, tmp_path, cfg, w, "BF16", prec, 5, 64, 5, 64,
          [(0, 4), (1, 4), (2, 2), (0, 1), (1, 3)], 4, seed=102)


@pytest.mark.parametrize("prec", [FP32, BF16])
def test_sj_model_768_wide(orc, tmp_path, prec):
    # 12 heads x 64 on the MFMA paths (tiled GEMMs, split-K residuals for the
    # short row, the flash attention kernel)
    cfg, w = synth.make_sj_model(hidden_size=768, num_layers=2, num_heads=12, vocab_size=3000,
                                 max_positions=512, head_layers=1, store="BF16", seed=103)
    check(orc, tmp_path, cfg, w, "BF16", prec, 3, 300, 100, 300, [(0, 5), (1, 5), (2, 2)], 5,
          seed=104)


@pytest.mark.parametrize("prec", [FP32, BF16])
def test_sj_model_768_short_batch(orc, tmp_path, prec):
    # at most 256 tokens: in bf16 the attention kernel folds the output
    # projection in (the BERT family's queries are not pre-scaled, so its
    # softmax scales the logits itself) and the layer norm adds the heads'
    # partials with Wo's bias
    cfg, w = synth.make_sj_model(hidden_size=768, num_layers=2, num_heads=12, vocab_size=3000,
                                 max_positions=512, head_layers=1, store="BF16", seed=107)
    check(orc, tmp_path, cfg, w, "BF16", prec, 2, 120, 60, 120, [(0, 5), (1, 4)], 5, seed=108)


def test_sj_model_padded_rows(orc, tmp_path):
    cfg, w = synth.make_sj_model(hidden_size=64, num_layers=1, num_heads=2, vocab_size=200,
                                 max_positions=40, store="F32", seed=105)
    check(orc, tmp_path, cfg, w, "F32", FP32, 3, 30, 5, 30, [(0, 3), (1, 3), (2, 2)], 3,
          seed=106, pad_rows=True)
