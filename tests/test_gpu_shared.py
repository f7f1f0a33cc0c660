"""sjh_model_forward_shared: B decision rows over U shared token sequences.

The result is defined as sjh_model_forward on the expanded batch
ids[row_seq] (src/model.cpp:309-536: the encoder reads the tokens only, the
head reads the hidden states plus the row's qtype).  Checked against the
oracle's forward on that expanded batch (probabilities and act 5e-3 at the
three calibration temperatures, labels exact, masked logits -1e4 exactly) and
against this library's own forward on the expanded batch at config 5's widths,
where the oracle is too slow to run."""
import numpy as np
import pytest

import snapjudge_amd as sj
from snapjudge_amd import synth

pytestmark = pytest.mark.gpu

FP32, BF16 = sj.SJH_PREC_FP32, sj.SJH_PREC_BF16


def probs_err(orc, lg, lr, mm):
    e = 0.0
    for b in range(len(lg)):
        k = int(mm[b].sum())
        for t in (0.5, 1.0, 5.0):
            e = max(e, float(np.abs(orc.calibrated_probs(lg[b, :k], t) -
                                    orc.calibrated_probs(lr[b, :k], t)).max()))
    return e


def labels(orc, lg, mm):
    return [int(np.argmax(orc.calibrated_probs(lg[b, :int(mm[b].sum())], 1.0)))
            for b in range(len(lg))]


def shared_batch(U, L, lo, hi, vocab, row_seq, K, seed):
    ids, mask, lens = synth.make_batch(U, L, lo, hi, vocab, seed=seed)
    rs = np.asarray(row_seq, dtype=np.int32)
    rng = np.random.default_rng(seed + 7)
    kinds = [(int(rng.integers(0, 3)), int(rng.integers(1, K + 1))) for _ in rs]
    mp, mm, qt = synth.make_markers(lens[rs], K, kinds, seed=seed)
    return ids, mask, rs, mp, mm, qt


@pytest.mark.parametrize("pad_rows", [False, True])
@pytest.mark.parametrize("prec", [FP32, BF16])
def test_shared_matches_oracle_on_expanded_batch(orc, prec, pad_rows):
    # 5 sequences, 13 rows: repeats, a sequence no row uses (3), rows out of
    # sequence order, a one-token sequence
    rl, enc, w = synth.make_model(hidden_size=128, num_hidden_layers=2, num_attention_heads=2,
                                  intermediate_size=192, vocab_size=800, store="BF16",
                                  max_position_embeddings=256, head_layers=2, n_act=3, seed=41)
    cfg = synth.flat_cfg(rl, enc)
    row_seq = [0, 0, 2, 4, 1, 2, 2, 0, 4, 4, 1, 0, 2]
    ids, mask, rs, mp, mm, qt = shared_batch(5, 96, 1, 96, cfg["vocab_size"], row_seq, 6, seed=42)
    mask[4, 1:] = 0
    ids[4, 1:] = 0
    lens = mask.sum(1)
    mp[rs == 4] = 0  # the one-token sequence: its markers all sit on position 0
    print(f"shared prec={prec} pad_rows={pad_rows} lens={lens.tolist()}", flush=True)
    om = orc.model(w, cfg)
    rlg, ract = om.forward(ids[rs], mask[rs], mp, mm, qt)
    m = sj.Model(w, cfg, precision=prec, pad_rows=pad_rows)
    lg, act = m.forward_shared(ids, mask, rs, mp, mm, qt)
    elg, eact = m.forward(ids[rs], mask[rs], mp, mm, qt)
    perr = probs_err(orc, lg, rlg, mm)
    aerr = float(np.abs(act - ract).max())
    print(f"  vs oracle: probs {perr:.3g} act {aerr:.3g}; vs forward: "
          f"{float(np.abs(act - eact).max()):.3g}", flush=True)
    assert perr <= 5e-3 and aerr <= 5e-3
    assert labels(orc, lg, mm) == labels(orc, rlg, mm)
    assert np.all(lg[mm == 0] == np.float32(-1e4))
    assert probs_err(orc, lg, elg, mm) <= 5e-3 and float(np.abs(act - eact).max()) <= 5e-3
    # a second call with fewer rows and sequences reuses the buffers
    lg2, act2 = m.forward_shared(ids[:3], mask[:3], rs[:4] % 3, mp[:4], mm[:4], qt[:4])
    rlg2, ract2 = om.forward(ids[:3][rs[:4] % 3], mask[:3][rs[:4] % 3], mp[:4], mm[:4], qt[:4])
    assert probs_err(orc, lg2, rlg2, mm[:4]) <= 5e-3
    assert float(np.abs(act2 - ract2).max()) <= 5e-3
    m.close()


def test_shared_sj_model(orc, tmp_path):
    cfg, w = synth.make_sj_model(hidden_size=64, num_layers=2, num_heads=4, vocab_size=500,
                                 intermediate_size=160, max_positions=64, head_layers=1,
                                 head_intermediate=96, store="BF16", seed=51)
    synth.write_sj_checkpoint(str(tmp_path), cfg, w, store="BF16")
    row_seq = [1, 0, 1, 2, 2, 1]
    ids, mask, rs, mp, mm, qt = shared_batch(3, 64, 4, 64, cfg["vocab_size"], row_seq, 5, seed=52)
    om = orc.sj_model(w, cfg)
    rlg, ract = om.forward(ids[rs], mask[rs], mp, mm, qt)
    m = sj.Model.load(str(tmp_path), precision=FP32)
    lg, act = m.forward_shared(ids, mask, rs, mp, mm, qt)
    assert probs_err(orc, lg, rlg, mm) <= 5e-3
    assert float(np.abs(act - ract).max()) <= 5e-3
    assert np.all(lg[mm == 0] == np.float32(-1e4))
    m.close()


@pytest.mark.parametrize("prec", [BF16, sj.SJH_PREC_FP8W])
def test_shared_cfg5_widths_match_forward(prec):
    # config 5's widths (D 1024, 16 heads, F 2624, a 2-layer head) at 2
    # encoder layers: 32 sequences x 8 questions, against forward on the
    # 256-row expanded batch.  Both take the persistent GEMMs (T >= 4096) and
    # every kernel's result for a row is independent of the other rows, so
    # the two agree bit for bit.  (The reference's forward on the bench's
    # config-5 decision step is checked in tests/test_gpu_bench_batches.py.)
    p = dict(synth.PRESETS["cfg5"])
    p.update(num_hidden_layers=2, max_position_embeddings=1024)
    rl, enc, w = synth.make_model(**p, head_layers=2, n_act=3, seed=61)
    cfg = synth.flat_cfg(rl, enc)
    row_seq = np.repeat(np.arange(32), 8)
    ids, mask, rs, mp, mm, qt = shared_batch(32, 512, 64, 512, cfg["vocab_size"], row_seq, 16,
                                             seed=62)
    print(f"cfg5 widths prec={prec} rows={len(rs)}", flush=True)
    m = sj.Model(w, cfg, precision=prec)
    lg, act = m.forward_shared(ids, mask, rs, mp, mm, qt)
    elg, eact = m.forward(ids[rs], mask[rs], mp, mm, qt)
    live = mm.astype(bool)
    derr = float(np.abs(lg[live] - elg[live]).max())
    aerr = float(np.abs(act - eact).max())
    print(f"  logits {derr:.3g} act {aerr:.3g}", flush=True)
    assert np.all(lg[~live] == np.float32(-1e4))
    assert derr == 0.0 and aerr == 0.0
    m.close()


def test_shared_rejects_bad_rows():
    rl, enc, w = synth.make_model(**synth.PRESETS["cfg1"], head_layers=1, n_act=3, seed=71)
    cfg = synth.flat_cfg(rl, enc)
    ids, mask, rs, mp, mm, qt = shared_batch(2, 32, 4, 32, cfg["vocab_size"], [0, 1], 3, seed=72)
    m = sj.Model(w, cfg, precision=FP32)
    with pytest.raises(sj.SjhError, match="row_seq"):
        m.forward_shared(ids, mask, np.array([0, 2], np.int32), mp, mm, qt)
    with pytest.raises(sj.SjhError, match="qtype"):
        m.forward_shared(ids, mask, rs, mp, mm, np.array([0, 3]))
    m.close()
