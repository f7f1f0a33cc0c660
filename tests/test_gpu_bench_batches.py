"""GPU parity on the bench's own batches of BASELINE configs 3 and 5, at full
depth, against fixtures from the compiled reference (tests/golden/make_goldens.py).

Config 3: the 22-layer/768 encoder (weights seed 0) on batch 64 x seq 512,
lengths U[64, 512] seed 1, in the bf16 mode (as bench.py runs it, graphs on) and
the fp32 mode.  The fixture holds DecisionModel::encode of the shortest, the
median and the longest row, each run alone (rows are independent,
src/tensor.cpp:179-185), at sampled positions.

Config 5: the 28-layer/1024 encoder with per-row e4m3 weights (weights seed 0)
on batch 32 x seq 1024, lengths U[256, 1024] seed 1, with the bench's 8 typed
questions per sequence (seed 3).  The reference ran on the dequantized twin of
the fp8 weights (decode(code) * scale, what an fp8 checkpoint stands for): its
encode of the shortest and the longest row alone, and its forward on each of
their 16 question rows.  The GPU runs the whole batch in SJH_PREC_FP8W, encode
and forward_shared (the bench's decision step).

Tolerances (north_star): hidden states max-abs 2e-2 in the bf16 and fp8-weight
modes (bf16 activations), 1e-4 in the fp32 mode; calibrated probabilities 5e-3;
argmax labels exact."""
import os

import numpy as np
import pytest

import snapjudge_amd as sj
from snapjudge_amd import synth

pytestmark = pytest.mark.gpu

BF16, FP32 = sj.SJH_PREC_BF16, sj.SJH_PREC_FP32
TOL = {BF16: 2e-2, FP32: 1e-4, sj.SJH_PREC_FP8W: 2e-2}


@pytest.fixture(scope="module")
def cfg3(golden_dir):
    g = np.load(os.path.join(golden_dir, "cfg3_b64s512.npz"))
    rl, enc, w = synth.make_model(**synth.PRESETS["cfg3"], seed=int(g["seed"]))
    cfg = synth.flat_cfg(rl, enc)
    ids, mask, lens = synth.make_batch(64, 512, 64, 512, cfg["vocab_size"], seed=int(g["batch_seed"]))
    assert np.array_equal(lens, g["lens"])  # the bench's batch
    return cfg, w, g, ids, mask, lens


@pytest.mark.parametrize("prec", [BF16, FP32])
def test_cfg3_bench_batch_full_depth_vs_reference_fixture(cfg3, prec):
    cfg, w, g, ids, mask, lens = cfg3
    print(f"cfg3 22 layers prec={prec} T={int(lens.sum())}", flush=True)
    m = sj.Model(w, cfg, precision=prec, use_graphs=True)
    h = m.encode(ids, mask)
    for i, b in enumerate(g["rows"]):
        pos = g[f"pos_{i}"]
        err = float(np.abs(h[b, pos] - g[f"hidden_{i}"]).max())
        print(f"cfg3 prec={prec} row {int(b)} (n={int(lens[b])}, {len(pos)} positions) max|d|={err:.3g}",
              flush=True)
        assert err <= TOL[prec]
    assert np.all(h[~mask.astype(bool)] == 0)
    if prec == BF16:
        # the batch reversed: the outputs are permuted and nothing else
        hr = m.encode(ids[::-1].copy(), mask[::-1].copy())
        assert np.array_equal(hr[::-1], h)
    m.close()


@pytest.fixture(scope="module")
def cfg5(golden_dir):
    g = np.load(os.path.join(golden_dir, "cfg5_b32s1024.npz"))
    rl, enc, w = synth.make_model(**synth.PRESETS["cfg5"], seed=int(g["seed"]))
    cfg = synth.flat_cfg(rl, enc)
    ids, mask, lens = synth.make_batch(32, 1024, 256, 1024, cfg["vocab_size"], seed=int(g["batch_seed"]))
    assert np.array_equal(lens, g["lens"])  # the bench's batch
    m = sj.Model(w, cfg, precision=sj.SJH_PREC_FP8W, use_graphs=True)
    del w
    yield cfg, m, g, ids, mask, lens
    m.close()


def test_cfg5_bench_batch_encode_vs_reference_fixture(cfg5):
    cfg, m, g, ids, mask, lens = cfg5
    print(f"cfg5 28 layers fp8w T={int(lens.sum())}", flush=True)
    h = m.encode(ids, mask)
    for i, b in enumerate(g["rows"]):
        pos = g[f"pos_{i}"]
        err = float(np.abs(h[b, pos] - g[f"hidden_{i}"]).max())
        print(f"cfg5 fp8w row {int(b)} (n={int(lens[b])}, {len(pos)} positions) max|d|={err:.3g}",
              flush=True)
        assert err <= TOL[sj.SJH_PREC_FP8W]
    assert np.all(h[~mask.astype(bool)] == 0)
    hr = m.encode(ids[::-1].copy(), mask[::-1].copy())
    assert np.array_equal(hr[::-1], h)


def test_cfg5_bench_decision_step_vs_reference_fixture(cfg5, orc):
    # the bench's decision step: forward_shared over the 32 sequences x 8
    # questions (256 rows); the fixture holds the reference's forward of the
    # question rows of the shortest and the longest sequence
    cfg, m, g, ids, mask, lens = cfg5
    row_seq, mp, mm, qt = synth.make_questions(lens, int(g["n_q"]), seed=int(g["question_seed"]))
    lg, act = m.forward_shared(ids, mask, row_seq, mp, mm, qt)
    assert np.all(lg[mm == 0] == np.float32(-1e4))
    perr = aerr = 0.0
    for k, r in enumerate(g["q_rows"]):
        nk = int(mm[r].sum())
        assert np.all(g["logits"][k, nk:] == np.float32(-1e4))
        pg = orc.calibrated_probs(lg[r, :nk], 1.0)
        pr = orc.calibrated_probs(g["logits"][k, :nk], 1.0)
        perr = max(perr, float(np.abs(pg - pr).max()))
        aerr = max(aerr, float(np.abs(act[r] - g["act"][k]).max()))
        assert int(np.argmax(pg)) == int(np.argmax(pr)), f"row {int(r)} label"
        assert int(np.argmax(act[r])) == int(np.argmax(g["act"][k]))
    print(f"cfg5 decision step: {len(g['q_rows'])} rows vs reference, probs max|d| {perr:.3g}, "
          f"act max|d| {aerr:.3g}", flush=True)
    assert perr <= 5e-3 and aerr <= 5e-3
