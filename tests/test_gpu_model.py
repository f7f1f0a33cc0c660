"""GPU parity of the whole DecisionModel forward (sjh_model_* C ABI).

Tolerances are the ones BASELINE.json's north_star states: hidden states
max-abs 1e-4 in the fp32 path and 2e-2 in the bf16 path (valid positions),
calibrated probabilities 5e-3, argmax labels bit-exact.  References: the
oracle run live on the same inputs (small cases), the fixtures recorded from
the compiled reference (tests/golden/*.npz), and, at full BASELINE shapes,
row-sampled oracle runs plus properties that hold at any size (a row's result
does not depend on the rest of the batch or on its padding)."""
import os

import numpy as np
import pytest

import snapjudge_amd as sj
from snapjudge_amd import synth

pytestmark = pytest.mark.gpu

FP32, BF16 = sj.SJH_PREC_FP32, sj.SJH_PREC_BF16
TOL = {FP32: 1e-4, BF16: 2e-2}


def valid_err(h, ref, mask):
    m = mask.astype(bool)
    return float(np.abs(h[m] - ref[m]).max())


# Calibration temperatures are clamped to [0.5, 5] (src/common.cpp:199-202);
# T = 0.5 doubles logit differences before the softmax, so the 5e-3 bound is
# checked at both ends of the range and at 1.
TEMPERATURES = (0.5, 1.0, 5.0)


def probs_err(orc, lg, lr, mm):
    e = 0.0
    for b in range(len(lg)):
        k = int(mm[b].sum())
        for t in TEMPERATURES:
            e = max(e, float(np.abs(orc.calibrated_probs(lg[b, :k], t) -
                                    orc.calibrated_probs(lr[b, :k], t)).max()))
    return e


def labels(orc, lg, mm):
    return [int(np.argmax(orc.calibrated_probs(lg[b, :int(mm[b].sum())], 1.0))) for b in range(len(lg))]


@pytest.fixture(scope="module")
def cfg1(golden_dir):
    g = np.load(os.path.join(golden_dir, "cfg1_forward.npz"))
    rl, enc, w = synth.make_model(**synth.PRESETS["cfg1"], seed=int(g["seed"]))
    return synth.flat_cfg(rl, enc), w, g


@pytest.mark.parametrize("prec", [FP32, BF16])
@pytest.mark.parametrize("graphs", [True, False])
def test_cfg1_forward_vs_reference_fixture(orc, cfg1, prec, graphs):
    cfg, w, g = cfg1
    print(f"cfg1 prec={prec} graphs={graphs}", flush=True)
    m = sj.Model(w, cfg, precision=prec, use_graphs=graphs)
    h = m.encode(g["ids"], g["mask"])
    assert valid_err(h, g["hidden"], g["mask"]) <= TOL[prec]
    assert np.all(h[~g["mask"].astype(bool)] == 0)  # packed mode leaves padding at 0
    lg, act = m.forward(g["ids"], g["mask"], g["marker_pos"], g["marker_mask"], g["qtype"])
    assert probs_err(orc, lg, g["logits"], g["marker_mask"]) <= 5e-3
    assert labels(orc, lg, g["marker_mask"]) == labels(orc, g["logits"], g["marker_mask"])
    assert np.all(lg[g["marker_mask"] == 0] == -1e4)
    assert float(np.abs(act - g["act"]).max()) <= 5e-3
    # repeated calls replay the same work: identical results
    lg2, act2 = m.forward(g["ids"], g["mask"], g["marker_pos"], g["marker_mask"], g["qtype"])
    assert np.array_equal(lg, lg2) and np.array_equal(act, act2)
    m.close()


@pytest.mark.parametrize("prec", [FP32, BF16])
def test_pad_rows_mode_matches_reference_at_every_position(orc, cfg1, prec):
    cfg, w, g = cfg1
    m = sj.Model(w, cfg, precision=prec, pad_rows=True)
    h = m.encode(g["ids"], g["mask"])
    # the reference computes padded query rows too; pad_rows reproduces them
    assert float(np.abs(h - g["hidden"]).max()) <= TOL[prec]
    m.close()


@pytest.mark.parametrize("prec", [FP32, BF16])
def test_tiny_checkpoint_sliding_window(orc, golden_dir, prec):
    rl, enc, w = synth.read_checkpoint(os.path.join(golden_dir, "tiny-ckpt"))
    cfg = synth.flat_cfg(rl, enc)
    ids, mask, lens = synth.make_batch(5, 40, 1, 40, cfg["vocab_size"], seed=4)
    mp, mm, qt = synth.make_markers(lens, 3, [(0, 3), (2, 2), (1, 3), (0, 2), (2, 2)], seed=4)
    om = orc.model(w, cfg)
    ref_h = om.encode(ids, mask)
    ref_lg, ref_act = om.forward(ids, mask, mp, mm, qt)
    m = sj.Model(w, cfg, precision=prec)
    assert valid_err(m.encode(ids, mask), ref_h, mask) <= TOL[prec]
    lg, act = m.forward(ids, mask, mp, mm, qt)
    assert probs_err(orc, lg, ref_lg, mm) <= 5e-3
    assert float(np.abs(act - ref_act).max()) <= 5e-3
    m.close()


@pytest.mark.parametrize("prec", [FP32, BF16])
def test_head_tail_masked_markers(orc, golden_dir, prec):
    # decision-head tail on the device: a row with every marker masked (all
    # logits -1e4, uniform softmax, kf = 2), a row with one live marker, and
    # a marker position past L (clamped to L - 1) in a row without padding
    rl, enc, w = synth.read_checkpoint(os.path.join(golden_dir, "tiny-ckpt"))
    cfg = synth.flat_cfg(rl, enc)
    ids, mask, lens = synth.make_batch(4, 32, 8, 32, cfg["vocab_size"], seed=9)
    mask[3, :] = 1
    lens[3] = 32
    mp, mm, qt = synth.make_markers(lens, 4, [(0, 4), (1, 3), (2, 2), (0, 4)], seed=9)
    mm[1, :] = 0
    mm[2, :] = 0
    mm[2, 0] = 1
    mp[3, 2] = 1000
    om = orc.model(w, cfg)
    ref_lg, ref_act = om.forward(ids, mask, mp, mm, qt)
    m = sj.Model(w, cfg, precision=prec)
    lg, act = m.forward(ids, mask, mp, mm, qt)
    assert np.all(lg[mm == 0] == np.float32(-1e4))
    live = [b for b in range(len(mm)) if mm[b].sum() > 0]
    assert probs_err(orc, lg[live], ref_lg[live], mm[live]) <= 5e-3
    assert float(np.abs(act - ref_act).max()) <= 5e-3
    m.close()


@pytest.mark.parametrize("prec", [FP32, BF16])
def test_sliding_lora_model(orc, prec):
    rl, enc, w = synth.make_model(hidden_size=128, num_hidden_layers=3, num_attention_heads=2,
                                  intermediate_size=192, vocab_size=1000, store="BF16",
                                  max_position_embeddings=256, head_layers=2, n_act=3,
                                  layer_types=["full_attention", "sliding_attention",
                                               "full_attention"],
                                  local_attention=16, theta_sliding=7000.0, lora_r=8, seed=5)
    cfg = synth.flat_cfg(rl, enc)
    ids, mask, lens = synth.make_batch(6, 200, 20, 200, cfg["vocab_size"], seed=6)
    mp, mm, qt = synth.make_markers(lens, 6, [(0, 6), (1, 5), (2, 2), (0, 4), (1, 5), (2, 2)], seed=6)
    om = orc.model(w, cfg)
    m = sj.Model(w, cfg, precision=prec)
    assert valid_err(m.encode(ids, mask), om.encode(ids, mask), mask) <= TOL[prec]
    lg, act = m.forward(ids, mask, mp, mm, qt)
    ref_lg, ref_act = om.forward(ids, mask, mp, mm, qt)
    assert probs_err(orc, lg, ref_lg, mm) <= 5e-3
    assert labels(orc, lg, mm) == labels(orc, ref_lg, mm)
    m.close()


@pytest.fixture(scope="module")
def cfg2(golden_dir):
    g = np.load(os.path.join(golden_dir, "cfg2_b1s128.npz"))
    rl, enc, w = synth.make_model(**synth.PRESETS["cfg2"], seed=int(g["seed"]))
    return synth.flat_cfg(rl, enc), w, g


@pytest.mark.parametrize("prec", [FP32, BF16])
def test_cfg2_full_depth_vs_reference_fixture(cfg2, prec):
    cfg, w, g = cfg2
    print(f"cfg2 22 layers prec={prec}", flush=True)
    m = sj.Model(w, cfg, precision=prec)
    h = m.encode(g["ids"], g["mask"])
    err = float(np.abs(h - g["hidden"]).max())
    print(f"cfg2 prec={prec} max|d|={err:.3g}", flush=True)
    assert err <= TOL[prec]
    m.close()


def test_cfg3_shape_sampled_rows_and_batch_invariance(orc):
    # BASELINE config 3's shape (B=64, S=512, n ~ U[64, 512], D=768, F=1152,
    # V=50368) through 2 layers; rows are independent, so sampled rows are
    # checked against the oracle run on each row alone.  Results do not depend
    # on padding or on the order of the batch (bit for bit); the GEMM tile
    # shape follows the token count, so a row alone is held to the tolerance.
    rl, enc, w = synth.make_model(**dict(synth.PRESETS["cfg2"], num_hidden_layers=2), seed=21)
    cfg = synth.flat_cfg(rl, enc)
    ids, mask, lens = synth.make_batch(64, 512, 64, 512, cfg["vocab_size"], seed=22)
    m = sj.Model(w, cfg, precision=BF16)
    h = m.encode(ids, mask)
    om = orc.model(w, cfg)
    order = np.argsort(lens)
    # the two shortest, the median and the two longest rows (n near 512: four
    # 128-query blocks, eight 64-key tiles per attention workgroup)
    for b in (order[0], order[1], order[32], order[-2], order[-1]):
        n = int(lens[b])
        ref = om.encode(ids[b:b + 1, :n], mask[b:b + 1, :n])[0]
        err = float(np.abs(h[b, :n] - ref).max())
        print(f"row {b} n={n} max|d|={err:.3g}", flush=True)
        assert err <= TOL[BF16]
        # the same row alone takes the short-batch GEMM path (split-K): same
        # tolerance against the oracle; with different padding, identical bits
        alone = m.encode(ids[b:b + 1, :n + 7], mask[b:b + 1, :n + 7])[0, :n]
        assert float(np.abs(alone - ref).max()) <= TOL[BF16]
        alone2 = m.encode(ids[b:b + 1, :n + 3], mask[b:b + 1, :n + 3])[0, :n]
        assert np.array_equal(alone, alone2)
    # reversing the batch order permutes the outputs and nothing else
    hr = m.encode(ids[::-1].copy(), mask[::-1].copy())
    assert np.array_equal(hr[::-1], h)
    m.close()


@pytest.mark.skip(reason="the folded LayerNorm path is switched off: its first GPU run faulted the "
                         "device and the cause is not found yet")
@pytest.mark.parametrize("offset", ["row", "block"])
def test_folded_layer_norm_under_large_row_offsets(orc, offset):
    # On the persistent kernel's batches (T >= 4096) the LayerNorms after the
    # residual GEMMs are folded: the residual epilogue rounds x to bf16 after
    # centring it on its 256-column block's mean, and the next GEMM finishes
    # the normalisation.  A rank-1 term added to every layer's Wo2 puts a
    # large offset on each row of the residual stream: the same for every
    # column ("row", ~100x the spread; LN removes it) or a different one per
    # 256-column block ("block"; the folded correction carries it).  Sampled
    # rows against the oracle, and against the same rows run alone (T < 4096:
    # standalone LayerNorms).
    rl, enc, w = synth.make_model(**dict(synth.PRESETS["cfg2"], num_hidden_layers=2), seed=26)
    cfg = synth.flat_cfg(rl, enc)
    D, F = cfg["hidden_size"], cfg["intermediate_size"]
    rng = np.random.default_rng(27)
    u = rng.standard_normal(F).astype(np.float32)
    if offset == "row":
        v = np.full(D, 20.0, np.float32)
    else:
        v = np.repeat(np.array([25.0, -20.0, 5.0], np.float32), D // 3)
    for i in range(cfg["num_hidden_layers"]):
        k = f"encoder.layers.{i}.mlp.Wo.weight"
        w[k] = synth.bf16_round(w[k] + np.outer(v, u).astype(np.float32) / np.sqrt(F))
    ids, mask, lens = synth.make_batch(12, 480, 380, 480, cfg["vocab_size"], seed=28)
    assert int(lens.sum()) >= 4096
    m = sj.Model(w, cfg, precision=BF16)
    h = m.encode(ids, mask)
    om = orc.model(w, cfg)
    for b in (int(np.argmin(lens)), int(np.argmax(lens))):
        n = int(lens[b])
        ref = om.encode(ids[b:b + 1, :n], mask[b:b + 1, :n])[0]
        err = float(np.abs(h[b, :n] - ref).max())
        alone = m.encode(ids[b:b + 1, :n], mask[b:b + 1, :n])[0]
        aerr = float(np.abs(alone - ref).max())
        print(f"{offset} offsets: row {b} n={n} batch max|d|={err:.3g}, alone max|d|={aerr:.3g}", flush=True)
        assert err <= TOL[BF16] and aerr <= TOL[BF16]
    m.close()


@pytest.mark.parametrize("offset", ["none", "row", "block"])
def test_residual_epilogue_layer_norm(orc, offset):
    # On one round of persistent 256 x 256 tiles (T >= 4096, at most 256
    # tiles) the residual GEMMs' epilogues also write the LayerNorm that reads
    # the residual stream next: the tiles of a 256-row panel publish their
    # rows' 256-column moments and each normalises its own block once the
    # panel's other tiles have arrived.  Checked against the standalone
    # LayerNorm launches (fuse_ln=0, bit for bit) and the oracle on sampled rows, with
    # large offsets on the residual stream: the same on every column of a row
    # ("row", ~100x the spread; the LayerNorm removes it) or different per
    # 256-column block ("block").  Two runs give the same bits, and so does
    # the path of tiles that give up waiting (fuse_ln=2: one poll, the panel's
    # last tile normalises their blocks from X), and so do the standalone
    # LayerNorm launches (the same statistics in the same order).
    rl, enc, w = synth.make_model(**dict(synth.PRESETS["cfg2"], num_hidden_layers=2), seed=26)
    cfg = synth.flat_cfg(rl, enc)
    D, F = cfg["hidden_size"], cfg["intermediate_size"]
    if offset != "none":
        rng = np.random.default_rng(27)
        u = rng.standard_normal(F).astype(np.float32)
        if offset == "row":
            v = np.full(D, 20.0, np.float32)
        else:
            v = np.repeat(np.array([25.0, -20.0, 5.0], np.float32), D // 3)
        for i in range(cfg["num_hidden_layers"]):
            k = f"encoder.layers.{i}.mlp.Wo.weight"
            w[k] = synth.bf16_round(w[k] + np.outer(v, u).astype(np.float32) / np.sqrt(F))
    ids, mask, lens = synth.make_batch(12, 480, 380, 480, cfg["vocab_size"], seed=28)
    T = int(lens.sum())
    assert 4096 <= T and 3 * ((T + 255) // 256) <= 256
    print(f"rln {offset}: T={T}", flush=True)
    fused = sj.Model(w, cfg, precision=BF16)
    h1 = fused.encode(ids, mask)
    h2 = fused.encode(ids, mask)
    assert np.array_equal(h1, h2)
    fused.close()
    gave_up = sj.Model(w, cfg, precision=BF16, fuse_ln=2)
    hg = gave_up.encode(ids, mask)
    gave_up.close()
    print(f"rln {offset}: one-poll path identical: {np.array_equal(hg, h1)}", flush=True)
    assert np.array_equal(hg, h1)
    plain = sj.Model(w, cfg, precision=BF16, fuse_ln=0)
    hp = plain.encode(ids, mask)
    plain.close()
    # the standalone LayerNorm computes the same statistics in the same order
    print(f"rln {offset}: fused vs standalone max|d|={valid_err(h1, hp, mask):.3g}", flush=True)
    assert np.array_equal(h1, hp)
    om = orc.model(w, cfg)
    for b in (int(np.argmin(lens)), int(np.argmax(lens))):
        n = int(lens[b])
        ref = om.encode(ids[b:b + 1, :n], mask[b:b + 1, :n])[0]
        err = float(np.abs(h1[b, :n] - ref).max())
        perr = float(np.abs(hp[b, :n] - ref).max())
        print(f"rln {offset}: row {b} n={n} max|d|={err:.3g} (standalone {perr:.3g})", flush=True)
        if offset == "block":
            # Per-block offsets survive the LayerNorm as block-wise offsets of
            # its output; through QKV they give large logits whose softmax
            # turns on bf16 roundings, so both bf16 paths leave the fp32
            # oracle by ~0.4 here.  The fused path is held to the standalone
            # path's accuracy.
            assert err <= 1.25 * perr + 1e-3
        else:
            assert err <= TOL[BF16] and perr <= TOL[BF16]


@pytest.mark.parametrize("D,H,F", [(512, 8, 768), (1024, 16, 2624)])
def test_residual_epilogue_layer_norm_widths(orc, D, H, F):
    # The residual epilogue that finishes the LayerNorm at two and four
    # 256-column blocks per row (D = 512 and 1024; config 5's widths), with
    # norm weights away from 1: bit for bit against the standalone LayerNorm
    # (fuse_ln=0) and the give-up path (fuse_ln=2), rows against the oracle.
    rl, enc, w = synth.make_model(hidden_size=D, num_hidden_layers=2, num_attention_heads=H,
                                  intermediate_size=F, vocab_size=50368, store="BF16", seed=71)
    cfg = synth.flat_cfg(rl, enc)
    rng = np.random.default_rng(72)
    for k in list(w):
        if k.endswith(("attn_norm.weight", "mlp_norm.weight")):
            w[k] = synth.bf16_round((1.0 + 0.2 * rng.standard_normal(D)).astype(np.float32))
    ids, mask, lens = synth.make_batch(12, 480, 380, 480, cfg["vocab_size"], seed=73)
    T = int(lens.sum())
    assert 4096 <= T and (D // 256) * ((T + 255) // 256) <= 256
    print(f"rln D={D}: T={T}", flush=True)
    fused = sj.Model(w, cfg, precision=BF16)
    h1 = fused.encode(ids, mask)
    fused.close()
    gave_up = sj.Model(w, cfg, precision=BF16, fuse_ln=2)
    hg = gave_up.encode(ids, mask)
    gave_up.close()
    plain = sj.Model(w, cfg, precision=BF16, fuse_ln=0)
    hp = plain.encode(ids, mask)
    plain.close()
    print(f"rln D={D}: one-poll identical {np.array_equal(hg, h1)}, standalone max|d|="
          f"{valid_err(h1, hp, mask):.3g}", flush=True)
    assert np.array_equal(hg, h1)
    assert np.array_equal(hp, h1)
    om = orc.model(w, cfg)
    for b in (int(np.argmin(lens)), int(np.argmax(lens))):
        n = int(lens[b])
        ref = om.encode(ids[b:b + 1, :n], mask[b:b + 1, :n])[0]
        err = float(np.abs(h1[b, :n] - ref).max())
        print(f"rln D={D}: row {b} n={n} max|d|={err:.3g}", flush=True)
        assert err <= TOL[BF16]


@pytest.mark.parametrize("preset,lens", [("cfg2", [128]), ("cfg2", [90, 70, 60]), ("cfg5", [128]),
                                         ("cfg5", [200, 56]), ("sliding", [200, 40])])
def test_attention_folds_output_projection_on_short_batches(orc, preset, lens):
    # Short batches (T <= 256): attention multiplies each head's output by its
    # 64-column slice of Wo (one workgroup per 128 Wo rows) and the LayerNorm
    # that reads X next adds the H partial products in head order, with no Wo
    # launch.  One and two query blocks, D 768 and 1024, two layers (the
    # second with an attention LayerNorm): repeated calls give the same bits,
    # the result stays within the bf16 tolerance of the two-launch path
    # (fuse_attn_wo=0: the sum over K runs in another order) and of the oracle
    # on every row.
    if preset == "sliding":  # a sliding-window layer (window 128) over a 200-token row
        p = dict(synth.PRESETS["cfg2"], num_hidden_layers=2, layer_types=["sliding_attention", "full_attention"],
                 local_attention=128)
    else:
        p = dict(synth.PRESETS[preset], num_hidden_layers=2)
    rl, enc, w = synth.make_model(**p, seed=81)
    cfg = synth.flat_cfg(rl, enc)
    ids, mask, lens = synth.batch_with_lens(np.array(lens), max(lens), cfg["vocab_size"], seed=82)
    print(f"attention + Wo {preset}: T={int(lens.sum())}", flush=True)
    fused = sj.Model(w, cfg, precision=BF16)
    h1 = fused.encode(ids, mask)
    h2 = fused.encode(ids, mask)
    fused.close()
    assert np.array_equal(h1, h2)
    plain = sj.Model(w, cfg, precision=BF16, fuse_attn_wo=0)
    hp = plain.encode(ids, mask)
    plain.close()
    d = valid_err(h1, hp, mask)
    print(f"attention + Wo {preset}: against the two-launch path max|d|={d:.3g}", flush=True)
    assert d <= TOL[BF16]
    om = orc.model(w, cfg)
    for b in range(len(lens)):
        n = int(lens[b])
        ref = om.encode(ids[b:b + 1, :n], mask[b:b + 1, :n])[0]
        err = float(np.abs(h1[b, :n] - ref).max())
        perr = float(np.abs(hp[b, :n] - ref).max())
        print(f"attention + Wo {preset}: row {b} n={n} max|d|={err:.3g} (two launches {perr:.3g})", flush=True)
        assert err <= TOL[BF16]


def test_more_than_256_sequences(orc):
    # More than 256 sequences: the sequence table, with the query-block prefix
    # that the attention work list is cut from, is filled on the host instead
    # of by the device kernel.  Sampled rows (one and two 128-query blocks,
    # both ends of the length order) against the oracle on each row alone;
    # reversing the batch permutes the outputs bit for bit.
    rl, enc, w = synth.make_model(**dict(synth.PRESETS["cfg2"], num_hidden_layers=2), seed=51)
    cfg = synth.flat_cfg(rl, enc)
    lens = np.random.default_rng(52).integers(1, 201, size=300)
    ids, mask, lens = synth.batch_with_lens(lens, int(lens.max()), cfg["vocab_size"], seed=53)
    m = sj.Model(w, cfg, precision=BF16)
    h = m.encode(ids, mask)
    om = orc.model(w, cfg)
    order = np.argsort(lens, kind="stable")
    for b in (order[0], order[150], order[-1], 0, 256, 299):
        n = int(lens[b])
        ref = om.encode(ids[b:b + 1, :n], mask[b:b + 1, :n])[0]
        err = float(np.abs(h[b, :n] - ref).max())
        print(f"B=300 row {b} n={n} max|d|={err:.3g}", flush=True)
        assert err <= TOL[BF16]
    hr = m.encode(ids[::-1].copy(), mask[::-1].copy())
    assert np.array_equal(hr[::-1], h)
    assert np.all(h[~mask.astype(bool)] == 0)
    m.close()


def test_attention_key_split_tail(orc):
    # Lengths 8000, 6000, 2100, 2100: the two shortest rows hold 34 of the
    # batch's 144 query blocks (at most a quarter) and at least 2048 keys
    # each, so their attention items run as two key halves whose partials a
    # merge kernel combines (the tied rows both split: the split never
    # depends on the batch order).  Each split row against the oracle on the
    # row alone; alone it runs unsplit (a batch of one), and the rounding of
    # the two-half sum shows in the bits.  Reversing the batch permutes the
    # outputs bit for bit.
    rl, enc, w = synth.make_model(**dict(synth.PRESETS["cfg4"], num_hidden_layers=2), seed=61)
    cfg = synth.flat_cfg(rl, enc)
    ids, mask, lens = synth.batch_with_lens(np.array([2100, 8000, 2100, 6000]), 8000, cfg["vocab_size"], seed=62)
    m = sj.Model(w, cfg, precision=BF16)
    h = m.encode(ids, mask)
    om = orc.model(w, cfg)
    for b in (0, 2):
        ref = om.encode(ids[b:b + 1, :2100], mask[b:b + 1, :2100])[0]
        err = float(np.abs(h[b, :2100] - ref).max())
        alone = m.encode(ids[b:b + 1, :2100], mask[b:b + 1, :2100])[0]
        print(f"split row {b} max|d|={err:.3g} alone {float(np.abs(alone - ref).max()):.3g}", flush=True)
        assert err <= TOL[BF16]
        assert not np.array_equal(alone, h[b, :2100])
    hr = m.encode(ids[::-1].copy(), mask[::-1].copy())
    assert np.array_equal(hr[::-1], h)
    assert np.all(h[~mask.astype(bool)] == 0)
    # 8000, 2100, 2100, 2100: the three tied rows hold 51 of 114 blocks
    # (more than a quarter) and no length change splits them off, so nothing
    # splits and each 2100 row equals its run alone bit for bit (the GEMMs
    # give the same bits for a row at any tile shape)
    ids3, mask3, _ = synth.batch_with_lens(np.array([8000, 2100, 2100, 2100]), 8000, cfg["vocab_size"], seed=63)
    h3 = m.encode(ids3, mask3)
    for b in (1, 3):
        assert np.array_equal(h3[b, :2100], m.encode(ids3[b:b + 1, :2100], mask3[b:b + 1, :2100])[0])
    m.close()


@pytest.fixture(scope="module")
def cfg4(golden_dir):
    g = np.load(os.path.join(golden_dir, "cfg4_b4s8192.npz"))
    rl, enc, w = synth.make_model(**synth.PRESETS["cfg4"], seed=int(g["seed"]))
    cfg = synth.flat_cfg(rl, enc)
    ids, mask, lens = synth.make_batch(4, 8192, 4096, 8192, cfg["vocab_size"], seed=int(g["batch_seed"]))
    assert np.array_equal(lens, g["lens"])  # the bench's batch
    return cfg, w, g, ids, mask, lens


@pytest.mark.parametrize("prec", [BF16, FP32])
def test_cfg4_full_depth_vs_reference_fixture(cfg4, prec):
    # BASELINE config 4 at full depth: 22 layers, batch 4 x seq 8192, lengths
    # U[4096, 8192] (T ~ 27k tokens on the persistent GEMMs, RoPE positions up
    # to 8191, attention over up to 8k keys).  The fixture holds the compiled
    # reference's encode of the shortest and the longest row, each run alone
    # (rows are independent), at sampled positions (first and last 16, every
    # 97th in between)
    cfg, w, g, ids, mask, lens = cfg4
    print(f"cfg4 22 layers prec={prec} T={int(lens.sum())}", flush=True)
    m = sj.Model(w, cfg, precision=prec)
    h = m.encode(ids, mask)
    m.close()
    for name, b in (("short", int(g["rows"][0])), ("long", int(g["rows"][1]))):
        pos = g["pos_" + name]
        err = float(np.abs(h[b, pos] - g["hidden_" + name]).max())
        print(f"cfg4 prec={prec} row {b} (n={int(lens[b])}, {len(pos)} positions) max|d|={err:.3g}",
              flush=True)
        assert err <= TOL[prec]
    assert np.all(h[~mask.astype(bool)] == 0)


def test_graph_replay_serves_a_shape_bucket():
    # Batches of different sizes, lengths and ids that fall in one shape
    # bucket replay one captured graph; each result equals the same batch run
    # launch by launch (bit for bit).  A batch in another bucket captures its
    # own graph; coming back to the first bucket replays it again.
    rl, enc, w = synth.make_model(**dict(synth.PRESETS["cfg2"], num_hidden_layers=2), seed=41)
    cfg = synth.flat_cfg(rl, enc)
    g_on = sj.Model(w, cfg, precision=BF16, use_graphs=True)
    g_off = sj.Model(w, cfg, precision=BF16, use_graphs=False)
    # one bucket: 5..8 sequences (8 table entries), 1921..2048 tokens (an
    # eighth of the octave above 1024), longest row 257..384 (three query blocks)
    V = cfg["vocab_size"]
    batches = [synth.batch_with_lens([384, 350, 330, 320, 300, 330], 384, V, seed=42),
               synth.batch_with_lens([290, 300, 270, 260, 280, 300, 280], 320, V, seed=43),
               synth.batch_with_lens([257, 250, 260, 240, 245, 255, 250, 265], 300, V, seed=44)]
    for ids, mask, lens in batches:
        assert 1920 < int(lens.sum()) <= 2048 and 256 < lens.max() <= 384
    other = synth.batch_with_lens([200, 150, 60], 200, V, seed=45)
    seen = []
    for i, (ids, mask, lens) in enumerate(batches + [other, batches[0]]):
        h = g_on.encode(ids, mask)
        want = g_off.encode(ids, mask)
        print(f"batch {i}: B={len(lens)} T={int(lens.sum())} graphs {g_on.graph_stats()}", flush=True)
        assert np.array_equal(h, want)
        seen.append(g_on.graph_stats())
    assert seen[2] == {"cached": 1, "captures": 1, "replays": 2}
    assert seen[3]["captures"] == 2 and seen[4] == {"cached": 2, "captures": 2, "replays": 3}
    g_on.close()
    g_off.close()


def test_graph_replay_with_residual_epilogue_layer_norm():
    # Batches of one shape bucket at T > 4096 (one round of persistent
    # residual tiles, whose epilogue finishes the LayerNorm through the row
    # panels' sync ints) replay one captured graph: every launch leaves the
    # ints at zero for the next replay.  Each result equals the launch-by-
    # launch run with the standalone LayerNorm, bit for bit.
    rl, enc, w = synth.make_model(**dict(synth.PRESETS["cfg2"], num_hidden_layers=2), seed=48)
    cfg = synth.flat_cfg(rl, enc)
    g_on = sj.Model(w, cfg, precision=BF16, use_graphs=True)
    g_off = sj.Model(w, cfg, precision=BF16, use_graphs=False, fuse_ln=0)
    V = cfg["vocab_size"]
    batches = [synth.batch_with_lens([370, 380, 360, 375, 365, 384, 372, 368, 377, 366, 371, 369], 384, V, seed=49),
               synth.batch_with_lens([384, 300, 380, 350, 383, 376, 379, 381, 382, 330, 378, 380, 10], 384, V,
                                     seed=50),
               synth.batch_with_lens([350, 360, 340, 370, 345, 355, 365, 380, 384, 375, 362, 358], 384, V, seed=51)]
    for ids, mask, lens in batches:
        assert 4096 < int(lens.sum()) <= 4608 and 256 < lens.max() <= 384
    for i, (ids, mask, lens) in enumerate(batches + [batches[0]]):
        h = g_on.encode(ids, mask)
        want = g_off.encode(ids, mask)
        print(f"batch {i}: B={len(lens)} T={int(lens.sum())} graphs {g_on.graph_stats()}", flush=True)
        assert np.array_equal(h, want)
    assert g_on.graph_stats() == {"cached": 1, "captures": 1, "replays": 3}
    g_on.close()
    g_off.close()


def test_graph_cache_eviction_waits_for_queued_launches():
    # More graphs than the cache holds (32), issued back to back with no host
    # synchronization: every capture past the 32nd evicts the least recently
    # used graph while its launch may still be queued.  Each output buffer is
    # its own graph key (plus four shape buckets), and every result equals the
    # launch-by-launch model's, bit for bit; a second round recaptures evicted
    # graphs.
    import torch

    rl, enc, w = synth.make_model(**dict(synth.PRESETS["cfg2"], num_hidden_layers=2), seed=47)
    cfg = synth.flat_cfg(rl, enc)
    D, V = cfg["hidden_size"], cfg["vocab_size"]
    g_on = sj.Model(w, cfg, precision=BF16, use_graphs=True)
    g_off = sj.Model(w, cfg, precision=BF16, use_graphs=False)
    lens = [1500, 900, 400, 130]  # four buckets; the first call sizes the workspace
    ids = torch.from_numpy(np.random.default_rng(48).integers(0, V, size=max(lens)).astype(np.int32)).cuda()
    want = {}
    for n in lens:
        out = torch.empty((n, D), dtype=torch.float32, device="cuda")
        g_off.encode_device(ids.data_ptr(), np.array([n], np.int32), out.data_ptr())
        torch.cuda.synchronize()
        want[n] = out.cpu().numpy()
    calls = [lens[i % 4] for i in range(40)]
    outs = [torch.full((n, D), float("nan"), dtype=torch.float32, device="cuda") for n in calls]
    torch.cuda.synchronize()
    for rnd in range(2):
        order = range(40) if rnd == 0 else range(12)
        for i in order:
            g_on.encode_device(ids.data_ptr(), np.array([calls[i]], np.int32), outs[i].data_ptr())
        torch.cuda.synchronize()
        gs = g_on.graph_stats()
        print(f"round {rnd}: graphs {gs}", flush=True)
        for i in order:
            assert np.array_equal(outs[i].cpu().numpy(), want[calls[i]]), f"call {i} n={calls[i]}"
            outs[i].fill_(float("nan"))
        assert gs["cached"] == 32
    assert gs["captures"] == 52 and gs["replays"] == 0
    g_on.close()
    g_off.close()


def test_calls_on_two_streams_and_forward_are_ordered():
    # encode_device calls on two streams and a forward() on the model's own
    # stream share one workspace: each waits for the previous call.  Issued
    # back to back with no host synchronization, every result equals the same
    # call made alone.
    import torch

    rl, enc, w = synth.make_model(**dict(synth.PRESETS["cfg2"], num_hidden_layers=2), seed=51)
    cfg = synth.flat_cfg(rl, enc)
    m = sj.Model(w, cfg, precision=BF16)
    D = cfg["hidden_size"]
    batches = [synth.make_batch(4, 256, 30 + 20 * i, 256, cfg["vocab_size"], seed=52 + i) for i in range(4)]
    fwd_ids, fwd_mask, fwd_lens = synth.make_batch(3, 128, 20, 128, cfg["vocab_size"], seed=60)
    mp, mm, qt = synth.make_markers(fwd_lens, 3, [(0, 3), (1, 3), (2, 2)], seed=60)
    d_ids, d_out, want = [], [], []
    for ids, mask, lens in batches:
        packed = np.concatenate([ids[b, :lens[b]] for b in range(len(lens))]).astype(np.int32)
        d_ids.append(torch.from_numpy(packed).cuda())
        d_out.append(torch.full((len(packed), D), float("nan"), dtype=torch.float32, device="cuda"))
        h = m.encode(ids, mask)
        want.append(np.concatenate([h[b, :lens[b]] for b in range(len(lens))]))
    lg_want, act_want = m.forward(fwd_ids, fwd_mask, mp, mm, qt)
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]  # default priority
    for rep in range(2):
        for i, (ids, mask, lens) in enumerate(batches):
            m.encode_device(d_ids[i].data_ptr(), lens.astype(np.int32), d_out[i].data_ptr(),
                            streams[i % 2].cuda_stream)
        lg, act = m.forward(fwd_ids, fwd_mask, mp, mm, qt)  # synchronizes its own stream
        torch.cuda.synchronize()
        for i in range(len(batches)):
            assert np.array_equal(d_out[i].cpu().numpy(), want[i]), (rep, i)
        assert np.array_equal(lg, lg_want) and np.array_equal(act, act_want)
        for t in d_out:
            t.fill_(float("nan"))
        torch.cuda.synchronize()
    m.close()


@pytest.mark.parametrize("prec", [FP32, BF16])
def test_hidden_wider_than_1024_at_batch_one(orc, prec):
    # D = 1536: the layer norms take the scalar row kernel, so the short
    # batch's residual GEMMs must not fold split-K partials into them
    rl, enc, w = synth.make_model(hidden_size=1536, num_hidden_layers=2, num_attention_heads=24,
                                  intermediate_size=1024, vocab_size=1000, store="BF16",
                                  max_position_embeddings=512, head_layers=1, seed=71)
    cfg = synth.flat_cfg(rl, enc)
    ids, mask, lens = synth.make_batch(1, 120, 120, 120, cfg["vocab_size"], seed=72)
    mp, mm, qt = synth.make_markers(lens, 4, [(0, 4)], seed=72)
    om = orc.model(w, cfg)
    m = sj.Model(w, cfg, precision=prec)
    assert valid_err(m.encode(ids, mask), om.encode(ids, mask), mask) <= TOL[prec]
    lg, act = m.forward(ids, mask, mp, mm, qt)
    ref_lg, ref_act = om.forward(ids, mask, mp, mm, qt)
    assert probs_err(orc, lg, ref_lg, mm) <= 5e-3
    assert float(np.abs(act - ref_act).max()) <= 5e-3
    m.close()


def test_encode_device_matches_encode():
    import torch

    rl, enc, w = synth.make_model(**dict(synth.PRESETS["cfg2"], num_hidden_layers=2), seed=31)
    cfg = synth.flat_cfg(rl, enc)
    ids, mask, lens = synth.make_batch(8, 300, 10, 300, cfg["vocab_size"], seed=32)
    m = sj.Model(w, cfg, precision=BF16)
    h = m.encode(ids, mask)
    packed = np.concatenate([ids[b, :lens[b]] for b in range(8)]).astype(np.int32)
    d_ids = torch.from_numpy(packed).cuda()
    d_out = torch.empty((len(packed), cfg["hidden_size"]), dtype=torch.float32, device="cuda")
    for _ in range(2):  # second call replays the captured graph
        m.encode_device(d_ids.data_ptr(), lens.astype(np.int32), d_out.data_ptr(),
                        torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        got = d_out.cpu().numpy()
        want = np.concatenate([h[b, :lens[b]] for b in range(8)])
        assert np.array_equal(got, want)
    m.close()


def test_input_validation_errors():
    rl, enc, w = synth.make_model(hidden_size=64, num_hidden_layers=1, num_attention_heads=4,
                                  intermediate_size=64, vocab_size=100, max_position_embeddings=32,
                                  head_layers=1)
    cfg = synth.flat_cfg(rl, enc)
    m = sj.Model(w, cfg, precision=FP32)
    ids = np.zeros((1, 40), np.int64)
    with pytest.raises(sj.SjhError, match="max_len"):
        m.encode(ids, np.ones_like(ids))
    ids = np.full((1, 8), 100, np.int64)
    with pytest.raises(sj.SjhError, match="vocabulary"):
        m.encode(ids, np.ones_like(ids))
    m.close()
