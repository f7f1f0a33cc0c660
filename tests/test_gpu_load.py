"""Checkpoints loaded straight to the device (sjh_model_load) against models
staged from fp32 host arrays (sjh_model_create) on the same weights: bit for
bit, whatever the stored type.  BF16 files are copied as they are; F32 and
F16 files are rounded to bf16 on the device (round to nearest even, as the
host path rounds); fp8 files carry the codes and scales of the pinned host
quantizer (sjh_quantize_fp8), and F32/BF16 files loaded in the fp8 mode are
quantized on the device, which must give the same codes and scales."""
import numpy as np
import pytest

import snapjudge_amd as sj
from snapjudge_amd import synth

pytestmark = pytest.mark.gpu

BF16, FP32, FP8W = sj.SJH_PREC_BF16, sj.SJH_PREC_FP32, sj.SJH_PREC_FP8W


def decision_model(seed, **kw):
    p = dict(hidden_size=128, num_hidden_layers=2, num_attention_heads=2, intermediate_size=192,
             vocab_size=1000, store="BF16", max_position_embeddings=256, head_layers=2, n_act=3,
             layer_types=["full_attention", "sliding_attention"], local_attention=16,
             theta_sliding=7000.0, lora_r=4, seed=seed)
    p.update(kw)
    return synth.make_model(**p)


def same_outputs(a, b, ids, mask, mp, mm, qt):
    assert np.array_equal(a.encode(ids, mask), b.encode(ids, mask))
    la, aa = a.forward(ids, mask, mp, mm, qt)
    lb, ab = b.forward(ids, mask, mp, mm, qt)
    assert np.array_equal(la, lb) and np.array_equal(aa, ab)


@pytest.mark.parametrize("store", ["BF16", "F32", "F16"])
@pytest.mark.parametrize("prec", [BF16, FP32])
def test_load_equals_create(tmp_path, store, prec):
    rl, enc, w = decision_model(91)
    synth.write_checkpoint(str(tmp_path), rl, enc, w, store=store)
    # the values the file holds, widened to fp32 on the host
    rl2, enc2, w2 = synth.read_checkpoint(str(tmp_path))
    cfg = synth.flat_cfg(rl2, enc2)
    ids, mask, lens = synth.make_batch(5, 120, 10, 120, cfg["vocab_size"], seed=92)
    mp, mm, qt = synth.make_markers(lens, 4, [(0, 4), (1, 4), (2, 2), (0, 3), (1, 2)], seed=92)
    print(f"store={store} prec={prec}", flush=True)
    a = sj.Model.load(str(tmp_path), precision=prec)
    b = sj.Model(w2, cfg, precision=prec)
    same_outputs(a, b, ids, mask, mp, mm, qt)
    a.close()
    b.close()


def test_fp8_checkpoint_and_device_quantizer(tmp_path):
    # hidden and intermediate sizes multiples of 64 (the fp8 GEMM's rows)
    rl, enc, w = decision_model(93, hidden_size=256, num_attention_heads=4, intermediate_size=320,
                                lora_r=0)
    cfg = synth.flat_cfg(rl, enc)
    ids, mask, lens = synth.make_batch(4, 250, 20, 250, cfg["vocab_size"], seed=94)
    mp, mm, qt = synth.make_markers(lens, 3, [(0, 3), (1, 3), (2, 2), (0, 2)], seed=94)
    synth.write_checkpoint(str(tmp_path / "bf16"), rl, enc, w, store="BF16")
    synth.write_checkpoint(str(tmp_path / "fp8"), rl, enc, synth.fp8_tensors(w, sj.quantize_fp8),
                           store="BF16")
    ref = sj.Model(w, cfg, precision=FP8W)  # device quantizer, from host fp32
    disk = sj.Model.load(str(tmp_path / "fp8"), precision=FP8W)  # host quantizer's codes
    dev = sj.Model.load(str(tmp_path / "bf16"), precision=FP8W)  # device quantizer, from bf16
    same_outputs(ref, disk, ids, mask, mp, mm, qt)
    same_outputs(ref, dev, ids, mask, mp, mm, qt)
    with pytest.raises(sj.SjhError, match="SJH_PREC_FP8W"):
        sj.Model.load(str(tmp_path / "fp8"), precision=BF16)
    for m in (ref, disk, dev):
        m.close()


def test_load_the_reference_tiny_checkpoint(golden_dir, orc):
    # the reference's own fixture (F32, a sliding layer), loaded from its files
    rl, enc, w = synth.read_checkpoint(golden_dir + "/tiny-ckpt")
    cfg = synth.flat_cfg(rl, enc)
    ids, mask, lens = synth.make_batch(4, 24, 1, 24, cfg["vocab_size"], seed=5)
    mp, mm, qt = synth.make_markers(lens, 3, [(0, 3), (2, 2), (1, 3), (2, 2)], seed=5)
    a = sj.Model.load(golden_dir + "/tiny-ckpt", precision=FP32)
    b = sj.Model(w, cfg, precision=FP32)
    same_outputs(a, b, ids, mask, mp, mm, qt)
    h = a.encode(ids, mask)
    ref = orc.model(w, cfg).encode(ids, mask)
    m = mask.astype(bool)
    assert float(np.abs(h[m] - ref[m]).max()) <= 1e-4
    a.close()
    b.close()
