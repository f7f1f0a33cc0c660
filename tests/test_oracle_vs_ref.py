"""The oracle against the reference's own CPU forward (oracle/_ref/libsjref.so,
compiled from the reference sources by oracle/Makefile).  Both are built with
-ffp-contract=off and follow the same operation order, so they must agree bit
for bit.  Skipped where the reference build is absent (e.g. on the GPU box
without the prebuilt library)."""
import numpy as np
import pytest

from oracle import RefModel
from snapjudge_amd import synth

pytestmark = pytest.mark.skipif(not RefModel.available(), reason="oracle/_ref not built")


def _compare(orc, tmp_path, rl, enc, w, store, B, L, lo, hi, kinds, K, seed):
    synth.write_checkpoint(str(tmp_path), rl, enc, w, store=store)
    rl2, enc2, w2 = synth.read_checkpoint(str(tmp_path))
    cfg = synth.flat_cfg(rl2, enc2)
    ref = RefModel(str(tmp_path))
    om = orc.model(w2, cfg)
    ids, mask, lens = synth.make_batch(B, L, lo, hi, cfg["vocab_size"], seed=seed)
    mp, mm, qt = synth.make_markers(lens, K, kinds, seed=seed)
    assert np.array_equal(om.encode(ids, mask), ref.encode(ids, mask))
    lo_, ao = om.forward(ids, mask, mp, mm, qt)
    lr, ar = ref.forward(ids, mask, mp, mm, qt)
    assert np.array_equal(lo_, lr)
    assert np.array_equal(ao, ar)
    cf, sf, cs, ss = ref.rope_tables()
    assert np.array_equal(cf, om.rope[0]) and np.array_equal(sf, om.rope[1])
    assert np.array_equal(cs, om.rope[2]) and np.array_equal(ss, om.rope[3])


def test_tiny_checkpoint_bit_exact(orc, golden_dir):
    ref = RefModel(golden_dir + "/tiny-ckpt")
    rl, enc, w = synth.read_checkpoint(golden_dir + "/tiny-ckpt")
    cfg = synth.flat_cfg(rl, enc)
    om = orc.model(w, cfg)
    ids, mask, lens = synth.make_batch(4, 24, 1, 24, cfg["vocab_size"], seed=5)
    mp, mm, qt = synth.make_markers(lens, 3, [(0, 3), (2, 2), (1, 3), (2, 2)], seed=5)
    assert np.array_equal(om.encode(ids, mask), ref.encode(ids, mask))
    a = om.forward(ids, mask, mp, mm, qt)
    b = ref.forward(ids, mask, mp, mm, qt)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


def test_cfg1_bit_exact(orc, tmp_path):
    rl, enc, w = synth.make_model(**synth.PRESETS["cfg1"], seed=11)
    _compare(orc, tmp_path, rl, enc, w, "F32", 8, 32, 8, 32,
             [(0, 4), (2, 2)] * 4, 4, seed=3)


def test_sliding_lora_bf16_bit_exact(orc, tmp_path):
    rl, enc, w = synth.make_model(hidden_size=64, num_hidden_layers=3, num_attention_heads=2,
                                  intermediate_size=96, vocab_size=300, store="BF16",
                                  max_position_embeddings=64, head_layers=1, n_act=3,
                                  layer_types=["full_attention", "sliding_attention",
                                               "full_attention"],
                                  local_attention=6, theta_sliding=5000.0, lora_r=4, seed=2)
    _compare(orc, tmp_path, rl, enc, w, "BF16", 5, 40, 3, 40,
             [(0, 5), (1, 5), (2, 2), (0, 3), (1, 4)], 5, seed=9)


def test_ops_bit_exact(orc):
    import ctypes as C

    L = RefModel.lib()
    rng = np.random.default_rng(4)
    a = rng.standard_normal((13, 40)).astype(np.float32)
    w = rng.standard_normal((17, 40)).astype(np.float32)
    b = rng.standard_normal(17).astype(np.float32)
    p = lambda x: x.ctypes.data_as(C.c_void_p)
    for act in (0, 1, 2):
        out = np.empty((13, 17), np.float32)
        L.sjref_gemm_nt(p(a), p(w), p(b), act, 13, 17, 40, p(out))
        assert np.array_equal(out, orc.gemm_nt(a, w, b, act))
    wi = rng.standard_normal((2 * 9, 40)).astype(np.float32)
    out = np.empty((13, 9), np.float32)
    L.sjref_gemm_geglu(p(a), p(wi), 13, 9, 40, p(out))
    assert np.array_equal(out, orc.gemm_geglu(a, wi))
    x = (rng.standard_normal((6, 50)) * 4 + 1).astype(np.float32)
    lw = rng.standard_normal(50).astype(np.float32)
    lb = rng.standard_normal(50).astype(np.float32)
    out = np.empty_like(x)
    L.sjref_layer_norm(p(x), 6, 50, p(lw), p(lb), C.c_float(1e-5), p(out))
    assert np.array_equal(out, orc.layer_norm(x, lw, lb, 1e-5))
    q, k, v = (rng.standard_normal((2, 3, 11, 8)).astype(np.float32) for _ in range(3))
    lens = np.array([11, 6], np.int64)
    for win in (0, 2):
        out = np.empty_like(q)
        L.sjref_attention(p(q), p(k), p(v), p(lens), 2, 3, 11, 8, win, p(out))
        assert np.array_equal(out, orc.attention(q, k, v, lens, win))


def test_sj_model_bit_exact(orc, tmp_path):
    # SjModel (src/sj_model.cpp): learned positions (rows past max_positions
    # clamp to the last one), biased LayerNorms, separate q/k/v/o with biases,
    # GELU FFNs, a head of two layers and the scorer; padded rows included
    from oracle import RefSjModel

    cfg, w = synth.make_sj_model(hidden_size=48, num_layers=2, num_heads=3, vocab_size=200,
                                 intermediate_size=80, max_positions=20, head_layers=2,
                                 head_intermediate=64, seed=13)
    synth.write_sj_checkpoint(str(tmp_path), cfg, w, store="F32")
    ref = RefSjModel(str(tmp_path))
    om = orc.sj_model(w, cfg)
    ids, mask, lens = synth.make_batch(4, 26, 3, 26, cfg["vocab_size"], seed=14)
    mp, mm, qt = synth.make_markers(lens, 4, [(0, 4), (1, 3), (2, 2), (0, 1)], seed=14)
    mp[1, 0] = 40  # clamped to L - 1
    assert np.array_equal(om.encode(ids, mask), ref.encode(ids, mask))
    lo_, ao = om.forward(ids, mask, mp, mm, qt)
    lr, ar = ref.forward(ids, mask, mp, mm, qt)
    assert np.array_equal(lo_, lr) and np.array_equal(ao, ar)
    assert np.all(lo_[mm == 0] == np.float32(-1e4))
    # act is {top1, 1 - top1} of the softmax over the (masked) logits
    for b in range(len(lo_)):
        p = np.exp(lo_[b].astype(np.float64) - lo_[b].max())
        assert abs(ao[b, 0] - (p / p.sum()).max()) < 1e-6
        assert abs(ao[b, 0] + ao[b, 1] - 1.0) < 1e-6


def test_sj_model_catches_a_dropped_bias(orc, tmp_path):
    # the oracle run without one layer's attention output bias no longer
    # matches the reference: the comparison above is sensitive to it
    from oracle import RefSjModel

    cfg, w = synth.make_sj_model(hidden_size=32, num_layers=1, num_heads=2, vocab_size=100,
                                 max_positions=16, seed=15)
    synth.write_sj_checkpoint(str(tmp_path), cfg, w, store="F32")
    ref = RefSjModel(str(tmp_path))
    w2 = dict(w)
    w2["sj.encoder.layers.0.attn.o.bias"] = np.zeros_like(w["sj.encoder.layers.0.attn.o.bias"])
    ids, mask, _ = synth.make_batch(2, 10, 4, 10, cfg["vocab_size"], seed=16)
    assert not np.allclose(orc.sj_model(w2, cfg).encode(ids, mask), ref.encode(ids, mask), atol=1e-4)
