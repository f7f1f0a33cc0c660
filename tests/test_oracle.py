"""Pins the oracle (oracle/sj_oracle.c) before anything is compared against it.

1. The reference's own golden vectors (tests/golden/tensor_ops.json, the file
   the reference's tests/test_tensor.cpp:58-100 checks its ops against, with
   the same tolerances).
2. Closed forms and invariants that a plausible slip (dropped term, swapped
   GEGLU halves, wrong RoPE pairing, wrong window edge, key padding leaking)
   would break.
3. The compiled reference (oracle/_ref) -- see test_oracle_vs_ref.py.
"""
import json
import math
import os

import numpy as np
import pytest


@pytest.fixture(scope="module")
def G(golden_dir):
    with open(os.path.join(golden_dir, "tensor_ops.json")) as f:
        return json.load(f)


def A(x):
    return np.asarray(x, dtype=np.float32)


def test_gemm_and_activations_vs_reference_golden(orc, G):
    a, w, b = A(G["gemm"]["a"]), A(G["gemm"]["w"]), A(G["gemm"]["bias"])
    assert np.abs(orc.gemm_nt(a, w, b, 0) - A(G["gemm"]["out"])).max() <= 1e-5
    assert np.abs(orc.gemm_nt(a, w, b, 1) - A(G["gemm_gelu"]["out"])).max() <= 1e-5
    assert np.abs(orc.gemm_nt(a, w, b, 2) - A(G["gemm_relu"]["out"])).max() <= 1e-5


def test_geglu_vs_reference_golden(orc, G):
    a, wi = A(G["gemm"]["a"]), A(G["geglu"]["wi"])
    got = orc.gemm_geglu(a, wi)
    assert np.abs(got - A(G["geglu"]["out"])).max() <= 1e-5
    # swapping the input and gate halves is a plausible slip: it must not match
    F = wi.shape[0] // 2
    swapped = orc.gemm_geglu(a, np.concatenate([wi[F:], wi[:F]]))
    assert np.abs(swapped - A(G["geglu"]["out"])).max() > 1e-3


def test_layer_norm_vs_reference_golden(orc, G):
    x, w, b = A(G["layer_norm"]["x"]), A(G["layer_norm"]["w"]), A(G["layer_norm"]["b"])
    assert np.abs(orc.layer_norm(x, w, b, 1e-5) - A(G["layer_norm"]["out"])).max() <= 1e-4
    assert np.abs(orc.layer_norm(x, w, None, 1e-5) - A(G["layer_norm"]["out_nobias"])).max() <= 1e-4


def test_softmax_vs_reference_golden(orc, G):
    assert np.abs(orc.softmax_rows(A(G["softmax"]["z"])) - A(G["softmax"]["out"])).max() <= 1e-6


def test_attention_vs_reference_golden(orc, G):
    q, k, v = A(G["attn_full"]["q"]), A(G["attn_full"]["k"]), A(G["attn_full"]["v"])
    lens = np.asarray(G["attn_full"]["lens"], np.int64)
    assert np.abs(orc.attention(q, k, v, lens, 0) - A(G["attn_full"]["out"])).max() <= 1e-5
    assert np.abs(orc.attention(q, k, v, lens, 2) - A(G["attn_window"]["out"])).max() <= 1e-5


def test_rope_vs_reference_golden(orc, G):
    r = G["rope"]
    got = orc.rope_inplace(A(r["qkv"]), A(r["cos"]), A(r["sin"]), r["L"], r["H"], r["Dh"])
    assert np.abs(got - A(r["out"])).max() <= 1e-5
    # the golden tables are the reference's table builder at theta 10000
    c, s = orc.rope_table(r["theta"], r["L"], r["Dh"])
    assert np.abs(c - A(r["cos"])).max() <= 1e-6 and np.abs(s - A(r["sin"])).max() <= 1e-6


def test_rope_table_closed_form(orc):
    c, s = orc.rope_table(160000.0, 300, 64)
    assert np.all(c[0] == 1.0) and np.all(s[0] == 0.0)
    assert np.abs(c * c + s * s - 1).max() < 1e-6
    # d = 0 has inverse frequency 1: angle = pos
    pos = np.arange(300)
    assert np.abs(c[:, 0] - np.cos(pos)).max() < 1e-6
    # highest pair: theta^(-2*31/64)
    inv = 160000.0 ** (-62 / 64)
    assert np.abs(s[:, 31] - np.sin(pos * inv)).max() < 1e-6


def test_rope_pairs_d_with_d_plus_half(orc):
    # one head, Dh = 4: row [x0 x1 x2 x3] rotates (x0, x2) and (x1, x3)
    L, H, Dh = 1, 1, 4
    qkv = np.zeros((1, 3 * H * Dh), np.float32)
    qkv[0, :4] = [1, 2, 3, 4]
    th = 0.3
    c = np.array([[math.cos(th), math.cos(th)]], np.float32)
    s = np.array([[math.sin(th), math.sin(th)]], np.float32)
    out = orc.rope_inplace(qkv, c, s, L, H, Dh)
    cs, sn = math.cos(th), math.sin(th)
    want = [1 * cs - 3 * sn, 2 * cs - 4 * sn, 3 * cs + 1 * sn, 4 * cs + 2 * sn]
    assert np.abs(out[0, :4] - want).max() < 1e-6
    assert np.all(out[0, 8:] == 0)  # v untouched


def test_layer_norm_moments(orc):
    rng = np.random.default_rng(0)
    x = (rng.standard_normal((7, 768)) * 3 + 5).astype(np.float32)
    y = orc.layer_norm(x, np.ones(768, np.float32), None, 1e-5)
    assert np.abs(y.mean(1)).max() < 1e-5
    assert np.abs(y.var(1) - 1).max() < 1e-4


def _np_attention(q, k, v, lens, window):
    B, H, L, Dh = q.shape
    out = np.zeros((B, H, L, Dh))
    for b in range(B):
        for i in range(L):
            lo, hi = 0, lens[b]
            if window > 0:
                lo, hi = max(0, i - window), min(lens[b], i + window + 1)
            if hi <= lo:
                continue
            s = np.einsum("hd,hjd->hj", q[b, :, i].astype(np.float64), k[b, :, lo:hi]) / math.sqrt(Dh)
            p = np.exp(s - s.max(1, keepdims=True))
            p /= p.sum(1, keepdims=True)
            out[b, :, i] = np.einsum("hj,hjd->hd", p, v[b, :, lo:hi])
    return out


@pytest.mark.parametrize("window", [0, 1, 3])
def test_attention_brute_force_and_padding(orc, window):
    rng = np.random.default_rng(window)
    B, H, L, Dh = 3, 2, 9, 8
    q, k, v = (rng.standard_normal((B, H, L, Dh)).astype(np.float32) for _ in range(3))
    lens = np.array([9, 5, 1], np.int64)
    got = orc.attention(q, k, v, lens, window)
    assert np.abs(got - _np_attention(q, k, v, lens, window)).max() < 1e-5
    # keys at or beyond len carry exactly zero weight
    k2, v2 = k.copy(), v.copy()
    k2[1, :, 5:] = 100.0
    v2[1, :, 5:] = -50.0
    assert np.array_equal(orc.attention(q, k2, v2, lens, window)[1], got[1])


def test_attention_constant_keys_average_values(orc):
    rng = np.random.default_rng(1)
    B, H, L, Dh = 1, 1, 6, 4
    q = rng.standard_normal((B, H, L, Dh)).astype(np.float32)
    k = np.ones((B, H, L, Dh), np.float32)
    v = rng.standard_normal((B, H, L, Dh)).astype(np.float32)
    out = orc.attention(q, k, v, np.array([4]), 0)
    assert np.abs(out[0, 0] - v[0, 0, :4].mean(0)).max() < 1e-6


def test_attention_len_zero_gives_zeros(orc):
    q = np.ones((1, 1, 3, 4), np.float32)
    out = orc.attention(q, q, q, np.array([0]), 0)
    assert np.all(out == 0)


def test_decode_math(orc):
    p = orc.calibrated_probs(np.array([1.0, 2.0, 3.0], np.float32), 2.0)
    z = np.array([0.5, 1.0, 1.5])
    assert np.abs(p - np.exp(z) / np.exp(z).sum()).max() < 1e-15
    assert orc.confidence(np.full(4, 0.25)) == pytest.approx(0.0, abs=1e-12)
    assert orc.confidence(np.array([1.0, 0, 0])) == pytest.approx(1.0, abs=1e-9)
    L = orc.L
    assert L.orc_round4(0.12344) == 0.1234 and L.orc_round4(0.12346) == 0.1235
    assert L.orc_round4(-0.33336) == -0.3334
    assert L.orc_clamp_temperature(0.1) == 0.5 and L.orc_clamp_temperature(9.0) == 5.0
    assert L.orc_clamp_temperature(float("nan")) == 1.0


def test_gelu_closed_form(orc):
    for x in (-3.0, -0.5, 0.0, 0.7, 2.5):
        assert orc.gelu(x) == pytest.approx(0.5 * x * (1 + math.erf(x / math.sqrt(2))), abs=1e-6)
