"""The algorithmic work behind bench.py's roofline figures (role_work,
gemm_flops_per_token, kernel_table), checked on the CPU against counts made
independently of those formulas: the per-token GEMM figures published for the
BASELINE configs, the multiply-adds implied by a synthetic model's own weight
shapes, a per-sequence count of the attention products, and the bytes of the
arrays each launch reads and writes once."""
import numpy as np
import pytest

import bench
from snapjudge_amd import synth

D, F, H, T = 64, 96, 4, 37
BF16, F32 = np.uint16, np.float32


def _layer_weights():
    _, _, w = synth.make_model(hidden_size=D, num_hidden_layers=1, num_attention_heads=H, intermediate_size=F,
                               vocab_size=128, seed=0)
    return {k: w[f"encoder.layers.0.{k}.weight"].shape for k in ("attn.Wqkv", "attn.Wo", "mlp.Wi", "mlp.Wo")}


def _nbytes(*shapes_and_types):
    return float(sum(np.empty(s, t).nbytes for s, t in shapes_and_types))


def test_gemm_flops_per_token_matches_the_published_figures():
    # 220.59 MFLOP per valid token at D 768 / F 1152 / 22 layers (configs 2-4)
    # and 686.29 at D 1024 / F 2624 / 28 layers (config 5)
    assert bench.gemm_flops_per_token(768, 1152, 22) / 1e6 == pytest.approx(220.59, abs=0.005)
    assert bench.gemm_flops_per_token(1024, 2624, 28) / 1e6 == pytest.approx(686.29, abs=0.005)


def test_gemm_roles_count_the_weight_shapes():
    # every projection is out[T, N] = A[T, K] . W[N, K]^T: 2 T N K FLOPs
    shp = _layer_weights()

    def flops(name):
        n, k = shp[name]
        return 2.0 * T * n * k

    assert bench.role_work("gemm_qkv_rope", T, D, F, 0)[0] == flops("attn.Wqkv")
    assert bench.role_work("gemm_wi_geglu", T, D, F, 0)[0] == flops("mlp.Wi")
    for role in ("gemm_wo_resid", "gemm_wo_resid_ln"):
        assert bench.role_work(role, T, D, F, 0)[0] == flops("attn.Wo")
    for role in ("gemm_wo2_resid", "gemm_wo2_resid_ln"):
        assert bench.role_work(role, T, D, F, 0)[0] == flops("mlp.Wo")
    layer = sum(bench.role_work(r, T, D, F, 0)[0]
                for r in ("gemm_qkv_rope", "gemm_wi_geglu", "gemm_wo_resid", "gemm_wo2_resid"))
    assert layer == pytest.approx(T * bench.gemm_flops_per_token(D, F, 1), rel=1e-12)


def test_gemm_roles_count_each_operand_once():
    shp = _layer_weights()
    x_rw = [((T, D), F32), ((T, D), F32)]  # the fp32 residual stream, read and written
    want = {
        "gemm_qkv_rope": [((T, D), BF16), (shp["attn.Wqkv"], BF16), ((T, 3 * D), BF16)],
        "gemm_wi_geglu": [((T, D), BF16), (shp["mlp.Wi"], BF16), ((T, F), BF16)],
        "gemm_wo_resid": [((T, D), BF16), (shp["attn.Wo"], BF16)] + x_rw,
        "gemm_wo2_resid": [((T, F), BF16), (shp["mlp.Wo"], BF16)] + x_rw,
        # and the LayerNorm's bf16 rows that the epilogue writes
        "gemm_wo_resid_ln": [((T, D), BF16), (shp["attn.Wo"], BF16), ((T, D), BF16)] + x_rw,
        "gemm_wo2_resid_ln": [((T, F), BF16), (shp["mlp.Wo"], BF16), ((T, D), BF16)] + x_rw,
        # q, k and v read, o written
        "attention": [((T, D), BF16)] * 4,
        # fp32 rows in, bf16 rows out; the final norm writes fp32
        "attn_norm": [((T, D), F32), ((T, D), BF16)],
        "mlp_norm": [((T, D), F32), ((T, D), BF16)],
        "final_norm": [((T, D), F32), ((T, D), F32)],
    }
    for role, arrays in want.items():
        assert bench.role_work(role, T, D, F, 0)[1] == _nbytes(*arrays), role


def test_attention_flops_count_every_score_and_weighted_value():
    Dh = D // H
    lens = [5, 17, 0, 64, 1]
    count = 0
    for n in lens:  # varlen, non-causal: each sequence attends only to itself
        for _ in range(H):
            count += 2 * n * n * Dh  # Q K^T: n x n scores of Dh multiply-adds
            count += 2 * n * n * Dh  # P V: n x Dh outputs of n multiply-adds
    sum_n2 = float(sum(n * n for n in lens))
    assert bench.role_work("attention", sum(lens), D, F, sum_n2)[0] == count


def test_kernel_table_averages_work_over_its_roles_by_launch():
    lens = np.array([5, 17, 64, 1])
    Tv = int(lens.sum())
    steps = 2
    # (total ms over the run, launches): 21 Wo and 22 Wo2 launches per step
    prof = {"gemm_wo_resid_ln": (0.5, 21 * steps), "gemm_wo2_resid_ln": (0.7, 22 * steps),
            "attn_norm": (0.04, 2 * steps)}
    tab = bench.kernel_table(prof, steps, Tv, D, F, 22, lens)
    g = tab["gemm_resid_ln"]
    n = 43 * steps
    w_wo = bench.role_work("gemm_wo_resid_ln", Tv, D, F, 0)[0]
    w_wo2 = bench.role_work("gemm_wo2_resid_ln", Tv, D, F, 0)[0]
    flops = (21 * w_wo + 22 * w_wo2) * steps / n
    avg_s = 1.2e-3 / n
    assert g["launches_per_step"] == 43
    assert g["ms_per_step"] == pytest.approx(0.6, abs=1e-4)
    assert g["work_per_launch"] == pytest.approx(flops)
    assert g["achieved"] == pytest.approx(flops / avg_s / 1e12, abs=0.01)
    assert g["frac"] == pytest.approx(g["achieved"] / bench.PEAK_BF16_TFLOPS, abs=1e-4)
    ln = tab["layer_norm"]  # bytes against the HBM peak
    assert ln["bound"] == "hbm" and ln["unit"] == "GB/s"
    assert ln["achieved"] == pytest.approx(6.0 * Tv * D / (0.04e-3 / (2 * steps)) / 1e9, abs=0.01)
    assert "attention" not in tab  # no launches, no row
