"""fp8 weight format of the SJH_PREC_FP8W mode, on the CPU (no GPU needed).

The quantizer (sjh_quantize_fp8, the host code the model staging uses) is
pinned against an independent brute-force restatement: the nearest finite OCP
e4m3fn value by exhaustive search over the code table, ties to the even code,
saturation at 448.  The code table itself is pinned by its closed form at
known points (zero, the subnormal steps, 1.0, the largest finite value, NaN).
That the GPU decodes every code to the same value is checked in
tests/test_gpu_fp8.py."""
import numpy as np
import pytest

import snapjudge_amd as sj

TABLE = sj.fp8_e4m3_table()


def brute_e4m3(x: np.ndarray) -> np.ndarray:
    pos = TABLE[:127].astype(np.float64)  # finite non-negative codes 0x00..0x7e
    out = np.empty(x.shape, np.uint8)
    for idx, v in np.ndenumerate(x.astype(np.float64)):
        sign = 0x80 if np.signbit(v) else 0
        if np.isnan(v):
            out[idx] = sign | 0x7F
            continue
        a = abs(v)
        if a >= 448.0:
            code = 0x7E
        else:
            d = np.abs(pos - a)
            cands = np.nonzero(d == d.min())[0]
            code = int(cands[0]) if len(cands) == 1 else int([c for c in cands if c % 2 == 0][0])
        out[idx] = sign | code
    return out


def test_code_table_closed_form():
    assert TABLE[0x00] == 0.0 and TABLE[0x80] == 0.0 and np.signbit(TABLE[0x80])
    assert TABLE[0x01] == 2.0 ** -9 and TABLE[0x07] == 7 * 2.0 ** -9
    assert TABLE[0x08] == 2.0 ** -6  # smallest normal
    assert TABLE[0x38] == 1.0 and TABLE[0xB8] == -1.0
    assert TABLE[0x7E] == 448.0 and TABLE[0xFE] == -448.0
    assert np.isnan(TABLE[0x7F]) and np.isnan(TABLE[0xFF])
    assert np.all(np.diff(TABLE[:127]) > 0)  # codes order like their values
    assert np.array_equal(TABLE[128:255], -TABLE[:127])


def test_rounding_ties_and_saturation_at_unit_scale():
    # a row whose largest magnitude is 448 has scale exactly 1, so the codes
    # are the rounding of the values themselves
    pos = TABLE[:127].astype(np.float64)
    mids = (pos[:-1] + pos[1:]) / 2  # exact ties (representable in fp32)
    vals = np.concatenate([
        mids, np.nextafter(mids.astype(np.float32), np.float32(0)),
        np.nextafter(mids.astype(np.float32), np.float32(np.inf)),
        pos, -mids, [0.0, -0.0, 1e-30, -1e-30, 2.0 ** -10, 3 * 2.0 ** -11, 447.9, -447.99],
        np.random.default_rng(0).uniform(-448, 448, 2000),
        np.random.default_rng(1).uniform(-0.02, 0.02, 500),
    ]).astype(np.float32)
    row = np.concatenate([[np.float32(448.0)], vals])[None, :]
    q, sc = sj.quantize_fp8(row)
    assert sc[0] == np.float32(1.0)
    assert np.array_equal(q[0], brute_e4m3(row[0]))
    # ties really went to the even code
    qm = q[0, 1:1 + len(mids)]
    assert np.all(qm % 2 == 0)


def test_rows_scale_and_codes_match_brute_force():
    rng = np.random.default_rng(2)
    w = (rng.standard_normal((40, 300)) * rng.uniform(1e-4, 3.0, (40, 1))).astype(np.float32)
    w[3] = 0.0  # all-zero row: scale 1, codes 0
    w[7, :5] = [1e-3, -2e-3, 5.0, -5.0, 0.0]
    q, sc = sj.quantize_fp8(w)
    amax = np.abs(w).max(axis=1)
    want_sc = np.where(amax > 0, amax / np.float32(448.0), np.float32(1.0)).astype(np.float32)
    assert np.array_equal(sc, want_sc)
    assert np.all(q[3] == 0) and sc[3] == 1.0
    scaled = (w / sc[:, None]).astype(np.float32)
    assert np.array_equal(q, brute_e4m3(scaled))
    # each row's largest magnitude is represented exactly (code 0x7e)
    assert np.all((q[np.arange(40) != 3] & 0x7F).max(axis=1) == 0x7E)
    # dequantization error: at most half a step of the e4m3 grid at that value
    # (the larger of the two neighbouring gaps, plus fp32 rounding of the scale)
    deq = TABLE[q] * sc[:, None]
    c = (q & 0x7F).astype(int)
    up = TABLE[np.minimum(c + 1, 0x7E)] - TABLE[c]
    down = TABLE[c] - TABLE[np.maximum(c - 1, 0)]
    step = np.maximum(up, down)
    assert np.all(np.abs(deq - w) <= 0.5 * step * sc[:, None] + 4e-7 * np.abs(w) + 1e-30)


def test_quantize_rejects_bad_shape():
    with pytest.raises(sj.SjhError):
        sj.check(sj.lib().sjh_quantize_fp8(None, -1, 4, None, None))
