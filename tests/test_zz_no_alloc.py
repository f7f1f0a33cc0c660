"""sjh_model_encode_device_noalloc against sjh_model_encode_device.

The allocation-free variant runs the same kernels on the same launch sizes
with its buffers in the library's fixed per-device scratch array, so its
output must equal encode_device's bit for bit: two calls in a row, the second
with a smaller batch (the short-batch split-K path), with the array's contents
left over from the first call, from another model on the same device, and on
the NULL stream.  A batch that does not fit the array is rejected before any
GPU work."""
import numpy as np
import pytest

import snapjudge_amd as sj
from snapjudge_amd import synth

pytestmark = pytest.mark.gpu


def packed(ids, lens):
    return np.concatenate([ids[b, :lens[b]] for b in range(len(lens))]).astype(np.int32)


def run(m, fn, ids, lens, D, stream):
    import torch

    d_ids = torch.from_numpy(packed(ids, lens)).cuda()
    out = torch.full((int(lens.sum()), D), float("nan"), dtype=torch.float32, device="cuda")
    getattr(m, fn)(d_ids.data_ptr(), lens.astype(np.int32), out.data_ptr(), stream)
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("prec", [sj.SJH_PREC_BF16, sj.SJH_PREC_FP32])
def test_noalloc_equals_encode_device(prec):
    import torch

    rl, enc, w = synth.make_model(**dict(synth.PRESETS["cfg2"], num_hidden_layers=2), seed=81)
    cfg = synth.flat_cfg(rl, enc)
    D, V = cfg["hidden_size"], cfg["vocab_size"]
    m = sj.Model(w, cfg, precision=prec)
    stream = torch.cuda.current_stream().cuda_stream
    # ~1900 tokens (bf16) / ~850 tokens (fp32: twice the bytes per token)
    big = (synth.make_batch(6, 400, 100, 400, V, seed=82) if prec == sj.SJH_PREC_BF16
           else synth.make_batch(4, 300, 100, 300, V, seed=82))
    small = synth.make_batch(2, 120, 40, 120, V, seed=83)   # <= 256 tokens: split-K residuals
    for name, (ids, _, lens) in (("big", big), ("small", small)):
        want = run(m, "encode_device", ids, lens, D, stream)
        got = run(m, "encode_device_noalloc", ids, lens, D, stream)
        print(f"prec={prec} {name}: T={int(lens.sum())} equal={np.array_equal(got, want)}", flush=True)
        assert np.isfinite(want).all()
        assert np.array_equal(got, want)
    # another model on the same device overwrites the shared array; the first
    # model's next call (NULL stream) is still exact
    rl2, enc2, w2 = synth.make_model(**dict(synth.PRESETS["cfg2"], num_hidden_layers=1), seed=84)
    m2 = sj.Model(w2, synth.flat_cfg(rl2, enc2), precision=prec)
    ids, _, lens = big
    other = run(m2, "encode_device_noalloc", ids, lens, D, stream)
    assert np.array_equal(other, run(m2, "encode_device", ids, lens, D, stream))
    ids, _, lens = small
    assert np.array_equal(run(m, "encode_device_noalloc", ids, lens, D, 0),
                          run(m, "encode_device", ids, lens, D, 0))
    m2.close()
    m.close()


def test_noalloc_rejects_batches_beyond_the_array():
    # the host rejects these before any launch; the id and output buffers are
    # nevertheless real and sized for the batch
    import torch

    rl, enc, w = synth.make_model(**dict(synth.PRESETS["cfg2"], num_hidden_layers=1), seed=85)
    cfg = synth.flat_cfg(rl, enc)
    D = cfg["hidden_size"]
    m = sj.Model(w, cfg, precision=sj.SJH_PREC_BF16)
    stream = torch.cuda.current_stream().cuda_stream
    for lens, msg in ((np.full(16, 512, np.int32), "scratch"),      # 8192 tokens, ~80 MB
                      (np.ones(300, np.int32), "256 sequences")):
        T = int(lens.sum())
        d_ids = torch.zeros(T, dtype=torch.int32, device="cuda")
        out = torch.zeros((T, D), dtype=torch.float32, device="cuda")
        with pytest.raises(sj.SjhError, match=msg) as e:
            m.encode_device_noalloc(d_ids.data_ptr(), lens, out.data_ptr(), stream)
        assert e.value.code == -1  # SJH_E_INVALID
    torch.cuda.synchronize()
    m.close()
