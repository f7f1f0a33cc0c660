"""CPU-side checks of the C ABI library: it loads, exports every symbol the
header declares, and its host-side validation rejects bad calls with a
status code and a message (no compute is launched)."""
import ctypes as C
import os
import re

import numpy as np
import pytest

import snapjudge_amd as sj

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include",
                      "snapjudge_hip.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sjh_[a-z_0-9]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = sj.lib()
    syms = declared_symbols()
    assert len(syms) >= 15
    for s in syms:
        assert hasattr(lib, s), f"{s} declared in snapjudge_hip.h but not exported"
    # and the Python binding covers exactly the declared surface
    assert set(sj._SIGS) == set(syms)


def test_version_and_default_options():
    lib = sj.lib()
    assert lib.sjh_version() == 1
    o = sj.Options()
    lib.sjh_default_options(C.byref(o))
    assert (o.precision, o.use_graphs, o.pad_rows, o.device, o.fuse_ln, o.fuse_attn_wo) == (sj.SJH_PREC_BF16, 1, 0, 0, 1, 1)


def test_null_arguments_are_rejected():
    lib = sj.lib()
    h = C.c_void_p()
    rc = lib.sjh_model_create(None, None, C.byref(h))
    assert rc == -1 and b"null" in lib.sjh_last_error()
    rc = lib.sjh_model_encode(None, None, None, 1, 1, None)
    assert rc == -1 and b"null model" in lib.sjh_last_error()


def test_kernel_launchers_validate_before_launch():
    lib = sj.lib()
    # K not positive
    rc = lib.sjh_gemm(C.c_void_p(16), C.c_void_p(16), None, C.c_void_p(16), 4, 4, 0, 0, sj.SJH_BF16,
                      None)
    assert rc == -1 and b"K must be positive" in lib.sjh_last_error()
    # bad dtype
    rc = lib.sjh_gemm(C.c_void_p(16), C.c_void_p(16), None, C.c_void_p(16), 4, 4, 4, 0, 7, None)
    assert rc == -1 and b"dtype" in lib.sjh_last_error()
    # unsupported head_dim for attention
    lens = np.zeros(1, np.int32)
    rc = lib.sjh_attn(C.c_void_p(16), lens.ctypes.data_as(C.c_void_p), C.c_void_p(16), 1, 4, 1, 24,
                      0, sj.SJH_F32, None)
    assert rc != 0 and b"head_dim" in lib.sjh_last_error()
    # rope with odd head dim
    rc = lib.sjh_rope(C.c_void_p(16), None, None, 4, 4, 1, 3, sj.SJH_F32, None)
    assert rc == -1 and b"even" in lib.sjh_last_error()
    # layer norm with D out of range
    rc = lib.sjh_add_ln(C.c_void_p(16), None, None, None, C.c_void_p(16), 4, 5000, 1e-5, 0, 0,
                        sj.SJH_F32, None)
    assert rc == -1 and b"D must be" in lib.sjh_last_error()


def test_model_create_without_gpu_fails_cleanly():
    try:
        import torch

        if torch.cuda.is_available():
            pytest.skip("a GPU is visible")
    except ImportError:
        pass
    from snapjudge_amd import synth

    rl, enc, w = synth.make_model(hidden_size=16, num_hidden_layers=1, num_attention_heads=2,
                                  intermediate_size=8, vocab_size=32, max_position_embeddings=16,
                                  head_layers=1)
    with pytest.raises(sj.SjhError) as e:
        sj.Model(w, synth.flat_cfg(rl, enc))
    assert e.value.code in (-1, -2)
