"""Checkpoint loading (sjh_model_load) before any device work: the files are
read and checked against the reference loaders' rules first
(src/safetensors.cpp:16-61, src/model.cpp:35-205, src/sj_model.cpp:87-204),
so every malformed checkpoint fails with SJH_E_INVALID and a message here,
without a GPU.  A well-formed one gets as far as device selection (this
container has no GPU: SJH_E_DEVICE).  The loaded values are checked on the
GPU (tests/test_gpu_load.py)."""
import json
import os
import struct

import numpy as np
import pytest

import snapjudge_amd as sj
from snapjudge_amd import synth

INVALID, DEVICE = -1, -2


def load_rc(path):
    try:
        torch = __import__("torch")
        if torch.cuda.is_available():
            pytest.skip("checks the loader ahead of device work; a GPU is present")
    except ImportError:
        pass
    import ctypes as C

    h = C.c_void_p()
    opt = sj.Options(sj.SJH_PREC_BF16, 0, 1, 0, 0)
    rc = sj.lib().sjh_model_load(os.fsencode(str(path)), C.byref(opt), C.byref(h))
    return rc, sj.lib().sjh_last_error().decode()


def small_decision(tmp_path, **kw):
    rl, enc, w = synth.make_model(hidden_size=64, num_hidden_layers=2, num_attention_heads=2,
                                  intermediate_size=96, vocab_size=300, store="BF16",
                                  max_position_embeddings=64, head_layers=1, seed=3)
    return rl, enc, w


def test_well_formed_checkpoints_reach_device_selection(tmp_path):
    rl, enc, w = small_decision(tmp_path)
    for store in ("F32", "F16", "BF16"):
        d = tmp_path / store
        synth.write_checkpoint(str(d), rl, enc, w, store=store)
        rc, msg = load_rc(d)
        assert rc == DEVICE, msg
    d = tmp_path / "fp8"
    synth.write_checkpoint(str(d), rl, enc, synth.fp8_tensors(w, sj.quantize_fp8), store="BF16")
    rc, msg = load_rc(d)
    assert rc == DEVICE, msg
    cfg, sw = synth.make_sj_model(hidden_size=32, num_layers=1, num_heads=2, vocab_size=50, seed=4)
    synth.write_sj_checkpoint(str(tmp_path / "sj"), cfg, sw, store="BF16")
    rc, msg = load_rc(tmp_path / "sj")
    assert rc == DEVICE, msg


@pytest.mark.parametrize("case,match", [
    ("no_config", "no checkpoint"),
    ("missing_head_layers", "missing configuration keys \\['head_layers'\\]"),
    ("missing_prefix", "missing 'scorer.' parameters"),
    ("bad_shape", r"tensor encoder.layers.1.attn.Wo.weight expected \[64,64\] but has \[64,63\]"),
    ("missing_tensor", "missing tensor encoder.final_norm.weight"),
    ("bad_dtype", "unsupported dtype I64 for type_emb.weight"),
    ("size_mismatch", "size mismatch"),
    ("out_of_bounds", "out of bounds"),
    ("bad_header", "bad JSON"),
    ("fp8_without_scale", "missing tensor encoder.layers.0.attn.Wo.weight_scale"),
    ("fp8_elsewhere", "unsupported dtype F8_E4M3 for type_emb.weight"),
    ("bad_lora", "lora_A.weight"),
    # a number written as a string: the reference's json.value throws a type
    # error rather than loading the default
    ("string_layers", "config key 'num_hidden_layers': type must be number, but is string"),
    ("null_eps", "config key 'norm_eps': type must be number, but is null"),
])
def test_malformed_decision_checkpoints(tmp_path, case, match):
    rl, enc, w = small_decision(tmp_path)
    d = tmp_path / "ck"
    t = dict(w)
    if case == "string_layers":
        enc = dict(enc, num_hidden_layers="2")
    if case == "null_eps":
        enc = dict(enc, norm_eps=None)
    if case == "missing_head_layers":
        rl = {k: v for k, v in rl.items() if k != "head_layers"}
    if case == "missing_prefix":
        t = {k: v for k, v in t.items() if not k.startswith("scorer.")}
    if case == "bad_shape":
        t["encoder.layers.1.attn.Wo.weight"] = t["encoder.layers.1.attn.Wo.weight"][:, :63].copy()
    if case == "missing_tensor":
        del t["encoder.final_norm.weight"]
    if case == "bad_dtype":
        t["type_emb.weight"] = ("I64", np.zeros((3, 64), np.int64))
    if case == "fp8_without_scale":
        q, _ = sj.quantize_fp8(t["encoder.layers.0.attn.Wo.weight"])
        t["encoder.layers.0.attn.Wo.weight"] = ("F8_E4M3", q)
    if case == "fp8_elsewhere":
        t["type_emb.weight"] = ("F8_E4M3", np.zeros((3, 64), np.uint8))
    if case == "bad_lora":
        t["lora_A.weight"] = np.zeros((4, 64), np.float32)
        t["lora_B.weight"] = np.zeros((64, 5), np.float32)
    synth.write_checkpoint(str(d), rl, enc, t, store="BF16")
    st = d / "model.safetensors"
    if case == "no_config":
        os.remove(d / "encoder" / "config.json")
    if case in ("size_mismatch", "out_of_bounds", "bad_header"):
        raw = bytearray(st.read_bytes())
        (hlen,) = struct.unpack("<Q", raw[:8])
        hdr = json.loads(raw[8:8 + hlen])
        if case == "size_mismatch":  # a BF16 tensor whose bytes do not match its shape
            hdr["type_emb.weight"]["shape"] = [3, 65]
        elif case == "out_of_bounds":
            hdr["type_emb.weight"]["data_offsets"][1] = len(raw) + 10
        hj = json.dumps(hdr).encode() if case != "bad_header" else raw[8:8 + hlen - 3]
        hj += b" " * ((8 - len(hj) % 8) % 8)
        body = raw[8 + hlen:]
        st.write_bytes(struct.pack("<Q", len(hj)) + hj + body)
    rc, msg = load_rc(d)
    assert rc == INVALID, msg
    assert __import__("re").search(match, msg), msg


@pytest.mark.parametrize("case,match", [
    ("missing_key", "config missing required keys"),
    ("bad_hidden", r"tensor sj.embeddings.word.weight expected \[50,48\] but has \[50,32\]"),
    ("missing_bias", "missing tensor sj.encoder.layers.0.attn.k.bias"),
])
def test_malformed_sj_checkpoints(tmp_path, case, match):
    # the reference's own rejection test changes hidden_size so that shapes
    # mismatch (tests/test_sj_model.cpp:61-70)
    cfg, w = synth.make_sj_model(hidden_size=32, num_layers=1, num_heads=2, vocab_size=50, seed=4)
    if case == "missing_key":
        del cfg["num_heads"]
    if case == "bad_hidden":
        cfg["hidden_size"] = 48
        cfg["intermediate_size"] = 128
        cfg["head_intermediate"] = 128
    if case == "missing_bias":
        del w["sj.encoder.layers.0.attn.k.bias"]
    synth.write_sj_checkpoint(str(tmp_path), cfg, w)
    rc, msg = load_rc(tmp_path)
    assert rc == INVALID, msg
    assert __import__("re").search(match, msg), msg
