"""Synthetic snapjudge checkpoints and batches for tests and benchmarks.

Checkpoints follow the reference's on-disk layout (what
DecisionModel::load, src/model.cpp:35-205, and Agent::Agent,
src/agent.cpp:59-85, read): ``rl_agent_config.json``, ``encoder/config.json``
and ``model.safetensors`` with the tensor names of src/model.cpp:96-171.
Weights are N(0, std) from a seeded numpy Generator; norms are 1, head biases
0.  With ``store="BF16"`` every weight is rounded to bf16 before it is used
anywhere, so the CPU reference (which widens BF16 to fp32 on load,
src/safetensors.cpp:109-135) and the GPU see identical values.

Presets are the five configurations of BASELINE.json.

SjModel checkpoints (snapjudge's own BERT-style model, src/sj_model.cpp:87-204)
are ``sj_config.json`` + ``model.safetensors`` with the ``sj.*`` tensor names;
make_sj_model draws their norm gains and every bias at random too, so that a
dropped bias or a swapped norm shows in parity.
"""
from __future__ import annotations

import json
import os
import struct

import numpy as np

# (name -> encoder dims) for the benchmark configurations
PRESETS = {
    "cfg1": dict(hidden_size=64, num_hidden_layers=2, num_attention_heads=4,
                 intermediate_size=128, vocab_size=512, theta_full=10000.0, store="F32",
                 max_position_embeddings=512),
    "cfg2": dict(hidden_size=768, num_hidden_layers=22, num_attention_heads=12,
                 intermediate_size=1152, vocab_size=50368, theta_full=160000.0, store="BF16",
                 max_position_embeddings=8192),
    "cfg5": dict(hidden_size=1024, num_hidden_layers=28, num_attention_heads=16,
                 intermediate_size=2624, vocab_size=50368, theta_full=160000.0, store="BF16",
                 max_position_embeddings=8192),
}
PRESETS["cfg3"] = PRESETS["cfg2"]
PRESETS["cfg4"] = PRESETS["cfg2"]


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round fp32 to the nearest bf16 (ties to even), returned as fp32."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return (u.astype(np.uint32) << 16).view(np.float32)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def make_model(hidden_size: int, num_hidden_layers: int, num_attention_heads: int,
               intermediate_size: int, vocab_size: int, theta_full: float = 10000.0,
               theta_sliding: float = 10000.0, store: str = "F32",
               max_position_embeddings: int = 8192, head_layers: int = 2, n_act: int = 2,
               layer_types: list | None = None, local_attention: int = 0, lora_r: int = 0,
               std: float = 0.02, seed: int = 0, scorer_bias: bool = True,
               rng_chunk: int = 1 << 22):
    """Return (rl_cfg, enc_cfg, tensors) with fp32 arrays (bf16-exact if store=BF16)."""
    D, F, V, L = hidden_size, intermediate_size, vocab_size, num_hidden_layers
    rng = np.random.default_rng(seed)
    rnd = bf16_round if store == "BF16" else (lambda a: a)

    def n(*shape):
        out = np.empty(shape, dtype=np.float32)
        flat = out.reshape(-1)
        for s in range(0, flat.size, rng_chunk):  # bounded temporaries for big tables
            e = min(flat.size, s + rng_chunk)
            flat[s:e] = rng.standard_normal(e - s, dtype=np.float32) * np.float32(std)
        return rnd(out)

    ones = lambda *s: np.ones(s, dtype=np.float32)
    zeros = lambda *s: np.zeros(s, dtype=np.float32)
    t = {}
    t["encoder.embeddings.tok_embeddings.weight"] = n(V, D)
    t["encoder.embeddings.norm.weight"] = ones(D)
    for i in range(L):
        p = f"encoder.layers.{i}."
        if i > 0:
            t[p + "attn_norm.weight"] = ones(D)
        t[p + "attn.Wqkv.weight"] = n(3 * D, D)
        t[p + "attn.Wo.weight"] = n(D, D)
        t[p + "mlp_norm.weight"] = ones(D)
        t[p + "mlp.Wi.weight"] = n(2 * F, D)
        t[p + "mlp.Wo.weight"] = n(D, F)
    t["encoder.final_norm.weight"] = ones(D)
    if lora_r:
        t["lora_A.weight"] = n(lora_r, D)
        t["lora_B.weight"] = n(D, lora_r)
    t["type_emb.weight"] = n(3, D)
    for i in range(head_layers):
        p = f"head.layers.{i}."
        t[p + "norm1.weight"], t[p + "norm1.bias"] = ones(D), zeros(D)
        t[p + "norm2.weight"], t[p + "norm2.bias"] = ones(D), zeros(D)
        t[p + "self_attn.in_proj_weight"], t[p + "self_attn.in_proj_bias"] = n(3 * D, D), n(3 * D)
        t[p + "self_attn.out_proj.weight"], t[p + "self_attn.out_proj.bias"] = n(D, D), n(D)
        t[p + "linear1.weight"], t[p + "linear1.bias"] = n(4 * D, D), n(4 * D)
        t[p + "linear2.weight"], t[p + "linear2.bias"] = n(D, 4 * D), n(D)
    t["scorer.0.weight"] = ones(D)
    if scorer_bias:
        t["scorer.0.bias"] = zeros(D)
    t["scorer.1.weight"] = n(D, D)
    if scorer_bias:
        t["scorer.1.bias"] = n(D)
    t["scorer.3.weight"] = n(1, D)
    if scorer_bias:
        t["scorer.3.bias"] = n(1)
    t["act_head.0.weight"], t["act_head.0.bias"] = n(256, D + 4), n(256)
    t["act_head.2.weight"], t["act_head.2.bias"] = n(n_act, 256), n(n_act)
    rl = {"encoder": "synthetic", "head_layers": head_layers, "max_len": max_position_embeddings,
          "head_max_len": 192, "act_costs": {f"a{i}": 1.0 for i in range(n_act - 1)},
          "temperature": [1.0, 1.0, 1.0], "temperature_by_options": {}}
    enc = {"hidden_size": D, "num_hidden_layers": L, "num_attention_heads": num_attention_heads,
           "intermediate_size": F, "max_position_embeddings": max_position_embeddings,
           "vocab_size": V, "norm_eps": 1e-5, "norm_bias": False,
           "local_attention": local_attention,
           "layer_types": layer_types or ["full_attention"] * L,
           "rope_parameters": {"full_attention": {"rope_theta": theta_full},
                               "sliding_attention": {"rope_theta": theta_sliding}}}
    return rl, enc, t


def flat_cfg(rl: dict, enc: dict) -> dict:
    """Merge the two config files the way DecisionModel::load reads them
    (src/model.cpp:59-87)."""
    rp = enc.get("rope_parameters", {})
    n_costs = len(rl["act_costs"]) if isinstance(rl.get("act_costs"), dict) else 0
    return {
        "hidden_size": enc["hidden_size"], "num_hidden_layers": enc["num_hidden_layers"],
        "num_attention_heads": enc["num_attention_heads"],
        "intermediate_size": enc["intermediate_size"], "vocab_size": enc["vocab_size"],
        "max_position_embeddings": enc.get("max_position_embeddings", 8192),
        "norm_eps": enc.get("norm_eps", 1e-5), "local_attention": enc.get("local_attention", 0),
        "layer_types": enc.get("layer_types", []),
        "rope_theta_full": rp.get("full_attention", {}).get("rope_theta", 10000.0),
        "rope_theta_sliding": rp.get("sliding_attention", {}).get("rope_theta", 10000.0),
        "head_layers": rl.get("head_layers", 2), "n_act": n_costs + 1,
        "max_len": rl.get("max_len", 512),
    }


# ---------------------------------------------------------------- safetensors
_DT = {"F32": (np.float32, 4), "F16": (np.float16, 2), "BF16": (np.uint16, 2)}


def write_safetensors(path: str, tensors: dict, store="F32") -> None:
    """Write a .safetensors file.  ``store`` is one dtype for every tensor
    ("F32", "F16", "BF16") or a function name -> dtype; a tensor given as
    (dtype, raw ndarray) is written as is (e.g. ("F8_E4M3", uint8 codes))."""
    header, blobs, off = {}, [], 0
    for k, v in tensors.items():
        if isinstance(v, tuple):
            dt, arr = v
            raw = np.ascontiguousarray(arr).tobytes()
            shape = list(arr.shape)
        else:
            dt = store(k) if callable(store) else store
            if dt == "BF16":
                raw = bf16_bits(v).tobytes()
            elif dt == "F16":
                raw = v.astype(np.float16).tobytes()
            else:
                raw = np.ascontiguousarray(v, dtype=np.float32).tobytes()
            shape = list(v.shape)
        header[k] = {"dtype": dt, "shape": shape, "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    hj = json.dumps(header).encode()
    hj += b" " * ((8 - len(hj) % 8) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hj)))
        f.write(hj)
        for b in blobs:
            f.write(b)


def write_checkpoint(path: str, rl: dict, enc: dict, tensors: dict, store="F32") -> None:
    os.makedirs(os.path.join(path, "encoder"), exist_ok=True)
    with open(os.path.join(path, "rl_agent_config.json"), "w") as f:
        json.dump(rl, f, indent=1)
    with open(os.path.join(path, "encoder", "config.json"), "w") as f:
        json.dump(enc, f, indent=1)
    write_safetensors(os.path.join(path, "model.safetensors"), tensors, store)


# ---------------------------------------------------------------- SjModel
def make_sj_model(hidden_size: int, num_layers: int, num_heads: int, vocab_size: int,
                  intermediate_size: int | None = None, max_positions: int = 512,
                  head_layers: int = 1, head_intermediate: int | None = None,
                  norm_eps: float = 1e-5, std: float = 0.02, seed: int = 0, store: str = "F32"):
    """(sj_config, tensors) of an SjModel (src/sj_model.cpp:87-204 names and
    shapes), fp32 arrays (bf16-exact with store="BF16")."""
    D, V = hidden_size, vocab_size
    F = intermediate_size or 4 * D
    HF = head_intermediate or 4 * D
    rng = np.random.default_rng(seed)
    rnd = bf16_round if store == "BF16" else (lambda a: a)

    def n(*shape, scale=std, mean=0.0):
        v = rng.standard_normal(int(np.prod(shape)), dtype=np.float32) * np.float32(scale)
        return rnd((v + np.float32(mean)).reshape(shape))

    t = {"sj.embeddings.word.weight": n(V, D), "sj.embeddings.position.weight": n(max_positions, D),
         "sj.embeddings.norm.weight": n(D, scale=0.05, mean=1.0), "sj.embeddings.norm.bias": n(D)}

    def layer(p, ff, n1="attn_norm", n2="ffn_norm"):
        t[p + n1 + ".weight"], t[p + n1 + ".bias"] = n(D, scale=0.05, mean=1.0), n(D)
        for x in "qkvo":
            t[p + f"attn.{x}.weight"], t[p + f"attn.{x}.bias"] = n(D, D), n(D)
        t[p + n2 + ".weight"], t[p + n2 + ".bias"] = n(D, scale=0.05, mean=1.0), n(D)
        t[p + "ffn.w1.weight"], t[p + "ffn.w1.bias"] = n(ff, D), n(ff)
        t[p + "ffn.w2.weight"], t[p + "ffn.w2.bias"] = n(D, ff), n(D)

    for i in range(num_layers):
        layer(f"sj.encoder.layers.{i}.", F)
    t["sj.encoder.final_norm.weight"] = n(D, scale=0.05, mean=1.0)
    t["sj.encoder.final_norm.bias"] = n(D)
    t["sj.type_emb.weight"] = n(3, D)
    for i in range(head_layers):
        layer(f"sj.head.layers.{i}.", HF, "norm1", "norm2")
    t["sj.scorer.norm.weight"], t["sj.scorer.norm.bias"] = n(D, scale=0.05, mean=1.0), n(D)
    t["sj.scorer.w1.weight"], t["sj.scorer.w1.bias"] = n(D, D), n(D)
    t["sj.scorer.w2.weight"], t["sj.scorer.w2.bias"] = n(1, D), n(1)
    cfg = {"vocab_size": V, "hidden_size": D, "num_layers": num_layers, "num_heads": num_heads,
           "intermediate_size": F, "max_positions": max_positions, "norm_eps": norm_eps,
           "head_layers": head_layers, "head_intermediate": HF, "max_len": max_positions,
           "head_max_len": 192, "n_types": 3, "cls_id": 1, "sep_id": 2, "mask_id": 4, "pad_id": 3}
    return cfg, t


def write_sj_checkpoint(path: str, cfg: dict, tensors: dict, store="F32") -> None:
    """sj_config.json + model.safetensors, the layout SjModel checkpoints use
    (src/sj_train.cpp:180-184)."""
    os.makedirs(path, exist_ok=True)
    with open(os.path.join(path, "sj_config.json"), "w") as f:
        json.dump(cfg, f, indent=1)
    write_safetensors(os.path.join(path, "model.safetensors"), tensors, store)


FP8_PROJECTIONS = ("attn.Wqkv.weight", "attn.Wo.weight", "mlp.Wi.weight", "mlp.Wo.weight")


def fp8_tensors(tensors: dict, quantize) -> dict:
    """The tensors of an SJH_PREC_FP8W checkpoint: each encoder projection as
    ("F8_E4M3", codes) plus "<name>_scale" (fp32, one per row), from the given
    per-row quantizer (snapjudge_amd.quantize_fp8); other tensors unchanged."""
    out = {}
    for k, v in tensors.items():
        if k.startswith("encoder.layers.") and k.split(".", 3)[-1] in FP8_PROJECTIONS:
            q, sc = quantize(v)
            out[k] = ("F8_E4M3", q)
            out[k + "_scale"] = ("F32", sc.astype(np.float32))
        else:
            out[k] = v
    return out


def read_checkpoint(path: str):
    """(rl_cfg, enc_cfg, tensors as fp32), widening F16/BF16 like
    src/safetensors.cpp:109-135."""
    with open(os.path.join(path, "rl_agent_config.json")) as f:
        rl = json.load(f)
    with open(os.path.join(path, "encoder", "config.json")) as f:
        enc = json.load(f)
    with open(os.path.join(path, "model.safetensors"), "rb") as f:
        buf = f.read()
    (hlen,) = struct.unpack("<Q", buf[:8])
    hdr = json.loads(buf[8:8 + hlen])
    base = 8 + hlen
    out = {}
    for k, e in hdr.items():
        if k == "__metadata__":
            continue
        a, b = e["data_offsets"]
        raw = buf[base + a:base + b]
        if e["dtype"] == "F32":
            v = np.frombuffer(raw, dtype=np.float32)
        elif e["dtype"] == "F16":
            v = np.frombuffer(raw, dtype=np.float16).astype(np.float32)
        elif e["dtype"] == "BF16":
            v = (np.frombuffer(raw, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)
        else:
            raise ValueError(f"unsupported dtype {e['dtype']} for {k}")
        out[k] = v.reshape(e["shape"]).copy()
    return rl, enc, out


# ---------------------------------------------------------------- batches
def make_batch(B: int, L: int, lo: int, hi: int, vocab: int, seed: int = 0, pad_id: int = 0):
    """Right-padded ids [B, L] int64 and mask [B, L] with lengths ~ U[lo, hi]."""
    rng = np.random.default_rng(seed)
    lens = rng.integers(lo, hi + 1, size=B)
    ids = np.full((B, L), pad_id, dtype=np.int64)
    mask = np.zeros((B, L), dtype=np.int64)
    for b, n in enumerate(lens):
        ids[b, :n] = rng.integers(0, vocab, size=n)
        mask[b, :n] = 1
    return ids, mask, lens.astype(np.int64)


def batch_with_lens(lens, L: int, vocab: int, seed: int = 0, pad_id: int = 0):
    """Right-padded ids [B, L] and mask for the given row lengths."""
    rng = np.random.default_rng(seed)
    lens = np.asarray(lens, dtype=np.int64)
    ids = np.full((len(lens), L), pad_id, dtype=np.int64)
    mask = np.zeros((len(lens), L), dtype=np.int64)
    for b, n in enumerate(lens):
        ids[b, :n] = rng.integers(0, vocab, size=n)
        mask[b, :n] = 1
    return ids, mask, lens


def make_markers(lens, K: int, kinds, seed: int = 0):
    """Marker positions [B, K] at distinct positions in [1, n-1] (n = row length),
    marker_mask [B, K] with kinds[b] valid markers, qtype [B]."""
    rng = np.random.default_rng(seed + 1)
    B = len(lens)
    mp = np.zeros((B, K), dtype=np.int64)
    mm = np.zeros((B, K), dtype=np.uint8)
    qt = np.zeros(B, dtype=np.int64)
    for b in range(B):
        qtype, k = kinds[b]
        n = int(lens[b])
        pos = rng.choice(np.arange(1, max(n, 2)), size=min(k, max(n - 1, 1)), replace=False)
        mp[b, :len(pos)] = np.sort(pos)
        mm[b, :len(pos)] = 1
        qt[b] = qtype
    return mp, mm, qt


# marker counts per qtype (src/common.cpp:12-13): choice K in [4, 16], score
# on a 1-5 scale, noul yes/no
QTYPE_MARKERS = {0: (4, 16), 1: (5, 5), 2: (2, 2)}


def make_questions(lens, n_q: int, seed: int = 3, K: int = 16):
    """Config 5's typed questions: every sequence carries n_q questions with a
    uniform qtype (choice / score / noul) and QTYPE_MARKERS markers each.
    Returns (row_seq [U*n_q] int32, marker_pos [U*n_q, K], marker_mask, qtype):
    the rows of the reference's forward are the sequences repeated n_q times
    (one qtype per row, src/model.cpp:410-416)."""
    rng = np.random.default_rng(seed)
    lens = np.asarray(lens)
    row_seq = np.repeat(np.arange(len(lens)), n_q).astype(np.int32)
    qt = rng.integers(0, 3, size=len(row_seq))
    kinds = [(int(t), int(rng.integers(QTYPE_MARKERS[int(t)][0], QTYPE_MARKERS[int(t)][1] + 1)))
             for t in qt]
    mp, mm, qt = make_markers(lens[row_seq], K, kinds, seed=seed)
    return row_seq, mp, mm, qt
