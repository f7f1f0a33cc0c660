"""snapjudge_amd -- MI355X (gfx950) encoder forward for snapjudge's DecisionModel.

The product is the native library ``libsnapjudge_hip.so`` (HIP kernels + C++
engine + C ABI, declared in ``include/snapjudge_hip.h``).  This module is a
thin ctypes binding over that C ABI, used by the tests and the benchmark the
way the reference's Go/C bindings use its engine ABI.  There is no CPU
fallback: if the library is missing or no gfx950 device is visible, calls
raise.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libsnapjudge_hip.so")

SJH_F32, SJH_BF16 = 0, 1
SJH_PREC_FP32, SJH_PREC_BF16, SJH_PREC_FP8W = 0, 1, 2

_fp = C.POINTER(C.c_float)
_i64p = C.POINTER(C.c_int64)
_i32p = C.POINTER(C.c_int32)
_u8p = C.POINTER(C.c_uint8)


class LayerDesc(C.Structure):
    _fields_ = [("attn_norm", _fp), ("wqkv", _fp), ("wo", _fp), ("mlp_norm", _fp),
                ("wi", _fp), ("wo2", _fp), ("window", C.c_int32), ("sliding", C.c_int32)]


class HeadDesc(C.Structure):
    _fields_ = [(n, _fp) for n in ("n1w", "n1b", "n2w", "n2b", "in_w", "in_b", "out_w",
                                   "out_b", "l1w", "l1b", "l2w", "l2b")]


class ModelDesc(C.Structure):
    _fields_ = [
        ("hidden_size", C.c_int32), ("num_heads", C.c_int32), ("intermediate_size", C.c_int32),
        ("vocab_size", C.c_int32), ("num_layers", C.c_int32), ("max_position", C.c_int32),
        ("n_act", C.c_int32), ("head_layers", C.c_int32), ("lora_r", C.c_int32),
        ("norm_eps", C.c_float), ("rope_theta_full", C.c_double),
        ("rope_theta_sliding", C.c_double),
        ("emb_w", _fp), ("emb_norm", _fp), ("final_norm", _fp),
        ("rope_cos_full", _fp), ("rope_sin_full", _fp),
        ("rope_cos_slide", _fp), ("rope_sin_slide", _fp),
        ("layers", C.POINTER(LayerDesc)), ("lora_a", _fp), ("lora_b", _fp),
        ("type_emb", _fp), ("head", C.POINTER(HeadDesc)),
        ("sc_ln_w", _fp), ("sc_ln_b", _fp), ("sc_w1", _fp), ("sc_b1", _fp),
        ("sc_w2", _fp), ("sc_b2", _fp),
        ("act_w1", _fp), ("act_b1", _fp), ("act_w2", _fp), ("act_b2", _fp),
    ]


class Options(C.Structure):
    _fields_ = [("precision", C.c_int32), ("max_len", C.c_int32), ("use_graphs", C.c_int32),
                ("pad_rows", C.c_int32), ("device", C.c_int32), ("fuse_ln", C.c_int32),
                ("fuse_attn_wo", C.c_int32)]


# Every symbol include/snapjudge_hip.h declares, with its ctypes signature.
_SIGS = {
    "sjh_last_error": (C.c_char_p, []),
    "sjh_version": (C.c_int, []),
    "sjh_default_options": (None, [C.POINTER(Options)]),
    "sjh_model_create": (C.c_int, [C.POINTER(ModelDesc), C.POINTER(Options), C.POINTER(C.c_void_p)]),
    "sjh_model_destroy": (None, [C.c_void_p]),
    "sjh_model_load": (C.c_int, [C.c_char_p, C.POINTER(Options), C.POINTER(C.c_void_p)]),
    "sjh_model_encode": (C.c_int, [C.c_void_p, _i64p, _i64p, C.c_int32, C.c_int32, _fp]),
    "sjh_model_forward": (C.c_int, [C.c_void_p, _i64p, _i64p, _i64p, _u8p, _i64p, C.c_int32,
                                    C.c_int32, C.c_int32, _fp, _fp]),
    "sjh_model_encode_device": (C.c_int, [C.c_void_p, C.c_void_p, _i32p, C.c_int32, C.c_void_p,
                                          C.c_void_p]),
    "sjh_model_forward_shared": (C.c_int, [C.c_void_p, _i64p, _i64p, C.c_int32, C.c_int32, _i32p,
                                           _i64p, _u8p, _i64p, C.c_int32, C.c_int32, _fp, _fp]),
    "sjh_model_encode_device_noalloc": (C.c_int, [C.c_void_p, C.c_void_p, _i32p, C.c_int32,
                                                  C.c_void_p, C.c_void_p]),
    "sjh_model_info": (C.c_int, [C.c_void_p, _i32p, _i32p, _i32p, _i32p]),
    "sjh_model_graph_stats": (C.c_int, [C.c_void_p, _i32p, _i64p, _i64p]),
    "sjh_model_profile": (C.c_int, [C.c_void_p, C.c_int32]),
    "sjh_model_profile_read": (C.c_int, [C.c_void_p, C.c_int32, C.POINTER(C.c_char_p),
                                         C.POINTER(C.c_double), _i64p, _i32p]),
    "sjh_gemm": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32, C.c_int32,
                           C.c_int32, C.c_int32, C.c_int32, C.c_void_p]),
    "sjh_quantize_fp8": (C.c_int, [_fp, C.c_int64, C.c_int64, _u8p, _fp]),
    "sjh_gemm_fp8w": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_void_p]),
    "sjh_gemm_geglu": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32, C.c_int32,
                                 C.c_int32, C.c_int32, C.c_void_p]),
    "sjh_gemm_residual": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32, C.c_int32,
                                    C.c_int32, C.c_int32, C.c_void_p]),
    "sjh_gemm_qkv_rope": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                    C.c_void_p, C.c_int32, C.c_int32, C.c_int32, C.c_int32,
                                    C.c_int32, C.c_int32, C.c_void_p]),
    "sjh_add_ln": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                             C.c_int32, C.c_int32, C.c_float, C.c_int32, C.c_int32, C.c_int32,
                             C.c_void_p]),
    "sjh_rope": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64, C.c_int32, C.c_int32,
                           C.c_int32, C.c_int32, C.c_void_p]),
    "sjh_attn": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32, C.c_int32, C.c_int32,
                           C.c_int32, C.c_int32, C.c_int32, C.c_void_p]),
    "sjh_attn_log2": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32, C.c_int32, C.c_int32,
                                C.c_int32, C.c_void_p]),
    "sjh_embed_ln": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32,
                               C.c_int32, C.c_float, C.c_int32, C.c_void_p]),
}

_LIB = None


def lib() -> C.CDLL:
    """Load libsnapjudge_hip.so (built in-tree); raise if it is missing."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with "
                               "`python -c 'import __graft_entry__ as g; g.build()'`")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = L
    return _LIB


class SjhError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


def check(rc: int) -> None:
    if rc != 0:
        raise SjhError(rc, lib().sjh_last_error().decode(errors="replace"))


def _ptr(a: np.ndarray | None):
    if a is None:
        return None
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"], "weights must be C-contiguous fp32"
    return a.ctypes.data_as(_fp)


def quantize_fp8(w: np.ndarray):
    """Per-row e4m3 codes and fp32 scales of a 2-D fp32 matrix (sjh_quantize_fp8)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, cols = w.shape
    q = np.empty((rows, cols), dtype=np.uint8)
    sc = np.empty(rows, dtype=np.float32)
    check(lib().sjh_quantize_fp8(w.ctypes.data_as(_fp), rows, cols, q.ctypes.data_as(_u8p),
                                 sc.ctypes.data_as(_fp)))
    return q, sc


FP8_PROJECTIONS = ("attn.Wqkv.weight", "attn.Wo.weight", "mlp.Wi.weight", "mlp.Wo.weight")


def fp8_dequantized(weights: "dict") -> "dict":
    """The weights an SJH_PREC_FP8W model computes with: every encoder
    projection replaced by decode(q) * scale of its sjh_quantize_fp8 codes (the
    reference forward on this dict is the fp8 model's oracle)."""
    table = fp8_e4m3_table()
    out = dict(weights)
    for k, v in weights.items():
        if k.startswith("encoder.layers.") and k.split(".", 3)[-1] in FP8_PROJECTIONS:
            q, sc = quantize_fp8(v)
            out[k] = (table[q] * sc[:, None]).astype(np.float32)
    return out


def fp8_e4m3_table() -> np.ndarray:
    """Value of each OCP e4m3fn code (bias 7, 3 mantissa bits, S.1111.111 NaN)."""
    c = np.arange(256)
    sign = np.where(c & 0x80, -1.0, 1.0)
    e, m = (c >> 3) & 15, c & 7
    v = np.where(e == 0, m * 2.0 ** -9, (1 + m / 8) * 2.0 ** (e - 7.0))
    v = np.where((e == 15) & (m == 7), np.nan, v)
    return (sign * v).astype(np.float32)


class Model:
    """A DecisionModel staged on the GPU (sjh_model_create)."""

    def __init__(self, weights: "dict", cfg: "dict", precision: int = SJH_PREC_BF16,
                 max_len: int = 0, use_graphs: bool = True, pad_rows: bool = False,
                 device: int = 0, fuse_ln: int = 1, fuse_attn_wo: int = 1):
        self._keep = []
        w = {k: np.ascontiguousarray(v, dtype=np.float32) for k, v in weights.items()}
        self._keep.append(w)
        D, L = cfg["hidden_size"], cfg["num_hidden_layers"]
        layers = (LayerDesc * L)()
        win = cfg.get("local_attention", 0) // 2 if cfg.get("local_attention", 0) > 0 else 0
        types = cfg.get("layer_types") or []
        for i in range(L):
            p = f"encoder.layers.{i}."
            lt = types[i] if i < len(types) else "full_attention"
            layers[i] = LayerDesc(_ptr(w.get(p + "attn_norm.weight")), _ptr(w[p + "attn.Wqkv.weight"]),
                                  _ptr(w[p + "attn.Wo.weight"]), _ptr(w[p + "mlp_norm.weight"]),
                                  _ptr(w[p + "mlp.Wi.weight"]), _ptr(w[p + "mlp.Wo.weight"]),
                                  win if lt == "sliding_attention" else 0,
                                  1 if lt == "sliding_attention" else 0)
        nh = cfg.get("head_layers", 0)
        heads = (HeadDesc * max(nh, 1))()
        for i in range(nh):
            p = f"head.layers.{i}."
            heads[i] = HeadDesc(*[_ptr(w[p + s]) for s in (
                "norm1.weight", "norm1.bias", "norm2.weight", "norm2.bias",
                "self_attn.in_proj_weight", "self_attn.in_proj_bias",
                "self_attn.out_proj.weight", "self_attn.out_proj.bias",
                "linear1.weight", "linear1.bias", "linear2.weight", "linear2.bias")])
        self._keep += [layers, heads]
        lora_r = w["lora_A.weight"].shape[0] if "lora_A.weight" in w else 0
        d = ModelDesc()
        d.hidden_size, d.num_heads = D, cfg["num_attention_heads"]
        d.intermediate_size, d.vocab_size = cfg["intermediate_size"], cfg["vocab_size"]
        d.num_layers, d.max_position = L, cfg.get("max_position_embeddings", 8192)
        d.n_act, d.head_layers, d.lora_r = cfg.get("n_act", 1), nh, lora_r
        d.norm_eps = cfg.get("norm_eps", 1e-5)
        d.rope_theta_full = cfg.get("rope_theta_full", 10000.0)
        d.rope_theta_sliding = cfg.get("rope_theta_sliding", 10000.0)
        d.emb_w = _ptr(w["encoder.embeddings.tok_embeddings.weight"])
        d.emb_norm = _ptr(w["encoder.embeddings.norm.weight"])
        d.final_norm = _ptr(w["encoder.final_norm.weight"])
        d.layers = layers
        d.lora_a = _ptr(w.get("lora_A.weight"))
        d.lora_b = _ptr(w.get("lora_B.weight"))
        d.type_emb = _ptr(w["type_emb.weight"])
        d.head = heads
        d.sc_ln_w, d.sc_ln_b = _ptr(w["scorer.0.weight"]), _ptr(w.get("scorer.0.bias"))
        d.sc_w1, d.sc_b1 = _ptr(w["scorer.1.weight"]), _ptr(w.get("scorer.1.bias"))
        d.sc_w2, d.sc_b2 = _ptr(w["scorer.3.weight"]), _ptr(w.get("scorer.3.bias"))
        d.act_w1, d.act_b1 = _ptr(w["act_head.0.weight"]), _ptr(w["act_head.0.bias"])
        d.act_w2, d.act_b2 = _ptr(w["act_head.2.weight"]), _ptr(w["act_head.2.bias"])
        opt = Options(precision, max_len, 1 if use_graphs else 0, 1 if pad_rows else 0, device,
                      int(fuse_ln), int(fuse_attn_wo))
        h = C.c_void_p()
        check(lib().sjh_model_create(C.byref(d), C.byref(opt), C.byref(h)))
        self._h = h
        self._keep = None  # the library copied everything it needs
        self.D = D
        self.n_act = d.n_act
        self.precision = precision

    @classmethod
    def load(cls, path: str, precision: int = SJH_PREC_BF16, max_len: int = 0,
             use_graphs: bool = True, pad_rows: bool = False, device: int = 0,
             fuse_ln: int = 1, fuse_attn_wo: int = 1) -> "Model":
        """A checkpoint directory loaded straight to the device (sjh_model_load):
        a DecisionModel (rl_agent_config.json + encoder/config.json) or an
        SjModel (sj_config.json), with model.safetensors."""
        self = cls.__new__(cls)
        opt = Options(precision, max_len, 1 if use_graphs else 0, 1 if pad_rows else 0, device,
                      int(fuse_ln), int(fuse_attn_wo))
        h = C.c_void_p()
        check(lib().sjh_model_load(os.fsencode(path), C.byref(opt), C.byref(h)))
        self._h = h
        self._keep = None
        D, n_act = C.c_int32(), C.c_int32()
        check(lib().sjh_model_info(h, C.byref(D), None, C.byref(n_act), None))
        self.D, self.n_act, self.precision = D.value, n_act.value, precision
        return self

    def close(self):
        if getattr(self, "_h", None):
            lib().sjh_model_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def encode(self, ids: np.ndarray, mask: np.ndarray) -> np.ndarray:
        ids = np.ascontiguousarray(ids, dtype=np.int64)
        mask = np.ascontiguousarray(mask, dtype=np.int64)
        B, L = ids.shape
        out = np.empty((B, L, self.D), dtype=np.float32)
        check(lib().sjh_model_encode(self._h, ids.ctypes.data_as(_i64p), mask.ctypes.data_as(_i64p),
                                     B, L, out.ctypes.data_as(_fp)))
        return out

    def forward(self, ids, mask, marker_pos, marker_mask, qtype):
        ids = np.ascontiguousarray(ids, dtype=np.int64)
        mask = np.ascontiguousarray(mask, dtype=np.int64)
        mp = np.ascontiguousarray(marker_pos, dtype=np.int64)
        mm = np.ascontiguousarray(marker_mask, dtype=np.uint8)
        qt = np.ascontiguousarray(qtype, dtype=np.int64)
        B, L = ids.shape
        K = mp.shape[1]
        logits = np.empty((B, K), dtype=np.float32)
        act = np.empty((B, self.n_act), dtype=np.float32)
        check(lib().sjh_model_forward(self._h, ids.ctypes.data_as(_i64p), mask.ctypes.data_as(_i64p),
                                      mp.ctypes.data_as(_i64p), mm.ctypes.data_as(_u8p),
                                      qt.ctypes.data_as(_i64p), B, L, K,
                                      logits.ctypes.data_as(_fp), act.ctypes.data_as(_fp)))
        return logits, act

    def forward_shared(self, ids, mask, row_seq, marker_pos, marker_mask, qtype):
        """forward on len(row_seq) rows; row b is sequence row_seq[b] of ids/mask."""
        ids = np.ascontiguousarray(ids, dtype=np.int64)
        mask = np.ascontiguousarray(mask, dtype=np.int64)
        rs = np.ascontiguousarray(row_seq, dtype=np.int32)
        mp = np.ascontiguousarray(marker_pos, dtype=np.int64)
        mm = np.ascontiguousarray(marker_mask, dtype=np.uint8)
        qt = np.ascontiguousarray(qtype, dtype=np.int64)
        U, L = ids.shape
        B, K = mp.shape
        assert len(rs) == B and mm.shape == (B, K) and len(qt) == B
        logits = np.empty((B, K), dtype=np.float32)
        act = np.empty((B, self.n_act), dtype=np.float32)
        check(lib().sjh_model_forward_shared(self._h, ids.ctypes.data_as(_i64p),
                                             mask.ctypes.data_as(_i64p), U, L,
                                             rs.ctypes.data_as(_i32p), mp.ctypes.data_as(_i64p),
                                             mm.ctypes.data_as(_u8p), qt.ctypes.data_as(_i64p),
                                             B, K, logits.ctypes.data_as(_fp),
                                             act.ctypes.data_as(_fp)))
        return logits, act

    def encode_device(self, d_ids: int, lens: np.ndarray, d_hidden: int, stream: int = 0):
        lens = np.ascontiguousarray(lens, dtype=np.int32)
        check(lib().sjh_model_encode_device(self._h, C.c_void_p(d_ids), lens.ctypes.data_as(_i32p),
                                            len(lens), C.c_void_p(d_hidden), C.c_void_p(stream)))

    def encode_device_noalloc(self, d_ids: int, lens: np.ndarray, d_hidden: int, stream: int = 0):
        lens = np.ascontiguousarray(lens, dtype=np.int32)
        check(lib().sjh_model_encode_device_noalloc(self._h, C.c_void_p(d_ids),
                                                    lens.ctypes.data_as(_i32p), len(lens),
                                                    C.c_void_p(d_hidden), C.c_void_p(stream)))

    def graph_stats(self) -> dict:
        n, cap, rep = C.c_int32(), C.c_int64(), C.c_int64()
        check(lib().sjh_model_graph_stats(self._h, C.byref(n), C.byref(cap), C.byref(rep)))
        return {"cached": n.value, "captures": cap.value, "replays": rep.value}

    def profile(self, on: bool):
        check(lib().sjh_model_profile(self._h, 1 if on else 0))

    def profile_read(self) -> dict:
        n = 64
        names = (C.c_char_p * n)()
        ms = (C.c_double * n)()
        cnt = (C.c_int64 * n)()
        got = C.c_int32()
        check(lib().sjh_model_profile_read(self._h, n, names, ms, cnt, C.byref(got)))
        return {names[i].decode(): (ms[i], cnt[i]) for i in range(got.value)}
