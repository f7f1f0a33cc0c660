"""ctypes bindings of the test-only checkers (see oracle/sj_oracle.h).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the product (snapjudge_amd).

  Oracle     -- liboracle.so, the C restatement of the reference path
               (DecisionModel; SjModel through Oracle.sj_model)
  RefModel   -- oracle/_ref/libsjref.so, the reference's own CPU forward
                (DecisionModel::load/encode/forward) compiled from its sources
  RefSjModel -- the same library's SjModel::load/encode/forward
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_LIB = os.path.join(HERE, "liboracle.so")
REF_LIB = os.path.join(HERE, "_ref", "libsjref.so")

_fp = C.POINTER(C.c_float)
_i64p = C.POINTER(C.c_int64)
_u8p = C.POINTER(C.c_uint8)


def build_oracle() -> None:
    subprocess.run(["make", "-s", "-C", HERE, "all"], check=True)


def build_ref() -> bool:
    """Compile the reference sources into _ref/ when the reference tree exists."""
    ref = os.environ.get("SNAPJUDGE_REF", "/root/reference")
    if not os.path.isdir(os.path.join(ref, "src")):
        return False
    subprocess.run(["make", "-s", "-C", HERE, "ref", f"REF={ref}"], check=True)
    return True


class OrcLayer(C.Structure):
    _fields_ = [("attn_norm", _fp), ("wqkv", _fp), ("wo", _fp), ("mlp_norm", _fp),
                ("wi", _fp), ("wo2", _fp), ("window", C.c_int32), ("sliding", C.c_int32)]


class OrcHead(C.Structure):
    _fields_ = [(n, _fp) for n in ("n1w", "n1b", "n2w", "n2b", "in_w", "in_b", "out_w", "out_b",
                                   "l1w", "l1b", "l2w", "l2b")]


class OrcModel(C.Structure):
    _fields_ = [(n, C.c_int64) for n in ("D", "H", "F", "V", "n_layers", "max_pos", "n_act",
                                         "head_layers", "lora_r")] + [
        ("eps", C.c_float),
        ("emb_w", _fp), ("emb_norm", _fp), ("final_norm", _fp),
        ("rope_cos_full", _fp), ("rope_sin_full", _fp), ("rope_cos_slide", _fp),
        ("rope_sin_slide", _fp), ("layers", C.POINTER(OrcLayer)), ("lora_a", _fp),
        ("lora_b", _fp), ("type_emb", _fp), ("head", C.POINTER(OrcHead)),
        ("sc_ln_w", _fp), ("sc_ln_b", _fp), ("sc_w1", _fp), ("sc_b1", _fp), ("sc_w2", _fp),
        ("sc_b2", _fp), ("act_w1", _fp), ("act_b1", _fp), ("act_w2", _fp), ("act_b2", _fp)]


def _p(a):
    if a is None:
        return None
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(_fp)


class Oracle:
    """The C restatement (liboracle.so)."""

    def __init__(self):
        if not os.path.exists(ORACLE_LIB):
            build_oracle()
        L = C.CDLL(ORACLE_LIB)
        v = C.c_void_p
        sig = {
            "orc_layer_norm": [v, C.c_int64, C.c_int64, v, v, C.c_float, v],
            "orc_softmax_rows": [v, C.c_int64, C.c_int64],
            "orc_gemm_nt": [v, v, v, C.c_int, C.c_int64, C.c_int64, C.c_int64, v],
            "orc_gemm_geglu": [v, v, C.c_int64, C.c_int64, C.c_int64, v],
            "orc_attention": [v, v, v, v, C.c_int64, C.c_int64, C.c_int64, C.c_int64, C.c_int, v],
            "orc_embedding": [v, C.c_int64, v, C.c_int64, v],
            "orc_rope_inplace": [v, C.c_int64, v, v, C.c_int64, C.c_int64, C.c_int64],
            "orc_rope_table": [C.c_double, C.c_int64, C.c_int64, v, v],
            "orc_encode": [v, v, v, C.c_int64, C.c_int64, v],
            "orc_forward": [v, v, v, v, v, v, C.c_int64, C.c_int64, C.c_int64, v, v, v],
            "orc_calibrated_probs": [v, C.c_int, C.c_double, v],
        }
        for name, args in sig.items():
            getattr(L, name).argtypes = args
            getattr(L, name).restype = C.c_int if name in ("orc_encode", "orc_forward") else None
        L.orc_gelu_erf.argtypes = [C.c_float]
        L.orc_gelu_erf.restype = C.c_float
        L.orc_confidence_from_probs.argtypes = [v, C.c_int]
        L.orc_confidence_from_probs.restype = C.c_double
        L.orc_round4.argtypes = [C.c_double]
        L.orc_round4.restype = C.c_double
        L.orc_clamp_temperature.argtypes = [C.c_double]
        L.orc_clamp_temperature.restype = C.c_double
        self.L = L

    @staticmethod
    def _a(x):
        return x.ctypes.data_as(C.c_void_p)

    # ---- ops
    def layer_norm(self, x, w, b, eps):
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty_like(x)
        D = x.shape[-1]
        self.L.orc_layer_norm(self._a(x), x.size // D, D, self._a(w) if w is not None else None,
                              self._a(b) if b is not None else None, eps, self._a(out))
        return out

    def gelu(self, x: float) -> float:
        return self.L.orc_gelu_erf(x)

    def softmax_rows(self, z):
        z = np.array(z, np.float32, copy=True)
        self.L.orc_softmax_rows(self._a(z), z.size // z.shape[-1], z.shape[-1])
        return z

    def gemm_nt(self, a, w, bias=None, act=0):
        a = np.ascontiguousarray(a, np.float32)
        w = np.ascontiguousarray(w, np.float32)
        M, K = a.shape
        N = w.shape[0]
        out = np.empty((M, N), np.float32)
        self.L.orc_gemm_nt(self._a(a), self._a(w),
                           self._a(np.ascontiguousarray(bias, np.float32)) if bias is not None else None,
                           act, M, N, K, self._a(out))
        return out

    def gemm_geglu(self, a, wi):
        a = np.ascontiguousarray(a, np.float32)
        wi = np.ascontiguousarray(wi, np.float32)
        M, K = a.shape
        F = wi.shape[0] // 2
        out = np.empty((M, F), np.float32)
        self.L.orc_gemm_geglu(self._a(a), self._a(wi), M, F, K, self._a(out))
        return out

    def attention(self, q, k, v, lens, window):
        q, k, v = (np.ascontiguousarray(t, np.float32) for t in (q, k, v))
        B, H, L, Dh = q.shape
        lens = np.ascontiguousarray(lens, np.int64)
        out = np.empty_like(q)
        self.L.orc_attention(self._a(q), self._a(k), self._a(v), self._a(lens), B, H, L, Dh,
                             window, self._a(out))
        return out

    def rope_inplace(self, qkv, cos_t, sin_t, L, H, Dh):
        qkv = np.array(qkv, np.float32, copy=True)
        cos_t = np.ascontiguousarray(cos_t, np.float32)
        sin_t = np.ascontiguousarray(sin_t, np.float32)
        self.L.orc_rope_inplace(self._a(qkv), qkv.shape[0], self._a(cos_t), self._a(sin_t), L, H, Dh)
        return qkv

    def rope_table(self, theta, max_pos, Dh):
        c = np.empty((max_pos, Dh // 2), np.float32)
        s = np.empty_like(c)
        self.L.orc_rope_table(theta, max_pos, Dh, self._a(c), self._a(s))
        return c, s

    def calibrated_probs(self, logits, t_scale):
        logits = np.ascontiguousarray(logits, np.float32)
        p = np.empty(len(logits), np.float64)
        self.L.orc_calibrated_probs(self._a(logits), len(logits), t_scale, self._a(p))
        return p

    def confidence(self, p):
        p = np.ascontiguousarray(p, np.float64)
        return self.L.orc_confidence_from_probs(self._a(p), len(p))

    # ---- model
    def model(self, weights: dict, cfg: dict) -> "OracleModel":
        return OracleModel(self, weights, cfg)

    def sj_model(self, weights: dict, cfg: dict) -> "OracleSjModel":
        return OracleSjModel(self, weights, cfg)


class OracleModel:
    def __init__(self, orc: Oracle, weights: dict, cfg: dict):
        self.orc = orc
        w = {k: np.ascontiguousarray(v, np.float32) for k, v in weights.items()}
        D, H, L = cfg["hidden_size"], cfg["num_attention_heads"], cfg["num_hidden_layers"]
        Dh = D // H
        maxp = cfg["max_position_embeddings"]
        cf, sf = orc.rope_table(cfg["rope_theta_full"], maxp, Dh)
        cs, ss = orc.rope_table(cfg["rope_theta_sliding"], maxp, Dh)
        win = cfg["local_attention"] // 2 if cfg["local_attention"] > 0 else 0
        types = cfg.get("layer_types") or []
        layers = (OrcLayer * L)()
        for i in range(L):
            p = f"encoder.layers.{i}."
            lt = types[i] if i < len(types) else "full_attention"
            sl = lt == "sliding_attention"
            layers[i] = OrcLayer(_p(w.get(p + "attn_norm.weight")), _p(w[p + "attn.Wqkv.weight"]),
                                 _p(w[p + "attn.Wo.weight"]), _p(w[p + "mlp_norm.weight"]),
                                 _p(w[p + "mlp.Wi.weight"]), _p(w[p + "mlp.Wo.weight"]),
                                 win if sl else 0, 1 if sl else 0)
        nh = cfg["head_layers"]
        heads = (OrcHead * max(nh, 1))()
        for i in range(nh):
            p = f"head.layers.{i}."
            heads[i] = OrcHead(*[_p(w[p + s]) for s in (
                "norm1.weight", "norm1.bias", "norm2.weight", "norm2.bias",
                "self_attn.in_proj_weight", "self_attn.in_proj_bias",
                "self_attn.out_proj.weight", "self_attn.out_proj.bias",
                "linear1.weight", "linear1.bias", "linear2.weight", "linear2.bias")])
        m = OrcModel()
        m.D, m.H, m.F, m.V = D, H, cfg["intermediate_size"], cfg["vocab_size"]
        m.n_layers, m.max_pos, m.n_act, m.head_layers = L, maxp, cfg["n_act"], nh
        m.lora_r = w["lora_A.weight"].shape[0] if "lora_A.weight" in w else 0
        m.eps = cfg["norm_eps"]
        m.emb_w = _p(w["encoder.embeddings.tok_embeddings.weight"])
        m.emb_norm = _p(w["encoder.embeddings.norm.weight"])
        m.final_norm = _p(w["encoder.final_norm.weight"])
        m.rope_cos_full, m.rope_sin_full = _p(cf), _p(sf)
        m.rope_cos_slide, m.rope_sin_slide = _p(cs), _p(ss)
        m.layers = layers
        m.lora_a, m.lora_b = _p(w.get("lora_A.weight")), _p(w.get("lora_B.weight"))
        m.type_emb = _p(w["type_emb.weight"])
        m.head = heads
        m.sc_ln_w, m.sc_ln_b = _p(w["scorer.0.weight"]), _p(w.get("scorer.0.bias"))
        m.sc_w1, m.sc_b1 = _p(w["scorer.1.weight"]), _p(w.get("scorer.1.bias"))
        m.sc_w2, m.sc_b2 = _p(w["scorer.3.weight"]), _p(w.get("scorer.3.bias"))
        m.act_w1, m.act_b1 = _p(w["act_head.0.weight"]), _p(w["act_head.0.bias"])
        m.act_w2, m.act_b2 = _p(w["act_head.2.weight"]), _p(w["act_head.2.bias"])
        self._keep = (w, cf, sf, cs, ss, layers, heads)
        self.m = m
        self.D, self.n_act = D, cfg["n_act"]
        self.rope = (cf, sf, cs, ss)

    def encode(self, ids, mask):
        ids = np.ascontiguousarray(ids, np.int64)
        mask = np.ascontiguousarray(mask, np.int64)
        B, L = ids.shape
        out = np.empty((B, L, self.D), np.float32)
        a = Oracle._a
        rc = self.orc.L.orc_encode(C.byref(self.m), a(ids), a(mask), B, L, a(out))
        assert rc == 0
        return out

    def forward(self, ids, mask, marker_pos, marker_mask, qtype, hidden=False):
        ids = np.ascontiguousarray(ids, np.int64)
        mask = np.ascontiguousarray(mask, np.int64)
        mp = np.ascontiguousarray(marker_pos, np.int64)
        mm = np.ascontiguousarray(marker_mask, np.uint8)
        qt = np.ascontiguousarray(qtype, np.int64)
        B, L = ids.shape
        K = mp.shape[1]
        logits = np.empty((B, K), np.float32)
        act = np.empty((B, self.n_act), np.float32)
        h = np.empty((B, L, self.D), np.float32) if hidden else None
        a = Oracle._a
        rc = self.orc.L.orc_forward(C.byref(self.m), a(ids), a(mask), a(mp), a(mm), a(qt), B, L, K,
                                    a(logits), a(act), a(h) if h is not None else None)
        assert rc == 0
        return (logits, act, h) if hidden else (logits, act)


class RefModel:
    """The reference's own CPU forward (oracle/_ref/libsjref.so) on a checkpoint dir."""

    _L = None

    @classmethod
    def lib(cls):
        if cls._L is None:
            if not os.path.exists(REF_LIB):
                raise FileNotFoundError(REF_LIB)
            L = C.CDLL(REF_LIB)
            v = C.c_void_p
            L.sjref_last_error.restype = C.c_char_p
            L.sjref_load.argtypes = [C.c_char_p]
            L.sjref_load.restype = v
            L.sjref_free.argtypes = [v]
            L.sjref_dims.argtypes = [v, v]
            L.sjref_rope_tables.argtypes = [v, v, v, v, v]
            L.sjref_encode.argtypes = [v, v, v, C.c_int64, C.c_int64, v]
            L.sjref_forward.argtypes = [v, v, v, v, v, v, C.c_int64, C.c_int64, C.c_int64, v, v]
            L.sjref_layer_norm.argtypes = [v, C.c_int64, C.c_int64, v, v, C.c_float, v]
            L.sjref_gemm_nt.argtypes = [v, v, v, C.c_int, C.c_int64, C.c_int64, C.c_int64, v]
            L.sjref_gemm_geglu.argtypes = [v, v, C.c_int64, C.c_int64, C.c_int64, v]
            L.sjref_attention.argtypes = [v, v, v, v, C.c_int64, C.c_int64, C.c_int64, C.c_int64,
                                          C.c_int, v]
            L.sjref_rope_inplace.argtypes = [v, C.c_int64, v, v, C.c_int64, C.c_int64, C.c_int64]
            L.sjref_softmax_rows.argtypes = [v, C.c_int64, C.c_int64]
            cls._L = L
        return cls._L

    @classmethod
    def available(cls) -> bool:
        return os.path.exists(REF_LIB)

    def __init__(self, ckpt_dir: str):
        L = self.lib()
        self.h = L.sjref_load(ckpt_dir.encode())
        if not self.h:
            raise RuntimeError(L.sjref_last_error().decode())
        dims = np.zeros(8, np.int64)
        L.sjref_dims(self.h, dims.ctypes.data_as(C.c_void_p))
        (self.D, self.H, self.Dh, self.F, self.n_layers, self.n_act, self.max_pos,
         self.head_layers) = (int(x) for x in dims)

    def __del__(self):
        if getattr(self, "h", None):
            self.lib().sjref_free(self.h)
            self.h = None

    def rope_tables(self):
        n = (self.max_pos, self.Dh // 2)
        t = [np.empty(n, np.float32) for _ in range(4)]
        self.lib().sjref_rope_tables(self.h, *[x.ctypes.data_as(C.c_void_p) for x in t])
        return t

    def encode(self, ids, mask):
        ids = np.ascontiguousarray(ids, np.int64)
        mask = np.ascontiguousarray(mask, np.int64)
        B, L = ids.shape
        out = np.empty((B, L, self.D), np.float32)
        a = Oracle._a
        if self.lib().sjref_encode(self.h, a(ids), a(mask), B, L, a(out)) != 0:
            raise RuntimeError(self.lib().sjref_last_error().decode())
        return out

    def forward(self, ids, mask, marker_pos, marker_mask, qtype):
        ids = np.ascontiguousarray(ids, np.int64)
        mask = np.ascontiguousarray(mask, np.int64)
        mp = np.ascontiguousarray(marker_pos, np.int64)
        mm = np.ascontiguousarray(marker_mask, np.uint8)
        qt = np.ascontiguousarray(qtype, np.int64)
        B, L = ids.shape
        K = mp.shape[1]
        logits = np.empty((B, K), np.float32)
        act = np.empty((B, self.n_act), np.float32)
        a = Oracle._a
        if self.lib().sjref_forward(self.h, a(ids), a(mask), a(mp), a(mm), a(qt), B, L, K,
                                    a(logits), a(act)) != 0:
            raise RuntimeError(self.lib().sjref_last_error().decode())
        return logits, act


# ---------------------------------------------------------------- SjModel
class OrcSjLayer(C.Structure):
    _fields_ = [(n, _fp) for n in ("an_w", "an_b", "q_w", "q_b", "k_w", "k_b", "v_w", "v_b",
                                   "o_w", "o_b", "fn_w", "fn_b", "w1_w", "w1_b", "w2_w", "w2_b")]


class OrcSjModel(C.Structure):
    _fields_ = [(n, C.c_int64) for n in ("D", "H", "F", "V", "n_layers", "max_pos", "head_layers",
                                         "head_ff")] + [
        ("eps", C.c_float), ("word_emb", _fp), ("pos_emb", _fp), ("emb_norm_w", _fp),
        ("emb_norm_b", _fp), ("layers", C.POINTER(OrcSjLayer)), ("final_norm_w", _fp),
        ("final_norm_b", _fp), ("type_emb", _fp), ("head", C.POINTER(OrcSjLayer)),
        ("sc_n_w", _fp), ("sc_n_b", _fp), ("sc_w1", _fp), ("sc_b1", _fp), ("sc_w2", _fp),
        ("sc_b2", _fp)]


def _sj_layer(w, p, n1, n2):
    g = lambda s: _p(w[p + s])
    return OrcSjLayer(g(n1 + ".weight"), g(n1 + ".bias"),
                      g("attn.q.weight"), g("attn.q.bias"), g("attn.k.weight"), g("attn.k.bias"),
                      g("attn.v.weight"), g("attn.v.bias"), g("attn.o.weight"), g("attn.o.bias"),
                      g(n2 + ".weight"), g(n2 + ".bias"), g("ffn.w1.weight"), g("ffn.w1.bias"),
                      g("ffn.w2.weight"), g("ffn.w2.bias"))


class OracleSjModel:
    """The C restatement of SjModel (orc_sj_encode / orc_sj_forward) on a
    tensor dict with the sj.* names and an sj_config dict."""

    def __init__(self, orc: "Oracle", weights: dict, cfg: dict):
        L = orc.L
        v = C.c_void_p
        L.orc_sj_encode.argtypes = [v, v, v, C.c_int64, C.c_int64, v]
        L.orc_sj_encode.restype = C.c_int
        L.orc_sj_forward.argtypes = [v, v, v, v, v, v, C.c_int64, C.c_int64, C.c_int64, v, v, v]
        L.orc_sj_forward.restype = C.c_int
        self.orc = orc
        w = {k: np.ascontiguousarray(x, np.float32) for k, x in weights.items()}
        D, nl, nh = cfg["hidden_size"], cfg["num_layers"], cfg.get("head_layers", 1)
        layers = (OrcSjLayer * nl)(*[_sj_layer(w, f"sj.encoder.layers.{i}.", "attn_norm", "ffn_norm")
                                     for i in range(nl)])
        head = (OrcSjLayer * max(nh, 1))(*[_sj_layer(w, f"sj.head.layers.{i}.", "norm1", "norm2")
                                           for i in range(nh)])
        m = OrcSjModel()
        m.D, m.H, m.F, m.V = D, cfg["num_heads"], cfg.get("intermediate_size", 4 * D), cfg["vocab_size"]
        m.n_layers, m.max_pos = nl, cfg.get("max_positions", 512)
        m.head_layers, m.head_ff = nh, cfg.get("head_intermediate", 4 * D)
        m.eps = cfg.get("norm_eps", 1e-5)
        m.word_emb, m.pos_emb = _p(w["sj.embeddings.word.weight"]), _p(w["sj.embeddings.position.weight"])
        m.emb_norm_w, m.emb_norm_b = _p(w["sj.embeddings.norm.weight"]), _p(w["sj.embeddings.norm.bias"])
        m.layers, m.head = layers, head
        m.final_norm_w = _p(w["sj.encoder.final_norm.weight"])
        m.final_norm_b = _p(w["sj.encoder.final_norm.bias"])
        m.type_emb = _p(w["sj.type_emb.weight"])
        m.sc_n_w, m.sc_n_b = _p(w["sj.scorer.norm.weight"]), _p(w["sj.scorer.norm.bias"])
        m.sc_w1, m.sc_b1 = _p(w["sj.scorer.w1.weight"]), _p(w["sj.scorer.w1.bias"])
        m.sc_w2, m.sc_b2 = _p(w["sj.scorer.w2.weight"]), _p(w["sj.scorer.w2.bias"])
        self._keep = (w, layers, head)
        self.m, self.D = m, D

    def encode(self, ids, mask):
        ids = np.ascontiguousarray(ids, np.int64)
        mask = np.ascontiguousarray(mask, np.int64)
        B, L = ids.shape
        out = np.empty((B, L, self.D), np.float32)
        a = Oracle._a
        assert self.orc.L.orc_sj_encode(C.byref(self.m), a(ids), a(mask), B, L, a(out)) == 0
        return out

    def forward(self, ids, mask, marker_pos, marker_mask, qtype, hidden=False):
        ids = np.ascontiguousarray(ids, np.int64)
        mask = np.ascontiguousarray(mask, np.int64)
        mp = np.ascontiguousarray(marker_pos, np.int64)
        mm = np.ascontiguousarray(marker_mask, np.uint8)
        qt = np.ascontiguousarray(qtype, np.int64)
        B, L = ids.shape
        K = mp.shape[1]
        logits = np.empty((B, K), np.float32)
        act = np.empty((B, 2), np.float32)
        h = np.empty((B, L, self.D), np.float32) if hidden else None
        a = Oracle._a
        assert self.orc.L.orc_sj_forward(C.byref(self.m), a(ids), a(mask), a(mp), a(mm), a(qt), B, L,
                                         K, a(logits), a(act), a(h) if h is not None else None) == 0
        return (logits, act, h) if hidden else (logits, act)


class RefSjModel:
    """The reference's own SjModel (oracle/_ref/libsjref.so) on a checkpoint
    dir with sj_config.json + model.safetensors."""

    def __init__(self, ckpt_dir: str):
        L = RefModel.lib()
        v = C.c_void_p
        L.sjref_sj_load.argtypes = [C.c_char_p]
        L.sjref_sj_load.restype = v
        L.sjref_sj_free.argtypes = [v]
        L.sjref_sj_encode.argtypes = [v, v, v, C.c_int64, C.c_int64, v]
        L.sjref_sj_forward.argtypes = [v, v, v, v, v, v, C.c_int64, C.c_int64, C.c_int64, v, v]
        self.L = L
        self.h = L.sjref_sj_load(ckpt_dir.encode())
        if not self.h:
            raise RuntimeError(L.sjref_last_error().decode())
        import json
        with open(os.path.join(ckpt_dir, "sj_config.json")) as f:
            self.D = json.load(f)["hidden_size"]

    def __del__(self):
        if getattr(self, "h", None):
            self.L.sjref_sj_free(self.h)
            self.h = None

    def encode(self, ids, mask):
        ids = np.ascontiguousarray(ids, np.int64)
        mask = np.ascontiguousarray(mask, np.int64)
        B, L = ids.shape
        out = np.empty((B, L, self.D), np.float32)
        a = Oracle._a
        if self.L.sjref_sj_encode(self.h, a(ids), a(mask), B, L, a(out)) != 0:
            raise RuntimeError(self.L.sjref_last_error().decode())
        return out

    def forward(self, ids, mask, marker_pos, marker_mask, qtype):
        ids = np.ascontiguousarray(ids, np.int64)
        mask = np.ascontiguousarray(mask, np.int64)
        mp = np.ascontiguousarray(marker_pos, np.int64)
        mm = np.ascontiguousarray(marker_mask, np.uint8)
        qt = np.ascontiguousarray(qtype, np.int64)
        B, L = ids.shape
        K = mp.shape[1]
        logits = np.empty((B, K), np.float32)
        act = np.empty((B, 2), np.float32)
        a = Oracle._a
        if self.L.sjref_sj_forward(self.h, a(ids), a(mask), a(mp), a(mm), a(qt), B, L, K,
                                   a(logits), a(act)) != 0:
            raise RuntimeError(self.L.sjref_last_error().decode())
        return logits, act
