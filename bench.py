"""Benchmark: snapjudge encoder forward on one MI355X.

Workload: the 22-layer / hidden 768 / 12x64 heads /
GEGLU 1152 / vocab 50368 ModernBERT-style DecisionModel encoder with
random N(0, 0.02) bf16 weights (seed 0), batch 64 x seq 512, row lengths
~ U[64, 512] (seed 1), right-padded.  One step = one encoder forward
(DecisionModel::encode, src/model.cpp:222-307) over the batch, with the token
ids already resident in HBM (sjh_model_encode_device).

value = valid (non-pad) encoder tokens per second over the timed steps (the
forward replayed as a captured hipGraph).  Also reported:
  roofline      -- the kernel with the most time per step.  Kernels are
                   grouped as rocprofv3 names them (one instantiation each:
                   QKV projection + RoPE, Wi + GEGLU, the residual GEMM that
                   serves both Wo and Wo2, attention, the fp32 -> bf16 layer
                   norm); achieved = algorithmic FLOPs (or bytes) per launch /
                   mean launch time, measured with a hipEvent pair around every
                   launch on the model's stream over a second pass of the same
                   steps, launched kernel by kernel; traffic = HBM bytes per
                   launch from the committed rocprofv3 counter summary.
                   `kernels` lists the same figures for every group;
  gemm_all_tflops -- all four projection GEMMs together;
  attention_mfma_frac -- the attention kernel's algorithmic FLOPs
                   (4*D*sum(n^2) per layer) over its time, vs bf16 peak;
  p50_latency_b1_ms -- config 2 (batch 1, seq 128, no padding) encoder
                   latency, hipGraph replay, p50 of 50, with the per-kernel
                   times of one launch-by-launch pass;
  b1_varlen     -- batch 1 with a new length ~ U[64, 128] every call: p50
                   and mean latency including the graph captures (one per
                   shape bucket);
  cpu_baseline  -- the reference's own CPU forward (oracle/_ref, compiled
                   from its sources, no-BLAS build) on a bounded sample of the
                   same workload, extrapolated by layers;
  other_configs -- configs 4 (batch 4 x seq 8192) and 5 (28-layer/1024
                   encoder with fp8 e4m3 weights, batch 32 x seq 1024): valid
                   tokens/s and per-kernel times, same method; for config 5
                   also the decision step over 8 typed questions per sequence
                   (256 rows, forward_shared, host arrays in and out).
--legs selects the legs (default all: cfg3,b1,cfg4,cfg5,cpu); a run without
cfg3 prints the other legs with a null value (profiling runs only).  The
extra leg `blas` (never by default) times config 3's four projection shapes
as plain GEMMs with torch.matmul (hipBLASLt) beside sjh_gemm.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "encoder tokens/sec at B64×S512 bf16 (1 GPU); attention MFMA % peak; p50 latency at B1"
PEAK_BF16_TFLOPS = 2500.0
GEMM_NAMES = ("gemm_qkv_rope", "gemm_wo_resid", "gemm_wi_geglu", "gemm_wo2_resid", "gemm_wo_resid_ln",
              "gemm_wo2_resid_ln")


PEAK_HBM_GBS = 8000.0
LEGS = ("cfg3", "b1", "cfg4", "cfg5", "cpu")
EXTRA_LEGS = ("blas",)  # run only when named

# rocprofv3 --pmc summary of config 3 (FETCH_SIZE and WRITE_SIZE passes, each
# scaled by the same counter on a plain copy of known size): lines
# "traffic_bytes_per_launch[<group>] = <bytes>"
CFG3_TRAFFIC = os.path.join(ROOT, "profiles", "encoder_cfg3_traffic.md")


def measured_traffic(path, group):
    """HBM bytes per launch of a kernel group recorded by the counter runs, or None."""
    import re

    try:
        with open(path) as f:
            m = re.search(r"traffic_bytes_per_launch\[" + re.escape(group) + r"\]\s*=\s*([0-9]+)", f.read())
    except OSError:
        return None
    return int(m.group(1)) if m else None


# Kernel groups: (event roles, rocprofv3 kernel, bound).  The roles of a group
# launch one kernel instantiation (rocprofv3 reports them as one kernel).
KERNEL_GROUPS = {
    "gemm_qkv_rope": (("gemm_qkv_rope",), "gemm_bf16_pers_kernel<256, 256, 4, 4, 2, 64, false, 2, "
                      "unsigned short, 0> (QKV projection + RoPE epilogue)", "mfma"),
    "gemm_wi_geglu": (("gemm_wi_geglu",), "gemm_bf16_pers_kernel<256, 256, 4, 4, 2, 64, false, 3, "
                      "unsigned short, 0> (Wi projection + GEGLU epilogue)", "mfma"),
    "gemm_resid_ln": (("gemm_wo_resid_ln", "gemm_wo2_resid_ln"), "gemm_bf16_pers_kernel<256, 256, 4, 4, "
                      "2, 64, false, 1, float, 3> (Wo and Wo2 projections + residual + LayerNorm epilogue)",
                      "mfma"),
    "gemm_resid": (("gemm_wo_resid", "gemm_wo2_resid"), "gemm_bf16_pers_kernel<256, 256, 4, 4, 2, "
                   "64, false, 1, float, 0> (Wo and Wo2 projections + residual epilogue)", "mfma"),
    "attention": (("attention",), "attn_bf16_mfma_kernel (varlen flash attention)", "mfma"),
    "layer_norm": (("attn_norm", "mlp_norm", "final_norm"), "ln_vec_kernel<3, true, float, NoRes, "
                   "unsigned short> (fp32 rows -> bf16 LayerNorm)", "hbm"),
}


def role_work(role, T, D, F, sum_n2):
    """Algorithmic work of one launch of an event role: (FLOPs, HBM bytes) over
    valid tokens -- every operand read once, every output written once."""
    return {
        "gemm_qkv_rope": (2.0 * T * D * 3 * D, 2.0 * (T * D + 3 * D * D + 3 * T * D)),
        "gemm_wi_geglu": (2.0 * T * D * 2 * F, 2.0 * (T * D + 2 * F * D + T * F)),
        "gemm_wo_resid": (2.0 * T * D * D, 2.0 * (T * D + D * D) + 8.0 * T * D),
        "gemm_wo2_resid": (2.0 * T * F * D, 2.0 * (T * F + D * F) + 8.0 * T * D),
        "gemm_wo_resid_ln": (2.0 * T * D * D, 2.0 * (T * D + D * D) + 10.0 * T * D),
        "gemm_wo2_resid_ln": (2.0 * T * F * D, 2.0 * (T * F + D * F) + 10.0 * T * D),
        "attention": (4.0 * D * sum_n2, 8.0 * T * D),
        "attn_norm": (0.0, 6.0 * T * D),
        "mlp_norm": (0.0, 6.0 * T * D),
        "final_norm": (0.0, 8.0 * T * D),
    }[role]


def kernel_table(prof, steps, T, D, F, NL, lens):
    """Per kernel group: launches and ms per step, mean launch time, and the
    algorithmic rate against its roofline (MFMA FLOPs for the GEMMs and
    attention, HBM bytes for the layer norms), with the other rate beside it.
    Work per launch is role_work's, averaged over the group's launches."""
    sum_n2 = float((lens.astype(np.float64) ** 2).sum())
    out = {}
    for grp, (roles, kname, bound) in KERNEL_GROUPS.items():
        ms = sum(prof[r][0] for r in roles if r in prof)
        n = sum(prof[r][1] for r in roles if r in prof)
        if n == 0:
            continue
        per_step = n // steps
        flops = sum(role_work(r, T, D, F, sum_n2)[0] * prof[r][1] for r in roles if r in prof) / n
        nbytes = sum(role_work(r, T, D, F, sum_n2)[1] * prof[r][1] for r in roles if r in prof) / n
        avg_s = ms / 1e3 / n
        tflops, gbs = flops / avg_s / 1e12, nbytes / avg_s / 1e9
        peak = PEAK_HBM_GBS if bound == "hbm" else PEAK_BF16_TFLOPS
        achieved = gbs if bound == "hbm" else tflops
        out[grp] = {"kernel": kname, "bound": bound, "launches_per_step": per_step,
                    "ms_per_step": round(ms / steps, 4), "avg_launch_us": round(avg_s * 1e6, 3),
                    "work_per_launch": flops if bound == "mfma" else nbytes,
                    "achieved": round(achieved, 2), "peak": peak,
                    "unit": "GB/s" if bound == "hbm" else "TFLOP/s",
                    "frac": round(achieved / peak, 4),
                    "tflops": round(tflops, 2), "hbm_gbs": round(gbs, 1)}
    return out


def gemm_flops_per_token(D, F, layers):
    return 2.0 * layers * (3 * D * D + D * D + 2 * D * F + D * F)


def host_cpu():
    """CPU model, logical CPUs of the host, and the CPUs this process may use
    (the box's share; capped at 16, the GPU box's per-GPU CPU share)."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    avail = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    return model, os.cpu_count(), min(avail, 16)


def cpu_baseline(w, rl, enc, ids, mask, lens, layers_full):
    """Reference CPU encode on 8 rows (length deciles of the batch) through the
    first 2 layers of the same model (about 10 s of CPU work), extrapolated to
    all layers: layers cost the same and rows are independent.
    SNAPJUDGE_THREADS (and OMP/OPENBLAS_NUM_THREADS) = the CPUs available to
    this process; in the reference that sizes the attention thread team
    (src/tensor.cpp:162-168), while its no-BLAS GEMM runs on one thread."""
    from oracle import RefModel
    from snapjudge_amd import synth

    if not RefModel.available():
        return None
    cpu_model, n_logical, threads = host_cpu()
    for k in ("SNAPJUDGE_THREADS", "OMP_NUM_THREADS", "OPENBLAS_NUM_THREADS"):
        os.environ[k] = str(threads)
    nl = 2
    keep = {k: v for k, v in w.items()
            if not k.startswith("encoder.layers.")
            or any(k.startswith(f"encoder.layers.{i}.") for i in range(nl))}
    enc1 = dict(enc, num_hidden_layers=nl, layer_types=enc["layer_types"][:nl])
    order = np.argsort(lens)
    rows = [order[int(q * (len(lens) - 1))] for q in (0.1, 0.2, 0.3, 0.4, 0.5, 0.6, 0.7, 0.8)]
    with tempfile.TemporaryDirectory() as d:
        synth.write_checkpoint(d, rl, enc1, keep, store="BF16")
        ref = RefModel(d)
        ntok, secs = 0, 0.0
        for b in rows:
            n = int(lens[b])
            t0 = time.perf_counter()
            ref.encode(ids[b:b + 1, :n], mask[b:b + 1, :n])
            secs += time.perf_counter() - t0
            ntok += n
    tps = ntok * nl / (secs * layers_full)
    return {"value": round(tps, 2), "unit": "tokens/s", "cores": threads, "kind": "reference",
            "cpu_model": cpu_model, "host_logical_cpus": n_logical,
            "blas": "none: reference built with SNAPJUDGE_NO_BLAS (its single-threaded in-tree "
                    "GEMM, src/cblas_fallback.cpp); no BLAS library in the image",
            "sample": f"reference DecisionModel::encode (SNAPJUDGE_THREADS={threads}) on "
                      f"{len(rows)} rows of the batch, each called alone (sum n = {ntok}), through "
                      f"{nl} of {layers_full} layers: {secs:.1f} s, extrapolated x{layers_full / nl:g}"}


def encoder_leg(sj, torch, model, ids, lens, D, steps, warmup, stream):
    """Time `steps` encoder forwards (graph replay) on ids already in HBM, then
    the same steps launch by launch with per-kernel events.  Returns
    (ms per step, valid tokens/s, per-kernel totals)."""
    B = len(lens)
    T = int(lens.sum())
    packed = np.concatenate([ids[b, :lens[b]] for b in range(B)]).astype(np.int32)
    d_ids = torch.from_numpy(packed).cuda()
    d_out = torch.empty((T, D), dtype=torch.float32, device="cuda")
    lens32 = lens.astype(np.int32)

    def step():
        model.encode_device(d_ids.data_ptr(), lens32, d_out.data_ptr(), stream)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    model.profile(True)  # per-launch events (graph replay is off while profiling)
    step()  # first launch-by-launch step, not counted
    torch.cuda.synchronize()
    model.profile(False)
    model.profile(True)  # restarts the totals
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    prof = model.profile_read()
    model.profile(False)
    return elapsed * 1e3 / steps, T * steps / elapsed, prof


def decision_leg(model, ids, mask, lens, n_q, steps, seed=3):
    """Config 5's decision step: each of the U sequences carries n_q typed
    questions (qtype uniform over choice / score / noul, src/common.cpp:12-13,
    with synth.QTYPE_MARKERS markers), U * n_q rows through forward_shared: the
    encoder on the U sequences, the head layers once per distinct (sequence,
    qtype) pair, the scorer and act head per row.  Host arrays in, logits and
    act out, as DecisionModel::forward's interface, so the time includes the
    host<->device copies.  For comparison, the same rows through forward on
    the U * n_q-row expansion (every row encoded and run through the head)."""
    from snapjudge_amd import synth

    U = len(lens)
    row_seq, mp, mm, qt = synth.make_questions(lens, n_q, seed=seed)
    pairs = len({(int(u), int(t)) for u, t in zip(row_seq, qt)})

    def timed(fn, n):
        fn()  # warm-up: graph capture, workspace growth
        t = []
        for _ in range(n):
            t0 = time.perf_counter()
            fn()
            t.append(time.perf_counter() - t0)
        return float(np.median(t)) * 1e3

    shared = timed(lambda: model.forward_shared(ids, mask, row_seq, mp, mm, qt), steps)
    xi, xm = ids[row_seq], mask[row_seq]
    expanded = timed(lambda: model.forward(xi, xm, mp, mm, qt), max(2, steps // 2))
    rows = len(row_seq)
    return {"rows": rows, "sequences": U, "head_pairs": pairs,
            "forward_shared_ms": round(shared, 3), "rows_per_s": round(rows / (shared / 1e3), 1),
            "expanded_forward_ms": round(expanded, 3),
            "expanded_rows_per_s": round(rows / (expanded / 1e3), 1)}


def extra_leg(sj, torch, name, preset, precision, B, S, lo, hi, steps, stream, questions=0):
    """BASELINE config 4 or 5 (encoder tokens/s; not the headline line), and
    with questions > 0 the decision step over that many questions per row."""
    from snapjudge_amd import synth

    rl, enc, w = synth.make_model(**synth.PRESETS[preset], seed=0)
    cfg = synth.flat_cfg(rl, enc)
    D, F, NL = cfg["hidden_size"], cfg["intermediate_size"], cfg["num_hidden_layers"]
    ids, mask, lens = synth.make_batch(B, S, lo, hi, cfg["vocab_size"], seed=1)
    model = sj.Model(w, cfg, precision=precision, use_graphs=True)
    del w
    ms, tps, prof = encoder_leg(sj, torch, model, ids, lens, D, steps, 2, stream)
    decision = decision_leg(model, ids, mask, lens, questions, steps) if questions else None
    model.close()
    T = int(lens.sum())
    gemm_ms = sum(prof[n][0] for n in GEMM_NAMES if n in prof)
    kt = kernel_table(prof, steps, T, D, F, NL, lens)
    dom = max(kt, key=lambda g: kt[g]["ms_per_step"])
    return {"workload": name, "valid_tokens_per_step": T, "ms_per_step": round(ms, 3),
            "valid_tokens_per_s": round(tps, 1),
            "gemm_tflops": round(gemm_flops_per_token(D, F, NL) * T * steps / (gemm_ms / 1e3) / 1e12, 2),
            "attention_tflops": kt["attention"]["achieved"] if "attention" in kt else None,
            "dominant_kernel": dom,
            "kernels": {g: {k: v for k, v in d.items() if k != "kernel"} for g, d in kt.items()},
            "kernel_ms_per_step": {k: round(v[0] / steps, 4) for k, v in sorted(prof.items())},
            **({"decision": decision} if decision else {})}


def b1_legs(sj, torch, w, cfg, stream):
    """Config 2 (batch 1, seq 128, no padding): p50 latency of a hipGraph
    replay over 50 calls, per-kernel times of one launch-by-launch pass, and
    the same encoder with a new length ~ U[64, 128] on every call (the graph
    of each shape bucket is captured on its first call, inside the timing)."""
    D = cfg["hidden_size"]
    lm = sj.Model(w, cfg, precision=sj.SJH_PREC_BF16, use_graphs=True)
    rng = np.random.default_rng(7)
    ids2 = rng.integers(0, cfg["vocab_size"], size=128).astype(np.int32)
    d_ids2 = torch.from_numpy(ids2).cuda()
    d_out2 = torch.empty((128, D), dtype=torch.float32, device="cuda")

    def call(n):
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        lm.encode_device(d_ids2.data_ptr(), np.array([n], np.int32), d_out2.data_ptr(), stream)
        torch.cuda.synchronize()
        return (time.perf_counter() - t1) * 1e3

    lat = [call(128) for _ in range(60)][10:]
    lm.profile(True)
    call(128)
    lm.profile(False)
    lm.profile(True)
    call(128)
    prof = lm.profile_read()
    lm.profile(False)
    lm.close()
    # varying lengths on a fresh model: captures are part of the measurement
    vm = sj.Model(w, cfg, precision=sj.SJH_PREC_BF16, use_graphs=True)
    lm = vm
    lens = np.random.default_rng(8).integers(64, 129, size=60)
    vlat = [call(int(n)) for n in lens]
    gs = vm.graph_stats()
    vm.close()
    p50 = float(np.median(lat))
    vp50 = float(np.median(vlat))
    return (round(p50, 4),
            {k: round(v[0], 4) for k, v in sorted(prof.items())},
            {"lengths": "U[64,128] seed 8, a new length every call", "calls": len(vlat),
             "p50_ms": round(vp50, 4), "mean_ms_incl_captures": round(float(np.mean(vlat)), 4),
             "max_ms": round(float(np.max(vlat)), 4), "graph_captures": gs["captures"],
             "graph_replays": gs["replays"], "p50_vs_fixed_shape": round(vp50 / p50, 4)})


def blas_leg(sj, torch, T, D, F, stream, iters=50):
    """The four projection products of config 3 (M = the batch's T valid
    tokens) as plain bf16 GEMMs, out = A . W^T with no epilogue: torch.matmul
    (hipBLASLt) beside this library's sjh_gemm on the same operands, each the
    mean of `iters` launches between a hipEvent pair on the current stream.
    A reference point for the GEMM kernels, not part of `value`."""
    import ctypes as C

    shapes = {"qkv": (3 * D, D), "wo": (D, D), "wi": (2 * F, D), "wo2": (D, F)}
    g = torch.Generator(device="cuda").manual_seed(5)
    out = {}
    for name, (N, K) in shapes.items():
        A = (torch.randn((T, K), device="cuda", generator=g) * 0.5).to(torch.bfloat16)
        W = (torch.randn((N, K), device="cuda", generator=g) * 0.02).to(torch.bfloat16)
        Cb = torch.empty((T, N), dtype=torch.bfloat16, device="cuda")
        Cs = torch.empty_like(Cb)

        def ours():
            sj.check(sj.lib().sjh_gemm(C.c_void_p(A.data_ptr()), C.c_void_p(W.data_ptr()), None,
                                       C.c_void_p(Cs.data_ptr()), T, N, K, 0, sj.SJH_BF16,
                                       C.c_void_p(stream)))

        def blas():
            torch.matmul(A, W.t(), out=Cb)

        res = {}
        for label, fn in (("hipblaslt", blas), ("sjh", ours)):
            for _ in range(5):
                fn()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            e0.record()
            for _ in range(iters):
                fn()
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / iters
            tf = 2.0 * T * N * K / (us * 1e-6) / 1e12
            res[label] = {"us": round(us, 2), "tflops": round(tf, 1), "frac": round(tf / PEAK_BF16_TFLOPS, 4)}
        res["max_abs_diff"] = float((Cb.float() - Cs.float()).abs().max())
        out[name] = {"M": T, "N": N, "K": K, **res}
        del A, W, Cb, Cs
    return out


def copy_probe(mib):
    """Plain device-to-device copy of a known size (torch's copy kernel): the
    calibration run for the FETCH_SIZE / WRITE_SIZE counters."""
    import torch

    n = mib * (1 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes_each_way": n * 4, "launches": 3}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--legs", default=",".join(LEGS),
                    help="comma-separated legs to run: " + ",".join(LEGS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-latency", action="store_true", help="skip the batch-1 legs")
    ap.add_argument("--no-cfg4", action="store_true", help="skip the config-4 (S=8192) leg")
    ap.add_argument("--no-cfg5", action="store_true", help="skip the config-5 (fp8) leg")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="also run a plain copy of MIB MiB (counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this build measures one GPU only; the encoder shards across GPUs by "
              "sequence with no exchange, but no multi-GPU path is built.", file=sys.stderr)
        sys.exit(2)
    legs = set(x.strip() for x in args.legs.split(",") if x.strip())
    bad = legs - set(LEGS) - set(EXTRA_LEGS)
    if bad:
        ap.error(f"unknown legs {sorted(bad)}")
    for flag, leg in ((args.no_cpu, "cpu"), (args.no_latency, "b1"), (args.no_cfg4, "cfg4"),
                      (args.no_cfg5, "cfg5")):
        if flag:
            legs.discard(leg)

    import torch

    import snapjudge_amd as sj
    from snapjudge_amd import synth

    B, S, LO, HI = 64, 512, 64, 512
    p = synth.PRESETS["cfg3"]
    rl, enc, w = synth.make_model(**p, seed=0)
    cfg = synth.flat_cfg(rl, enc)
    D, F, NL = cfg["hidden_size"], cfg["intermediate_size"], cfg["num_hidden_layers"]
    ids, mask, lens = synth.make_batch(B, S, LO, HI, cfg["vocab_size"], seed=1)
    T = int(lens.sum())
    stream = torch.cuda.current_stream().cuda_stream

    value = ms_per_step = None
    roofline, kernels, prof, gemm_tflops, attn_frac = None, {}, {}, None, None
    if "cfg3" in legs:
        # Timed region: the encoder forward replayed as a captured hipGraph (one
        # graph per batch shape bucket, so the launches go out back to back).  A
        # second pass over the same number of steps, launched kernel by kernel
        # with a hipEvent pair around every launch on the model's stream, gives
        # the per-kernel durations the roofline uses; it is not part of `value`.
        model = sj.Model(w, cfg, precision=sj.SJH_PREC_BF16, use_graphs=True)
        ms_per_step, value, prof = encoder_leg(sj, torch, model, ids, lens, D, args.steps,
                                               args.warmup, stream)
        model.close()
        del model
        kt = kernel_table(prof, args.steps, T, D, F, NL, lens)
        dom = max(kt, key=lambda g: kt[g]["ms_per_step"])
        d = kt[dom]
        roofline = {"bound": d["bound"], "achieved": d["achieved"], "peak": d["peak"],
                    "unit": d["unit"], "frac": d["frac"],
                    "traffic": measured_traffic(CFG3_TRAFFIC, dom), "kernel": d["kernel"],
                    "group": dom, "work_per_launch": d["work_per_launch"],
                    "launches_per_step": d["launches_per_step"],
                    "avg_launch_us": d["avg_launch_us"], "ms_per_step": d["ms_per_step"]}
        for g, dd in kt.items():
            kernels[g] = {k: v for k, v in dd.items() if k != "kernel"}
            kernels[g]["traffic"] = measured_traffic(CFG3_TRAFFIC, g)
        gemm_ms = sum(prof[n][0] for n in GEMM_NAMES if n in prof)
        gemm_tflops = round(gemm_flops_per_token(D, F, NL) * T * args.steps / (gemm_ms / 1e3) / 1e12, 2)
        attn_frac = kt["attention"]["frac"] if "attention" in kt else None

    p50 = b1_kernels = b1_var = None
    if "b1" in legs:
        p50, b1_kernels, b1_var = b1_legs(sj, torch, w, cfg, stream)

    extra = {}
    if "cfg4" in legs:
        extra["cfg4"] = extra_leg(sj, torch, "BASELINE config 4: same encoder, batch 4 x seq 8192, "
                                  "lengths U[4096,8192] seed 1, bf16", "cfg4", sj.SJH_PREC_BF16,
                                  4, 8192, 4096, 8192, 5, stream)
    if "cfg5" in legs:
        extra["cfg5"] = extra_leg(sj, torch, "BASELINE config 5: 28-layer/1024 encoder, GEGLU 2624, "
                                  "per-row fp8 e4m3 projection weights (bf16 activations), batch "
                                  "32 x seq 1024, lengths U[256,1024] seed 1", "cfg5",
                                  sj.SJH_PREC_FP8W, 32, 1024, 256, 1024, 5, stream, questions=8)
    if "blas" in legs:
        extra["blas_cfg3_shapes"] = blas_leg(sj, torch, T, D, F, stream)
    cpu = cpu_baseline(w, rl, enc, ids, mask, lens, NL) if "cpu" in legs else None
    out = {
        "metric": METRIC, "value": round(value, 1) if value else None, "unit": "tokens/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4) if ms_per_step else None,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "BASELINE config 3: 22-layer/768 ModernBERT-style encoder, "
                               "bf16 weights N(0,0.02) seed 0, batch 64 x seq 512, "
                               "lengths U[64,512] seed 1 (valid tokens only)",
                   "global_batch": B, "seq_len": S, "valid_tokens_per_step": T,
                   "parallelism": "none (1 GPU)"},
        "roofline": roofline,
        "kernels": kernels,
        "gemm_all_tflops": gemm_tflops,
        "attention_mfma_frac": attn_frac,
        "p50_latency_b1_ms": p50,
        "b1_kernel_ms": b1_kernels,
        "b1_varlen": b1_var,
        "padded_tokens_per_s": round(B * S / (ms_per_step / 1e3), 1) if ms_per_step else None,
        "kernel_ms_per_step": {k: round(v[0] / args.steps, 4) for k, v in sorted(prof.items())},
        "cpu_baseline": cpu,
        "other_configs": extra,
    }
    print(json.dumps(out), flush=True)
    if args.copy_probe:
        copy_probe(args.copy_probe)


if __name__ == "__main__":
    main()
