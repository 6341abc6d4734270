"""Benchmark of the quantized-linear path on one MI355X.

Workload (the configuration the headline metric is quoted on): the full
Wan2.1-1.3B block-linear set in FP8 for one 3-frame chunk (M = 4680
tokens), 30 layers x 4 DMD steps, 7 linears per layer-step (self-attn QKV,
O; cross-attn Q, K/V on 512 text tokens, O; FFN up with GELU, FFN down),
with 30 distinct layers of random-init FP8 per-output-channel weights
resident in HBM (1.48 GB).  Activations are ~N(0,1), rounded to bf16, and
reach each linear in the form its producer writes it in the DiT block of
this backend: per-token e4m3 (codes + one f32 scale per row) from the fused
AdaLN norms for QKV, cross-attn Q and FFN up (layer_norm / residual_norm
quantize in the same pass that writes them) and for the text tokens
(quantized once per prompt); MX e4m3 (one power-of-two scale per 32
columns of a row) from attention's epilogue for O and cross-attn O and from
FFN up's epilogue for FFN down.  So no linear of the chunk runs a separate
quantization pass.  The same chunk on bf16 inputs, where each linear first
quantizes its input per token to e4m3, is timed too
(ms_per_chunk_bf16_input), and so is the one with a bf16 FFN hand-off.
The cross-attention K/V projections of the 30 layers all read the same 512
text tokens, so each step runs them as one linear over the layers'
concatenated weights [30 x 3072, 1536] (the reference computes them per
prompt, one linear per layer: dit.rs:470-492; head_split reads each layer's
slice of the output by stride).  One "step" is one chunk: 724
Backend::linear calls (6 per layer-step, dit.rs:602-759, plus one K/V call
per step).  Inputs are synthetic and resident before timing starts.

Timed two ways over the same calls: eagerly (one C-ABI call per linear from
Python) and as one replayed HIP graph of the whole chunk; `value` is the
faster.  The roofline object covers the dominant kernel, the fp8 GEMM: the
chunk's 724 GEMM launches run back to back (eagerly) inside a HIP-event
region on the context stream, so the average launch duration is the GEMM's
alone (rocprofv3 --kernel-trace of `bench.py --gemm-only` reports the same
kernels' average).  The CPU oracle is timed on a bounded row sample of the
same GEMMs beside it.

  python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu] [--no-graph]
"""

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "lightx2v-rs_amd"))

PEAK_FP8_TFLOPS = 5000.0   # MI355X dense fp8 MFMA
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
HBM_GBS = 8000.0

DIM, FFN, TEXT, LAYERS, DMD = 1536, 8960, 512, 30, 4
M = 4680  # 3 latent frames x 30 x 52 patches (832x480)

# (name, rows, N, K, act, input) -- crates/lightx2v-model/src/dit.rs:602-759 call sites
GEMMS = [
    ("qkv", M, 3 * DIM, DIM, 0, "x_attn"),
    ("o", M, DIM, DIM, 0, "x_o"),
    ("q2", M, DIM, DIM, 0, "x_q2"),
    ("kv2", TEXT, 2 * DIM, DIM, 0, "x_text"),
    ("o2", M, DIM, DIM, 0, "x_o2"),
    ("ffn1", M, FFN, DIM, 1, "x_ffn"),
    ("ffn2", M, DIM, FFN, 0, "y_ffn1"),
]
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gemm_fp8_chunk_traffic.json")


def flops_of(gemms):
    return sum(2.0 * r * n * k for _, r, n, k, _, _ in gemms)


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def per_config(be, H):
    """The baseline's other configs (1, 2, 3 and 5), one linear per shape:
    weights quantized on the device from the Rng's normals, inputs resident,
    30 back-to-back launches timed in a HIP-event region after ~50 ms of
    untimed launches.  Each is reported against the peak of the MFMA it runs
    on (fp8 for FP8 weights, bf16 for Q8 / Q4, which the GEMM dequantizes to
    bf16)."""
    import numpy as np
    out = {}

    def weight(kind, n, k, std, seed, heavy=False, group=None):
        tmp = be.alloc(n * k, H.DTYPE_F32)
        be.fill_normal(tmp, seed, std)
        if heavy:  # 1% of the weight's K columns x20 (columns k % 100 == 37)
            w = be.download(tmp).reshape(n, k)
            w[:, 37::100] *= 20.0
            tmp.free()
            be.set_act_dtype(H.DTYPE_F32)
            tmp = be.upload(w.ravel())
        if kind == "native":
            w = be.weight(be.download(tmp), n, k)
        elif kind == "fp8":
            w = be.quantize_fp8(tmp, n, k, group or k)
        elif kind == "q8":
            w = be.quantize_q8(tmp, n, k, 32)
        else:
            w = be.quantize_q4_sym(tmp, n, k, 32)
        tmp.free()
        return w

    def alg_bytes(rows, n, k, xdt, ydt, kind, group):
        """|X| + |W codes| + |scales (+ zeros)| + |bias| + |Y|, each once at its
        dtype ("e4m3": codes + a row scale; "mx": codes + one scale byte per 32)."""
        def tensor(r, c, dt):
            if dt == "e4m3":
                return r * c + r * 4
            if dt == "mx":
                return r * c + r * c // 32
            return r * c * {H.DTYPE_F32: 4, H.DTYPE_BF16: 2}[dt]
        codes = n * k // 2 if kind == "q4" else (n * k * 2 if kind == "native" else n * k)
        scales = 0 if kind == "native" else n * (k // group) * 4 * (2 if kind == "q4" else 1)
        return tensor(rows, k, xdt) + codes + scales + n * 4 + tensor(rows, n, ydt)

    def time_linear(name, x, rows, k, w, n, act, xdt, ydt, peak, path, kind="fp8", group=None):
        if ydt == "mx":
            y = be.alloc_mx(rows, n)
        else:
            be.set_act_dtype(ydt)
            y = be.alloc(rows * n)
        b = be.alloc(n, H.DTYPE_F32)
        be.fill_normal(b, 7, 0.01)
        # untimed warm-up for ~50 ms: the clock settles after the allocations and fills
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < 0.05:
            for _ in range(5):
                be.linear(x, 0, rows, w, b, act, y, 0)
            be.sync()
        be.profile_region("c_" + name, True)
        for _ in range(30):
            be.linear(x, 0, rows, w, b, act, y, 0)
        be.profile_region("c_" + name, False)
        us = be.profile_kernel("c_" + name)[1] * 1e3 / 30
        # the kernel configuration that ran (the profile report's name for it)
        be.profile_reset()
        be.profile_enable(True)
        try:
            be.linear(x, 0, rows, w, b, act, y, 0)
            ran = sorted(kk for kk in be.profile_stats() if kk.startswith("gemm"))
        finally:
            be.profile_enable(False)
            be.profile_reset()
        fl = 2.0 * rows * n * k
        tf = fl / (us * 1e-6) / 1e12
        nb = alg_bytes(rows, n, k, xdt, ydt, kind, group or k)
        ai = fl / nb
        bound = min(peak, ai * HBM_GBS / 1e3)  # TFLOP/s: the MFMA peak or AI x 8 TB/s
        out[name] = {"shape": f"{rows}x{k}->{n}", "us_per_linear": round(us, 2), "tflops": round(tf, 1),
                     "peak_tflops": peak, "pct_peak": round(100.0 * tf / peak, 1),
                     "alg_bytes": nb, "ai_flop_per_byte": round(ai, 1),
                     "bound": "hbm" if bound < peak else "mfma", "bound_tflops": round(bound, 1),
                     "us_at_bound": round(fl / (bound * 1e12) * 1e6, 2), "pct_bound": round(100.0 * tf / bound, 1),
                     "hbm_gbs": round(nb / (us * 1e-6) / 1e9, 1), "path": path, "kernel": ",".join(ran)}
        y.free()
        b.free()

    fp8_path = "per-token e4m3 activations (quantized inside linear) x FP8 weight, fp8 MFMA"
    fp8_g128_path = ("per-token e4m3 activations x FP8 weight with one scale per 128 columns, fp8 MFMA (each "
                     "128-column stage's partial sums scaled by the group's scale)")
    g128_chunk_path = ("the chunk's input as its producer writes it (per-token e4m3: QKV, cross Q, the text K/V, "
                       "FFN up; MX e4m3: O, cross O, FFN down) x FP8 weight with one scale per 128 columns, fp8 "
                       "MFMA; bf16 output (FFN up: MX e4m3)")
    # config 1: FP8 self-attn Q projection, f32 activations in and out
    be.set_act_dtype(H.DTYPE_F32)
    x = be.alloc(M * DIM)
    be.fill_normal(x, 1001, 1.0)
    w = weight("fp8", DIM, DIM, 0.02, 1002)
    time_linear("cfg1_fp8_q_proj_f32", x, M, DIM, w, DIM, 0, H.DTYPE_F32, H.DTYPE_F32, PEAK_FP8_TFLOPS, fp8_path)
    w.free()
    # the same with group-128 scales (the reference's FP8 default, quant.rs:21)
    w = weight("fp8", DIM, DIM, 0.02, 1002, group=128)
    time_linear("cfg1_fp8_g128_q_proj_f32", x, M, DIM, w, DIM, 0, H.DTYPE_F32, H.DTYPE_F32, PEAK_FP8_TFLOPS,
                fp8_g128_path, group=128)
    w.free()
    x.free()
    # config 4's seven GEMMs with group-128 weights, each on the input its producer
    # writes in the chunk and with the chunk's output (as the headline times them)
    for name, rows, n, k, act, _ in GEMMS:
        be.set_act_dtype(H.DTYPE_BF16)
        xb = be.alloc(rows * k)
        be.fill_normal(xb, 1041, 1.0)
        if name in ("o", "o2", "ffn2"):
            x, xdt = be.alloc_mx(rows, k), "mx"
            be.quantize_mx(xb, 0, rows, x)
        else:
            x, xdt = be.alloc_e4m3(rows, k), "e4m3"
            be.quantize_act(xb, 0, rows, x)
        xb.free()
        w = weight("fp8", n, k, 0.02, 1042 + n + k, group=128)
        time_linear(f"cfg4_g128_{name}", x, rows, k, w, n, act, xdt, "mx" if name == "ffn1" else H.DTYPE_BF16,
                    PEAK_FP8_TFLOPS, g128_chunk_path, group=128)
        w.free()
        if name == "kv2":
            # the chunk's form of it: the 30 layers' K/V weights in one call
            # (the text is the same for every layer); its time per layer
            kvn = LAYERS * n
            w = weight("fp8", kvn, k, 0.02, 1043 + n + k, group=128)
            time_linear("cfg4_g128_kv2_all_layers", x, rows, k, w, kvn, act, xdt, H.DTYPE_BF16, PEAK_FP8_TFLOPS,
                        g128_chunk_path + "; the 30 layers' weights concatenated, one call", group=128)
            out["cfg4_g128_kv2_all_layers"]["us_per_layer"] = round(out["cfg4_g128_kv2_all_layers"]["us_per_linear"]
                                                                    / LAYERS, 2)
            w.free()
        x.free()
    # config 2: Q8 (per-32 scales) FFN up + GELU, bf16 activations
    be.set_act_dtype(H.DTYPE_BF16)
    x = be.alloc(M * DIM)
    be.fill_normal(x, 1011, 1.0)
    w = weight("q8", FFN, DIM, 0.02, 1012)
    time_linear("cfg2_q8_ffn_up_gelu", x, M, DIM, w, FFN, 1, H.DTYPE_BF16, H.DTYPE_BF16, PEAK_BF16_TFLOPS,
                "bf16 activations x Q8 weight dequantized to bf16 inside the GEMM, bf16 MFMA", kind="q8", group=32)
    w.free()
    x.free()
    # config 3: Q4 (symmetric, per-32 scales) FFN down, input = GELU of N(0,1); plain and heavy-tailed
    be.set_act_dtype(H.DTYPE_F32)
    xr = be.alloc(M * FFN)
    be.fill_normal(xr, 1021, 1.0)
    v = be.download(xr)
    xr.free()
    g = 0.5 * v * (1.0 + np.tanh(np.float32(0.7978845608) * (v + np.float32(0.044715) * v * v * v)))
    be.set_act_dtype(H.DTYPE_BF16)
    x = be.upload(g.astype(np.float32))
    del v, g
    for heavy in (False, True):
        w = weight("q4", DIM, FFN, 0.02, 1022, heavy=heavy)
        time_linear("cfg3_q4_ffn_down" + ("_heavy_tailed" if heavy else ""), x, M, FFN, w, DIM, 0,
                    H.DTYPE_BF16, H.DTYPE_BF16, PEAK_BF16_TFLOPS,
                    "bf16 activations x Q4 weight dequantized to bf16 inside the GEMM, bf16 MFMA", kind="q4", group=32)
        w.free()
    x.free()
    # config 5: Wan2.2-TI2V-5B shapes in FP8, M = 2640 and 880
    for rows in (2640, 880):
        for nm, n, k, act in (("qkv", 3 * 3072, 3072, 0), ("o", 3072, 3072, 0), ("ffn1", 14336, 3072, 1),
                              ("ffn2", 3072, 14336, 0)):
            be.set_act_dtype(H.DTYPE_BF16)
            x = be.alloc(rows * k)
            be.fill_normal(x, 1031 + rows, 1.0)
            w = weight("fp8", n, k, 0.015, 1032 + n + k)
            time_linear(f"cfg5_{nm}_m{rows}", x, rows, k, w, n, act, H.DTYPE_BF16, H.DTYPE_BF16,
                        PEAK_FP8_TFLOPS, fp8_path)
            w.free()
            x.free()
    # native f32 weights (Backend::weight) at Wan2.1-1.3B's non-block linears: patch_embed, proj_out and
    # the text MLP (dit.rs:540-561, 772-781, 450-469), through the weights' bf16 copy on the bf16 MFMA
    native_path = "bf16 activations x the native f32 weight's bf16 copy, bf16 MFMA"
    for nm, rows, n, k, act in (("patch_embed", M, DIM, 64, 0), ("proj_out", M, 64, DIM, 0),
                                ("text_mlp1", TEXT, DIM, 4096, 1), ("text_mlp2", TEXT, DIM, DIM, 0)):
        be.set_act_dtype(H.DTYPE_BF16)
        x = be.alloc(rows * k)
        be.fill_normal(x, 1051 + k, 1.0)
        w = weight("native", n, k, 0.02, 1052 + n + k)
        time_linear(f"native_{nm}", x, rows, k, w, n, act, H.DTYPE_BF16, H.DTYPE_BF16, PEAK_BF16_TFLOPS,
                    native_path, kind="native")
        w.free()
        x.free()
    be.set_act_dtype(H.DTYPE_BF16)
    return out


def yardstick(be, H):
    """hipBLASLt's fp8 GEMM through torch._scaled_mm (e4m3 x e4m3, per-tensor
    scales, bf16 output) beside this build's GEMM on pre-quantized per-token
    e4m3 activations (per-channel weight scales, bias; FFN up with GELU), at
    the chunk's shapes: 100 launches each after a warm-up, CUDA / HIP events.
    A reference point for the GEMM alone, not part of the metric."""
    import torch

    dev = torch.device("cuda:0")

    def ev_time(fn, it=100):
        for _ in range(10):
            fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(it):
            fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / it * 1e3

    shapes = [(nm, r, n, k, act) for nm, r, n, k, act, _ in GEMMS]
    shapes.append(("kv2_all_layers", TEXT, LAYERS * 2 * DIM, DIM, 0))
    # two large shapes: what the library reaches where launch, prologue and
    # epilogue costs vanish against the K loop (a measured fp8 ceiling)
    shapes.append(("large_4096x4096_14336", 4096, 14336, 4096, 0))
    shapes.append(("large_8192_cube", 8192, 8192, 8192, 0))
    res = {}
    for nm, rows, n, k, act in shapes:
        a8 = torch.randn(rows, k, device=dev).to(torch.float8_e4m3fn)
        w8 = (0.02 * torch.randn(n, k, device=dev)).to(torch.float8_e4m3fn)
        one = torch.ones((), device=dev)
        t_blas = ev_time(lambda: torch._scaled_mm(a8, w8.t(), scale_a=one, scale_b=one, out_dtype=torch.bfloat16))
        del a8, w8
        torch.cuda.empty_cache()
        be.set_act_dtype(H.DTYPE_F32)
        xf = be.alloc(rows * k)
        be.fill_normal(xf, 11, 1.0)
        xq = be.alloc_e4m3(rows, k)
        be.quantize_act(xf, 0, rows, xq)
        tmp = be.alloc(n * k)
        be.fill_normal(tmp, 12, 0.02)
        w = be.quantize_fp8(tmp, n, k, k)
        bias = be.alloc(n)
        be.fill_normal(bias, 13, 0.01)
        be.set_act_dtype(H.DTYPE_BF16)
        y = be.alloc(rows * n)
        for _ in range(10):
            be.linear(xq, 0, rows, w, bias, act, y, 0)
        be.profile_region("y_" + nm, True)
        for _ in range(100):
            be.linear(xq, 0, rows, w, bias, act, y, 0)
        be.profile_region("y_" + nm, False)
        t_ours = be.profile_kernel("y_" + nm)[1] * 1e3 / 100
        for h in (xf, xq, tmp, bias, y):
            h.free()
        w.free()
        res[nm] = {"shape": f"{rows}x{k}->{n}", "hipblaslt_us": round(t_blas, 2), "this_build_us": round(t_ours, 2),
                   "hipblaslt_tflops": round(2.0 * rows * n * k / t_blas / 1e6, 1),
                   "this_build_tflops": round(2.0 * rows * n * k / t_ours / 1e6, 1)}
        log(f"yardstick {nm} {rows}x{k}->{n}: hipBLASLt {t_blas:.2f} us, this build {t_ours:.2f} us")
    # bf16: hipBLASLt's GEMM (torch.mm, bf16 x bf16 -> bf16) beside this build's
    # Q8 / Q4 linears (per-32 scales, dequantized to bf16 in the K loop) and its
    # native bf16-weight linear at configs 2 and 3's shapes, and 8192^3
    res16 = {}
    for nm, rows, n, k, act in (("cfg2_ffn_up", M, FFN, DIM, 1), ("cfg3_ffn_down", M, DIM, FFN, 0),
                                ("large_8192_cube", 8192, 8192, 8192, 0)):
        xb = torch.randn(rows, k, device=dev, dtype=torch.bfloat16)
        wb = 0.02 * torch.randn(n, k, device=dev, dtype=torch.bfloat16)
        t_blas = ev_time(lambda: torch.mm(xb, wb.t()))
        del xb, wb
        torch.cuda.empty_cache()
        be.set_act_dtype(H.DTYPE_BF16)
        x = be.alloc(rows * k)
        be.fill_normal(x, 21, 1.0)
        tmp = be.alloc(n * k, H.DTYPE_F32)
        be.fill_normal(tmp, 22, 0.02)
        ws = {"native_bf16": be.weight(be.download(tmp), n, k)}
        if not nm.startswith("large"):
            ws["q8_g32"] = be.quantize_q8(tmp, n, k, 32)
            ws["q4_g32"] = be.quantize_q4_sym(tmp, n, k, 32)
        tmp.free()
        bias = be.alloc(n, H.DTYPE_F32)
        be.fill_normal(bias, 23, 0.01)
        y = be.alloc(rows * n)
        entry = {"shape": f"{rows}x{k}->{n}", "hipblaslt_us": round(t_blas, 2),
                 "hipblaslt_tflops": round(2.0 * rows * n * k / t_blas / 1e6, 1)}
        for wn, w in ws.items():
            for _ in range(10):
                be.linear(x, 0, rows, w, bias, act, y, 0)
            be.profile_region("y16_" + nm + wn, True)
            for _ in range(30):
                be.linear(x, 0, rows, w, bias, act, y, 0)
            be.profile_region("y16_" + nm + wn, False)
            t = be.profile_kernel("y16_" + nm + wn)[1] * 1e3 / 30
            entry[wn + "_us"] = round(t, 2)
            entry[wn + "_tflops"] = round(2.0 * rows * n * k / t / 1e6, 1)
            w.free()
        for h in (x, bias, y):
            h.free()
        res16[nm] = entry
        log(f"yardstick bf16 {nm} {rows}x{k}->{n}: hipBLASLt {t_blas:.2f} us, " +
            ", ".join(f"{kk[:-3]} {vv} us" for kk, vv in entry.items() if kk.endswith("_us") and kk != "hipblaslt_us"))
    print(json.dumps({"yardstick": "hipBLASLt fp8 GEMM (torch._scaled_mm) vs this build, chunk shapes and two large ones",
                      "torch": torch.__version__, "shapes": res,
                      "bf16": {"what": "hipBLASLt bf16 GEMM (torch.mm) vs this build's Q8 / Q4 / native bf16 linears "
                                       "(bias; GELU at FFN up)", "shapes": res16}}), flush=True)


def cpu_baseline(seconds_target=12.0):
    """The CPU oracle (crates/lightx2v-cpu/src/lib.rs:296-326 restated: a
    sequential f32 acc += x*w per output, then bias, then GELU) on a row
    sample of one layer-step's 7 FP8 GEMMs (weights dequantized as the
    oracle's weight_fp8 does), timed twice in this run: on one thread (the
    reference's CpuBackend is single-threaded, lib.rs:107-149) and with
    OpenMP over output rows on every host core this process may use
    (bit-identical outputs).  Each leg runs about seconds_target / 2."""
    import numpy as np

    import oracle as O

    nproc = os.cpu_count() or 1
    affinity = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else nproc
    omp = os.environ.get("OMP_NUM_THREADS")
    threads = max(1, min(affinity, int(omp))) if omp and omp.isdigit() else affinity
    ws = {}
    for i, (name, rows, n, k, act, _) in enumerate(GEMMS):
        wf = O.Rng(1002 + i).normal(n * k).reshape(n, k) * np.float32(0.02)
        q, s = O.fp8_quantize(wf, n, k, k, True)
        ws[name] = (O.fp8_dequantize(q, s, n, k, k), O.Rng(1003 + i).normal(n) * np.float32(0.01))

    def run(sample_rows, nt):
        fl = 0.0
        t = 0.0
        for name, rows, n, k, act, _ in GEMMS:
            r = min(rows, sample_rows)
            x = O.Rng(1001).normal(r * k).reshape(r, k)
            wd, b = ws[name]
            t0 = time.perf_counter()
            O.linear(x, wd, b, act, nthreads=nt)
            t += time.perf_counter() - t0
            fl += 2.0 * r * n * k
        return fl, t

    def leg(nt):
        fl, t = run(max(1, nt), nt)
        rows = int(max(nt, min(M, max(1, nt) * (seconds_target / 2) / max(t, 1e-3))))
        fl, t = run(rows, nt)
        return fl / t / 1e12, rows, fl, t

    v1, r1, f1, t1 = leg(1)
    vn, rn, fn, tn = leg(threads)
    step_flops = flops_of(GEMMS) * LAYERS * DMD
    return {
        "value": vn,
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"oracle linear (sequential f32 per output, OpenMP over rows) on {rn} rows of each of one "
                   f"layer-step's 7 FP8 GEMMs (weights dequantized): {fn / 1e9:.1f} GFLOP in {tn:.1f} s on "
                   f"{threads} threads (host nproc {nproc}, {affinity} usable by this process)"),
        "single_thread": {
            "value": v1, "cores": 1,
            "sample": f"the same on {r1} rows per GEMM, one thread: {f1 / 1e9:.2f} GFLOP in {t1:.1f} s",
        },
        "chunk_s_extrapolated": {"single_thread": step_flops / (v1 * 1e12), "all_cores": step_flops / (vn * 1e12),
                                 "what": "the chunk's 47.4 TFLOP at the sampled rates (an extrapolation)"},
        "nproc": nproc,
        "affinity": affinity,
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=int(os.environ.get("WORLD_SIZE", "1")))
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=20.0, help="CPU baseline: both legs together")
    ap.add_argument("--no-configs", action="store_true", help="skip the per-config linears")
    ap.add_argument("--no-graph", action="store_true",
                    help="time eagerly only (rocprofv3 cannot trace hipGraphLaunch here)")
    ap.add_argument("--yardstick", action="store_true",
                    help="time hipBLASLt's fp8 GEMM (torch._scaled_mm, per-tensor scales, bf16 out) against "
                         "this build's GEMM at the chunk's shapes, print one JSON line, exit")
    ap.add_argument("--gemm-only", action="store_true",
                    help="run the chunk's GEMMs --steps times on pre-quantized activations and the counter "
                         "calibration kernel, then exit (the workload of the rocprofv3 summaries in profiles/)")
    ap.add_argument("--data-probe", action="store_true",
                    help="time the chunk's GEMMs (as --gemm-only) on the random activations, then on all-zero "
                         "activations, print one JSON line, exit: the matrix cores' data-dependent power draw")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: the linear path shards over token rows with no exchange, "
              f"so a multi-GPU figure is not run here (--gpus {args.gpus}).", file=sys.stderr)
        sys.exit(2)

    if args.yardstick:
        import torch

        torch.cuda.init()  # before the library's context: torch must see the device first

    import lightx2v_hip as H

    be = H.HipBackend(0)
    log(f"bench: {be.name()}")
    if args.yardstick:
        yardstick(be, H)
        return
    be.set_act_dtype(H.DTYPE_BF16)

    # ---- resident synthetic inputs and weights --------------------------------
    t0 = time.perf_counter()
    acts = {}
    for i, nm in enumerate(["x_attn", "x_o", "x_q2", "x_o2", "x_ffn"]):
        acts[nm] = be.alloc(M * DIM)
        be.fill_normal(acts[nm], 1001 + 7 * i, 1.0)
    acts["x_text"] = be.alloc(TEXT * DIM)
    be.fill_normal(acts["x_text"], 1099, 1.0)
    outs = {name: be.alloc(rows * n * (LAYERS if name == "kv2" else 1)) for name, rows, n, _, _, _ in GEMMS}
    KVW = LAYERS * 2 * DIM  # columns of the concatenated cross-attention K/V output
    ffn_mx = be.alloc_mx(M, FFN)  # FFN up -> FFN down in MX e4m3
    acts["y_ffn1"] = outs["ffn1"]
    tmp = be.alloc(FFN * DIM, H.DTYPE_F32)
    tmp_kv = be.alloc(KVW * DIM, H.DTYPE_F32)

    def make_layers(group):
        """Per layer: the weights of the six per-layer linears; then the
        layers' cross-attention K/V weights as one [30 x 3072, 1536] weight
        (scales and bias concatenated the same way)."""
        out = []
        for l in range(LAYERS):
            lw = {}
            for j, (name, rows, n, k, act, _) in enumerate(GEMMS):
                if name == "kv2":
                    continue
                seed = 10_000 * (l + 1) + 10 * j
                be.fill_normal(tmp, seed, 0.02)
                w = be.quantize_fp8(tmp, n, k, group or k)
                b = be.alloc(n, H.DTYPE_F32)
                be.fill_normal(b, seed + 1, 0.01)
                lw[name] = (w, b)
            out.append(lw)
        be.fill_normal(tmp_kv, 9_999, 0.02)
        kvw = be.quantize_fp8(tmp_kv, KVW, DIM, group or DIM)
        kvb = be.alloc(KVW, H.DTYPE_F32)
        be.fill_normal(kvb, 9_998, 0.01)
        return out, (kvw, kvb)

    layers, kv_all = make_layers(None)
    be.sync()
    wbytes = (sum(w.info()["device_bytes"] for lw in layers for w, _ in lw.values()) +
              kv_all[0].info()["device_bytes"])
    log(f"bench: setup {time.perf_counter() - t0:.1f} s, {wbytes / 1e9:.2f} GB FP8 weights resident")

    def chunk(mx_handoff):
        """The chunk on bf16 inputs: each linear quantizes its input per
        token first (FFN up -> FFN down in MX e4m3, or in bf16)."""
        def run():
            for _ in range(DMD):
                be.linear(acts["x_text"], 0, TEXT, *kv_all, 0, outs["kv2"], 0)
                for lw in layers:
                    for name, rows, n, k, act, src in GEMMS:
                        if name == "kv2":
                            continue
                        w, b = lw[name]
                        x, y = acts[src], outs[name]
                        if mx_handoff and name == "ffn1":
                            y = ffn_mx
                        if mx_handoff and name == "ffn2":
                            x = ffn_mx
                        be.linear(x, 0, rows, w, b, act, y, 0)
        return run

    step_flops = flops_of(GEMMS) * LAYERS * DMD
    n_linear = ((len(GEMMS) - 1) * LAYERS + 1) * DMD

    # The linears' inputs in the forms their producers write them in the DiT
    # block: per-token e4m3 from the fused norms (QKV, cross Q, FFN up) and
    # for the text (once per prompt); MX e4m3 from attention's epilogue (O,
    # cross O) and from FFN up's (FFN down).
    MX_IN = ("x_o", "x_o2")
    per_token = [g for g in GEMMS if g[0] != "ffn2"]
    qin = {}
    for _, rows, _, k, _, src in per_token:
        if src in MX_IN:
            qin[src] = be.alloc_mx(rows, k)
            be.quantize_mx(acts[src], 0, rows, qin[src])
        else:
            qin[src] = be.alloc_e4m3(rows, k)
            be.quantize_act(acts[src], 0, rows, qin[src])
    gx = {name: (ffn_mx if name == "ffn2" else qin[src]) for name, _, _, _, _, src in GEMMS}
    gy = {name: (ffn_mx if name == "ffn1" else outs[name]) for name, _, _, _, _, _ in GEMMS}
    # the bf16-input chunk's per-token quantization, timed on its own
    xq = {src: be.alloc_e4m3(rows, k) for _, rows, _, k, _, src in per_token}

    def gemm_step():
        """The headline chunk: every linear on its producer-written input."""
        for _ in range(DMD):
            be.linear(gx["kv2"], 0, TEXT, *kv_all, 0, gy["kv2"], 0)
            for lw in layers:
                for name, rows, n, k, act, src in GEMMS:
                    if name == "kv2":
                        continue
                    w, b = lw[name]
                    be.linear(gx[name], 0, rows, w, b, act, gy[name], 0)

    step = gemm_step

    def calibrate():
        """The rocprofv3 FETCH_SIZE / WRITE_SIZE calibration: one plain
        streaming kernel of known bytes (k_convert, f32 -> bf16: 1 GiB read,
        512 MiB written, both past the 256 MB Infinity Cache)."""
        cal_n = 256 << 20
        ca, cb = be.alloc(cal_n, H.DTYPE_F32), be.alloc(cal_n, H.DTYPE_BF16)
        be.copy(ca, 0, cb, 0, cal_n)
        be.sync()
        ca.free()
        cb.free()

    if args.gemm_only:
        for _ in range(max(1, args.steps)):
            gemm_step()
        be.sync()
        calibrate()
        log(f"bench: --gemm-only: {n_linear} GEMM launches and the calibration kernel")
        return

    def timed(fn, steps, warmup):
        for _ in range(warmup):
            fn()
        be.sync()
        t0 = time.perf_counter()
        for _ in range(steps):
            fn()
        be.sync()
        return (time.perf_counter() - t0) * 1e3 / steps

    if args.data_probe:
        # The same launches, shapes and weights; only the activation values
        # differ (zeros quantize to zero codes with scale 1).  FFN down's MX
        # input is what FFN up writes: GELU(bias) when its input is zero.
        ms_rand = timed(gemm_step, args.steps, args.warmup)
        for _, rows, _, k, _, src in per_token:
            be.fill_normal(acts[src], 1, 0.0)
            if src in MX_IN:
                be.quantize_mx(acts[src], 0, rows, qin[src])
            else:
                be.quantize_act(acts[src], 0, rows, qin[src])
        be.sync()
        ms_zero = timed(gemm_step, args.steps, args.warmup)
        log(f"bench: --data-probe: random {ms_rand:.2f} ms, zero {ms_zero:.2f} ms per chunk of GEMMs")
        print(json.dumps({"data_probe": "the chunk's 724 GEMM launches, random vs all-zero activations",
                          "ms_random": round(ms_rand, 3), "ms_zero": round(ms_zero, 3),
                          "tflops_random": round(step_flops / ms_rand / 1e9, 1),
                          "tflops_zero": round(step_flops / ms_zero / 1e9, 1),
                          "ratio": round(ms_rand / ms_zero, 3), "steps": args.steps}))
        return

    # ---- eager, then one replayed graph per chunk --------------------------------
    def eager_and_graph(fn, what):
        ms_e = timed(fn, args.steps, args.warmup)
        ms_g = None
        if not args.no_graph:
            be.graph_begin()
            fn()
            g = be.graph_end()
            ms_g = timed(g.launch, args.steps, args.warmup)
            g.free()
        log(f"bench: {what}: eager {ms_e:.2f} ms/chunk" + (f", graph {ms_g:.2f} ms/chunk" if ms_g else ""))
        return ms_e, ms_g

    ms_eager, ms_graph = eager_and_graph(step, "chunk (producer-written e4m3 / MX inputs)")
    ms = min(ms_eager, ms_graph) if ms_graph else ms_eager
    log(f"bench: chunk {ms:.2f} ms, {step_flops / ms / 1e9:.1f} TFLOP/s")
    # the chunk on bf16 inputs (each linear quantizes per token first)
    ms_bf16_e, ms_bf16_g = eager_and_graph(chunk(True), "chunk on bf16 inputs")
    ms_bf16_input = min(ms_bf16_e, ms_bf16_g) if ms_bf16_g else ms_bf16_e
    # ... and with the FFN hand-off in bf16 too (per-token e4m3 inside FFN down)
    ms_bf16_handoff = timed(chunk(False), args.steps, args.warmup)
    log(f"bench: bf16 inputs and bf16 FFN hand-off (eager) {ms_bf16_handoff:.2f} ms/chunk")
    # the chunk with group-128 weights (the reference's FP8 format, quant.rs:21),
    # eager, on the same producer-written inputs as the headline chunk
    # (per-token e4m3 for QKV, cross Q, FFN up and the text K/V; MX e4m3 for
    # O, cross O and FFN down, FFN up writing MX)
    g128, kv_g128 = make_layers(128)

    def chunk_g128():
        for _ in range(DMD):
            be.linear(gx["kv2"], 0, TEXT, *kv_g128, 0, gy["kv2"], 0)
            for lw in g128:
                for name, rows, n, k, act, src in GEMMS:
                    if name == "kv2":
                        continue
                    w, b = lw[name]
                    be.linear(gx[name], 0, rows, w, b, act, gy[name], 0)

    ms_g128 = timed(chunk_g128, args.steps, args.warmup)
    log(f"bench: group-128 weights (eager) {ms_g128:.2f} ms/chunk")
    for lw in g128:
        for w, b in lw.values():
            w.free()
            b.free()
    kv_g128[0].free()
    kv_g128[1].free()
    del g128
    tmp.free()
    tmp_kv.free()
    value = step_flops / ms / 1e9

    # ---- the block's linear path with its producers and consumers ---------------
    # (crates/lightx2v-model/src/dit.rs:590-770 minus attention and the KV
    # cache): AdaLN layer_norm -> QKV; O -> residual_norm (gated, affine) ->
    # cross Q; cross O -> residual_norm (mod) -> FFN up -> FFN down ->
    # gate_residual, per layer with its own modulation table.  "unfused":
    # the norms write bf16 and each linear quantizes its input per token;
    # "fused": the norms write the e4m3 input directly (no quantize pass) and
    # FFN down adds its gated output into h in its epilogue (linear_residual).
    NK = H.NormKind
    h = be.alloc(M * DIM)
    be.fill_normal(h, 1201, 1.0)
    normed = be.alloc(M * DIM)
    xq_blk = be.alloc_e4m3(M, DIM)
    # head_split's outputs and parameters: q / k / v of the chunk and the
    # text, [heads, rows, 128] bf16; RMS weights per layer; RoPE tables
    # [M, 64] (dit.rs:612-641, 705, 477-489)
    HD = 128
    hq, hk, hv = (be.alloc(M * DIM) for _ in range(3))
    hk2, hv2 = be.alloc(TEXT * DIM), be.alloc(TEXT * DIM)
    rcos, rsin = be.alloc(M * HD // 2, H.DTYPE_F32), be.alloc(M * HD // 2, H.DTYPE_F32)
    be.fill_normal(rcos, 1601, 0.7)
    be.fill_normal(rsin, 1602, 0.7)
    lrms = []
    lmods, lnw = [], []
    for l in range(LAYERS):
        rw = [be.alloc(DIM, H.DTYPE_F32) for _ in range(4)]  # norm_q1, norm_k1, norm_q2, norm_k2
        for i, b in enumerate(rw):
            be.fill_normal(b, 1700 + 4 * l + i, 0.1)
        lrms.append(rw)
        md = be.alloc(6 * DIM, H.DTYPE_F32)
        be.fill_normal(md, 1300 + l, 0.1)
        nw, nb = be.alloc(DIM, H.DTYPE_F32), be.alloc(DIM, H.DTYPE_F32)
        be.fill_normal(nw, 1400 + l, 0.1)
        be.fill_normal(nb, 1500 + l, 0.1)
        lmods.append(md)
        lnw.append((nw, nb))

    def block_path(fused):
        def run():
            xin = xq_blk if fused else normed
            for _ in range(DMD):
                # every layer's text K / V in one call; each layer's slices by stride
                be.linear(acts["x_text"], 0, TEXT, *kv_all, 0, outs["kv2"], 0)
                for l, lw in enumerate(layers):
                    md, (nw, nb) = lmods[l], lnw[l]
                    nq1, nk1, nq2, nk2 = lrms[l]
                    be.layer_norm(h, M, DIM, NK.mod(1, 0), md, 1e-6, xin)
                    be.linear(xin, 0, M, *lw["qkv"], 0, outs["qkv"], 0)
                    be.head_split(outs["qkv"], M, 3 * DIM, 0, DIM // HD, HD, nq1, (rcos, rsin), 1e-6, hq)
                    be.head_split(outs["qkv"], M, 3 * DIM, DIM, DIM // HD, HD, nk1, (rcos, rsin), 1e-6, hk)
                    be.head_split(outs["qkv"], M, 3 * DIM, 2 * DIM, DIM // HD, HD, None, None, 1e-6, hv)
                    be.linear(acts["x_o"], 0, M, *lw["o"], 0, outs["o"], 0)
                    be.residual_norm(h, outs["o"], M, DIM, md, 2, NK.affine(nw, nb), 1e-6, xin)
                    be.linear(xin, 0, M, *lw["q2"], 0, outs["q2"], 0)
                    be.head_split(outs["q2"], M, DIM, 0, DIM // HD, HD, nq2, None, 1e-6, hq)
                    be.head_split(outs["kv2"], TEXT, KVW, 2 * DIM * l, DIM // HD, HD, nk2, None, 1e-6, hk2)
                    be.head_split(outs["kv2"], TEXT, KVW, 2 * DIM * l + DIM, DIM // HD, HD, None, None, 1e-6, hv2)
                    be.linear(acts["x_o2"], 0, M, *lw["o2"], 0, outs["o2"], 0)
                    be.residual_norm(h, outs["o2"], M, DIM, md, None, NK.mod(4, 3), 1e-6, xin)
                    be.linear(xin, 0, M, *lw["ffn1"], 1, ffn_mx, 0)
                    if fused:  # the gate-residual add in FFN down's epilogue
                        be.linear_residual(ffn_mx, 0, M, *lw["ffn2"], 0, h, 0, md, 5)
                    else:
                        be.linear(ffn_mx, 0, M, *lw["ffn2"], 0, outs["ffn2"], 0)
                        be.gate_residual(h, outs["ffn2"], M, DIM, md, 5)
        return run

    block = {}
    for nm, fused in (("unfused", False), ("fused", True)):
        fn = block_path(fused)
        ms_e = timed(fn, args.steps, args.warmup)
        ms_g = None
        if not args.no_graph:
            be.graph_begin()
            fn()
            g = be.graph_end()
            ms_g = timed(g.launch, args.steps, args.warmup)
            g.free()
        block[nm] = round(min(ms_e, ms_g) if ms_g else ms_e, 3)
    log(f"bench: block linear path with norms: unfused {block['unfused']:.2f} ms/chunk, "
        f"fused {block['fused']:.2f} ms/chunk")

    # ---- the dominant kernel alone: the headline chunk's GEMM launches ----------
    # (gemm_step: FFN up writes the MX buffer FFN down reads; the other inputs
    # per-token or MX e4m3 as their producers write them).  act_quant_step is
    # the per-token quantization the bf16-input chunk adds to its linears.
    def act_quant_step():
        for _ in range(DMD):
            be.quantize_act(acts["x_text"], 0, TEXT, xq["x_text"])
            for _ in range(LAYERS):
                for name, rows, _, k, _, src in per_token:
                    if name != "kv2":
                        be.quantize_act(acts[src], 0, rows, xq[src])

    reps = max(1, min(args.steps, 3))
    region = {}
    for name, fn in (("gemm_fp8_chunk", gemm_step), ("act_quant_chunk", act_quant_step)):
        fn()
        be.profile_region(name, True)
        for _ in range(reps):
            fn()
        be.profile_region(name, False)
        _, t = be.profile_kernel(name)
        region[name] = t / reps
    gemm_ms = region["gemm_fp8_chunk"]
    # algorithmic bytes of the chunk's GEMMs as run here: e4m3 X (+ f32 row
    # scales, or one E8M0 byte per 32 for the MX inputs of O, cross O and FFN
    # down), e4m3 W + f32 channel scales, f32 bias, bf16 Y (MX e4m3 + scales
    # for FFN up), averaged per launch
    def x_bytes(nm, r, k):
        return r * k + (r * k // 32 if nm in ("o", "o2", "ffn2") else r * 4)

    alg_step = sum(x_bytes(nm, r, k) * (1 if nm == "kv2" else LAYERS) +
                   (n * k + n * 8 + (r * n + r * n // 32 if nm == "ffn1" else 2 * r * n)) * LAYERS
                   for nm, r, n, k, _, _ in GEMMS)
    alg_per_launch = alg_step / ((len(GEMMS) - 1) * LAYERS + 1)
    achieved = step_flops / gemm_ms / 1e9
    log(f"bench: GEMM-only {gemm_ms:.2f} ms/chunk ({gemm_ms * 1e3 / n_linear:.2f} us/launch, "
        f"{achieved:.1f} TFLOP/s); bf16 inputs' act quant {region['act_quant_chunk']:.2f} ms/chunk")

    # per-shape GEMM time (layer 0 weights, 50 back-to-back launches in a region)
    per = {}
    for name, rows, n, k, act, src in GEMMS:
        # the K / V call covers all the layers: its per-layer share is reported
        w, b = kv_all if name == "kv2" else layers[0][name]
        be.linear(gx[name], 0, rows, w, b, act, gy[name], 0)
        be.profile_region("g_" + name, True)
        for _ in range(50):
            be.linear(gx[name], 0, rows, w, b, act, gy[name], 0)
        be.profile_region("g_" + name, False)
        us = be.profile_kernel("g_" + name)[1] * 1e3 / 50 / (LAYERS if name == "kv2" else 1)
        uq = 0.0  # FFN down's input is quantized in FFN up's epilogue
        if name != "ffn2":
            be.profile_region("q_" + name, True)
            for _ in range(50):
                be.quantize_act(acts[src], 0, rows, xq[src])
            be.profile_region("q_" + name, False)
            uq = be.profile_kernel("q_" + name)[1] * 1e3 / 50 / (LAYERS if name == "kv2" else 1)
        per[name] = {"shape": f"{rows}x{k}->{n}" + (f", the {LAYERS} layers in one call (per layer)"
                                                   if name == "kv2" else ""),
                     "input": "MX e4m3" if name in ("o", "o2", "ffn2") else "per-token e4m3",
                     "gemm_us": round(us, 2), "bf16_input_act_quant_us": round(uq, 2),
                     "tflops": round(2.0 * rows * n * k / (us * 1e-6) / 1e12, 1),
                     "pct_fp8_peak": round(2.0 * rows * n * k / (us * 1e-6) / 1e12 / PEAK_FP8_TFLOPS * 100, 1)}

    # ---- head_split at the chunk's q (RMS + RoPE), 20 calls in a region ----
    be.head_split(outs["qkv"], M, 3 * DIM, 0, DIM // HD, HD, lrms[0][0], (rcos, rsin), 1e-6, hq)
    be.profile_region("hsplit", True)
    for _ in range(20):
        be.head_split(outs["qkv"], M, 3 * DIM, 0, DIM // HD, HD, lrms[0][0], (rcos, rsin), 1e-6, hq)
    be.profile_region("hsplit", False)
    hs_us = be.profile_kernel("hsplit")[1] * 1e3 / 20
    hs_bytes = M * DIM * 2 * 2 + M * HD // 2 * 4 * 2 + DIM * 4
    head_split = {"shape": f"q of the chunk's QKV: {M} rows x {DIM} of {3 * DIM}, RMS + RoPE, bf16 -> "
                           f"[{DIM // HD}, {M}, {HD}]", "us": round(hs_us, 2), "alg_bytes": hs_bytes,
                  "hbm_gbs": round(hs_bytes / (hs_us * 1e-6) / 1e9, 1),
                  "pct_hbm": round(100.0 * hs_bytes / (hs_us * 1e-6) / 1e9 / HBM_GBS, 1)}
    log(f"bench: head_split {hs_us:.1f} us ({head_split['hbm_gbs']} GB/s)")

    def region_us(name, fn, n):
        be.sync()
        be.profile_region(name, True)
        for _ in range(n):
            fn()
        be.profile_region(name, False)
        return be.profile_kernel(name)[1] * 1e3 / n

    # ---- causal attention at the chunk's shape (not part of the linear metric) ----
    # 12 heads x 128, the 3-frame chunk's 4680 queries against one cached
    # 1560-token frame plus the chunk (6240 keys), frame-causal MemRoPE-style
    # mask resident on the device (crates/lightx2v-model/src/dit.rs:655-668).
    import numpy as np
    heads, hd, frame = DIM // 128, 128, 1560
    sk = M + frame
    qf = (np.arange(M) + frame) // frame
    kf = np.arange(sk) // frame
    amask = kf[None, :] <= qf[:, None]
    aq, ak, av = be.alloc(heads * M * hd), be.alloc(heads * sk * hd), be.alloc(heads * sk * hd)
    for i, bb in enumerate((aq, ak, av)):
        be.fill_normal(bb, 1600 + i, 1.0)
    aout = be.alloc(M * heads * hd)
    am = be.mask_upload(amask, M, sk)
    be.causal_attention(aq, ak, av, heads, M, sk, hd, am, aout)
    be.profile_region("attn", True)
    for _ in range(20):
        be.causal_attention(aq, ak, av, heads, M, sk, hd, am, aout)
    be.profile_region("attn", False)
    attn_us = be.profile_kernel("attn")[1] * 1e3 / 20
    pairs = float(amask.sum()) * heads
    attn = {"shape": f"{heads} heads x {hd}, sq {M}, sk {sk}, frame-causal mask",
            "us": round(attn_us, 2),
            "tflops_allowed_pairs": round(4.0 * hd * pairs / (attn_us * 1e-6) / 1e12, 1),
            "pct_bf16_peak": round(4.0 * hd * pairs / (attn_us * 1e-6) / 1e12 / PEAK_BF16_TFLOPS * 100, 1),
            "kernel": "k_attn_mfma (bf16 MFMA, online softmax)"}
    log(f"bench: causal attention {attn_us:.1f} us ({attn['tflops_allowed_pairs']} TFLOP/s over allowed pairs)")
    # attention -> O linear (layer 0's weights): the bf16 hand-off (the linear
    # quantizes per token first) against the MX e4m3 hand-off written by the
    # attention epilogue
    amx = be.alloc_mx(M, heads * hd)
    ow, ob = layers[0]["o"]

    def attn_o(dst):
        def run():
            be.causal_attention(aq, ak, av, heads, M, sk, hd, am, dst)
            be.linear(dst, 0, M, ow, ob, 0, outs["o"], 0)
        return run

    attn_o(amx)()
    ao16_us = region_us("attn_o16", attn_o(aout), 10)
    aomx_us = region_us("attn_omx", attn_o(amx), 10)
    attn["attention_then_o_linear_us"] = {"bf16_handoff": round(ao16_us, 2), "mx_handoff": round(aomx_us, 2)}
    log(f"bench: attention + O linear: bf16 hand-off {ao16_us:.1f} us, MX hand-off {aomx_us:.1f} us")
    am.free()
    for bb in (aq, ak, av, aout, amx):
        bb.free()

    # ---- KV cache at steady state (not part of the linear metric) ----
    # One layer's MemRoPE cache after 6 chunks (12 frames of 1560 tokens, bf16,
    # K / V [heads, cap, 128]): the re-run steps' put (overwrite in place) and
    # update (nothing moves), the chunk's first step (append + seed / evict
    # gather), and attention of the chunk over the cache in place with the
    # DiT's mask (key temporal <= query temporal, dit.rs:636-668).
    rows = M
    cfg = H.MemRopeConfig()
    kvc = be.kv_cache_new(heads, hd, 12 * frame)
    kb_, vb_ = be.alloc(heads * rows * hd), be.alloc(heads * rows * hd)
    be.fill_normal(kb_, 1700, 1.0)
    be.fill_normal(vb_, 1701, 1.0)
    temporal = [np.array([c * 3 + i // frame for i in range(rows)], np.uint64) for c in range(40)]
    for c in range(6):
        kvc.put(kb_, vb_, rows, temporal[c])
        kvc.memrope_update(cfg, frame)
    be.sync()
    tq = temporal[5].astype(np.int64)
    kmask = np.array(kvc.temporal())[None, :] <= tq[:, None]
    # the step's mask, built on the device from the temporal indices (the
    # reference builds the [sq, sk] bools on the host, dit.rs:643-653)
    be.sync()
    t0 = time.perf_counter()
    km = be.mask_temporal(temporal[5], kvc.temporal())
    mask_ms = (time.perf_counter() - t0) * 1e3
    t0 = time.perf_counter()
    be.mask_upload(kmask, rows, len(kvc)).free()
    upload_ms = (time.perf_counter() - t0) * 1e3
    qb_, ob_ = be.alloc(heads * rows * hd), be.alloc(rows * heads * hd)
    be.fill_normal(qb_, 1702, 1.0)
    kvc.attention(qb_, rows, km, ob_)

    kv_attn_us = region_us("kv_attn", lambda: kvc.attention(qb_, rows, km, ob_), 10)
    put_us = region_us("kv_put", lambda: (kvc.put(kb_, vb_, rows, temporal[5]), kvc.memrope_update(cfg, frame)), 10)
    nxt = [6]

    def first_step():
        kvc.put(kb_, vb_, rows, temporal[nxt[0]])
        kvc.memrope_update(cfg, frame)
        nxt[0] += 1

    evict_us = region_us("kv_evict", first_step, 5)
    kpairs = float(kmask.sum()) * heads
    kv = {"shape": f"{heads} heads x {hd}, {len(kvc)} cached rows (12 frames of {frame}), chunk of {rows} queries, bf16",
          "attention_in_place_us": round(kv_attn_us, 2),
          "attention_tflops_allowed_pairs": round(4.0 * hd * kpairs / (kv_attn_us * 1e-6) / 1e12, 1),
          "put_and_update_rerun_step_us": round(put_us, 2),
          "put_and_update_first_step_us": round(evict_us, 2),
          "step_mask_ms": {"device_from_temporal": round(mask_ms, 3), "host_bools_uploaded": round(upload_ms, 3)},
          "kernels": "k_kv_copy, k_kv_remap (HBM), k_attn_mfma"}
    log(f"bench: kv cache attention {kv_attn_us:.1f} us, re-run put+update {put_us:.1f} us, "
        f"first step {evict_us:.1f} us")
    km.free()
    kvc.free()
    for bb in (kb_, vb_, qb_, ob_):
        bb.free()

    calibrate()

    configs = None
    if not args.no_configs:
        configs = per_config(be, H)
        log("bench: configs " + ", ".join(f"{k} {v['us_per_linear']:.1f} us ({v['pct_peak']:.0f}%)"
                                          for k, v in configs.items()))

    # roofline.traffic: the calibrated FETCH_SIZE + WRITE_SIZE bytes per launch
    # of the chunk's GEMMs (two rocprofv3 --pmc passes of --gemm-only, in the
    # committed summary)
    traffic = None
    if os.path.exists(TRAFFIC_FILE):
        tj = json.load(open(TRAFFIC_FILE))
        traffic = tj.get("l2_miss_bytes_per_launch", tj.get("hbm_bytes_per_launch"))

    cpu = None
    if not args.no_cpu:
        sys.path.insert(0, ROOT)
        cpu = cpu_baseline(args.cpu_seconds)
        log(f"bench: cpu baseline {cpu['value'] * 1e3:.2f} GFLOP/s on {cpu['cores']} threads")

    out = {
        "metric": "quant-linear TFLOP/s and % MFMA peak; DiT 30-layer linear ms per 3-frame chunk",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8",
        "data": "synthetic (random-init FP8 per-channel weights ~N(0,0.02); activations ~N(0,1) rounded to bf16, "
                "reaching each linear as its producer writes it: per-token or MX e4m3)",
        "config": {
            "workload": "cfg4: Wan2.1-1.3B 30-layer x 4-step FP8 block-linear set, one 3-frame chunk",
            "tokens": M, "text_tokens": TEXT, "layers": LAYERS, "dmd_steps": DMD,
            "gemms_per_layer_step": len(GEMMS), "linear_calls_per_step": n_linear, "tflop_per_step": round(step_flops / 1e12, 3),
            "activations": "bf16 values ~N(0,1) in the form each linear's producer writes: per-token e4m3 "
                           "(fused norms: QKV, cross Q, FFN up; the text once per prompt), MX e4m3 (attention's "
                           "epilogue: O, cross O; FFN up's epilogue: FFN down); bf16 out (FFN up: MX e4m3)",
            "weights_gb": round(wbytes / 1e9, 3),
            "cross_kv": "the 30 layers' K/V projections (512 text tokens) as one linear per step over their "
                        "concatenated weights",
        },
        "pct_fp8_peak": round(value / PEAK_FP8_TFLOPS * 100, 2),
        "ms_per_chunk": round(ms, 3),
        "ms_per_chunk_eager": round(ms_eager, 3),
        "ms_per_chunk_graph": round(ms_graph, 3) if ms_graph else None,
        "ms_per_chunk_bf16_input": round(ms_bf16_input, 3),
        "ms_per_chunk_bf16_input_eager_graph": [round(ms_bf16_e, 3), round(ms_bf16_g, 3) if ms_bf16_g else None],
        "ms_per_chunk_bf16_input_bf16_ffn_handoff": round(ms_bf16_handoff, 3),
        "ms_per_chunk_g128_weights": round(ms_g128, 3),
        "gemm_only_ms_per_chunk": round(gemm_ms, 3),
        "block_path_ms_per_chunk": {
            "unfused": block["unfused"], "fused": block["fused"],
            "what": "the chunk's 840 linears plus their producers and consumers (layer_norm, 2 residual_norm, "
                    "6 head_split (q / k RMS + RoPE, v; cross q; text k / v), gate_residual per layer-step; "
                    "attention and the KV cache excluded); fused = the norms write the FP8 linears' e4m3 inputs "
                    "in the same pass and FFN down's epilogue does the gate-residual add",
        },
        "act_quant_ms_per_chunk": 0.0,
        "act_quant_ms_per_chunk_bf16_input": round(region["act_quant_chunk"], 3),
        "per_gemm": per,
        "head_split": head_split,
        "causal_attention": attn,
        "kv_cache": kv,
        "per_config": configs,
        "roofline": {
            "bound": "mfma",
            "achieved": round(achieved, 1),
            "peak": PEAK_FP8_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_FP8_TFLOPS, 4),
            "traffic": traffic,
            "kernel": ("fp8 GEMM, all 7 shapes of the chunk (k_gemm_fp8_dma 128x256 for O, cross Q, cross O and "
                       "FFN down; the persistent k_gemm_fp8_ov 256x128 with the epilogue overlapped for QKV; the "
                       "persistent k_gemm_fp8_w4 256x256, one wave per SIMD, for FFN up and the 30-layer K/V call)"),
            "avg_launch_us": round(gemm_ms * 1e3 / n_linear, 2),
            # traffic (calibrated FETCH_SIZE + WRITE_SIZE) counts the L2's misses,
            # served by the 256 MB Infinity Cache or by HBM: gfx950's counters
            # have no HBM-only byte count, so this is L2-miss traffic per second
            "l2_miss_gbs": round(traffic / (gemm_ms * 1e-3 / n_linear) / 1e9, 1) if traffic else None,
            "alg_gbs": round(alg_per_launch / (gemm_ms * 1e-3 / n_linear) / 1e9, 1),
            "alg_bytes_per_launch": round(alg_per_launch),
            "launches_per_step": n_linear,
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    be.close()


if __name__ == "__main__":
    main()
