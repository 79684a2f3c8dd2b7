#!/usr/bin/env python3
"""Benchmark: dense bf16 linear layer on one MI355X through libinvision_hip.so.

    python bench.py [--steps K] [--warmup W] [--warmup-seconds S] [--gpus 1] [--workload c2] [--all]
                    [--no-cpu-baseline]

A step is one Y = X . W^T + bias over the workload's full shape, with X, W,
bias and Y resident in HBM (device pointers through the C ABI).  The default
workload is the FLUX2-Klein-4B fused QKV projection, M x K x N = 4608 x 3072 x
9216, bf16 X and W, fp32 bias and output, fp32 accumulation.

Warm-up runs at least W steps and at least S seconds of back-to-back steps
(default 1.5 s): the GPU's clock needs on the order of a second of sustained
load to reach its steady state, and a short warm-up times the ramp instead of
the kernel.  The line reports the warm-up steps actually run.

Prints ONE JSON line on stdout.  `roofline` uses the dense bf16 MFMA peak;
`achieved` is 2*M*N*K per launch over the average launch time measured with
HIP events on the library's stream across the timed steps.  `cpu_baseline` is
the reference's CPU GEMM algorithm (the oracle's restatement of qgemm/gemm_nt,
src/quicknncpu.pas:1241-1337) timed on this host, with the reference's own
sgemm2.cpp alongside when it was built.  Extra per-workload lines (--all) go to
stderr.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "GEMM TFLOP/s + % bf16 MFMA peak at 4608×3072×9216 (1 GPU)"
PEAK_BF16_TFLOPS = 2516.6   # 256 CU x 2.4 GHz x 4096 bf16 FLOP/clk/CU (dense)
PEAK_HBM_GBS = 8000.0

# name -> (description, M, K, N, bias, epilogue, x dtype, y dtype)
WORKLOADS = {
    "c1": ("single linear + bias (QNNLinear), fp32 X", 256, 3072, 3072, True, "none", "f32", "f32"),
    "c2": ("FLUX2-Klein-4B fused QKV projection", 4608, 3072, 9216, True, "none", "bf16", "f32"),
    "c3_up": ("DiT MLP up + SiLU, bf16 H out", 4608, 3072, 9216, True, "silu", "bf16", "bf16"),
    "c3_down": ("DiT MLP down", 4608, 9216, 3072, True, "none", "bf16", "f32"),
    "c4_gate_up": ("Qwen3-4B gate/up at M=512", 512, 2560, 9728, False, "none", "bf16", "f32"),
    "c4_down": ("Qwen3-4B down at M=512", 512, 9728, 2560, False, "none", "bf16", "f32"),
    "c5_qkv": ("Z-Image block QKV, 2 CFG branches", 9216, 3840, 11520, True, "none", "bf16", "f32"),
    "c5_out": ("Z-Image attention out", 9216, 3840, 3840, True, "none", "bf16", "f32"),
    "c5_up": ("Z-Image MLP up", 9216, 3840, 15360, True, "none", "bf16", "f32"),
    "c5_down": ("Z-Image MLP down", 9216, 15360, 3840, True, "none", "bf16", "f32"),
    "c5_adaln": ("Z-Image AdaLN modulation M=2", 2, 3840, 23040, True, "none", "bf16", "f32"),
    # N is the SwiGLU output width F: the GEMM runs over the 2F gate/up rows
    "flux2_swiglu": ("FLUX2 MLP gate/up with fused SiLU(gate)*up, bf16 H", 4608, 3072, 9216, True, "swiglu", "bf16",
                     "bf16"),
    "flux2_gated_out": ("FLUX2 attention out-projection into the gated fp32 residual", 4608, 3072, 3072, False,
                        "gated_add", "bf16", "f32"),
    "flux2_adaln_qkv": ("FLUX2 AdaLN of the fp32 residual stream fused into the QKV projection", 4608, 3072, 9216,
                        False, "adaln", "f32", "f32"),
}


# Attention shapes: (description, heads, kv_heads, seq_q, seq_k, head_dim, causal).
ATTN_WORKLOADS = {
    "flux2_attention": ("FLUX2-Klein-4B joint attention at 1024x1024 (4096 image + 512 text tokens)", 24, 24, 4608,
                        4608, 128, False),
    "zimage_attention": ("Z-Image block attention, 4096 tokens", 30, 30, 4096, 4096, 128, False),
    "qwen3_prefill_attention": ("Qwen3-4B causal grouped-query attention, 512 tokens", 32, 8, 512, 512, 128, True),
    # fp32 Q, K, V from the projections; each head's RMSNorm and the interleaved rotary
    # embedding of Q and K applied while they are staged (inv_hip_attention_qk_norm_rope)
    "flux2_qk_norm_rope_attention": ("FLUX2-Klein-4B QK norm + RoPE + joint attention, fp32 Q/K/V in", 24, 24, 4608,
                                     4608, 128, False),
}
ATTN_PREP = {"flux2_qk_norm_rope_attention"}

# VAE convolutions (QNNConv2d): (description, batch, in_ch, out_ch, H, W, kH, kW, stride, padding).  The
# decoder of a 1024x1024 image runs at 128, 256, 512 and 1024 pixels with 512, 512, 256 and 128
# channels (base 128, multipliers 1, 2, 4, 4: src/quicknn_vae.pas:560-627, 934-943).
CONV_WORKLOADS = {
    "vae_conv3x3_512ch_256px": ("FLUX2 VAE decoder ResNet conv at 256x256, 512 -> 512 channels", 1, 512, 512, 256,
                                256, 3, 3, 1, 1),
    "vae_conv3x3_128ch_1024px": ("FLUX2 VAE decoder ResNet conv at 1024x1024, 128 -> 128 channels", 1, 128, 128, 1024,
                                 1024, 3, 3, 1, 1),
    "vae_conv3x3_512ch_128px": ("VAE decoder mid-block ResNet conv at 128x128, 512 -> 512 channels", 1, 512, 512, 128,
                                128, 3, 3, 1, 1),
    "vae_conv3x3_256ch_512px": ("VAE decoder ResNet conv at 512x512, 256 -> 256 channels", 1, 256, 256, 512, 512, 3,
                                3, 1, 1),
    "vae_conv1x1_512ch_128px": ("VAE mid-block attention q/k/v projection (1x1) at 128x128, 512 channels", 1, 512,
                                512, 128, 128, 1, 1, 1, 0),
    "vae_conv1x1_256to128_1024px": ("VAE decoder ResNet skip (1x1) at 1024x1024, 256 -> 128 channels", 1, 256, 128,
                                    1024, 1024, 1, 1, 1, 0),
    "vae_conv_out_128to3_1024px": ("VAE decoder conv_out at 1024x1024, 128 -> 3 channels", 1, 128, 3, 1024, 1024, 3,
                                   3, 1, 1),
}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def make_inputs(M, K, N, seed=0):
    """Synthetic inputs of the workload's distributions, drawn in the order X, W, bias from the
    reference's sampler (src/quicknn_sample.pas:212-276) seeded with `seed`: X ~ N(0,1) (fp32; the
    bf16 workloads round it RNE), W ~ N(0,0.02) rounded to bf16, bias ~ N(0,0.01) fp32."""
    from invision_amd import quicknn_hip as q
    from invision_amd.bf16 import as_bf16_bits
    q.rng_seed(seed)
    X = q.randn((M, K), 1.0)
    W = as_bf16_bits(q.randn((N, K), 0.02, round_bf16=True))
    b = q.randn((N,), 0.01)
    return X, W, b


def gemm_parity_tol(epi, ydt):
    """Normwise tolerance of the sampled-row check against numpy float64 on the same bf16-rounded X
    (measured ~1e-6 for fp32 outputs): fp32 Y 1e-4; a bf16 Y adds half an ulp (2^-8); the AdaLN
    prologue normalises in fp32, and an element near a bf16 rounding boundary may round the other way
    than in the float64 check, so it gets the fp32-activation bound 2e-3."""
    tol = 2e-3 if epi == "adaln" else 1e-4
    return tol + (2.0 ** -8 if ydt == "bf16" else 0.0)


def gemm_rows(N, epi):
    """Weight rows the GEMM runs over (a gate/up pair has two per output column)."""
    return 2 * N if epi == "swiglu" else N


def algorithmic_bytes(M, K, N, bias, xdt, ydt, epi="none"):
    xs = 2 if xdt == "bf16" else 4
    ys = 2 if ydt == "bf16" else 4
    R = gemm_rows(N, epi)
    b = M * K * xs + R * K * 2 + M * N * ys + (4 * R if bias else 0)
    if epi == "gated_add":
        b += M * N * ys + 4 * N  # the residual read back, and the gate
    return b


MALL_BYTES = 256 << 20  # MI355X Infinity Cache


def run_workload(name, steps, warmup, check=True, host_path=False, warmup_seconds=0.0, cold=False):
    """Time one GEMM workload on device-resident operands.  cold=True rotates over enough copies of
    the weight (together more than twice the 256 MB Infinity Cache) that every launch reads its
    weight from HBM rather than from the cache the previous launch filled."""
    from invision_amd import hip
    from invision_amd import quicknn_hip as q
    from invision_amd.bf16 import as_bf16_bits, bf16_bits_to_f32

    desc, M, K, N, has_bias, epi, xdt, ydt = WORKLOADS[name]
    log(f"[bench] {name}: {desc} M={M} K={K} N={N} epilogue={epi} x={xdt} y={ydt}{' (cold weights)' if cold else ''}")
    R = gemm_rows(N, epi)
    X, W, b = make_inputs(M, K, R)
    Xin = as_bf16_bits(X) if xdt == "bf16" else X
    ncopies = (2 * MALL_BYTES) // (R * K * 2) + 2 if cold else 1
    ws = []
    for _ in range(ncopies):
        if epi == "swiglu":
            ws.append(q.Weight.gate_up(W[:N], W[N:], b[:N] if has_bias else None, b[N:] if has_bias else None))
        else:
            ws.append(q.Weight(W, b if has_bias else None))
    w = ws[0]
    turn = [0]

    def next_weight():
        turn[0] += 1
        return ws[turn[0] % ncopies]
    xd = q.DeviceArray.from_host(Xin, xdt)
    yd = q.DeviceArray((M, N), ydt)
    gd = None
    if epi == "adaln":
        rng = np.random.default_rng(3)
        shift = (rng.standard_normal(K, dtype=np.float32) * np.float32(0.3)).astype(np.float32)
        scale = (rng.standard_normal(K, dtype=np.float32) * np.float32(0.3)).astype(np.float32)
        sd, hd = q.DeviceArray.from_host(scale, "f32"), q.DeviceArray.from_host(shift, "f32")
    if epi == "gated_add":
        rng = np.random.default_rng(1)
        Y0 = rng.standard_normal((M, N), dtype=np.float32)
        yd.copy_from(Y0)
        gate = (rng.standard_normal(N, dtype=np.float32) * np.float32(0.5)).astype(np.float32)
        gd = q.DeviceArray.from_host(gate, "f32")

    def launch():
        wt = next_weight() if cold else w
        if epi == "adaln":
            hip.call("inv_hip_linear_norm", xd.ptr, hip.INV_NORM_ADALN, sd.ptr, hd.ptr, q.EPSILON, wt.handle, None,
                     yd.ptr, yd.inv_dtype, M, K, N, hip.INV_EPI_NONE, hip.INV_FLAG_DEVICE_PTRS | hip.INV_FLAG_ASYNC)
        elif epi == "gated_add":
            q.linear_gated_add_device(xd, wt, yd, M, gate=gd, asynchronous=True)
        else:
            q.linear_device(xd, wt, yd, M, epilogue=epi, asynchronous=True)

    if epi == "gated_add" and check:
        # parity on the first call's update, before timing accumulates into Y
        launch()
        hip.call("inv_hip_synchronize")
        Y1 = yd.to_host()
    warm_steps, tw = 0, time.perf_counter()
    while warm_steps < warmup or time.perf_counter() - tw < warmup_seconds:
        for _ in range(25):
            launch()
        warm_steps += 25
        hip.call("inv_hip_synchronize")
    # Timed region: host wall clock bracketed by synchronizations, and HIP
    # events on the library stream around the same launches.
    t0 = time.perf_counter()
    hip.call("inv_hip_timer_start")
    for _ in range(steps):
        launch()
    import ctypes
    ms = ctypes.c_float()
    hip.call("inv_hip_timer_stop", ctypes.byref(ms))
    hip.call("inv_hip_synchronize")
    t1 = time.perf_counter()
    wall_ms = (t1 - t0) * 1e3 / steps
    gpu_ms = ms.value / steps
    # Per-launch spread: each launch bracketed by its own events (outside the timed region).
    per = []
    for _ in range(min(steps, 30)):
        hip.call("inv_hip_timer_start")
        launch()
        hip.call("inv_hip_timer_stop", ctypes.byref(ms))
        per.append(ms.value)
    p10, p50, p90 = (float(v) for v in np.percentile(per, [10, 50, 90]))
    flops = 2.0 * M * R * K
    res = {"name": name + ("_cold" if cold else ""), "M": M, "K": K, "N": N, "gemm_rows": R,
           "weight_copies": ncopies, "warmup_steps": warm_steps, "wall_ms": wall_ms,
           "kernel_ms": gpu_ms, "tflops_wall": flops / (wall_ms * 1e-3) / 1e12,
           "tflops_kernel": flops / (gpu_ms * 1e-3) / 1e12,
           "bytes": algorithmic_bytes(M, K, N, has_bias, xdt, ydt, epi)}
    res["gbs_kernel"] = res["bytes"] / (gpu_ms * 1e-3) / 1e9
    res["launch_ms_p10_p50_p90"] = [round(p10, 5), round(p50, 5), round(p90, 5)]
    if host_path and epi in ("none", "silu", "gelu"):
        # The reference's own calling convention: fp32 X and Y in host memory,
        # copied over PCIe on every call (pinned bounce buffers), X rounded to
        # bf16 by the host on its way up.  Reported beside the device-resident
        # rate, never as it.
        # Y is the caller's buffer, written on every call (as the reference's
        # dst TMemoryBlock), not a fresh array whose first touch would be timed.
        Xh = np.ascontiguousarray(X if xdt == "f32" else bf16_bits_to_f32(Xin))
        Yh = np.zeros((M, R), np.float32)
        host_call = lambda: hip.call("inv_hip_linear", Xh.ctypes.data, hip.INV_DT_F32, w.handle, None, Yh.ctypes.data,
                                     hip.INV_DT_F32, M, K, R, hip.INV_EPI_NONE if epi == "none" else
                                     (hip.INV_EPI_SILU if epi == "silu" else hip.INV_EPI_GELU_ERF), 0)
        host_ms, res["host_fp32_io_serial_ms"] = host_times(host_call)
        res["host_fp32_io_ms"] = host_ms
        res["host_fp32_io_tflops"] = flops / (host_ms * 1e-3) / 1e12
    if check:
        # Spot parity on a few rows with numpy float64 (independent of the oracle).
        Y = Y1 if epi == "gated_add" else yd.to_host()
        Yf = bf16_bits_to_f32(Y) if ydt == "bf16" else Y.astype(np.float64)
        rows = np.unique(np.linspace(0, M - 1, num=min(M, 6)).astype(int))
        Xs = X[rows]
        if epi == "adaln":
            Xs = Xs.astype(np.float64)
            mu = Xs.mean(1, keepdims=True)
            Xs = (1 + scale) * ((Xs - mu) / np.sqrt(((Xs - mu) ** 2).mean(1, keepdims=True) + 1e-6)) + shift
        Xr = bf16_bits_to_f32(as_bf16_bits(np.asarray(Xs, np.float32))).astype(np.float64)
        ref = Xr @ bf16_bits_to_f32(W).astype(np.float64).T
        if has_bias:
            ref += b.astype(np.float64)
        if epi == "silu":
            ref = ref / (1.0 + np.exp(-ref))
        elif epi == "swiglu":
            g, u = ref[:, :N], ref[:, N:]
            ref = g / (1.0 + np.exp(-g)) * u
        elif epi == "gated_add":
            ref = gate.astype(np.float64) * ref  # compared on the update Y1 - Y0
            Yf = Yf[rows] - Y0[rows]
            rows = slice(None)
        err = float(np.max(np.abs(Yf[rows] - ref)) / np.max(np.abs(ref)))
        res["parity_normwise_sampled_rows"] = err
        res["parity_tol"] = gemm_parity_tol(epi, ydt)
        res["parity_ok"] = bool(err <= res["parity_tol"])
    xd.free()
    yd.free()
    for wt in ws:
        wt.free()
    if gd is not None:
        gd.free()
    if epi == "adaln":
        sd.free()
        hd.free()
    return res


def gemm_constant_operands(name, seconds=1.5, steps=200):
    """The same GEMM launch with every X and W element 2^-7 (exact in bf16): identical instructions
    and memory traffic, operands that do not toggle.  Its rate against the random-operand rate shows
    how much of the gap to peak is the data-dependent power of the matrix cores."""
    import ctypes
    from invision_amd import hip
    from invision_amd import quicknn_hip as q
    from invision_amd.bf16 import as_bf16_bits
    desc, M, K, N, has_bias, epi, xdt, ydt = WORKLOADS[name]
    w = q.Weight(as_bf16_bits(np.full((N, K), 2.0 ** -7, np.float32)), np.zeros(N, np.float32) if has_bias else None)
    xd = q.DeviceArray.from_host(as_bf16_bits(np.full((M, K), 2.0 ** -7, np.float32)), "bf16")
    yd = q.DeviceArray((M, N), ydt)
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(25):
            q.linear_device(xd, w, yd, M, asynchronous=True)
        hip.call("inv_hip_synchronize")
    ms = ctypes.c_float()
    hip.call("inv_hip_timer_start")
    for _ in range(steps):
        q.linear_device(xd, w, yd, M, asynchronous=True)
    hip.call("inv_hip_timer_stop", ctypes.byref(ms))
    ok = bool(np.all(yd.to_host()[:4] == np.float32(K * 2.0 ** -14)))  # exact: K products of 2^-14
    for a in (w, xd, yd):
        a.free()
    return {"tflops": round(2.0 * M * N * K / (ms.value / steps * 1e-3) / 1e12, 1), "exact": ok}


def mfma_ceiling(gemm_tflops):
    """The register-only MFMA loop of libinv_probe.so on this GPU, now: the rate a
    GEMM on the same operand distributions could reach with zero memory traffic
    under the board's power limit, and the same with constant operands."""
    import ctypes
    from invision_amd import build as B
    if not os.path.exists(B.PROBE_PATH):
        log("[bench] libinv_probe.so not built: no MFMA ceiling")
        return None
    lib = ctypes.CDLL(B.PROBE_PATH)
    lib.inv_probe_mfma_ceiling.restype = ctypes.c_int
    lib.inv_probe_mfma_ceiling.argtypes = [ctypes.c_double, ctypes.c_double, ctypes.POINTER(ctypes.c_double),
                                           ctypes.POINTER(ctypes.c_double)]
    r, c = ctypes.c_double(), ctypes.c_double()
    rc = lib.inv_probe_mfma_ceiling(1.0, 1.0, ctypes.byref(r), ctypes.byref(c))
    if rc != 0:
        log(f"[bench] MFMA ceiling probe failed ({rc})")
        return None
    out = {"random_operands_tflops": round(r.value, 1), "constant_operands_tflops": round(c.value, 1),
           "gemm_frac_of_random_ceiling": round(gemm_tflops / r.value, 4),
           "what": "v_mfma_f32_32x32x16_bf16 over a 128x128 wave tile from registers only, 1 wave/SIMD, all CUs, "
                   "sustained 1 s; W ~ N(0,0.02) and X ~ N(0,1) in bf16, or constant operands"}
    log(f"[bench] MFMA ceiling: {json.dumps(out)}")
    return out


def vendor_gemm(workload):
    """The same GEMM through torch on this GPU (its bf16 matmul runs hipBLASLt on ROCm), on the
    same X, W and bias values (make_inputs), as a same-run comparator for the headline kernel.
    torch carries its own HIP runtime, so it runs in a child process that never loads this
    library; the inputs go to it through .npy files."""
    import subprocess
    import tempfile
    desc, M, K, N, has_bias, epi, xdt, ydt = WORKLOADS[workload]
    X, W, b = make_inputs(M, K, N)
    with tempfile.TemporaryDirectory(dir="/tmp") as d:
        np.save(os.path.join(d, "x.npy"), X)
        np.save(os.path.join(d, "w.npy"), W)
        np.save(os.path.join(d, "b.npy"), b)
        r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--vendor-gemm-child", d,
                            "--workload", workload], capture_output=True, text=True, timeout=300)
    if r.returncode != 0:
        raise RuntimeError(f"comparator exited {r.returncode}: {r.stderr[-500:]}")
    return json.loads(r.stdout.strip().splitlines()[-1])


def vendor_gemm_child(d, workload, steps=50, warmup_seconds=1.0):
    """Child side of vendor_gemm: Y = X . W^T + bias by torch.addmm on bf16 X and W, fp32 output
    where torch offers out_dtype=float32 for bf16 operands, else bf16 output (half the bytes
    written); prints one JSON line."""
    import torch
    from invision_amd.bf16 import round_bf16
    desc, M, K, N, has_bias, epi, xdt, ydt = WORKLOADS[workload]
    X, W, b = (np.load(os.path.join(d, f + ".npy")) for f in ("x", "w", "b"))
    dev = torch.device("cuda:0")
    xt = torch.from_numpy(round_bf16(X)).to(dev).to(torch.bfloat16)
    wt = torch.from_numpy(W.view(np.int16)).to(dev).view(torch.bfloat16)
    bt = torch.from_numpy(b).to(dev)
    wtt = wt.t()
    fn, out = (lambda: torch.addmm(bt, xt, wtt, out_dtype=torch.float32)), "f32"
    try:
        y = fn()
    except Exception:
        bb = bt.to(torch.bfloat16)
        fn, out = (lambda: torch.addmm(bb, xt, wtt)), "bf16"
        y = fn()
    torch.cuda.synchronize()
    ref = round_bf16(X[:8]).astype(np.float64) @ ((W.astype(np.uint32) << 16).view(np.float32)
                                                   .astype(np.float64)).T + b
    err = float(np.abs(y[:8].float().cpu().numpy() - ref).max() / np.abs(ref).max())
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < warmup_seconds:
        for _ in range(10):
            fn()
        torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    print(json.dumps({"what": f"torch.addmm on the same bf16 X, W and fp32 bias, {out} Y, torch {torch.__version__}"
                              f" (hipBLASLt)", "tflops": round(2.0 * M * N * K / (ms * 1e-3) / 1e12, 1),
                      "ms": round(ms, 5), "normwise_err_first_rows": err}), flush=True)
    return 0


def time_host_call(call):
    """Wall milliseconds per call of a host-pointer entry point (one untimed call,
    then at least 3 calls and 1 s)."""
    call()
    reps, th = 0, time.perf_counter()
    while reps < 3 or time.perf_counter() - th < 1.0:
        call()
        reps += 1
    return (time.perf_counter() - th) * 1e3 / reps


def host_times(call):
    """(banded, serial) wall ms of a host-pointer call: the library's default
    overlaps upload, kernels and download in bands; INV_HIP_HOST_PIPELINE=0 is
    the one serial pass."""
    banded = time_host_call(call)
    prev = os.environ.get("INV_HIP_HOST_PIPELINE")
    os.environ["INV_HIP_HOST_PIPELINE"] = "0"
    try:
        serial = time_host_call(call)
    finally:
        if prev is None:
            del os.environ["INV_HIP_HOST_PIPELINE"]
        else:
            os.environ["INV_HIP_HOST_PIPELINE"] = prev
    return banded, serial


def run_attention(name, steps, warmup_seconds=0.5, check=True, host_path=False):
    """inv_hip_attention on resident bf16 Q, K, V; FLOP = 4 * seq_q * seq_k * head_dim * heads
    (halved for causal: the keys after the diagonal are skipped).  host_path: also
    the wall time of the call on fp32 Q, K, V and O in host memory (the reference's
    calling convention), banded and serial."""
    import ctypes
    from invision_amd import hip
    from invision_amd import quicknn_hip as q
    from invision_amd.bf16 import as_bf16_bits, bf16_bits_to_f32
    desc, heads, kvh, sq, sk, d, causal = ATTN_WORKLOADS[name]
    log(f"[bench] {name}: {desc} heads={heads} kv_heads={kvh} seq_q={sq} seq_k={sk} head_dim={d} causal={causal}")
    rng = np.random.default_rng(2)
    prep = name in ATTN_PREP
    Qf, Kf, Vf = (rng.standard_normal(sh, dtype=np.float32) for sh in ((sq, heads * d), (sk, kvh * d), (sk, kvh * d)))
    if prep:
        wq, wk = (np.float32(1.0) + np.float32(0.1) * rng.standard_normal(d, dtype=np.float32) for _ in range(2))
        th = rng.uniform(-np.pi, np.pi, (max(sq, sk), d // 2)).repeat(2, axis=1)  # pairs share an angle
        cos_t, sin_t = np.cos(th).astype(np.float32), np.sin(th).astype(np.float32)
        qd, kd, vd, wqd, wkd, cd, sd = (q.DeviceArray.from_host(a, "f32") for a in (Qf, Kf, Vf, wq, wk, cos_t, sin_t))
        Q, K, V = Qf, Kf, Vf
    else:
        Q, K, V = (as_bf16_bits(a) for a in (Qf, Kf, Vf))
        qd, kd, vd = (q.DeviceArray.from_host(a, "bf16") for a in (Q, K, V))
    od = q.DeviceArray((sq, heads * d), "bf16")

    def launch():
        if prep:
            hip.call("inv_hip_attention_qk_norm_rope", qd.ptr, 0, kd.ptr, 0, vd.ptr, 0, od.ptr, hip.INV_DT_BF16,
                     heads, kvh, sq, sk, d, 1.0 / float(np.sqrt(d)), wqd.ptr, wkd.ptr, hip.INV_ROPE_INTERLEAVED,
                     cd.ptr, sd.ptr, cd.ptr, sd.ptr, None, hip.INV_FLAG_DEVICE_PTRS | hip.INV_FLAG_ASYNC)
        else:
            q.attention_device(qd, kd, vd, od, heads=heads, head_dim=d, kv_heads=kvh, causal=causal,
                               asynchronous=True)

    warm, tw = 0, time.perf_counter()
    while warm < 3 or time.perf_counter() - tw < warmup_seconds:
        for _ in range(10):
            launch()
        warm += 10
        hip.call("inv_hip_synchronize")
    ms = ctypes.c_float()
    t0 = time.perf_counter()
    hip.call("inv_hip_timer_start")
    for _ in range(steps):
        launch()
    hip.call("inv_hip_timer_stop", ctypes.byref(ms))
    hip.call("inv_hip_synchronize")
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    gpu_ms = ms.value / steps
    flops = 4.0 * sq * sk * d * heads * (0.5 if causal else 1.0)
    res = {"name": name, "heads": heads, "kv_heads": kvh, "seq_q": sq, "seq_k": sk, "head_dim": d, "causal": causal,
           "warmup_steps": warm, "wall_ms": wall_ms, "kernel_ms": gpu_ms, "tflops_kernel": flops / (gpu_ms * 1e-3) / 1e12,
           "tflops_wall": flops / (wall_ms * 1e-3) / 1e12}
    if check:
        import math
        # fp64 spot check of a few query rows of head 0 (numpy, independent of the oracle)
        O = bf16_bits_to_f32(od.to_host())
        rows = np.unique(np.linspace(0, sq - 1, num=min(sq, 4)).astype(int))
        if prep:
            def norm_rope(x, w, tok):  # head 0: RMSNorm over d, then pairs (2k, 2k+1) rotated
                x = x.astype(np.float64)
                x = x / np.sqrt((x ** 2).mean(1, keepdims=True) + 1e-6) * w
                c, s_ = cos_t[tok].astype(np.float64), sin_t[tok].astype(np.float64)
                y = np.empty_like(x)
                y[:, 0::2] = x[:, 0::2] * c[:, 0::2] - x[:, 1::2] * s_[:, 0::2]
                y[:, 1::2] = x[:, 1::2] * c[:, 0::2] + x[:, 0::2] * s_[:, 0::2]
                return y
            qh = norm_rope(Qf[rows, :d], wq, rows)
            kh = norm_rope(Kf[:, :d], wk, np.arange(sk))
            vh = Vf[:, :d].astype(np.float64)
        else:
            qh = bf16_bits_to_f32(Q)[rows, :d].astype(np.float64)
            kh = bf16_bits_to_f32(K)[:, :d].astype(np.float64)
            vh = bf16_bits_to_f32(V)[:, :d].astype(np.float64)
        S = qh @ kh.T / math.sqrt(d)
        if causal:
            S[np.arange(sk)[None, :] > rows[:, None] + (sk - sq)] = -np.inf
        P = np.exp(S - S.max(1, keepdims=True))
        ref = (P / P.sum(1, keepdims=True)) @ vh
        res["parity_normwise_sampled_rows"] = float(np.max(np.abs(O[rows, :d] - ref)) / np.max(np.abs(ref)))
        # bf16 Q/K/V and softmax weights (4e-3) plus the bf16 output (2^-8); the norm + rotary workload
        # is checked against unrounded fp32 inputs, which adds their bf16 rounding (1.5e-2 in the tests)
        res["parity_tol"] = (1.5e-2 if prep else 4e-3) + 2.0 ** -8
        res["parity_ok"] = bool(res["parity_normwise_sampled_rows"] <= res["parity_tol"])
    if host_path and not prep:
        Oh = np.zeros((sq, heads * d), np.float32)
        host_call = lambda: hip.call("inv_hip_attention", Qf.ctypes.data, Kf.ctypes.data, Vf.ctypes.data,
                                     Oh.ctypes.data, hip.INV_DT_F32, hip.INV_DT_F32, heads, kvh, sq, sk, d,
                                     1.0 / float(np.sqrt(d)), hip.INV_ATTN_CAUSAL if causal else 0)
        res["host_fp32_io_ms"], res["host_fp32_io_serial_ms"] = host_times(host_call)
    for a in (qd, kd, vd, od) + ((wqd, wkd, cd, sd) if prep else ()):
        a.free()
    return res


def run_conv(name, steps, warmup_seconds=0.5, check=True, host_path=False):
    """inv_hip_conv2d on a device-resident fp32 NCHW image (im2col into the bf16
    patch matrix, then the GEMM with the per-channel bias); FLOP = 2 * out_ch *
    outH * outW * in_ch * kH * kW.  The patch matrix is written once per call:
    outH * outW * round_up(K, 64) * 2 bytes.  host_path: also the wall time of
    the call on an fp32 image and output in host memory."""
    import ctypes
    from invision_amd import hip
    from invision_amd import quicknn_hip as q
    from invision_amd.bf16 import round_bf16
    desc, b, c, oc, H, W, kH, kW, s, p = CONV_WORKLOADS[name]
    log(f"[bench] {name}: {desc} batch={b} in_ch={c} out_ch={oc} {H}x{W} k={kH}x{kW} stride={s} pad={p}")
    rng = np.random.default_rng(4)
    K = c * kH * kW
    x = rng.standard_normal((b, c, H, W), dtype=np.float32)
    w = rng.standard_normal((oc, K), dtype=np.float32) * np.float32(1.0 / np.sqrt(K))
    bias = rng.standard_normal(oc, dtype=np.float32) * np.float32(0.01)
    _, _, oH, oW = q.QNNConv2DShape(b, oc, H, W, kH, kW, p, s)
    wt = q.Weight(w, bias)
    xd = q.DeviceArray.from_host(x, "f32")
    yd = q.DeviceArray((b, oc, oH, oW), "f32")
    flags = hip.INV_FLAG_DEVICE_PTRS | hip.INV_FLAG_ASYNC

    def launch():
        hip.call("inv_hip_conv2d", xd.ptr, wt.handle, None, yd.ptr, c, oc, H, W, kH, kW, s, p, b, flags)

    warm, tw = 0, time.perf_counter()
    while warm < 3 or time.perf_counter() - tw < warmup_seconds:
        launch()
        warm += 1
        hip.call("inv_hip_synchronize")
    ms = ctypes.c_float()
    hip.call("inv_hip_timer_start")
    for _ in range(steps):
        launch()
    hip.call("inv_hip_timer_stop", ctypes.byref(ms))
    hip.call("inv_hip_synchronize")
    t = ms.value / steps
    flops = 2.0 * b * oc * oH * oW * K
    col_bytes = oH * oW * ((K + 63) // 64 * 64) * 2
    res = {"name": name, "batch": b, "in_ch": c, "out_ch": oc, "H": H, "W": W, "kH": kH, "kW": kW, "stride": s,
           "padding": p, "warmup_steps": warm, "kernel_ms": t, "gflop": flops / 1e9,
           "tflops_kernel": flops / (t * 1e-3) / 1e12, "patch_matrix_bytes": col_bytes}
    if check:
        # fp64 spot check of 8 output pixels over every output channel (numpy, independent of the oracle)
        y = yd.to_host()
        xb = np.pad(round_bf16(x).astype(np.float64), ((0, 0), (0, 0), (p, p), (p, p)))
        wr = round_bf16(w).astype(np.float64)
        pix = np.unique(np.linspace(0, oH * oW - 1, num=8).astype(int))
        err, top = 0.0, 0.0
        for pp in pix:
            oh, ow = divmod(int(pp), oW)
            patch = xb[0, :, oh * s:oh * s + kH, ow * s:ow * s + kW].reshape(-1)
            ref = wr @ patch + bias
            err = max(err, float(np.abs(y[0, :, oh, ow] - ref).max()))
            top = max(top, float(np.abs(ref).max()))
        res["parity_normwise_sampled_pixels"] = err / top
        res["parity_tol"] = 1e-4  # same bf16 image and filter values, fp32 accumulation
        res["parity_ok"] = bool(err / top <= res["parity_tol"])
    if host_path:
        yh = np.zeros((b, oc, oH, oW), np.float32)
        res["host_fp32_io_ms"] = time_host_call(
            lambda: hip.call("inv_hip_conv2d", x.ctypes.data, wt.handle, None, yh.ctypes.data, c, oc, H, W, kH, kW,
                             s, p, b, 0))
    xd.free()
    yd.free()
    wt.free()
    return res


def run_block(steps, warmup_seconds=0.5):
    """A FLUX2-Klein-4B double block at 1024x1024 with its text and image streams
    taken as one 4608-token stream under one weight set (24 heads of 128, MLP
    9216), device-resident, in the
    reference's order (src/quicknn_transformers.pas:1400-1460): AdaLN + QKV
    projection (one GEMM), QK norm + RoPE + attention (one call), gated output
    projection, AdaLN + SwiGLU gate/up (one GEMM), gated down projection.
    FLOP: the five GEMMs' 2*M*N*K plus attention's 4*seq^2*D*heads."""
    import ctypes
    from invision_amd import hip
    from invision_amd import quicknn_hip as q
    S, H, heads, D, F = 4608, 3072, 24, 128, 9216
    log(f"[bench] flux2_double_block_image_stream: tokens={S} hidden={H} heads={heads} mlp={F}")
    rng = np.random.default_rng(3)
    bf = lambda shape: (rng.standard_normal(shape, dtype=np.float32) * np.float32(0.02))
    wqkv = q.Weight(bf((3 * H, H)))
    wo = q.Weight(bf((H, H)), rng.standard_normal(H, dtype=np.float32) * np.float32(0.01))
    wgu = q.Weight.gate_up(q.as_bf16_bits(bf((F, H))), q.as_bf16_bits(bf((F, H))))
    wd = q.Weight(bf((H, F)), rng.standard_normal(H, dtype=np.float32) * np.float32(0.01))
    vec = lambda n, s: q.DeviceArray.from_host((rng.standard_normal(n, dtype=np.float32) * np.float32(s)), "f32")
    x = q.DeviceArray.from_host(rng.standard_normal((S, H), dtype=np.float32), "f32")
    sh1, sc1, g1, sh2, sc2, g2 = (vec(H, 0.1) for _ in range(6))
    qw, kw = (q.DeviceArray.from_host(np.ones(D, np.float32) + rng.standard_normal(D, dtype=np.float32) * np.float32(0.1),
                                      "f32") for _ in range(2))
    th = rng.uniform(-np.pi, np.pi, (S, D // 2)).repeat(2, axis=1)
    ct, st = (q.DeviceArray.from_host(f(th).astype(np.float32), "f32") for f in (np.cos, np.sin))
    qkv = q.DeviceArray((S, 3 * H), "f32")
    attn = q.DeviceArray((S, H), "bf16")
    h = q.DeviceArray((S, F), "bf16")
    dev = hip.INV_FLAG_DEVICE_PTRS | hip.INV_FLAG_ASYNC

    def block():
        hip.call("inv_hip_linear_norm", x.ptr, hip.INV_NORM_ADALN, sc1.ptr, sh1.ptr, q.EPSILON, wqkv.handle, None,
                 qkv.ptr, hip.INV_DT_F32, S, H, 3 * H, hip.INV_EPI_NONE, dev)
        # Q, K and V read in place from the thirds of the fused projection (token stride 3H)
        hip.call("inv_hip_attention_qk_norm_rope", qkv.ptr, 3 * H, qkv.ptr + H * 4, 3 * H, qkv.ptr + 2 * H * 4, 3 * H,
                 attn.ptr, hip.INV_DT_BF16, heads, heads, S, S, D, 1.0 / float(np.sqrt(D)), qw.ptr, kw.ptr,
                 hip.INV_ROPE_INTERLEAVED, ct.ptr, st.ptr, ct.ptr, st.ptr, None, dev)
        hip.call("inv_hip_linear_gated_add", attn.ptr, hip.INV_DT_BF16, wo.handle, None, g1.ptr, x.ptr, S, H, H, dev)
        hip.call("inv_hip_linear_norm", x.ptr, hip.INV_NORM_ADALN, sc2.ptr, sh2.ptr, q.EPSILON, wgu.handle, None, h.ptr,
                 hip.INV_DT_BF16, S, H, F, hip.INV_EPI_SWIGLU, dev)
        hip.call("inv_hip_linear_gated_add", h.ptr, hip.INV_DT_BF16, wd.handle, None, g2.ptr, x.ptr, S, F, H, dev)

    warm, tw = 0, time.perf_counter()
    while warm < 3 or time.perf_counter() - tw < warmup_seconds:
        block()
        warm += 1
        hip.call("inv_hip_synchronize")
    ms = ctypes.c_float()
    hip.call("inv_hip_timer_start")
    for _ in range(steps):
        block()
    hip.call("inv_hip_timer_stop", ctypes.byref(ms))
    t = ms.value / steps
    gemm = 2.0 * S * H * (3 * H) + 2.0 * S * H * H + 2.0 * S * (2 * F) * H + 2.0 * S * H * F
    flops = gemm + 4.0 * S * S * D * heads
    for a in (x, sh1, sc1, g1, sh2, sc2, g2, qw, kw, ct, st, qkv, attn, h):
        a.free()
    for w in (wqkv, wo, wgu, wd):
        w.free()
    return {"name": "flux2_double_block_image_stream", "tokens": S, "hidden": H, "heads": heads, "mlp": F,
            "warmup_steps": warm, "kernel_ms": t, "gflop": flops / 1e9, "tflops_kernel": flops / (t * 1e-3) / 1e12}


def _median_run(fn, runs=5):
    """One warm-up call, then the median wall time (s) of `runs` calls."""
    import statistics
    fn()
    ts = []
    for _ in range(runs):
        t = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t)
    return statistics.median(ts)


def cpu_share():
    """CPUs this process may run on (its affinity), capped at 16: the GPU box grants a 16-CPU share of
    its host to a one-GPU job whatever nproc reports, and more threads only oversubscribe it."""
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count() or 1
    return max(1, min(16, avail))


def cpu_baseline(name):
    """The reference's CPU GEMM on this host (a baseline, not the target), following the CPU timing
    method of the benchmark plan: median of 5 runs after 1 warm-up, with every CPU of this job's
    share and with 1 thread, on identical fp32 inputs (X ~ N(0,1), W ~ N(0,0.02) widened from bf16).

    - value: the qgemm / gemm_nt fallback the reference binds when no BLAS library is found
      (src/quicknncpu.pas:1176-1180, 1241-1337, src/ops_avx2.inc:1407-1508), restated in
      oracle/oracle.c (kind "port"), over the full shape with all threads;
    - openblas_cblas_sgemm: OpenBLAS cblas_sgemm, the library the reference binds by default on Linux
      (src/quicknncpu.pas:3967-3981, the call at :350), here numpy's bundled OpenBLAS build (the host
      has no system libopenblas), reached by numpy's matmul with the same RowMajor NoTrans/Trans GEMM;
    - reference_sgemm2: the reference's own src/sgemm2.cpp (OpenMP, 4x4x128 tiles) compiled unchanged;
    - bf16_widening: BF16ToSingle of the whole weight (src/quicknn_common.pas:1991-2008), the per-load
      and per-call conversion the reference performs before an fp32 GEMM.
    The 1-thread figures run on the first 256 rows of X (the GEMM's rate per row is flat in M)."""
    import threadpoolctl

    import oracle
    from invision_amd import quicknn_hip as q
    desc, M, K, N, has_bias, epi, xdt, ydt = WORKLOADS[name]
    threads = cpu_share()
    X, Wb, _ = make_inputs(M, K, N)
    A = np.ascontiguousarray(X)
    B = oracle.bf16_to_f32(Wb)
    C = np.zeros((M, N), np.float32)
    m1 = min(M, 256)
    fl = lambda m: 2.0 * m * N * K

    def entry(seconds, m, nthr):
        return {"ms": round(seconds * 1e3, 3), "tflops": round(fl(m) / seconds / 1e12, 4), "threads": nthr,
                "shape": f"{m}x{K}x{N}"}

    t_all = _median_run(lambda: oracle.qgemm(oracle.NO_TRANS, oracle.TRANS, M, N, K, 1.0, A, K, B, K, 0.0, C, N,
                                             threads))
    t_one = _median_run(lambda: oracle.qgemm(oracle.NO_TRANS, oracle.TRANS, m1, N, K, 1.0, A, K, B, K, 0.0, C, N, 1))
    out = {"value": fl(M) / t_all / 1e12, "unit": "TFLOP/s", "cores": threads, "kind": "port",
           "sample": f"the full {M}x{K}x{N} fp32 GEMM, median of 5 runs after 1 warm-up, {threads} threads: the "
                     f"reference's qgemm/gemm_nt fallback (8-row tiles over threads, 8-lane AVX2 FMA dots) restated "
                     f"in oracle/oracle.c; 1-thread figures on {m1} rows",
           "qgemm_port": {"all_threads": entry(t_all, M, threads), "one_thread": entry(t_one, m1, 1)}}
    with threadpoolctl.threadpool_limits(limits=threads, user_api="blas"):
        t_b = _median_run(lambda: np.matmul(A, B.T, out=C))
    with threadpoolctl.threadpool_limits(limits=1, user_api="blas"):
        t_b1 = _median_run(lambda: np.matmul(A[:m1], B.T, out=C[:m1]))
    info = [i for i in threadpoolctl.threadpool_info() if i.get("internal_api") == "openblas"]
    out["openblas_cblas_sgemm"] = {"all_threads": entry(t_b, M, threads), "one_thread": entry(t_b1, m1, 1),
                                   "library": (f"OpenBLAS {info[0].get('version')} ({info[0].get('architecture')}), "
                                               f"numpy's bundled build") if info else "numpy's bundled BLAS"}
    if oracle.ref_lib() is not None:
        with threadpoolctl.threadpool_limits(limits=threads, user_api="openmp"):
            t_r = _median_run(lambda: oracle.sgemm2_ref_nt(A, B))
        with threadpoolctl.threadpool_limits(limits=1, user_api="openmp"):
            t_r1 = _median_run(lambda: oracle.sgemm2_ref_nt(A[:m1], B))
        out["reference_sgemm2"] = {"all_threads": entry(t_r, M, threads), "one_thread": entry(t_r1, m1, 1)}
    t_w = _median_run(lambda: oracle.bf16_to_f32(Wb))
    out["bf16_widening"] = {"ms": round(t_w * 1e3, 3), "elements": int(Wb.size), "threads": 1,
                            "gbs": round(Wb.size * 6 / t_w / 1e9, 2)}
    out["nproc"] = os.cpu_count()
    try:
        out["cpu_model"] = next(l.split(":", 1)[1].strip() for l in open("/proc/cpuinfo") if "model name" in l)
    except Exception:
        pass
    return out


def profile_run(args):
    """Launches for counter collection: copy_words16 over 512 MiB (known traffic:
    512 MiB read + 512 MiB written per launch), then the workload."""
    from invision_amd import hip
    from invision_amd import quicknn_hip as q
    n = 512 << 20
    a = q.DeviceArray((n // 4,), "f32")
    b = q.DeviceArray((n // 4,), "f32")
    a.fill_zero()
    for _ in range(5):
        hip.call("inv_hip_memcpy_d2d", b.ptr, a.ptr, n)
    a.free()
    b.free()
    log(f"[profile] copy calibration: 5 x copy_words16 of {n} bytes")
    if args.workload in ATTN_WORKLOADS:
        res = run_attention(args.workload, args.steps, warmup_seconds=args.warmup_seconds, check=False)
    elif args.workload in CONV_WORKLOADS:
        res = run_conv(args.workload, args.steps, warmup_seconds=args.warmup_seconds, check=False)
    else:
        res = run_workload(args.workload, args.steps, args.warmup, check=False, warmup_seconds=args.warmup_seconds,
                           cold=args.cold)
    log(f"[profile] {json.dumps(res)}")
    print(json.dumps({"profile_run": args.workload, "copy_bytes": n, **res}), flush=True)
    q.shutdown()
    return 0


# Per-kernel activity counters of one rocprofv3 pass (7 SQ + 1 GRBM counters: within one pass's limits).
BUSY_COUNTERS = ("GRBM_GUI_ACTIVE SQ_BUSY_CU_CYCLES SQ_VALU_MFMA_BUSY_CYCLES SQ_INSTS_VALU_MFMA_MOPS_BF16 "
                 "SQ_WAVE_CYCLES SQ_WAIT_INST_LDS SQ_LDS_BANK_CONFLICT SQ_INSTS_LDS")
L2_COUNTERS = "TCC_HIT_sum TCC_MISS_sum"


def profile_passes(workload, out_dir, cold=False):
    """The rocprofv3 runs a profile summary is made from, each in its own process started from /tmp:
    (name, argv, time limit in s).  A kernel trace over the timed launches, then one counter pass
    each for FETCH_SIZE, WRITE_SIZE, the activity counters and the L2 hit counters."""
    bench = os.path.join(ROOT, "bench.py")
    run = ["python3", bench, "--profile-run", "--workload", workload] + (["--cold"] if cold else [])
    short = ["--steps", "5", "--warmup", "1", "--warmup-seconds", "0"]

    def pmc(name, counters, tail, limit):
        return (name, ["rocprofv3", "--pmc"] + counters.split() + ["-d", os.path.join(out_dir, name), "-o", workload,
                                                                  "--output-format", "csv", "--"] + run + tail, limit)
    return [("trace", ["rocprofv3", "--kernel-trace", "--stats", "-d", os.path.join(out_dir, "trace"), "-o", workload,
                       "--output-format", "csv", "--"] + run + ["--steps", "50", "--warmup", "5"], 240),
            pmc("fetch", "FETCH_SIZE", short, 90),
            pmc("write", "WRITE_SIZE", short, 90),
            pmc("busy", BUSY_COUNTERS, ["--steps", "20", "--warmup", "5", "--warmup-seconds", "0.5"], 120),
            pmc("l2", L2_COUNTERS, short, 90)]


def shown(argv):
    """A pass's command line as the summaries print it (the repository root as <repo>)."""
    return "cd /tmp && TMPDIR=/tmp " + " ".join(argv).replace(ROOT, "<repo>")


def profile_all(workload, out_dir, cold=False):
    """Run every pass of profile_passes() as a child process (this process never touches the GPU),
    then write the profiles/ summary; the raw trace and counter tables are deleted afterwards."""
    import glob
    import subprocess
    os.makedirs(out_dir, exist_ok=True)
    env = dict(os.environ, TMPDIR="/tmp")
    dirs = {}
    for name, argv, limit in profile_passes(workload, out_dir, cold):
        log(f"[profile-all] {workload}{' cold' if cold else ''}: {name} pass", )
        logf = os.path.join(out_dir, name + ".log")
        try:
            with open(logf, "w") as lf:
                rc = subprocess.run(argv, cwd="/tmp", env=env, stdout=lf, stderr=subprocess.STDOUT,
                                    timeout=limit).returncode
        except subprocess.TimeoutExpired:
            log(f"[profile-all] {name} pass exceeded {limit} s; stopping")
            return 1
        if rc != 0:
            log(f"[profile-all] {name} pass failed ({rc}):\n" + "".join(open(logf).readlines()[-15:]))
            return 1
        dirs[name] = os.path.join(out_dir, name)
    summarize_profile(workload, dirs["trace"], dirs["fetch"], dirs["write"], dirs["busy"], dirs["l2"], cold=cold,
                      out_dir=out_dir)
    for pat in ("*kernel_trace.csv", "*counter_collection.csv", "*agent_info.csv"):
        for f in glob.glob(os.path.join(out_dir, "**", pat), recursive=True):
            os.remove(f)
    return 0


def summarize_profile(workload, trace_dir, fetch_dir, write_dir, busy_dir=None, l2_dir=None, cold=False,
                      kernel="gemm_nt_bf16_kernel", steps=50, out_dir=None):
    """Turn the rocprofv3 runs of profile_passes() into profiles/gemm_<workload>_<MxKxN>.md and
    profiles/gemm_<workload>_traffic.json (HBM bytes per launch, read by the bench line's roofline).

    FETCH_SIZE / WRITE_SIZE are scaled by what they read for copy_words16 over 512 MiB (512 MiB read and
    512 MiB written per launch), launched by --profile-run before the workload."""
    import csv
    import glob
    import statistics

    def find(d, suffix):
        f = sorted(glob.glob(os.path.join(d, "**", "*" + suffix), recursive=True))
        if not f:
            raise FileNotFoundError(f"no *{suffix} under {d}")
        return f[0]

    def counters(d):
        by = {}
        for r in csv.DictReader(open(find(d, "counter_collection.csv"))):
            by.setdefault(r["Kernel_Name"], []).append(float(r["Counter_Value"]))
        return by

    def named_counters(d, kname):
        """{kernel: {counter: [(value, duration ns)]}} of the dispatches of the kernels matching kname."""
        by = {}
        for r in csv.DictReader(open(find(d, "counter_collection.csv"))):
            if kname in r["Kernel_Name"]:
                dur = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
                by.setdefault(r["Kernel_Name"], {}).setdefault(r["Counter_Name"], []).append(
                    (float(r["Counter_Value"]), dur))
        return by

    def per_call(by, c):
        """A counter per call: the sum over the call's GEMM launches of each launch's median."""
        return sum(statistics.median(v for v, _ in per[c]) for per in by.values())

    desc, M, K, N, has_bias, epi, xdt, ydt = WORKLOADS[workload]
    flops = 2.0 * M * N * K
    alg = algorithmic_bytes(M, K, N, has_bias, xdt, ydt, epi)
    stats = list(csv.DictReader(open(find(trace_dir, "kernel_stats.csv"))))
    fe, wr = counters(fetch_dir), counters(write_dir)
    copyk = next(k for k in fe if "copy_words16" in k)
    # A call's GEMM launches: one, or two with a split tail (the whole rounds as
    # tiles, then the last round's tiles split two ways along K); per-call
    # figures sum them.
    gks = [k for k in fe if kernel in k]
    gk = " + ".join(gks)
    copy_bytes = 512 << 20
    f_scale = copy_bytes / (statistics.median(fe[copyk]) * 1024)
    w_scale = copy_bytes / (statistics.median(wr[copyk]) * 1024)
    fe_call = sum(statistics.median(fe[k]) for k in gks)
    wr_call = sum(statistics.median(wr[k]) for k in wr if kernel in k)
    g_fetch = fe_call * 1024 * f_scale
    g_write = wr_call * 1024 * w_scale
    srow = next(r for r in stats if kernel in r["Name"])
    # Steady state: the timed launches of run_workload, i.e. the `steps` GEMM
    # dispatches before its final 30 isolated ones (the warm-up before them
    # includes the clock ramp, which the stats table averages in).
    trace = [r for r in csv.DictReader(open(find(trace_dir, "kernel_trace.csv"))) if kernel in r["Kernel_Name"]]
    trace.sort(key=lambda r: int(r["Start_Timestamp"]))
    by_name = {}
    for r in trace:
        by_name.setdefault(r["Kernel_Name"], []).append(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
    avg_ns, timed = 0.0, []
    for durs in by_name.values():
        timed = durs[-(steps + 30):-30] if len(durs) > steps + 30 else durs
        avg_ns += float(sum(timed)) / len(timed)
    passes = {name: shown(argv) for name, argv, _ in profile_passes(workload, os.path.dirname(trace_dir), cold)}
    cmds = {k: passes[k] for k in ("trace", "fetch", "write", "busy", "l2")}
    tfl = flops / avg_ns / 1e3
    lines = [f"# {workload}: {desc}, Y[{M}x{N}] = X[{M}x{K}] . W[{N}x{K}]^T (rocprofv3)", "",
             "Kernel trace and stats:", "", "```", cmds["trace"], "```", "",
             "| Kernel | Calls | Average (us) | Min (us) | Max (us) |", "|---|---|---|---|---|"]
    for r in stats:
        lines.append(f"| `{r['Name'][:110]}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.1f} | "
                     f"{float(r['MinNs']) / 1e3:.1f} | {float(r['MaxNs']) / 1e3:.1f} |")
    lines += ["", f"GEMM average over the {len(timed)} timed calls (after the warm-up; {len(by_name)} launch"
                  f"{'es' if len(by_name) > 1 else ''} each): {avg_ns / 1e3:.1f} us -> "
                  f"{tfl:.1f} TFLOP/s ({tfl / PEAK_BF16_TFLOPS * 100:.1f}% of the {PEAK_BF16_TFLOPS} TFLOP/s bf16 "
                  f"dense MFMA peak).  The table's averages include the warm-up launches.", "",
              "Counter passes (one counter per run):", "", "```", cmds["fetch"], cmds["write"], "```", "",
              "| Kernel | FETCH_SIZE (KiB, median) | WRITE_SIZE (KiB, median) |", "|---|---|---|",
              f"| copy_words16, 512 MiB read + 512 MiB written | {statistics.median(fe[copyk]):.0f} | "
              f"{statistics.median(wr[copyk]):.0f} |",
              f"| GEMM{' (per call: its launches summed)' if len(gks) > 1 else ''} | {fe_call:.0f} | {wr_call:.0f} |",
              "",
              f"Calibration against the copy kernel: FETCH_SIZE x {f_scale:.3f}, WRITE_SIZE x {w_scale:.3f} "
              f"(bytes per KiB the counter reports).", "",
              f"GEMM per launch: {g_fetch / 1e6:.1f} MB fetched from beyond L2 + {g_write / 1e6:.1f} MB written = "
              f"{(g_fetch + g_write) / 1e6:.1f} MB; algorithmic minimum {alg / 1e6:.1f} MB "
              f"({(g_fetch + g_write) / alg:.2f}x); {(g_fetch + g_write) / avg_ns:.0f} GB/s over the timed "
              f"launches ({(g_fetch + g_write) / avg_ns / PEAK_HBM_GBS * 100:.1f}% of {PEAK_HBM_GBS:.0f} GB/s), "
              f"algorithmic {alg / avg_ns:.0f} GB/s.", ""]
    t_mfma = flops / (PEAK_BF16_TFLOPS * 1e12) * 1e9
    t_hbm = alg / (PEAK_HBM_GBS * 1e9) * 1e9
    bound = "MFMA" if t_mfma >= t_hbm else "HBM"
    lines += [f"Roofline: the MFMA bound is {t_mfma / 1e3:.2f} us (2*M*N*K at {PEAK_BF16_TFLOPS} TFLOP/s), the HBM "
              f"bound {t_hbm / 1e3:.2f} us (the algorithmic bytes at {PEAK_HBM_GBS:.0f} GB/s); the launch at "
              f"{avg_ns / 1e3:.2f} us is {max(t_mfma, t_hbm) / avg_ns * 100:.1f}% of the binding ({bound}) bound.", ""]
    extra = {"roofline_bound": bound.lower(), "roofline_frac": max(t_mfma, t_hbm) / avg_ns}
    if busy_dir:
        bc = named_counters(busy_dir, kernel)
        med = lambda c: per_call(bc, c)
        dur = sum(statistics.median(d for _, d in per["GRBM_GUI_ACTIVE"]) for per in bc.values())
        cus = 256
        mfma_cyc = med("SQ_VALU_MFMA_BUSY_CYCLES") / (cus * 4)  # per SIMD
        mops = med("SQ_INSTS_VALU_MFMA_MOPS_BF16") * 512.0
        waves = med("SQ_WAVE_CYCLES")
        extra.update({"mfma_busy_cycles_per_simd": mfma_cyc, "mfma_flops_counted": mops, "flops_expected": flops,
                      "lds_wait_frac_of_wave_cycles": med("SQ_WAIT_INST_LDS") / waves,
                      "lds_bank_conflicts": med("SQ_LDS_BANK_CONFLICT"), "counter_pass_duration_ns": dur})
        lines += ["Activity counters (one pass, their own run):", "", "```", cmds["busy"], "```", "",
                  "| Counter | Median per dispatch (per call) |", "|---|---|"]
        lines += [f"| {c} | {med(c):.4g} |" for c in sorted(next(iter(bc.values())))]
        lines += ["", f"- Work check: SQ_INSTS_VALU_MFMA_MOPS_BF16 x 512 = {mops:.4g} FLOP against 2*M*N*K = "
                      f"{flops:.4g} ({mops / flops:.3f}x; tiles past the matrix edges multiply zero padding).",
                  f"- MFMA pipe: SQ_VALU_MFMA_BUSY_CYCLES / ({cus} CUs x 4 SIMDs) = {mfma_cyc:.4g} busy cycles per "
                  f"SIMD (the MFMA count times its issue cycles); over the {avg_ns / 1e3:.1f} us launch that is "
                  f"{mfma_cyc / (avg_ns * 2.4) * 100:.1f}% of the cycles at the 2.4 GHz peak clock "
                  f"(= the fraction of dense peak) and {mfma_cyc / (avg_ns * 1.7) * 100:.1f}% at 1.7 GHz, the "
                  f"clock the chip holds under random-operand MFMA load.",
                  f"- LDS: SQ_WAIT_INST_LDS is {extra['lds_wait_frac_of_wave_cycles'] * 100:.1f}% of "
                  f"SQ_WAVE_CYCLES; {extra['lds_bank_conflicts']:.0f} bank-conflict cycles.",
                  f"- GRBM_GUI_ACTIVE spans the counting window, which extends past the dispatch, so no clock is "
                  f"derived from it.", ""]
    if l2_dir:
        lc = named_counters(l2_dir, kernel)
        hit = per_call(lc, "TCC_HIT_sum")
        miss = per_call(lc, "TCC_MISS_sum")
        extra["l2_hit_frac"] = hit / max(1.0, hit + miss)
        lines += ["L2 (one pass, its own run):", "", "```", cmds["l2"], "```", "",
                  f"TCC_HIT_sum {hit:.4g}, TCC_MISS_sum {miss:.4g} per dispatch: L2 hit rate "
                  f"{extra['l2_hit_frac'] * 100:.1f}%.", ""]
    os.makedirs(os.path.join(ROOT, "profiles"), exist_ok=True)
    tag = workload + ("_cold" if cold else "")
    md = os.path.join(ROOT, "profiles", f"gemm_{tag}_{M}x{K}x{N}.md")
    open(md, "w").write("\n".join(lines) + "\n")
    tj = os.path.join(ROOT, "profiles", f"gemm_{tag}_traffic.json")
    json.dump({"workload": tag, "kernel": gk[:160], "fetch_bytes_per_launch": round(g_fetch),
               "write_bytes_per_launch": round(g_write), "hbm_bytes_per_launch": round(g_fetch + g_write),
               "algorithmic_bytes": alg, "fetch_scale": f_scale, "write_scale": w_scale, "avg_kernel_ns": avg_ns,
               **extra,
               "note": "bytes between L2 and the fabric (HBM or Infinity Cache); counters scaled by a copy "
                       "kernel of known size"}, open(tj, "w"), indent=1)
    if out_dir:
        import shutil
        shutil.copy(md, out_dir)
        shutil.copy(tj, out_dir)
    print(open(md).read())
    return 0


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10, help="minimum warm-up steps")
    ap.add_argument("--warmup-seconds", type=float, default=1.5,
                    help="minimum seconds of back-to-back warm-up steps before timing")
    ap.add_argument("--workload", default="c2", choices=sorted(WORKLOADS) + sorted(ATTN_WORKLOADS) + sorted(CONV_WORKLOADS),
                    help="GEMM shape for the bench line; attention shapes only with --profile-run")
    ap.add_argument("--all", action="store_true", help="also time every workload shape (stderr)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-vendor-gemm", action="store_true", help="skip the torch/hipBLASLt comparator")
    ap.add_argument("--vendor-gemm-child", metavar="DIR", help=argparse.SUPPRESS)
    ap.add_argument("--no-mfma-ceiling", action="store_true",
                    help="skip the register-only MFMA ceiling measured on the same GPU (~5 s)")
    ap.add_argument("--profile-run", action="store_true",
                    help="for rocprofv3 passes: a 512 MiB copy-kernel calibration (5 launches), then --steps "
                         "launches of the workload; no CPU baseline")
    ap.add_argument("--cold", action="store_true",
                    help="with --profile-run: rotate over weight copies larger than twice the Infinity Cache")
    ap.add_argument("--summarize-profile", nargs="+", metavar="DIR",
                    help="TRACE_DIR FETCH_DIR WRITE_DIR [BUSY_DIR [L2_DIR]]: write profiles/ summaries for "
                         "--workload from the rocprofv3 runs of profile_passes() (no GPU needed)")
    ap.add_argument("--profile-all", metavar="OUT_DIR",
                    help="run every rocprofv3 pass for --workload (child processes; raw output under OUT_DIR) and "
                         "write its profiles/ summary")
    args = ap.parse_args()
    if args.vendor_gemm_child:
        return vendor_gemm_child(args.vendor_gemm_child, args.workload)
    if args.profile_all:
        return profile_all(args.workload, os.path.abspath(args.profile_all), cold=args.cold)
    if args.summarize_profile:
        dirs = list(args.summarize_profile) + [None] * (5 - len(args.summarize_profile))
        return summarize_profile(args.workload, *dirs[:5], cold=args.cold)
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (run with --gpus 1)", file=sys.stderr)
        return 2

    from invision_amd import quicknn_hip as q
    info = q.device_info()
    log(f"[bench] device: {info}")
    if args.profile_run:
        return profile_run(args)
    if args.workload in ATTN_WORKLOADS or args.workload in CONV_WORKLOADS:
        print("the bench line is a GEMM shape; attention and convolution shapes run with --all or --profile-run",
              file=sys.stderr)
        return 2

    res = run_workload(args.workload, args.steps, args.warmup, host_path=True, warmup_seconds=args.warmup_seconds)
    log(f"[bench] {json.dumps(res)}")
    failed = [] if res.get("parity_ok", True) else [args.workload]
    if args.all:
        extra = []
        for name in WORKLOADS:
            if name != args.workload:
                extra.append(run_workload(name, max(5, args.steps // 2), 3,
                                          warmup_seconds=min(args.warmup_seconds, 0.5)))
                log(f"[bench] {json.dumps(extra[-1])}")
                if name == "c5_adaln":
                    extra.append(run_workload(name, max(5, args.steps // 2), 3, warmup_seconds=0.5, cold=True))
                    log(f"[bench] {json.dumps(extra[-1])}")
        for name in ATTN_WORKLOADS:
            extra.append(run_attention(name, max(5, args.steps // 4), warmup_seconds=min(args.warmup_seconds, 0.5),
                                       host_path=True))
            log(f"[bench] {json.dumps(extra[-1])}")
        r = run_block(max(5, args.steps // 20), warmup_seconds=min(args.warmup_seconds, 0.5))
        log(f"[bench] {json.dumps(r)}")
        for name in CONV_WORKLOADS:
            extra.append(run_conv(name, max(5, args.steps // 20), warmup_seconds=min(args.warmup_seconds, 0.5),
                                  host_path=True))
            log(f"[bench] {json.dumps(extra[-1])}")
        failed += [r["name"] for r in extra if not r.get("parity_ok", True)]

    ceiling = None if args.no_mfma_ceiling else mfma_ceiling(res["tflops_kernel"])
    if ceiling is not None and WORKLOADS[args.workload][5] == "none" and WORKLOADS[args.workload][6] == "bf16":
        const = gemm_constant_operands(args.workload)
        ceiling["gemm_constant_operands_tflops"] = const["tflops"]
        ceiling["gemm_constant_operands_exact"] = const["exact"]
        log(f"[bench] GEMM with constant operands: {const}")
    vendor = None
    if not args.no_vendor_gemm and WORKLOADS[args.workload][5] == "none" and WORKLOADS[args.workload][6] == "bf16":
        try:
            vendor = vendor_gemm(args.workload)
            log(f"[bench] vendor GEMM: {vendor}")
        except Exception as e:  # a comparator only: its failure does not void the line
            log(f"[bench] vendor GEMM comparator failed: {e!r}")
    desc, M, K, N, has_bias, epi, xdt, ydt = WORKLOADS[args.workload]
    achieved = res["tflops_kernel"]
    traffic = None
    tf = os.path.join(ROOT, "profiles", f"gemm_{args.workload}_traffic.json")
    if os.path.exists(tf):
        try:
            traffic = json.load(open(tf)).get("hbm_bytes_per_launch")
        except Exception:
            traffic = None
    headline_ok = res.get("parity_ok", True)
    if not headline_ok:
        log(f"[bench] PARITY FAILURE on {args.workload}: sampled-row error {res.get('parity_normwise_sampled_rows')} "
            f"> {res.get('parity_tol')}; no headline value is reported")
    line = {
        "metric": METRIC,
        "value": round(res["tflops_wall"], 2) if headline_ok else None,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": res["warmup_steps"],
        "ms_per_step": round(res["wall_ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": f"{desc}: Y[{M}x{N}] = X[{M}x{K}] . W[{N}x{K}]^T + bias, bf16 X/W, fp32 "
                               f"accumulate, fp32 bias and Y, device-resident",
                   "M": M, "K": K, "N": N, "x_dtype": xdt, "y_dtype": ydt, "bias": has_bias, "epilogue": epi,
                   "parallelism": "1 GPU"},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_BF16_TFLOPS, 4), "traffic": traffic},
        "parity_normwise_sampled_rows": res.get("parity_normwise_sampled_rows"),
        "parity_tol": res.get("parity_tol"),
        "launch_ms_p10_p50_p90": res["launch_ms_p10_p50_p90"],
        "host_fp32_io_tflops": round(res["host_fp32_io_tflops"], 2) if "host_fp32_io_tflops" in res else None,
        "host_fp32_io_ms": round(res["host_fp32_io_ms"], 3) if "host_fp32_io_ms" in res else None,
        "host_fp32_io_serial_ms": round(res["host_fp32_io_serial_ms"], 3) if "host_fp32_io_serial_ms" in res else None,
        "device": info["name"],
        "mfma_ceiling": ceiling,
        "vendor_gemm": vendor,
    }
    if not args.no_cpu_baseline:
        log("[bench] cpu baseline ...")
        cb = cpu_baseline(args.workload)
        # the GPU's kernel rate over each CPU leg's all-threads rate on the same GEMM
        if headline_ok and cb:
            cb["gpu_speedup"] = {"vs_port": round(achieved / cb["value"], 1),
                                 "vs_openblas": round(achieved / cb["openblas_cblas_sgemm"]["all_threads"]["tflops"], 1)}
            if "reference_sgemm2" in cb:
                cb["gpu_speedup"]["vs_reference_sgemm2"] = round(
                    achieved / cb["reference_sgemm2"]["all_threads"]["tflops"], 1)
        line["cpu_baseline"] = cb
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line), flush=True)
    q.shutdown()
    if failed:
        log(f"[bench] parity failures: {failed}")
        return 1
    return 0


if __name__ == "__main__":
    sys.exit(main())
