"""Benchmark of the quantised FFN path on one MI355X.

Headline (BASELINE.json metric, config 1): decode Q6_K GEMV HBM GB/s.  One step
= the ffn_down GEMV (Q6_K 3840 x 15360, rotating over 16 distinct weight copies
so the 256 MB Infinity Cache cannot serve it) followed by the lm-head GEMV
(Q6_K 262144 x 3840), both batch 1, CDNA4 layout, inputs resident in HBM.
value = algorithmic bytes (weights + x + y) per step / time per step.

Also reported under "extra": config 0 (Q4_K GEMV), config 2 (decode FFN block
over 48 distinct layers) and config 3 (prefill FFN block at batch 1024,
tokens/s, both accumulation modes).

usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--quick]
"""
import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [os.path.join(ROOT, "neutron-star_amd")]

import numpy as np  # noqa: E402

METRIC = "Q4_K/Q6_K GEMV HBM GB/s (decode); FFN prefill tokens/s @ batch 1024"
HBM_PEAK_GBS = 8000.0
FP16_MFMA_PEAK_TFLOPS = 2500.0
D, F, V = 3840, 15360, 262144

# algorithmic bytes (weights + fp32 x + fp32 y), SURVEY 8(d) per-unit figures
BYTES_Q4_GATE = 15360 * 15 * 144 + 3840 * 4 + 15360 * 4          # 33,254,400
BYTES_Q6_DOWN = 3840 * 60 * 210 + 15360 * 4 + 3840 * 4            # 48,460,800
BYTES_Q6_LMHEAD = 262144 * 15 * 210 + 3840 * 4 + 262144 * 4       # 826,817,536
BYTES_FFN_LAYER = 2 * 15360 * 15 * 144 + 3840 * 60 * 210         # 114,739,200 (weights)
FLOPS_PREFILL_LAYER = 2 * 1024 * 15360 * 3840 * 2 + 2 * 1024 * 3840 * 15360  # 362,387,865,600


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--quick", action="store_true", help="headline only (no extra configs)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for {args.gpus}); the multi-GPU design is "
              "described in DESIGN.md and is not run.", file=sys.stderr)
        sys.exit(2)

    import torch
    import nsffn as N

    assert torch.cuda.is_available(), "no GPU visible"
    torch.cuda.set_device(0)
    ctx = N.Context(0)
    stream = torch.cuda.current_stream()
    nthreads = N.default_threads()

    def upload(host, qtype, cols, rows):
        return torch.from_numpy(N.retile(host, qtype, cols, rows, N.ROW_MAJOR, N.CDNA4)).cuda()

    # ---- config 1 inputs -------------------------------------------------------
    t_gen = time.perf_counter()
    lm_host = N.synth_weights(N.Q6_K, 0x1B, V, D)
    lm = upload(lm_host, N.Q6_K, D, V)
    down_host0 = N.synth_weights(N.Q6_K, 0xD0, D, F)
    downs = [upload(down_host0, N.Q6_K, F, D)]
    for i in range(1, 16):
        downs.append(upload(N.synth_weights(N.Q6_K, 0xD0 + i, D, F), N.Q6_K, F, D))
    x_lm_h = N.synth_normal_f32(0x71, D)
    x_dn_h = N.synth_normal_f32(0x72, F)
    x_lm, x_dn = torch.from_numpy(x_lm_h).cuda(), torch.from_numpy(x_dn_h).cuda()
    y_lm = torch.empty(V, dtype=torch.float32, device="cuda")
    y_dn = torch.empty(D, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    log(f"inputs ready in {time.perf_counter() - t_gen:.1f}s")

    def step(i, ev=None):
        ctx.matmul(downs[i % 16], N.Q6_K, N.CDNA4, F, D, 1, x_dn, y_dn)
        if ev is not None:
            ev[0].record(stream)
        ctx.matmul(lm, N.Q6_K, N.CDNA4, D, V, 1, x_lm, y_lm)
        if ev is not None:
            ev[1].record(stream)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(i, evs[i])
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    wall = t1 - t0
    ms_per_step = 1e3 * wall / args.steps
    bytes_step = BYTES_Q6_DOWN + BYTES_Q6_LMHEAD
    value = bytes_step / (wall / args.steps) / 1e9
    lm_ms = float(np.mean([a.elapsed_time(b) for a, b in evs]))
    lm_gbs = BYTES_Q6_LMHEAD / (lm_ms * 1e-3) / 1e9
    log(f"config1: {ms_per_step:.4f} ms/step, {value:.1f} GB/s; lm-head {lm_ms * 1e3:.1f} us = {lm_gbs:.1f} GB/s")

    extra = {"lm_head_us": round(lm_ms * 1e3, 2), "lm_head_GBps": round(lm_gbs, 1)}

    def timed(fn, n, warm=3):
        for i in range(warm):
            fn(i)
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for i in range(n):
            fn(i)
        b.record(stream)
        torch.cuda.synchronize()
        return a.elapsed_time(b) / n  # ms

    # down GEMV alone (rotating copies)
    dn_ms = timed(lambda i: ctx.matmul(downs[i % 16], N.Q6_K, N.CDNA4, F, D, 1, x_dn, y_dn), 64)
    extra["cfg1a_down_us"] = round(dn_ms * 1e3, 2)
    extra["cfg1a_down_GBps"] = round(BYTES_Q6_DOWN / (dn_ms * 1e-3) / 1e9, 1)

    if not args.quick:
        # ---- config 0: Q4_K GEMV 15360 x 3840, 16 rotating copies -------------
        gates = [upload(N.synth_weights(N.Q4_K, 0x60 + i, F, D), N.Q4_K, D, F) for i in range(16)]
        y_g = torch.empty(F, dtype=torch.float32, device="cuda")
        g_ms = timed(lambda i: ctx.matmul(gates[i % 16], N.Q4_K, N.CDNA4, D, F, 1, x_lm, y_g), 64)
        extra["cfg0_q4k_gemv_us"] = round(g_ms * 1e3, 2)
        extra["cfg0_q4k_gemv_GBps"] = round(BYTES_Q4_GATE / (g_ms * 1e-3) / 1e9, 1)
        # ---- config 2: decode FFN block, 16 distinct layers in rotation -------
        ups = [upload(N.synth_weights(N.Q4_K, 0x80 + i, F, D), N.Q4_K, D, F) for i in range(16)]
        h_d = torch.empty(F, dtype=torch.float32, device="cuda")

        def block(i):
            ctx.gate_up_geglu_decode(gates[i % 16], ups[i % 16], N.CDNA4, D, F, x_lm, h_d)
            ctx.matmul(downs[i % 16], N.Q6_K, N.CDNA4, F, D, 1, h_d, y_dn)

        b_ms = timed(block, 48)
        extra["cfg2_ffn_block_decode_us"] = round(b_ms * 1e3, 2)
        extra["cfg2_ffn_block_decode_GBps"] = round(BYTES_FFN_LAYER / (b_ms * 1e-3) / 1e9, 1)
        del ups
        # ---- config 3: prefill FFN block at batch 1024 --------------------------
        B = 1024
        xp = torch.from_numpy(N.synth_normal_f16(0x90, B * D).view(np.int16)).cuda()
        hp = torch.empty((B, F), dtype=torch.int16, device="cuda")
        yp = torch.empty((B, D), dtype=torch.float32, device="cuda")
        for fast, name in ((False, "fp32acc"), (True, "fp16acc")):
            def pre(i, fast=fast):
                ctx.gate_up_geglu_rm32(gates[i % 16], gates[(i + 1) % 16], N.CDNA4, D, F, B, xp, hp, fast)
                ctx.ffn_down(downs[i % 16], N.Q6_K, N.CDNA4, F, D, B, hp, yp, True, fast)
            p_ms = timed(pre, 8, warm=2)
            gu_ms = timed(lambda i, fast=fast: ctx.gate_up_geglu_rm32(gates[i % 16], gates[(i + 1) % 16], N.CDNA4,
                                                                      D, F, B, xp, hp, fast), 8, warm=1)
            dn2_ms = timed(lambda i, fast=fast: ctx.ffn_down(downs[i % 16], N.Q6_K, N.CDNA4, F, D, B, hp, yp, True,
                                                             fast), 8, warm=1)
            extra[f"cfg3_prefill_{name}_tokens_per_s"] = round(B / (p_ms * 1e-3), 1)
            extra[f"cfg3_prefill_{name}_block_ms"] = round(p_ms, 4)
            extra[f"cfg3_prefill_{name}_TFLOPs"] = round(FLOPS_PREFILL_LAYER / (p_ms * 1e-3) / 1e12, 1)
            extra[f"cfg3_{name}_gate_up_ms"] = round(gu_ms, 4)
            extra[f"cfg3_{name}_down_ms"] = round(dn2_ms, 4)
            log(f"config3 {name}: {p_ms:.3f} ms/block = {B / (p_ms * 1e-3):.0f} tok/s "
                f"(gate/up {gu_ms:.3f} ms, down {dn2_ms:.3f} ms)")
        del gates

    # ---- CPU baseline: the oracle on one full config-1 step --------------------
    cpu = None
    if not args.no_cpu:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import ns_oracle as O

        # repeat whole config-1 steps until at least 10 s of CPU time have passed
        reps = 0
        t = time.perf_counter()
        while True:
            ref_dn = O.gemv(N.Q6_K, O.ROW_MAJOR, down_host0, F, D, x_dn_h, nthreads=nthreads)
            ref_lm = O.gemv(N.Q6_K, O.ROW_MAJOR, lm_host, D, V, x_lm_h, nthreads=nthreads)
            reps += 1
            dt = time.perf_counter() - t
            if dt >= 10.0 or reps >= 200:
                break
        cpu = {"value": round(reps * bytes_step / dt / 1e9, 3), "unit": "GB/s", "cores": nthreads, "kind": "port",
               "sample": f"{reps} full config-1 steps (Q6_K down 3840x15360 + lm-head 262144x3840 GEMV) by the "
                         f"oracle's dequant-once sequential-fp32 dot, {dt:.2f} s on {cpu_model()}"}
        # the same inputs on the GPU: a free parity check of the measured kernels
        ctx.matmul(downs[0], N.Q6_K, N.CDNA4, F, D, 1, x_dn, y_dn)
        ctx.matmul(lm, N.Q6_K, N.CDNA4, D, V, 1, x_lm, y_lm)
        torch.cuda.synchronize()

        def rel(a, b):
            return float(np.max(np.abs(a - b)) / np.max(np.abs(b)))
        extra["parity_rel_err_down"] = rel(y_dn.cpu().numpy(), ref_dn)
        extra["parity_rel_err_lm_head"] = rel(y_lm.cpu().numpy(), ref_lm)
        log(f"cpu baseline {cpu['value']} GB/s in {dt:.2f}s; parity {extra['parity_rel_err_down']:.2e} "
            f"{extra['parity_rel_err_lm_head']:.2e}")

    out = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded generator, BASELINE config 1 distributions)",
        "config": {"workload": "config 1: Q6_K ffn_down 3840x15360 (16 rotating copies) + Q6_K lm-head "
                               "262144x3840 GEMV, batch 1, CDNA4 layout",
                   "batch": 1, "bytes_per_step": bytes_step},
        "roofline": {"bound": "hbm", "achieved": round(lm_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(lm_gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "gemv_kernel<Q6_K, CDNA4> (lm-head)"},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(out), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
