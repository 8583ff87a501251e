#!/usr/bin/env python3
"""Benchmark of the HIP quantized-linear hot path on one MI355X.

Metric: Q4_K matvec GB/s (% of HBM peak) at Llama-3-8B shapes; prefill GEMM
TOPS (% of dense int8 MFMA peak).

A step is one batch-1 decode token through every linear layer of a Llama-3-8B-shaped decoder
32 layers x {q 4096x4096, k 1024x4096, v 1024x4096, o 4096x4096,
gate 14336x4096, up 14336x4096, down 4096x14336} in Q4_K, plus the 128256x4096 Q6_K lm_head.
Each layer runs four fused matvec launches (q/k/v, o, gate/up, down) on f32 inputs, which the
kernels quantize as they stage them;
weights are random-init (synthetic, 4.36 GB resident, so the 256 MB Infinity Cache cannot
serve them). The step is captured once as a HIP graph and replayed. `value` is the step's
algorithmic bytes (file-layout weight bytes + f32 activations in + f32 outputs) / step time.

Also reported:
  roofline      the dominant kernel (Q4_K matvec, 14336x4096, batch 1), timed with HIP events
                over back-to-back launches that rotate through the 64 distinct gate/up matrices
  prefill       GEMM at 512 tokens, in TOPS against the 5.0 POPS dense int8 MFMA peak: Q4_K at the
                8B FFN shapes (14336x4096, 4096x14336) and the Qwen3-0.6B FFN shapes (3072x1024,
                1024x3072), IQ4_NL 14336x4096 and Q6_K 4096x14336
  extra         the decode step at batch 8 (config 4); config 5's batch-1 matvecs (IQ4_NL
                14336x4096, Q6_K 4096x14336) rotating over at least 512 MB of matrices each; config 1 (the Q8_0
                3072x1024 matvec, rotating over 160 copies); config 2 (a batch-1 decode step of a
                Qwen3-0.6B-shaped decoder, tokens/s); the whole-network pass on Qwen3-0.6B and
                Llama-3-8B shapes (prefill, one-token decode, and 8 sequences decoded together in one
                pass over their own cache slots, with and without reading their logits); decode
                attention at ~6000 positions (one layer of Llama-3-8B's attention shapes)
  measured_peaks  this GPU's dense int8 MFMA rate and HBM read rate from probe kernels
                (hk_amd/csrc/peak.hip), quoted beside the published peaks the fractions use
  cpu_baseline  hk's CPU decode kernel restated with its SIMD paths (oracle/hk_cpu_simd.c, best
                instruction set of the host chosen at run time) on the host's physical cores, on a
                bounded sample (the 14336x4096 Q4_K matvec, repeated for ~10 s), plus one thread
  wall_s        wall-clock seconds of each phase of this run
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, GB/s
INT8_PEAK_TOPS = 5000.0      # MI355X dense int8 MFMA, TOPS

LLAMA8B = dict(hidden=4096, ffn=14336, kv=1024, layers=32, vocab=128256)


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--layers", type=int, default=LLAMA8B["layers"])
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--only", choices=["all", "decode", "kernel", "prefill", "extra", "copy"], default="all",
                   help="run one part only (profiling); 'copy' runs a plain 256 MiB device copy 20 times, "
                        "the calibration for the HBM traffic counters")
    return p.parse_args()


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path (asked for {args.gpus}).",
              file=sys.stderr)
        sys.exit(2)

    T0 = time.perf_counter()
    phases = {}
    mark = [T0]

    def phase(name):
        now = time.perf_counter()
        phases[name] = round(now - mark[0], 2)
        mark[0] = now

    import torch

    from hk_amd import Engine, formats as F, synth
    FMT_NAME = F.NAMES

    torch.cuda.init()
    dev = torch.device("cuda:0")
    if args.only == "copy":
        src = torch.ones(64 << 20, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(20):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": src.numel() * 4, "launches": 20}))
        return
    eng = Engine(0)
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    eng.set_stream(stream.cuda_stream)
    H, FF, KV, V = LLAMA8B["hidden"], LLAMA8B["ffn"], LLAMA8B["kv"], LLAMA8B["vocab"]
    L = args.layers

    def upload_synth(t, rows, cols, seed):
        raw = synth.weights_torch(t, rows, cols, seed, device=dev)
        m = eng.upload(raw, t, rows, cols)
        del raw
        return m

    # ---- weights: 32 layers of Q4_K + Q6_K lm_head ----
    shapes = [("q", H, H), ("k", KV, H), ("v", KV, H), ("o", H, H), ("gate", FF, H), ("up", FF, H), ("down", H, FF)]
    layers = []
    for li in range(L):
        layers.append({name: upload_synth(F.Q4_K, r, c, synth.seed_for(4, li * 10 + i))
                       for i, (name, r, c) in enumerate(shapes)})
    lm_head = upload_synth(F.Q6_K, V, H, synth.seed_for(4, 999))
    torch.cuda.synchronize()
    phase("import_and_weights")

    # ---- activations (resident): one input per distinct product input ----
    x_h = torch.randn(1, H, device=dev)
    x_f = torch.randn(1, FF, device=dev)
    outs = {name: torch.empty(1, r, device=dev) for name, r, _ in shapes}
    logits = torch.empty(1, V, device=dev)

    def step():
        # Per layer: q/k/v fused, o, gate/up fused, down; each launch quantizes its own input.
        for lw in layers:
            eng.matvec_parts([lw["q"], lw["k"], lw["v"]], [outs["q"], outs["k"], outs["v"]], 1, x=x_h)
            eng.matvec_parts([lw["o"]], [outs["o"]], 1, x=x_h)
            eng.matvec_parts([lw["gate"], lw["up"]], [outs["gate"], outs["up"]], 1, x=x_h)
            eng.matvec_parts([lw["down"]], [outs["down"]], 1, x=x_f)
        eng.matvec_parts([lm_head], [logits], 1, x=x_h)

    weight_bytes = sum(m.file_bytes for lw in layers for m in lw.values()) + lm_head.file_bytes
    act_bytes = 0
    for _ in range(L):
        act_bytes += 3 * 4 * H + 4 * FF                               # f32 inputs, once per launch
        act_bytes += 4 * sum(r for _, r, _ in shapes)                 # f32 outputs
    act_bytes += 4 * H + 4 * V
    step_bytes = weight_bytes + act_bytes

    result = {}
    if args.only in ("all", "decode"):
        for _ in range(max(1, args.warmup)):
            step()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        cap = torch.cuda.Stream()
        cap.wait_stream(stream)
        with torch.cuda.graph(g, stream=cap):
            eng.set_stream(cap.cuda_stream)
            step()
        eng.set_stream(stream.cuda_stream)
        torch.cuda.synchronize()
        for _ in range(args.warmup):
            g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record(stream)
        for _ in range(args.steps):
            g.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        ms = e0.elapsed_time(e1) / args.steps
        phase("decode_step")
        result["decode"] = dict(ms_per_step=ms, wall_ms_per_step=1e3 * wall / args.steps,
                                gbs=step_bytes / (ms * 1e-3) / 1e9, tokens_per_s=1e3 / ms,
                                weight_bytes=weight_bytes, step_bytes=step_bytes)

    # ---- dominant kernel: the fused gate/up Q4_K matvec (2 x 14336x4096, batch 1), rotating
    # over the 32 layers' distinct matrices (2.1 GB, so HBM, not the Infinity Cache, serves them).
    # The launches are captured in a HIP graph so host launch cost cannot starve the GPU.
    if args.only in ("all", "kernel"):
        pairs = [(lw["gate"], lw["up"]) for lw in layers]
        ys = [outs["gate"], outs["up"]]

        def gate_up():
            for g_, u_ in pairs:
                eng.matvec_parts([g_, u_], ys, 1, x=x_h)

        gate_up()
        torch.cuda.synchronize()
        gk = torch.cuda.CUDAGraph()
        cap = torch.cuda.Stream()
        cap.wait_stream(stream)
        with torch.cuda.graph(gk, stream=cap):
            eng.set_stream(cap.cuda_stream)
            gate_up()
        eng.set_stream(stream.cuda_stream)
        gk.replay()
        torch.cuda.synchronize()
        reps = max(4, args.steps)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            gk.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        us = 1e3 * e0.elapsed_time(e1) / (reps * len(pairs))
        kbytes = 2 * pairs[0][0].file_bytes + 4 * H + 2 * 4 * FF
        phase("roofline_kernel")
        result["kernel"] = dict(name="mmvr_kernel<Q4_K, NT=1, C=1> (gate+up fused, f32 input quantized in-kernel)",
                                shape="2x14336x4096",
                                launches=reps * len(pairs), avg_us=us, bytes_per_launch=kbytes,
                                gbs=kbytes / (us * 1e-6) / 1e9)

    # ---- prefill GEMM, 512 tokens ----
    if args.only in ("all", "prefill"):
        pre = []
        # The headline shape first, then BASELINE configs 3 (Qwen3-0.6B FFN) and 5 (8B FFN in the
        # mixed formats), and the 8B down projection.
        for (name, t, m_, k_) in [("llama8b-ffn-up", F.Q4_K, FF, H), ("qwen3-0.6b-ffn-up", F.Q4_K, 3072, 1024),
                                  ("qwen3-0.6b-ffn-down", F.Q4_K, 1024, 3072),
                                  ("llama8b-ffn-down", F.Q4_K, H, FF),
                                  ("llama8b-ffn-up", F.IQ4_NL, FF, H), ("llama8b-ffn-down", F.Q6_K, H, FF)] + \
                                 [("llama8b-ffn-up", t, FF, H) for t in (F.Q4_0, F.Q4_1, F.Q5_0, F.Q5_1, F.Q5_K, F.IQ4_XS)] + \
                                 [("llama8b-ffn-down", F.Q5_K, H, FF)]:
            n = 512
            reuse = layers[0]["gate"] if (t, m_, k_) == (F.Q4_K, FF, H) else None
            w = reuse or upload_synth(t, m_, k_, synth.seed_for(3, m_ + k_ + t))
            x = torch.randn(n, k_, device=dev)
            xq = torch.empty(eng.act_bytes(n, k_), dtype=torch.uint8, device=dev)
            yy = torch.empty(n, m_, device=dev)
            eng.qact(x, n, k_, F.ACT_KIND[t], xq)
            us = time_graph(torch, eng, stream, lambda: eng.gemm(w, xq, yy, n), 5)
            tops = 2.0 * m_ * n * k_ / (us * 1e-6) / 1e12
            pre.append(dict(shape=f"{m_}x{k_}x{n}", fmt=FMT_NAME[t], workload=name, avg_us=round(us, 2),
                            tops=round(tops, 2), frac_int8_peak=round(tops / INT8_PEAK_TOPS, 4)))
            if (t, m_, k_) == (F.Q4_K, FF, H):
                # The same GEMM with its activation quantization (qact of the f32 input) in the
                # timed region: prefill of one layer input as the engine runs it.
                us_q = time_graph(torch, eng, stream,
                                  lambda: (eng.qact(x, n, k_, F.ACT_Q8K, xq), eng.gemm(w, xq, yy, n)), 5)
                tq = 2.0 * m_ * n * k_ / (us_q * 1e-6) / 1e12
                pre.append(dict(shape=f"{m_}x{k_}x{n}", fmt=FMT_NAME[t], workload=name + " (qact + gemm)",
                                avg_us=round(us_q, 2), tops=round(tq, 2), frac_int8_peak=round(tq / INT8_PEAK_TOPS, 4)))
            if reuse is None:
                eng.free(w)
        result["prefill"] = pre
        phase("prefill")

    # ---- BASELINE config 4 at batch 8 (the decode step for 8 tokens) and config 5's batch-1
    # matvecs (IQ4_NL gate/up, Q6_K down, the other formats' gate/up), each rotating over at least
    # 512 MB of distinct matrices so that the 256 MB Infinity Cache cannot serve them.
    if args.only in ("all", "extra"):
        extra = {}
        x_h8 = torch.randn(8, H, device=dev)
        x_f8 = torch.randn(8, FF, device=dev)
        outs8 = {name: torch.empty(8, r, device=dev) for name, r, _ in shapes}
        logits8 = torch.empty(8, V, device=dev)

        xq_h8 = torch.empty(eng.act_bytes(8, H), dtype=torch.uint8, device=dev)
        xq_f8 = torch.empty(eng.act_bytes(8, FF), dtype=torch.uint8, device=dev)

        def step8():
            # Each product quantizes its own input (a decoder's four projections read four
            # different vectors), then runs on the prepared activations: the Q4_K layers on the
            # small-batch MFMA kernel, the Q6_K lm_head on the decode kernel.
            for lw in layers:
                eng.qact(x_h8, 8, H, F.ACT_Q8K, xq_h8)
                eng.matvec_parts([lw["q"], lw["k"], lw["v"]], [outs8["q"], outs8["k"], outs8["v"]], 8, xq=xq_h8)
                eng.qact(x_h8, 8, H, F.ACT_Q8K, xq_h8)
                eng.matvec_parts([lw["o"]], [outs8["o"]], 8, xq=xq_h8)
                eng.qact(x_h8, 8, H, F.ACT_Q8K, xq_h8)
                eng.matvec_parts([lw["gate"], lw["up"]], [outs8["gate"], outs8["up"]], 8, xq=xq_h8)
                eng.qact(x_f8, 8, FF, F.ACT_Q8K, xq_f8)
                eng.matvec_parts([lw["down"]], [outs8["down"]], 8, xq=xq_f8)
            eng.qact(x_h8, 8, H, F.ACT_Q8K, xq_h8)
            eng.matvec_parts([lm_head], [logits8], 8, xq=xq_h8)

        def step8_f32():
            for lw in layers:
                eng.matvec_parts([lw["q"], lw["k"], lw["v"]], [outs8["q"], outs8["k"], outs8["v"]], 8, x=x_h8)
                eng.matvec_parts([lw["o"]], [outs8["o"]], 8, x=x_h8)
                eng.matvec_parts([lw["gate"], lw["up"]], [outs8["gate"], outs8["up"]], 8, x=x_h8)
                eng.matvec_parts([lw["down"]], [outs8["down"]], 8, x=x_f8)
            eng.matvec_parts([lm_head], [logits8], 8, x=x_h8)

        us8 = time_graph(torch, eng, stream, step8, max(3, args.steps // 5), per_graph=1)
        us8f = time_graph(torch, eng, stream, step8_f32, max(3, args.steps // 5), per_graph=1)
        extra["decode_batch8_f32_inputs_ms"] = round(us8f / 1e3, 4)
        b8_bytes = weight_bytes + 8 * act_bytes
        extra["decode_batch8"] = dict(ms_per_step=round(us8 / 1e3, 4), tokens_per_s=round(8e6 / us8, 1),
                                      gbs=round(b8_bytes / (us8 * 1e-6) / 1e9, 1),
                                      frac_hbm_peak=round(b8_bytes / (us8 * 1e-6) / 1e9 / HBM_PEAK_GBS, 4))
        mv = []
        for (name, t, m_, k_) in [("llama8b-ffn-up", F.IQ4_NL, FF, H), ("llama8b-ffn-down", F.Q6_K, H, FF)] + \
                                 [("llama8b-ffn-up", t, FF, H) for t in (F.Q4_0, F.Q4_1, F.Q5_0, F.Q5_1, F.Q5_K, F.IQ4_XS)]:
            # at least 512 MB of distinct weights in the rotation (16+ copies at 4.5 bits per weight)
            ncopy = max(12, -(-(512 << 20) // F.matrix_bytes(t, m_, k_)))
            ws = [upload_synth(t, m_, k_, synth.seed_for(5, 100 * t + i)) for i in range(ncopy)]
            xv = torch.randn(1, k_, device=dev)
            yv = torch.empty(1, m_, device=dev)

            def rot():
                for w_ in ws:
                    eng.matvec_parts([w_], [yv], 1, x=xv)

            us = time_graph(torch, eng, stream, rot, 5, per_graph=1) / len(ws)
            mv.append(dict(shape=f"{m_}x{k_}", fmt=FMT_NAME[t], workload=name, avg_us=round(us, 2),
                           gbs=round(ws[0].file_bytes / (us * 1e-6) / 1e9, 1),
                           frac_hbm_peak=round(ws[0].file_bytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)))
            for w_ in ws:
                eng.free(w_)
        extra["matvec_batch1"] = mv

        # Config 1: the Q8_0 3072x1024 matvec at batch 1 (f32 input quantized in-kernel), rotating
        # over 160 copies (535 MB, past the Infinity Cache).
        ws = [upload_synth(F.Q8_0, 3072, 1024, synth.seed_for(1, i)) for i in range(160)]
        xv = torch.randn(1, 1024, device=dev)
        yv = torch.empty(1, 3072, device=dev)

        def rot1():
            for w_ in ws:
                eng.matvec_parts([w_], [yv], 1, x=xv)

        us = time_graph(torch, eng, stream, rot1, 5, per_graph=1) / len(ws)
        b1 = ws[0].file_bytes + 4 * 1024 + 4 * 3072
        extra["config1_q8_0_matvec"] = dict(shape="3072x1024", avg_us=round(us, 2), gbs=round(b1 / (us * 1e-6) / 1e9, 1),
                                            frac_hbm_peak=round(b1 / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4))
        for w_ in ws:
            eng.free(w_)

        # Upload from host memory: the file bytes of a 14336x4096 matrix from an mmap'd file view
        # (hk loads tensors as views of the mmap'd container), through hkhip_upload (H2D copy, then
        # the on-device repack for the formats whose blocks are not 16-byte aligned).
        import tempfile

        import numpy as np
        up = []
        for t in (F.Q4_K, F.IQ4_NL, F.Q6_K):
            raw = synth.weights_np(t, FF, H, seed=synth.seed_for(6, t))
            with tempfile.NamedTemporaryFile(dir="/tmp", suffix=".bin") as fh:
                raw.tofile(fh.name)
                view = np.memmap(fh.name, dtype=np.uint8, mode="r").reshape(raw.shape)
                eng.free(eng.upload(view, t, FF, H))  # warm-up
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                for _ in range(3):
                    eng.free(eng.upload(view, t, FF, H))
                torch.cuda.synchronize()
                dt = (time.perf_counter() - t0) / 3
                del view
            up.append(dict(fmt=FMT_NAME[t], shape=f"{FF}x{H}", ms=round(dt * 1e3, 2), gbs=round(raw.nbytes / dt / 1e9, 2)))
        extra["upload_from_mmap"] = up

        # Config 2: a batch-1 decode step through every linear layer of a Qwen3-0.6B-shaped decoder
        # (28 x {q 2048x1024, k/v 1024x1024, o 1024x2048, gate/up 3072x1024, down 1024x3072} Q4_K +
        # the 151936x1024 Q6_K lm_head), four fused launches per layer as in the 8B step.
        qshapes = [("q", 2048, 1024), ("k", 1024, 1024), ("v", 1024, 1024), ("o", 1024, 2048),
                   ("gate", 3072, 1024), ("up", 3072, 1024), ("down", 1024, 3072)]
        qlayers = [{nm: upload_synth(F.Q4_K, r, c, synth.seed_for(2, li * 10 + i)) for i, (nm, r, c) in enumerate(qshapes)}
                   for li in range(28)]
        qhead = upload_synth(F.Q6_K, 151936, 1024, synth.seed_for(2, 999))
        qx = {c: torch.randn(1, c, device=dev) for c in (1024, 2048, 3072)}
        qo = {nm: torch.empty(1, r, device=dev) for nm, r, _ in qshapes}
        qlog = torch.empty(1, 151936, device=dev)

        def qstep():
            for lw in qlayers:
                eng.matvec_parts([lw["q"], lw["k"], lw["v"]], [qo["q"], qo["k"], qo["v"]], 1, x=qx[1024])
                eng.matvec_parts([lw["o"]], [qo["o"]], 1, x=qx[2048])
                eng.matvec_parts([lw["gate"], lw["up"]], [qo["gate"], qo["up"]], 1, x=qx[1024])
                eng.matvec_parts([lw["down"]], [qo["down"]], 1, x=qx[3072])
            eng.matvec_parts([qhead], [qlog], 1, x=qx[1024])

        usq = time_graph(torch, eng, stream, qstep, max(5, args.steps // 2), per_graph=1)
        qbytes = sum(m.file_bytes for lw in qlayers for m in lw.values()) + qhead.file_bytes
        qbytes += 28 * 4 * (1024 + 2048 + 1024 + 3072 + sum(r for _, r, _ in qshapes)) + 4 * (1024 + 151936)
        extra["config2_qwen3_0_6b_decode"] = dict(ms_per_step=round(usq / 1e3, 4), tokens_per_s=round(1e6 / usq, 1),
                                                  step_bytes=qbytes, gbs=round(qbytes / (usq * 1e-6) / 1e9, 1),
                                                  frac_hbm_peak=round(qbytes / (usq * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                                                  launches=4 * 28 + 1)
        for lw in qlayers:
            for m in lw.values():
                eng.free(m)
        eng.free(qhead)
        extra["network_qwen3_0_6b"] = network_bench(torch, eng, F, synth)
        extra["network_llama3_8b"] = network_bench(torch, eng, F, synth, "llama3_8b")
        extra["long_context_attention"] = long_context_bench(torch, eng, F, synth)
        result["extra"] = extra
        phase("extra")

    # ---- this GPU's measured peaks, quoted beside the published ones (the fractions use those) ----
    peaks = None
    if args.only == "all":
        peaks = measured_peaks()
        phase("measured_peaks")

    # ---- CPU baseline: the oracle on the host cores, bounded sample ----
    cpu = None
    if not args.no_cpu and args.only == "all":
        cpu = cpu_baseline(args.cpu_seconds)
        phase("cpu_baseline")

    dec = result.get("decode", {})
    ker = result.get("kernel", {})
    line = {
        "metric": "Q4_K matvec GB/s (% HBM peak) at 8B shapes; prefill GEMM TOPS (% MFMA)",
        "value": round(dec.get("gbs", 0.0), 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dec.get("ms_per_step", 0.0), 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (random-init Q4_K / Q6_K blocks, N(0,1) activations)",
        "config": {"workload": "llama3-8b decode step, all linear layers, batch 1 (config 4)",
                   "layers": L, "hidden": H, "ffn": FF, "kv": KV, "vocab": V,
                   "weights": "Q4_K layers + Q6_K lm_head", "step_bytes": dec.get("step_bytes"),
                   "tokens_per_s": round(dec.get("tokens_per_s", 0.0), 1),
                   "frac_hbm_peak": round(dec.get("gbs", 0.0) / HBM_PEAK_GBS, 4),
                   "graph": "one HIP graph per step"},
        "roofline": {"bound": "hbm", "achieved": round(ker.get("gbs", 0.0), 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(ker.get("gbs", 0.0) / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(),
                     "kernel": ker.get("name"), "shape": ker.get("shape"), "avg_us": ker.get("avg_us"),
                     "bytes_per_launch": ker.get("bytes_per_launch")},
        "prefill": result.get("prefill"),
        "extra": result.get("extra"),
        "measured_peaks": peaks,
        "cpu_baseline": cpu,
        "wall_s": dict(phases, total=round(time.perf_counter() - T0, 2)),
    }
    print(json.dumps(line), flush=True)
    eng.close()


def long_context_bench(torch, eng, F, synth):
    """Decode attention at long context: a one-layer network with Llama-3-8B's attention shapes
    (dim 4096, 32 query / 8 key-value heads of 128, pairwise RoPE; FFN 256 and a 256-token
    vocabulary, so the products stay small beside the attention), max_ctx 8192; 8 sequences
    prefilled to 5800-6150 positions and then decoded together (one token each per pass), and one
    sequence at 6000 positions decoded alone; with the kernel each pass chooses (attn_gqa 0) and
    with the per-head kernel forced (2). Host clock per pass (graph replays); also the 6000-token
    prompt's prefill pass (one layer: its GEMMs and the MFMA prefill attention)."""
    import numpy as np

    from hk_amd.net import Config, Net, Options

    cfg = Config(dim=4096, n_layers=1, n_heads=32, n_kv_heads=8, head_dim=128, ffn_dim=256, vocab=256,
                 max_ctx=8192, rope_neox=False, rope_base=500000.0, rms_eps=1e-5)
    model = synth.model_np(cfg, F.Q4_K, seed=synth.seed_for(4, 600), out_fmt=F.Q6_K, embd_fmt=F.Q8_0, qk_norm=False)
    lens = [5800 + 50 * i for i in range(8)]
    out = {"context": "8 sequences at positions 5800-6170 (one token each per pass); one at 6000-6019"}
    for mode, name in ((0, "chosen"), (2, "per_head")):
        rng = np.random.default_rng(11)
        with Net(eng, cfg, Options(slots=9, attn_gqa=mode)) as net:
            net.load(model)
            for i, ln in enumerate(lens):
                net.forward_items([(1 + i, int(t), p) for p, t in enumerate(rng.integers(0, cfg.vocab, ln))])
            step = lambda k: [(1 + i, int(rng.integers(0, cfg.vocab)), ln + k) for i, ln in enumerate(lens)]
            for k in range(4):
                net.forward_items(step(k))
            t0 = time.perf_counter()
            for k in range(4, 20):
                net.forward_items(step(k))
            multi_s = (time.perf_counter() - t0) / 16
            torch.cuda.synchronize()
            prompt = [(99, int(t), p) for p, t in enumerate(rng.integers(0, cfg.vocab, 6000))]
            t0 = time.perf_counter()
            net.forward_items(prompt)
            torch.cuda.synchronize()
            prefill_s = time.perf_counter() - t0
            for k in range(4):
                net.forward_items([(99, 5, 6000 + k)])
            t0 = time.perf_counter()
            for k in range(4, 20):
                net.forward_items([(99, 5, 6000 + k)])
            one_s = (time.perf_counter() - t0) / 16
            ok = bool(np.isfinite(net.logits_rows([0])).all())
        out[name] = {"sessions8_ms_per_pass": round(multi_s * 1e3, 3), "one_token_ms_per_pass": round(one_s * 1e3, 3),
                     "finite_logits": ok}
        if mode == 0:  # the prefill kernels do not depend on the decode attention choice
            out["prefill_6000_ms"] = round(prefill_s * 1e3, 2)
    return out


def network_bench(torch, eng, F, synth, which: str = "qwen3_0_6b"):
    """The whole-network device pass (hk_amd.net) on a random model of a real shape: a 512-token
    prompt prefill, then 64 decode passes of one token (one HIP graph replay each, positions
    512..575), timed on the host clock around each call (the call returns when its pass is done).
      qwen3_0_6b: config 2's shapes (28 layers, dim 1024, 16 query / 8 key-value heads of 128, q/k
        norms, FFN 3072, vocabulary 151936); Q4_K layers, Q6_K output and embedding.
      llama3_8b:  config 4's shapes (32 layers, dim 4096, 32 / 8 heads of 128, FFN 14336,
        vocabulary 128256, llama3 RoPE scaling: factor 8 over 8192 positions, base 500000);
        Q4_K layers and embedding, Q6_K output. Every layer gets the same random matrices (their
        own device copies: no layer reads another's), which keeps the host synthesis short."""
    import numpy as np

    from hk_amd.net import Config, Net, Options
    from hk_amd.rope import RopeScaling

    if which == "llama3_8b":
        cfg = Config(dim=4096, n_layers=32, n_heads=32, n_kv_heads=8, head_dim=128, ffn_dim=14336, vocab=128256,
                     max_ctx=2048, rope_neox=False, rope_base=500000.0, rms_eps=1e-5,
                     rope_scaling=RopeScaling("llama3", 8.0, 8192, 1.0, 4.0))
        one = synth.model_np(Config(dim=4096, n_layers=1, n_heads=32, n_kv_heads=8, head_dim=128, ffn_dim=14336,
                                    vocab=8, max_ctx=16), F.Q4_K, seed=synth.seed_for(4, 500), qk_norm=False)
        rng_w = np.random.default_rng(synth.seed_for(4, 501))
        model = {"layers": one["layers"] * cfg.n_layers, "out_norm": (1.0 + 0.1 * rng_w.standard_normal(4096)).astype(np.float32),
                 "tok_embd": (synth.weights_np(F.Q4_K, cfg.vocab, cfg.dim, synth.seed_for(4, 502)), F.Q4_K),
                 "output": (synth.weights_np(F.Q6_K, cfg.vocab, cfg.dim, synth.seed_for(4, 503)), F.Q6_K)}
        n_layers_desc = "32 layers (dim 4096, GQA 32/8, FFN 14336, llama3-scaled RoPE)"
    else:
        cfg = Config(dim=1024, n_layers=28, n_heads=16, n_kv_heads=8, head_dim=128, ffn_dim=3072, vocab=151936,
                     max_ctx=2048, rope_neox=True, rope_base=1e6)
        model = synth.model_np(cfg, F.Q4_K, seed=synth.seed_for(2, 500), out_fmt=F.Q6_K, embd_fmt=F.Q6_K)
        n_layers_desc = "28 layers (dim 1024, GQA 16/8 with q/k norms, FFN 3072)"
    rng = np.random.default_rng(7)
    with Net(eng, cfg, Options(slots=9)) as net:
        net.load(model)
        del model
        prompt = rng.integers(0, cfg.vocab, 512)
        net.forward(prompt, 0)  # warm-up (first GEMM launches)
        t0 = time.perf_counter()
        net.forward(prompt, 0)
        pre_s = time.perf_counter() - t0
        toks = rng.integers(0, cfg.vocab, 64)
        for i in range(4):  # eager run, capture, replays
            net.forward(toks[i:i + 1], 512 + i)
        t0 = time.perf_counter()
        for i in range(64):
            net.forward(toks[i:i + 1], 512 + i)
        dec_s = (time.perf_counter() - t0) / 64
        ok = bool(np.isfinite(net.logits()).all())
        # hk's server case (kv.zig:22-29): 8 sequences, each prefilled to its own length (256 +
        # 32 i), then decoded together, one token each per pass (forward(items)); the timed passes
        # also read the 8 logit rows back to the host (logits(indices)).
        lens = [256 + 32 * i for i in range(8)]
        for i, ln in enumerate(lens):
            net.forward_items([(1 + i, int(t), p) for p, t in enumerate(rng.integers(0, cfg.vocab, ln))])
        step = lambda k: [(1 + i, int(rng.integers(0, cfg.vocab)), ln + k) for i, ln in enumerate(lens)]
        for k in range(4):
            net.forward_items(step(k))
        t0 = time.perf_counter()
        for k in range(4, 36):
            net.forward_items(step(k))
        multi_s = (time.perf_counter() - t0) / 32
        t0 = time.perf_counter()
        for k in range(36, 68):
            net.forward_items(step(k))
            rows = net.logits_view(list(range(8)))  # the engine's own rows, as hk's Device.logits
        multi_lg_s = (time.perf_counter() - t0) / 32
        ok = ok and bool(np.isfinite(rows).all())
    return {"prefill_512_ms": round(pre_s * 1e3, 2), "prefill_tokens_per_s": round(512 / pre_s, 1),
            "decode_ms_per_token": round(dec_s * 1e3, 3), "decode_tokens_per_s": round(1 / dec_s, 1),
            "context": "positions 512-575", "finite_logits": ok,
            "sessions8_ms_per_pass": round(multi_s * 1e3, 3), "sessions8_tokens_per_s": round(8 / multi_s, 1),
            "sessions8_with_logits_ms_per_pass": round(multi_lg_s * 1e3, 3),
            "sessions8_context": "8 sequences at positions 260-515, one token each per pass",
            "what": f"whole network on the device: embedding, {n_layers_desc}: RMS norm fused into the products' "
                    "input quantization, rope, f16 KV cache, prefill attention on f16 MFMAs, decode attention over "
                    "context chunks (per query head, or per GQA group on f16 MFMAs for large passes); logits; "
                    "host wall clock per forward call"}


def measured_peaks():
    """Dense int8 MFMA rate and HBM streaming-read rate of this GPU, from the probe kernels of
    hk_amd/csrc/peak.hip (libhkpeak.so, built with the engine); None if the probe library is absent.
    The roofline fractions stay against the published peaks (8 TB/s, 5.0 POPS)."""
    import ctypes

    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "hk_amd", "libhkpeak.so")
    if not os.path.exists(path):
        return None
    lib = ctypes.CDLL(path)
    lib.hkpeak_mfma_i8_tops.restype = ctypes.c_double
    lib.hkpeak_mfma_i8_tops.argtypes = [ctypes.c_int]
    lib.hkpeak_read_gbs.restype = ctypes.c_double
    lib.hkpeak_read_gbs.argtypes = [ctypes.c_uint64, ctypes.c_int]
    tops = lib.hkpeak_mfma_i8_tops(5)
    gbs = lib.hkpeak_read_gbs(2 << 30, 5)
    return {"mfma_i8_tops": round(tops, 1), "mfma_i8_frac_of_published": round(tops / INT8_PEAK_TOPS, 4),
            "hbm_read_gbs": round(gbs, 1), "hbm_read_frac_of_published": round(gbs / HBM_PEAK_GBS, 4),
            "how": "int8 MFMA: 4 independent v_mfma_i32_32x32x32_i8 chains per wave, 4 waves per SIMD, "
                   "pseudo-random operands, median of 5 x ~5 ms; HBM: grid-strided 16-B reads of a 2 GiB buffer, "
                   "median of 5"}


def measured_traffic():
    """HBM bytes per launch of the roofline kernel, as measured with rocprofv3 PMC counters
    (FETCH_SIZE + WRITE_SIZE, each scaled by what the counter reads for a plain copy of known
    size) and recorded in profiles/; None when no measurement is recorded."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "mmvr_q4k_gate_up_traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get("traffic_bytes")
    except (OSError, ValueError):
        return None


def time_graph(torch, eng, stream, fn, reps: int, per_graph: int = 10) -> float:
    """Average microseconds of one call of fn's GPU work: per_graph calls are captured back to back
    in one HIP graph (so the graph's own launch cost is spread over them) and the graph is
    replayed reps times."""
    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    cap.wait_stream(stream)
    with torch.cuda.graph(g, stream=cap):
        eng.set_stream(cap.cuda_stream)
        for _ in range(per_graph):
            fn()
    eng.set_stream(stream.cuda_stream)
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        g.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    return 1e3 * e0.elapsed_time(e1) / (reps * per_graph)


def physical_cores() -> int:
    """Physical cores among the CPUs this process may run on (hyperthread siblings count once)."""
    cpus = sorted(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else list(range(os.cpu_count() or 1))
    seen = set()
    for c in cpus:
        base = f"/sys/devices/system/cpu/cpu{c}/topology/"
        try:
            with open(base + "physical_package_id") as f1, open(base + "core_id") as f2:
                seen.add((f1.read().strip(), f2.read().strip()))
        except OSError:
            seen.add(("cpu", str(c)))
    return max(1, len(seen))


def cpu_model() -> str:
    fields = {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if ":" in line:
                    key, val = (p.strip() for p in line.split(":", 1))
                    fields.setdefault(key, val)
                if not line.strip() and fields:
                    break
    except OSError:
        return "unknown"
    name = fields.get("model name", "unknown")
    return f"{name} (vendor {fields.get('vendor_id', '?')}, family {fields.get('cpu family', '?')}, " \
           f"model {fields.get('model', '?')}, stepping {fields.get('stepping', '?')})"


def cpu_baseline(seconds: float):
    """hk's CPU decode kernel (its SIMD restatement, oracle/hk_cpu_simd.c: the dpu primitive of
    isa.zig on the best instruction set this host has, 16 KiB row chunks as matmul.zig hands them
    out) on the host's physical cores: the Q4_K 14336x4096 batch-1 matvec, repeated for about
    `seconds`, plus a single-thread figure. Reported in GB/s of weights + activations."""
    import numpy as np

    from hk_amd import formats as F, synth
    from oracle import oracle as O

    cores = physical_cores()
    level = O.simd_level()
    m, k = LLAMA8B["ffn"], LLAMA8B["hidden"]
    raw = synth.weights_np(F.Q4_K, m, k, synth.seed_for(4, 0))
    # 16 copies (528 MB) read in turn, so that the host's last-level cache cannot hold the weights
    copies = [raw.copy() for _ in range(16)]
    x = synth.activations_np(1, k, 1)[0]
    O.matvec_q4k_simd(raw, m, k, x, threads=cores, level=level)
    reps, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        O.matvec_q4k_simd(copies[reps % len(copies)], m, k, x, threads=cores, level=level)
        reps += 1
    dt = (time.perf_counter() - t0) / reps
    nbytes = raw.nbytes + 4 * k + 4 * m
    # The same product on one thread, for a figure comparable to hk-kernels' single-thread runs.
    reps1, t1 = 0, time.perf_counter()
    while time.perf_counter() - t1 < max(1.0, seconds / 4):
        O.matvec_q4k_simd(copies[reps1 % len(copies)], m, k, x, threads=1, level=level)
        reps1 += 1
    dt1 = (time.perf_counter() - t1) / reps1
    return {"value": round(nbytes / dt / 1e9, 2), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"Q4_K 14336x4096 matvec, batch 1, {reps} reps in {seconds:.0f} s over 16 copies (528 MB); hk's decode kernel "
                      f"({O.simd_level_name(level)} dot primitive, 16 KiB row chunks, OpenMP over {cores} physical cores)",
            "isa": O.simd_level_name(level),
            "single_thread_value": round(nbytes / dt1 / 1e9, 2), "cpu_model": cpu_model()}


if __name__ == "__main__":
    main()
