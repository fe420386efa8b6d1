"""Benchmark of the MI355X W4 quantized-matmul hot path (one JSON line on stdout).

Headline workload ("batched-agent decode MLP"): one step runs the decode MLP at each
M in {1, 8, 32, 128}: A[M, 5120] -> gate_up (4-bit, N = 2 x 17408, K = 5120) -> SwiGLU -> down (4-bit, N = 5120,
K = 17408), all through the C ABI (libinferd_amd.so). Weights are seeded synthetic MLX-affine 4-bit group-64
(q ~ U{0..15}, s ~ U(0.005, 0.02) bf16, b = bf16(-8 s)); activations bf16 N(0, 1). Weight copies are rotated so the
timed loop streams >= 3x the 256 MB Infinity Cache, as the reference cycles copies (engine/tools/moe_bench.mm:4-5).

value = algorithmic HBM bytes of the step / step time (GB/s): 150,405,120 weight bytes per M plus 90,112 activation
bytes per row (A in, the SwiGLU output written and read, the result; the gate/up product is never stored). The
reference's unfused count (229,376 B per row, with the gate/up product written and read) is reported beside it as
value_unfused_count. Each call of a step reads a weight copy no call of the previous five MLPs read.
The line also carries the measured HBM-read and MFMA ceilings of this GPU beside the datasheet peaks ("ceilings";
roofline.peak_measured / frac_measured). The other BASELINE configs are reported under "breakdown" (prefill TFLOP/s,
W4A8 TOPS, MoE tok/s, config-0 GB/s).
"""
from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

SETTLE_MS = 30.0  # minimum warmup load before a timed region (see --warmup)
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
INT8_PEAK_TOPS = 5000.0
LLC_BYTES = 256 << 20

H_DEC, I_DEC = 5120, 17408
W_BYTES_PER_WEIGHT = 0.5625  # packed nibbles + bf16 scale and bias per 64
ROW_BYTES_FUSED = (H_DEC + 2 * I_DEC + H_DEC) * 2  # A in, h out + in, y out: 90,112 B per row
ROW_BYTES_UNFUSED = (H_DEC + 2 * 2 * I_DEC + 2 * I_DEC + H_DEC) * 2  # + the gate/up product out and in: 229,376 B


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    # The GPU's clock needs about 20-30 ms of load to settle after an idle spell (the first calls run fast, then slow
    # while the power controller overshoots, then settle): the warmup runs at least --warmup steps and at least
    # kSettleMs of load, so the timed steps run in the steady state that continuous serving runs in.
    p.add_argument("--steps", type=int, default=40)
    p.add_argument("--warmup", type=int, default=100)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    p.add_argument("--no-breakdown", action="store_true", help="headline workload only")
    p.add_argument("--only", default="",
                   help="profiling: run one config only (c0, c1, c2, c3, c4, w8), or 'copy' (256 MiB device copy that "
                        "calibrates the FETCH_SIZE / WRITE_SIZE counters)")
    return p.parse_args()


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}): it measures one GPU's share of the "
              "path, and no multi-GPU run is built", file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch

    from inferd_amd import ops
    from inferd_amd.ops import MoeW, QLinear

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(1234)

    def qlin(N, K):
        wq = torch.randint(-2 ** 31, 2 ** 31 - 1, (N, K // 8), dtype=torch.int32, device=dev, generator=gen)
        s = (torch.rand((N, K // 64), device=dev, generator=gen) * 0.015 + 0.005).to(torch.bfloat16)
        b = (-8.0 * s.float()).to(torch.bfloat16)
        return QLinear(wq, s, b, N, K)

    def copies_for(nbytes):
        return max(1, -(-3 * LLC_BYTES // nbytes))

    def act(M, K, scale_rows=False):
        x = torch.randn((M, K), device=dev, generator=gen)
        if scale_rows:
            x = x * (torch.rand((M, 1), device=dev, generator=gen) * 1.5 + 0.5)
        return x.to(torch.bfloat16)

    def timed(fn, n, warm, settle_ms=30.0):
        # warm calls, then more until the call has loaded the GPU for settle_ms (the clock's settling time), so that
        # every breakdown figure is a steady-state one like the headline's
        for i in range(warm):
            fn(i)
        torch.cuda.synchronize()
        t0, i = time.perf_counter(), warm
        while (time.perf_counter() - t0) * 1e3 < settle_ms:
            for _ in range(4):
                fn(i)
                i += 1
            torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(n):
            fn(i)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n  # ms per call

    out = {}
    Ms = (1, 8, 32, 128)

    # ---- measured ceilings on this GPU, beside the datasheet peaks: one coalesced read of a 2 GiB buffer (8x the
    # Infinity Cache) and MFMA-only loops of the two shapes the kernels use (bf16 32x32x16, int8 32x32x32), each on
    # 512 blocks of 4 waves (two waves per SIMD)
    ceilings = {}
    if args.only in ("", "ceilings"):
        big = torch.empty(2 << 30, dtype=torch.uint8, device=dev)
        big.fill_(1)
        sink = torch.zeros(4096, dtype=torch.uint8, device=dev)
        ms = timed(lambda i: ops.probe_stream_read(big, sink), 10, 2)
        ceilings["hbm_read_gbs"] = big.numel() / (ms * 1e-3) / 1e9
        del big
        mo = torch.empty(512 * 256, dtype=torch.float32, device=dev)
        for int8, key, scale in ((False, "bf16_mfma_tflops", 1e12), (True, "int8_mfma_tops", 1e12)):
            ops_n = ops.probe_mfma(int8, 2000, 512, mo)
            ms = timed(lambda i: ops.probe_mfma(int8, 2000, 512, mo), 5, 1)
            ceilings[key] = ops_n / (ms * 1e-3) / scale
        out["ceilings"] = ceilings
        if args.only == "ceilings":
            print(json.dumps({k: round(v, 1) for k, v in ceilings.items()}), flush=True)
            return

    if args.only == "copy":
        # calibration for the FETCH_SIZE / WRITE_SIZE counters: a plain device copy of exactly 256 MiB each way
        src = torch.empty(128 << 20, dtype=torch.bfloat16, device=dev).normal_(generator=gen)
        dst = torch.empty_like(src)
        ms = timed(lambda i: dst.copy_(src), 20, 3)
        print(json.dumps({"copy_bytes_each_way": src.numel() * 2, "us": round(ms * 1e3, 2),
                          "gbs": round(2 * src.numel() * 2 / (ms * 1e-3) / 1e9, 1)}), flush=True)
        return

    # ---- headline: decode MLP (config 1) -----------------------------------------------------------------------
    if args.only in ("", "c1"):
        w_bytes = (2 * I_DEC * H_DEC + H_DEC * I_DEC) * W_BYTES_PER_WEIGHT
        ncp = copies_for(int(w_bytes))
        # MLX-layout weights are repacked once into the T64 layout (outside the timed region, as the reference
        # flips its weights once at load); copy 0 keeps its MLX form for the CPU baseline.
        host_layer = (qlin(2 * I_DEC, H_DEC), qlin(H_DEC, I_DEC))
        layers = [(ops.pack_t64(host_layer[0]), ops.pack_t64(host_layer[1]))]
        for _ in range(ncp - 1):
            gu_, dn_ = qlin(2 * I_DEC, H_DEC), qlin(H_DEC, I_DEC)
            layers.append((ops.pack_t64(gu_), ops.pack_t64(dn_)))
            del gu_, dn_
        A = {M: act(M, H_DEC) for M in Ms}
        Hh = {M: torch.empty((M, I_DEC), dtype=torch.bfloat16, device=dev) for M in Ms}
        Y = {M: torch.empty((M, H_DEC), dtype=torch.bfloat16, device=dev) for M in Ms}

        def mlp(M, c):
            # gate_up with its SwiGLU in one call (the reference's gemm + silu_mul pair), then down, on weight copy c
            gu, dn = layers[c % ncp]
            ops.gemm_t64_swiglu(A[M], gu, out=Hh[M])
            ops.gemm_t64(Hh[M], dn, Y[M])

        def step(i):
            # every call of the step reads a copy no call of the previous ncp - 1 MLPs read (ncp x 150 MB > 3 x LLC)
            for j, M in enumerate(Ms):
                mlp(M, i * len(Ms) + j)

        # at least args.warmup untimed steps, and at least SETTLE_MS of them (in batches of 8, so that the GPU stays
        # loaded between the host's checks)
        t0, i = time.perf_counter(), 0
        while i < args.warmup or (time.perf_counter() - t0) * 1e3 < SETTLE_MS:
            for _ in range(8 if i >= args.warmup else args.warmup):
                step(i)
                i += 1
            torch.cuda.synchronize()
        warm_steps = i
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(args.steps):
            step(i)
        e1.record()
        torch.cuda.synchronize()
        ms_step = e0.elapsed_time(e1) / args.steps
        # the bytes the step's calls move at minimum: weights, plus per row A in, h out and in, y out (the SwiGLU is
        # fused into gate_up, which never stores its product): 90,112 B. The reference's unfused sequence
        # gemm -> silu_mul -> gemm also writes and re-reads the gate/up product (229,376 B per row); that count is
        # reported beside it, labelled, never as the value.
        step_bytes = sum(w_bytes + M * ROW_BYTES_FUSED for M in Ms)
        step_bytes_unfused = sum(w_bytes + M * ROW_BYTES_UNFUSED for M in Ms)
        value = step_bytes / (ms_step * 1e-3) / 1e9

        # per-call timing (HIP events on the launch stream): the dominant call is the roofline kernel; bytes are each
        # call's own algorithmic traffic (weights, activation in, output)
        calls = {}
        for M in Ms:
            gu_b = 2 * I_DEC * H_DEC * W_BYTES_PER_WEIGHT + M * H_DEC * 2 + M * I_DEC * 2
            dn_b = H_DEC * I_DEC * W_BYTES_PER_WEIGHT + M * I_DEC * 2 + M * H_DEC * 2
            ms_gu = timed(lambda i: ops.gemm_t64_swiglu(A[M], layers[i % ncp][0], out=Hh[M]), args.steps * 2, 3)
            ms_dn = timed(lambda i: ops.gemm_t64(Hh[M], layers[i % ncp][1], Y[M]), args.steps * 2, 3)
            calls[f"gate_up_swiglu_M{M}"] = (ms_gu, gu_b, 2.0 * M * 2 * I_DEC * H_DEC)
            calls[f"down_M{M}"] = (ms_dn, dn_b, 2.0 * M * H_DEC * I_DEC)
        # the whole dense MLP block (rmsnorm, gate_up + SwiGLU, down with the residual add) as one operator
        nw = (torch.rand((H_DEC,), device=dev, generator=gen) + 0.5).to(torch.bfloat16)
        Xb = {M: act(M, H_DEC) for M in Ms}
        mlp_block = {}
        for M in Ms:
            ms_b = timed(lambda i: ops.mlp_decode(Xb[M], nw, 1e-6, *layers[i % ncp]), args.steps * 2, 3)
            mlp_block[f"M{M}"] = dict(us=ms_b * 1e3, gbs=(w_bytes + M * (4 * H_DEC + 2 * I_DEC) * 2) / (ms_b * 1e-3) / 1e9)
        out["mlp_block"] = mlp_block
        # the reference's default decode route for flipped weights (qwen35.h:1576): per-(row, 64-group) int8
        # activations, W4A8 gate_up, silu_mul_a8 (the next GEMM's int8 rows, core.metal:789-814), W4A8 down, both
        # GEMMs on the T64 copies (int8 rows as exact bf16 integers through the affine T64 kernels); bytes as value's
        # plus the gate/up product written and read (229,376 B per row: no SwiGLU epilogue on this route)
        w4a8_route = {}
        GUb = {M: torch.empty((M, 2 * I_DEC), dtype=torch.bfloat16, device=dev) for M in Ms}

        def w4a8_mlp(M, c):
            gu, dn = layers[c % ncp]
            U, XS = ops.a8_quant(A[M], False)
            ops.gemm_t64_w4a8(U, XS, gu, GUb[M], per_token=False)
            Uh, XSh = ops.silu_mul_a8(GUb[M], False)
            ops.gemm_t64_w4a8(Uh, XSh, dn, Y[M], per_token=False)

        for M in Ms:
            if M < 3:
                continue  # the reference takes the decode GEMV up to qmv_max = 2 rows
            ms_w = timed(lambda i: w4a8_mlp(M, i), args.steps, 3)
            w4a8_route[f"M{M}"] = dict(us=ms_w * 1e3, gbs=(w_bytes + M * ROW_BYTES_UNFUSED) / (ms_w * 1e-3) / 1e9)
        out["w4a8_route"] = w4a8_route
        dom = max(calls, key=lambda k: calls[k][0])
        ms_d, b_d, f_d = calls[dom]
        achieved = b_d / (ms_d * 1e-3) / 1e9
        out["headline"] = dict(ms_step=ms_step, value=value, step_bytes=step_bytes, copies=ncp, warmup_run=warm_steps,
                               value_unfused_count=step_bytes_unfused / (ms_step * 1e-3) / 1e9)
        out["dominant"] = dict(name=dom, ms=ms_d, bytes=b_d, flops=f_d, gbs=achieved,
                               tflops=f_d / (ms_d * 1e-3) / 1e12)
        out["per_M"] = {
            f"M{M}": dict(
                gate_up_swiglu_us=calls[f"gate_up_swiglu_M{M}"][0] * 1e3, down_us=calls[f"down_M{M}"][0] * 1e3,
                gate_up_swiglu_gbs=calls[f"gate_up_swiglu_M{M}"][1] / (calls[f"gate_up_swiglu_M{M}"][0] * 1e-3) / 1e9,
                down_gbs=calls[f"down_M{M}"][1] / (calls[f"down_M{M}"][0] * 1e-3) / 1e9)
            for M in Ms}
        del layers
    else:
        host_layer = None

    breakdown = {}
    if not args.no_breakdown or args.only:
        # ---- config 0: single qmv M=1, K=N=5120 ---------------------------------------------------------------
        if args.only in ("", "c0"):
            nb = int(5120 * 5120 * W_BYTES_PER_WEIGHT)
            ncp = copies_for(nb)
            Ws = [ops.pack_t64(qlin(5120, 5120)) for _ in range(ncp)]
            A0 = act(1, 5120)
            C0 = torch.empty((1, 5120), dtype=torch.bfloat16, device=dev)
            ms = timed(lambda i: ops.gemm_t64(A0, Ws[i % ncp], C0), 200, 20)
            byts = nb + 5120 * 2 * 2
            breakdown["c0_qmv_M1"] = dict(us=ms * 1e3, gbs=byts / (ms * 1e-3) / 1e9,
                                          frac_hbm=byts / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, copies=ncp)
            del Ws
            # four such linears sharing the input (a layer's q/k/v/o-sized projections) in one launch
            # (ifd_gemm_t64_multi), against four single launches of the same weights
            nl = 4
            nsets = copies_for(nl * nb)
            sets = [[ops.pack_t64(qlin(5120, 5120)) for _ in range(nl)] for _ in range(nsets)]
            Cm = [torch.empty((1, 5120), dtype=torch.bfloat16, device=dev) for _ in range(nl)]
            mcalls = [ops.gemm_t64_multi_call(A0, S, Cm) for S in sets]
            ms_m = timed(lambda i: mcalls[i % nsets](), 200, 20)

            def singles(i):
                for W, C in zip(sets[i % nsets], Cm):
                    ops.gemm_t64(A0, W, C)

            ms_s = timed(singles, 100, 10)
            breakdown["c0_multi4_M1"] = dict(us=ms_m * 1e3, us_per_linear=ms_m * 1e3 / nl,
                                             gbs=nl * byts / (ms_m * 1e-3) / 1e9,
                                             frac_hbm=nl * byts / (ms_m * 1e-3) / 1e9 / HBM_PEAK_GBS,
                                             singles_us_per_linear=ms_s * 1e3 / nl, copies=nsets)
            del sets, mcalls
        # ---- config 2: prefill qmm M=4096, K=5120, N=17408 ----------------------------------------------------
        if args.only in ("", "c2"):
            W2 = [ops.pack_t64(qlin(17408, 5120)) for _ in range(2)]
            A2 = act(4096, 5120, scale_rows=True)
            C2 = torch.empty((4096, 17408), dtype=torch.bfloat16, device=dev)
            ms = timed(lambda i: ops.gemm_t64(A2, W2[i % 2], C2), 10, 2)
            fl = 2.0 * 4096 * 17408 * 5120
            breakdown["c2_qmm_M4096"] = dict(us=ms * 1e3, tflops=fl / (ms * 1e-3) / 1e12,
                                             frac_bf16=fl / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS)
            del W2, A2, C2
        # ---- config 3: W4A8 M=2048, K=N=5120, per-token int8 --------------------------------------------------
        if args.only in ("", "c3"):
            W3 = [ops.pack_t64(qlin(5120, 5120)) for _ in range(4)]
            A3 = act(2048, 5120)
            U3, XS3 = ops.a8_quant(A3, True)
            C3 = torch.empty((2048, 5120), dtype=torch.bfloat16, device=dev)
            ms = timed(lambda i: ops.gemm_t64_w4a8(U3, XS3, W3[i % 4], C3), 20, 3)
            ms_q = timed(lambda i: ops.a8_quant(A3, True), 20, 3)
            op = 2.0 * 2048 * 5120 * 5120
            breakdown["c3_w4a8_M2048"] = dict(us=ms * 1e3, tops=op / (ms * 1e-3) / 1e12,
                                              frac_int8=op / (ms * 1e-3) / 1e12 / INT8_PEAK_TOPS,
                                              a8_quant_us=ms_q * 1e3)
            del W3
        # ---- 8-bit weights (config 0's shape and config 3's W8A8 shape) -----------------------------------------
        if args.only in ("", "w8"):
            def qlin8(N, K):
                wq = torch.randint(-2 ** 31, 2 ** 31 - 1, (N, K // 4), dtype=torch.int32, device=dev, generator=gen)
                s = ((torch.rand((N, K // 64), device=dev, generator=gen) * 0.015 + 0.005) / 16).to(torch.bfloat16)
                b = (-128.0 * s.float()).to(torch.bfloat16)
                return QLinear(wq, s, b, N, K, bits=8)

            nb8 = int(5120 * 5120 * (1 + 4 / 64))
            ncp = copies_for(nb8)
            W8 = [qlin8(5120, 5120) for _ in range(ncp)]
            w8 = {}
            for M in (1, 8, 32):
                A8 = act(M, 5120)
                C8 = torch.empty((M, 5120), dtype=torch.bfloat16, device=dev)
                ms = timed(lambda i: ops.gemm(A8, W8[i % ncp], C8), 200, 20)
                byts = nb8 + M * 5120 * 2 * 2
                w8[f"M{M}"] = dict(us=ms * 1e3, gbs=byts / (ms * 1e-3) / 1e9,
                                   frac_hbm=byts / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS)
            A8 = act(2048, 5120)
            U8, XS8 = ops.a8_quant(A8, True)
            C8 = torch.empty((2048, 5120), dtype=torch.bfloat16, device=dev)
            ms = timed(lambda i: ops.qmm_w4a8(U8, XS8, True, W8[i % 4], C8), 20, 3)
            op = 2.0 * 2048 * 5120 * 5120
            w8["w8a8_M2048"] = dict(us=ms * 1e3, tops=op / (ms * 1e-3) / 1e12,
                                    frac_int8=op / (ms * 1e-3) / 1e12 / INT8_PEAK_TOPS)
            T8 = [ops.pack_t64x8(W8[i % ncp]) for i in range(4)]
            ms = timed(lambda i: ops.gemm_t64x8_w8a8(U8, XS8, T8[i % 4], C8), 20, 3)
            w8["w8a8_t64x8_M2048"] = dict(us=ms * 1e3, tops=op / (ms * 1e-3) / 1e12,
                                          frac_int8=op / (ms * 1e-3) / 1e12 / INT8_PEAK_TOPS)
            del T8
            breakdown["w8_5120x5120"] = dict(w8, copies=ncp)
            del W8
            # the decode MLP's gate_up shape (N = 34816, K = 5120): long enough to stream at bandwidth
            nbg = int(34816 * 5120 * (1 + 4 / 64))
            ncg = copies_for(nbg)
            Wg = [qlin8(34816, 5120) for _ in range(ncg)]
            wg = {}
            for M in (1, 8, 32, 128):
                Ag = act(M, 5120)
                Cg = torch.empty((M, 34816), dtype=torch.bfloat16, device=dev)
                ms = timed(lambda i: ops.gemm(Ag, Wg[i % ncg], Cg), 40, 5)
                byts = nbg + M * (5120 + 34816) * 2
                wg[f"M{M}"] = dict(us=ms * 1e3, gbs=byts / (ms * 1e-3) / 1e9,
                                   frac_hbm=byts / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS)
            # the same layers repacked as T64x8, on the stream-K bf16 GEMM
            Tg = [ops.pack_t64x8(w) for w in Wg]
            for M in (1, 8, 32, 128):
                Ag = act(M, 5120)
                Cg = torch.empty((M, 34816), dtype=torch.bfloat16, device=dev)
                ms = timed(lambda i: ops.gemm_t64x8(Ag, Tg[i % ncg], Cg), 40, 5)
                byts = nbg + M * (5120 + 34816) * 2
                wg[f"t64x8_M{M}"] = dict(us=ms * 1e3, gbs=byts / (ms * 1e-3) / 1e9,
                                         frac_hbm=byts / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS)
            del Tg
            breakdown["w8_34816x5120"] = dict(wg, copies=ncg)
            del Wg
        # ---- config 4: MoE FFN H=2048, E=512, top-10, I=512, + shared expert ----------------------------------
        if args.only in ("", "c4"):
            E, H, I, k = 512, 2048, 512, 10

            def moew(N, K):
                q = qlin(E * N, K)
                return MoeW(q.wq.view(E, N, K // 8), q.s.view(E, N, K // 64), q.b.view(E, N, K // 64), E, N, K)

            ncp = 2
            lay = [(moew(2 * I, H), moew(H, I), qlin(2 * I, H), qlin(H, I)) for _ in range(ncp)]
            # the same experts repacked once into T64 stacks (the shared expert rides along as expert E)
            tlay = [(ops.pack_t64_stack(egu), ops.pack_t64_stack(edn), ops.pack_t64(sgu), ops.pack_t64(sdn))
                    for egu, edn, sgu, sdn in lay]
            router = (torch.randn((E, H), device=dev, generator=gen) * 0.02).to(torch.bfloat16)
            moe = {}
            e_bytes = (2 * I * H + H * I) * W_BYTES_PER_WEIGHT  # one expert's gate/up + down: 1,769,472 B
            for T in (16, 128, 2048):
                xn = act(T, H)
                outb = torch.zeros((T, H), dtype=torch.bfloat16, device=dev)

                def run_t64(i):
                    tgu, tdn, sgu, sdn = tlay[i % ncp]
                    ops.moe_ffn_t64(xn, router, tgu, tdn, k, shared=(sgu, sdn), shared_gate=False,
                                    logits_bf16=T >= 64, out=outb)

                def run(i):
                    egu, edn, sgu, sdn = lay[i % ncp]
                    ops.moe_ffn(xn, router, egu, edn, k, shared=(sgu, sdn), shared_gate=False,
                                logits_bf16=T >= 64, out=outb)

                ms = timed(run_t64, 10, 3)
                ms_mlx = timed(run, 5, 2)
                # algorithmic bytes: the distinct experts a uniform router touches, U(T) = E (1 - (1 - k/E)^T), the
                # shared expert, the router and the tokens in and out
                U = E * (1.0 - (1.0 - k / E) ** T)
                byts = (U + 1) * e_bytes + E * H * 2 + 2 * T * H * 2
                moe[f"T{T}"] = dict(us=ms * 1e3, tok_s=T / (ms * 1e-3), gbs=byts / (ms * 1e-3) / 1e9,
                                    frac_hbm=byts / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, mlx_layout_us=ms_mlx * 1e3)
            # the drop-in operator itself: Qwen35::encode_moe (rmsnorm, router, routing, the sorted route on the
            # loader's T64 copies with the shared expert as expert E, combine into x; at T = 8 the per-row route on
            # those copies, the shared expert as one more slot), timed by its own C++ program over this library; and
            # the same operator on the MLX-layout stacks alone
            for key, extra in (("encode_moe_t64", []), ("encode_moe_mlx", ["--mlx"])):
                prog = os.path.join(ROOT, "inferd_amd", "encode_moe_bench")
                if not os.path.exists(prog):
                    raise RuntimeError(f"{prog} is missing: run `python -m inferd_amd.build`")
                r = subprocess.run([prog, *extra, "8", "16", "128", "2048"], capture_output=True, text=True,
                                   timeout=600)
                if r.returncode != 0:
                    raise RuntimeError(f"encode_moe_bench failed ({r.returncode}): {r.stdout} {r.stderr}")
                op = json.loads(r.stdout.strip().splitlines()[-1])
                for T in (8, 16, 128, 2048):
                    U = E * (1.0 - (1.0 - k / E) ** T)
                    byts = (U + 1) * e_bytes + E * H * 2 + 2 * T * H * 2
                    op[f"T{T}"]["frac_hbm"] = byts / (op[f"T{T}"]["us"] * 1e-6) / 1e9 / HBM_PEAK_GBS
                moe[key] = op
            # decode batches (T <= 8): the four-launch decode MoE, each distinct expert read once, streaming the
            # T64 stacks (what encode_moe runs when the loader made them) and the MLX-layout stacks
            for T in (1, 2, 4, 8):
                xn = act(T, H)
                outb = torch.zeros((T, H), dtype=torch.bfloat16, device=dev)

                def run_dec_t64(i):
                    tgu, tdn, sgu, sdn = tlay[i % ncp]
                    ops.moe_decode_t64(xn, router, tgu, tdn, k, shared=(sgu, sdn), shared_gate=False, out=outb)

                def run_dec(i):
                    egu, edn, sgu, sdn = lay[i % ncp]
                    ops.moe_decode(xn, router, egu, edn, k, shared=(sgu, sdn), shared_gate=False, out=outb)

                ms = timed(run_dec_t64, 50, 5)
                ms_mlx = timed(run_dec, 50, 5)
                U = E * (1.0 - (1.0 - k / E) ** T)
                byts = (U + 1) * e_bytes + E * H * 2 + 2 * T * H * 2
                moe[f"decode_T{T}"] = dict(us=ms * 1e3, tok_s=T / (ms * 1e-3),
                                           frac_hbm=byts / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                                           mlx_layout_us=ms_mlx * 1e3)
            breakdown["c4_moe"] = moe
            del lay, tlay

    if breakdown:
        out["breakdown"] = breakdown

    # ---- CPU baseline: the oracle on this host's cores, bounded sample ---------------------------------------------
    cpu = None
    if not args.no_cpu and host_layer is not None:
        from oracle import oracle as orc
        ncores = len(os.sched_getaffinity(0))
        gu, dn = host_layer

        def h16(t):
            return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)

        def h32(t):
            return t.detach().cpu().numpy().view(np.uint32)

        gw = (h32(gu.wq), h16(gu.s), h16(gu.b))
        dw = (h32(dn.wq), h16(dn.s), h16(dn.b))
        # sample: whole headline steps (the decode MLP at M = 1, 8, 32, 128, every weight streamed by every pass, the
        # oracle's qmv arithmetic), repeated until at least 10 s of CPU work; the same metric and byte count as value
        rng = np.random.default_rng(0)
        t0 = time.perf_counter()
        nbytes, nsteps = 0, 0
        while time.perf_counter() - t0 < 10.0:
            for M in Ms:
                Ah = orc.f32_to_bf16(rng.standard_normal((M, H_DEC)).astype(np.float32))
                gy = orc.qmv(Ah, *gw, nthreads=ncores)
                hh = orc.silu_mul(orc.f32_to_bf16(gy))
                orc.qmv(hh, *dw, nthreads=ncores)
                nbytes += (2 * I_DEC * H_DEC + H_DEC * I_DEC) * W_BYTES_PER_WEIGHT + M * ROW_BYTES_FUSED
            nsteps += 1
        dt = time.perf_counter() - t0
        cpu = dict(value=nbytes / dt / 1e9, unit="GB/s", cores=ncores, kind="port",
                   sample=f"{nsteps} headline steps (decode MLP at M = 1, 8, 32, 128: gate_up 5120->34816, SwiGLU, "
                          f"down 17408->5120), the oracle's qmv arithmetic on {ncores} threads, {dt:.1f} s")

    line = {
        "metric": "W4 qmatmul HBM GB/s at decode M<=128; TFLOP/s at prefill M=4096; MoE tok/s",
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded 4-bit affine weights, bf16 N(0,1) activations)",
    }
    # HBM bytes per call of a bench call, from the FETCH_SIZE / WRITE_SIZE counter runs of the same workload scaled by
    # a plain 256 MiB device copy (profiles/traffic_c1_c0_c4.md); calls not measured report null
    measured_traffic = {"gate_up_swiglu_M128": 216816249}

    def roofline(d):
        # the bound is the larger of the call's two floors: its algorithmic bytes at HBM peak, its flops at dense
        # bf16 MFMA peak
        mfma = d["flops"] / (BF16_PEAK_TFLOPS * 1e12) > d["bytes"] / (HBM_PEAK_GBS * 1e9)
        ach, peak = (d["tflops"], BF16_PEAK_TFLOPS) if mfma else (d["gbs"], HBM_PEAK_GBS)
        r = {"kernel": d["name"], "bound": "mfma" if mfma else "hbm", "achieved": round(ach, 1), "peak": peak,
             "unit": "TFLOP/s" if mfma else "GB/s", "frac": round(ach / peak, 4),
             "traffic": measured_traffic.get(d["name"]),
             "us": round(d["ms"] * 1e3, 2), "gbs": round(d["gbs"], 1), "tflops": round(d["tflops"], 1)}
        pm = ceilings.get("bf16_mfma_tflops" if mfma else "hbm_read_gbs")
        if pm:  # the same achieved figure against this GPU's measured ceiling
            r["peak_measured"] = round(pm, 1)
            r["frac_measured"] = round(ach / pm, 4)
        return r

    if "headline" in out:
        h, d = out["headline"], out["dominant"]
        line.update({
            "value": round(h["value"], 1),
            "ms_per_step": round(h["ms_step"], 4),
            "warmup_steps_run": h["warmup_run"],
            "config": {"workload": "decode MLP (BASELINE config 1): M in {1,8,32,128}, gate_up 5120->34816, "
                                   "SwiGLU, down 17408->5120, 4-bit g64 weights in the T64 layout",
                       "weight_copies": h["copies"]},
            "roofline": roofline(d),
            "value_unfused_count": round(h["value_unfused_count"], 1),
            "per_M": {k: {kk: round(vv, 2) for kk, vv in v.items()} for k, v in out["per_M"].items()},
            "mlp_block": {k: {kk: round(vv, 2) for kk, vv in v.items()} for k, v in out["mlp_block"].items()},
            "w4a8_route": {k: {kk: round(vv, 2) for kk, vv in v.items()} for k, v in out["w4a8_route"].items()},
        })
    if cpu:
        line["cpu_baseline"] = {k: (round(v, 3) if isinstance(v, float) else v) for k, v in cpu.items()}
    if ceilings:
        line["ceilings"] = {"measured": {k: round(v, 1) for k, v in ceilings.items()},
                            "datasheet": {"hbm_read_gbs": HBM_PEAK_GBS, "bf16_mfma_tflops": BF16_PEAK_TFLOPS,
                                          "int8_mfma_tops": INT8_PEAK_TOPS}}
    if "breakdown" in out:
        line["breakdown"] = json.loads(json.dumps(out["breakdown"]), parse_float=lambda x: round(float(x), 4))
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
