#!/usr/bin/env python3
"""Throughput of the AWQ INT4 hot path on one MI355X.

Headline (`value`): decode dequant-GEMV at M=1 on the Llama-3-8B gate/up shape
(K=4096 -> N=14336, group 128; f32 activations ~N(0,1), f16 scales
U[0.002, 0.02], uniform 4-bit weights/zeros in AutoAWQ packing, f32 output),
in GB/s of algorithmic HBM bytes per call:
    K*N/2 + (K/g)*(N/8)*4 + (K/g)*N*2 + M*K*4 + M*N*4  = 30,580,736 B.
Secondary objects in the same JSON line: the decode at M=4 and 8 and a
measured read-stream ceiling (a plain streaming-read kernel from the bench
helper library over buffers of the decode call's size); prefill at M=2048 on
the same shape (fp16 activations, fp16 MFMA, fp32 accumulation; TFLOP/s of
2*M*N*K), with M=16, 64, 512 beside it; the standalone dequantize of K=14336,
N=4096, g64 (f32 out; GB/s of read+write); the gate and up projections of the
same shape with SiLU(gate) * up as one awq_gemm_silu_mul launch against the
unfused sequence (two awq_gemm launches and torch's SiLU and multiply) at
M = 1, 16, 64.

Step: one replay of a HIP graph of 100 back-to-back decode calls over
rotated weight copies; `--steps` timed steps (100 x steps calls) after
`--warmup` untimed steps. `ms_per_step` is the time of one such step;
`value` and `roofline` are per call.

Method: inputs resident in HBM before timing; the decode and the prefill
rows rotate over ceil(512 MB / weight bytes) independent weight copies so the
256 MB MALL cannot serve them. Calls are captured in a HIP graph (one graph =
many back-to-back launches on the stream) and the graph is replayed; HIP
events on that stream bracket the timed replays, after untimed calls
(`--warmup` for the decode; 200, about 50 ms, for the M=2048 prefill and the
dense GEMM beside it, since the clock ramps up over tens of milliseconds of
matrix-core work after the memory-bound phases) and a device synchronise on
both sides. The M=2048 prefill also replays about 200 untimed calls right
before the timed ones with no synchronisation in between: after the idle gap
of the synchronise the clock ramps again (measured 238 us per call without
them, 222 us with them, on one box). The rows of `decode_rows`,
`prefill_rows`, the fp32 prefill, the gate/up SiLU pair and `--sweep` replay
about 20 ms of untimed calls the same way before timing (mid-size prefill
points measured 2-12 % slow without). `roofline.achieved` = algorithmic bytes
(flops) per launch / average launch duration from those events.
Beside each graph-replay figure, `eager_us_per_call` times the reference
bench's own protocol (benches/awq_kernel_gemm.rs:318-340): wall clock around
launch + stream synchronise, 3 warm-up and 10 timed calls, so it includes the
host-side call cost and the launch latency.
cpu_baseline: the oracle's C restatement of the reference's f32 loop on the
host cores (OpenMP), on a bounded sample of the same decode workload, with the
host CPU model. `config1_decode_4096x4096_f32_scales` holds the CPU-baseline
configuration (4096 -> 4096, g128, f32 scales, M = 1) with the GPU and CPU
timings side by side.
"""
import argparse
import json
import math
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "cube-awq_amd"))

METRIC = "M=1 decode GB/s (% of HBM peak) + M=2048 prefill TFLOPS, 4096x14336 AWQ g128"
HBM_PEAK_GBS = 8000.0
FP16_MFMA_PEAK_TFLOPS = 2500.0  # dense fp16 MFMA, MI355X published figure
CALLS_PER_STEP = 100  # decode calls per timed step (one graph replay)
TRAFFIC_FILE = os.path.join(REPO, "profiles", "hbm_traffic.json")


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200,
                    help="timed steps (one step = a graph replay of 100 decode calls)")
    ap.add_argument("--warmup", type=int, default=5, help="untimed steps")
    ap.add_argument("--only", choices=["decode", "prefill", "dequant", "copy"], default=None,
                    help="run one workload only (profiling runs); 'copy' is a plain 256 MiB "
                         "device copy used to calibrate the FETCH_SIZE / WRITE_SIZE counters")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--point", default=None, metavar="M,K,N,DTYPE",
                    help="instead of the headline line: time one awq_gemm point (g128, f16 scales, "
                         "DTYPE activations and output: f32/f16/bf16) over --steps x 100 graph-replayed "
                         "calls on rotated weight copies, for profiling one kernel route")
    ap.add_argument("--sweep", action="store_true",
                    help="instead of the headline line: one JSON line per point of the decode sweep "
                         "(Llama-3-8B shapes, M = 1, 4, 8, f32 x), the prefill sweep (Llama-3-8B "
                         "shapes, M = 64, 512, 2048, f16 x) and the Llama-3-70B projections "
                         "(M = 1, 8, 128, 1024, 4096, f16 x)")
    return ap.parse_args()


# Sweep points: (name, x dtype, shapes K -> N, row counts[, scale dtype]),
# g128, f16 scales unless named, output in the activation dtype (f32 for the
# decode sweep). reference_qwen2_f32: the reference benchmark's own cases
# (benches/awq_kernel_gemm.rs:575-685, Qwen2-0.5B projections, f32 everything;
# decode b1/b8, prefill s128/s512), also timed by its eager protocol.
SWEEPS = [
    ("decode_llama3_8b", "f32", [(4096, 4096), (4096, 1024), (4096, 14336), (14336, 4096)], (1, 4, 8)),
    ("prefill_llama3_8b", "f16", [(4096, 4096), (4096, 14336), (14336, 4096)], (64, 512, 2048)),
    ("prefill_f32_llama3_8b", "f32", [(4096, 4096), (4096, 14336), (14336, 4096)], (17, 64, 128, 512, 2048)),
    ("llama3_70b", "f16", [(8192, 8192), (8192, 1024), (8192, 28672), (28672, 8192)], (1, 8, 128, 1024, 4096)),
    ("reference_qwen2_f32", "f32", [(896, 896), (896, 4864), (4864, 896)], (1, 8, 128, 512), "f32"),
]
FP32_PEAK_TFLOPS = 157.3  # dense fp32, MI355X published figure


def sweep(dev, np, torch, synth, _lib, call_gemm, graph_time, points=None, steps_override=None,
          eager_time=None):
    """One JSON line per (sweep, shape, M): time per call from HIP events over
    graph-replayed launches on rotated weight copies (as the headline), GB/s
    of algorithmic bytes K*N/2 + (K/g)*(N/8)*4 + (K/g)*N*2 + M*K*xs + M*N*ys,
    TFLOP/s of 2*M*N*K, and both as fractions of the HBM and fp16 MFMA peaks.
    `points` replaces SWEEPS with [(name, x dtype, [(K, N)], rows)]."""
    G = 128
    dt = {"f32": (_lib.AWQ_F32, torch.float32, np.float32, 4), "f16": (_lib.AWQ_F16, torch.float16, np.float16, 2),
          "bf16": (_lib.AWQ_BF16, torch.bfloat16, "bfloat16", 2)}
    for entry in (points or SWEEPS):
        name, xdt, shapes, rows = entry[:4]
        sdt = entry[4] if len(entry) > 4 else "f16"
        xt, tdt, ndt, xs = dt[xdt]
        st, _, sndt, ss = dt[sdt]
        for K, N in shapes:
            qw = torch.from_numpy(synth.packed_nibbles(synth.TID_QWEIGHT, K, N // 8).view(np.int32)).to(dev)
            qz = torch.from_numpy(synth.packed_nibbles(synth.TID_QZEROS, K // G, N // 8).view(np.int32)).to(dev)
            sc = torch.from_numpy(synth.uniform(synth.TID_SCALES, (K // G, N), 0.002, 0.02, sndt)).to(dev)
            w_bytes = K * N // 2 + (K // G) * (N // 8) * 4 + (K // G) * N * ss
            copies = max(1, math.ceil(512e6 / w_bytes))
            ws = [(qw.clone(), qz.clone(), sc.clone()) for _ in range(copies)]
            for M in rows:
                xh = synth.normal(synth.TID_X, (M, K), ndt)
                x = (torch.from_numpy(xh.view(np.int16)).view(torch.bfloat16) if xdt == "bf16"
                     else torch.from_numpy(xh)).to(dev)
                y = torch.empty((M, N), dtype=tdt, device=dev)

                def launch(i, x=x, y=y, M=M):
                    w = ws[i % copies]
                    call_gemm(x, xt, w[0], w[1], w[2], st, y, xt, M, K, N, G)

                flops = 2.0 * M * N * K
                # at least ~10 ms of calls per point (the matrix cores settle at a
                # power-limited clock after the first few milliseconds)
                steps = 2000 if flops < 2e10 else 200 if flops < 5e11 else 50
                if steps_override:
                    steps = steps_override
                warm = 5 if flops < 5e11 else 100  # clock ramp on long matrix-core runs
                ms, _, _ = graph_time(launch, min(100, steps), warm, steps, warm_replays=-1)
                nbytes = w_bytes + M * K * xs + M * N * xs
                gbs = nbytes / (ms * 1e-3) / 1e9
                tflops = flops / (ms * 1e-3) / 1e12
                line = dict(sweep=name, M=M, K=K, N=N, x=xdt, scales=sdt, us=round(ms * 1e3, 2),
                            gbs=round(gbs, 1), hbm_frac=round(gbs / HBM_PEAK_GBS, 4), tflops=round(tflops, 1),
                            mfma_frac=round(tflops / FP16_MFMA_PEAK_TFLOPS, 4))
                if xdt == "f32":
                    line["fp32_peak_frac"] = round(tflops / FP32_PEAK_TFLOPS, 4)
                if eager_time is not None and name.startswith("reference"):
                    line["eager_us"] = round(eager_time(launch) * 1e3, 2)
                print(json.dumps(line), flush=True)
                del x, y
            del ws, qw, qz, sc
            torch.cuda.empty_cache()


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: there is no multi-GPU path here; a sharded "
              "deployment runs this single-GPU kernel on each GPU's shard.", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import cube_awq
    from cube_awq import _lib, synth

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    L = cube_awq.lib()

    def cur_stream():
        # the stream torch is issuing on (the capture stream inside torch.cuda.graph)
        return torch.cuda.current_stream().cuda_stream

    def call_gemm(x, xt, qw, qz, sc, st, y, yt, M, K, N, g):
        rc = L.awq_gemm(x.data_ptr(), xt, qw.data_ptr(), qz.data_ptr(), sc.data_ptr(), st, None,
                        _lib.AWQ_F32, y.data_ptr(), yt, M, K, N, g, cur_stream())
        if rc:
            _lib.check(rc)

    run_stream = torch.cuda.Stream()  # warm-up, capture, replay and events all on it

    def graph_time(launch, per_graph, warmup, steps, warm_replays=0):
        """ms per call over exactly `steps` calls: `launch(i)` captured into a
        graph of `per_graph` calls (plus one graph for the remainder), replayed;
        events on the launch stream, device synchronised on both sides.
        `warm_replays` untimed replays run right before the timed ones, with
        no synchronisation in between, so the timed calls start on a GPU that
        is already busy (matrix-core-heavy calls run at a lower clock for
        tens of milliseconds after an idle gap); -1: as many as make about
        20 ms, from one timed replay."""
        per_graph = max(1, min(per_graph, steps))
        torch.cuda.synchronize()
        with torch.cuda.stream(run_stream):
            # Warm-up on the capture stream: the library's per-stream split-K
            # workspace is allocated here, never inside the capture.
            for i in range(max(warmup, 1)):
                launch(i)
        torch.cuda.synchronize()
        reps, rem = divmod(steps, per_graph)
        graphs = []
        for n_calls, n_reps in ((per_graph, reps), (rem, 1)):
            if n_calls == 0 or n_reps == 0:
                continue
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=run_stream):
                for i in range(n_calls):
                    launch(i)
            graphs.append((g, n_reps))
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(run_stream):
            graphs[0][0].replay()  # untimed: first replay uploads the graph
            torch.cuda.synchronize()
            if warm_replays < 0:
                w0, w1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                w0.record(run_stream)
                graphs[0][0].replay()
                w1.record(run_stream)
                w1.synchronize()
                warm_replays = min(200, math.ceil(20.0 / max(w0.elapsed_time(w1), 1e-3)))
            for _ in range(warm_replays):
                graphs[0][0].replay()
            t0 = time.perf_counter()
            e0.record(run_stream)
            for g, n_reps in graphs:
                for _ in range(n_reps):
                    g.replay()
            e1.record(run_stream)
            e1.synchronize()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        ms = e0.elapsed_time(e1) / steps
        return ms, steps, wall

    def eager_time(launch, warm=3, runs=10):
        """ms per call by the reference bench's protocol: wall clock around
        launch + stream synchronise, `warm` untimed and `runs` timed calls."""
        torch.cuda.synchronize()
        with torch.cuda.stream(run_stream):
            for i in range(warm):
                launch(i)
                run_stream.synchronize()
            t0 = time.perf_counter()
            for i in range(runs):
                launch(warm + i)
                run_stream.synchronize()
            el = time.perf_counter() - t0
        return el / runs * 1e3

    if args.point:
        pm, pk, pn, pdt = args.point.split(",")
        sweep(dev, np, torch, synth, _lib, call_gemm, graph_time,
              points=[("point", pdt, [(int(pk), int(pn))], (int(pm),))], steps_override=args.steps * 100)
        return
    if args.sweep:
        sweep(dev, np, torch, synth, _lib, call_gemm, graph_time, eager_time=eager_time)
        return

    out = {}
    traffic = {}
    if os.path.exists(TRAFFIC_FILE):
        with open(TRAFFIC_FILE) as f:
            traffic = json.load(f)

    # ---------------- decode M=1, 4096 -> 14336 -------------------------------------------
    M, K, N, G = 1, 4096, 14336, 128
    dec_bytes = K * N // 2 + (K // G) * (N // 8) * 4 + (K // G) * N * 2 + M * K * 4 + M * N * 4
    if args.only in (None, "decode"):
        qw = torch.from_numpy(synth.packed_nibbles(synth.TID_QWEIGHT, K, N // 8).view(np.int32)).to(dev)
        qz = torch.from_numpy(synth.packed_nibbles(synth.TID_QZEROS, K // G, N // 8).view(np.int32)).to(dev)
        sc = torch.from_numpy(synth.uniform(synth.TID_SCALES, (K // G, N), 0.002, 0.02, np.float16)).to(dev)
        x = torch.from_numpy(synth.normal(synth.TID_X, (M, K), np.float32)).to(dev)
        # 17 copies: any copy is reused only after >= 15 other calls (459 MB) even
        # across graph replays of 100 calls, so the 256 MB MALL cannot hold it.
        copies = math.ceil(512e6 / dec_bytes)
        ws = [(qw.clone(), qz.clone(), sc.clone()) for _ in range(copies)]
        y = torch.empty((M, N), dtype=torch.float32, device=dev)

        def dec(i):
            w = ws[i % copies]
            call_gemm(x, _lib.AWQ_F32, w[0], w[1], w[2], _lib.AWQ_F16, y, _lib.AWQ_F32, M, K, N, G)

        ms, calls, wall = graph_time(dec, CALLS_PER_STEP, args.warmup * CALLS_PER_STEP,
                                     args.steps * CALLS_PER_STEP)
        gbs = dec_bytes / (ms * 1e-3) / 1e9
        out["decode"] = dict(ms=ms, calls=calls, wall_s=wall, gbs=gbs, bytes=dec_bytes, copies=copies,
                             eager_ms=eager_time(dec))

        if args.only is None:
            # The other decode rows of the same shape (matrix-core kernel).
            out["decode_rows"] = {}
            for mr in (4, 8):
                xr = torch.from_numpy(synth.normal(synth.TID_X, (mr, K), np.float32)).to(dev)
                yr = torch.empty((mr, N), dtype=torch.float32, device=dev)
                r_bytes = dec_bytes + (mr - 1) * (K + N) * 4

                def dec_r(i, xr=xr, yr=yr, mr=mr):
                    w = ws[i % copies]
                    call_gemm(xr, _lib.AWQ_F32, w[0], w[1], w[2], _lib.AWQ_F16, yr, _lib.AWQ_F32, mr, K, N, G)

                rms, _, _ = graph_time(dec_r, 100, 50, 2000, warm_replays=-1)
                out["decode_rows"][mr] = dict(us=rms * 1e3, gbs=r_bytes / (rms * 1e-3) / 1e9)

            # The CPU-baseline configuration: 4096 -> 4096, g128, f32 x, f32
            # scales, f32 y, M = 1 (graph-replayed and eager, rotated copies).
            K1, N1 = 4096, 4096
            c1_bytes = K1 * N1 // 2 + (K1 // G) * (N1 // 8) * 4 + (K1 // G) * N1 * 4 + K1 * 4 + N1 * 4
            c1_copies = math.ceil(512e6 / c1_bytes)
            c1qw = torch.from_numpy(synth.packed_nibbles(synth.TID_QWEIGHT, K1, N1 // 8).view(np.int32)).to(dev)
            c1qz = torch.from_numpy(synth.packed_nibbles(synth.TID_QZEROS, K1 // G, N1 // 8).view(np.int32)).to(dev)
            c1sc = torch.from_numpy(synth.uniform(synth.TID_SCALES, (K1 // G, N1), 0.002, 0.02, np.float32)).to(dev)
            c1w = [(c1qw.clone(), c1qz.clone(), c1sc.clone()) for _ in range(c1_copies)]
            c1x = torch.from_numpy(synth.normal(synth.TID_X, (1, K1), np.float32)).to(dev)
            c1y = torch.empty((1, N1), dtype=torch.float32, device=dev)

            def cfg1(i):
                w = c1w[i % c1_copies]
                call_gemm(c1x, _lib.AWQ_F32, w[0], w[1], w[2], _lib.AWQ_F32, c1y, _lib.AWQ_F32, 1, K1, N1, G)

            c1ms, _, _ = graph_time(cfg1, 100, 100, 2000)
            out["config1"] = dict(us=c1ms * 1e3, gbs=c1_bytes / (c1ms * 1e-3) / 1e9, bytes=c1_bytes,
                                  eager_us=eager_time(cfg1) * 1e3)
            del c1w, c1qw, c1qz, c1sc

            # Measured read-stream ceiling: a plain streaming-read kernel (the
            # bench helper library, not the AWQ library) over buffers of the
            # decode call's size, rotated the same way, timed the same way.
            import ctypes
            hl = ctypes.CDLL(os.path.join(REPO, "cube-awq_amd", "lib", "libawq_bench_gfx950.so"))
            hl.awqbench_read_stream.restype = ctypes.c_int
            hl.awqbench_read_stream.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
                                                ctypes.c_int, ctypes.c_void_p]
            rs_bytes = dec_bytes // 16 * 16
            bufs = [torch.ones(rs_bytes // 4, dtype=torch.float32, device=dev) for _ in range(copies)]
            grid = 2048
            sink = torch.zeros(grid, dtype=torch.int32, device=dev)

            def stream(i):
                rc = hl.awqbench_read_stream(bufs[i % copies].data_ptr(), rs_bytes, sink.data_ptr(),
                                             grid, cur_stream())
                if rc:
                    raise RuntimeError(f"read-stream launch failed: {rc}")

            sms, _, _ = graph_time(stream, 100, 50, 2000)
            out["read_stream"] = dict(us=sms * 1e3, gbs=rs_bytes / (sms * 1e-3) / 1e9)
            del bufs
        del ws

        if args.only is None:
            # Llama-3-8B MLP input half, gate and up 4096 -> 14336 each: one
            # awq_gemm_silu_mul launch over the column-interleaved weights
            # (28672 wide) against the unfused sequence (two awq_gemm launches
            # and torch's SiLU * up), both on rotated weight copies.
            NI = 2 * N
            gu_bytes = K * NI // 2 + (K // G) * (NI // 8) * 4 + (K // G) * NI * 2
            gcopies = math.ceil(512e6 / gu_bytes)
            fqw = torch.from_numpy(synth.packed_nibbles(synth.TID_QWEIGHT, K, NI // 8).view(np.int32)).to(dev)
            fqz = torch.from_numpy(synth.packed_nibbles(synth.TID_QZEROS, K // G, NI // 8).view(np.int32)).to(dev)
            fsc = torch.from_numpy(synth.uniform(synth.TID_SCALES, (K // G, NI), 0.002, 0.02, np.float16)).to(dev)
            h = N // 8
            # per copy: the fused tensors, then gate and up (halves of the same
            # columns) as separate contiguous tensors for the unfused sequence
            gw = [(fqw.clone(), fqz.clone(), fsc.clone(),
                   fqw[:, :h].contiguous(), fqz[:, :h].contiguous(), fsc[:, :N].contiguous(),
                   fqw[:, h:].contiguous(), fqz[:, h:].contiguous(), fsc[:, N:].contiguous())
                  for _ in range(gcopies)]
            del fqw, fqz, fsc
            out["gate_up_silu"] = {}
            for mr, xdt in ((1, np.float32), (16, np.float16), (64, np.float16)):
                xt = _lib.AWQ_F32 if xdt == np.float32 else _lib.AWQ_F16
                tdt = torch.float32 if xdt == np.float32 else torch.float16
                xr = torch.from_numpy(synth.normal(synth.TID_X, (mr, K), xdt)).to(dev)
                yf = torch.empty((mr, N), dtype=tdt, device=dev)
                yg = torch.empty((mr, N), dtype=tdt, device=dev)
                yu = torch.empty((mr, N), dtype=tdt, device=dev)
                ys = torch.empty((mr, N), dtype=tdt, device=dev)

                def fused(i, xr=xr, yf=yf, mr=mr, xt=xt):
                    w = gw[i % gcopies]
                    rc = L.awq_gemm_silu_mul(xr.data_ptr(), xt, w[0].data_ptr(), w[1].data_ptr(), w[2].data_ptr(),
                                             _lib.AWQ_F16, None, _lib.AWQ_F32, yf.data_ptr(), xt, mr, K, NI, G,
                                             cur_stream())
                    if rc:
                        _lib.check(rc)

                def unfused(i, xr=xr, yg=yg, yu=yu, ys=ys, mr=mr, xt=xt):
                    w = gw[i % gcopies]
                    call_gemm(xr, xt, w[3], w[4], w[5], _lib.AWQ_F16, yg, xt, mr, K, N, G)
                    call_gemm(xr, xt, w[6], w[7], w[8], _lib.AWQ_F16, yu, xt, mr, K, N, G)
                    torch.mul(torch.nn.functional.silu(yg), yu, out=ys)

                fms, _, _ = graph_time(fused, 50, 20, 500, warm_replays=-1)
                ums, _, _ = graph_time(unfused, 50, 20, 500, warm_replays=-1)
                out["gate_up_silu"][mr] = dict(fused_us=fms * 1e3, unfused_us=ums * 1e3)
            del gw

    # ---------------- prefill M=2048, 4096 -> 14336 ---------------------------------------
    PM = 2048
    pf_flops = 2.0 * PM * N * K
    if args.only in (None, "prefill"):
        qw = torch.from_numpy(synth.packed_nibbles(synth.TID_QWEIGHT, K, N // 8).view(np.int32)).to(dev)
        qz = torch.from_numpy(synth.packed_nibbles(synth.TID_QZEROS, K // G, N // 8).view(np.int32)).to(dev)
        sc = torch.from_numpy(synth.uniform(synth.TID_SCALES, (K // G, N), 0.002, 0.02, np.float16)).to(dev)
        # Rotated weight copies (>= 512 MB, as for the decode): each call reads
        # its weights from HBM, not from the 256 MB MALL.
        pcopies = math.ceil(512e6 / (K * N // 2))
        pw = [(qw.clone(), qz.clone(), sc.clone()) for _ in range(pcopies)]
        xp = torch.from_numpy(synth.normal(synth.TID_X, (PM, K), np.float16)).to(dev)
        yp = torch.empty((PM, N), dtype=torch.float16, device=dev)

        def pre(i):
            w = pw[i % pcopies]
            call_gemm(xp, _lib.AWQ_F16, w[0], w[1], w[2], _lib.AWQ_F16, yp, _lib.AWQ_F16, PM, K, N, G)

        # 200 untimed calls (~50 ms) first: after the memory-bound decode phase
        # the clock takes tens of milliseconds of matrix-core work to ramp up
        # (measured: the first 50 calls averaged 285 us, the following ones 240).
        steps = 100 if args.only is None else max(10, args.steps // 100)
        ms, calls, wall = graph_time(pre, pcopies, 200, steps, warm_replays=math.ceil(200 / pcopies))
        out["prefill"] = dict(ms=ms, calls=calls, wall_s=wall, tflops=pf_flops / (ms * 1e-3) / 1e12, copies=pcopies,
                              eager_ms=eager_time(pre))
        if args.only is None:
            # The other prefill rows of the same shape.
            out["prefill_rows"] = {}
            for mr in (16, 64, 512):
                xr = xp[:mr].contiguous()
                yr = torch.empty((mr, N), dtype=torch.float16, device=dev)

                def pre_r(i, xr=xr, yr=yr, mr=mr):
                    w = pw[i % pcopies]
                    call_gemm(xr, _lib.AWQ_F16, w[0], w[1], w[2], _lib.AWQ_F16, yr, _lib.AWQ_F16, mr, K, N, G)

                rms, _, _ = graph_time(pre_r, 20, 10, 200, warm_replays=-1)
                out["prefill_rows"][mr] = dict(us=rms * 1e3, tflops=2.0 * mr * N * K / (rms * 1e-3) / 1e12)
            # fp32 activations (the reference's own float type) at prefill
            # sizes: x split into f16 hi + lo on the matrix cores, f32 output.
            out["prefill_f32_rows"] = {}
            for mr in (128, 512, 2048):
                xf = torch.from_numpy(synth.normal(synth.TID_X, (mr, K), np.float32)).to(dev)
                yf = torch.empty((mr, N), dtype=torch.float32, device=dev)

                def pre_f(i, xf=xf, yf=yf, mr=mr):
                    w = pw[i % pcopies]
                    call_gemm(xf, _lib.AWQ_F32, w[0], w[1], w[2], _lib.AWQ_F16, yf, _lib.AWQ_F32, mr, K, N, G)

                rms, _, _ = graph_time(pre_f, pcopies, 20, 50, warm_replays=-1)
                out["prefill_f32_rows"][mr] = dict(us=rms * 1e3, tflops=2.0 * mr * N * K / (rms * 1e-3) / 1e12)
                del xf, yf
            # Context, not a roofline: the library dense fp16 GEMM (torch ->
            # hipBLASLt) of the same shape on unquantised f16 weights, W given
            # as [N, K] (its faster layout). The fused kernel additionally
            # dequantises W on the fly.
            wd = torch.randn((N, K), dtype=torch.float16, device=dev,
                             generator=torch.Generator(device=dev).manual_seed(7))
            yd = torch.empty((PM, N), dtype=torch.float16, device=dev)

            def dense(i):
                torch.matmul(xp, wd.t(), out=yd)

            try:
                dms, _, _ = graph_time(dense, 10, 200, 100)  # same warm-up and count as the fused call
                out["prefill"]["dense_tflops"] = pf_flops / (dms * 1e-3) / 1e12
            except RuntimeError as e:  # informational only: never fail the bench on it
                print(f"dense comparison skipped: {e}", file=sys.stderr)
            del wd, yd

    # ---------------- dequantize K=14336, N=4096, g64 -------------------------------------
    DK, DN, DG = 14336, 4096, 64
    dq_bytes = DK * DN // 2 + (DK // DG) * DN // 2 + (DK // DG) * DN * 4 + DK * DN * 4
    if args.only in (None, "dequant"):
        dqw = torch.from_numpy(synth.packed_nibbles(synth.TID_QWEIGHT, DK, DN // 8).view(np.int32)).to(dev)
        dqz = torch.from_numpy(synth.packed_nibbles(synth.TID_QZEROS, DK // DG, DN // 8).view(np.int32)).to(dev)
        dsc = torch.from_numpy(synth.uniform(synth.TID_SCALES, (DK // DG, DN), 0.002, 0.02, np.float32)).to(dev)
        dout = torch.empty((DK, DN), dtype=torch.float32, device=dev)

        def deq(i):
            rc = L.awq_dequantize(dqw.data_ptr(), dqz.data_ptr(), dsc.data_ptr(), _lib.AWQ_F32,
                                  dout.data_ptr(), _lib.AWQ_F32, DK, DN, DG,
                                  _lib.AWQ_ORDER_SEQUENTIAL, cur_stream())
            if rc:
                _lib.check(rc)

        steps = 200 if args.only is None else max(20, args.steps // 20)
        ms, calls, wall = graph_time(deq, 20, 10, steps)
        out["dequant"] = dict(ms=ms, calls=calls, wall_s=wall, gbs=dq_bytes / (ms * 1e-3) / 1e9,
                              bytes=dq_bytes)

    # ---------------- counter calibration: plain 256 MiB device copy ----------------------
    if args.only == "copy":
        src = torch.ones(64 << 20, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(max(1, args.warmup)):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_each_way": src.numel() * 4, "calls": max(1, args.warmup)}))
        return

    # ---------------- CPU baseline (oracle, host cores) -----------------------------------
    cpu = None
    if not args.no_cpu_baseline and args.only in (None, "decode"):
        sys.path.insert(0, os.path.join(REPO, "oracle"))
        import awq_oracle as oracle
        hx = synth.normal(synth.TID_X, (M, K), np.float32)
        hqw = synth.packed_nibbles(synth.TID_QWEIGHT, K, N // 8)
        hqz = synth.packed_nibbles(synth.TID_QZEROS, K // G, N // 8)
        hsc = synth.uniform(synth.TID_SCALES, (K // G, N), 0.002, 0.02, np.float16).astype(np.float32)
        oracle.gemm_f32(hx, hqw, hqz, hsc, G)  # warm-up
        n = 0
        t0 = time.perf_counter()
        while True:
            oracle.gemm_f32(hx, hqw, hqz, hsc, G)
            n += 1
            el = time.perf_counter() - t0
            if el >= args.cpu_seconds and n >= 3:
                break
        cpu_model = "unknown"
        try:
            with open("/proc/cpuinfo") as f:
                for line in f:
                    if line.startswith("model name"):
                        cpu_model = line.split(":", 1)[1].strip()
                        break
        except OSError:
            pass
        cpu = dict(value=dec_bytes / (el / n) / 1e9, unit="GB/s", cores=oracle.num_threads(),
                   kind="port", cpu_model=cpu_model, host_cpus=os.cpu_count(),
                   sample=f"{n} calls of the M=1 4096x14336 g128 decode (oracle f32 loop, "
                          f"{el:.1f} s, OpenMP over {oracle.num_threads()} threads)")
        if "config1" in out:
            # The same loop on the CPU-baseline configuration (4096 -> 4096, f32
            # scales), timed by the reference bench's protocol (3 warm-up, then
            # wall clock over >= 10 calls and >= 2 s).
            K1, N1 = 4096, 4096
            c1x = synth.normal(synth.TID_X, (1, K1), np.float32)
            c1qw = synth.packed_nibbles(synth.TID_QWEIGHT, K1, N1 // 8)
            c1qz = synth.packed_nibbles(synth.TID_QZEROS, K1 // G, N1 // 8)
            c1sc = synth.uniform(synth.TID_SCALES, (K1 // G, N1), 0.002, 0.02, np.float32)
            for _ in range(3):
                oracle.gemm_f32(c1x, c1qw, c1qz, c1sc, G)
            n1 = 0
            t0 = time.perf_counter()
            while True:
                oracle.gemm_f32(c1x, c1qw, c1qz, c1sc, G)
                n1 += 1
                el1 = time.perf_counter() - t0
                if n1 >= 10 and el1 >= 2.0:
                    break
            out["config1"]["cpu_us"] = el1 / n1 * 1e6
            out["config1"]["cpu_calls"] = n1

    res = {
        "metric": METRIC,
        "value": None,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": None,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: SplitMix64-seeded uniform 4-bit weights/zeros (AutoAWQ packing), "
                "N(0,1) activations, U[0.002,0.02] scales",
        "config": {"workload": "AWQ decode dequant-GEMV M=1, K=4096 -> N=14336 (Llama-3-8B "
                               "gate/up), group 128, f32 activations, f16 scales, f32 output",
                   "M": M, "K": K, "N": N, "group_size": G, "parallelism": "single GPU"},
    }
    if "decode" in out:
        d = out["decode"]
        res["value"] = round(d["gbs"], 2)
        res["ms_per_step"] = d["ms"] * CALLS_PER_STEP
        res["steps"] = d["calls"] // CALLS_PER_STEP
        res["config"]["calls_per_step"] = CALLS_PER_STEP
        tr = traffic.get("decode_m1_4096x14336")
        res["roofline"] = {"bound": "hbm", "achieved": round(d["gbs"], 2), "peak": HBM_PEAK_GBS,
                           "unit": "GB/s", "frac": round(d["gbs"] / HBM_PEAK_GBS, 4),
                           "traffic": tr, "algorithmic_bytes": dec_bytes,
                           "rotating_copies": d["copies"], "us_per_call": round(d["ms"] * 1e3, 3),
                           "eager_us_per_call": round(d["eager_ms"] * 1e3, 2)}
        if "read_stream" in out:
            r = out["read_stream"]
            res["roofline"]["measured_read_stream_gbs"] = round(r["gbs"], 1)
            res["roofline"]["frac_of_read_stream"] = round(d["gbs"] / r["gbs"], 4)
        if "decode_rows" in out:
            res["decode_rows_4096x14336"] = {
                f"M={m}": {"us_per_call": round(v["us"], 3), "gbs": round(v["gbs"], 1)}
                for m, v in out["decode_rows"].items()}
    if cpu:
        res["cpu_baseline"] = {k: (round(v, 4) if isinstance(v, float) else v) for k, v in cpu.items()}
    if "config1" in out:
        c = out["config1"]
        row = {"us_per_call": round(c["us"], 3), "gbs": round(c["gbs"], 1),
               "hbm_frac": round(c["gbs"] / HBM_PEAK_GBS, 4), "eager_us_per_call": round(c["eager_us"], 2),
               "algorithmic_bytes": c["bytes"]}
        if "cpu_us" in c:
            row["cpu_us_per_call"] = round(c["cpu_us"], 1)
            row["cpu_gbs"] = round(c["bytes"] / (c["cpu_us"] * 1e-6) / 1e9, 3)
            row["cpu"] = f"oracle f32 loop, OpenMP over {cpu['cores']} threads, {cpu['cpu_model']}, {c['cpu_calls']} calls"
            row["gpu_over_cpu"] = round(c["cpu_us"] / c["us"], 1)
        res["config1_decode_4096x4096_f32_scales"] = row
    if "prefill" in out:
        p = out["prefill"]
        res["prefill_m2048"] = {"tflops": round(p["tflops"], 2), "ms_per_call": round(p["ms"], 4),
                                "eager_ms_per_call": round(p["eager_ms"], 4),
                                "roofline": {"bound": "mfma", "achieved": round(p["tflops"], 2),
                                             "peak": FP16_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                                             "frac": round(p["tflops"] / FP16_MFMA_PEAK_TFLOPS, 4),
                                             "traffic": traffic.get("prefill_m2048_4096x14336")},
                                "dtype": "f16 in, fp32 accumulate, f16 out", "calls": p["calls"],
                                "rotating_copies": p["copies"]}
        if "dense_tflops" in p:
            res["prefill_m2048"]["dense_fp16_library_gemm_tflops"] = round(p["dense_tflops"], 2)
    if "gate_up_silu" in out:
        res["gate_up_silu_4096x2x14336"] = {
            f"M={m}": {"fused_us": round(v["fused_us"], 2), "unfused_us": round(v["unfused_us"], 2),
                       "speedup": round(v["unfused_us"] / v["fused_us"], 2)}
            for m, v in out["gate_up_silu"].items()}
    if "prefill_f32_rows" in out:
        res["prefill_f32_4096x14336"] = {
            f"M={m}": {"us_per_call": round(v["us"], 2), "tflops": round(v["tflops"], 1),
                       "frac_of_fp32_peak": round(v["tflops"] / FP32_PEAK_TFLOPS, 3),
                       "frac_of_fp16_mfma_peak": round(v["tflops"] / FP16_MFMA_PEAK_TFLOPS, 4)}
            for m, v in out["prefill_f32_rows"].items()}
        res["prefill_f32_4096x14336"]["dtype"] = "f32 in (split f16 hi + lo), fp32 accumulate, f32 out"
    if "prefill_rows" in out:
        res["prefill_rows_4096x14336"] = {
            f"M={m}": {"us_per_call": round(v["us"], 2), "tflops": round(v["tflops"], 1)}
            for m, v in out["prefill_rows"].items()}
    if "dequant" in out:
        q = out["dequant"]
        res["dequant_k14336_n4096_g64"] = {
            "gbs": round(q["gbs"], 2), "us_per_call": round(q["ms"] * 1e3, 2),
            "roofline": {"bound": "hbm", "achieved": round(q["gbs"], 2), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(q["gbs"] / HBM_PEAK_GBS, 4),
                         "traffic": traffic.get("dequant_14336x4096_g64")},
            "calls": q["calls"]}
    print(json.dumps(res))


if __name__ == "__main__":
    main()
