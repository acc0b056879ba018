#!/usr/bin/env python3
"""Benchmark of the MI355X W8A8 FP8 linear path (one JSON line on stdout).

Workload: the M = 1 decode GEMV over every
Qwen3-4B FP8 linear shape -- fused QKV 6144x2560, o_proj 2560x4096, fused
gate_up 19456x2560, down_proj 2560x9728 -- each with dynamic 1x128-group
activation quantization, 128x128 block-scaled E4M3 weights, fp32
accumulation and bf16 output. One step is one pass over the four shapes
(one decoder layer's FP8 linears). Inputs are synthetic: the seeded
splitmix64 + Box-Muller generator of the parity tests, run on the host
(W ~ N(0, 0.02) in bf16, quantized per 128x128 block by the library;
x ~ N(0, 1) in bf16), every input checked against its committed FNV-1a
digest ("input_digests").
Every shape's weights are rotated over enough distinct copies (>= 640 MB)
that the 256 MB Infinity Cache cannot hold them between launches.

value = algorithmic bytes per step / wall time per step (GB/s), timed over
--steps steps (rounded up to whole graphs of 50 steps) replayed from a HIP
graph and bracketed by device synchronizations. Algorithmic bytes of one
FP8 linear = N*K + ceil(N/128)*(K/128)*4 + M*K*2 + M*N*2.

"roofline" covers the dominant kernel (the fused M = 1 weight-streaming
kernel, the only kernel of the step): achieved = algorithmic bytes of the
timed steps / the time between HIP events recorded on the replay stream
around the timed graph replays.
"detail" adds per-shape figures, the bf16 lm_head, the batched-decode M
sweep (configs[2], per call graph-replayed over rotated weights, as the
M = 1 line) and the prefill GEMM at M = 512 and 4096 (configs[3], quant +
GEMM per call, graph-replayed the same way) in TFLOP/s against the 5.0
PFLOP/s dense FP8 peak.
"cpu_baseline" times the CPU restatement of the same arithmetic
(oracle/heph_oracle.c: quantize, dequantize, f32-accumulated matmul) on the
host's cores over a bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
FP8_PEAK_TFLOPS = 5000.0       # MI355X dense FP8 MFMA
ROTATE_BYTES = 640 << 20       # > 2x the 256 MB Infinity Cache
GRAPH_STEPS = 50               # steps captured per HIP graph

SHAPES = [("qkv", 6144, 2560), ("o_proj", 2560, 4096), ("gate_up", 19456, 2560),
          ("down", 2560, 9728)]
Q_PROJ = ("q_proj", 4096, 2560)
LM_HEAD = ("lm_head", 151936, 2560)


TRAFFIC_PROFILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                               "fp8_gemv_m1_pmc_traffic.md")
PREFILL_TRAFFIC_PROFILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                                       "fp8_gemm_m4096_pmc_traffic.md")


def profiled_traffic(path=TRAFFIC_PROFILE):
    """HBM bytes per step measured by the committed rocprofv3 PMC summary
    (FETCH_SIZE + WRITE_SIZE, calibrated by a copy of known size), or None."""
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_step:"):
                    return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


BENCH_LIB = os.path.join(os.path.dirname(os.path.abspath(__file__)), "hephaestus_amd",
                         "libhephbench.so")

# Seeds of the synthetic inputs (hephaestus_amd/bench_csrc/synth.cpp, the
# parity tests' splitmix64 + Box-Muller stream). Weights: W ~ N(0, 0.02)
# rounded to bf16 (the checkpoint dtype FP8 staging starts from) and
# quantized per 128 x 128 block by the library; activations: x ~ N(0, 1) in
# bf16, with ~0.1 % of entries x 50 where a configuration asks for outliers.
CONFIG0_SEED = 0                 # configs[0]'s activation row
WEIGHT_SEEDS = {"qkv": 100, "o_proj": 101, "gate_up": 102, "down": 103, "q_proj": 7,
                "lm_head": 9}

# FNV-1a 64 digests of the inputs as generated here and on the GPU box:
# <shape>_w_bf16 the generated weights, <shape>_w_e4m3 / <shape>_scale_inv the
# library's quantization of them copied back from the GPU, x_* the
# activation rows (x_m1_k<K>: the M = 1 rows of seed K). tests/test_bench_synth.py
# derives every one from the generator and the CPU quantizer.
BENCH_DIGESTS = {
    "qkv_w_bf16": "612137bbc3d5d4b6", "qkv_w_e4m3": "bfc7373ef4d6d4a3",
    "qkv_scale_inv": "b4b83f5d901d6e30",
    "o_proj_w_bf16": "adea71fe3c873096", "o_proj_w_e4m3": "baa6e6e5d986a82e",
    "o_proj_scale_inv": "f23d23453abccea5",
    "gate_up_w_bf16": "f06f48183227526e", "gate_up_w_e4m3": "dcb1ea786f46ec8f",
    "gate_up_scale_inv": "df2bb0da8c37348e",
    "down_w_bf16": "9201ededf4bfeab4", "down_w_e4m3": "a2c565dce55f9db7",
    "down_scale_inv": "5be0ebc17ef0c8cf",
    "q_proj_w_bf16": "d0076a63d0e81feb", "q_proj_w_e4m3": "746abfc13619fe61",
    "q_proj_scale_inv": "981e450e75ad742c",
    "lm_head_w_bf16": "3fd6190e415a50eb",
    "x_config0": "64959a856e22d0ff",
    "x_m1_k2560": "2183ab0aabdb581f", "x_m1_k4096": "061f45ac35038d6c",
    "x_m1_k9728": "0e151c44c17df616",
}

_SYNTH = None
INPUT_CHECKS = {}                # digest name -> matched


def synth():
    """libhephbench.so's generator and digest entry points (ctypes)."""
    global _SYNTH
    if _SYNTH is None:
        import ctypes
        lib = ctypes.CDLL(BENCH_LIB)
        u64, sz, f32, f64, vp = (ctypes.c_uint64, ctypes.c_size_t, ctypes.c_float,
                                 ctypes.c_double, ctypes.c_void_p)
        lib.heph_bench_gen_normal.argtypes = [u64, u64, sz, f32, f32, vp]
        lib.heph_bench_gen_normal.restype = None
        lib.heph_bench_gen_normal_bf16.argtypes = [u64, u64, sz, f32, f32, vp]
        lib.heph_bench_gen_normal_bf16.restype = None
        lib.heph_bench_gen_act_bf16.argtypes = [u64, sz, f64, f32, vp]
        lib.heph_bench_gen_act_bf16.restype = None
        lib.heph_bench_fnv1a64.argtypes = [vp, sz]
        lib.heph_bench_fnv1a64.restype = u64
        _SYNTH = lib
    return _SYNTH


def fnv1a64(a) -> str:
    """Digest of a contiguous numpy array's bytes."""
    import numpy as np
    a = np.ascontiguousarray(a)
    return "%016x" % synth().heph_bench_fnv1a64(a.ctypes.data, a.nbytes)


def check_digest(name, a):
    """Records whether array a matches the committed digest `name`."""
    want = BENCH_DIGESTS.get(name)
    if want is None:
        return
    ok = fnv1a64(a) == want
    INPUT_CHECKS[name] = ok
    if not ok:
        print(f"bench: input {name} does not match its committed digest", file=sys.stderr,
              flush=True)


def host_normal_bf16(seed, n, mean, std):
    import numpy as np
    out = np.empty(n, np.uint16)
    synth().heph_bench_gen_normal_bf16(seed, 0, n, mean, std, out.ctypes.data)
    return out


def host_normal_f32(seed, n, mean, std):
    import numpy as np
    out = np.empty(n, np.float32)
    synth().heph_bench_gen_normal(seed, 0, n, mean, std, out.ctypes.data)
    return out


def bf16_to_device(bits, shape):
    """uint16 bf16 bit patterns (host) -> bf16 tensor on cuda:0."""
    import torch
    return torch.from_numpy(bits.view("int16")).view(torch.bfloat16).reshape(shape).to("cuda")


def achievable_read(sizes, timer_graph_calls=20):
    """The plain-read denominator: graph-replayed time of a streaming read
    (hephaestus_amd/bench_csrc/hbm_read.hip) of each size in bytes, every
    call on the next window of a 1 GiB buffer so that the windows rotate
    past the 256 MB Infinity Cache as the GEMV's weight copies do; the best
    of three grid sizes. Returns {bytes: {"us", "GBs", "blocks"}}."""
    import ctypes
    import torch
    lib = ctypes.CDLL(BENCH_LIB)
    lib.heph_bench_read.restype = ctypes.c_int
    lib.heph_bench_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int,
                                    ctypes.c_void_p, ctypes.c_void_p]
    pool = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
    pool.fill_(1)
    sink = torch.empty(1 << 16, dtype=torch.int32, device="cuda")
    out = {}
    for size in sizes:
        size = (size + 4095) // 4096 * 4096
        best = None
        for blocks in (1024, 2048, 4096):
            slots = max(1, (1 << 30) // size)
            it = [0]

            def run(size=size, blocks=blocks, slots=slots, it=it):
                off = (it[0] % slots) * size
                it[0] += 1
                st = lib.heph_bench_read(pool.data_ptr() + off, size, blocks, sink.data_ptr(),
                                         torch.cuda.current_stream().cuda_stream)
                if st:
                    raise RuntimeError(f"heph_bench_read failed: {st}")
            run()
            ms = graph_call_ms(run, timer_graph_calls if size < (256 << 20) else 4)
            if best is None or ms < best[0]:
                best = (ms, blocks)
        ms, blocks = best
        out[size] = {"us": round(ms * 1e3, 3), "GBs": round(size / (ms * 1e-3) / 1e9, 1),
                     "blocks": blocks}
    del pool
    return out


def achievable_mfma(blocks=1024, iters=16384):
    """The MFMA denominator: FP8 TFLOP/s of a loop of independent
    v_mfma_f32_16x16x128_f8f6f4 on pseudo-random E4M3 register operands
    (four sets, cycled, so the multipliers switch as on real data) with no
    memory traffic (hephaestus_amd/bench_csrc/hbm_read.hip), 4 waves per
    workgroup, after one untimed launch; HIP events over three launches."""
    import ctypes
    import torch
    lib = ctypes.CDLL(BENCH_LIB)
    lib.heph_bench_mfma.restype = ctypes.c_int
    lib.heph_bench_mfma.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    sink = torch.empty(blocks * 256, dtype=torch.float32, device="cuda")

    def run():
        st = lib.heph_bench_mfma(blocks, iters, sink.data_ptr(),
                                 torch.cuda.current_stream().cuda_stream)
        if st:
            raise RuntimeError(f"heph_bench_mfma failed: {st}")
    run()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(3):
        run()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / 3
    flops = blocks * 4.0 * iters * 8 * 65536
    tf = flops / (ms * 1e-3) / 1e12
    return {"TFLOPs": round(tf, 1), "frac_of_peak": round(tf / FP8_PEAK_TFLOPS, 4),
            "ms_per_launch": round(ms, 3),
            "method": f"{blocks} workgroups x 4 waves x {iters} rounds of 8 independent "
                      "16x16x128 FP8 MFMAs, pseudo-random register operands cycled over 4 "
                      "sets, HIP events over 3 launches"}


def vendor_fp8_gemm(M=4096, calls=10):
    """hipBLASLt's FP8 GEMM through torch._scaled_mm on the configs[3] shapes
    at M rows (4096 or 512): E4M3 operands with one fp32 scale per tensor (the vendor
    library has no 128x128 block-scale mode), bf16 out, weights rotated past
    the Infinity Cache as for this library's GEMM; per call (HIP events
    around `calls` calls after ~20 ms of the same calls). A comparison, not
    a parity check."""
    import torch
    out = {}
    if not hasattr(torch, "_scaled_mm"):
        return {"error": "torch._scaled_mm unavailable"}
    one = torch.ones((), dtype=torch.float32, device="cuda")
    tot_fl, tot_us = 0.0, 0.0
    for i, (name, N, K) in enumerate(SHAPES):
        a = act(M, K, seed=M + 7).to(torch.float8_e4m3fn)
        copies = max(1, math.ceil(ROTATE_BYTES / (N * K)))
        w0 = torch.from_numpy(host_normal_f32(300 + i, N * K, 0.0, 0.5)).reshape(N, K)
        w0 = w0.to("cuda").to(torch.float8_e4m3fn)
        ws = [w0] + [w0.clone() for _ in range(copies - 1)]
        it = [0]

        def run(ws=ws, it=it, a=a):
            w = ws[it[0] % len(ws)]
            it[0] += 1
            return torch._scaled_mm(a, w.t(), scale_a=one, scale_b=one, out_dtype=torch.bfloat16)
        try:
            run()
        except Exception as e:          # no FP8 GEMM for this build / device
            return {"error": f"torch._scaled_mm failed: {type(e).__name__}: {e}"[:200]}
        t_end = time.perf_counter() + 0.02
        while time.perf_counter() < t_end:
            for _ in range(4):
                run()
            torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(calls):
            run()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / calls
        fl = 2.0 * M * N * K
        out[name] = {"us": round(us, 2), "TFLOPs": round(fl / (us * 1e-6) / 1e12, 1)}
        tot_fl += fl
        tot_us += us
        del ws
    out["all"] = {"us": round(tot_us, 2), "TFLOPs": round(tot_fl / (tot_us * 1e-6) / 1e12, 1)}
    return out


def fp8_bytes(M, N, K):
    return N * K + (-(-N // 128)) * (K // 128) * 4 + M * K * 2 + M * N * 2


def bf16_bytes(M, N, K, out_bytes=4):
    return 2 * N * K + 2 * M * K + out_bytes * M * N


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--quick", action="store_true", help="skip the detail sweeps")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--prefill-pass", action="store_true",
                    help="only run the configs[3] M = 4096 prefill launches eagerly (per "
                         "shape 100 + --steps GEMM launches on quantized activations, then "
                         "--steps quantizer launches; for rocprofv3 traces and counters); "
                         "prints no JSON")
    ap.add_argument("--prefill-m", type=int, default=4096,
                    help="rows of the --prefill-pass launches (configs[3]: 512 or 4096)")
    ap.add_argument("--decode-pass", action="store_true",
                    help="only run configs[4] decode steps eagerly (random-init Qwen3-4B, "
                         "4096 cached tokens; for rocprofv3 traces); prints no JSON")
    ap.add_argument("--pmc-pass", action="store_true",
                    help="only run the M = 1, 16 and 32 launches (2 eager calls, then a "
                         "HIP graph of --steps calls replayed 4 times, per shape) plus a 256 "
                         "MiB device copy (for rocprofv3 --pmc traffic counts and kernel "
                         "traces); prints no JSON")
    ap.add_argument("--pmc-m", default="1,16,32",
                    help="comma-separated row counts of the --pmc-pass launches")
    return ap.parse_args()


def prefill_pass(steps, M=4096):
    """configs[3] at M rows (4096 or 512), per shape: the activations quantized once,
    then the GEMM alone (SKIP_QUANT, as the bench's kernel-only prefill
    figure) eagerly over the rotated weight copies (weights come from HBM,
    not the Infinity Cache), 100 launches before the `steps` counted ones so
    that every shape runs at the clock sustained under FP8 MFMA load; then
    `steps` launches of the activation quantizer alone."""
    import torch
    from hephaestus_amd import kernels as HK
    torch.cuda.set_device(0)
    for i, (name, N, K) in enumerate(SHAPES):
        lin = Linear(name, N, K, M, seed=WEIGHT_SEEDS[name])
        x = act(M, K, seed=M + 1, outliers=True)
        c = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
        HK.quantize_act_rows_fp8(lin.q_ws, lin.s_ws, x, M, K)
        for _ in range(100 + steps):
            w, s = lin.next()
            HK.linear_fp8(c, None, w, s, lin.q_ws, lin.s_ws, M, N, K, do_quantize=False)
        torch.cuda.synchronize()
        kern = HK.last_kernel()
        for _ in range(steps):
            HK.quantize_act_rows_fp8(lin.q_ws, lin.s_ws, x, M, K)
        torch.cuda.synchronize()
        print(f"prefill-pass {name} M={M} N={N} K={K} kernel={kern}: 1 quantizer launch, "
              f"{100 + steps} GEMM launches (the last {steps} are the measured ones), "
              f"{steps} quantizer launches", flush=True)
        del lin
    a = torch.ones(256 << 20, dtype=torch.uint8, device="cuda")
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    print("prefill-pass copy 268435456 bytes x3", flush=True)


def decode_pass(steps):
    """`steps` eager decode steps at position 4096 after two
    warm-up steps, each step ending in a device synchronization."""
    import torch
    from hephaestus_amd import decode as DEC
    from hephaestus_amd.loader import Qwen3Config
    torch.cuda.set_device(0)
    cfg = Qwen3Config()
    w = DEC.random_init(cfg, seed=4)
    kv = DEC.KVCache(cfg, 4097)
    kv.fill_synthetic(4096, seed=5)
    dec = DEC.Qwen3Decoder(w, kv)
    for i in range(2 + steps):
        dec.step(12345, 4096)
        torch.cuda.synchronize()
    print(f"decode-pass steps={2 + steps} (the last {steps} are the measured ones) "
          f"argmax={int(dec.next_token.item())}", flush=True)


def pmc_pass(steps, Ms=(1, 16, 32)):
    """Launches of every shape at M = 1, then the configs[2] batched decode
    sizes (by default M = 16 and 32; bf16 rows, default route), and one
    plain copy of known size.

    Under rocprofv3 --pmc FETCH_SIZE (or WRITE_SIZE) the copy kernel's count
    calibrates the counter: bytes = count * (copy bytes / copy count)."""
    import torch
    from hephaestus_amd import kernels as HK
    torch.cuda.set_device(0)
    lins = [Linear(n, N, K, 32, seed=WEIGHT_SEEDS[n]) for i, (n, N, K) in enumerate(SHAPES)]
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    for M in Ms:
        for lin in lins:
            x = act(M, lin.K, seed=lin.K + M)
            c = torch.empty(M, lin.N, dtype=torch.bfloat16, device="cuda")

            def call(lin=lin, x=x, c=c, M=M):
                w, s = lin.next()
                HK.linear_fp8(c, x, w, s, lin.q_ws, lin.s_ws, M, lin.N, lin.K)
            # two eager calls, then `steps` calls captured in a HIP graph:
            # back to back on the GPU, as in bench.py's timed region
            with torch.cuda.stream(stream):
                call()
                call()
                torch.cuda.synchronize()
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph, stream=stream):
                    for _ in range(steps):
                        call()
            # four replays back to back: the first ones bring the shader
            # clock up from the idle gaps of the set-up; read the last
            for _ in range(4):
                graph.replay()
            torch.cuda.synchronize()
            print(f"pmc-pass M={M} {lin.name} N={lin.N} K={lin.K} kernel={HK.last_kernel()} "
                  f"calls=2 eager + 4 x {steps} graph-replayed (the last {steps} are the "
                  f"measured ones)", flush=True)
    a = torch.ones(256 << 20, dtype=torch.uint8, device="cuda")
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    print("pmc-pass copy 268435456 bytes x3", flush=True)


class Linear:
    """One FP8 linear with rotated weight copies and its own workspace."""

    def __init__(self, name, N, K, M_max, seed, rotate=True):
        import torch
        from hephaestus_amd import kernels as HK
        from hephaestus_amd.weights import quantize_weight_fp8
        self.name, self.N, self.K = name, N, K
        wh = host_normal_bf16(seed, N * K, 0.0, 0.02)
        w = bf16_to_device(wh, (N, K))
        q, s = quantize_weight_fp8(w)
        del w
        if seed == WEIGHT_SEEDS.get(name):
            check_digest(f"{name}_w_bf16", wh)
            check_digest(f"{name}_w_e4m3", q.cpu().numpy())
            check_digest(f"{name}_scale_inv", s.cpu().numpy())
        del wh
        copies = max(1, math.ceil(ROTATE_BYTES / (N * K))) if rotate else 1
        self.w = [q] + [q.clone() for _ in range(copies - 1)]
        self.s = [s] + [s.clone() for _ in range(copies - 1)]
        self.q_ws, self.s_ws = HK.workspace(M_max, K, n=N)
        self.i = 0

    def next(self):
        w, s = self.w[self.i], self.s[self.i]
        self.i = (self.i + 1) % len(self.w)
        return w, s


def act(M, K, seed, outliers=False, digest=None):
    """M x K bf16 activations of `seed` on cuda:0 (outliers: ~0.1 % x 50);
    checked against the committed digest `digest` when given."""
    import numpy as np
    xh = np.empty(M * K, np.uint16)
    synth().heph_bench_gen_act_bf16(seed, M * K, 1e-3 if outliers else 0.0, 50.0,
                                    xh.ctypes.data)
    if digest:
        check_digest(digest, xh)
    return bf16_to_device(xh, (M, K))


def time_calls(fn, n, timer):
    """Run fn() n times with kernel-boundary timing; returns summed ms."""
    import torch
    timer.reset()
    for _ in range(n):
        timer.arm()
        fn()
    torch.cuda.synchronize()
    return sum(timer.durations_ms())


def graph_call_ms(fn, n):
    """Capture n calls of fn() (each rotating its weights) in a HIP graph,
    replay it once, then return the wall time per call of three timed
    replays (ms): the launches' host cost is off the GPU's critical path, as
    in the timed region of the M = 1 line."""
    import torch
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        fn()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for _ in range(n):
                fn()
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(3):
        graph.replay()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / (3 * n)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(the FP8 linear path has no multi-GPU mode here)", file=sys.stderr)
        sys.exit(2)
    if args.pmc_pass:
        pmc_pass(max(1, min(args.steps, 20)), tuple(int(m) for m in args.pmc_m.split(",")))
        return
    if args.prefill_pass:
        prefill_pass(max(1, min(args.steps, 20)), args.prefill_m)
        return
    if args.decode_pass:
        decode_pass(max(1, min(args.steps, 20)))
        return
    import torch
    from hephaestus_amd import kernels as HK
    from hephaestus_amd.timing import KernelTimer

    torch.cuda.set_device(0)
    props = torch.cuda.get_device_properties(0)
    lins = [Linear(n, N, K, 32, seed=WEIGHT_SEEDS[n]) for i, (n, N, K) in enumerate(SHAPES)]
    xs = {K: act(1, K, seed=K, digest=f"x_m1_k{K}") for K in {K for _, _, K in SHAPES}}
    outs = [torch.empty(1, N, dtype=torch.bfloat16, device="cuda") for _, N, _ in SHAPES]

    def step(timer=None):
        for lin, c in zip(lins, outs):
            w, s = lin.next()
            if timer is not None:
                timer.arm()
            HK.linear_fp8(c, xs[lin.K], w, s, lin.q_ws, lin.s_ws, 1, lin.N, lin.K)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # The timed region replays a HIP graph holding GRAPH_STEPS steps (each
    # captured step reads its own rotation of weight copies), so host-side
    # launch cost is not on the GPU's critical path.
    graph_steps = min(GRAPH_STEPS, args.steps)
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        step()                           # first use on the capture stream
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=stream):
            for _ in range(graph_steps):
                step()
    torch.cuda.synchronize()
    replays = -(-args.steps // graph_steps)
    graph.replay()
    torch.cuda.synchronize()
    # HIP events on the stream the replays launch on bracket the timed region:
    # back-to-back launches of the GEMV kernel only, so their time per step is
    # the kernels' own (the roofline's `achieved`); the wall clock gives `value`
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record()
    for _ in range(replays):
        graph.replay()
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    steps_timed = replays * graph_steps
    region_ms = ev0.elapsed_time(ev1)

    # Per-launch durations: the same launches issued eagerly, each stamped at
    # its own begin and end (hipExtLaunchKernel events cannot sit inside a
    # graph); each starts on an idle GPU, so these read ~5-15 % above the
    # graph-replayed kernels.
    timer = KernelTimer(len(lins) * args.steps)
    for _ in range(args.steps):
        step(timer)
    torch.cuda.synchronize()
    kernel_names = [HK.last_kernel()]
    durs = timer.durations_ms()
    timer.close()

    step_bytes = sum(fp8_bytes(1, N, K) for _, N, K in SHAPES)
    ms_per_step = wall * 1e3 / steps_timed
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    per_shape = {}
    for j, (name, N, K) in enumerate(SHAPES):
        d = durs[j::len(SHAPES)]
        avg_us = 1e3 * sum(d) / len(d)
        per_shape[name] = {"N": N, "K": K, "eager_kernel_us": round(avg_us, 3),
                           "eager_GBs": round(fp8_bytes(1, N, K) / (avg_us * 1e-6) / 1e9, 1),
                           "copies": len(lins[j].w)}
    kern_ms = sum(durs)
    achieved = step_bytes * steps_timed / (region_ms * 1e-3) / 1e9

    # each shape alone, graph-replayed per call (as the configs[2] sweep and
    # the plain read below), against the plain read of its weight bytes
    reads = achievable_read([N * K for _, N, K in SHAPES] + [1 << 30])
    for j, (name, N, K) in enumerate(SHAPES):
        lin, c = lins[j], outs[j]

        def run_1(lin=lin, c=c):
            w, s = lin.next()
            HK.linear_fp8(c, xs[lin.K], w, s, lin.q_ws, lin.s_ws, 1, lin.N, lin.K)
        ms = graph_call_ms(run_1, 20)
        rd = reads[(N * K + 4095) // 4096 * 4096]
        gbs = fp8_bytes(1, N, K) / (ms * 1e-3) / 1e9
        per_shape[name].update({"graph_us": round(ms * 1e3, 3), "graph_GBs": round(gbs, 1),
                                "frac_of_8TBs": round(gbs / HBM_PEAK_GBS, 4),
                                "plain_read_us": rd["us"], "plain_read_GBs": rd["GBs"],
                                "frac_of_plain_read": round(rd["us"] / (ms * 1e3), 4)})
    detail = {"m1_shapes": per_shape,
              "timed_region_us_per_step_hip_events": round(1e3 * region_ms / steps_timed, 3),
              "eager_kernel_time_per_step_us": round(1e3 * kern_ms / args.steps, 3),
              "achievable_read": {"method": "graph-replayed plain streaming read of the same "
                                            "byte count over a rotating window of a 1 GiB "
                                            "buffer (libhephbench.so), best of 1024/2048/4096 "
                                            "workgroups",
                                  "sizes": {str(k): v for k, v in reads.items()},
                                  "read_1GiB_GBs": reads[1 << 30]["GBs"]}}
    if not args.quick:
        detail.update(detail_sweeps(lins))

    cpu = None if args.no_cpu else cpu_baseline(lins, xs, args.cpu_seconds)

    line = {
        "metric": "FP8 GEMV GB/s (% of HBM peak) at M=1; prefill FP8 GEMM TFLOP/s at M=4096",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps_timed,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8_e4m3 x fp8_e4m3 -> f32 acc -> bf16",
        "data": "synthetic (seeded splitmix64 + Box-Muller host generator, "
                "bench_csrc/synth.cpp; bf16 weights quantized per 128x128 block on "
                "the GPU; digests checked)",
        "config": {"workload": "configs[1]: M=1 FP8 GEMV over Qwen3-4B linears "
                               "(qkv 6144x2560, o 2560x4096, gate_up 19456x2560, "
                               "down 2560x9728), fused 1x128 act quant, bf16 out",
                   "M": 1, "step": "one pass over the 4 shapes", "device": props.name,
                   "arch": props.gcnArchName},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": profiled_traffic(),
                     "traffic_source": "rocprofv3 FETCH_SIZE + WRITE_SIZE per step, "
                                       "profiles/fp8_gemv_m1_pmc_traffic.md",
                     "kernel": kernel_names[-1],
                     "bytes_per_step": step_bytes},
        "cpu_baseline": cpu,
        "input_digests": {"checked": len(INPUT_CHECKS),
                          "ok": bool(INPUT_CHECKS) and all(INPUT_CHECKS.values()),
                          "mismatched": sorted(k for k, v in INPUT_CHECKS.items() if not v)},
        "detail": detail,
    }
    pk = detail.get("prefill_m4096_kernel")
    path_tf = detail.get("prefill_m4096_TFLOPs")
    if pk and path_tf:
        # headline: the path (activation quantizer + GEMM, graph-replayed per
        # call), the work BASELINE's metric counts; the GEMM alone beside it
        line["prefill_roofline"] = {
            "bound": "mfma", "achieved": path_tf, "peak": FP8_PEAK_TFLOPS,
            "unit": "TFLOP/s", "frac": round(path_tf / FP8_PEAK_TFLOPS, 4),
            "what": "quantizer + GEMM per call",
            "kernel_only_TFLOPs": pk["TFLOPs"],
            "kernel_only_frac": round(pk["TFLOPs"] / FP8_PEAK_TFLOPS, 4),
            "traffic": profiled_traffic(PREFILL_TRAFFIC_PROFILE),
            "traffic_source": "rocprofv3 FETCH_SIZE + WRITE_SIZE per 4-shape step, "
                              "profiles/fp8_gemm_m4096_pmc_traffic.md",
            "kernel": ", ".join(sorted(set(pk["kernels"]))),
            "flops_per_step": pk["flops_per_step"],
            "workload": "configs[3] M=4096 over the 4 config-1 shapes: per call the "
                        "activation quantizer then the GEMM (kernel_only: the GEMM "
                        "alone on activations quantized beforehand), weights rotated "
                        "past the Infinity Cache"}
        am = detail.get("achievable_mfma")
        if am and am.get("TFLOPs"):
            line["prefill_roofline"]["kernel_only_frac_of_achievable_mfma"] = round(
                pk["TFLOPs"] / am["TFLOPs"], 4)
        vg = (detail.get("vendor_fp8_gemm_m4096") or {}).get("all")
        if vg:
            line["prefill_roofline"]["kernel_only_vs_hipblaslt_per_tensor_fp8"] = round(
                pk["TFLOPs"] / vg["TFLOPs"], 3)
    print(json.dumps(line))


def detail_sweeps(lins):
    import torch
    from hephaestus_amd import kernels as HK
    from hephaestus_amd.timing import KernelTimer
    out = {}
    timer = KernelTimer(64)

    # config 0: q_proj at M = 1
    qp = Linear(*Q_PROJ, 1, seed=WEIGHT_SEEDS["q_proj"])
    x = act(1, qp.K, seed=CONFIG0_SEED, digest="x_config0")
    c = torch.empty(1, qp.N, dtype=torch.bfloat16, device="cuda")

    def run_q():
        w, s = qp.next()
        HK.linear_fp8(c, x, w, s, qp.q_ws, qp.s_ws, 1, qp.N, qp.K)
    run_q()
    ms = time_calls(run_q, 50, timer) / 50
    out["config0_q_proj_m1"] = {"kernel_us": round(ms * 1e3, 3),
                                "GBs": round(fp8_bytes(1, qp.N, qp.K) / (ms * 1e-3) / 1e9, 1)}
    del qp

    # bf16 lm_head at M = 1 (f32 logits), two weight copies (> 1.5 GB)
    name, N, K = LM_HEAD
    wh = host_normal_bf16(WEIGHT_SEEDS["lm_head"], N * K, 0.0, 0.02)
    check_digest("lm_head_w_bf16", wh)
    lw = [bf16_to_device(wh, (N, K))]
    lw.append(lw[0].clone())
    del wh
    xl = act(1, K, seed=10)
    logits = torch.empty(1, N, dtype=torch.float32, device="cuda")
    it = [0]

    def run_lm():
        HK.linear(logits, xl, lw[it[0] % 2], 1, N, K)
        it[0] += 1
    run_lm()
    ms = time_calls(run_lm, 20, timer) / 20
    out["lm_head_bf16_m1"] = {"kernel_us": round(ms * 1e3, 3),
                              "GBs": round(bf16_bytes(1, N, K) / (ms * 1e-3) / 1e9, 1),
                              "frac": round(bf16_bytes(1, N, K) / (ms * 1e-3) / 1e9
                                            / HBM_PEAK_GBS, 4)}
    del lw

    # batched decode M in {2..32}; time per call graph-replayed
    # (every kernel of the call: quantizer, main kernel, K-split reduction)
    small = {}
    for M in (2, 4, 8, 16, 32):
        row = {}
        for lin in lins:
            xm = act(M, lin.K, seed=M)
            cm = torch.empty(M, lin.N, dtype=torch.bfloat16, device="cuda")

            def run_m(lin=lin, xm=xm, cm=cm, M=M):
                w, s = lin.next()
                HK.linear_fp8(cm, xm, w, s, lin.q_ws, lin.s_ws, M, lin.N, lin.K)
            run_m()
            ms = graph_call_ms(run_m, 20)
            row[lin.name] = round(fp8_bytes(M, lin.N, lin.K) / (ms * 1e-3) / 1e9, 1)
        small[f"M={M}"] = row
    out["small_m_GBs"] = small

    # prefill GEMM, quant + GEMM (+ K-split reduction) path time
    # per call, graph-replayed over the rotated weight copies as the M = 1
    # and configs[2] lines (timed eagerly, M = 512 calls are bound by the
    # host's launch rate), TFLOP/s
    pre = {}
    for M in (512, 4096):
        row = {}
        for lin in lins:
            xm = act(M, lin.K, seed=M + 1, outliers=True)
            cm = torch.empty(M, lin.N, dtype=torch.bfloat16, device="cuda")
            q_ws, s_ws = HK.workspace(M, lin.K, n=lin.N)

            def run_p(lin=lin, xm=xm, cm=cm, M=M, q_ws=q_ws, s_ws=s_ws):
                w, s = lin.next()
                HK.linear_fp8(cm, xm, w, s, q_ws, s_ws, M, lin.N, lin.K)
            # ~20 ms of the same launches first: the shader clock settles
            # under sustained FP8 MFMA load, and a first shape timed from idle
            # would run at a boosted clock
            t_end = time.perf_counter() + 0.02
            while time.perf_counter() < t_end:
                for _ in range(8):
                    run_p()
                torch.cuda.synchronize()
            ms = graph_call_ms(run_p, 20)
            tf = 2.0 * M * lin.N * lin.K / (ms * 1e-3) / 1e12
            row[lin.name] = {"us": round(ms * 1e3, 2), "TFLOPs": round(tf, 1),
                             "frac": round(tf / FP8_PEAK_TFLOPS, 4)}
        pre[f"M={M}"] = row
    out["prefill"] = pre
    out["prefill_m4096_kernel"] = prefill_kernel_times(lins)
    out["achievable_mfma"] = achievable_mfma()
    out["vendor_fp8_gemm_m4096"] = vendor_fp8_gemm()
    out["vendor_fp8_gemm_m512"] = vendor_fp8_gemm(M=512, calls=20)
    out["prefill_producer_path"] = prefill_producer_path(lins)
    out["decode_step_config4"] = decode_step_timing()
    t4096 = sum(2.0 * 4096 * l.N * l.K for l in lins)
    us4096 = sum(v["us"] for v in pre["M=4096"].values())
    out["prefill_m4096_TFLOPs"] = round(t4096 / (us4096 * 1e-6) / 1e12, 1)
    out["prefill_m4096_frac"] = round(out["prefill_m4096_TFLOPs"] / FP8_PEAK_TFLOPS, 4)
    timer.close()
    return out


def prefill_kernel_times(lins, M=4096, calls=10):
    """configs[3] at M = 4096, the GEMM kernel alone: the activations are
    quantized once, then each call runs with SKIP_QUANT over the rotated
    weight copies; after ~20 ms of the same launches (the clock settles
    under sustained MFMA load), HIP events on the launch stream around
    `calls` back-to-back calls, as vendor_fp8_gemm times hipBLASLt (stamps
    around each launch leave gaps in which the clock recovers, and read up
    to ~15 % faster than the sustained rate)."""
    import torch
    from hephaestus_amd import kernels as HK
    per, names = {}, []
    for lin in lins:
        xm = act(M, lin.K, seed=M + 1, outliers=True)
        cm = torch.empty(M, lin.N, dtype=torch.bfloat16, device="cuda")
        q_ws, s_ws = HK.workspace(M, lin.K, n=lin.N)
        HK.quantize_act_rows_fp8(q_ws, s_ws, xm, M, lin.K)

        def run(lin=lin, cm=cm, q_ws=q_ws, s_ws=s_ws):
            w, s = lin.next()
            HK.linear_fp8(cm, None, w, s, q_ws, s_ws, M, lin.N, lin.K, do_quantize=False)
        t_end = time.perf_counter() + 0.02
        while time.perf_counter() < t_end:
            for _ in range(8):
                run()
            torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(calls):
            run()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / calls
        names.append(HK.last_kernel())
        tf = 2.0 * M * lin.N * lin.K / (ms * 1e-3) / 1e12
        per[lin.name] = {"kernel_us": round(ms * 1e3, 2), "TFLOPs": round(tf, 1),
                         "frac": round(tf / FP8_PEAK_TFLOPS, 4), "kernel": names[-1]}
    flops = sum(2.0 * M * l.N * l.K for l in lins)
    us = sum(v["kernel_us"] for v in per.values())
    return {"shapes": per, "kernels": names, "flops_per_step": flops,
            "kernel_us_per_step": round(us, 2),
            "TFLOPs": round(flops / (us * 1e-6) / 1e12, 1)}


def prefill_producer_path(lins, Ms=(512, 4096)):
    """configs[3] as a prefill layer feeds its linears: the op that produces
    each linear's input quantizes it (qkv and gate_up: RMSNorm of the hidden
    rows, heph_rmsnorm_quant_fp8; down: SwiGLU of the gate and up rows,
    heph_silu_mul_quant_fp8) and the GEMM runs with SKIP_QUANT, against the
    unfused producer + quantizer + GEMM; o_proj's input comes from prefill
    attention, outside this library, so it keeps quantizer + GEMM in both.
    Per call graph-replayed over rotated weights; us and TFLOP/s of the
    GEMM's work."""
    import torch
    from hephaestus_amd import decode as DEC
    from hephaestus_amd import kernels as HK
    out = {}
    for M in Ms:
        row = {}
        for lin in lins:
            N, K = lin.N, lin.K
            cm = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
            q_ws, s_ws = HK.workspace(M, K, n=N)
            if lin.name == "down":
                gate = act(M, K, seed=M + 2)
                upv = act(M, K, seed=M + 5)
                y = torch.empty(M, K, dtype=torch.bfloat16, device="cuda")

                def unfused(lin=lin, gate=gate, upv=upv, y=y, cm=cm, q_ws=q_ws, s_ws=s_ws, M=M, K=K, N=N):
                    w, s = lin.next()
                    DEC.silu_mul(y, gate, upv, M * K)            # elementwise over all rows
                    HK.linear_fp8(cm, y, w, s, q_ws, s_ws, M, N, K)

                def fused(lin=lin, gate=gate, upv=upv, cm=cm, q_ws=q_ws, s_ws=s_ws, M=M, K=K, N=N):
                    w, s = lin.next()
                    HK.silu_mul_quant_fp8(q_ws, s_ws, gate, upv, M, K)
                    HK.linear_fp8(cm, None, w, s, q_ws, s_ws, M, N, K, do_quantize=False)
            elif lin.name in ("qkv", "gate_up"):
                src = act(M, K, seed=M + 3)
                gam = bf16_to_device(host_normal_bf16(M + 6, K, 1.0, 0.1), (K,))
                y = torch.empty(M, K, dtype=torch.bfloat16, device="cuda")

                def unfused(lin=lin, src=src, gam=gam, y=y, cm=cm, q_ws=q_ws, s_ws=s_ws, M=M, K=K, N=N):
                    w, s = lin.next()
                    DEC.rmsnorm(y, src, gam)
                    HK.linear_fp8(cm, y, w, s, q_ws, s_ws, M, N, K)

                def fused(lin=lin, src=src, gam=gam, cm=cm, q_ws=q_ws, s_ws=s_ws, M=M, K=K, N=N):
                    w, s = lin.next()
                    HK.rmsnorm_quant_fp8(q_ws, s_ws, src, gam, M, K)
                    HK.linear_fp8(cm, None, w, s, q_ws, s_ws, M, N, K, do_quantize=False)
            else:
                src = act(M, K, seed=M + 4)

                def unfused(lin=lin, src=src, cm=cm, q_ws=q_ws, s_ws=s_ws, M=M, K=K, N=N):
                    w, s = lin.next()
                    HK.linear_fp8(cm, src, w, s, q_ws, s_ws, M, N, K)
                fused = unfused
            t_end = time.perf_counter() + 0.02
            while time.perf_counter() < t_end:
                for _ in range(8):
                    fused()
                torch.cuda.synchronize()
            ms_u = graph_call_ms(unfused, 20)
            ms_f = graph_call_ms(fused, 20)
            fl = 2.0 * M * N * K
            row[lin.name] = {"unfused_us": round(ms_u * 1e3, 2), "fused_us": round(ms_f * 1e3, 2),
                             "unfused_TFLOPs": round(fl / (ms_u * 1e-3) / 1e12, 1),
                             "fused_TFLOPs": round(fl / (ms_f * 1e-3) / 1e12, 1)}
        tot_u = sum(v["unfused_us"] for v in row.values())
        tot_f = sum(v["fused_us"] for v in row.values())
        fl = sum(2.0 * M * l.N * l.K for l in lins)
        row["all"] = {"unfused_us": round(tot_u, 2), "fused_us": round(tot_f, 2),
                      "fused_TFLOPs": round(fl / (tot_f * 1e-6) / 1e12, 1),
                      "unfused_TFLOPs": round(fl / (tot_u * 1e-6) / 1e12, 1)}
        out[f"M={M}"] = row
    return out


def decode_step_timing(steps=20):
    """one random-init Qwen3-4B W8A8 decode step at position 4096
    (36 layers, FP8 KV cache of 4096 synthetic tokens), replayed from a HIP
    graph; ms per token and the FP8 weight bytes streamed per ms."""
    import torch
    from hephaestus_amd import decode as DEC
    from hephaestus_amd.loader import Qwen3Config
    cfg = Qwen3Config()
    w = DEC.random_init(cfg, seed=4)
    kv = DEC.KVCache(cfg, 4097)
    kv.fill_synthetic(4096, seed=5)
    dec = DEC.Qwen3Decoder(w, kv)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        dec.step(12345, 4096)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            dec.step(12345, 4096)
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        graph.replay()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    wbytes = DEC.n_params_bytes(cfg)
    kv_bytes = cfg.n_layers * 4097 * cfg.n_kv_heads * cfg.head_dim * 2
    return {"ms_per_token": round(ms, 4), "tokens_per_s": round(1e3 / ms, 1),
            "fp8_weight_bytes": wbytes, "kv_bytes": kv_bytes,
            "GBs_weights_plus_kv": round((wbytes + kv_bytes) / (ms * 1e-3) / 1e9, 1),
            "argmax": int(dec.next_token.item())}


def cpu_threads():
    """Host threads for the CPU baseline: OMP_NUM_THREADS when set (the GPU
    boxes set it to the cores one GPU's share of the host holds), else every
    core this process may run on."""
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        return int(env)
    return len(os.sched_getaffinity(0))


def cpu_baseline(lins, xs, seconds):
    """The oracle's quantize + dequant-matmul (f32 accumulation) on the host
    cores over the same four shapes and the same weights: M = 1 (configs[1],
    GB/s, the bench's unit) for ~seconds, then the M = 512 prefill leg
    (configs[3], TFLOP/s) for about as long again."""
    import numpy as np
    import torch
    from oracle import oracle as O
    O.build()
    threads = cpu_threads()
    host = []
    for lin in lins:
        host.append((lin.w[0].cpu().numpy(), lin.s[0].cpu().numpy(),
                     xs[lin.K].view(torch.int16).cpu().numpy().view(np.uint16),
                     lin.N, lin.K))
    budget = seconds / len(host)
    tot_bytes, tot_s, reps = 0, 0.0, {}
    for qw, sw, x, N, K in host:
        O.quant_linear(x, qw, sw, nthreads=threads)       # warm
        n, t0 = 0, time.perf_counter()
        while True:
            O.quant_linear(x, qw, sw, nthreads=threads)
            n += 1
            el = time.perf_counter() - t0
            if el >= budget:
                break
        tot_bytes += n * fp8_bytes(1, N, K)
        tot_s += el
        reps[N * 100000 + K] = n
    # configs[3] M = 512 leg: one call per shape, repeated while the budget lasts
    M = 512
    flops, pre_s, pre_calls, t_end = 0.0, 0.0, 0, time.perf_counter() + seconds
    xm = {K: O.gen_act_bf16(M + 1, M, K, outlier_p=1e-3) for K in {h[4] for h in host}}
    while True:
        for qw, sw, _, N, K in host:
            t0 = time.perf_counter()
            O.quant_linear(xm[K], qw, sw, nthreads=threads)
            pre_s += time.perf_counter() - t0
            flops += 2.0 * M * N * K
            pre_calls += 1
        if time.perf_counter() >= t_end:
            break
    cpu_name = ""
    try:
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name"):
                cpu_name = ln.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": round(tot_bytes / tot_s / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "port",
            "nproc": os.cpu_count(), "affinity_cores": len(os.sched_getaffinity(0)),
            "omp_num_threads_env": os.environ.get("OMP_NUM_THREADS"),
            "prefill_m512": {"TFLOPs": round(flops / pre_s / 1e12, 4), "calls": pre_calls,
                             "seconds": round(pre_s, 2)},
            "sample": f"oracle quant + f32 dequant-matmul on {threads} threads: M=1 over the 4 "
                      f"config-1 shapes for ~{seconds:.0f} s ({sum(reps.values())} calls), then "
                      f"the configs[3] M=512 leg ({pre_calls} calls, {pre_s:.1f} s); "
                      f"CPU: {cpu_name}"}


if __name__ == "__main__":
    main()
