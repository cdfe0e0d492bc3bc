"""Benchmark of the FP8 hot path on one MI355X.

Workload (the DeepSeek-V3 projection): X[8192, 7168] bf16
~N(0,1) with 1% of entries x20, W[2048, 7168] bf16 ~N(0, 0.02).  One step = the
reference forward (src/kernels.py:740-752): 1x128 row-wise quantization of X,
128x128 block quantization of W, block-scaled FP8 GEMM Y = X W^T with bf16 output.
Inputs are resident in HBM and rotate over 3 copies (> 256 MB) so the quantizers
read HBM, not the 256 MB Infinity Cache.

Prints ONE JSON line.  value = 2*M*N*K / step time (TFLOP/s of the whole step);
"roofline" describes the dominant kernel (the GEMM) against dense FP8 MFMA peak;
"components" gives each kernel's time and roofline fraction; "cpu_baseline" times
the CPU oracle (torch-CPU restatement of the reference path) on a bounded sample.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "FP8 block GEMM TFLOPS + % MFMA peak; quantizer GB/s as % of HBM BW"
PEAK_FP8_TFLOPS = 5000.0     # MI355X dense FP8 MFMA
PEAK_HBM_GBPS = 8000.0       # MI355X HBM3E
M, N, K = 8192, 2048, 7168


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--only", choices=["step", "gemm", "scaled_mm", "quant_x", "quant_w", "quant_fwd", "moe_gateup", "moe_down", "bwd_pair",
                                      "dual_quant", "requant", "dgrad", "wgrad", "moe_dual", "moe_requant",
                                      "moe_wgrad", "moe_dgrad", "moe_layer", "moe_layer_fwd", "moe_route",
                                      "moe_gather", "moe_combine", "moe_combine_bwd", "indexer", "indexer_wgrad", "indexer_full", "copy", "mfma_ceiling",
                                      "traffic_ceiling", "config1", "config5"],
                   default=None,
                   help="run only one kernel in a loop (for profiler runs)")
    p.add_argument("--no-extra", action="store_true",
                   help="skip the config-3 (MoE), config-4 (backward) and config-5 (training) timings")
    return p.parse_args()


# Untimed steps run before the warmup steps of the step timing.  After any idle spell (50 ms
# is enough) the GPU comes back at a lower working clock and needs ~150 config-2 steps
# (~25 ms) to reach its steady rate: measured in blocks of 10 steps from a cold start,
# 174, 195, 182, 174, ... 156, 153, 151, 150 us per step.  A training loop runs at that
# steady rate; a timed region of a few ms right after the setup's idle spell would time the
# ramp instead.  The timed region is unchanged: exactly `steps` steps.
SETTLE_MS = 60.0


def settle(fn, ms=SETTLE_MS):
    """Run fn untimed until `ms` of wall time have passed; returns the number of calls."""
    import torch

    n, t0 = 0, time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < ms:
        for _ in range(10):
            fn(n)
            n += 1
        torch.cuda.synchronize()
    return n


def time_loop(fn, iters, warmup, settle_ms=0.0):
    import torch

    if settle_ms > 0:
        settle(fn, settle_ms)
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(iters):
        fn(i)
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / iters * 1e3  # us per call


_BUSY = []


def kernel_loop(fn, iters, warmup, settle_ms=30.0):
    """Device time per call of a component.  Copies of a 256 MiB buffer queued first keep
    the GPU busy (at its working clock) while the host enqueues the `iters` calls, so the
    events bracket back-to-back kernels and not the host's launch overhead (which the step
    timing above does include).  Untimed calls for `settle_ms` first bring the clock to its
    steady rate for this component."""
    import torch

    if settle_ms > 0:
        settle(fn, settle_ms)
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    # host time per call, to size the queued work that covers the enqueueing
    t0 = time.perf_counter()
    for i in range(3):
        fn(i)
    torch.cuda.synchronize()
    host_s = (time.perf_counter() - t0) / 3
    if not _BUSY:
        src = torch.ones(128 * 1024 * 1024, dtype=torch.bfloat16, device="cuda")
        _BUSY.extend([src, torch.empty_like(src)])
    src, dst = _BUSY
    # a 256 MiB copy takes ~90 us; twice the measured host time, since a profiler's
    # per-launch cost varies from call to call
    for _ in range(2 + int(2 * host_s * iters / 80e-6)):
        dst.copy_(src)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(iters):
        fn(i)
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / iters * 1e3  # us per call


def mfma_ceiling_setup(dev):
    """bench_ceiling.so (bench_ceiling.hip): the GEMM's inner MFMA + promotion-FMA mix with
    no memory traffic, on random e4m3 operand bytes (NaN codes excluded).  Returns
    (callable(promote, shape=16) -> None, FLOP per launch); shape 32 runs the same work as
    32 x 32 x 64 MFMAs."""
    import ctypes

    import torch

    path = os.path.join(ROOT, "bench_ceiling.so")
    if not os.path.exists(path):
        raise RuntimeError(f"{path} not found: build it with __graft_entry__.build()")
    lib = ctypes.CDLL(path)
    lib.bench_mfma_ceiling.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                       ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    blocks, iters = 256, 200
    g = torch.Generator(device=dev).manual_seed(7)
    codes = torch.randint(0, 256, (blocks * 512 * 48 * 4,), dtype=torch.uint8, device=dev, generator=g)
    codes = torch.where((codes & 0x7F) == 0x7F, codes - 1, codes)
    out = torch.empty(blocks * 512, dtype=torch.float32, device=dev)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def run(promote, shape=16):
        rc = lib.bench_mfma_ceiling(ctypes.c_void_p(codes.data_ptr()), ctypes.c_void_p(out.data_ptr()),
                                    blocks, iters, int(promote), int(shape), st)
        if rc != 0:
            raise RuntimeError(f"bench_mfma_ceiling failed ({rc})")

    return run, float(blocks * 8 * iters * 32) * 2 * 16 * 16 * 128


def stream_mix_ceilings(dev, mixes, iters=20):
    """bench_ceiling.so's k_stream_mix: for each HBM-bound kernel, the rate at which its read
    : write byte mix moves in linear, coalesced 16-byte order (no arithmetic, no transposes),
    best over four grids.  mixes: name -> (bytes read, R, W, input buffers rotated); the
    kernel reads R and writes W chunks per unit, so it writes bytes_read * W / R.  Returns
    name -> {"gbps", "us", "grid", "bytes"}."""
    import ctypes

    import torch

    lib = ctypes.CDLL(os.path.join(ROOT, "bench_ceiling.so"))
    lib.bench_stream_mix.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int,
                                     ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    res = {}
    for name, (rd, r, w, nbuf) in mixes.items():
        units = rd // (16 * r)
        srcs = [torch.ones(r * units * 16, dtype=torch.uint8, device=dev) for _ in range(nbuf)]
        dst = torch.empty(w * units * 16, dtype=torch.uint8, device=dev)
        best = None
        for grid in (1024, 2048, 4096, 8192):
            def run(i, grid=grid):
                rc = lib.bench_stream_mix(ctypes.c_void_p(srcs[i % nbuf].data_ptr()), ctypes.c_void_p(dst.data_ptr()),
                                          units, r, w, grid, st)
                if rc != 0:
                    raise RuntimeError(f"bench_stream_mix failed ({rc})")
            us = kernel_loop(run, iters, 3)
            if best is None or us < best[0]:
                best = (us, grid)
        moved = units * 16 * (r + w)
        res[name] = {"gbps": round(moved / best[0] / 1e3, 1), "us": round(best[0], 2), "grid": best[1],
                     "bytes": moved, "read_write": f"{r}:{w}"}
        del srcs, dst
    torch.cuda.empty_cache()
    return res


def config1_step(dev, steps):
    """Config 1 on the GPU: X[2048,512] bf16, W[1024,512] bf16 (seed 1), the forward
    quantizer pair in one launch and the GEMM, bf16 out.  Launch-bound at this size: the
    device time of the two kernels and the step time with its host launch overhead."""
    import torch

    from cinnamon_amd import kernels

    g = torch.Generator().manual_seed(1)
    x = torch.randn(2048, 512, generator=g).to(torch.bfloat16).to(dev)
    w = (torch.randn(1024, 512, generator=g) * 0.02).to(torch.bfloat16).to(dev)
    y = torch.empty(2048, 1024, dtype=torch.bfloat16, device=dev)

    def step(i):
        a, sa, b, _, sb = kernels.quantize_fp8_forward(x, w, col_scales=True)
        kernels.fp8_gemm_bs(a, sa, b, sb, torch.bfloat16, out=y)

    dev_us = kernel_loop(step, max(steps, 50), 5)
    step_us = time_loop(step, max(steps, 50), 5)
    fl = 2.0 * 2048 * 1024 * 512
    return {"what": "config 1: forward quantizer pair + GEMM, X[2048,512] x W[1024,512]^T, bf16 out",
            "device_us": round(dev_us, 2), "step_us": round(step_us, 2),
            "tflops_device": round(fl / dev_us / 1e6, 1)}


def config5_training(dev, steps=4):
    """Config 5: training steps of the MLA + MoE model of tests/c5_model.py (8 layers,
    d_model 1024, 16 + 1 experts, batch 16 x 1024 tokens, 633M parameters) with its Linear
    and expert layers on the FP8 path, against the same model kept in fp32 with the
    reference's per-expert loop; same weights and token batches.  Tokens per second over
    the steps after the first (test_c5_training.py checks the losses agree)."""
    import torch

    from tests.c5_model import C5Config, C5Model, to_fp8, train

    c = C5Config()
    torch.manual_seed(5)
    ref = C5Model(c).to(dev)
    fp8 = to_fp8(ref)
    g = torch.Generator().manual_seed(5)
    batches = [torch.randint(0, c.vocab_size, (16, 1025), generator=g).to(dev) for _ in range(steps)]
    sync = torch.cuda.synchronize
    l8, _, t8 = train(fp8, batches, sync)
    del fp8
    torch.cuda.empty_cache()
    lr, _, tr = train(ref, batches, sync)
    del ref
    torch.cuda.empty_cache()
    tok = 16 * 1024
    return {"what": "config 5 training steps (tests/c5_model.py, fp32 model, FP8 Linear and expert layers) "
                    "against the same model in fp32 with the per-expert loop",
            "steps": steps, "tokens_per_step": tok,
            "tokens_per_s_fp8": round(tok * (steps - 1) / sum(t8[1:])),
            "tokens_per_s_fp32_reference": round(tok * (steps - 1) / sum(tr[1:])),
            "loss_fp8": [round(v, 4) for v in l8], "loss_fp32_reference": [round(v, 4) for v in lr]}


# config 3 sizes (moe_setup): tokens, top-k, d_model, expert hidden
C3_T, C3_TOPK, C3_D, C3_H = 16384, 8, 7168, 2048


def stream_mixes(nbuf):
    """The byte mix of each HBM-bound kernel in this benchmark: name -> (bytes read, R, W,
    input buffers rotated), with R : W its read : write ratio (scales aside)."""
    A = C3_T * C3_TOPK
    return {
        "quant_x_rowwise": (M * K * 2, 2, 1, nbuf),          # bf16 in, e4m3 out
        "quant_w_blockwise": (N * K * 2, 2, 1, nbuf),
        "quant_fwd_fused": ((M + N) * K * 2, 2, 1, nbuf),
        "dual_quant_dy": (M * N * 2, 1, 1, 1),               # bf16 in, two e4m3 layouts out
        "requant_x_block_t": (M * K, 1, 1, 1),               # e4m3 in, e4m3 out
        "swiglu_dual_grouped_dh12": (A * C3_H * 4 + A * 2 * C3_H * 2, 2, 1, 1),  # dh fp32 + h12 bf16 in
        "requant_grouped_x": (A * C3_D, 1, 1, 1),
        "gather_quant": (C3_T * C3_D * 2, 1, 4, 1),          # bf16 tokens in, k code rows each out
        "combine": (A * C3_D * 2, 4, 1, 1),                  # fp16 rows in, fp32 tokens out
    }


def _cpu_time(fn, runs, warmup=1):
    """Median wall time (s) of fn() over `runs` timed runs after `warmup` untimed ones."""
    for _ in range(warmup):
        fn()
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    ts.sort()
    return ts[len(ts) // 2]


def cpu_baseline():
    """Time the oracle (torch-CPU restatement of the reference path, src/kernels.py:50-62,
    111-123, 262-281 and the fp32 matmul of the dequantized operands) per config, on all host
    cores.  Each config reports its quantize time and its dequantize + matmul time: configs 1,
    2 and 4 in full, config 3 on 128 rows of each of 4 experts with the full config's time
    scaled from that sample (about 40 s of CPU work in all)."""
    import torch

    from oracle import fp8_oracle as orc

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    runs = 3
    res = {}

    def gen(seed, *shape, std=1.0, outliers=False):
        g = torch.Generator().manual_seed(seed)
        x = torch.randn(*shape, generator=g) * std
        if outliers:
            x[torch.rand(*shape, generator=g) < 0.01] *= 20
        return x.to(torch.bfloat16)

    def t_kn(codes):
        return codes.view(torch.uint8).t().contiguous()

    def record(name, rows, full_rows, q_s, mm_s, flop, what, fixed_q_s=0.0, fixed_scale=1.0):
        # fixed_q_s: the part of the quantize time that does not scale with the rows (the
        # weights), which the full config has fixed_scale times of
        scale = full_rows / rows
        res[name] = {"sample": what, "rows": rows, "full_rows": full_rows,
                     "quantize_ms": round(q_s * 1e3, 2), "dequant_matmul_ms": round(mm_s * 1e3, 2),
                     "tflops": round(flop / (q_s + mm_s) / 1e12, 4),
                     "full_config_ms_estimate": round(((q_s - fixed_q_s) * scale + fixed_q_s * fixed_scale
                                                        + mm_s * scale) * 1e3, 1)}

    # config 1: X[2048, 512], W[1024, 512] (seed 1), always in full
    x1, w1 = gen(1, 2048, 512), gen(1, 1024, 512, std=0.02)
    q1 = _cpu_time(lambda: (orc.quant_rowwise(x1), orc.quant_blockwise(w1)), runs)
    a1, s1 = orc.quant_rowwise(x1)
    b1, t1 = orc.quant_blockwise(w1)
    mm1 = _cpu_time(lambda: orc.gemm_ref(a1, s1, t_kn(b1), t1.t().contiguous()), runs)
    record("config1", 2048, 2048, q1, mm1, 2.0 * 2048 * 1024 * 512, "X[2048,512] x W[1024,512]^T, in full")

    # config 2: X[M, 7168] rows (seed 2), W[2048, 7168] quantized in full
    r2 = M
    x2, w2 = gen(2, r2, K, outliers=True), gen(2, N, K, std=0.02)
    q2 = _cpu_time(lambda: (orc.quant_rowwise(x2), orc.quant_blockwise(w2)), runs)
    a2, s2 = orc.quant_rowwise(x2)
    b2, t2 = orc.quant_blockwise(w2)
    bkn, tkn = t_kn(b2), t2.t().contiguous()
    mm2 = _cpu_time(lambda: orc.gemm_ref(a2, s2, bkn, tkn), runs)
    qw2 = _cpu_time(lambda: orc.quant_blockwise(w2), runs)
    record("config2", r2, M, q2, mm2, 2.0 * r2 * N * K,
           "X[8192,7168] x W[2048,7168]^T in full", fixed_q_s=qw2)

    # config 4: the backward of config 2 on r4 token rows: dual quantization of dY[r4, 2048]
    # (seed 4), re-quantization of the rows' X codes into 128x128 blocks, dgrad
    # dY.W -> [r4, 7168] and the wgrad contribution dY^T.X -> [2048, 7168]
    r4 = M
    dy = gen(4, r4, N, std=1e-3)
    xa, xsa = a2[:r4], s2[:r4]

    def c4_quant():
        orc.quant_rowwise(dy, 128, True)
        orc.quant_rowwise(dy.t().contiguous(), 128, True)
        orc.quant_blockwise(orc.dequant_rowwise(xa, xsa), 128, 128, False)

    q4 = _cpu_time(c4_quant, runs)
    gq, gs = orc.quant_rowwise(dy, 128, True)
    gqt, gst = orc.quant_rowwise(dy.t().contiguous(), 128, True)
    xb, xbs = orc.quant_blockwise(orc.dequant_rowwise(xa, xsa), 128, 128, False)

    def c4_mm():
        orc.gemm_ref(gq, gs, b2.view(torch.uint8), t2)        # dgrad: B = W [2048, 7168]
        orc.gemm_ref(gqt, gst, xb.view(torch.uint8), xbs)     # wgrad: B = X blocks [r4, 7168]

    mm4 = _cpu_time(c4_mm, runs)
    record("config4", r4, M, q4, mm4, 2 * 2.0 * r4 * N * K,
           "dY[8192,2048] in full: dual quant, X re-quant, dgrad and wgrad")

    # config 3: 4 of the 32 experts (the two largest and the two smallest of the Zipf routing,
    # seed 3), r3 rows of each: gate/up [r3,7168]x[4096,7168]^T and down [r3,2048]x[7168,2048]^T,
    # both expert weights quantized per expert
    g3 = torch.Generator().manual_seed(3)
    pz = torch.tensor([(e + 1) ** -1.1 for e in range(32)])
    cnt = torch.bincount(torch.multinomial(pz.expand(16384, 32), 8, replacement=False, generator=g3).reshape(-1),
                         minlength=32)
    order = cnt.argsort(descending=True)
    experts = [int(order[0]), int(order[1]), int(order[-2]), int(order[-1])]
    r3 = [128] * 4
    xs3 = [gen(30 + i, r, K) for i, r in enumerate(r3)]
    hs3 = [gen(40 + i, r, 2048) for i, r in enumerate(r3)]
    w12 = [gen(50 + i, 4096, K, std=0.02) for i in range(4)]
    w3 = [gen(60 + i, K, 2048, std=0.02) for i in range(4)]

    def c3_quant():
        for i in range(4):
            orc.quant_rowwise(xs3[i])
            orc.quant_rowwise(hs3[i])
            orc.quant_blockwise(w12[i])
            orc.quant_blockwise(w3[i])

    q3 = _cpu_time(c3_quant, runs)
    ops = []
    for i in range(4):
        xa3, xs3_ = orc.quant_rowwise(xs3[i])
        ha3, hs3_ = orc.quant_rowwise(hs3[i])
        wa, wsa = orc.quant_blockwise(w12[i])
        wb, wsb = orc.quant_blockwise(w3[i])
        ops.append((xa3, xs3_, t_kn(wa), wsa.t().contiguous(), ha3, hs3_, t_kn(wb), wsb.t().contiguous()))

    def c3_mm():
        for xa3, xs3_, wa, wsa, ha3, hs3_, wb, wsb in ops:
            orc.gemm_ref(xa3, xs3_, wa, wsa)
            orc.gemm_ref(ha3, hs3_, wb, wsb)

    mm3 = _cpu_time(c3_mm, runs)
    qw3 = _cpu_time(lambda: [(orc.quant_blockwise(w12[i]), orc.quant_blockwise(w3[i])) for i in range(4)],
                    runs)
    record("config3", sum(r3), int(cnt.sum()), q3, mm3, sum(2.0 * r * K * 4096 + 2.0 * r * 2048 * K for r in r3),
           f"experts {experts} (rows {[int(cnt[e]) for e in experts]}), 128 rows of each; gate/up and down, "
           "both weights quantized (full-config estimate: all 131072 rows and the 32 experts' weights)",
           fixed_q_s=qw3, fixed_scale=8.0)

    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    c2 = res["config2"]
    return {
        "value": c2["tflops"],
        "unit": "TFLOP/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"config 2 forward in full (X[8192,7168], W[2048,7168]): oracle quantize "
                  f"{c2['quantize_ms']} ms + dequantize and fp32 matmul {c2['dequant_matmul_ms']} ms, median of "
                  f"{runs}; configs 1, 3 (4 experts x 128 rows) and 4 in per_config; CPU {model}",
        "per_config": res,
    }


def measured_traffic(profile="profiles/k_gemm_fp8_bs_256_config2_fwd.txt"):
    """HBM bytes per GEMM launch from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE summary
    (copy-calibrated); None if the summary is absent."""
    path = os.path.join(ROOT, profile)
    try:
        for line in open(path):
            if "total" in line and "MB" in line:
                return int(float(line.rsplit("total", 1)[1].split("MB")[0]) * 1e6), profile
    except OSError:
        pass
    return None, None


def measured_mfma(profile="profiles/k_gemm_fp8_bs_256_config2_fwd.txt"):
    """The committed rocprofv3 MFMA-counter figures of the GEMM: FP8 FLOP per launch
    (SQ_INSTS_VALU_MFMA_MOPS_F8 x 512), average clock (GRBM_GUI_ACTIVE) and MfmaUtil
    (SQ_VALU_MFMA_BUSY_CYCLES over active cycles x SIMDs); None if the summary is absent."""
    out = {}
    try:
        for line in open(os.path.join(ROOT, profile)):
            if "SQ_INSTS_VALU_MFMA_MOPS_F8 x 512 =" in line:
                out["mfma_flop_per_launch"] = float(line.split("=")[1].split("GFLOP")[0]) * 1e9
            elif "MHz average clock" in line:
                out["clock_mhz"] = float(line.split("->")[1].split("MHz")[0])
            elif line.strip().startswith("MfmaUtil"):
                out["mfma_util"] = round(float(line.rsplit("=", 1)[1].strip().rstrip("%")) / 100, 4)
    except (OSError, ValueError, IndexError):
        return None
    if len(out) != 3:
        return None
    out["source"] = profile
    return out


def moe_setup(dev):
    """Config 3: 32 experts, d_model 7168, expert hidden 2048, 16384 tokens, top-8 routing
    with Zipf(1.1) expert popularity (sampled without replacement), bf16 ~N(0,1)
    activations and ~N(0,0.02) weights.  Large operands come from the GPU generator."""
    import torch

    from cinnamon_amd import kernels

    E, D, H, T, topk = 32, 7168, 2048, 16384, 8
    g = torch.Generator(device=dev).manual_seed(3)
    p = torch.tensor([(e + 1) ** -1.1 for e in range(E)], device=dev)
    sel = torch.multinomial(p.expand(T, E), topk, replacement=False, generator=g)
    counts = torch.bincount(sel.reshape(-1), minlength=E)
    ends = counts.cumsum(0)
    starts = ends - counts
    A = T * topk
    x = torch.randn(A, D, device=dev, generator=g).to(torch.bfloat16)
    h = torch.randn(A, H, device=dev, generator=g).to(torch.bfloat16)
    w12 = (torch.randn(E * 2 * H, D, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    w3 = (torch.randn(E * D, H, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    w12q, w12s = kernels.quantize_fp8_blockwise(w12)
    w3q, w3s = kernels.quantize_fp8_blockwise(w3)
    del w12, w3
    return dict(E=E, D=D, H=H, A=A, T=T, topk=topk, sel=sel, x=x, h=h, starts=starts, ends=ends, counts=counts,
                w12q=w12q.view(E, 2 * H, D), w12s=w12s.view(E, 2 * H // 128, D // 128),
                w3q=w3q.view(E, D, H), w3s=w3s.view(E, D // 128, H // 128))


def moe_bwd_setup(dev, moe):
    """Config-3 backward operands for the gate/up GEMM: dH [A, H] fp32 ~N(0, 1e-3) (the down
    GEMM's dgrad output), the saved gate/up output h12 [A, 2H] bf16 ~N(0, 1), and the stacked
    transposed w12 codes [D, E*2H] (the grouped dgrad's B operand)."""
    import torch

    from cinnamon_amd import kernels

    g = torch.Generator(device=dev).manual_seed(33)
    E, D, H, A = moe["E"], moe["D"], moe["H"], moe["A"]
    dh = torch.randn(A, H, device=dev, generator=g) * 1e-3
    h12 = torch.randn(A, 2 * H, device=dev, generator=g).to(torch.bfloat16)
    w12 = (torch.randn(E * 2 * H, D, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    _, w12qt, w12s = kernels.quantize_fp8_blockwise_t(w12, with_rowmajor=False)
    del w12
    return dict(dh=dh, h12=h12, w12qt=w12qt, w12s=w12s)


def bwd_setup(dev, xs0, w0):
    """Config 4: backward of the config-2 shapes; dY[8192, 2048] bf16 ~N(0, 1e-3)."""
    import torch

    from cinnamon_amd import kernels

    g = torch.Generator(device=dev).manual_seed(4)
    dy = (torch.randn(M, N, device=dev, generator=g) * 1e-3).to(torch.bfloat16)
    xq, xs = kernels.quantize_fp8_rowwise(xs0, col_scales=True)
    _, wqt, ws = kernels.quantize_fp8_blockwise_t(w0.float(), with_rowmajor=False)
    return dict(dy=dy, xq=xq, xs=xs, wqt=wqt, ws=ws)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the multi-GPU "
              "sharding is a design note, not a measured path.", file=sys.stderr)
        sys.exit(2)

    import torch

    from cinnamon_amd import kernels

    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(2)
    nbuf = 3
    xs = []
    for i in range(nbuf):
        x = torch.randn(M, K, generator=g)
        x[torch.rand(M, K, generator=g) < 0.01] *= 20
        xs.append(x.to(torch.bfloat16).to(dev))
    ws = [(torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16).to(dev) for _ in range(nbuf)]
    del x

    # pre-quantized operands for the GEMM-only timing
    xq, xsc = kernels.quantize_fp8_rowwise(xs[0], col_scales=True)
    wq, wsc = kernels.quantize_fp8_blockwise(ws[0])
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)

    def step(i):
        # X row tiles and W blocks in one launch (cin_quant_fwd), then the GEMM; X's scales
        # column-major, as the FP8 linear keeps them
        a, sa, b, _, sb = kernels.quantize_fp8_forward(xs[i % nbuf], ws[i % nbuf], col_scales=True)
        kernels.fp8_gemm_bs(a, sa, b, sb, torch.bfloat16, out=y)

    def gemm(i):
        kernels.fp8_gemm_bs(xq, xsc, wq, wsc, torch.bfloat16, out=y)

    # for comparison: the vendor library's FP8 GEMM (hipBLASLt through torch._scaled_mm) on the
    # same codes with one scale per tensor, i.e. without the per-block promotion
    one = torch.ones((), dtype=torch.float32, device=dev)

    def scaled_mm(i):
        torch._scaled_mm(xq, wq.t(), scale_a=one, scale_b=one, out_dtype=torch.bfloat16)

    def quant_x(i):
        kernels.quantize_fp8_rowwise(xs[i % nbuf])

    def quant_w(i):
        kernels.quantize_fp8_blockwise(ws[i % nbuf])

    def quant_fwd(i):
        kernels.quantize_fp8_forward(xs[i % nbuf], ws[i % nbuf], col_scales=True)

    from cinnamon_amd import layers

    moe = bwd = None
    full = args.only is None and not args.no_extra
    if full or (args.only or "").startswith("moe"):
        moe = moe_setup(dev)
        # the experts' activation scales are column-major, as layers.experts_forward keeps them
        hq, hs = kernels.quantize_fp8_rowwise(moe["h"], col_scales=True)
        xq3, xs3 = kernels.quantize_fp8_rowwise(moe["x"], col_scales=True)
        y12 = torch.empty((moe["A"], 2 * moe["H"]), dtype=torch.bfloat16, device=dev)
        y3 = torch.empty((moe["A"], moe["D"]), dtype=torch.bfloat16, device=dev)

    def moe_gateup(i):
        layers.fp8_grouped_gemm(xq3, xs3, moe["w12q"], moe["w12s"], moe["starts"], moe["ends"], out=y12)

    def moe_down(i):
        layers.fp8_grouped_gemm(hq, hs, moe["w3q"], moe["w3s"], moe["starts"], moe["ends"], out=y3)

    # config-3 backward of the gate/up GEMM (the larger one): SwiGLU backward fused with the
    # grouped dual quantization of its output dH12 [A, 2H], grouped re-quantization of the saved X codes, grouped wgrad
    # dW12 [E, 2H, D] and grouped dgrad dX [A, D]
    mb = None
    if full or args.only in ("moe_dual", "moe_requant", "moe_wgrad", "moe_dgrad"):
        if moe is None:
            moe = moe_setup(dev)
            xq3, xs3 = kernels.quantize_fp8_rowwise(moe["x"], col_scales=True)
        mb = moe_bwd_setup(dev, moe)
        gq3, gs3, gqt3, gst3 = layers.swiglu_backward_dual_grouped(mb["dh"], mb["h12"], moe["starts"],
                                                                   moe["ends"], col_scales=True)
        xbt3, xbs3 = layers.requantize_grouped_t(xq3, xs3, moe["starts"], moe["ends"])
        dx3 = torch.empty((moe["A"], moe["D"]), dtype=torch.bfloat16, device=dev)

    def moe_dual(i):
        layers.swiglu_backward_dual_grouped(mb["dh"], mb["h12"], moe["starts"], moe["ends"], col_scales=True)

    def moe_requant(i):
        layers.requantize_grouped_t(xq3, xs3, moe["starts"], moe["ends"])

    def moe_wgrad(i):
        layers.fp8_grouped_wgrad(gqt3, gst3, xbt3, xbs3, moe["starts"], moe["ends"], moe["A"],
                                 out_dtype=torch.bfloat16)

    def moe_dgrad(i):
        layers.fp8_grouped_dgrad(gq3, gs3, mb["w12qt"], mb["w12s"], moe["starts"], moe["ends"],
                                 2 * moe["H"], out=dx3)

    # config 3 experts layer end to end (layers.GroupedExperts, FP8 forward and backward):
    # weights quantized inside every call, as in training
    ml = None
    if full or args.only in ("moe_layer", "moe_layer_fwd"):
        if moe is None:
            moe = moe_setup(dev)
        g3 = torch.Generator(device=dev).manual_seed(34)
        ml = layers.GroupedExperts(moe["E"], moe["D"], moe["H"]).to(dev)
        ml_x = moe["x"].detach().clone().requires_grad_(True)
        ml_g = torch.randn(moe["A"], moe["D"], device=dev, generator=g3) * 1e-3

    def moe_layer(i):
        ml_x.grad = None
        ml.zero_grad(set_to_none=True)
        ml(ml_x, moe["starts"], moe["ends"]).backward(ml_g)

    def moe_layer_fwd(i):
        with torch.no_grad():
            ml(ml_x, moe["starts"], moe["ends"])

    # the whole routed block of MoE.forward (src/layers.py:126-157), forward + backward, on
    # the same FP8 experts: cinnamon_amd.moe.routed_experts against the reference's torch
    # routing (sort, gather, bincount, .item(), gated scatter_add_) around them
    def moe_routed_setup():
        g6 = torch.Generator(device=dev).manual_seed(37)
        T3, k3 = moe["T"], moe["topk"]
        sc = torch.rand(T3, k3, device=dev, generator=g6)
        return dict(x=moe["x"][:T3].detach().clone().requires_grad_(True),
                    sc=(sc / sc.sum(-1, keepdim=True)).requires_grad_(True),
                    dout=torch.randn(T3, moe["D"], device=dev, generator=g6) * 1e-3)

    def moe_routed_fused(i):
        r = mr
        r["x"].grad = r["sc"].grad = None
        ml.zero_grad(set_to_none=True)
        out, _ = moe_ops_r.routed_experts(ml, r["x"], moe["sel"], r["sc"])
        out.backward(r["dout"])

    def moe_routed_torch(i):
        r = mr
        r["x"].grad = r["sc"].grad = None
        ml.zero_grad(set_to_none=True)
        k3 = moe["topk"]
        flat = moe["sel"].reshape(-1)
        sorted_idx, order = flat.sort()
        tok = order // k3
        sorted_x = r["x"][tok]
        cnt = torch.bincount(sorted_idx, minlength=moe["E"])
        ends = cnt.cumsum(0)
        starts = ends - cnt
        int(cnt.max().item())
        sorted_out = ml(sorted_x, starts, ends)
        w = sorted_out * r["sc"].reshape(-1)[order][:, None]
        out = torch.zeros(moe["T"], moe["D"], device=dev, dtype=w.dtype)
        out.scatter_add_(0, tok.unsqueeze(1).expand_as(w), w)
        out.backward(r["dout"])

    # config 3 dispatch and combine around the experts (cinnamon_amd.moe) against the
    # reference's torch formulation of the same block (src/layers.py:133-154)
    md = None
    if full or args.only in ("moe_route", "moe_gather", "moe_combine", "moe_combine_bwd"):
        from cinnamon_amd import moe as moe_ops
        if moe is None:
            moe = moe_setup(dev)
        g4 = torch.Generator(device=dev).manual_seed(35)
        T3, k3 = moe["T"], moe["topk"]
        sc3 = torch.rand(T3, k3, device=dev, generator=g4)
        sc3 = (sc3 / sc3.sum(-1, keepdim=True)).to(torch.bfloat16)
        md = dict(x=moe["x"][:T3], sel=moe["sel"], scores=sc3,
                  ys=torch.randn(moe["A"], moe["D"], device=dev, generator=g4))
        md["perm"], md["inv"], *_ = moe_ops.moe_route(md["sel"], moe["E"])
        md["ys16"] = md["ys"].half()  # routed_experts stores the sorted outputs in fp16
        md["dout"] = torch.randn(T3, moe["D"], device=dev, generator=g4)

    def moe_route(i):
        moe_ops.moe_route(md["sel"], moe["E"])

    def moe_gather(i):
        moe_ops.moe_gather_quantize(md["x"], md["perm"], moe["topk"], inv=md["inv"], col_scales=True)

    def moe_combine(i):
        moe_ops.moe_combine(md["ys16"], md["scores"], md["inv"])

    def moe_combine_bwd(i):
        moe_ops.moe_combine_backward(md["dout"], md["ys16"], md["scores"], md["perm"], md["inv"],
                                     dy_dtype=torch.bfloat16)

    def moe_dispatch_fused(i):
        perm, inv, *_ = moe_ops.moe_route(md["sel"], moe["E"])
        moe_ops.moe_gather_quantize(md["x"], perm, moe["topk"], inv=inv, col_scales=True)

    def moe_dispatch_torch(i):
        k = moe["topk"]
        _, order = md["sel"].reshape(-1).sort()
        tok = order // k
        sorted_x = md["x"][tok]
        cnt = torch.bincount(md["sel"].reshape(-1), minlength=moe["E"])
        cnt.cumsum(0)
        int(cnt.max().item())
        kernels.quantize_fp8_rowwise(sorted_x)

    def moe_combine_torch(i):
        k = moe["topk"]
        _, order = md["sel"].reshape(-1).sort()
        tok = order // k
        w = md["ys"] * md["scores"].reshape(-1)[order][:, None]
        torch.zeros(moe["T"], moe["D"], device=dev, dtype=w.dtype).scatter_add_(
            0, tok.unsqueeze(1).expand_as(w), w)

    # DSA indexer scores on FP8 q / k (src/attention.py:288-300) at the model's indexer shape:
    # 4 heads, d_indexer_head 64 widened to 128 by PoPE, 16 sequences of 1024 tokens
    ix = None
    if full or args.only in ("indexer", "indexer_wgrad", "indexer_full"):
        g5 = torch.Generator(device=dev).manual_seed(36)
        IB, IL, IH, ID = 16, 1024, 4, 128
        ix = dict(q=torch.randn(IB, IL, IH, ID, device=dev, generator=g5).to(torch.bfloat16),
                  k=torch.randn(IB, IL, ID, device=dev, generator=g5).to(torch.bfloat16),
                  w=torch.randn(IB, IL, IH, device=dev, generator=g5) * 0.5, shape=(IB, IL, IH, ID))
        q8, qsc = kernels.quantize_fp8_rowwise(ix["q"].reshape(-1, ID), block_size=128)
        k8, ksc = kernels.quantize_fp8_rowwise(ix["k"].reshape(-1, ID), block_size=128)
        ix["q8"], ix["qs"] = q8.view(IB, IL, IH, ID), qsc.view(IB, IL, IH)
        ix["k8"], ix["ks"] = k8.view(IB, IL, ID), ksc.view(IB, IL)
        ix["g"] = torch.randn(IB, IL, IL, device=dev, generator=g5)

    def indexer(i):
        torch.ops.cinnamon_amd.indexer_scores_fp8(ix["q8"], ix["qs"], ix["k8"], ix["ks"], ix["w"], 0.125)

    def indexer_wgrad(i):
        torch.ops.cinnamon_amd.indexer_weights_grad_fp8(ix["q8"], ix["qs"], ix["k8"], ix["ks"], ix["g"], 0.125)

    def indexer_full(i):
        kernels.indexer_scores_fp8(ix["q"], ix["k"], ix["w"], 0.125)

    def indexer_two_call(i):
        # both quantizations in one launch, then the scoring kernel on the codes
        c = torch.ops.cinnamon_amd.indexer_quantize(ix["q"], ix["k"])
        torch.ops.cinnamon_amd.indexer_scores_fp8(*c, ix["w"], 0.125)

    def indexer_fused(i):
        torch.ops.cinnamon_amd.indexer_scores_fp8_q(ix["q"], ix["k8"], ix["ks"], ix["w"], 0.125, False)

    def indexer_full_fwd_bwd(i):
        w = ix["w"].detach().requires_grad_(True)
        kernels.indexer_scores_fp8(ix["q"], ix["k"], w, 0.125).backward(ix["g"])

    def indexer_torch(i):
        IB, IL, IH, ID = ix["shape"]
        q8, qsc = kernels.quantize_fp8_rowwise(ix["q"].reshape(-1, ID), block_size=128)
        k8, ksc = kernels.quantize_fp8_rowwise(ix["k"].reshape(-1, ID), block_size=128)
        logits = torch.einsum("bthd,bsd->bths", q8.view(IB, IL, IH, ID).float(), k8.view(IB, IL, ID).float())
        logits = torch.relu(logits) * (qsc.view(IB, IL, IH) * ix["w"] * 0.125).unsqueeze(-1)
        return logits.sum(dim=2) * ksc.view(IB, IL).unsqueeze(1)

    def indexer_torch_fwd_bwd(i):
        w = ix["w"].detach().requires_grad_(True)
        IB, IL, IH, ID = ix["shape"]
        q8, qsc = kernels.quantize_fp8_rowwise(ix["q"].reshape(-1, ID), block_size=128)
        k8, ksc = kernels.quantize_fp8_rowwise(ix["k"].reshape(-1, ID), block_size=128)
        logits = torch.einsum("bthd,bsd->bths", q8.view(IB, IL, IH, ID).float(), k8.view(IB, IL, ID).float())
        logits = torch.relu(logits) * (qsc.view(IB, IL, IH) * w * 0.125).unsqueeze(-1)
        (logits.sum(dim=2) * ksc.view(IB, IL).unsqueeze(1)).backward(ix["g"])

    if full or args.only in ("dual_quant", "requant", "dgrad", "wgrad", "bwd_pair"):
        bwd = bwd_setup(dev, xs[0], ws[0])
        gq, gs, gqt, gst = kernels.quantize_fp8_dual(bwd["dy"], col_scales=True)
        xbt, xbs = kernels.requantize_rowwise_to_blockwise(bwd["xq"], bwd["xs"], transposed=True)
        dx = torch.empty((M, K), dtype=torch.bfloat16, device=dev)
        dw = torch.empty((N, K), dtype=torch.bfloat16, device=dev)

    def dual_quant(i):
        kernels.quantize_fp8_dual(bwd["dy"], col_scales=True)

    def requant(i):
        kernels.requantize_rowwise_to_blockwise(bwd["xq"], bwd["xs"], transposed=True)

    def bwd_pair(i):
        # both quantizations above in one launch (FP8MatmulFunction.backward calls this)
        kernels.quantize_fp8_backward(bwd["dy"], bwd["xq"], bwd["xs"], col_scales=True)

    def dgrad(i):
        kernels.fp8_gemm_bs(gq, gs, bwd["wqt"], bwd["ws"].t(), torch.bfloat16, out=dx)

    def wgrad(i):
        kernels.fp8_gemm_bs(gqt, gst, xbt, xbs.t(), torch.bfloat16, out=dw)

    if args.only == "mfma_ceiling":
        run_ceiling, ceil_flop = mfma_ceiling_setup(dev)
        res = {}
        # alternating rounds: the power-limited clock drifts over a run
        for rnd in range(2):
            for shape in (16, 32):
                for promote in (1, 0):
                    us = kernel_loop(lambda i: run_ceiling(promote, shape), args.steps, args.warmup)
                    key = f"mfma{shape}_" + ("promotion" if promote else "hardware_accumulation")
                    res.setdefault(key, []).append({"us_per_call": round(us, 2),
                                                    "tflops": round(ceil_flop / us / 1e6, 1)})
        print(json.dumps({"only": "mfma_ceiling", **res}))
        return
    if args.only == "config1":
        print(json.dumps({"only": "config1", **config1_step(dev, args.steps)}))
        return
    if args.only == "config5":
        print(json.dumps({"only": "config5", **config5_training(dev)}))
        return
    if args.only == "traffic_ceiling":
        print(json.dumps({"only": "traffic_ceiling", **stream_mix_ceilings(dev, stream_mixes(nbuf), args.steps)}))
        return
    if args.only == "copy":
        # calibration for HBM byte counters: a plain copy of 512 MiB (read 512 MiB, write 512 MiB)
        src = torch.empty(256 * 1024 * 1024, dtype=torch.bfloat16, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        us = time_loop(lambda i: dst.copy_(src), args.steps, args.warmup)
        print(json.dumps({"only": "copy", "bytes_read": src.numel() * 2, "bytes_written": src.numel() * 2,
                          "us_per_call": us}))
        return
    if args.only:
        fn = {"step": step, "gemm": gemm, "scaled_mm": scaled_mm, "quant_x": quant_x, "quant_w": quant_w, "quant_fwd": quant_fwd,
              "moe_gateup": moe_gateup, "moe_down": moe_down, "dual_quant": dual_quant,
              "bwd_pair": bwd_pair,
              "requant": requant, "dgrad": dgrad, "wgrad": wgrad, "moe_dual": moe_dual,
              "moe_requant": moe_requant, "moe_wgrad": moe_wgrad, "moe_dgrad": moe_dgrad,
              "moe_layer": moe_layer, "moe_layer_fwd": moe_layer_fwd, "moe_route": moe_route, "moe_gather": moe_gather,
              "moe_combine": moe_combine, "moe_combine_bwd": moe_combine_bwd, "indexer": indexer, "indexer_wgrad": indexer_wgrad,
              "indexer_full": indexer_full}[args.only]
        if args.only == "step":
            us = time_loop(fn, args.steps, args.warmup, settle_ms=SETTLE_MS)
        else:
            us = kernel_loop(fn, args.steps, args.warmup)
        print(json.dumps({"only": args.only, "us_per_call": us}))
        return

    # the timed region: exactly `steps` steps, synchronized on both sides
    torch.cuda.synchronize()
    step_us = time_loop(step, args.steps, args.warmup, settle_ms=SETTLE_MS)
    gemm_us = kernel_loop(gemm, max(args.steps, 50), 5)
    try:
        smm_us = kernel_loop(scaled_mm, max(args.steps, 50), 5)
    except RuntimeError as e:  # an FP8 GEMM torch was built without
        smm_us, smm_err = None, str(e)[:200]
    qx_us = kernel_loop(quant_x, max(args.steps, 50), 5)
    qw_us = kernel_loop(quant_w, max(args.steps, 50), 5)
    qf_us = kernel_loop(quant_fwd, max(args.steps, 50), 5)
    # the MFMA rate this GPU sustains on random e4m3 operands under its power limit, for the
    # GEMM's own MFMA + promotion-FMA mix with no memory traffic at all
    run_ceiling, ceil_flop = mfma_ceiling_setup(dev)
    ceil_us = kernel_loop(lambda i: run_ceiling(1), 20, 3)
    ceil_hw_us = kernel_loop(lambda i: run_ceiling(0), 20, 3)
    ceil_tflops, ceil_hw_tflops = ceil_flop / ceil_us / 1e6, ceil_flop / ceil_hw_us / 1e6

    flops = 2.0 * M * N * K
    qx_bytes = M * K * 2 + M * K + M * (K // 128) * 4        # read bf16, write e4m3 + scales
    qw_bytes = N * K * 2 + N * K + (N // 128) * (K // 128) * 4
    gemm_bytes = M * K + N * K + M * N * 2 + (M * K // 128 + (N // 128) * (K // 128)) * 4
    gemm_tflops = flops / (gemm_us * 1e-6) / 1e12
    qx_gbps = qx_bytes / (qx_us * 1e-6) / 1e9
    qw_gbps = qw_bytes / (qw_us * 1e-6) / 1e9
    qf_gbps = (qx_bytes + qw_bytes) / (qf_us * 1e-6) / 1e9

    out = {
        "metric": METRIC,
        "value": round(flops / (step_us * 1e-6) / 1e12, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle_ms": SETTLE_MS,
        "ms_per_step": round(step_us / 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8_e4m3 (fp32 accumulate)",
        "data": "synthetic",
        "config": {
            "workload": "config 2 dense forward: rowwise 1x128 quant of X[8192,7168] bf16 (1% x20 "
                        "outliers) + 128x128 quant of W[2048,7168] bf16 + block-scaled FP8 GEMM, bf16 out",
            "M": M, "N": N, "K": K, "seed": 2, "rotating_input_buffers": nbuf,
        },
        "roofline": {
            "bound": "mfma",
            "achieved": round(gemm_tflops, 2),
            "peak": PEAK_FP8_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(gemm_tflops / PEAK_FP8_TFLOPS, 4),
            "traffic": measured_traffic()[0],
            "traffic_source": measured_traffic()[1],
            "counters": measured_mfma(),
            "ceiling": {
                "what": "register-only loop of the GEMM's MFMA + per-block promotion FMA mix on random "
                        "e4m3 operands (bench_ceiling.hip): the rate the power limit allows with no "
                        "operand traffic; with MFMA accumulation in hardware instead (no block "
                        "scales to apply) for comparison",
                "tflops": round(ceil_tflops, 1),
                "frac_of_peak": round(ceil_tflops / PEAK_FP8_TFLOPS, 4),
                "hardware_accumulation_tflops": round(ceil_hw_tflops, 1),
                "gemm_frac_of_ceiling": round(gemm_tflops / ceil_tflops, 4),
            },
            "kernel": "k_gemm_fp8_bs_256",
            "algorithmic_work": "2*M*N*K = %.4g FLOP per launch" % flops,
        },
        "components": {
            "gemm": {"us": round(gemm_us, 2), "tflops": round(gemm_tflops, 2),
                     "frac_of_fp8_peak": round(gemm_tflops / PEAK_FP8_TFLOPS, 4),
                     "min_bytes": gemm_bytes},
            "hipblaslt_per_tensor_fp8": (
                {"what": "torch._scaled_mm (hipBLASLt) on the same e4m3 codes with one scale per "
                         "tensor: the GEMM without per-block promotion, not the block-scaled result",
                 "us": round(smm_us, 2), "tflops": round(flops / (smm_us * 1e-6) / 1e12, 1)}
                if smm_us is not None else {"error": smm_err}),
            "quant_x_rowwise": {"us": round(qx_us, 2), "gbps": round(qx_gbps, 1),
                                "frac_of_hbm": round(qx_gbps / PEAK_HBM_GBPS, 4), "bytes": qx_bytes},
            "quant_w_blockwise": {"us": round(qw_us, 2), "gbps": round(qw_gbps, 1),
                                  "frac_of_hbm": round(qw_gbps / PEAK_HBM_GBPS, 4), "bytes": qw_bytes},
            "quant_fwd_fused": {"what": "X row tiles and W blocks in one launch, as in the step",
                                "us": round(qf_us, 2), "gbps": round(qf_gbps, 1),
                                "frac_of_hbm": round(qf_gbps / PEAK_HBM_GBPS, 4),
                                "bytes": qx_bytes + qw_bytes},
        },
    }
    if moe is not None:
        A, D, H = moe["A"], moe["D"], moe["H"]
        gu_us = kernel_loop(moe_gateup, 10, 2)
        dn_us = kernel_loop(moe_down, 10, 2)
        gu_fl, dn_fl = 2.0 * A * D * 2 * H, 2.0 * A * H * D
        out["components"]["config3_moe_forward"] = {
            "tokens": 16384, "topk": 8, "rows": A, "experts": moe["E"],
            "expert_rows_max": int(moe["counts"].max()), "expert_rows_min": int(moe["counts"].min()),
            "gate_up": {"us": round(gu_us, 1), "tflops": round(gu_fl / gu_us / 1e6, 1),
                        "frac_of_fp8_peak": round(gu_fl / gu_us / 1e6 / PEAK_FP8_TFLOPS, 4)},
            "down": {"us": round(dn_us, 1), "tflops": round(dn_fl / dn_us / 1e6, 1),
                     "frac_of_fp8_peak": round(dn_fl / dn_us / 1e6 / PEAK_FP8_TFLOPS, 4)},
        }
    if ml is not None:
        from cinnamon_amd import moe as moe_ops_r
        mr = moe_routed_setup()
        rf_ms = time_loop(moe_routed_fused, 3, 1) / 1e3
        rt_ms = time_loop(moe_routed_torch, 3, 1) / 1e3
        del mr
        A, D, H = moe["A"], moe["D"], moe["H"]
        f_ms = time_loop(moe_layer_fwd, 3, 1) / 1e3
        fb_ms = time_loop(moe_layer, 3, 1) / 1e3
        fl = 2.0 * A * D * 2 * H + 2.0 * A * H * D
        out["components"]["config3_experts_layer"] = {
            "what": "layers.GroupedExperts (FP8) on the config-3 rows: weight quantization, "
                    "gate/up GEMM, SwiGLU + quantization, down GEMM; backward adds the grouped "
                    "dual/re-quantizers, SwiGLU backward, dgrad and wgrad of both GEMMs",
            "forward_ms": round(f_ms, 2), "forward_backward_ms": round(fb_ms, 2),
            "tokens_per_s_fwd_bwd": round(moe["A"] / (fb_ms * 1e-3) / 8),
            "routed_block_fwd_bwd_ms": round(rf_ms, 2),
            "routed_block_fwd_bwd_ms_torch_routing": round(rt_ms, 2),
            "gemm_tflops_fwd_bwd": round(3 * fl / (fb_ms * 1e-3) / 1e12, 1),
        }
    if md is not None:
        A, D, T3 = moe["A"], moe["D"], moe["T"]
        r_us = kernel_loop(moe_route, 20, 3)
        g_us = kernel_loop(moe_gather, 10, 2)
        c_us = kernel_loop(moe_combine, 5, 1)
        cb_us = kernel_loop(moe_combine_bwd, 5, 1)
        fused_us = time_loop(moe_dispatch_fused, 5, 1)
        torch_us = time_loop(moe_dispatch_torch, 5, 1)
        ctorch_us = time_loop(moe_combine_torch, 3, 1)
        # bytes: the gather reads each token row once (its k re-reads hit the caches) and
        # writes A code rows + scales; the combine reads the fp16 sorted rows and writes the
        # fp32 token rows (the torch formulation reads the reference's fp32 sorted_out)
        g_bytes = T3 * D * 2 + A * D + A * (D // 128) * 4
        c_bytes = A * D * 2 + T3 * D * 4 + A * 2 + A * 4
        out["components"]["config3_moe_dispatch"] = {
            "what": "cinnamon_amd.moe on the config-3 routing (16384 tokens, top-8, 32 Zipf experts, "
                    "d 7168) against the reference's torch formulation on the same GPU",
            "route_us": round(r_us, 1),
            "gather_quant_us": round(g_us, 1), "gather_quant_gbps": round(g_bytes / g_us / 1e3, 1),
            "gather_quant_frac_of_hbm": round(g_bytes / g_us / 1e3 / PEAK_HBM_GBPS, 4),
            "dispatch_us": round(fused_us, 1),
            "torch_sort_gather_bincount_item_quant_us": round(torch_us, 1),
            "combine_us": round(c_us, 1), "combine_gbps": round(c_bytes / c_us / 1e3, 1),
            "combine_frac_of_hbm": round(c_bytes / c_us / 1e3 / PEAK_HBM_GBPS, 4),
            "torch_sort_mul_scatter_add_us": round(ctorch_us, 1),
            "combine_backward_us": round(cb_us, 1),
        }
    if ix is not None:
        IB, IL, IH, ID = ix["shape"]
        k_us = kernel_loop(indexer, 20, 3)
        kf_us = kernel_loop(indexer_fused, 20, 3)
        kc_us = kernel_loop(indexer_full, 20, 3)
        k2_us = kernel_loop(indexer_two_call, 20, 3)
        kb_us = kernel_loop(indexer_wgrad, 20, 3)
        f_us = time_loop(indexer_full, 10, 2)
        t_us = time_loop(indexer_torch, 5, 1)
        fb_us = time_loop(indexer_full_fwd_bwd, 10, 2)
        tb_us = time_loop(indexer_torch_fwd_bwd, 3, 1)
        # bytes: q and k codes + scales + weights read once, scores written once (fp32)
        i_bytes = IB * IL * IH * ID + IB * IL * ID + IB * IL * IH * 8 + IB * IL * 4 + IB * IL * IL * 4
        i_flops = 2.0 * IB * IL * IL * IH * ID
        out["components"]["config5_indexer_scores"] = {
            "what": "kernels.indexer_scores_fp8 on 16 x 1024 tokens, 4 heads, d 128, against the "
                    "reference's FP8 einsum formulation (quantize, fp32 einsum, relu, weight, head "
                    "sum) on the same GPU.  kernel_us: the scoring kernel on codes; fused_q_kernel_us: "
                    "the one that quantizes q itself; call_device_us: the whole call's device time "
                    "(k quantization + fused kernel), against the two-call form (both "
                    "quantizations, then scoring on codes)",
            "kernel_us": round(k_us, 1), "kernel_gbps": round(i_bytes / k_us / 1e3, 1),
            "kernel_frac_of_hbm": round(i_bytes / k_us / 1e3 / PEAK_HBM_GBPS, 4),
            "kernel_tflops": round(i_flops / k_us / 1e6, 1),
            "fused_q_kernel_us": round(kf_us, 1),
            "call_device_us": round(kc_us, 1),
            "call_device_us_two_call": round(k2_us, 1),
            "weights_grad_kernel_us": round(kb_us, 1),
            "weights_grad_kernel_frac_of_hbm": round(i_bytes / kb_us / 1e3 / PEAK_HBM_GBPS, 4),
            "with_quantization_us": round(f_us, 1),
            "torch_einsum_us": round(t_us, 1),
            "forward_backward_us": round(fb_us, 1),
            "torch_einsum_forward_backward_us": round(tb_us, 1),
        }
    if mb is not None:
        A, D, H = moe["A"], moe["D"], moe["H"]
        cap = layers.padded_capacity(A, moe["E"])
        md_us = kernel_loop(moe_dual, 5, 1)
        mr_us = kernel_loop(moe_requant, 5, 1)
        mw_us = kernel_loop(moe_wgrad, 3, 1)
        mg_us = kernel_loop(moe_dgrad, 3, 1)
        fl = 2.0 * A * D * 2 * H
        # bytes: the fused SwiGLU backward + dual reads dH fp32 and h12 bf16, writes dH12's row
        # codes + scales and padded column codes + scales;
        # requant reads X codes + row scales, writes padded transposed codes + block scales
        md_bytes = A * H * 4 + A * 2 * H * 2 + A * 2 * H + A * (2 * H // 128) * 4 + 2 * H * cap + 2 * H * (cap // 128) * 4
        mr_bytes = A * D + A * (D // 128) * 4 + D * cap + (cap // 128) * (D // 128) * 4
        out["components"]["config3_moe_backward_gateup"] = {
            "swiglu_dual_grouped_dh12": {"us": round(md_us, 1), "gbps": round(md_bytes / md_us / 1e3, 1),
                                         "frac_of_hbm": round(md_bytes / md_us / 1e3 / PEAK_HBM_GBPS, 4)},
            "requant_grouped_x": {"us": round(mr_us, 1), "gbps": round(mr_bytes / mr_us / 1e3, 1),
                                  "frac_of_hbm": round(mr_bytes / mr_us / 1e3 / PEAK_HBM_GBPS, 4)},
            "wgrad_grouped_dw12": {"us": round(mw_us, 1), "tflops": round(fl / mw_us / 1e6, 1),
                                   "frac_of_fp8_peak": round(fl / mw_us / 1e6 / PEAK_FP8_TFLOPS, 4)},
            "dgrad_grouped_dx": {"us": round(mg_us, 1), "tflops": round(fl / mg_us / 1e6, 1),
                                 "frac_of_fp8_peak": round(fl / mg_us / 1e6 / PEAK_FP8_TFLOPS, 4)},
        }
    if bwd is not None:
        dq_us = kernel_loop(dual_quant, 20, 3)
        rq_us = kernel_loop(requant, 20, 3)
        bp_us = kernel_loop(bwd_pair, 20, 3)
        dg_us = kernel_loop(dgrad, 20, 3)
        wg_us = kernel_loop(wgrad, 20, 3)
        dq_bytes = M * N * 2 + 2 * M * N + 4 * (M * (N // 128) + N * (M // 128))
        rq_bytes = M * K + M * (K // 128) * 4 + K * M + (M // 128) * (K // 128) * 4
        out["components"]["config4_backward"] = {
            "dual_quant_dy": {"us": round(dq_us, 2), "gbps": round(dq_bytes / dq_us / 1e3, 1),
                              "frac_of_hbm": round(dq_bytes / dq_us / 1e3 / PEAK_HBM_GBPS, 4)},
            "requant_x_block_t": {"us": round(rq_us, 2), "gbps": round(rq_bytes / rq_us / 1e3, 1),
                                  "frac_of_hbm": round(rq_bytes / rq_us / 1e3 / PEAK_HBM_GBPS, 4)},
            "dual_and_requant_one_launch": {"us": round(bp_us, 2),
                                            "gbps": round((dq_bytes + rq_bytes) / bp_us / 1e3, 1),
                                            "frac_of_hbm": round((dq_bytes + rq_bytes) / bp_us / 1e3 / PEAK_HBM_GBPS, 4)},
            "dgrad": {"us": round(dg_us, 1), "tflops": round(flops / dg_us / 1e6, 1),
                      "frac_of_fp8_peak": round(flops / dg_us / 1e6 / PEAK_FP8_TFLOPS, 4)},
            "wgrad": {"us": round(wg_us, 1), "tflops": round(flops / wg_us / 1e6, 1),
                      "frac_of_fp8_peak": round(flops / wg_us / 1e6 / PEAK_FP8_TFLOPS, 4)},
        }
    out["components"]["config1"] = config1_step(dev, args.steps)
    if not args.no_extra:
        out["components"]["config5_training"] = config5_training(dev)
    # each HBM-bound kernel against its own byte mix moved in the friendliest pattern
    comps = out["components"]
    where = {"quant_x_rowwise": comps, "quant_w_blockwise": comps, "quant_fwd_fused": comps,
             "dual_quant_dy": comps.get("config4_backward"), "requant_x_block_t": comps.get("config4_backward"),
             "swiglu_dual_grouped_dh12": comps.get("config3_moe_backward_gateup"),
             "requant_grouped_x": comps.get("config3_moe_backward_gateup")}
    mixes = {k: v for k, v in stream_mixes(nbuf).items() if where.get(k) is not None}
    if "config3_moe_dispatch" in comps:
        mixes.update({k: stream_mixes(nbuf)[k] for k in ("gather_quant", "combine")})
    ceil = stream_mix_ceilings(dev, mixes)
    for k, c in ceil.items():
        if k in ("gather_quant", "combine"):
            d = comps["config3_moe_dispatch"]
            d[f"{k}_traffic_ceiling_gbps"] = c["gbps"]
            d[f"{k}_frac_of_traffic_ceiling"] = round(d[f"{k}_gbps"] / c["gbps"], 4)
        else:
            d = where[k][k]
            d["traffic_ceiling_gbps"] = c["gbps"]
            d["frac_of_traffic_ceiling"] = round(d["gbps"] / c["gbps"], 4)
    out["roofline"]["hbm_traffic_ceilings"] = {
        "what": "bench_ceiling.hip k_stream_mix: each kernel's read : write byte ratio moved in linear "
                "16-byte coalesced order with no arithmetic (best of 4 grids); the rate the HBM "
                "system gives that mix, against which frac_of_traffic_ceiling is taken",
        **ceil}
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline()
    print(json.dumps(out))


if __name__ == "__main__":
    main()
