"""Benchmark of mtlattn on one MI355X, printing ONE JSON line.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]

Headline (BASELINE.json metric): fwd+bwd TFLOP/s of causal GQA prefill,
8 x 4096 tokens, Hq=32, Hkv=8, D=128, bf16 (config C3). One step = the forward
with LSE plus the backward (dQ with the delta row-dot fused in, dK/dV) -- the
work of one autograd step of the op, through the same `_C` calls autograd makes. FLOPs
count attended pairs only (the reference's convention, mtlattn/bench.py:25-32):
fwd 4*D*Hq*pairs, bwd 2.5x that, fwd+bwd 14*D*Hq*pairs. Inputs are synthetic
N(0,1) and resident in HBM before timing. The secondary line item is split-KV
decode HBM GB/s (config C5); the other prefill configs (C1, C2, C4) follow
as fwd+bwd TFLOP/s and fraction of peak under "other_configs".

Per-kernel times: each kernel is launched alone through the C ABI
(mtlattn_amd/capi.py) on torch's current stream, K times back to back between
two HIP events recorded on that same stream; the average launch duration is
the figure. Algorithmic FLOPs per kernel split the 14*D*Hq*pairs of a step by
the products each kernel must do: forward 4 (S, P.V), dK/dV 8 (S, dP, dV, dK),
dQ 2 (dQ; its S and dP recomputation is not algorithmic work), preprocess 0.
"""

import argparse
import json
import math
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2500.0      # MI355X dense bf16 MFMA (spec)
PEAK_FP32_TFLOPS = 157.3       # MI355X fp32 (spec)
PEAK_HBM_GBS = 8000.0          # MI355X HBM3E (spec)
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic.json")

C3 = dict(B=8, L=4096, Hq=32, Hkv=8, D=128)
C3_WORKLOAD = "C3 causal GQA prefill fwd+bwd: 8 seqs x 4096, Hq=32, Hkv=8, D=128, bf16"
C5_WORKLOAD = "C5 split-KV decode: 64 seqs q_len=1, kv U[8192,65536] (seeded), Hq=64, Hkv=8, D=128, bf16"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    # GPU clocks ramp for ~60 ms of sustained load: the default warmup covers it
    ap.add_argument("--warmup", type=int, default=30)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-configs", action="store_true", help="skip the C1/C2/C4 lines")
    ap.add_argument("--no-peaks", action="store_true", help="skip the measured-ceiling kernels")
    ap.add_argument("--only", choices=["c1", "c2", "c3", "c4", "c4nb", "c5", "copy", "peaks", "rates"], default=None,
                    help="run one workload (or the 1 GiB copy used to calibrate HBM byte counters) "
                         "and print only its timing: the short program profilers wrap")
    return ap.parse_args()


def c3_pairs(L=4096, B=8):
    return B * L * (L + 1) // 2


def avg_launch_ms(fn, n, stream):
    """Average duration of `fn` (one kernel launch) over n back-to-back
    launches, from two HIP events recorded on `stream`."""
    import torch
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(n):
        fn()
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / n


def warm(step, min_ms):
    """Runs `step` (synchronised) until at least min_ms of it has run: GPU
    clocks ramp under sustained load."""
    import torch
    t0 = time.perf_counter()
    while True:
        step()
        torch.cuda.synchronize()
        if (time.perf_counter() - t0) * 1e3 >= min_ms:
            return


def step_kernel_ms(calls, n, stream):
    """Average duration of each call in `calls` (one kernel launch each, run
    in order as one step) over n steps, from HIP events recorded on `stream`
    between consecutive launches."""
    import torch
    names = list(calls)
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(len(names) + 1)] for _ in range(n)]
    torch.cuda.synchronize()
    for i in range(n):
        ev[i][0].record(stream)
        for j, name in enumerate(names):
            calls[name]()
            ev[i][j + 1].record(stream)
    torch.cuda.synchronize()
    return {name: sum(ev[i][j].elapsed_time(ev[i][j + 1]) for i in range(n)) / n for j, name in enumerate(names)}


def c3_inputs(seed):
    import torch
    B, L, Hq, Hkv, D = (C3[x] for x in ("B", "L", "Hq", "Hkv", "D"))
    g = torch.Generator().manual_seed(seed)
    M = B * L
    mk = lambda h: torch.randn(M, h, D, generator=g).to(torch.bfloat16)
    q, k, v, do = mk(Hq), mk(Hkv), mk(Hkv), mk(Hq)
    cu = torch.arange(0, M + 1, L, dtype=torch.int32)
    return q, k, v, do, cu


def bench_c3(args):
    import torch
    import mtlattn
    from mtlattn_amd import capi
    C = mtlattn._C
    B, L, Hq, Hkv, D = (C3[x] for x in ("B", "L", "Hq", "Hkv", "D"))
    q, k, v, do, cu = (t.cuda() for t in c3_inputs(args.seed))
    M = B * L
    scale = 1.0 / math.sqrt(D)
    lse = torch.empty(M, Hq, dtype=torch.float32, device="cuda")
    state = {}

    def step():
        state["o"] = C.varlen_attention(q, k, v, cu, cu, L, scale, True, 0, lse, None)
        state["g"] = C.varlen_attention_bwd(q, k, v, state["o"], do, lse, cu, cu, scale, True, 0, None)

    # the same step as four C-ABI calls (one kernel each) on torch's stream;
    # the step proper runs dQ with delta fused in (no preprocess launch), the
    # separate entries time the preprocess and a dQ that reads delta
    stream = torch.cuda.current_stream()
    sh = stream.cuda_stream
    p = capi.problem_for(q, k, cu, cu, L, scale, causal=True)
    rs = Hq * D
    rk = Hkv * D
    delta = torch.empty(M, Hq, dtype=torch.float32, device="cuda")
    dq = torch.empty_like(q)
    dk, dv = torch.empty_like(k), torch.empty_like(v)
    out2 = torch.empty_like(q)
    bf = capi.DTYPE_BF16
    calls = {
        "fwd_mfma": lambda: capi.call("mtlattn_varlen_fwd", p, q.data_ptr(), rs, k.data_ptr(), rk, v.data_ptr(), rk,
                                      out2.data_ptr(), lse.data_ptr(), None, 0, sh),
        "bwd_preprocess": lambda: capi.call("mtlattn_bwd_preprocess", p, out2.data_ptr(), rs, do.data_ptr(), rs,
                                            delta.data_ptr(), sh),
        "bwd_dq": lambda: capi.call("mtlattn_bwd_dq", p, q.data_ptr(), rs, k.data_ptr(), rk, v.data_ptr(), rk,
                                    do.data_ptr(), rs, lse.data_ptr(), delta.data_ptr(), dq.data_ptr(), bf, sh),
        "bwd_dkv": lambda: capi.call("mtlattn_bwd_dkv", p, q.data_ptr(), rs, k.data_ptr(), rk, v.data_ptr(), rk,
                                     do.data_ptr(), rs, lse.data_ptr(), delta.data_ptr(), dk.data_ptr(),
                                     dv.data_ptr(), bf, sh),
    }

    # --warmup steps, and at least 100 ms of steps so the clocks have ramped
    # (as for the other configs)
    for _ in range(args.warmup):
        step()
    warm(step, 100.0)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    # Per-kernel durations, straight after the timed steps (clocks and caches
    # as there): HIP events on the launch stream between the four kernels of
    # each step, over as many steps as the timed region.
    n = args.steps
    kern_ms = step_kernel_ms(calls, n, stream)
    o = state["o"]
    fin = bool(torch.isfinite(o.float()).all().item()) and all(
        bool(torch.isfinite(t.float()).all().item()) for t in state["g"])
    pairs = c3_pairs(L, B)
    unit = D * Hq * pairs
    algo = {"fwd_mfma": 4.0 * unit, "bwd_preprocess": 0.0, "bwd_dq": 2.0 * unit, "bwd_dkv": 8.0 * unit}
    flops = 14.0 * unit
    return {"ms_per_step": wall_ms, "tflops": flops / (wall_ms * 1e-3) / 1e12, "pairs": pairs, "flops": flops,
            "kern_ms": kern_ms, "algo_flop": algo, "launches_timed": n, "finite": fin}


def _attended_pairs(lens, causal, window):
    pairs = 0
    for L in lens:
        if not causal:
            pairs += L * L
        elif window <= 0:
            pairs += L * (L + 1) // 2
        else:
            w = min(L, window)
            pairs += w * (w + 1) // 2 + (L - w) * window
    return pairs


def bench_configs(args, only=None):
    """The other prefill configs of BASELINE.json (C1, C2, C4): fwd+bwd per
    step through `_C`, as for C3. Synthetic N(0,1) inputs generated on the
    device; C2's lengths and C4's bias follow the config sheet."""
    import torch
    import mtlattn
    C = mtlattn._C
    gl = torch.Generator().manual_seed(args.seed)
    c2_lens = torch.randint(256, 4097, (32,), generator=gl).tolist()
    cfgs = [
        ("C1", "fp32 plumbing: lens {17,64,129,250}, Hq=Hkv=4, D=64, non-causal", [17, 64, 129, 250], 4, 4, 64,
         torch.float32, False, 0, False),
        ("C2", "bf16 ragged: 32 seqs, L ~ U[256,4096] (seeded), Hq=Hkv=16, D=64, non-causal", c2_lens, 16, 16, 64,
         torch.bfloat16, False, 0, False),
        ("C4", "bf16 4x16384, Hq=32, Hkv=8, D=128, causal, window 4096, fp32 bias [65536,1,16384] = -(i-j)/16",
         [16384] * 4, 32, 8, 128, torch.bfloat16, True, 4096, True),
    ]
    if only == "C4NB":   # C4's shape without the bias (for the bias's cost; not a bench line)
        cfgs = [("C4NB", "bf16 4x16384, Hq=32, Hkv=8, D=128, causal, window 4096, no bias", [16384] * 4, 32, 8, 128,
                 torch.bfloat16, True, 4096, False)]
    out = {}
    for name, desc, lens, hq, hkv, d, dt, causal, window, with_bias in cfgs:
        if only is not None and name != only:
            continue
        g = torch.Generator(device="cuda").manual_seed(args.seed + 7)
        T = sum(lens)
        q = torch.randn(T, hq, d, device="cuda", generator=g).to(dt)
        k = torch.randn(T, hkv, d, device="cuda", generator=g).to(dt)
        v = torch.randn(T, hkv, d, device="cuda", generator=g).to(dt)
        do = torch.randn(T, hq, d, device="cuda", generator=g).to(dt)
        cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32, device="cuda")
        bias = None
        if with_bias:
            L = lens[0]
            i = torch.arange(L, device="cuda")[:, None]
            j = torch.arange(L, device="cuda")[None, :]
            blk = torch.where(j <= i, -(i - j).float() / 16.0, torch.zeros((), device="cuda"))
            bias = blk.unsqueeze(1).repeat(len(lens), 1, 1)
            del i, j, blk
        lse = torch.empty(T, hq, dtype=torch.float32, device="cuda")
        scale = 1.0 / math.sqrt(d)
        max_q = max(lens)
        st = {}

        def step():
            st["o"] = C.varlen_attention(q, k, v, cu, cu, max_q, scale, causal, window, lse, bias)
            st["g"] = C.varlen_attention_bwd(q, k, v, st["o"], do, lse, cu, cu, scale, causal, window, bias)

        warm(step, 100.0)
        n = max(3, args.steps // 4)
        t0 = time.perf_counter()
        for _ in range(n):
            step()
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / n
        pairs = _attended_pairs(lens, causal, window)
        flops = 14.0 * d * hq * pairs
        tf = flops / (ms * 1e-3) / 1e12
        peak = PEAK_FP32_TFLOPS if dt == torch.float32 else PEAK_BF16_TFLOPS
        out[name] = {"workload": desc, "ms_per_step": round(ms, 4), "tflops": round(tf, 2),
                     "frac_of_peak": round(tf / peak, 4), "peak_tflops": peak, "attended_pairs_per_head": pairs,
                     "steps": n, "dtype": "fp32" if dt == torch.float32 else "bf16"}
        del q, k, v, do, bias, lse, st
        torch.cuda.empty_cache()
    return out


def c5_inputs(seed):
    import torch
    B = 64
    gl = torch.Generator().manual_seed(seed)
    kv_lens = torch.randint(8192, 65537, (B,), generator=gl).tolist()
    return kv_lens


def bench_c5(args):
    import torch
    import mtlattn
    C = mtlattn._C
    B, Hq, Hkv, D = 64, 64, 8, 128
    kv_lens = c5_inputs(args.seed)
    g = torch.Generator().manual_seed(args.seed + 1)
    Mk = sum(kv_lens)
    q = torch.randn(B, Hq, D, generator=g).to(torch.bfloat16).cuda()
    k = torch.empty(Mk, Hkv, D, dtype=torch.bfloat16, device="cuda")
    v = torch.empty(Mk, Hkv, D, dtype=torch.bfloat16, device="cuda")
    gd = torch.Generator(device="cuda").manual_seed(args.seed + 2)
    k.normal_(generator=gd)
    v.normal_(generator=gd)
    cu_q = torch.arange(0, B + 1, dtype=torch.int32, device="cuda")
    cu_kv = torch.tensor([0] + list(torch.tensor(kv_lens).cumsum(0).tolist()), dtype=torch.int32, device="cuda")
    scale = 1.0 / math.sqrt(D)

    def run():
        return C.varlen_attention(q, k, v, cu_q, cu_kv, 1, scale, True, 0, None, None)

    for _ in range(max(3, args.warmup)):
        run()
    warm(run, 100.0)
    ms = avg_launch_ms(run, max(10, args.steps), torch.cuda.current_stream())
    nbytes = Mk * Hkv * D * 2 * 2 + B * Hq * D * 2 * 2
    out = run()
    torch.cuda.synchronize()
    return {"ms": ms, "GBps": nbytes / (ms * 1e-3) / 1e9, "bytes": nbytes, "sum_kv": Mk,
            "finite": bool(torch.isfinite(out.float()).all().item())}


def copy_calibration(args):
    """A plain 1 GiB device-to-device copy: the known-size kernel the HBM byte
    counters (FETCH_SIZE / WRITE_SIZE) are scaled by."""
    import torch
    n = 1 << 30
    a = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
    b = torch.empty_like(a)
    for _ in range(max(1, args.steps)):
        b.copy_(a)
    torch.cuda.synchronize()
    return n


def measured_peaks():
    """Ceilings of this GPU measured with the calibration kernels
    (mtlattn_amd/csrc/calib.hip): sustained bf16 MFMA throughput of a
    register-only v_mfma_f32_32x32x16 stream on every CU, and HBM read
    bandwidth of a 4 GiB 16-byte-load stream; each after 100 ms of warm-up,
    then 10 launches between HIP events. Also the shader clock of the first
    wave during each (s_memtime cycles over s_memrealtime 100 MHz ticks)."""
    import ctypes
    import torch
    lib = ctypes.CDLL(os.path.join(ROOT, "mtlattn_amd", "libmtlattn_calib.so"))
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    lib.mtlattn_calib_mfma.argtypes = [ctypes.c_int, ctypes.c_int, vp, vp, vp]
    lib.mtlattn_calib_read.argtypes = [vp, i64, ctypes.c_int, vp, vp, vp]
    stream = torch.cuda.current_stream()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    clk = torch.zeros(2, dtype=torch.int64, device="cuda")

    def mhz():
        c = clk.cpu().tolist()
        return round(c[0] / (c[1] / 100.0), 1) if c[1] > 0 else None

    blocks, iters = cus * 4, 2048
    sink = torch.empty(blocks * 512, dtype=torch.float32, device="cuda")
    run = lambda: lib.mtlattn_calib_mfma(blocks, iters, sink.data_ptr(), clk.data_ptr(), stream.cuda_stream)
    warm(run, 100.0)
    ms = avg_launch_ms(run, 10, stream)
    mfma_tf = blocks * 8 * iters * 8 * 32768.0 / (ms * 1e-3) / 1e12
    mfma_mhz = mhz()
    nbytes = 4 << 30
    buf = torch.ones(nbytes // 4, dtype=torch.int32, device="cuda")
    rblocks = cus * 8
    rsink = torch.empty(rblocks * 4, dtype=torch.int32, device="cuda")
    run = lambda: lib.mtlattn_calib_read(buf.data_ptr(), nbytes, rblocks, rsink.data_ptr(), clk.data_ptr(),
                                         stream.cuda_stream)
    warm(run, 100.0)
    ms_r = avg_launch_ms(run, 10, stream)
    read_gbs = nbytes / (ms_r * 1e-3) / 1e9
    read_mhz = mhz()
    del buf
    torch.cuda.empty_cache()
    return {"mfma_bf16_tflops": round(mfma_tf, 1), "mfma_clock_mhz": mfma_mhz,
            "hbm_read_gbs": round(read_gbs, 1), "read_clock_mhz": read_mhz, "cus": cus,
            "how": "calib.hip: register-only v_mfma_f32_32x32x16_bf16 stream (4 chains, 8 waves per CU-block, "
                   f"{blocks} blocks) and a 4 GiB read stream (16-byte nontemporal loads, {rblocks} blocks "
                   "of contiguous spans); "
                   "HIP events over 10 launches after 100 ms warm-up"}


def issue_rates():
    """Per-SIMD issue rates measured with the rate probes of
    mtlattn_amd/csrc/calib.hip: one block of 8 waves per CU, waves 0-3 in one
    role and waves 4-7 (the other wave of each SIMD) in another. For each
    pairing, the shader cycles per instruction of each side and the clock."""
    import ctypes
    import torch
    lib = ctypes.CDLL(os.path.join(ROOT, "mtlattn_amd", "libmtlattn_calib.so"))
    vp = ctypes.c_void_p
    lib.mtlattn_calib_rates.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, vp, vp, vp]
    lib.mtlattn_calib_rate_ops.argtypes = [ctypes.c_int]
    names = {0: "idle", 1: "v_exp_f32", 2: "v_fmac_f32", 3: "mfma32x32x16 (VGPR acc)", 4: "mfma32x32x16 (AGPR acc)",
             5: "ds_read_b128", 6: "mfma + 2 v_exp + 2 v_fmac (one wave)", 7: "mfma + 4 v_exp (one wave)",
             8: "mfma (LDS operand) + 2 v_exp + 2 v_fmac (one wave)",
             9: "mfma + softmax chain: 2 fma->exp, cvt, dot2 (one wave)",
             10: "global_load_lds_dwordx4 (1 KB, L2-resident)",
             11: "mfma + 1 direct load per 4 MFMAs (one wave)",
             12: "mfma (LDS operand shared by 2 MFMAs) + 2 v_exp + 2 v_fmac (one wave)"}
    iters = {1: 2000, 2: 4000, 3: 1000, 4: 1000, 5: 1000, 6: 1000, 7: 1000, 8: 1000, 9: 1000, 10: 1000, 11: 1000,
             12: 1000}
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    sink = torch.empty(cus * 512, dtype=torch.float32, device="cuda")
    cyc = torch.zeros(cus * 16, dtype=torch.int64, device="cuda")
    stream = torch.cuda.current_stream()
    pairs = [(1, 0), (1, 1), (2, 0), (2, 2), (3, 0), (4, 0), (3, 3), (4, 4), (3, 1), (4, 1), (3, 2), (4, 2),
             (5, 0), (5, 5), (3, 5), (6, 0), (7, 0), (6, 6), (7, 7), (6, 3),
             (8, 0), (8, 8), (9, 0), (9, 9), (10, 0), (10, 10), (3, 10), (11, 0), (11, 11), (12, 0), (12, 12)]
    out = []
    for ra, rb in pairs:
        n = max(iters.get(ra, 1), iters.get(rb, 1))
        for _ in range(3):   # the first launches run while the clock ramps
            rc = lib.mtlattn_calib_rates(ra, rb, n, cus, sink.data_ptr(), cyc.data_ptr(), stream.cuda_stream)
            assert rc == 0, rc
        torch.cuda.synchronize()
        c = cyc.view(cus, 8, 2).double()
        side = []
        for role, waves in ((ra, slice(0, 4)), (rb, slice(4, 8))):
            if role == 0:
                side.append(None)
                continue
            cycles = c[:, waves, 0].mean().item()
            ops = n * lib.mtlattn_calib_rate_ops(role)
            side.append({"role": names[role], "cycles_per_instr": round(cycles / ops, 2)})
        ticks = c[:, 0:4, 1].mean().item() if ra else c[:, 4:8, 1].mean().item()
        cyc_a = c[:, 0:4, 0].mean().item() if ra else c[:, 4:8, 0].mean().item()
        out.append({"waves_0_3": side[0], "waves_4_7": side[1], "iters": n,
                    "clock_mhz": round(cyc_a / (ticks / 100.0), 0) if ticks > 0 else None})
    return {"cus": cus, "pairs": out,
            "how": "calib.hip calib_rates_kernel: inline-asm streams, one 8-wave block per CU, "
                   "s_memtime cycles per wave over the instruction count; third of three launches"}


def host_cpu():
    """Model, sockets and physical cores of the host (from /proc/cpuinfo),
    the CPUs this process may run on, and the torch thread count used: the
    OMP_NUM_THREADS the GPU host sets (its CPU share for one GPU), else the
    CPUs available, at most 16."""
    info = {"model": platform.processor() or platform.machine(), "sockets": None, "physical_cores": None}
    try:
        with open("/proc/cpuinfo") as f:
            blocks = f.read().split("\n\n")
        phys, cores = set(), {}
        for b in blocks:
            kv = dict(l.split(":", 1) for l in b.splitlines() if ":" in l)
            kv = {k.strip(): v.strip() for k, v in kv.items()}
            if "model name" in kv:
                info["model"] = kv["model name"]
            if "physical id" in kv:
                phys.add(kv["physical id"])
                if "core id" in kv:
                    cores.setdefault(kv["physical id"], set()).add(kv["core id"])
        if phys:
            info["sockets"] = len(phys)
            info["physical_cores"] = sum(len(c) for c in cores.values()) or None
    except OSError:
        pass
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count() or 1
    info["logical_cpus"] = os.cpu_count()
    info["cpus_available"] = avail
    omp = os.environ.get("OMP_NUM_THREADS", "")
    info["threads"] = min(int(omp), avail) if omp.isdigit() and int(omp) > 0 else min(16, avail)
    info["threads_from"] = "OMP_NUM_THREADS" if omp.isdigit() and int(omp) > 0 else "min(16, cpus available)"
    return info


def cpu_baseline_others(seed, threads, budget_s=3.0):
    """The oracle on bounded samples of C1 (whole), C2 (sequences until the
    budget), C4 (query blocks of one sequence until the budget) and C5
    (forward of sequences until the budget), each reported in its metric's
    unit: TFLOP/s of attended-pair FLOPs, or GB/s of C5's algorithmic bytes."""
    import torch
    import oracle
    torch.set_num_threads(threads)
    out = {}
    g = torch.Generator().manual_seed(seed + 7)

    def timed(fn):
        t0 = time.perf_counter()
        fn()
        return time.perf_counter() - t0

    # C1: fp32 fwd+bwd, whole config
    lens = [17, 64, 129, 250]
    T = sum(lens)
    q, k, v, do = (torch.randn(T, 4, 64, generator=g) for _ in range(4))
    cu = torch.tensor([0, 17, 81, 210, 460], dtype=torch.int32)
    dt = timed(lambda: oracle.varlen_forward_backward(q, k, v, do, cu, cu))
    pairs = sum(L * L for L in lens)
    out["C1"] = {"value": round(14.0 * 64 * 4 * pairs / dt / 1e12, 5), "unit": "TFLOP/s",
                 "sample": f"whole config, fp32 fwd+bwd, {dt:.2f} s"}
    # C2: bf16 inputs, ragged non-causal D=64, sequences until the budget
    gl = torch.Generator().manual_seed(seed)
    c2 = torch.randint(256, 4097, (32,), generator=gl).tolist()
    T = sum(c2)
    q, k, v, do = (torch.randn(T, 16, 64, generator=g).to(torch.bfloat16) for _ in range(4))
    cu = torch.tensor([0] + torch.tensor(c2).cumsum(0).tolist(), dtype=torch.int32)
    done, t0 = [], time.perf_counter()
    for s in range(32):
        oracle.varlen_forward_backward_blocked(q, k, v, do, cu, cu, seqs=[s], q_block=1024)
        done.append(s)
        if time.perf_counter() - t0 >= budget_s:
            break
    dt = time.perf_counter() - t0
    pairs = sum(c2[s] ** 2 for s in done)
    out["C2"] = {"value": round(14.0 * 64 * 16 * pairs / dt / 1e12, 5), "unit": "TFLOP/s",
                 "sample": f"{len(done)} of 32 sequences fwd+bwd, {dt:.2f} s"}
    del q, k, v, do
    # C4: one sequence of 16384, window 4096, fp32 bias -(i-j)/16, query
    # blocks of 1024 from the start until the budget
    L, W, D = 16384, 4096, 128
    q = torch.randn(L, 32, D, generator=g).to(torch.bfloat16)
    k = torch.randn(L, 8, D, generator=g).to(torch.bfloat16)
    v = torch.randn(L, 8, D, generator=g).to(torch.bfloat16)
    do = torch.randn(L, 32, D, generator=g).to(torch.bfloat16)
    i = torch.arange(L)[:, None]
    rows, t0, pairs = 0, time.perf_counter(), 0
    while rows < L:
        n = min(1024, L - rows)
        cq = torch.tensor([0, n], dtype=torch.int32)
        kv0 = max(0, rows - W + 1)
        ck = torch.tensor([0, rows + n - kv0], dtype=torch.int32)
        qi = i[rows:rows + n]
        j = torch.arange(kv0, rows + n)[None, :]
        b = torch.where(j <= qi, -(qi - j).float() / 16.0, torch.zeros(())).unsqueeze(1)
        oracle.varlen_forward_backward_blocked(q[rows:rows + n], k[kv0:rows + n], v[kv0:rows + n], do[rows:rows + n],
                                               cq, ck, 1 / math.sqrt(D), True, W, b, q_block=1024)
        pairs += sum(min(r + 1, W) for r in range(rows, rows + n))
        rows += n
        if time.perf_counter() - t0 >= budget_s:
            break
    dt = time.perf_counter() - t0
    out["C4"] = {"value": round(14.0 * D * 32 * pairs / dt / 1e12, 5), "unit": "TFLOP/s",
                 "sample": f"first {rows} of 65536 query rows (sequence 0, its key band and bias), fwd+bwd, "
                           f"{dt:.2f} s"}
    del q, k, v, do
    # C5: decode forward, sequences until the budget (oracle time only)
    kv_lens = c5_inputs(seed)
    dt, done_kv, n = 0.0, 0, 0
    for L in kv_lens:
        q = torch.randn(1, 64, D, generator=g).to(torch.bfloat16)
        k = torch.randn(L, 8, D, generator=g).to(torch.bfloat16)
        v = torch.randn(L, 8, D, generator=g).to(torch.bfloat16)
        cq, ck = torch.tensor([0, 1], dtype=torch.int32), torch.tensor([0, L], dtype=torch.int32)
        dt += timed(lambda: oracle.varlen_forward_backward_blocked(q, k, v, None, cq, ck, 1 / math.sqrt(D), True,
                                                                   backward=False, q_block=1))
        done_kv += L
        n += 1
        if dt >= budget_s:
            break
    nbytes = done_kv * 8 * D * 2 * 2 + n * 64 * D * 2 * 2
    out["C5"] = {"value": round(nbytes / dt / 1e9, 3), "unit": "GB/s",
                 "sample": f"{n} of 64 sequences (sum kv {done_kv}), forward, {dt:.2f} s"}
    return out


def cpu_baseline(seed, budget_s=12.0):
    """The oracle (torch CPU fp32, explicit fwd+bwd formulas) on C3, one
    sequence (all 8 kv heads, 32 query heads) at a time until `budget_s` of
    CPU time is spent: a bounded sample of the same workload."""
    import torch
    import oracle
    host = host_cpu()
    threads = host["threads"]
    torch.set_num_threads(threads)
    B, L, Hq, Hkv, D = (C3[x] for x in ("B", "L", "Hq", "Hkv", "D"))
    q, k, v, do, cu = c3_inputs(seed)
    done = 0
    t0 = time.perf_counter()
    for s in range(B):
        oracle.varlen_forward_backward_blocked(q, k, v, do, cu, cu, causal=True, seqs=[s], q_block=512)
        done += 1
        if time.perf_counter() - t0 >= budget_s:
            break
    dt = time.perf_counter() - t0
    sample_pairs = L * (L + 1) // 2 * done
    flops = 14.0 * D * Hq * sample_pairs
    return {"value": round(flops / dt / 1e12, 5), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": f"C3 fwd+bwd, {done} of {B} sequences (all 32 query heads), "
                      f"{sample_pairs * Hq} attended pairs, {dt:.1f} s; oracle "
                      f"varlen_forward_backward_blocked fp32, torch {threads} threads",
            "host": host, "other_configs": cpu_baseline_others(seed, threads)}


def load_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 --pmc
    summary (FETCH_SIZE, WRITE_SIZE scaled by the copy calibration)."""
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
        return t["kernels"][kernel]["hbm_bytes"]
    except (OSError, KeyError, ValueError):
        return None


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "how the path shards over GPUs is documented, not run.", file=sys.stderr)
        sys.exit(2)
    import torch
    assert torch.cuda.is_available(), "bench.py needs a HIP device"
    if args.only == "copy":
        n = copy_calibration(args)
        print(json.dumps({"copy_bytes": n, "launches": max(1, args.steps)}), flush=True)
        return
    if args.only == "c3":
        c3 = bench_c3(args)
        print(json.dumps({"c3_ms_per_step": c3["ms_per_step"], "tflops": c3["tflops"],
                          "kern_ms": c3["kern_ms"]}), flush=True)
        return
    if args.only == "c5":
        dec = bench_c5(args)
        print(json.dumps({"c5_ms": dec["ms"], "GBps": dec["GBps"]}), flush=True)
        return
    if args.only in ("c1", "c2", "c4", "c4nb"):
        print(json.dumps(bench_configs(args, args.only.upper())), flush=True)
        return
    if args.only == "peaks":
        print(json.dumps(measured_peaks()), flush=True)
        return
    if args.only == "rates":
        print(json.dumps(issue_rates()), flush=True)
        return
    c3 = bench_c3(args)
    dec = None if args.no_decode else bench_c5(args)
    others = None if args.no_configs else bench_configs(args)
    peaks = None if args.no_peaks else measured_peaks()
    cpu = None if args.no_cpu_baseline else cpu_baseline(args.seed)
    km, algo = c3["kern_ms"], c3["algo_flop"]
    dom = max(km, key=km.get)
    ach = algo[dom] / (km[dom] * 1e-3) / 1e12
    line = {
        "metric": "fwd+bwd TFLOP/s causal GQA 8x4096 D128 bf16; split-KV decode HBM GB/s",
        "value": round(c3["tflops"], 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(c3["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic N(0,1), seeded",
        "config": {"workload": C3_WORKLOAD, "global_batch": C3["B"], "seq_len": C3["L"],
                   "parallelism": "single GPU", "attended_pairs_per_head": c3["pairs"],
                   "flop_per_step": c3["flops"]},
        "roofline": {"bound": "mfma", "achieved": round(ach, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(ach / PEAK_BF16_TFLOPS, 4), "traffic": load_traffic(dom), "kernel": dom,
                     "kernel_ms": round(km[dom], 4), "algorithmic_flop": algo[dom],
                     "peak_measured": None if peaks is None else peaks["mfma_bf16_tflops"],
                     "frac_measured": None if peaks is None else round(ach / peaks["mfma_bf16_tflops"], 4),
                     "step_frac": round(c3["tflops"] / PEAK_BF16_TFLOPS, 4),
                     "step_frac_measured": None if peaks is None else round(c3["tflops"] / peaks["mfma_bf16_tflops"],
                                                                             4)},
        "measured_peaks": peaks,
        "kernels": {n: {"ms": round(t, 4),
                        "tflops": round(algo[n] / (t * 1e-3) / 1e12, 2) if algo[n] else None}
                    for n, t in km.items()},
        "decode": None if dec is None else {
            "workload": C5_WORKLOAD,
            "ms": round(dec["ms"], 4), "GBps": round(dec["GBps"], 1), "bytes": dec["bytes"],
            "roofline": {"bound": "hbm", "achieved": round(dec["GBps"], 1), "peak": PEAK_HBM_GBS,
                         "unit": "GB/s", "frac": round(dec["GBps"] / PEAK_HBM_GBS, 4),
                         "peak_measured": None if peaks is None else peaks["hbm_read_gbs"],
                         "frac_measured": None if peaks is None else round(dec["GBps"] / peaks["hbm_read_gbs"], 4)},
            "outputs_finite": dec["finite"]},
        "other_configs": others,
        "outputs_finite": c3["finite"],
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
