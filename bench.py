"""Headline benchmark: effective TOPS of the full `sageattn` call on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload c3c] [--no-cpu]

A "step" is one full call (K/V prologue + main loop, Q quantized in the main loop) on synthetic
inputs already resident in HBM. The default workload is BASELINE's headline, configs[2]: fp16,
B=1, H=48, N=47520, D=128, causal, smooth_k on, HND. Ops convention 4*B*H*N^2*D, halved when
causal (the reference's `bench/bench_attention.py:140`).

The method follows the reference's (`docs/METHOD.md:14-45`, `bench/bench_attention.py:49-58`):
1. W untimed warm-up calls, then an untimed clock-settling phase by time: at least `--settle`
   seconds (default 4) and 40 calls, continued in half-second chunks while the shader clock still
   rises (at most 10 s). Recorded as `settle` (calls, seconds, the clock readings, and the board
   power and power cap at its end, `board_power`: the card lowers its clock to hold the cap).
2. The timed region: exactly K calls of the public `sageattn(...)` (with `--kernel` other than 0,
   of `sk1_forward` with that kernel), bracketed by device synchronizations, with the shader
   clock read before and after. `ms_per_step` and `value` come from it.
3. An A/A twin: the same call timed as two candidates over 10 interleaved rounds (order rotated
   each round, one HIP event pair per batch of calls); `aa_ratio` = median B / median A, whose
   distance from 1 is the noise floor of this run.
4. The prologue/main-loop split: K calls of `sk1_forward` with HIP events on the launch stream
   between its launches.
5. The MFMA ceiling at this run's clock: the library's register-resident probe
   (`sage_mfma_peak_probe`, int8 and e4m3), reported as `measured_peak` beside the documented
   5.0 POPS.

Prints ONE JSON line. Besides the contract fields it carries
* `roofline`: the main-loop kernel's achieved TFLOP/s (algorithmic ops per launch / its mean
  launch duration from step 4) against the int8/fp8 dense MFMA peak, and against the measured
  one (`frac_of_measured`); `traffic` is its HBM bytes per launch from the committed rocprofv3
  FETCH_SIZE/WRITE_SIZE summary for the workload (null when none is committed);
* `prologue`: the prologue pair's achieved HBM GB/s on its algorithmic bytes (K read twice with
  smooth_k: once for the mean, once to quantize), and `frac_single_read`, the same time against
  the bytes of one K read (the prologue's byte floor);
* `cpu_baseline`: the CPU emulation of the reference scheme (`oracle/`, a "port") and torch CPU
  SDPA, timed on a bounded sample of the same workload on this host's cores;
* `first_call`: a fresh child process's import, library load and first call of the workload's
  shape (the reference quotes its first call in a fresh process, `README.md:77-79`).
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "sageattention-rdna4_amd"))

METRIC = "effective TOPS (full call incl. quant) fp16 B1 H48 D128 N47520 causal; % MFMA peak"
PEAK_TOPS = 5000.0          # MI355X dense int8 (5.0 POPS) and fp8 (5.0 PFLOP/s) MFMA peak
HBM_PEAK_GBPS = 8000.0
# s_memrealtime's rate on MI355X (hipDeviceAttributeWallClockRate reads 100000 kHz; a probe's
# tick span over its event-timed launch measured 99.8-99.96 MHz)
REALTIME_MHZ = 100.0

WORKLOADS = {
    # name: (dtype, B, H, N, causal, layout, k_offset_std, outlier_frac, std[, head_dim])
    "c3c": ("fp16", 1, 48, 47520, True, "HND", 2.0, 0.0, 1.0),     # headline (configs[2], causal)
    "c3n": ("fp16", 1, 48, 47520, False, "HND", 2.0, 0.0, 1.0),
    "c2c": ("fp16", 1, 48, 8771, True, "HND", 2.0, 0.001, 1.0),
    "c2n": ("fp16", 1, 48, 8771, False, "HND", 2.0, 0.001, 1.0),
    "c4": ("bf16", 1, 48, 16384, True, "HND", 2.0, 0.001, 1.5),
    "c1": ("fp16", 1, 48, 1024, False, "HND", 2.0, 0.0, 1.0),
    "c5_288": ("fp16", 1, 48, 288, False, "HND", 0.0, 0.0, 1.0),
    "c5_4096": ("fp16", 1, 48, 4096, False, "HND", 0.0, 0.0, 1.0),
    "c5_b8": ("fp16", 8, 24, 4096, False, "NHD", 0.0, 0.0, 1.0),
    # head_dim 64: the reference's F165 shapes (SDXL 1024^2 level 1, CogVideoX-2B) and the
    # headline length
    "d64_sdxl": ("fp16", 1, 10, 4096, False, "HND", 2.0, 0.0, 1.0, 64),
    "d64_cogvx": ("fp16", 1, 30, 17550, False, "HND", 2.0, 0.0, 1.0, 64),
    "d64_c3c": ("fp16", 1, 48, 47520, True, "HND", 2.0, 0.0, 1.0, 64),
}


def head_dim(wl):
    return wl[9] if len(wl) > 9 else 128


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def make_inputs(wl, seed=0):
    import torch
    dt, B, H, N, causal, layout, off, outl, std = wl[:9]
    D = head_dim(wl)
    dtype = torch.float16 if dt == "fp16" else torch.bfloat16
    g = torch.Generator().manual_seed(seed)
    out = []
    for i in range(3):
        x = torch.randn(B, H, N, D, generator=g, dtype=torch.float32)
        if std != 1.0:
            x.mul_(std)
        if i == 1 and off:
            x.add_(torch.randn(B, H, 1, D, generator=g) * off)
        if i == 1 and outl:
            n_out = int(round(outl * N))
            for b in range(B):
                for h in range(H):
                    idx = torch.randperm(N, generator=g)[:n_out]
                    x[b, h, idx] *= 50.0
        x = x.to(dtype)
        if layout == "NHD":
            x = x.transpose(1, 2).contiguous()
        out.append(x)
    return out


def ops_of(B, H, N, causal, D=128):
    return 4.0 * B * H * N * N * D * (0.5 if causal else 1.0)


def prologue_bytes(B, H, N, smooth_k=True, D=128):
    """Algorithmic HBM bytes of the prologue pair: K read twice (mean + quant) when smooth_k, V read
    once, K8 and V8T written, SK and SV written, SV read and rewritten by the fold."""
    n_pad = (N + 63) // 64 * 64
    el = B * H * N * D * 2
    q8 = B * H * n_pad * D
    return (2 if smooth_k else 1) * el + el + 2 * q8 + 4 * B * H * n_pad * 4


def profiled_traffic(workload):
    """HBM bytes per main-loop launch for `workload`, from the committed rocprofv3 summary
    (FETCH_SIZE and WRITE_SIZE scaled by a plain copy; see profiles/), or None."""
    import re
    path = os.path.join(ROOT, "profiles", "attn_fwd_%s_hbm_traffic.md" % workload)
    if not os.path.exists(path):
        return None
    pat = re.compile(r"^traffic_bytes_per_launch\[%s\] = (\d+)$" % re.escape(workload))
    with open(path) as f:
        for line in f:
            m = pat.match(line.strip())
            if m:
                return int(m.group(1))
    return None


def cpu_baseline(wl, q, k, v, budget_s=20.0):
    """Time the oracle (CPU emulation of the reference scheme) and torch CPU SDPA on a bounded
    sample of the workload: plane 0, the last `rows` query rows (the longest causal rows), with the
    sample's prologue (mean, K/V quantization, fold) included."""
    import torch
    import torch.nn.functional as F
    sys.path.insert(0, ROOT)
    import oracle
    dt, B, H, N, causal, layout, *_ = wl
    qh, kh, vh = (oracle.to_hnd(t, layout)[0:1, 0:1].contiguous() for t in (q, k, v))
    n_pad = oracle.n_pad_for(N)
    D = head_dim(wl)
    sm = D ** -0.5
    int8 = dt == "fp16"

    def run(rows):
        r0 = N - rows
        t0 = time.perf_counter()
        kr, vr, qr = kh[0], vh[0], qh[0]
        mean = oracle.kseq_mean(kr)
        k8, sk = oracle.quant_k(kr, n_pad, mean=mean, int8=int8)
        v8t, sv = oracle.quant_v(vr, n_pad)
        s, svp = oracle.fold_v_scale(sv)
        q8, sq, cq = oracle.quant_q(qr[:, r0:], sm, int8=int8)
        oracle.attention_tiles(q8, cq, k8, sk, v8t, svp, s, N, causal, q.dtype, row0=r0)
        t_emu = time.perf_counter() - t0
        t0 = time.perf_counter()
        qs = qr[:, r0:].float()
        if causal:
            mask = torch.arange(N)[None, :] <= torch.arange(r0, N)[:, None]
            F.scaled_dot_product_attention(qs, kr.float(), vr.float(), attn_mask=mask)
        else:
            F.scaled_dot_product_attention(qs, kr.float(), vr.float())
        t_sdpa = time.perf_counter() - t0
        ops = sum(4.0 * D * ((r + 1) if causal else N) for r in range(r0, N))
        return ops, t_emu, t_sdpa

    # Two short runs fix the sample's fixed cost (the plane's prologue) and its cost per query row;
    # the timed run is then sized to take about `budget_s` seconds of CPU.
    _, te1, ts1 = run(64)
    _, te2, ts2 = run(192)
    per_row = max((te2 + ts2 - te1 - ts1) / 128.0, 1e-6)
    fixed = max(te1 + ts1 - 64 * per_row, 0.0)
    rows = int(min(N, max(64.0, (budget_s - fixed) / per_row)) // 64 * 64) or 64
    ops, te, ts = run(rows)
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return dict(value=ops / te / 1e9, unit="GOPS", cores=torch.get_num_threads(), kind="port",
                cpu_model=model, torch_version=torch.__version__,
                sample="plane 0 of %d, last %d query rows of N=%d%s, with that plane's prologue; "
                       "ops %.3e, emulation %.2f s" % (B * H, rows, N, " (causal)" if causal else "",
                                                       ops, te),
                sdpa_cpu_gops=ops / ts / 1e9, sdpa_cpu_s=ts, host_cpus=os.cpu_count())


def sclk_mhz():
    """The GPU's current shader clock in MHz, read from sysfs (`pp_dpm_sclk`, where the current
    level carries a `*`): a plain file read, so no other program is started from this process.
    None where it is unavailable. With several AMD cards it reports the first one that has it."""
    import glob
    import re
    for path in sorted(glob.glob("/sys/class/drm/card*/device/pp_dpm_sclk")):
        try:
            with open(path) as f:
                for line in f:
                    if "*" in line:
                        m = re.search(r"(\d+)\s*Mhz", line, re.IGNORECASE)
                        if m:
                            return int(m.group(1))
        except OSError:
            continue
    return None


def board_power(root="/sys/class/drm"):
    """The board's power draw and power cap in W, read from sysfs hwmon (`power1_average`, else
    `power1_input`; `power1_cap`; microwatts): plain file reads. None for what is unreadable; with
    several AMD cards, the first one that reports a power draw."""
    import glob

    def read_w(path):
        try:
            with open(path) as f:
                return int(f.read().strip()) / 1e6
        except (OSError, ValueError):
            return None
    for d in sorted(glob.glob(os.path.join(root, "card*", "device", "hwmon", "hwmon*"))):
        draw = read_w(os.path.join(d, "power1_average"))
        if draw is None:
            draw = read_w(os.path.join(d, "power1_input"))
        if draw is not None:
            return {"watts": round(draw, 1), "cap_watts": read_w(os.path.join(d, "power1_cap"))}
    return None


def settle(call, sync, *, min_calls=40, min_s=4.0, max_s=10.0, chunk_s=0.5, max_calls=20000,
           clock=None, now=time.perf_counter):
    """Untimed clock settling by time, not by call count (the reference's rule,
    `docs/METHOD.md:23-25`): calls (each followed by `sync`) until at least `min_calls` calls and
    `min_s` seconds have passed, then on in `chunk_s` chunks while the shader clock reading still
    rises, until `max_s`; `max_calls` caps the count so a call that returns at once cannot spin
    forever. Returns the calls made, the seconds spent and the clock readings (MHz, None where
    unreadable) at the start, after the floor and after each chunk."""
    clock = clock or sclk_mhz
    t0 = now()
    trace = [clock()]
    n = 0
    while (n < min_calls or now() - t0 < min_s) and n < max_calls:
        call()
        sync()
        n += 1
    trace.append(clock())
    while now() - t0 < max_s and n < max_calls:
        t1 = now()
        while now() - t1 < chunk_s and n < max_calls:
            call()
            sync()
            n += 1
        trace.append(clock())
        if trace[-2] is None or trace[-1] is None or trace[-1] <= trace[-2]:
            break
    return {"calls": n, "seconds": round(now() - t0, 3), "sclk_mhz": trace}


def aa_twin(call, make_event, sync, *, rounds=10, batch=5):
    """The A/A twin (`docs/METHOD.md:14-22`): the same call measured as two candidates, A and B,
    over `rounds` interleaved rounds with the order swapped every round; each measurement is one
    event pair around a batch of `batch` calls. Returns both medians (ms per call), their ratio
    B/A (whose distance from 1 is the run's noise floor) and each candidate's min-max."""
    import statistics
    res = {"A": [], "B": []}
    for r in range(rounds):
        for name in (("A", "B") if r % 2 == 0 else ("B", "A")):
            e0, e1 = make_event(), make_event()
            e0.record()
            for _ in range(batch):
                call()
            e1.record()
            sync()
            res[name].append(e0.elapsed_time(e1) / batch)
    ma, mb = statistics.median(res["A"]), statistics.median(res["B"])
    return {"rounds": rounds, "batch": batch, "ms_a": round(ma, 4), "ms_b": round(mb, 4),
            "ratio": round(mb / ma, 4),
            "range_a": [round(min(res["A"]), 4), round(max(res["A"]), 4)],
            "range_b": [round(min(res["B"]), 4), round(max(res["B"]), 4)]}


def mfma_peak(lib, qk_int8, make_event, sync, *, target_ms=25.0, reps=5):
    """The dense MFMA rate at this run's clock, from the library's register-resident probe: one
    short launch sizes the iteration count to about `target_ms` per launch, then `reps` launches
    are timed with event pairs. Returns TOPS of the median launch and the shader clock (MHz) its
    first wave ran at."""
    import statistics
    import torch
    blocks = 4 * torch.cuda.get_device_properties(0).multi_processor_count

    clocks = torch.zeros(2, dtype=torch.int64, device="cuda:0")

    def timed(iters):
        e0, e1 = make_event(), make_event()
        e0.record()
        ops = lib.mfma_peak_probe(qk_int8, blocks, iters, clocks)
        e1.record()
        sync()
        cyc, ticks = (int(x) for x in clocks.cpu())
        return ops, e0.elapsed_time(e1), cyc, ticks

    timed(2000)                  # the first launch also pays its code object's first use
    _, ms, _, _ = timed(2000)
    iters = max(2000, int(2000 * target_ms / max(ms, 1e-3)))
    runs = sorted((timed(iters) for _ in range(reps)), key=lambda r: r[1])
    ops, ms, cyc, ticks = runs[len(runs) // 2]
    # the first wave's shader-clock cycles over its constant-rate ticks (s_memrealtime counts at
    # REALTIME_MHZ) give the clock the matrix cores ran at
    mhz = cyc / ticks * REALTIME_MHZ if ticks else None
    return ops / (ms * 1e-3) / 1e12, mhz


def copy_calibration(mib, reps):
    """A plain device-to-device copy of `mib` MiB, `reps` times: each launch reads and writes
    exactly mib MiB, which calibrates what the HBM counters report per algorithmic byte."""
    import torch
    n = mib * (1 << 20)
    src = torch.empty(n, dtype=torch.uint8, device="cuda:0").fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_per_launch": n, "reps": reps}), flush=True)
    return 0


def first_call_child(workload):
    """Run in a fresh child process: time the import of torch, the import of the package, the
    library load, and the first and second `sageattn` calls of `workload`'s shape (inputs made on
    the GPU, outside the timed calls). Prints one JSON line."""
    t0 = time.perf_counter()
    import torch
    t1 = time.perf_counter()
    from sageattention import sageattn
    from sageattention.sk1_backend import SageLib
    t2 = time.perf_counter()
    SageLib.get()
    t3 = time.perf_counter()
    dt, B, H, N, causal, layout, *_ = WORKLOADS[workload]
    D = head_dim(WORKLOADS[workload])
    shape = (B, H, N, D) if layout == "HND" else (B, N, H, D)
    dtype = torch.float16 if dt == "fp16" else torch.bfloat16
    q, k, v = (torch.randn(shape, device="cuda:0", dtype=dtype) for _ in range(3))
    torch.cuda.synchronize()
    t4 = time.perf_counter()
    sageattn(q, k, v, tensor_layout=layout, is_causal=causal, smooth_k=True)
    torch.cuda.synchronize()
    t5 = time.perf_counter()
    sageattn(q, k, v, tensor_layout=layout, is_causal=causal, smooth_k=True)
    torch.cuda.synchronize()
    t6 = time.perf_counter()
    print(json.dumps({"import_torch_s": round(t1 - t0, 4), "import_package_s": round(t2 - t1, 4),
                      "library_load_s": round(t3 - t2, 4), "first_call_s": round(t5 - t4, 4),
                      "second_call_s": round(t6 - t5, 4),
                      "import_to_first_result_s": round((t1 - t0) + (t3 - t1) + (t5 - t4), 4)}),
          flush=True)
    return 0


def first_call_latency(workload, timeout_s=600):
    """`first_call_child` in a fresh process (started before this process touches the GPU), or
    the reason it could not be measured."""
    import subprocess
    try:
        res = subprocess.run([sys.executable, os.path.abspath(__file__), "--first-call-child",
                              "--workload", workload], capture_output=True, text=True,
                             timeout=timeout_s)
    except subprocess.TimeoutExpired:
        return {"error": "timed out after %d s" % timeout_s}
    lines = [ln for ln in res.stdout.splitlines() if ln.startswith("{")]
    if res.returncode != 0 or not lines:
        return {"error": "child exited %d: %s" % (res.returncode, res.stderr.strip()[-300:])}
    out = json.loads(lines[-1])
    out["process"] = "fresh child process, the workload's shape; inputs made on the GPU"
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=50)
    # the shader clock ramps up over the first seconds of calls (measured 1819 MHz at the start of
    # a timed region after a 5-call warm-up, 2212 MHz at its end): settle by time as well
    ap.add_argument("--settle", type=float, default=4.0,
                    help="seconds of untimed calls after the warm-up (at least; see settle()); "
                         "0 skips the phase (counter-collection runs)")
    ap.add_argument("--aa-rounds", type=int, default=10,
                    help="rounds of the A/A twin (0 skips it: counter-collection runs)")
    ap.add_argument("--no-peak", action="store_true",
                    help="skip the MFMA ceiling probe (counter-collection runs)")
    ap.add_argument("--workload", default="c3c", choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-budget", type=float, default=20.0)
    ap.add_argument("--kernel", type=int, default=0, choices=(0, 1, 2, 3, 4),
                    help="main-loop kernel: 0 the library's choice by grid fill, 1 the 128-query "
                         "kernel, 2 the 256-query ping-pong, 3 the pipelined 128-query kernel, "
                         "4 its key split (non-causal head_dim 64)")
    ap.add_argument("--no-first-call", action="store_true",
                    help="skip the fresh-process first-call latency (import, library load, first "
                         "call)")
    ap.add_argument("--first-call-child", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="instead of the benchmark, run a plain device copy of this many MiB "
                         "(the reference kernel for scaling rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this build measures one GPU only (every GPU box here has one GPU); "
              "--gpus %d is not supported" % args.gpus, file=sys.stderr)
        return 2
    if args.first_call_child:
        return first_call_child(args.workload)
    # before this process initializes the GPU: the first call in a fresh process
    first = None if args.no_first_call or args.copy_mib else first_call_latency(args.workload)
    if first is not None:
        log("first call:", first)

    import torch
    if args.copy_mib:
        return copy_calibration(args.copy_mib, max(args.steps, 1))
    from sageattention import sageattn
    from sageattention.sk1_backend import SageLib, sk1_forward

    wl = WORKLOADS[args.workload]
    dt, B, H, N, causal, layout, *_ = wl
    D = head_dim(wl)
    q, k, v = make_inputs(wl)
    dev = torch.device("cuda:0")
    qd, kd, vd = (t.to(dev) for t in (q, k, v))
    lib = SageLib.get()
    split_call = lambda ev=None: sk1_forward(lib, qd, kd, vd, tensor_layout=layout,
                                             is_causal=causal, smooth_k=True, events=ev,
                                             kernel=args.kernel)
    if args.kernel == 0:
        call = lambda: sageattn(qd, kd, vd, tensor_layout=layout, is_causal=causal, smooth_k=True)
        timed_call = "sageattn"
    else:
        call = split_call
        timed_call = "sk1_forward(kernel=%d)" % args.kernel
    # the kernel the timed call runs: the library's own automatic choice for kernel 0
    kcode = args.kernel or lib.kernel_choice(B, H, N, D, causal)
    kname = {1: "attn_fwd_kernel", 2: "attn_fwd_pp_kernel", 3: "attn_fwd_pl_kernel",
             4: "attn_fwd_pl_kernel (key split)"}[kcode]
    sync = torch.cuda.synchronize
    event = lambda: torch.cuda.Event(enable_timing=True)  # noqa: E731
    for _ in range(args.warmup):
        call()
    sync()
    st = settle(call, sync, min_s=args.settle) if args.settle > 0 else None
    if st is not None:
        st["board_power"] = board_power()
    log("settle:", st)

    # the timed region: exactly K calls
    sync()
    clk0 = sclk_mhz()
    e0, e1 = event(), event()
    sync()
    t0 = time.perf_counter()
    e0.record()
    for _ in range(args.steps):
        call()
    e1.record()
    sync()
    wall = time.perf_counter() - t0
    clk1 = sclk_mhz()
    ms_step = wall * 1e3 / args.steps
    ev_ms = e0.elapsed_time(e1) / args.steps

    aa = (aa_twin(call, event, sync, rounds=args.aa_rounds,
                  batch=max(1, min(10, int(100.0 / max(ms_step, 1e-3)))))
          if args.aa_rounds > 0 else None)
    log("A/A twin:", aa)

    # the prologue / main-loop split, from events between sk1_forward's launches
    evs = [[event() for _ in range(3)] for _ in range(args.steps)]
    sync()
    for i in range(args.steps):
        split_call(evs[i])
    sync()
    steps_ms = sorted(e[0].elapsed_time(e[2]) for e in evs)
    pro_ms = sum(e[0].elapsed_time(e[1]) for e in evs) / args.steps
    attn_ms = sum(e[1].elapsed_time(e[2]) for e in evs) / args.steps
    split_ms = sum(e[0].elapsed_time(e[2]) for e in evs) / args.steps

    peak, measured = None, None
    if not args.no_peak:
        clk_p0 = sclk_mhz()
        i8_tops, i8_mhz = mfma_peak(lib, True, event, sync)
        f8_tops, f8_mhz = mfma_peak(lib, False, event, sync)
        peak = {"int8_tops": round(i8_tops, 1), "fp8_tops": round(f8_tops, 1),
                "int8_run_mhz": None if i8_mhz is None else round(i8_mhz),
                "fp8_run_mhz": None if f8_mhz is None else round(f8_mhz),
                "documented_tops": PEAK_TOPS,
                "sclk_mhz": {"before": clk_p0, "after": sclk_mhz()},
                "probe": "sage_mfma_peak_probe: %d blocks x 4 waves, 4 independent "
                         "register-resident MFMAs per wave per round"
                         % (4 * torch.cuda.get_device_properties(0).multi_processor_count)}
        log("measured MFMA peak:", peak)
        measured = peak["int8_tops"] if dt == "fp16" else peak["fp8_tops"]

    ops = ops_of(B, H, N, causal, D)
    value = ops / (ms_step * 1e-3) / 1e12
    attn_tflops = ops / (attn_ms * 1e-3) / 1e12
    pbytes = prologue_bytes(B, H, N, D=D)
    pro_gbps = pbytes / (pro_ms * 1e-3) / 1e9
    # the same data flow with K read once (the smooth_k mean and the quantization from one read):
    # the byte floor of the prologue, whatever the number of passes
    floor_bytes = prologue_bytes(B, H, N, smooth_k=False, D=D)
    floor_gbps = floor_bytes / (pro_ms * 1e-3) / 1e9
    log("workload %s: %.3f ms/step (events %.3f), split: prologue %.3f ms (%.0f GB/s), main loop"
        " %.3f ms (%.1f TFLOP/s)" % (args.workload, ms_step, ev_ms, pro_ms, pro_gbps, attn_ms,
                                     attn_tflops))

    cpu = None
    if not args.no_cpu:
        del qd, kd, vd
        cpu = cpu_baseline(wl, q, k, v, budget_s=args.cpu_budget)
        log("cpu baseline:", cpu)

    res = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8" if dt == "fp16" else "fp8",
        "data": "synthetic",
        "pct_mfma_peak": round(100.0 * value / PEAK_TOPS, 2),
        "config": {"workload": "%s: %s B=%d H=%d N=%d D=%d %s smooth_k %s" % (
            args.workload, dt, B, H, N, D, "causal" if causal else "non-causal", layout),
            "global_batch": B, "seq_len": N, "parallelism": "single-gpu"},
        "timed_call": timed_call,
        "settle": st,
        "aa_ratio": None if aa is None else aa["ratio"],
        "aa_twin": aa,
        "measured_peak": peak,
        "roofline": {"bound": "mfma", "achieved": round(attn_tflops, 1), "peak": PEAK_TOPS,
                     "unit": "TFLOP/s", "frac": round(attn_tflops / PEAK_TOPS, 4),
                     "frac_of_measured": (None if measured is None
                                          else round(attn_tflops / measured, 4)),
                     "traffic": profiled_traffic(args.workload), "kernel": kname,
                     "ms": round(attn_ms, 4)},
        "prologue": {"ms": round(pro_ms, 4), "bytes": pbytes, "achieved_GBps": round(pro_gbps, 1),
                     "peak_GBps": HBM_PEAK_GBPS, "frac": round(pro_gbps / HBM_PEAK_GBPS, 4),
                     "single_read_bytes": floor_bytes,
                     "frac_single_read": round(floor_gbps / HBM_PEAK_GBPS, 4)},
        "cpu_baseline": cpu,
        "first_call": first,
        # the timed region's HIP-event time per call, the split pass's per-call times, and the
        # shader clock before and after the timed region: box-to-box clock differences are the
        # largest source of spread between runs
        "event_ms_per_step": round(ev_ms, 4),
        "split_step_ms": {"mean": round(split_ms, 4), "min": round(steps_ms[0], 4),
                          "median": round(steps_ms[len(steps_ms) // 2], 4),
                          "max": round(steps_ms[-1], 4)},
        "sclk_mhz": {"before": clk0, "after": clk1},
    }
    print(json.dumps(res), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
