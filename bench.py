"""Benchmark of the MI355X block-FP8 W8A8 GEMM (BASELINE.json metric).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--only qkv|side|prefill|mlp|moe|ceiling]
    python bench.py --profile config2 [--steps K --warmup W]       # the timed step's graphs, for rocprofv3 runs
    python bench.py --profile prefill|mlp|moe [--reps R]           # eager launches, for rocprofv3 runs
    python bench.py --rocprof-summary DIR [--steps K]              # tables of a rocprofv3 csv output

Workload (one "step"): BASELINE.json configs[1] decode sweep -- one block-FP8
GEMM at each M in {1, 2, 4, 8, 16} with N=6144, K=4096 (QKV projection),
E4M3 weights with fp32 128x128 block scales, bf16 activations quantized per
1x128 group inside the op, bf16 output.  Inputs are synthetic (seeded
N(0,0.02) weights with 5% x8 blocks, N(0,1) activations with 1% x20 outlier
channels) and resident in HBM before timing starts.  Weight copies totalling
>= 512 MB are rotated so the 256 MB Infinity Cache cannot serve them.  The
weights are in the load-time packed layout (ops.pack_weight, the same codes in
matrix-instruction fragment order; results bit-identical to row-major
weights); the row-major kernel times are reported beside them.

value = algorithmic bytes of the sweep / time per sweep (GB/s), with bytes per
GEMM B = N*K + 4*ceil(N/128)*ceil(K/128) + 2*M*K + 2*M*N.  Side measurements
in the same JSON line: the prefill config (M=4096, N=K=7168; TFLOP/s against
the dense FP8 MFMA peak), the MLP-pair decode config, the MoE layer (512
tokens, 8 experts, top-2, H=4096, I=14336), the per-M sweep, the
roofline of the dominant kernel (the decode GEMM with the quantizer fused: the
step's five launches, timed region / 5; HIP events on its stream), the
prefill kernel's roofline against the dense FP8 MFMA peak (roofline_prefill),
the streaming-read ceiling of this GPU at the decode footprints
(stream_ceiling, tests/csrc/libgk_probe.so) and the CPU oracle baseline timed on this
host (config 2 M=16 as cpu_baseline; configs 3, 4 and 5 beside it).
"""

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "gaudi-kernels_amd", "python"))
sys.path.insert(0, ROOT)

import torch  # noqa: E402

METRIC = "block-FP8 GEMM GB/s & TFLOP/s (% roofline) at M=1..16 and M=4096"
PEAK_HBM_GBS = 8000.0
PEAK_FP8_TFLOPS = 5033.0   # dense, 256 CU x 8192 FLOP/clk x 2.4 GHz
MALL_ROTATE_BYTES = 512 << 20
# The roofline kernel: the decode GEMM with the 1x128 quantizer fused, on packed weights, at config 2
# (NW=8, R=2, U=4, bf16 activations read directly, WPACK, one token tile) -- each op of the step is one
# launch of it.
DECODE_KERNEL = "gk::gemm_decode_kernel<8,2,4,false,false,false,true,true,1>"
# The prefill roofline kernel: the 256 x 256 LDS-tiled MFMA kernel on packed weights (config 4), launched as the
# split kernel: one launch with 256-wide tiles on 4096 columns and 192-wide tiles on the other 3072.
PREFILL_KERNEL = "gk::gemm_prefill256_split_kernel<false,true>"
SIMD_NUM = 1024  # 256 CUs x 4 SIMDs (MI355X)


def gemm_bytes(m, n, k, bias=False):
    nb, g = (n + 127) // 128, (k + 127) // 128
    return n * k + 4 * nb * g + 2 * m * k + 2 * m * n + (4 * n if bias else 0)


def gemm_flops(m, n, k):
    return 2 * m * n * k


def log(msg):
    print(msg, file=sys.stderr, flush=True)


class Rotation:
    """Distinct device copies of one weight/scale pair totalling >= MALL_ROTATE_BYTES.

    packed=True: each copy is the load-time packed layout (ops.pack_weight) of the weight.
    """

    def __init__(self, w, s, min_bytes=MALL_ROTATE_BYTES, packed=False):
        copies = max(1, -(-min_bytes // (w.numel() + 4 * s.numel())))
        wd, sd = w.cuda(), s.cuda()
        if packed:
            from gaudi_kernels import ops
            self.items = [(ops.pack_weight(wd), sd if i == 0 else sd.clone()) for i in range(copies)]
        else:
            self.items = [(wd, sd)] + [(wd.clone(), sd.clone()) for _ in range(copies - 1)]
        self.i = 0

    def next(self):
        item = self.items[self.i]
        self.i = (self.i + 1) % len(self.items)
        return item


def capture(fn, iters):
    """HIP graph of `iters` back-to-back fn() calls (kernel launches only; no host work at replay)."""
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        fn()  # first call outside capture (library / allocator warm-up)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(iters):
            fn()
    torch.cuda.synchronize()
    return graph


def time_graph(graph, iters_in_graph, replays=3, warm_s=0.02):
    """Average ms per captured call, HIP events on the replay stream (torch's current stream).

    Untimed replays first, for at least `warm_s` seconds and three replays: a graph's first replays after
    other work run slower (measured on MI355X: the config 4 op 241, 221, then 216 us; a decode graph's
    first replays 1.3 and 0.2 us per step above its later ones), so the timed replays start steady."""
    t_end = time.perf_counter() + warm_s
    done = 0
    while done < 3 or time.perf_counter() < t_end:
        graph.replay()
        torch.cuda.synchronize()
        done += 1
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(replays):
        graph.replay()
    end.record()
    end.synchronize()
    return start.elapsed_time(end) / (replays * iters_in_graph)


def time_loop(fn, iters, warmup):
    """Average ms per fn() call: `warmup` eager calls, then a graph of `iters` calls replayed."""
    for _ in range(warmup):
        fn()
    return time_graph(capture(fn, iters), iters)


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "block_fp8_gemm_bench.md")
PROFILE_DIR = os.path.join(ROOT, "profiles")


def profile_lines():
    """Lines of every committed rocprofv3 summary under profiles/ (traffic: and mfma: lines are read from them)."""
    import glob
    lines = []
    for path in sorted(glob.glob(os.path.join(PROFILE_DIR, "*.md"))):
        try:
            lines += open(path).read().splitlines()
        except OSError:
            pass
    return lines


def measured_traffic(kernel_prefix, workload):
    """HBM bytes of one op on `workload`: the sum over the launches of kernels whose names start with
    `kernel_prefix`, from the committed rocprofv3 --pmc summaries (FETCH_SIZE and WRITE_SIZE scaled by a
    plain-copy calibration), or None if not recorded."""
    import re
    total, seen = 0, set()
    for line in profile_lines():
        m = re.match(r"traffic: kernel=(\S+) workload=(\S+) .* bytes=(\d+)", line)
        if m and m.group(1).startswith(kernel_prefix) and m.group(2) == workload and m.group(1) not in seen:
            seen.add(m.group(1))
            total += int(m.group(3))
    return total if seen else None


def measured_mfma(kernel_prefix, workload):
    """(MFMA busy fraction, F8 MFMA FLOPs, GRBM_GUI_ACTIVE cycles) of one op on `workload` from the committed
    rocprofv3 --pmc summaries: FLOPs and cycles summed over the launches of kernels whose names start with
    `kernel_prefix`, the busy fraction weighted by each launch's cycles; None if not recorded."""
    import re
    busy, flops, cycles, seen = 0.0, 0.0, 0.0, set()
    for line in profile_lines():
        m = re.match(r"mfma: kernel=(\S+) workload=(\S+) .*busy_frac=([0-9.]+) .*f8_flops=([0-9.e+]+) .*gui_cycles=([0-9.]+)",
                     line)
        if m and m.group(1).startswith(kernel_prefix) and m.group(2) == workload and m.group(1) not in seen:
            seen.add(m.group(1))
            busy += float(m.group(3)) * float(m.group(5))
            flops += float(m.group(4))
            cycles += float(m.group(5))
    return (busy / cycles, flops, cycles) if seen and cycles > 0 else None


def measured_trace(kernel_prefix, workload):
    """Kernel-trace figures of the timed step from the committed rocprofv3 summaries (`--profile config2` under
    `--kernel-trace`, summarized by `--rocprof-summary DIR --steps K`): the roofline kernel's average duration over
    the timed launches and the span of the timed steps per step; None if not recorded."""
    import re
    for line in profile_lines():
        m = re.match(r"trace: kernel=(\S+) workload=(\S+) launches=(\d+) steps=(\d+) avg_us=([0-9.]+) "
                     r"span_per_step_us=([0-9.]+)", line)
        if m and m.group(1).startswith(kernel_prefix) and m.group(2) == workload:
            return {"avg_launch_us": float(m.group(5)), "span_per_step_us": float(m.group(6)),
                    "launches": int(m.group(3)), "steps": int(m.group(4)),
                    "source": "profiles/block_fp8_gemm_bench.md (rocprofv3 --kernel-trace of the step graphs)"}
    return None


def kernel_short_name(name):
    """Kernel name without its parameter list (and without the anonymous-namespace marker)."""
    return name.replace("(anonymous namespace)::", "").split("(")[0]


def rocprof_summary(directory, steps=20):
    """Markdown tables from rocprofv3 csv output: kernel trace durations and PMC counters per dispatch shape.

    Dispatches are grouped by (kernel, grid size): one kernel name covers
    several GEMM shapes in one bench run.  Counter values are rocprofv3's
    (KiB per dispatch for FETCH_SIZE / WRITE_SIZE), unscaled.
    """
    import csv
    import glob
    from collections import defaultdict

    def med(v):
        v = sorted(v)
        return v[len(v) // 2]

    for path in sorted(glob.glob(os.path.join(directory, "**", "*_kernel_trace.csv"), recursive=True)):
        agg = defaultdict(list)
        for r in csv.DictReader(open(path)):
            grid = f"{r['Grid_Size_X']}x{r['Grid_Size_Y']}x{r['Grid_Size_Z']}"
            agg[(kernel_short_name(r["Kernel_Name"]), grid, r["Workgroup_Size_X"])].append(
                int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
        print(f"### kernel trace: {os.path.relpath(path, directory)}\n")
        print("| kernel | grid (threads) | wg | calls | avg us | median us | min us |")
        print("|---|---|---|---|---|---|---|")
        for (name, grid, wg), v in sorted(agg.items(), key=lambda kv: -sum(kv[1])):
            print(f"| `{name}` | {grid} | {wg} | {len(v)} | {sum(v) / len(v) / 1e3:.2f} | {med(v) / 1e3:.2f} | "
                  f"{min(v) / 1e3:.2f} |")
        print()
        # The timed step of `--profile config2`: its last len(CONFIG2_MS) x steps dispatches of the roofline kernel
        # (the warm-up graph's come first): their average duration and the span from the first start to the last
        # end, per step.
        rows = sorted((int(r["Start_Timestamp"]), int(r["End_Timestamp"])) for r in csv.DictReader(open(path))
                      if kernel_short_name(r["Kernel_Name"]).replace("void ", "").replace(" ", "") ==
                      DECODE_KERNEL.replace(" ", "") and r["Grid_Size_X"] == "98304")
        n_timed = len(CONFIG2_MS) * steps
        if len(rows) >= n_timed:
            timed = rows[-n_timed:]
            avg = sum(e - b for b, e in timed) / n_timed / 1e3
            span = (timed[-1][1] - timed[0][0]) / steps / 1e3
            print(f"trace: kernel={DECODE_KERNEL.replace(' ', '')} workload=config2_step launches={n_timed} "
                  f"steps={steps} avg_us={avg:.3f} span_per_step_us={span:.3f}\n")
    counters = defaultdict(list)
    copy = defaultdict(list)  # counter -> values of the calibration copies
    for path in sorted(glob.glob(os.path.join(directory, "**", "*_counter_collection.csv"), recursive=True)):
        agg = defaultdict(list)
        copies = defaultdict(list)
        for r in csv.DictReader(open(path)):
            agg[(kernel_short_name(r["Kernel_Name"]), r["Grid_Size"], r["Counter_Name"])].append(
                float(r["Counter_Value"]))
            if r["Kernel_Name"] == "__amd_rocclr_copyBuffer":
                copies[r["Counter_Name"]].append((int(r["Dispatch_Id"]), float(r["Counter_Value"])))
        # a --profile run starts with the three 256 MiB calibration copies (copy_calibration); later
        # copies (input set-up) have other sizes
        for ctr, v in copies.items():
            copy[ctr] += [val for _, val in sorted(v)[:3]]
        print(f"### counters: {os.path.relpath(path, directory)}\n")
        print("| kernel | grid (threads) | counter | dispatches | median | min | max |")
        print("|---|---|---|---|---|---|---|")
        for (name, grid, ctr), v in sorted(agg.items()):
            print(f"| `{name}` | {grid} | {ctr} | {len(v)} | {med(v):.1f} | {min(v):.1f} | {max(v):.1f} |")
            counters[(name, grid, ctr)] += v
        print()
    # Traffic: the 256 MiB calibration copies (the first three __amd_rocclr_copyBuffer dispatches of each
    # --profile run) calibrate the counters; each gk GEMM dispatch shape gets a line.
    copy = {c: med(v) for c, v in copy.items()}
    copy_bytes = 256 << 20
    if "FETCH_SIZE" in copy and "WRITE_SIZE" in copy:
        fs, ws = copy_bytes / 1024 / copy["FETCH_SIZE"], copy_bytes / 1024 / copy["WRITE_SIZE"]
        print(f"copy calibration: FETCH_SIZE {copy['FETCH_SIZE']:.1f} KiB and WRITE_SIZE {copy['WRITE_SIZE']:.1f} KiB "
              f"for {copy_bytes} bytes each way: scales {fs:.4f} / {ws:.4f}\n")
        for (name, grid, ctr), v in sorted(counters.items()):
            short = name.replace("void ", "")
            if ctr != "FETCH_SIZE" or not short.startswith("gk::gemm_"):
                continue
            wv = counters.get((name, grid, "WRITE_SIZE"))
            if not wv:
                continue
            f_kib, w_kib = med(v), med(wv)
            total = int(round(f_kib * 1024 * fs + w_kib * 1024 * ws))
            print(f"traffic: kernel={short.replace(' ', '')} workload={workload_of(short, grid)} "
                  f"grid={grid} fetch_kib={f_kib:.1f} write_kib={w_kib:.1f} fetch_scale={fs:.4f} write_scale={ws:.4f} "
                  f"bytes={total}\n")
    # Matrix-core evidence: MfmaUtil (SQ_VALU_MFMA_BUSY_CYCLES over GRBM_GUI_ACTIVE x SIMDs, percent),
    # SQ_INSTS_VALU_MFMA_MOPS_F8 (FLOPs / 512) and GRBM_GUI_ACTIVE per dispatch shape.
    for (name, grid, ctr), v in sorted(counters.items()):
        short = name.replace("void ", "")
        if ctr != "MfmaUtil" or not short.startswith("gk::gemm_"):
            continue
        mops = counters.get((name, grid, "SQ_INSTS_VALU_MFMA_MOPS_F8"))
        gui = counters.get((name, grid, "GRBM_GUI_ACTIVE"))
        if not mops or not gui:
            continue
        print(f"mfma: kernel={short.replace(' ', '')} workload={workload_of(short, grid)} grid={grid} "
              f"busy_frac={med(v) / 100:.4f} f8_flops={med(mops) * 512:.6e} gui_cycles={med(gui):.0f}\n")


# Dispatch grids (threads) of the bench workloads' GEMM kernels -> workload names in profile summaries.
WORKLOAD_BY_GRID = {"98304": "config2", "114688": "config3_gate_up", "131072": "config3_down",
                    "688128": "config5_gate_up", "196608": "config5_down"}


def workload_of(kernel, grid):
    """Workload of a GEMM dispatch in a profile summary: by grid, except the config 4 prefill launch (the split
    kernel, 512 workgroups of 512 threads)."""
    if "prefill256_split" in kernel:
        return "config4"
    return WORKLOAD_BY_GRID.get(grid, "grid" + grid)


def copy_calibration():
    """Plain device-to-device copy of 256 MiB: the calibration kernel for the FETCH_SIZE / WRITE_SIZE counters of
    `rocprofv3 --pmc` runs of this script (the GEMM counters are scaled by what they read here)."""
    copy_bytes = 256 << 20
    csrc = torch.empty(copy_bytes, dtype=torch.uint8, device="cuda")
    cdst = torch.empty_like(csrc)
    for _ in range(3):
        cdst.copy_(csrc)
    torch.cuda.synchronize()


CONFIG2_MS = (1, 2, 4, 8, 16)
CONFIG2_NK = (6144, 4096)


class Config2Step:
    """The timed step (config 2 decode sweep: one block-FP8 GEMM op at each M in CONFIG2_MS, N=6144, K=4096,
    packed weights rotated over >= 512 MB) and its two HIP graphs: `warm` (W untimed steps) and `timed` (K steps).
    bench.py times `timed` after replaying `warm`; `--profile config2` replays the same two graphs under rocprofv3,
    so the profile covers exactly the timed launches."""

    def __init__(self, steps, warmup):
        from gaudi_kernels import ops
        from oracle import synth
        n, k = CONFIG2_NK
        self.w, self.s = synth.weight(n, k, seed=2000)
        self.rot = Rotation(self.w, self.s, packed=True)
        self.xs = {m: synth.activations(m, k, seed=2001 + m).cuda() for m in CONFIG2_MS}
        self.outs = {m: torch.empty((m, n), dtype=torch.bfloat16, device="cuda") for m in CONFIG2_MS}
        self.wss = {m: ops.make_workspace(m, n, k) for m in CONFIG2_MS}
        self.bytes = sum(gemm_bytes(m, n, k) for m in CONFIG2_MS)
        self.flops = sum(gemm_flops(m, n, k) for m in CONFIG2_MS)
        self.steps = steps

        def step():
            for m in CONFIG2_MS:
                wd, sd = self.rot.next()
                ops.block_fp8_gemm(self.xs[m], wd, sd, out=self.outs[m], workspace=self.wss[m])

        # The K timed steps (and the W warm-up steps) are captured as HIP graphs so
        # that the GPU runs them back to back without per-launch host work.
        self.warm = capture(step, max(1, warmup))
        self.timed = capture(step, steps)

    def release(self):
        del self.warm, self.timed


def run_profile(workload, reps, steps=20, warmup=5):
    """One workload's launches for rocprofv3 (kernel trace or counters), no timing.  config2: the timed step's own
    graphs (`warm` replayed, then `timed` once, as bench.py does; `steps`/`warmup` as its --steps/--warmup), so the
    last 5 x steps roofline-kernel dispatches of the trace are the timed region.  Others: eager launches of the
    same inputs and ops as the timed measurements."""
    from gaudi_kernels import ops
    from oracle import synth

    ops.require_device()
    copy_calibration()
    log(f"[profile] {workload}, {reps} reps")
    if workload == "config2":
        c2 = Config2Step(steps, warmup)
        c2.warm.replay()
        torch.cuda.synchronize()
        c2.timed.replay()
        torch.cuda.synchronize()
        log(f"[profile] config2 step graph: {warmup} warm-up steps, then {steps} timed steps of "
            f"{len(CONFIG2_MS)} launches")
        c2.release()
    elif workload == "prefill":
        m, n, k = 4096, 7168, 7168
        w, s = synth.weight(n, k, seed=4000)
        x = synth.activations(m, k, seed=4001).cuda()
        p, sd = ops.pack_weight(w.cuda()), s.cuda()
        o = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
        for _ in range(reps):
            ops.block_fp8_gemm(x, p, sd, out=o)
    elif workload == "mlp":
        m = 16
        for (n, k, seed) in ((28672, 4096, 3000), (4096, 14336, 3100)):
            w, s = synth.weight(n, k, seed=seed)
            x = synth.activations(m, k, seed=seed + 1).cuda()
            p, sd = ops.pack_weight(w.cuda()), s.cuda()
            for _ in range(reps):
                ops.block_fp8_gemm(x, p, sd)
    elif workload == "moe":
        x5, lg5, wg, sg, wdn, sdn = moe_inputs()
        pg, pdn = ops.pack_experts(wg), ops.pack_experts(wdn)
        for _ in range(reps):
            ops.moe_block_fp8(x5, lg5, pg, sg, pdn, sdn, top_k=2)
    torch.cuda.synchronize()
    log("[profile] done")


def moe_inputs(device="cuda"):
    """Config 5 (512 tokens, 8 experts, top-2, H=4096, I=14336) on `device`."""
    from oracle import synth
    t5, h5, i5, e5 = 512, 4096, 14336, 8
    wg, sg, wdn, sdn = [], [], [], []
    for i in range(e5):
        a, b = synth.weight(2 * i5, h5, seed=5010 + i, device=device)
        c, d = synth.weight(h5, i5, seed=6010 + i, device=device)
        wg.append(a); sg.append(b); wdn.append(c); sdn.append(d)
    x5 = synth.activations(t5, h5, seed=5001).to(device)
    lg5 = torch.randn(t5, e5, generator=torch.Generator().manual_seed(5002)).to(device)
    return x5, lg5, torch.stack(wg), torch.stack(sg), torch.stack(wdn), torch.stack(sdn)


def stream_ceiling():
    """Best streaming-read rate (GB/s) of a plain read kernel (tests/csrc/libgk_probe.so) at the decode footprints: config 2's
    weights (25.17 MB) and config 3's gate_up weights (117.44 MB), buffers rotated over >= 512 MB like the GEMMs,
    workgroup counts 256..4096."""
    import ctypes
    path = os.path.join(ROOT, "tests", "csrc", "libgk_probe.so")
    lib = ctypes.CDLL(path)
    lib.gk_probe_stream_read.restype = ctypes.c_int
    lib.gk_probe_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int,
                                         ctypes.c_void_p]
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")
    out = {}
    for label, nbytes in (("config2_25MB", 6144 * 4096), ("config3_gate_up_117MB", 28672 * 4096)):
        copies = max(2, -(-MALL_ROTATE_BYTES // nbytes))
        bufs = [torch.full((nbytes,), i + 1, dtype=torch.uint8, device="cuda") for i in range(copies)]
        best = None
        for wgs in (256, 512, 1024, 2048, 4096):
            state = {"i": 0}

            def read():
                b = bufs[state["i"]]
                state["i"] = (state["i"] + 1) % copies
                st = lib.gk_probe_stream_read(ctypes.c_void_p(b.data_ptr()), nbytes, ctypes.c_void_p(sink.data_ptr()),
                                              wgs, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
                assert st == 0, st

            t = time_loop(read, 4 * copies, 3)
            gbs = nbytes / (t * 1e-3) / 1e9
            if best is None or gbs > best[0]:
                best = (gbs, wgs, t * 1e3)
        out[label] = {"bytes": nbytes, "GBps": round(best[0], 1), "hbm_frac": round(best[0] / PEAK_HBM_GBS, 4),
                      "us": round(best[2], 2), "workgroups": best[1]}
        del bufs
        torch.cuda.empty_cache()
    return out


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baselines(w2, s2):
    """The oracle (oracle/block_fp8.reference, oracle/moe.moe_reference: block_fp8_oracle.py:11-46 batched over
    rows) on this host's cores.  Returns (headline config 2 M=16 entry, per-config entries)."""
    from oracle import block_fp8, moe, synth
    cores = os.cpu_count() or 1
    torch.set_num_threads(cores)
    model = cpu_model()

    def median_time(fn, min_runs=3, budget_s=10.0):
        fn()  # warm-up
        times = []
        t_budget = time.perf_counter()
        while len(times) < min_runs or (time.perf_counter() - t_budget < budget_s and len(times) < 10):
            t1 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t1)
            if len(times) >= 1 and time.perf_counter() - t_budget > 3 * budget_s:
                break
        return sorted(times)[len(times) // 2], len(times)

    base = {"cores": cores, "cpu_model": model, "kind": "port"}
    # config 2, M = 16 (the headline unit: GB/s)
    n, k, m = 6144, 4096, 16
    xc = synth.activations(m, k, seed=2001 + m)
    t2, r2 = median_time(lambda: block_fp8.reference(xc, w2, s2, row_chunk=16))
    headline = {"value": round(gemm_bytes(m, n, k) / t2 / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": "port",
                "sample": f"oracle/block_fp8.reference, config2 M=16 N=6144 K=4096 in full, median of {r2} runs "
                          f"({t2 * 1e3:.0f} ms each), torch threads={cores}, cpu {model}"}
    per = {"config2_m16": {**base, "s": round(t2, 4), "GBps": headline["value"], "runs": r2, "sample": "full"}}
    # config 3: the MLP pair at M = 16, in full
    tot_t, tot_b = 0.0, 0
    for (nn, kk, seed) in ((28672, 4096, 3000), (4096, 14336, 3100)):
        w3, s3 = synth.weight(nn, kk, seed=seed)
        x3 = synth.activations(16, kk, seed=seed + 1)
        t3, _ = median_time(lambda: block_fp8.reference(x3, w3, s3, row_chunk=16), min_runs=1, budget_s=3.0)
        tot_t += t3
        tot_b += gemm_bytes(16, nn, kk)
        del w3, s3
    per["config3_mlp_pair_m16"] = {**base, "s": round(tot_t, 4), "GBps": round(tot_b / tot_t / 1e9, 3),
                                   "sample": "full (gate_up N=28672 K=4096 + down N=4096 K=14336, M=16)"}
    # config 4: 64-row chunks, two timed and extrapolated to the 64 chunks of M = 4096
    m4, n4, k4 = 4096, 7168, 7168
    w4, s4 = synth.weight(n4, k4, seed=4000)
    x4 = synth.activations(128, k4, seed=4001)
    block_fp8.reference(x4[:64], w4, s4, row_chunk=64)  # warm-up
    t1 = time.perf_counter()
    block_fp8.reference(x4, w4, s4, row_chunk=64)
    tc = (time.perf_counter() - t1) / 2
    t4 = tc * (m4 // 64)
    per["config4_prefill"] = {**base, "s": round(t4, 2), "TFLOPs": round(gemm_flops(m4, n4, k4) / t4 / 1e12, 5),
                              "sample": f"extrapolated: 2 of 64 row chunks of 64 timed ({tc:.2f} s per chunk) x 64",
                              "extrapolated": True}
    del w4, s4
    # config 5: the MoE layer in full
    x5, lg5, wg, sg, wdn, sdn = moe_inputs(device="cpu")
    t1 = time.perf_counter()
    moe.moe_reference(x5, lg5, wg, sg, wdn, sdn, top_k=2)
    t5 = time.perf_counter() - t1
    w_bytes = wg.numel() + wdn.numel() + 4 * (sg.numel() + sdn.numel())
    f5 = 2 * 512 * 2 * (2 * 14336 * 4096 + 4096 * 14336)
    per["config5_moe"] = {**base, "s": round(t5, 2), "GBps": round(w_bytes / t5 / 1e9, 3),
                          "TFLOPs": round(f5 / t5 / 1e12, 5), "sample": "full (one run), oracle/moe.moe_reference"}
    return headline, per


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--only", choices=["decode", "qkv", "side", "prefill", "mlp", "moe", "ceiling"], default=None)
    ap.add_argument("--rocprof-summary", metavar="DIR", default=None,
                    help="print per-kernel, per-grid tables of a rocprofv3 csv output directory and exit")
    ap.add_argument("--profile", choices=["config2", "prefill", "mlp", "moe"], default=None,
                    help="run one workload's ops eagerly (for rocprofv3) and exit")
    ap.add_argument("--reps", type=int, default=5)
    args = ap.parse_args()
    if args.rocprof_summary:
        rocprof_summary(args.rocprof_summary, args.steps)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (under tensor parallelism each GPU "
              "runs this GEMM on its own shard of the weights); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    if args.profile:
        run_profile(args.profile, args.reps, args.steps, args.warmup)
        return

    from gaudi_kernels import ops
    from oracle import synth

    ops.require_device()
    dev_name = torch.cuda.get_device_name(0)
    log(f"[bench] device {dev_name}")
    result = {}

    # ---- config 2: decode sweep (the timed step) ----------------------------------------------
    n, k = CONFIG2_NK
    ms_list = CONFIG2_MS
    c2 = Config2Step(args.steps, args.warmup)
    w, s, rot, xs, outs, wss = c2.w, c2.s, c2.rot, c2.xs, c2.outs, c2.wss
    rot_row = Rotation(w, s)
    sweep_bytes, sweep_flops = c2.bytes, c2.flops
    log(f"[bench] decode sweep: {len(rot.items)} weight copies, warmup {args.warmup}, steps {args.steps}")
    c2.warm.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    c2.timed.replay()
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    c2.release()
    ms_per_step = ev0.elapsed_time(ev1) / args.steps
    value = sweep_bytes / (ms_per_step * 1e-3) / 1e9
    log(f"[bench] decode sweep {ms_per_step * 1e3:.1f} us/step, {value:.0f} GB/s (wall {wall:.3f}s)")

    # Per M: the whole op -- at N = 6144, K = 4096 one launch of the decode
    # kernel with the quantizer fused, the step's only kernel, whose roofline
    # is reported over the step's five launches -- and, beside it, the decode
    # kernel alone on activations quantized beforehand (the block_fp8_gemm_q
    # path).
    per_m = {}
    launch_us = []
    for m in ms_list:
        op_ms = time_loop(lambda: ops.block_fp8_gemm(xs[m], *rot.next(), out=outs[m], workspace=wss[m]), 100, 10)
        # the op's own activation layout for M <= 16: the decode fragment layout
        q, sa = ops.act_quant(xs[m], decode_layout=True)
        kern_ms = time_loop(lambda: ops.block_fp8_gemm_q(q, sa, m, *rot.next(), out=outs[m], decode_layout=True),
                            100, 10)
        row_ms = time_loop(lambda: ops.block_fp8_gemm_q(q, sa, m, *rot_row.next(), out=outs[m], decode_layout=True),
                           100, 10)
        b = gemm_bytes(m, n, k)
        per_m[str(m)] = {"op_us": round(op_ms * 1e3, 2), "op_GBps": round(b / (op_ms * 1e-3) / 1e9, 1),
                         "op_hbm_frac": round(b / (op_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                         "q_path_kernel_us": round(kern_ms * 1e3, 2),
                         "q_path_kernel_GBps": round(b / (kern_ms * 1e-3) / 1e9, 1),
                         "q_path_kernel_rowmajor_us": round(row_ms * 1e3, 2)}
        launch_us.append(op_ms * 1e3)
        log(f"[bench]   M={m}: op {op_ms * 1e3:.2f} us ({per_m[str(m)]['op_GBps']} GB/s), "
            f"kernel on pre-quantized activations {kern_ms * 1e3:.2f} us "
            f"({per_m[str(m)]['q_path_kernel_GBps']} GB/s), row-major weights {row_ms * 1e3:.2f} us")
    del rot, rot_row, c2
    torch.cuda.empty_cache()

    copy_calibration()

    # The roofline kernel's average launch over the timed region: the step is the kernel's five launches (one per
    # M) and nothing else, so a launch takes ms_per_step / 5 (HIP events on the replay stream, the launch gaps of
    # the graph included).  Algorithmic bytes per launch: the mean over M = 1..16 of
    # N*K + 4*(N/128)*(K/128) + 2*M*K + 2*M*N.  The committed kernel trace of the same graphs
    # (`--profile config2`) gives the kernel-only duration and the span of the timed steps beside it.
    avg_bytes = sweep_bytes / len(ms_list)
    avg_us = ms_per_step * 1e3 / len(ms_list)
    achieved = avg_bytes / (avg_us * 1e-6) / 1e9
    trace = measured_trace(DECODE_KERNEL, "config2_step")
    result["roofline"] = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                          "frac": round(achieved / PEAK_HBM_GBS, 4),
                          "traffic": measured_traffic(DECODE_KERNEL, "config2"),
                          "traffic_source": "profiles/ (rocprofv3 FETCH_SIZE/WRITE_SIZE of the timed step graphs)",
                          "kernel": f"{DECODE_KERNEL} (quantizer fused; M=1,2,4,8,16, N=6144, K=4096, packed weights)",
                          "bytes_per_launch": int(avg_bytes), "avg_launch_us": round(avg_us, 3),
                          "launch_us_source": "timed region: ms_per_step / 5 launches (HIP events, gaps included)",
                          "profile": trace,
                          "steady_state_launch_us": {str(m): round(t, 3) for m, t in zip(ms_list, launch_us)},
                          "m16": {"achieved": round(gemm_bytes(16, n, k) / (launch_us[-1] * 1e-6) / 1e9, 1),
                                  "launch_us": round(launch_us[-1], 3)}}
    result["decode_sweep"] = per_m

    # ---- the streaming-read ceiling at the decode footprints --------------------------------------
    if args.only in (None, "ceiling"):
        ceil = stream_ceiling()
        ceil["decode_roofline_frac_of_ceiling"] = round(result["roofline"]["achieved"] / ceil["config2_25MB"]["GBps"], 4)
        result["stream_ceiling"] = ceil
        log(f"[bench] stream ceiling: {ceil}")

    # ---- config 2 as a layer step: fused add + RMSNorm feeding the QKV GEMM --------------------------
    # (a) one norm kernel that also writes the 1x128 codes in the decode layout, then the GEMM on them;
    # (b) the reference's op split: fused add + RMSNorm to bf16, then the GEMM op (quantizer fused).
    if args.only in (None, "qkv"):
        w, s = synth.weight(n, k, seed=2000)
        rot = Rotation(w, s, packed=True)
        gamma = (torch.rand(k, generator=torch.Generator().manual_seed(2100)) + 0.5).bfloat16().cuda()
        chain = {}
        for m in ms_list:
            xm = synth.activations(m, k, seed=2200 + m).cuda()
            rm = synth.activations(m, k, seed=2300 + m).cuda()
            om = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")

            def fused_chain():
                q, sa, _ = ops.rms_norm_quant(xm, gamma, 1e-6, residual=rm, decode_layout=True)
                ops.block_fp8_gemm_q(q, sa, m, *rot.next(), out=om, decode_layout=True)

            def split_chain():
                _, h = ops.fused_add_rms_norm(xm, rm, gamma, 1e-6)
                ops.block_fp8_gemm(h, *rot.next(), out=om, workspace=wss[m])

            t_norm = time_loop(lambda: ops.rms_norm_quant(xm, gamma, 1e-6, residual=rm, decode_layout=True), 100, 10)
            t_fused = time_loop(fused_chain, 100, 10)
            t_split = time_loop(split_chain, 100, 10)
            chain[str(m)] = {"norm_quant_us": round(t_norm * 1e3, 2), "fused_chain_us": round(t_fused * 1e3, 2),
                             "split_chain_us": round(t_split * 1e3, 2)}
        result["qkv_chain"] = chain
        log(f"[bench] qkv chain (fused add + RMSNorm -> QKV GEMM): {chain}")
        del rot
        torch.cuda.empty_cache()

    # ---- the path's neighbours: load-time codec and packing, per-token / per-channel GEMM, gated
    # activations fused with the quantizer (side measurements, bytes / FLOPs as stated per entry) ----------
    if args.only in (None, "side"):
        side = {}
        w4, s4 = synth.weight(7168, 7168, seed=4000)
        w4d, s4d = w4.cuda(), s4.cuda()
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

        def timed_sync(fn, reps=10):
            fn()
            torch.cuda.synchronize()
            ev0.record()
            for _ in range(reps):
                fn()
            ev1.record()
            torch.cuda.synchronize()
            return ev0.elapsed_time(ev1) / reps

        # codec: 2 B per code (read + write) + 8 B per scale; the call reads a status word back (synchronizes)
        t = timed_sync(lambda: ops.codec_ocp_to_half(w4d, s4d))
        side["codec_ocp_to_half_51M"] = {"us": round(t * 1e3, 1),
                                         "GBps": round((2 * w4.numel() + 8 * s4.numel()) / (t * 1e-3) / 1e9, 1)}
        t = time_loop(lambda: ops.pack_weight(w4d), 20, 3)  # 2 B per weight byte
        side["pack_weight_51M"] = {"us": round(t * 1e3, 1), "GBps": round(2 * w4.numel() / (t * 1e-3) / 1e9, 1)}
        # per-token / per-channel: token quantizer + channel GEMM, N = 6144, K = 4096 decode (one fused launch,
        # ops.token_channel_gemm; the two launches beside it) and config 4 prefill
        sw2 = (torch.rand(n, generator=torch.Generator().manual_seed(7)) + 0.5).cuda()
        wch = Rotation(synth.weight(n, k, seed=2000)[0], torch.zeros(1), min_bytes=MALL_ROTATE_BYTES)
        for m in (1, 16):
            xm = synth.activations(m, k, seed=2400 + m).cuda()

            def chan2():
                q, sa = ops.token_quant(xm)
                ops.channel_gemm(q, sa, wch.next()[0], sw2)

            t2 = time_loop(chan2, 100, 10)
            t = time_loop(lambda: ops.token_channel_gemm(xm, wch.next()[0], sw2), 100, 10)
            side[f"token_channel_gemm_m{m}"] = {"us": round(t * 1e3, 2),
                                                "GBps": round((n * k + 2 * m * k + 2 * m * n + 4 * n) / (t * 1e-3) / 1e9, 1),
                                                "two_launch_us": round(t2 * 1e3, 2)}
        del wch
        x4 = synth.activations(4096, 7168, seed=4001).cuda()
        sw4 = (torch.rand(7168, generator=torch.Generator().manual_seed(8)) + 0.5).cuda()

        def chan4():
            q, sa = ops.token_quant(x4)
            ops.channel_gemm(q, sa, w4d, sw4)

        t = time_loop(chan4, 10, 2)
        side["token_channel_gemm_m4096"] = {"us": round(t * 1e3, 1),
                                            "TFLOPs": round(gemm_flops(4096, 7168, 7168) / (t * 1e-3) / 1e12, 1)}
        # gated activation + 1x128 quantizer: 4 B in, 1 B + 4/128 B out per output element
        for rows in (16, 4096):
            gu = synth.activations(rows, 2 * 14336, seed=2500 + rows).cuda()
            per = rows * 14336 * (4 + 1 + 4 / 128)
            for name, fn in (("silu_mul_quant", lambda: ops.silu_mul_quant(gu)),
                             ("gelu_mul_quant", lambda: ops.gelu_mul_quant(gu))):
                t = time_loop(fn, 50, 5)
                side[f"{name}_{rows}x14336"] = {"us": round(t * 1e3, 2), "GBps": round(per / (t * 1e-3) / 1e9, 1)}
        result["side_ops"] = side
        log(f"[bench] side ops: {side}")
        del w4d, s4d, x4
        torch.cuda.empty_cache()

    # ---- config 3: MLP pair decode at M=16 ------------------------------------------------------
    if args.only in (None, "mlp"):
        m = 16
        pair = []
        for (nn, kk, seed) in ((28672, 4096, 3000), (4096, 14336, 3100)):
            w3, s3 = synth.weight(nn, kk, seed=seed)
            x3 = synth.activations(m, kk, seed=seed + 1).cuda()
            o3 = torch.empty((m, nn), dtype=torch.bfloat16, device="cuda")
            ws3 = ops.make_workspace(m, nn, kk)
            times = []
            for packed in (True, False):
                r3 = Rotation(w3, s3, packed=packed)
                times.append(time_loop(lambda: ops.block_fp8_gemm(x3, *r3.next(), out=o3, workspace=ws3), 30, 5))
                del r3
                torch.cuda.empty_cache()
            pair.append((nn, kk, times[0], times[1]))
        tb = sum(gemm_bytes(m, nn, kk) for nn, kk, _, _ in pair)
        tt = sum(t for _, _, t, _ in pair)
        result["mlp_pair_m16"] = {"us": round(tt * 1e3, 2), "GBps": round(tb / (tt * 1e-3) / 1e9, 1),
                                  "hbm_frac": round(tb / (tt * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                                  "gate_up_us": round(pair[0][2] * 1e3, 2), "down_us": round(pair[1][2] * 1e3, 2),
                                  "rowmajor_gate_up_us": round(pair[0][3] * 1e3, 2),
                                  "rowmajor_down_us": round(pair[1][3] * 1e3, 2)}
        log(f"[bench] mlp pair: {result['mlp_pair_m16']}")

    # ---- config 4: prefill ------------------------------------------------------------------------
    if args.only in (None, "prefill"):
        m, nn, kk = 4096, 7168, 7168
        w4, s4 = synth.weight(nn, kk, seed=4000)
        x4 = synth.activations(m, kk, seed=4001).cuda()
        # weight copies rotated (>= 512 MB with the codes and the output) so that the MALL does not hold them
        r4 = Rotation(w4, s4, min_bytes=384 << 20, packed=True)
        r4r = Rotation(w4, s4, min_bytes=384 << 20)
        o4 = torch.empty((m, nn), dtype=torch.bfloat16, device="cuda")
        ws4 = ops.make_workspace(m, nn, kk)
        ms4 = time_loop(lambda: ops.block_fp8_gemm(x4, *r4.next(), out=o4, workspace=ws4), 2 * len(r4.items), 3)
        _, m_pad, _ = ops.plan(m, nn, kk)
        q4, sa4 = ops.act_quant(x4, m_pad=m_pad)
        ms4k = time_loop(lambda: ops.block_fp8_gemm_q(q4, sa4, m, *r4.next(), out=o4), 2 * len(r4.items), 3)
        ms4r = time_loop(lambda: ops.block_fp8_gemm_q(q4, sa4, m, *r4r.next(), out=o4), 2 * len(r4r.items), 3)
        del r4, r4r
        torch.cuda.empty_cache()
        f = gemm_flops(m, nn, kk)
        result["prefill_m4096"] = {"op_us": round(ms4 * 1e3, 1), "gemm_kernel_us": round(ms4k * 1e3, 1),
                                   "op_TFLOPs": round(f / (ms4 * 1e-3) / 1e12, 1),
                                   "op_mfma_frac": round(f / (ms4 * 1e-3) / 1e12 / PEAK_FP8_TFLOPS, 4),
                                   "gemm_kernel_TFLOPs": round(f / (ms4k * 1e-3) / 1e12, 1),
                                   "gemm_kernel_mfma_frac": round(f / (ms4k * 1e-3) / 1e12 / PEAK_FP8_TFLOPS, 4),
                                   "gemm_kernel_rowmajor_us": round(ms4r * 1e3, 1),
                                   "weights": "packed, rotated copies (not MALL-resident)"}
        # The prefill kernel's roofline: FLOPs of one launch over its average launch duration (graph replay of
        # back-to-back launches on the replay stream, HIP events), against the dense FP8 MFMA peak.
        achieved = f / (ms4k * 1e-3) / 1e12
        counters = measured_mfma(PREFILL_KERNEL, "config4")
        result["roofline_prefill"] = {
            "bound": "mfma", "achieved": round(achieved, 1), "peak": PEAK_FP8_TFLOPS, "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_FP8_TFLOPS, 4), "traffic": measured_traffic(PREFILL_KERNEL, "config4"),
            "kernel": f"{PREFILL_KERNEL} (config 4: M=4096, N=K=7168, one launch: 256-wide tiles on 4096 "
                      "columns and 192-wide on 3072; packed weights, activations quantized beforehand)",
            "flops_per_op": f, "avg_op_us": round(ms4k * 1e3, 2),
            "op_frac": round(f / (ms4 * 1e-3) / 1e12 / PEAK_FP8_TFLOPS, 4),
            "counters": None if counters is None else {
                "mfma_busy_frac": counters[0], "f8_mfma_flops": counters[1], "gui_active_cycles": counters[2],
                "source": "profiles/prefill_moe_gemm_counters.md (rocprofv3 --pmc MfmaUtil SQ_INSTS_VALU_MFMA_MOPS_F8 "
                          "GRBM_GUI_ACTIVE)"}}
        log(f"[bench] prefill: {result['prefill_m4096']}")

    # ---- config 5: MoE layer ----------------------------------------------------------------------
    if args.only in (None, "moe"):
        t5, h5, i5, e5, k5 = 512, 4096, 14336, 8, 2
        x5, lg5, wg, sg, wdn, sdn = moe_inputs()
        o5 = torch.empty((t5, h5), dtype=torch.bfloat16, device="cuda")
        ws5 = torch.empty(ops.moe_workspace_bytes(t5, h5, i5, e5, k5), dtype=torch.uint8, device="cuda")
        ms5r = time_loop(lambda: ops.moe_block_fp8(x5, lg5, wg, sg, wdn, sdn, top_k=k5, out=o5, workspace=ws5),
                         20, 3)
        # expert weights in the load-time packed layout (bit-identical results)
        pg, pdn = ops.pack_experts(wg), ops.pack_experts(wdn)
        ms5 = time_loop(lambda: ops.moe_block_fp8(x5, lg5, pg, sg, pdn, sdn, top_k=k5, out=o5, workspace=ws5),
                        20, 3)
        del pg, pdn
        off = ops.moe_route(lg5, k5)[4].cpu()
        rows_used = int(off[-1])
        w_bytes = wg.numel() + wdn.numel() + 4 * (sg.numel() + sdn.numel())
        io_bytes = 2 * t5 * h5 * 2 + 4 * t5 * e5
        f_useful = 2 * t5 * k5 * (2 * i5 * h5 + h5 * i5)
        f_padded = 2 * rows_used * (2 * i5 * h5 + h5 * i5)
        result["moe_config5"] = {
            "us": round(ms5 * 1e3, 1),
            "weight_GBps": round((w_bytes + io_bytes) / (ms5 * 1e-3) / 1e9, 1),
            "hbm_frac": round((w_bytes + io_bytes) / (ms5 * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
            "TFLOPs": round(f_useful / (ms5 * 1e-3) / 1e12, 1),
            "padded_TFLOPs": round(f_padded / (ms5 * 1e-3) / 1e12, 1),
            "rows_used": rows_used, "rows_routed": t5 * k5, "weight_bytes": w_bytes,
            "rowmajor_us": round(ms5r * 1e3, 1)}
        log(f"[bench] moe: {result['moe_config5']}")
        del wg, sg, wdn, sdn, ws5
        torch.cuda.empty_cache()

    # ---- CPU baseline: the oracle on this host ----------------------------------------------------
    cpu = None
    if not args.no_cpu:
        cpu, per_cfg = cpu_baselines(w, s)
        result["cpu_baseline_configs"] = per_cfg
        log(f"[bench] cpu baseline: {cpu} {per_cfg}")

    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp8e4m3", "data": "synthetic",
        "config": {"workload": "config2 QKV decode sweep: block-FP8 GEMM at M=1,2,4,8,16, N=6144, K=4096, "
                               "128x128 fp32 weight scales, 1x128 activation groups, bf16 out; weights in the "
                               "load-time packed layout",
                   "sweep_bytes": sweep_bytes, "sweep_flops": sweep_flops, "device": dev_name},
        **result,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
