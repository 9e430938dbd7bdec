#!/usr/bin/env python3
"""Benchmark of the MI355X backend: Real-ESRGAN general x4v3
(SRVGGNetCompact) on a 1x3x256x384 image, per-image latency on one GPU,
plus the conv sweep's MFMA utilisation and the CPU baseline.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-sweep]

A step is one forward pass of the whole network over one synthetic image
(seeded uniform [0, 1) input, Kaiming-normal random-init weights) with the
input already resident in HBM: a step is one launch, the whole network as
one chain (ien_model_run_device with graphs on: a run of one launch is
launched directly).  Prints one JSON line.

roofline: the dominant kernel is that launch, conv_pair<chain>: the first
layer (3 -> 64), the 32 body layers (3x3 64->64 + PReLU each, 16 pairs)
and the last layer (64 -> 48) plus the pixel shuffle and the image added.
Its algorithmic work per launch is 2 * 98304 px * 576 * 64 * 32 (body)
+ 2 * 98304 * 27 * 64 (first) + 2 * 98304 * 576 * 48 (last) = 237.7 GFLOP
(the halo recomputed by neighbouring tiles is not counted); its average
duration is measured with HIP events on the library's stream over a graph of
100 back-to-back runs, after 100 untimed ones (the clock settles under
sustained load: a run's duration drifts by up to 25 % over the first tens of
milliseconds).  `traffic` (HBM bytes per launch from rocprofv3 FETCH_SIZE /
WRITE_SIZE, scaled by a copy kernel of known size) is read from
profiles/realesrgan_chain_256x384_hbm_traffic.txt when that summary exists.

cpu_baseline: the oracle -- the C restatement of the reference's CPU f32
path (crates/realesrgan-native/src/network.rs over native-engine's
Winograd F(4x4, 3x3) and indirect GEMM) -- timed on this host's cores on
the same image, median of 5 runs after a warm-up (README.md:26-27).  Every
other configuration carries its own cpu_baseline from the same protocol
(models[*].cpu_baseline, gemm_sweep_cpu).

host_path_ms: ien_model_run with host buffers (upload, launches, download
of the f32 output, synchronisation) beside the device-resident `value`.

measured_peaks: this device's sustained rates beside the published peaks
the roofline uses (2516.6 TFLOP/s f16 dense, 8 TB/s HBM): a register-only
MFMA loop on every SIMD and a 1 GiB device copy read from HBM.
"""

import argparse
import json
import os
import pathlib
import re
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "image-engine-native_amd"))

MFMA_F16_PEAK_TFLOPS = 2516.6  # MI355X dense f16 MFMA
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
SCUNET_GFLOP = 944.9           # 1x3x512x768, incl. 46.7 GFLOP of window attention
METRIC = "ms/image at 1 MI355X per model; conv/attn GEMM MFMA util % of f16 peak"


def log(msg):
    print(f"bench: {msg}", file=sys.stderr, flush=True)


# Device bytes in use (hipMemGetInfo) before the library's context opened:
# each configuration reports what it holds above that.
_DEVICE_BASE = 0


def device_in_use():
    import torch

    free, total = torch.cuda.mem_get_info()
    return total - free


def device_mib(extra_note=None):
    """Device memory the run holds: the context (its split-K workspace and
    chain flags), the model (weights, maps grown to this size, Swin scratch,
    plans) and the run's input and output tensors, in MiB above what was in
    use before the context opened. The library never shrinks its maps, so
    this is the configuration's peak; read before the model is freed."""
    import torch

    torch.cuda.synchronize()
    return round((device_in_use() - _DEVICE_BASE) / 2**20, 1)


def host_peak_mib():
    """VmHWM of this process (realesrgan-bench.rs:82-87 prints the same)."""
    try:
        for line in open("/proc/self/status"):
            if line.startswith("VmHWM"):
                return round(int(line.split()[1]) / 1024, 1)
    except OSError:
        pass
    return None


def conv_flops(h, w, cin, cout, size):
    return 2.0 * h * w * cout * cin * size * size


def event_time(fn, reps, stream):
    """Average milliseconds of one `fn` (which launches on `stream`): `reps`
    back-to-back calls captured into one HIP graph (so host launch overhead
    does not starve the GPU), replayed between two HIP events recorded on
    that stream."""
    import torch

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for _ in range(reps):
            fn()
    graph.replay()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    graph.replay()
    end.record(stream)
    end.synchronize()
    return start.elapsed_time(end) / reps


class SweepCase:
    """One conv-sweep shape (NCHW, f16, N(0, 1)) set up on the device the
    way the benchmark times it: `launch()` runs the product (or the
    depthwise pass) through the library into `out` (C x H*W f16);
    `x`, `wt`, `bias` are the host inputs (x C x H x W)."""

    def __init__(self, ctx, name):
        import torch

        import ien
        import synthetic

        (self.name, self.kind, cin, cout, size, h, w), x, wt, bias = synthetic.sweep_case(name)
        self.cin, self.cout, self.size, self.h, self.w = cin, cout, size, h, w
        self.x, self.wt, self.bias = x, wt, bias
        xt = torch.from_numpy(x).half().cuda()
        self._m = None
        if self.kind == "conv":
            m = ien.Matrix(ctx, wt, bias)
            inp = ien.image_input(xt, h, w, cin, layout=ien.NCHW, size=size)
            out = torch.empty((cout, h * w), dtype=torch.float16, device="cuda")

            def launch():
                ien.multiply_ex(ctx, inp, 0, h * w, m, out, h * w, layout=ien.NCHW)

            self._m = m
            self.flops = conv_flops(h, w, cin, cout, size)
            self.nbytes = 2.0 * (cin + cout) * h * w + 2.0 * wt.size
        else:
            wd = torch.from_numpy(wt).cuda()
            bd = torch.from_numpy(bias).cuda()
            out = torch.empty((cin, h * w), dtype=torch.float16, device="cuda")

            def launch():
                ien.depthwise(ctx, xt, h, w, cin, ien.NCHW, wd, size, bd, out)

            self.flops = 2.0 * h * w * cin * size * size
            self.nbytes = 2.0 * 2 * cin * h * w + 4.0 * wt.size
        self.out = out
        self.launch = launch

    def free(self):
        if self._m is not None:
            self._m.free()
            self._m = None


def sweep(ctx, stream, reps):
    """Each conv-sweep shape (NCHW, f16, N(0,1)) through the library."""
    import synthetic

    results = []
    counters = sweep_counters_from_profiles()
    for entry in synthetic.SWEEP:
        case = SweepCase(ctx, entry[0])
        for _ in range(5):
            case.launch()
        ms = event_time(case.launch, reps, stream)
        tflops = case.flops / (ms * 1e-3) / 1e12
        gbs = case.nbytes / (ms * 1e-3) / 1e9
        row = {"shape": case.name, "us": round(ms * 1e3, 2), "tflops": round(tflops, 1),
               "mfma_util_pct": round(100 * tflops / MFMA_F16_PEAK_TFLOPS, 1),
               "hbm_gbs": round(gbs, 0), "hbm_pct": round(100 * gbs / HBM_PEAK_GBS, 1)}
        if case.name in counters:
            row["rocprof"] = counters[case.name]
        results.append(row)
        case.free()
    return results


def elementwise(ctx, stream, reps, copy_tbps=None):
    """The memory-bound passes at a shape a model runs them, each timed like
    the sweep (a graph of `reps` back-to-back launches after 20 untimed):
    algorithmic bytes (every input read once, every output written once),
    GB/s, % of the 8 TB/s HBM peak and, when given, of the measured device
    copy rate, and the time a device copy of the same bytes takes timed the
    same way (`of_same_size_copy_pct`: that time over the pass's, 100 when
    the pass moves its bytes as fast as a copy of that size).  Each pass
    cycles over enough copies of its buffers that the
    launches between two uses of one copy touch more than 512 MiB: twice the
    256 MiB memory-side cache, so every launch reads and writes HBM."""
    import itertools

    import numpy as np
    import torch

    import ien

    dev, f16 = "cuda", torch.float16
    rng = np.random.default_rng(5)

    def halves(*shape):
        return torch.from_numpy(rng.standard_normal(shape).astype(np.float16)).to(dev)

    def floats(*shape):
        return torch.from_numpy(rng.standard_normal(shape).astype(np.float32)).to(dev)

    # (name, algorithmic bytes, make): make() allocates one copy of the
    # pass's buffers and returns its launch.
    cases = []

    # LayerNorm: BiRefNet 1024x1024, the patch embedding's norm (256x256 tokens x 96) and
    # stage 1's merge norm (128x128 x 384), in place.
    def layer_norm(rows, c):
        x, g, b = halves(rows, c), floats(c), floats(c)
        return lambda: ien.layer_norm(ctx, x, rows, c, c, g, b)

    for rows, c in ((65536, 96), (16384, 384)):
        cases.append((f"layer_norm {rows}x{c}", 2 * rows * c * 2, lambda rows=rows, c=c: layer_norm(rows, c)))

    # Bilinear align-corners: BiRefNet's half-size stage-1 map (128x128 x 96) to 256x256,
    # into a 192-channel map.
    def resize():
        src, dst = halves(128 * 128, 96), halves(256 * 256, 192)
        return lambda: ien.resize(ctx, src, 128, 128, 96, 96, dst, 256, 256, 192)

    cases.append(("resize 128x128x96 -> 256x256", 2 * (128 * 128 + 256 * 256) * 96, resize))

    # Window gather with the block's LayerNorm: SCUNet level 1 (512x768, 32 channels, windows
    # of 8 shifted by 4).
    w = ien.windows(8, 4, 512, 768)

    def window_gather():
        wmap, wg, wb = halves(512 * 768, 32), floats(32), floats(32)
        tokens = torch.empty((ien.window_count(w) * 64, 32), dtype=f16, device=dev)
        return lambda: ien.window_gather(ctx, w, wmap, 32, 32, wg, wb, tokens)

    cases.append(("window_gather 512x768x32 w8 s4", 2 * 2 * 512 * 768 * 32, window_gather))

    # 2x2 gather and scatter: SCUNet's halving (512x768 x 64 -> 256x384 rows of 256) and doubling.
    def gather_2x2():
        gmap, grows = halves(512 * 768, 64), torch.empty((256 * 384, 256), dtype=f16, device=dev)
        return lambda: ien.gather_2x2(ctx, gmap, 512, 768, 64, 64, ien.ORDER_ROW_MAJOR, grows)

    cases.append(("gather_2x2 512x768x64", 2 * 2 * 512 * 768 * 64, gather_2x2))

    def scatter_2x2():
        srows, smap = halves(256 * 384, 128), torch.empty((512 * 768, 32), dtype=f16, device=dev)
        return lambda: ien.scatter_2x2(ctx, srows, 128, 256, 384, 32, smap, 32)

    cases.append(("scatter_2x2 256x384x128 -> 512x768x32", 2 * 2 * 256 * 384 * 128, scatter_2x2))

    # Residual add: SCUNet level 1 (512x768 x 64).
    def add():
        ax, ay = halves(512 * 768 * 64), halves(512 * 768 * 64)
        return lambda: ien.add(ctx, ax, ay)

    cases.append(("add 512x768x64", 3 * 512 * 768 * 64 * 2, add))

    # Pixel shuffle x4 plus the repeated image: Real-ESRGAN at 256x384 (the path outside the chain).
    def shuffle():
        last, img = halves(256 * 384, 48), floats(256, 384, 3)
        sh_out = torch.empty((1024, 1536, 3), dtype=torch.float32, device=dev)
        return lambda: ien.pixel_shuffle_add(ctx, last, 48, img, 384, 256, sh_out)

    cases.append(("pixel_shuffle_add 256x384", 256 * 384 * (48 * 2 + 12) + 1024 * 1536 * 12, shuffle))

    # f32 -> f16: BiRefNet's 1024x1024 RGB input; u8 -> f32: the same as bytes.
    def to_halves():
        fimg, himg = floats(1024 * 1024 * 3), torch.empty(1024 * 1024 * 3, dtype=f16, device=dev)
        return lambda: ien.floats_to_halves(ctx, fimg, himg)

    cases.append(("floats_to_halves 1024x1024x3", 1024 * 1024 * 3 * 6, to_halves))

    def to_floats():
        bimg = torch.from_numpy(rng.integers(0, 256, 1024 * 1024 * 3, dtype=np.uint8)).to(dev)
        fimg = torch.empty(1024 * 1024 * 3, dtype=torch.float32, device=dev)
        return lambda: ien.bytes_to_floats(ctx, bimg, fimg)

    cases.append(("bytes_to_floats 1024x1024x3", 1024 * 1024 * 3 * 5, to_floats))

    # The same bytes moved by a plain device copy (half of them read, half
    # written), timed the same way: what a pass of that size can reach when
    # its fixed costs (the launch, the first loads' latency, the tail) weigh
    # as much as its traffic.
    def same_size_copy(nbytes):
        n = max(8, int(nbytes) // 4)  # halves: 2n bytes read + 2n written
        src, dst = halves(n), torch.empty(n, dtype=f16, device=dev)
        return lambda: dst.copy_(src)

    def timed(nbytes, make):
        copies = max(2, -(-(512 << 20) // int(nbytes)) + 1)
        launches = [make() for _ in range(copies)]
        turn = itertools.cycle(launches)
        launch = lambda: next(turn)()  # noqa: E731
        for _ in range(20):
            launch()
        ms = event_time(launch, reps, stream)
        del launches, launch, turn
        torch.cuda.empty_cache()
        return ms, copies

    results = []
    for name, nbytes, make in cases:
        ms, copies = timed(nbytes, make)
        copy_ms, _ = timed(nbytes, lambda nbytes=nbytes: same_size_copy(nbytes))
        gbs = nbytes / (ms * 1e-3) / 1e9
        row = {"pass": name, "bytes": int(nbytes), "us": round(ms * 1e3, 2), "gbs": round(gbs, 0),
               "hbm_pct": round(100 * gbs / HBM_PEAK_GBS, 1), "copies": copies,
               "same_size_copy_us": round(copy_ms * 1e3, 2),
               "of_same_size_copy_pct": round(100 * copy_ms / ms, 1)}
        if copy_tbps:
            row["copy_pct"] = round(100 * gbs / (copy_tbps * 1000), 1)
        results.append(row)
    return results


def counters_from_profiles(cfg):
    """The counter-derived figures of one configuration from its committed
    summary (profiles/<cfg>_counters.md, made from `--counter-probe` runs
    under rocprofv3 --pmc): rocprof_frac (algorithmic GFLOP over the
    serialized kernel time, of the f16 peak), mfma_busy_pct, traffic bytes
    per image and their ratio to the compulsory bytes; None without it."""
    path = ROOT / "profiles" / f"{cfg}_counters.md"
    if not path.exists():
        return None
    out = {}
    for key in ("rocprof_frac", "mfma_busy_pct", "traffic_bytes_per_image", "traffic_ratio", "serial_kernel_us"):
        m = re.search(rf"^{key}:\s*([0-9.eE+-]+)", path.read_text(), re.M)
        if m:
            out[key] = float(m.group(1))
    out["source"] = f"profiles/{cfg}_counters.md"
    return out


def sweep_counters_from_profiles():
    """Per sweep shape: traffic bytes per launch, its ratio to the
    algorithmic bytes, MFMA busy % and rocprof_frac (profiles/sweep_counters.md)."""
    path = ROOT / "profiles" / "sweep_counters.md"
    if not path.exists():
        return {}
    out = {}
    for m in re.finditer(r"^shape (\S+): (.*)$", path.read_text(), re.M):
        f = m.group(2).split()
        out[m.group(1)] = {f[i]: float(f[i + 1]) for i in range(0, len(f) - 1, 2)}
    return out


def traffic_from_profiles():
    path = ROOT / "profiles" / "realesrgan_chain_256x384_hbm_traffic.txt"
    if not path.exists():
        return None
    m = re.search(r"^traffic_bytes_per_launch:\s*([0-9.eE+]+)", path.read_text(), re.M)
    return float(m.group(1)) if m else None


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_threads():
    return len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()


def cpu_time(fn, runs):
    """Median seconds of `runs` calls of fn after one warm-up call (the
    reference's protocol, README.md:26-27)."""
    fn()
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2]


def oracle_module():
    sys.path.insert(0, str(ROOT))
    from oracle import oracle as O

    return O


def cpu_leg(fn, runs, what):
    """cpu_baseline of one configuration: the oracle (C restatement of the
    reference CPU f32 path) on this host's cores."""
    threads = cpu_threads()
    sec = cpu_time(lambda: fn(threads), runs)
    return {"value": round(sec * 1e3, 1), "unit": "ms/image", "cores": threads, "kind": "port",
            "sample": f"{what}, median of {runs} runs after a warm-up, {threads} threads on {cpu_model()}; "
                      f"the oracle (C restatement of the reference CPU f32 path, not the reference's "
                      f"AVX2 build: a conservative baseline)"}


def cpu_baseline(tensors, image, runs):
    O = oracle_module()
    import synthetic

    layers = synthetic.esrgan_layers(tensors)
    return cpu_leg(lambda t: O.realesrgan_run(layers, image, threads=t), runs, "one full 1x3x256x384 image")


def cpu_sweep(runs):
    """The conv sweep's shapes on the oracle: conv3 (Winograd, the
    reference's 3x3 path), multiply (1x1) and the direct depthwise sum."""
    import numpy as np

    O = oracle_module()
    import synthetic

    out = []
    threads = cpu_threads()
    for entry in synthetic.SWEEP:
        (name, kind, cin, cout, size, h, w), x, wt, bias = synthetic.sweep_case(entry[0])
        x = np.ascontiguousarray(x.transpose(1, 2, 0))
        if kind == "depthwise":
            fn = lambda: O.depthwise(x, wt, bias, threads=threads)
        elif size == 3:
            fn = lambda: O.conv3(x, wt, bias, threads=threads)
        else:
            fn = lambda: O.multiply_conv(x, wt, bias, size=size, threads=threads)
        out.append({"shape": name, "ms": round(cpu_time(fn, runs) * 1e3, 2)})
    return {"shapes": out, "cores": threads, "kind": "port",
            "sample": f"each shape once per run, median of {runs} runs after a warm-up, {threads} threads "
                      f"on {cpu_model()}; the oracle (conv3 F(4x4)/F(2x2) for 3x3, multiply for 1x1)"}


def esrgan_flops(H, W):
    """Algorithmic FLOPs of one Real-ESRGAN x4v3 run: the first layer
    (3 -> 64), the 32 body layers (64 -> 64) and the last (64 -> 48), all 3x3."""
    return (conv_flops(H, W, 3, 64, 3) + 32 * conv_flops(H, W, 64, 64, 3)
            + conv_flops(H, W, 64, 48, 3))


def counter_probe(ctx, name, runs):
    """Counter-pass workload of one configuration (for rocprofv3 --pmc):
    `runs` eager runs of its model on its synthetic input (one dispatch a
    kernel; the branches on their streams), or every sweep shape `runs`
    times; then a copy of 1 GiB (a kernel of known traffic, for scaling
    FETCH_SIZE and WRITE_SIZE) whose source was written before 512 MiB of
    other writes, so that it is read from HBM rather than from the 256 MiB
    memory-side cache."""
    import torch

    import ien
    import synthetic

    dev = "cuda"
    if name == "sweep":
        for entry in synthetic.SWEEP:
            case = SweepCase(ctx, entry[0])
            for _ in range(runs):
                case.launch()
            torch.cuda.synchronize()
            case.free()
        what = f"each conv-sweep shape x{runs}"
    else:
        if name == "esrgan":
            h, w, kind, tensors = 256, 384, ien.MODEL_REALESRGAN, synthetic.esrgan_tensors()
            image, mask, out = synthetic.esrgan_image(h, w), None, (4 * h, 4 * w, 3)
        elif name == "scunet":
            h, w, kind, tensors = 512, 768, ien.MODEL_SCUNET, synthetic.scunet_tensors()
            image, mask, out = synthetic.scunet_image(h, w), None, (h, w, 3)
        elif name == "lama":
            h, w, kind, tensors = 512, 512, ien.MODEL_LAMA, synthetic.lama_tensors()
            image, mask, out = synthetic.lama_image(h, w), synthetic.lama_mask(h, w), (h, w, 3)
        elif name == "birefnet":
            h = w = 1024
            kind, tensors = ien.MODEL_BIREFNET, synthetic.birefnet_tensors()
            image, mask, out = synthetic.birefnet_image(h), None, (h, w)
        else:
            sys.exit(f"unknown counter probe {name!r}")
        model = ien.Model(ctx, kind, tensors=tensors)
        d_in = torch.from_numpy(image).to(dev)
        d_mask = None if mask is None else torch.from_numpy(mask).to(dev)
        d_out = torch.empty(out, dtype=torch.float32, device=dev)
        for _ in range(runs):
            model.run_device(d_in, w, h, d_out, d_mask=d_mask)
        torch.cuda.synchronize()
        model.free()
        what = f"the {name} model x{runs} (eager)"
    a = torch.empty(512 << 20, dtype=torch.float16, device=dev).fill_(1)
    flush = torch.empty(256 << 20, dtype=torch.float16, device=dev).fill_(2)
    c = torch.empty_like(a)
    torch.cuda.synchronize()
    c.copy_(a)
    torch.cuda.synchronize()
    del flush
    print(f"counter probe: {what}, then a 1073741824-byte copy", flush=True)


def traffic_probe(ctx):
    """The dominant kernel's counter-pass workload: the Real-ESRGAN model's
    one launch x10 (eager, the seeded image), then the 1 GiB copy."""
    counter_probe(ctx, "esrgan", 10)


def measured_peaks(ctx, stream, mfma=True):
    """This device's sustained rates beside the published peaks: a
    register-only f16 MFMA loop on every SIMD (ien_measure_mfma; skipped
    without `mfma`) and a 1 GiB device-to-device copy read from HBM (its
    source written before 512 MiB of other writes, so not served by the
    256 MiB memory-side cache), timed with HIP events; the copy's rate
    counts bytes read plus written."""
    import torch

    import ien

    tf, mfma_ms = ien.measure_mfma(ctx, 100000) if mfma else (float("nan"), float("nan"))
    a = torch.empty(512 << 20, dtype=torch.float16, device="cuda").fill_(1)
    c = torch.empty_like(a)
    rates = []
    for _ in range(3):
        flush = torch.empty(256 << 20, dtype=torch.float16, device="cuda").fill_(2)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        c.copy_(a)
        e1.record()
        e1.synchronize()
        rates.append(2 * a.numel() * 2 / (e0.elapsed_time(e1) * 1e-3) / 1e12)
        del flush
    copy = sorted(rates)[1]
    del a, c
    return {"mfma_f16_tflops": round(tf, 1), "mfma_frac_of_published": round(tf / MFMA_F16_PEAK_TFLOPS, 3),
            "mfma_loop_ms": round(mfma_ms, 3), "copy_tbps": round(copy, 3),
            "copy_frac_of_published": round(copy / (HBM_PEAK_GBS / 1000), 3),
            "copy_bytes": 2 << 30}


def host_path_ms(run, reps=3):
    """Median milliseconds of ien_model_run (host buffers: upload, the
    launches, download and synchronisation), after a warm-up."""
    return round(cpu_time(run, reps) * 1e3, 3)


def scunet_leg(ctx, steps, warmup, cpu_runs=0):
    """SCUNet (configuration 3) at 1 x 3 x 512 x 768 with its trunc-normal
    random-init weights, graph replay, input and output in HBM."""
    import torch

    import ien
    import synthetic

    h, w = 512, 768
    tensors = synthetic.scunet_tensors()
    image = synthetic.scunet_image(h, w)
    model = ien.Model(ctx, ien.MODEL_SCUNET, tensors=tensors)
    host_ms = host_path_ms(lambda: model.run(image))
    d_in = torch.from_numpy(image).cuda()
    d_out = torch.empty((h, w, 3), dtype=torch.float32, device="cuda")
    model.set_graph(True)
    for _ in range(warmup):
        model.run_device(d_in, w, h, d_out)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        model.run_device(d_in, w, h, d_out)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    ok = bool(torch.isfinite(d_out).all())
    dev_mib = device_mib()
    model.free()
    del d_in, d_out
    torch.cuda.empty_cache()
    if not ok:
        sys.exit("SCUNet: non-finite output")
    leg = {"workload": "SCUNet 1x3x512x768 (28 Swin-Conv blocks, 64/128/256/512)", "ms_per_image": round(ms, 3),
           "images_per_s": round(1e3 / ms, 2), "gflop_per_image": SCUNET_GFLOP,
           "tflops": round(SCUNET_GFLOP / ms, 1), "mfma_frac": round(SCUNET_GFLOP / ms / MFMA_F16_PEAK_TFLOPS, 4),
           "host_path_ms": host_ms, "device_peak_mib": dev_mib}
    if cpu_runs:
        O = oracle_module()
        names = synthetic.scunet_names()
        leg["cpu_baseline"] = cpu_leg(lambda t: O.scunet_run(tensors, names, image, threads=t), cpu_runs,
                                      "one full 1x3x512x768 image")
    return leg


def lama_gflop(h=512, w=512):
    """Multiply-adds x 2 of Big LaMa's convolutions and products at h x w
    (the Fourier transforms' own arithmetic not counted)."""
    p = h * w
    e = p // 64
    half = (w // 8) // 2 + 1
    macs = p * 196 * 64 + (p // 4) * 576 * 128 + (p // 16) * 1152 * 256 + e * 2304 * 512
    ffc = e * 4608 * 128 + e * 1152 * 384 + e * 384 * 192 + (h // 8) * half * 384 * 384 + e * 192 * 384
    macs += 36 * ffc
    macs += e * 9 * 512 * 256 + (p // 16) * 9 * 256 * 128 + (p // 4) * 9 * 128 * 64 + p * 3136 * 3
    return 2 * macs / 1e9


def lama_leg(ctx, steps, warmup, cpu_runs=0):
    """Big LaMa (configuration 4) at 1 x 4 x 512 x 512 (RGB plus a ~25 %
    rectangle mask) with He-normal random-init weights, graph replay, inputs
    and output in HBM."""
    import torch

    import ien
    import synthetic

    h, w = 512, 512
    tensors = synthetic.lama_tensors()
    image, mask = synthetic.lama_image(h, w), synthetic.lama_mask(h, w)
    model = ien.Model(ctx, ien.MODEL_LAMA, tensors=tensors)
    host_ms = host_path_ms(lambda: model.run(image, mask=mask))
    d_in = torch.from_numpy(image).cuda()
    d_mask = torch.from_numpy(mask).cuda()
    d_out = torch.empty((h, w, 3), dtype=torch.float32, device="cuda")
    model.set_graph(True)
    for _ in range(warmup):
        model.run_device(d_in, w, h, d_out, d_mask=d_mask)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        model.run_device(d_in, w, h, d_out, d_mask=d_mask)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    ok = bool(torch.isfinite(d_out).all())
    dev_mib = device_mib()
    model.free()
    del d_in, d_out
    torch.cuda.empty_cache()
    if not ok:
        sys.exit("LaMa: non-finite output")
    gflop = round(lama_gflop(h, w), 1)
    leg = {"workload": "Big LaMa 1x4x512x512 (18 FFC blocks at 64x64x512)", "ms_per_image": round(ms, 3),
           "images_per_s": round(1e3 / ms, 2), "gflop_per_image": gflop, "tflops": round(gflop / ms, 1),
           "mfma_frac": round(gflop / ms / MFMA_F16_PEAK_TFLOPS, 4), "host_path_ms": host_ms,
           "device_peak_mib": dev_mib}
    if cpu_runs:
        O = oracle_module()
        names = synthetic.lama_names()
        leg["cpu_baseline"] = cpu_leg(lambda t: O.lama_run(tensors, names, image, mask, threads=t), cpu_runs,
                                      "one full 1x4x512x512 image and mask")
    return leg


def birefnet_gflop(side=1024, window=12, padded=True):
    """Multiply-adds x 2 of BiRefNet-lite at side x side: both backbone runs
    (the window products over the grids padded to whole windows, as the
    kernels compute them, or over the tokens alone), the decoder's
    convolutions and products, the head and the full-resolution branch's two
    convolutions."""
    n = window * window
    macs = 0
    for s0 in (side, side // 2):
        g = s0 // 4
        macs += g * g * 48 * 96
        for s, (c, depth) in enumerate(((96, 2), (192, 2), (384, 6), (768, 2))):
            gp = -(-g // window) * window if padded else g
            tp = gp * gp
            macs += depth * (tp * c * 3 * c + tp * 2 * n * c + tp * c * c + g * g * 8 * c * c)
            if s < 3:
                macs += (g // 2) ** 2 * 4 * c * 2 * c
                g //= 2

    def block(g, cin, cout, gate):
        m = g * g * (9 * cin * 64 + 64 * 256 * (1 + 1 + 9 + 49) + 1024 * 64 + 9 * 64 * cout)
        return m + (g * g * (9 * cout * 16 + 16) if gate else 0)

    g4 = side >> 5
    macs += block(g4, 2880, 1536, False)
    for i, ((cin, cout), (pc_in, pc_out)) in enumerate(zip(((1728, 768), (960, 384), (480, 192), (240, 96)),
                                                           ((3072, 192), (768, 192), (192, 96), (48, 48)))):
        g = side >> (3 - i + 2)
        macs += block(g, cin, cout, i < 3)
        if i:
            c = (768, 384, 192)[i - 1]
            macs += g * g * c * c
        macs += g * g * 9 * pc_in * 64 + g * g * 9 * 64 * pc_out
    macs += (side // 4) ** 2 * 96 + side * side * (27 * 64 + 576)
    return 2 * macs / 1e9


def birefnet_leg(ctx, steps, warmup, cpu_runs=0):
    """BiRefNet-lite (configuration 5) at 1 x 3 x 1024 x 1024 N(0, 1),
    window 12, deformable-free ASPP, trunc-normal Swin init, graph replay,
    input and logits in HBM."""
    import torch

    import ien
    import synthetic

    side = 1024
    tensors = synthetic.birefnet_tensors()
    image = synthetic.birefnet_image(side)
    model = ien.Model(ctx, ien.MODEL_BIREFNET, tensors=tensors)
    host_ms = host_path_ms(lambda: model.run(image))
    d_in = torch.from_numpy(image).cuda()
    d_out = torch.empty((side, side), dtype=torch.float32, device="cuda")
    model.set_graph(True)
    for _ in range(warmup):
        model.run_device(d_in, side, side, d_out)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        model.run_device(d_in, side, side, d_out)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    ok = bool(torch.isfinite(d_out).all())
    dev_mib = device_mib()
    model.free()
    del d_in, d_out
    torch.cuda.empty_cache()
    if not ok:
        sys.exit("BiRefNet: non-finite output")
    gflop = round(birefnet_gflop(side, 12), 1)
    leg = {"workload": "BiRefNet-lite 1x3x1024x1024 (Swin-T window 12, deformable-free ASPP)",
           "ms_per_image": round(ms, 3), "images_per_s": round(1e3 / ms, 2), "gflop_per_image": gflop,
           "gflop_unpadded_windows": round(birefnet_gflop(side, 12, padded=False), 1),
           "tflops": round(gflop / ms, 1), "mfma_frac": round(gflop / ms / MFMA_F16_PEAK_TFLOPS, 4),
           "host_path_ms": host_ms, "device_peak_mib": dev_mib}
    if cpu_runs:
        O = oracle_module()
        names = synthetic.birefnet_names(12)
        leg["cpu_baseline"] = cpu_leg(lambda t: O.birefnet_run(tensors, names, image, 12, threads=t), cpu_runs,
                                      "one full 1x3x1024x1024 image")
    return leg


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    ap.add_argument("--cpu-runs", type=int, default=5,
                    help="timed oracle runs per configuration (median, after one warm-up)")
    ap.add_argument("--no-sweep", action="store_true", help="skip the conv sweep")
    ap.add_argument("--no-elementwise", action="store_true", help="skip the memory-bound passes")
    ap.add_argument("--counter-probe", choices=["esrgan", "scunet", "lama", "birefnet", "sweep"],
                    help="only run one configuration eagerly, then a 1 GiB copy (for rocprofv3 --pmc passes)")
    ap.add_argument("--probe-runs", type=int, default=3, help="runs of the counter probe's workload")
    ap.add_argument("--elementwise-only", action="store_true",
                    help="only time the memory-bound passes (and the device copy they are set beside)")
    ap.add_argument("--kernel-reps", type=int, default=100)
    ap.add_argument("--no-models", action="store_true", help="skip the other models (SCUNet, LaMa, BiRefNet)")
    ap.add_argument("--birefnet-only", action="store_true",
                    help="only the BiRefNet leg (the workload of its kernel profile)")
    ap.add_argument("--lama-only", action="store_true",
                    help="only the LaMa leg (the workload of its kernel profile)")
    ap.add_argument("--scunet-only", action="store_true",
                    help="only the SCUNet leg (the workload of its kernel profile)")
    ap.add_argument("--sweep-only", action="store_true",
                    help="only the conv sweep (the workload of its kernel profile)")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="only run the body chain 10 times and a 1 GiB device copy "
                         "(the workload of the FETCH_SIZE / WRITE_SIZE counter passes)")
    ap.add_argument("--peaks", action="store_true",
                    help="only the measured peaks (MFMA loop, device copy)")
    ap.add_argument("--serial-branches", action="store_true",
                    help="run the models' branch streams one after the other (for profiles that "
                         "attribute time to single kernels; not for the bench line)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py runs on one GPU only: this backend has no multi-GPU path "
              "(one image per GPU; see the sharding notes of the design)", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import ien
    import synthetic

    if args.serial_branches:
        os.environ["IEN_SERIAL_BRANCHES"] = "1"
    if not torch.cuda.is_available():
        sys.exit("bench.py needs a GPU")
    torch.cuda.set_device(0)
    global _DEVICE_BASE
    torch.zeros(1, device="cuda")
    _DEVICE_BASE = device_in_use()
    ctx = ien.Context(0)
    stream = ctx.stream
    H, W = 256, 384
    tensors = synthetic.esrgan_tensors()
    if args.peaks:
        print(json.dumps({"measured_peaks": measured_peaks(ctx, stream)}), flush=True)
        return
    if args.traffic_probe:
        traffic_probe(ctx)
        return
    if args.counter_probe:
        counter_probe(ctx, args.counter_probe, args.probe_runs)
        return
    if args.scunet_only:
        print(json.dumps(scunet_leg(ctx, max(1, args.steps // 10), 10)), flush=True)
        return
    if args.lama_only:
        print(json.dumps(lama_leg(ctx, max(1, args.steps // 10), 10)), flush=True)
        return
    if args.birefnet_only:
        print(json.dumps(birefnet_leg(ctx, max(1, args.steps // 10), 10)), flush=True)
        return
    if args.sweep_only:
        print(json.dumps({"gemm_sweep": sweep(ctx, stream, args.kernel_reps)}), flush=True)
        return
    if args.elementwise_only:
        copy = measured_peaks(ctx, stream, mfma=False)["copy_tbps"]
        print(json.dumps({"elementwise": elementwise(ctx, stream, args.kernel_reps, copy)}), flush=True)
        return
    image = synthetic.esrgan_image(H, W)
    model = ien.Model(ctx, ien.MODEL_REALESRGAN, tensors=tensors)
    d_in = torch.from_numpy(image).cuda()
    d_out = torch.empty((4 * H, 4 * W, 3), dtype=torch.float32, device="cuda")
    model.set_graph(True)

    for _ in range(args.warmup):
        model.run_device(d_in, W, H, d_out)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        model.run_device(d_in, W, H, d_out)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_per_step = elapsed * 1e3 / args.steps
    if not bool(torch.isfinite(d_out).all()):
        sys.exit("non-finite output")

    # Dominant kernel: the step's one launch (the whole network as one
    # chain), 100 back-to-back runs from one graph after 100 untimed ones.
    model.set_graph(False)
    run = lambda: model.run_device(d_in, W, H, d_out)  # noqa: E731
    for _ in range(100):
        run()
    kms = event_time(run, 100, stream)
    model.set_graph(True)
    flops = esrgan_flops(H, W)
    achieved = flops / (kms * 1e-3) / 1e12
    roofline = {"bound": "mfma", "achieved": round(achieved, 1), "peak": MFMA_F16_PEAK_TFLOPS,
                "unit": "TFLOP/s", "frac": round(achieved / MFMA_F16_PEAK_TFLOPS, 4),
                "traffic": traffic_from_profiles(),
                "kernel": "conv_pair<chain> (the whole network in one launch: first layer, 32 body "
                          "layers 3x3 64->64 + PReLU, last layer + pixel shuffle, 256x384)",
                "kernel_us": round(kms * 1e3, 2), "flop_per_launch": flops,
                "rocprof": counters_from_profiles("esrgan")}

    host_ms = host_path_ms(lambda: model.run(image))
    memory = {"device_peak_mib": device_mib(), "host_peak_mib": host_peak_mib(),
              "what": "device: the context, the model and the run's input and output, above what was in "
                      "use before the context opened (hipMemGetInfo); host: VmHWM after the Real-ESRGAN "
                      "runs, before any CPU baseline"}
    cpu_runs = 0 if args.no_cpu else args.cpu_runs
    log("Real-ESRGAN timed")
    gemm_sweep = None if args.no_sweep else sweep(ctx, stream, args.kernel_reps)
    log("conv sweep timed")
    models = None
    if not args.no_models:
        models = {}
        for name, leg in (("scunet", scunet_leg), ("lama", lama_leg), ("birefnet", birefnet_leg)):
            models[name] = leg(ctx, max(10, args.steps // 10), 10, cpu_runs)
            models[name]["rocprof"] = counters_from_profiles(name)
            log(f"{name} timed")
    cpu = cpu_baseline(tensors, image, cpu_runs) if cpu_runs else None
    sweep_cpu = cpu_sweep(cpu_runs) if cpu_runs and not args.no_sweep else None
    peaks = measured_peaks(ctx, stream)
    passes = None if args.no_elementwise else elementwise(ctx, stream, args.kernel_reps, peaks["copy_tbps"])
    log("memory-bound passes timed")

    line = {
        "metric": METRIC,
        "value": round(ms_per_step, 4),
        "unit": "ms/image",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded uniform [0,1) image, Kaiming-normal random-init weights)",
        "config": {"workload": "Real-ESRGAN general x4v3 (SRVGGNetCompact), 1x3x256x384 -> 1x3x1024x1536",
                   "global_batch": 1, "height": H, "width": W, "layers": 34, "parallelism": "none",
                   "execution": "one launch per image (the whole network as one chain)"},
        "images_per_s": round(1e3 / ms_per_step, 1),
        "host_path_ms": host_ms,
        "memory": memory,
        "roofline": roofline,
        "cpu_baseline": cpu,
        "gemm_sweep": gemm_sweep,
        "gemm_sweep_cpu": sweep_cpu,
        "elementwise": passes,
        "models": models,
        "measured_peaks": peaks,
        "device": ctx.name,
    }
    model.free()
    ctx.close()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
