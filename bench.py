#!/usr/bin/env python3
"""bench.py -- INT4 GEMV HBM GB/s at the Llama-3-8B decode shapes (plus the FP8
E4M3 per-token quantizer's GB/s) on one MI355X.

A step is one Llama-3-8B decode layer's four INT4 GEMVs (M = 1, group size
128, bf16 activation and output, fp32 accumulation): fused QKV (K 4096,
N 6144), O (4096, 4096), fused gate/up (4096, 28672), down (14336, 4096).
`value` is algorithmic bytes per step (packed weights + fp32 scales + zero
nibbles + x + y: 116 858 880 B) times steps over the wall-clock time of the
timed steps, bracketed by torch.cuda.synchronize().  Inputs are resident in
HBM and rotate over enough copies (> 1 GiB) that the 256 MB Infinity Cache
cannot hold them.  The four GEMVs read independent inputs, and a step is one
kc_gemv_int4_bf16_chain call, which runs them as ONE launch of the fused tile
(gemv_run_kernel); the same call captured in a HIP graph, and the four
kc_gemv_int4_bf16 launches back to back, are timed beside it, and `value` is
the fastest of these (all in `config.launch_modes_GBps`).  The same chain
with each GEMV reading the previous one's output (QKV -> O -> gate/up ->
down, which the library runs launch by launch) is reported as
`dependent_chain`.

`roofline` is for the dominant kernel, the fused launch of the whole layer:
its algorithmic bytes per launch over its average duration, timed with HIP
events on the launch stream; `cpu_baseline` times the CPU oracle's scalar GEMV on the same
inputs on one host thread.  The other BASELINE configurations are reported
beside it, each as algorithmic bytes over the average launch duration:
`gemv_cfg0` (fp32 reference-ABI GEMV, 4096 x 4096), `gemm_cfg3` (MFMA
small-batch GEMM, M = 4/16/64, K 8192, N 28672), `fp8_quant` (cfg1 per-token X
and per-channel W, fp32 [4096, 4096]) and `fp8_cfg4` (SmoothQuant statistics
and the two fused quantizers on bf16 X [16384, 8192] and W [28672, 8192]),
`fp8_gemm_cfg4` (the W8A8 FP8 GEMM on those codes, TFLOP/s against the FP8
matrix peak, with torch._scaled_mm on the same codes beside it) and
`convert_int4` (GPTQ and AWQ checkpoints of the gate/up layer to the layout) and
`decode_fusion` (the RMSNorm in front of the QKV and gate/up GEMVs, fused into
the GEMV, against two launches).

    python bench.py [--gpus 1] [--steps 200] [--warmup 20]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT / "kernel-craft_amd" / "python", ROOT / "oracle"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

METRIC = "INT4 GEMV HBM GB/s (% of peak) at M=1 8B shapes; FP8 quant GB/s"
PEAK_HBM_GBS = 8000.0          # MI355X HBM3E, AMD published
PEAK_FP8_TFLOPS = 5000.0       # MI355X dense FP8 matrix peak, AMD published
GS = 128
LLAMA = [("qkv", 6144, 4096), ("o_proj", 4096, 4096), ("gate_up", 28672, 4096),
         ("down", 4096, 14336)]                        # (name, N, K)
DOMINANT = 2                                           # gate/up
ROTATE_BYTES = 1 << 30


def gemv_bytes(n: int, k: int, gs: int = GS, xb: int = 2, yb: int = 2) -> int:
    g = k // gs
    return n * k // 2 + n * g * 4 + n * g // 2 + k * xb + n * yb


def fp8_bytes(rows: int, cols: int) -> int:
    return rows * cols * 4 + rows * cols + rows * 4


GEMV_SOURCES = ("kernel-craft_amd/csrc/gemv_chain.hip", "kernel-craft_amd/csrc/int4_decode.hpp",
                "kernel-craft_amd/csrc/kc_common.hpp")


def source_sha256(paths=GEMV_SOURCES) -> str:
    """sha256 over the dominant kernel's source files, in order."""
    import hashlib
    h = hashlib.sha256()
    for rel in paths:
        h.update((ROOT / rel).read_bytes())
    return h.hexdigest()


def read_traffic(path: Path):
    """(HBM bytes per launch of the dominant kernel, note) from the committed
    rocprofv3 --pmc summary: its `hbm_bytes_per_launch: N` line counts only
    when its `source_sha256:` line matches the sources built now, so that a
    changed kernel never reports the previous kernel's traffic (None then)."""
    try:
        fields = {}
        for line in path.read_text().splitlines():
            if ":" in line and line.strip().split(":", 1)[0] in ("hbm_bytes_per_launch",
                                                               "source_sha256"):
                k, v = line.strip().split(":", 1)
                fields[k] = v.strip()
        if fields.get("source_sha256") != source_sha256():
            return None, f"{path.name}: measured on other kernel sources; re-profile"
        return int(fields["hbm_bytes_per_launch"]), f"{path.name} (sources match)"
    except (OSError, ValueError, KeyError):
        return None, f"{path.name}: unreadable"


def log(*a) -> None:
    print(*a, file=sys.stderr, flush=True)


_SLEEP_CYCLES_PER_MS = None


def enqueue_backlog(torch, ms: float = 20.0) -> None:
    """Queue ~`ms` of idle GPU time (a spinning single-wave kernel) so the
    launches that follow are issued ahead of the GPU and run back to back:
    events then time kernels, not the host.  The backlog must not touch
    memory: a bandwidth-heavy backlog (e.g. filling a large buffer) leaves
    the HBM-bound kernels measured after it about 10 % slower."""
    global _SLEEP_CYCLES_PER_MS
    if _SLEEP_CYCLES_PER_MS is None:  # calibrate torch.cuda._sleep once
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        torch.cuda._sleep(1_000_000)
        e1.record()
        torch.cuda.synchronize()
        _SLEEP_CYCLES_PER_MS = 1_000_000 / max(e0.elapsed_time(e1), 1e-3)
    torch.cuda._sleep(int(_SLEEP_CYCLES_PER_MS * ms))


def time_launches(torch, launch, reps: int) -> float:
    """Average microseconds per launch of `launch(j)` over `reps` back-to-back
    launches on the current stream, timed with HIP events behind a backlog."""
    launch(0)
    torch.cuda.synchronize()
    enqueue_backlog(torch)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for j in range(reps):
        launch(j)
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / reps


def hbm(nbytes: int, us: float) -> dict:
    gbs = nbytes / (us * 1e-6) / 1e9
    return {"avg_us": round(us, 3), "bytes": nbytes, "GBps": round(gbs, 1),
            "frac": round(gbs / PEAK_HBM_GBS, 4)}


def measure_floors(torch, dev, quick: bool = False) -> dict:
    """What plain streams achieve on this GPU, as floors for the path's
    kernels: reads of each GEMV's weight bytes (packed + scales + zeros) and of
    512 MiB; read+write streams with the FP8 quantizers' 4:1 (fp32 -> E4M3)
    and 2:1 (bf16 -> E4M3) traffic at the cfg1 / cfg4 sizes; an empty launch.
    Each is the best over grid sizes and loads in flight per thread
    (build/libkc_probes.so), timed like the path's kernels (events, backlog,
    inputs rotated over 1.5 GiB so that the Infinity Cache cannot serve them)."""
    import ctypes
    probes = ctypes.CDLL(str(ROOT / "build" / "libkc_probes.so"))
    probes.kcp_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
                                       ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    probes.kcp_stream_copy.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
                                       ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    probes.kcp_empty.argtypes = [ctypes.c_int, ctypes.c_void_p]
    buf_bytes = 3 << 29                                       # 1.5 GiB
    buf = torch.empty(buf_bytes, dtype=torch.uint8, device=dev).fill_(3)
    grids = (512, 1024, 2048, 4096) if quick else (512, 1024, 2048, 4096, 8192)
    sink = torch.zeros(max(grids) * 256, dtype=torch.int32, device=dev)
    out = torch.empty(256 << 20, dtype=torch.uint8, device=dev)

    def stream() -> int:
        return torch.cuda.current_stream().cuda_stream

    def best(nbytes, launch_fn, unrolls):
        nbytes -= nbytes % 16
        slots = max(1, (buf_bytes - nbytes) // max(nbytes, 1 << 20))
        reps = 50 if nbytes <= (64 << 20) else 10
        res = None
        for grid in grids:
            for u in unrolls:
                def launch(j, grid=grid, u=u):
                    off = (j % (slots + 1)) * (buf_bytes - nbytes) // max(slots, 1)
                    off -= off % 256
                    rc = launch_fn(buf.data_ptr() + off, nbytes, grid, u)
                    if rc:
                        raise RuntimeError(f"probe launch failed: hipError {rc}")
                us = time_launches(torch, launch, reps)
                if res is None or us < res["avg_us"]:
                    res = {"avg_us": round(us, 3), "grid": grid, "unroll": u}
        return res

    floors = {"read": {}, "copy": {}}
    reads = [(nm, n * k // 2 + n * (k // GS) * 4 + n * (k // GS) // 2) for nm, n, k in LLAMA]
    reads += [("cfg0_weights", 4096 * 2048 + 4096 * 32 * 4 + 4096 * 16),
              ("cfg3_weights", 28672 * 4096 + 28672 * 64 * 4 + 28672 * 32),
              ("512MiB", 512 << 20)]
    for nm, nb in reads:
        r = best(nb, lambda ptr, n, g, u: probes.kcp_stream_read(ptr, n, sink.data_ptr(), g, u,
                                                                  stream()), (4, 8, 16))
        r.update(hbm(nb - nb % 16, r["avg_us"]))
        floors["read"][nm] = r
    copies = [("cfg1_fp32_to_e4m3", 4096 * 4096 * 4, 4),
              ("cfg4_x_bf16_to_e4m3", 16384 * 8192 * 2, 2),
              ("cfg4_w_bf16_to_e4m3", 28672 * 8192 * 2, 2)]
    for nm, nb, ratio in copies:
        r = best(nb, lambda ptr, n, g, u, ratio=ratio: probes.kcp_stream_copy(
            ptr, n, out.data_ptr(), ratio, g, u, stream()), (1, 4, 8))
        r.update(hbm(nb + nb // ratio, r["avg_us"]))
        floors["copy"][nm] = r
    floors["empty_launch_us"] = round(time_launches(
        torch, lambda j: probes.kcp_empty(256, stream()), 200), 3)
    del buf, out, sink
    return floors


def counter_probe(args, torch, lib, dev) -> int:
    """Launch sequences for the rocprofv3 --pmc passes in profiles/ (one kind
    of kernel at a time, so that per-dispatch counters are easy to read)."""
    gen = torch.Generator(device=dev)
    gen.manual_seed(77)
    stream = torch.cuda.current_stream().cuda_stream
    if args.quant_probe:
        n = 4096
        xs = [torch.randn(n, n, device=dev, generator=gen) for _ in range(18)]   # 1.2 GB
        q = torch.empty(n, n, dtype=torch.int8, device=dev)
        s = torch.empty(n, device=dev)
        for j in range(20):
            st = lib.kc_quantize_fp8_per_token_f32(xs[j % len(xs)].data_ptr(), q.data_ptr(),
                                                   s.data_ptr(), n, n, stream)
            if st:
                raise RuntimeError(lib.kc_last_error_string().decode())
        torch.cuda.synchronize()
        src = torch.empty(64 << 20, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(20):
            dst.copy_(src)
        torch.cuda.synchronize()
        print("quant probe done: 20 x cfg1 per-token quantizer, 20 x copy of 67108864 B", flush=True)
        return 0
    # cfg3 GEMMs
    n, k = 28672, 8192
    g = k // GS
    w = [(torch.randint(0, 256, (n, k // 2), dtype=torch.uint8, device=dev, generator=gen),
          torch.empty(n, g, device=dev).uniform_(0.005, 0.02, generator=gen),
          torch.randint(0, 256, (n, g // 2), dtype=torch.uint8, device=dev, generator=gen))
         for _ in range(8)]                                                      # 1 GB
    ws = []                                                                      # the same, shuffled
    for p, _, _ in w:
        sbuf = torch.empty(lib.kc_shuffled_int4_bytes(n, k), dtype=torch.uint8, device=dev)
        if lib.kc_shuffle_int4_mfma(p.data_ptr(), sbuf.data_ptr(), n, k, stream):
            raise RuntimeError(lib.kc_last_error_string().decode())
        ws.append(sbuf)
    torch.cuda.synchronize()
    for fn, shuffled in ((lib.kc_gemm_int4_bf16, False), (lib.kc_gemm_int4_bf16_shuffled, True)):
        for m in (4, 16, 64):
            x = torch.randn(m, k, device=dev, generator=gen).to(torch.bfloat16)
            y = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
            for j in range(10):
                p, sc, z = w[j % len(w)]
                wp = ws[j % len(ws)] if shuffled else p
                st = fn(wp.data_ptr(), sc.data_ptr(), z.data_ptr(), x.data_ptr(), y.data_ptr(), m, n,
                        k, GS, stream)
                if st:
                    raise RuntimeError(lib.kc_last_error_string().decode())
            torch.cuda.synchronize()
    del w, ws
    # the FP8 W8A8 GEMM at the cfg4 consumer shape
    t4, d4, n4 = 16384, 8192, 28672
    qx = torch.randint(-128, 128, (t4, d4), dtype=torch.int8, device=dev, generator=gen)
    qw = torch.randint(-128, 128, (n4, d4), dtype=torch.int8, device=dev, generator=gen)
    qx[(qx & 0x7F) == 0x7F] = 0                    # no NaN codes
    qw[(qw & 0x7F) == 0x7F] = 0
    sx = torch.rand(t4, device=dev, generator=gen)
    sw = torch.rand(n4, device=dev, generator=gen)
    y4 = torch.empty(t4, n4, dtype=torch.bfloat16, device=dev)
    for _ in range(3):
        st = lib.kc_gemm_fp8_w8a8_bf16(qx.data_ptr(), sx.data_ptr(), qw.data_ptr(), sw.data_ptr(),
                                       y4.data_ptr(), t4, n4, d4, stream)
        if st:
            raise RuntimeError(lib.kc_last_error_string().decode())
    torch.cuda.synchronize()
    # the vendor library on the same codes and scales, for its counters beside ours
    a8, b8 = qx.view(torch.float8_e4m3fn), qw.view(torch.float8_e4m3fn)
    for _ in range(3):
        torch._scaled_mm(a8, b8.t(), scale_a=sx.view(-1, 1), scale_b=sw.view(1, -1),
                         out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    print("mfma probe done: 10 x cfg3 GEMM at M 4, 16, 64 on the reference layout, then on the "
          "shuffled layout; 3 x FP8 GEMM 16384 x 28672 x 8192, then 3 x torch._scaled_mm on the "
          "same codes", flush=True)
    return 0


def cpu_info() -> tuple:
    """(threads the CPU legs use, the CPU model): this process's affinity,
    capped by OMP_NUM_THREADS and at 16 (the GPU box's share of host cores)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    try:
        n = min(n, int(os.environ.get("OMP_NUM_THREADS", n)))
    except ValueError:
        pass
    model = "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return max(1, min(n, 16)), model


def cpu_baseline(torch, np, layer, xs, layer_bytes: int, seconds: float) -> dict:
    """The CPU oracle's scalar loops timed on this host, on the same
    algorithmic-byte basis as the GPU numbers: the decode layer's four INT4
    GEMVs (the metric), and the cfg1 FP8 per-token quantizer (the reference
    has no CPU FP8 path, so the oracle's is the baseline).  Each on one
    thread and on all the threads cpu_info() allows; `seconds` bounds the
    whole sample."""
    import kc_oracle
    threads, model = cpu_info()
    host = []
    for i, (_, n, k) in enumerate(LLAMA):
        p, s, z = layer[i]
        host.append((p.cpu().numpy(), s.cpu().numpy(), z.cpu().numpy(),
                     xs[i].view(torch.int16).cpu().numpy().view(np.uint16), n, k))
    rng = np.random.default_rng(1)
    x1 = rng.standard_normal((4096, 4096)).astype(np.float32)
    x1[:, rng.choice(4096, 41, replace=False)] *= np.float32(50.0)

    def run(fn, budget):
        fn()                                          # warm (pages, threads)
        count, t0 = 0, time.perf_counter()
        while True:
            fn()
            count += 1
            if time.perf_counter() - t0 >= budget:
                return count, time.perf_counter() - t0

    def layer_fn(t):
        return lambda: [kc_oracle.gemv_int4_bf16_f32(p, s, z, xb, n, k, GS, threads=t)
                        for p, s, z, xb, n, k in host]

    legs = {}
    for key, t, share in (("single", 1, 0.4), ("all_cores", threads, 0.2)):
        cnt, el = run(layer_fn(t), seconds * share)
        legs[key] = {"value": round(cnt * layer_bytes / el / 1e9, 3), "unit": "GB/s",
                     "threads": t, "sample": f"{cnt} decode layers ({layer_bytes} B each) "
                                             f"in {el:.2f} s"}
    fp8 = {}
    fb = fp8_bytes(4096, 4096)
    for key, t, share in (("single", 1, 0.25), ("all_cores", threads, 0.15)):
        cnt, el = run(lambda t=t: kc_oracle.quantize_fp8_per_token(x1, threads=t), seconds * share)
        fp8[key] = {"value": round(cnt * fb / el / 1e9, 3), "unit": "GB/s", "threads": t,
                    "sample": f"{cnt} x cfg1 X fp32 [4096, 4096] ({fb} B) in {el:.2f} s"}
    out = {"value": legs["all_cores"]["value"], "unit": "GB/s", "cores": threads,
           "kind": "port",
           "sample": (f"oracle scalar C loops (kco_gemv_int4_bf16_f32, rows split over "
                      f"{threads} OpenMP threads) over the decode layer's 4 GEMVs: "
                      f"{legs['all_cores']['sample']}"),
           "single": legs["single"], "all_cores": legs["all_cores"], "fp8_cfg1": fp8,
           "cpu_model": model, "affinity_cpus": len(os.sched_getaffinity(0))
           if hasattr(os, "sched_getaffinity") else None}
    log(f"# cpu baseline ({model}, {threads} threads): GEMV layer single "
        f"{legs['single']['value']} GB/s, all {legs['all_cores']['value']} GB/s; fp8 cfg1 single "
        f"{fp8['single']['value']} GB/s, all {fp8['all_cores']['value']} GB/s")
    return out


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--cpu-seconds", type=float, default=15.0,
                    help="bound on the CPU-baseline sample (0 skips it)")
    ap.add_argument("--no-graph", action="store_true", help="eager launches instead of HIP graphs")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="for rocprofv3 --pmc: launch the decode layer's fused run (one chain "
                         "call) and a plain 64 MiB device copy (the counter calibration) 20 "
                         "times each, then exit")
    ap.add_argument("--quant-probe", action="store_true",
                    help="for rocprofv3 --pmc: launch the cfg1 FP8 per-token quantizer 20 "
                         "times over rotating inputs and the 64 MiB copy 20 times, then exit")
    ap.add_argument("--gemv-probe", action="store_true",
                    help="for rocprofv3 --pmc: each decode-layer GEMV and the cfg0 fp32 GEMV 20 "
                         "times, the stream-read floor kernel over each shape's packed weights "
                         "20 times, and the 64 MiB copy 20 times, then exit")
    ap.add_argument("--floor-probe", action="store_true",
                    help="measure only the stream floors (reads of each GEMV's weight bytes, "
                         "quantizer-shaped copies, an empty launch), print them as JSON, exit")
    ap.add_argument("--mfma-probe", action="store_true",
                    help="for rocprofv3 --pmc: launch the cfg3 GEMMs (M 4, 16, 64; reference, then "
                         "shuffled layout) 10 times "
                         "each and the FP8 W8A8 GEMM (cfg4 shape) 3 times, then exit")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py: this build runs on one GPU only (the quantized GEMV/FP8 path has no "
              "multi-GPU code); run with --gpus 1", file=sys.stderr)
        return 2

    import numpy as np
    import torch
    import kernel_craft_torch_ops as ops

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 1
    lib = ops._get_lib()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    log(f"# {lib.kc_version().decode()} on {torch.cuda.get_device_name(dev)}")

    if args.quant_probe or args.mfma_probe:
        return counter_probe(args, torch, lib, dev)
    if args.floor_probe:
        print(json.dumps({"floors": measure_floors(torch, dev)}), flush=True)
        return 0

    # ---- inputs (BASELINE cfg2 distributions), rotated over > 1 GiB --------
    layer_bytes = sum(gemv_bytes(n, k) for _, n, k in LLAMA)
    w_bytes = sum(n * k // 2 + n * (k // GS) * 4 + n * (k // GS) // 2 for _, n, k in LLAMA)
    copies = max(2, math.ceil(ROTATE_BYTES / w_bytes))
    gen = torch.Generator(device=dev)
    gen.manual_seed(2024)

    def new_weights(n: int, k: int) -> tuple:
        g = k // GS
        packed = torch.randint(0, 256, (n, k // 2), dtype=torch.uint8, device=dev, generator=gen)
        scales = torch.empty(n, g, device=dev).uniform_(0.005, 0.02, generator=gen)
        zeros = torch.randint(0, 256, (n, g // 2), dtype=torch.uint8, device=dev, generator=gen)
        return packed, scales, zeros
    layers = [[new_weights(n, k) for _, n, k in LLAMA] for _ in range(copies)]
    # a timing loop that launches one projection back to back rotates over
    # that projection's own copies, at least ROTATE_BYTES of them: the layer's
    # ten copies of QKV (135 MB) or O (90 MB) alone would fit in the cache
    pools = []
    for i, (_, n, k) in enumerate(LLAMA):
        need = max(copies, math.ceil(ROTATE_BYTES / (n * k // 2 + n * (k // GS) * 9 // 2)))
        pools.append([layers[r][i] for r in range(copies)]
                     + [new_weights(n, k) for _ in range(need - copies)])
    xs = [torch.randn(k, device=dev, generator=gen).to(torch.bfloat16) for _, _, k in LLAMA]
    ys = [torch.empty(n, dtype=torch.bfloat16, device=dev) for _, n, _ in LLAMA]
    fn = lib.kc_gemv_int4_bf16

    def launch_w(w: tuple, i: int) -> None:
        _, n, k = LLAMA[i]
        p, s, z = w
        st = fn(p.data_ptr(), s.data_ptr(), z.data_ptr(), xs[i].data_ptr(), ys[i].data_ptr(),
                n, k, GS, torch.cuda.current_stream().cuda_stream)
        if st:
            raise RuntimeError(f"kc_gemv_int4_bf16 failed: {lib.kc_last_error_string().decode()}")

    def launch(r: int, i: int) -> None:         # copy r of the layer
        launch_w(layers[r][i], i)

    def launch_op(j: int, i: int) -> None:      # the j-th launch of projection i alone
        launch_w(pools[i][j % len(pools[i])], i)

    if args.gemv_probe:
        # every decode shape and the cfg0 fp32 GEMV, 20 launches each over
        # rotating weights, each followed by 20 launches of the stream-read
        # floor kernel over the same number of bytes (packed + scales +
        # zeros, from a 1.5 GiB buffer at rotating offsets, with the grid and
        # unroll measure_floors found best for that size on MI355X), then the
        # 64 MiB copy that calibrates FETCH_SIZE
        import ctypes
        probes = ctypes.CDLL(str(ROOT / "build" / "libkc_probes.so"))
        probes.kcp_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
                                           ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
        floor_shape = {"qkv": (4096, 16), "o_proj": (2048, 8), "gate_up": (2048, 16),
                       "down": (2048, 16)}
        sink = torch.zeros(4096 * 256, dtype=torch.int32, device=dev)
        fbuf_bytes = 3 << 29
        fbuf = torch.empty(fbuf_bytes, dtype=torch.uint8, device=dev).fill_(3)
        x32 = torch.randn(4096, device=dev, generator=gen)
        y32 = torch.empty(4096, device=dev)
        for i, (name, n, k) in enumerate(LLAMA):
            for j in range(20):
                launch_op(j, i)
            torch.cuda.synchronize()
            wb = n * k // 2 + n * (k // GS) * 4 + n * (k // GS) // 2
            wb -= wb % 16
            slots = (fbuf_bytes - wb) // wb
            grid, unroll = floor_shape[name]
            for j in range(20):
                off = (j % (slots + 1)) * ((fbuf_bytes - wb) // slots)
                off -= off % 256
                assert off + wb <= fbuf_bytes
                rc = probes.kcp_stream_read(fbuf.data_ptr() + off, wb, sink.data_ptr(), grid,
                                            unroll, torch.cuda.current_stream().cuda_stream)
                if rc:
                    raise RuntimeError(f"probe launch failed: hipError {rc}")
            torch.cuda.synchronize()
            print(f"gemv probe: {name} x 20, floor read of {wb} B x 20", flush=True)
        del fbuf
        # the decode layer's four GEMVs in one launch of the fused tile
        import ctypes
        arrs = []
        for r in range(copies):
            arr = (ops.GemvOp * len(LLAMA))()
            for i, (_, n, k) in enumerate(LLAMA):
                p, s_, z = layers[r][i]
                arr[i] = ops.GemvOp(p.data_ptr(), s_.data_ptr(), z.data_ptr(), xs[i].data_ptr(),
                                    ys[i].data_ptr(), n, k, GS, 0)
            arrs.append(arr)
        for j in range(20):
            st = lib.kc_gemv_int4_bf16_chain(ctypes.cast(arrs[j % copies], ctypes.c_void_p),
                                             len(LLAMA), torch.cuda.current_stream().cuda_stream)
            if st:
                raise RuntimeError(lib.kc_last_error_string().decode())
        torch.cuda.synchronize()
        print("gemv probe: the fused decode layer x 20", flush=True)
        o = 1                                    # O projection's weights, fp32 x and y
        for j in range(20):
            p, s_, z = pools[o][j % len(pools[o])]
            st = lib.kc_gemv_int4_f32_async(p.data_ptr(), s_.data_ptr(), z.data_ptr(),
                                            x32.data_ptr(), y32.data_ptr(), 4096, 4096, GS,
                                            torch.cuda.current_stream().cuda_stream)
            if st:
                raise RuntimeError(lib.kc_last_error_string().decode())
        torch.cuda.synchronize()
        src = torch.empty(64 << 20, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(20):
            dst.copy_(src)
        torch.cuda.synchronize()
        print("gemv probe done: cfg0 x 20, 20 x copy of 67108864 B", flush=True)
        return 0


    # ---- parity guard: every shape against an fp32 reference --------------
    for i, (name, n, k) in enumerate(LLAMA):
        launch(0, i)
        p, s, z = layers[0][i]
        W = torch.empty(n, k, dtype=torch.float32, device=dev)
        lib.launch_dequantize_int4(p.data_ptr(), s.data_ptr(), z.data_ptr(), W.data_ptr(),
                                   n, k, GS, torch.cuda.current_stream().cuda_stream)
        ref = W @ xs[i].float()
        err = (ys[i].float() - ref).norm() / ref.norm()
        del W
        if not err < 1e-2:
            print(f"bench.py: parity guard failed for {name}: rel L2 {err:.3e}", file=sys.stderr)
            return 1
        log(f"# parity {name}: rel L2 {err:.2e}")

    # ---- a step: the layer's four GEMVs from one chain call (one launch of the
    # fused tile: the inputs are independent), the same call replayed from a
    # HIP graph, and the four stand-alone launches; `value` is the fastest.
    import ctypes

    def chain_arrays(xs_, ys_):
        arrs = []
        for r in range(copies):
            arr = (ops.GemvOp * len(LLAMA))()
            for i, (_, n, k) in enumerate(LLAMA):
                p, s, z = layers[r][i]
                arr[i] = ops.GemvOp(p.data_ptr(), s.data_ptr(), z.data_ptr(), xs_[i].data_ptr(),
                                    ys_[i].data_ptr(), n, k, GS, 0)
            arrs.append(arr)
        return arrs

    chains = chain_arrays(xs, ys)
    # the host work of a step is one foreign call with arguments prepared
    # here (the op array's address, the stream handle), as a native caller's
    # would be: with ~21 us of GPU work per step, per-step Python overhead
    # (torch.cuda.current_stream() alone costs microseconds) would otherwise
    # leave the GPU waiting for the host
    chain_fn = lib.kc_gemv_int4_bf16_chain
    n_ops = len(LLAMA)
    main_stream = torch.cuda.current_stream().cuda_stream

    def chain_ptrs(arrs):
        return [ctypes.cast(a, ctypes.c_void_p) for a in arrs]

    chain_p = chain_ptrs(chains)

    def step_chain(j: int, arrs=chain_p, stream=None) -> None:
        st = chain_fn(arrs[j % copies], n_ops, main_stream if stream is None else stream)
        if st:
            raise RuntimeError(f"kc_gemv_int4_bf16_chain failed: {lib.kc_last_error_string().decode()}")

    per_op_args = [[(p.data_ptr(), s_.data_ptr(), z.data_ptr(), xs[i].data_ptr(), ys[i].data_ptr(),
                     n, k, GS) for i, ((_, n, k), (p, s_, z)) in enumerate(zip(LLAMA, layers[r]))]
                   for r in range(copies)]

    def step_per_op(j: int) -> None:
        for a in per_op_args[j % copies]:
            if fn(*a, main_stream):
                raise RuntimeError(f"kc_gemv_int4_bf16 failed: {lib.kc_last_error_string().decode()}")

    if args.traffic_probe:
        src = torch.empty(64 << 20, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for j in range(20):
            step_chain(j)
        torch.cuda.synchronize()
        for _ in range(20):
            dst.copy_(src)
        torch.cuda.synchronize()
        print("traffic probe done: 20 x the decode layer's fused run, 20 x copy of 67108864 B",
              flush=True)
        return 0

    # parity of the fused run: every projection of the chain's output against
    # its own stand-alone launch (the chain's tile repeats the per-lane-x
    # GEMV; gate/up's stand-alone kernel sums in another order)
    step_chain(0)
    torch.cuda.synchronize()
    fused_out = [y.clone() for y in ys]
    for i, (name, n, k) in enumerate(LLAMA):
        launch(0, i)
        torch.cuda.synchronize()
        err = ((fused_out[i].float() - ys[i].float()).norm() / ys[i].float().norm()).item()
        if not err < 3e-3:
            print(f"bench.py: fused run differs from the stand-alone GEMV for {name}: rel L2 "
                  f"{err:.3e}", file=sys.stderr)
            return 1
        log(f"# fused run {name}: rel L2 {err:.2e} against the stand-alone launch")

    graphs = None
    if not args.no_graph:
        try:
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            graphs = []
            with torch.cuda.stream(side):
                for r in range(copies):
                    gph = torch.cuda.CUDAGraph()
                    with torch.cuda.graph(gph, stream=side):
                        step_chain(r, stream=side.cuda_stream)
                    graphs.append(gph)
            torch.cuda.current_stream().wait_stream(side)
        except Exception as e:  # pragma: no cover - depends on the runtime
            log(f"# graph capture unavailable ({e})")
            graphs = None

    def step_graph(j: int) -> None:
        graphs[j % copies].replay()

    def timed(step) -> float:
        torch.cuda.synchronize()
        for j in range(args.warmup):
            step(j)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for j in range(args.steps):
            step(args.warmup + j)
        torch.cuda.synchronize()
        return time.perf_counter() - t0

    modes = {"one_launch_chain": timed(step_chain), "per_op_launches": timed(step_per_op)}
    if graphs is not None:
        modes["hip_graph"] = timed(step_graph)
    for m, t in modes.items():
        log(f"# {m}: {args.steps} steps in {t * 1e3:.3f} ms -> "
            f"{layer_bytes * args.steps / t / 1e9:.1f} GB/s")
    launch_mode = min(modes, key=modes.get)
    elapsed = modes[launch_mode]
    value = layer_bytes * args.steps / elapsed / 1e9
    modes_gbs = {m: round(layer_bytes * args.steps / t / 1e9, 1) for m, t in modes.items()}

    # the decode layer wired as in a decoder: each GEMV reads the previous
    # one's output (O's x from QKV's y, gate/up's from O's, down's from
    # gate/up's), which the chain runs launch by launch
    ys_dep = [torch.empty(n, dtype=torch.bfloat16, device=dev) for _, n, _ in LLAMA]
    xs_dep = [xs[0]] + [ys_dep[i - 1][:k] for i, (_, _, k) in enumerate(LLAMA) if i > 0]
    chains_dep = chain_arrays(xs_dep, ys_dep)
    chain_dep_p = chain_ptrs(chains_dep)
    t_dep = timed(lambda j: step_chain(j, chain_dep_p))
    dependent = {"GBps": round(layer_bytes * args.steps / t_dep / 1e9, 1),
                 "us_per_step": round(t_dep * 1e6 / args.steps, 3),
                 "config": "QKV -> O -> gate/up -> down, each x a slice of the previous y; "
                           "kc_gemv_int4_bf16_chain runs dependent ops launch by launch"}
    log(f"# dependent chain: {dependent['us_per_step']} us/step, {dependent['GBps']} GB/s")

    # ---- the fused launch timed alone (events, backlogged, rotating copies)
    reps = 100
    enqueue_backlog(torch)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for j in range(reps):
        step_chain(j)
    e1.record()
    torch.cuda.synchronize()
    run_us = e0.elapsed_time(e1) * 1e3 / reps
    log(f"# fused run (gemv_run_kernel, the layer in one launch): {run_us:.2f} us/launch, "
        f"{layer_bytes / run_us / 1e3:.1f} GB/s")

    # ---- per-kernel durations with HIP events (launch stream, backlogged) ---
    reps = 100
    kernel_us = {}
    for i, (name, n, k) in enumerate(LLAMA):
        enqueue_backlog(torch)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for j in range(reps):
            launch_op(j, i)
        e1.record()
        torch.cuda.synchronize()
        kernel_us[name] = e0.elapsed_time(e1) * 1e3 / reps
        log(f"# {name:8s} N={n:6d} K={k:6d}: {kernel_us[name]:7.2f} us/launch, "
            f"{gemv_bytes(n, k) / kernel_us[name] / 1e3:7.1f} GB/s")
    # ---- the same GEMVs on the pre-shuffled layout (kc_shuffle_int4_mfma once,
    # then kc_gemm_int4_bf16_shuffled at M = 1): the matrix-core GEMV, which
    # reads each 16-row tile 1 KB at a time; same bytes, same rotation
    ys_sh = [torch.empty(1, n, dtype=torch.bfloat16, device=dev) for _, n, _ in LLAMA]
    xs2 = [x.view(1, -1) for x in xs]
    shuffled_us = {}
    for i, (name, n, k) in enumerate(LLAMA):
        shuf = []
        for p, _, _ in pools[i]:
            sbuf = torch.empty(lib.kc_shuffled_int4_bytes(n, k), dtype=torch.uint8, device=dev)
            if lib.kc_shuffle_int4_mfma(p.data_ptr(), sbuf.data_ptr(), n, k,
                                        torch.cuda.current_stream().cuda_stream):
                raise RuntimeError(f"kc_shuffle_int4_mfma: {lib.kc_last_error_string().decode()}")
            shuf.append(sbuf)

        def launch_shuf(j: int, i=i, n=n, k=k, shuf=shuf) -> None:
            r = j % len(shuf)
            _, s_, z = pools[i][r]
            st = lib.kc_gemm_int4_bf16_shuffled(shuf[r].data_ptr(), s_.data_ptr(), z.data_ptr(),
                                                xs2[i].data_ptr(), ys_sh[i].data_ptr(), 1, n, k,
                                                GS, torch.cuda.current_stream().cuda_stream)
            if st:
                raise RuntimeError(f"kc_gemm_int4_bf16_shuffled: "
                                   f"{lib.kc_last_error_string().decode()}")
        launch_shuf(0)
        launch_op(0, i)
        torch.cuda.synchronize()
        err = ((ys_sh[i].float().view(-1) - ys[i].float()).norm() / ys[i].float().norm()).item()
        if not err < 3e-3:
            print(f"bench.py: shuffled-layout GEMV disagrees for {name}: rel L2 {err:.3e}",
                  file=sys.stderr)
            return 1
        shuffled_us[name] = time_launches(torch, launch_shuf, reps)
        del shuf
        log(f"# {name:8s} shuffled layout: {shuffled_us[name]:7.2f} us/launch "
            f"(reference layout {kernel_us[name]:.2f})")
    shuffled = {"kernel_us": {k: round(v, 3) for k, v in shuffled_us.items()},
                "sum_us": round(sum(shuffled_us.values()), 3),
                "reference_layout_sum_us": round(sum(kernel_us.values()), 3),
                "config": "the decode layer's GEMVs at M = 1 on the pre-shuffled layout "
                          "(kc_shuffle_int4_mfma, kc_gemm_int4_bf16_shuffled), one launch each, "
                          "events as kernel_us"}

    achieved = layer_bytes / (run_us * 1e-6) / 1e9
    traffic, traffic_note = read_traffic(ROOT / "profiles" / "gemv_run_decode_layer_traffic.md")
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS,
                "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": traffic,
                "traffic_source": traffic_note,
                "kernel": "gemv_run_kernel: the decode layer's four GEMVs in one launch",
                "bytes_per_launch": layer_bytes, "avg_us": round(run_us, 3)}

    def stream_ptr() -> int:
        return torch.cuda.current_stream().cuda_stream

    def ck(status: int, name: str) -> None:
        if status:
            raise RuntimeError(f"{name}: {lib.kc_last_error_string().decode()}")

    # ---- BASELINE cfg0: the reference-ABI GEMV (fp32 x and y), 4096 x 4096 --
    n0 = k0 = 4096
    c0_copies = max(2, math.ceil(ROTATE_BYTES / (n0 * k0 // 2)))
    c0 = []
    for _ in range(c0_copies):
        c0.append((torch.randint(0, 256, (n0, k0 // 2), dtype=torch.uint8, device=dev, generator=gen),
                   torch.empty(n0, k0 // GS, device=dev).uniform_(0.005, 0.02, generator=gen),
                   torch.randint(0, 256, (n0, k0 // GS // 2), dtype=torch.uint8, device=dev,
                                 generator=gen)))
    x0 = torch.randn(k0, device=dev, generator=gen)
    y0 = torch.empty(n0, device=dev)

    def launch_cfg0(j: int) -> None:
        p, sc, z = c0[j % c0_copies]
        ck(lib.kc_gemv_int4_f32_async(p.data_ptr(), sc.data_ptr(), z.data_ptr(), x0.data_ptr(),
                                      y0.data_ptr(), n0, k0, GS, stream_ptr()),
           "kc_gemv_int4_f32_async")
    cfg0 = hbm(gemv_bytes(n0, k0, xb=4, yb=4), time_launches(torch, launch_cfg0, reps))
    cfg0["config"] = "cfg0: INT4 GEMV M=1 N=K=4096 gs 128, fp32 x/y (reference ABI kernel)"
    log(f"# cfg0 fp32 GEMV 4096x4096: {cfg0['avg_us']} us, {cfg0['GBps']} GB/s")
    del c0

    # ---- BASELINE cfg3: INT4 small-batch GEMM on MFMA, K 8192, N 28672 -----
    n3, k3 = 28672, 8192
    w3_bytes = n3 * k3 // 2 + n3 * (k3 // GS) * 4 + n3 * (k3 // GS) // 2
    c3_copies = max(2, math.ceil(ROTATE_BYTES / w3_bytes))
    c3 = []
    for _ in range(c3_copies):
        c3.append((torch.randint(0, 256, (n3, k3 // 2), dtype=torch.uint8, device=dev, generator=gen),
                   torch.empty(n3, k3 // GS, device=dev).uniform_(0.005, 0.02, generator=gen),
                   torch.randint(0, 256, (n3, k3 // GS // 2), dtype=torch.uint8, device=dev,
                                 generator=gen)))
    cfg3 = {}
    for m in (4, 16, 64):
        x3 = torch.randn(m, k3, device=dev, generator=gen).to(torch.bfloat16)
        y3 = torch.empty(m, n3, dtype=torch.bfloat16, device=dev)

        def launch_cfg3(j: int, m=m, x3=x3, y3=y3) -> None:
            p, sc, z = c3[j % c3_copies]
            ck(lib.kc_gemm_int4_bf16(p.data_ptr(), sc.data_ptr(), z.data_ptr(), x3.data_ptr(),
                                     y3.data_ptr(), m, n3, k3, GS, stream_ptr()), "kc_gemm_int4_bf16")
        nbytes = w3_bytes + m * k3 * 2 + m * n3 * 2
        r = hbm(nbytes, time_launches(torch, launch_cfg3, 50))
        r["TFLOPs"] = round(2.0 * m * n3 * k3 / (r["avg_us"] * 1e-6) / 1e12, 2)
        cfg3[f"M{m}"] = r
        log(f"# cfg3 MFMA GEMM M={m:2d}: {r['avg_us']} us, {r['GBps']} GB/s, {r['TFLOPs']} TFLOP/s")
    # the same GEMMs on the pre-shuffled layout
    c3s = []
    for p, _, _ in c3:
        sbuf = torch.empty(lib.kc_shuffled_int4_bytes(n3, k3), dtype=torch.uint8, device=dev)
        ck(lib.kc_shuffle_int4_mfma(p.data_ptr(), sbuf.data_ptr(), n3, k3, stream_ptr()),
           "kc_shuffle_int4_mfma")
        c3s.append(sbuf)
    cfg3_shuf = {}
    for m in (4, 16, 64):
        x3 = torch.randn(m, k3, device=dev, generator=gen).to(torch.bfloat16)
        y3 = torch.empty(m, n3, dtype=torch.bfloat16, device=dev)
        y3r = torch.empty(m, n3, dtype=torch.bfloat16, device=dev)

        def launch_cfg3s(j: int, m=m, x3=x3, y3=y3) -> None:
            _, sc, z = c3[j % c3_copies]
            ck(lib.kc_gemm_int4_bf16_shuffled(c3s[j % c3_copies].data_ptr(), sc.data_ptr(),
                                              z.data_ptr(), x3.data_ptr(), y3.data_ptr(), m, n3, k3,
                                              GS, stream_ptr()), "kc_gemm_int4_bf16_shuffled")
        p, sc, z = c3[0]
        ck(lib.kc_gemm_int4_bf16(p.data_ptr(), sc.data_ptr(), z.data_ptr(), x3.data_ptr(),
                                 y3r.data_ptr(), m, n3, k3, GS, stream_ptr()), "kc_gemm_int4_bf16")
        launch_cfg3s(0)
        torch.cuda.synchronize()
        # the same K-split kernel reads both layouts at K 8192 (on the
        # reference layout in pairs of T-blocks): bit-identical outputs
        same = torch.equal(y3.view(torch.int16), y3r.view(torch.int16))
        if not same:
            print(f"bench.py: shuffled-layout GEMM differs at M={m}", file=sys.stderr)
            return 1
        nbytes = w3_bytes + m * k3 * 2 + m * n3 * 2
        r = hbm(nbytes, time_launches(torch, launch_cfg3s, 50))
        r["TFLOPs"] = round(2.0 * m * n3 * k3 / (r["avg_us"] * 1e-6) / 1e12, 2)
        cfg3_shuf[f"M{m}"] = r
        log(f"# cfg3 GEMM, shuffled layout, M={m:2d}: {r['avg_us']} us, {r['GBps']} GB/s")
    del c3, c3s

    # ---- BASELINE cfg1: FP8 per-token X and per-channel W, fp32 [4096, 4096] -
    frows = fcols = 4096
    fcopies = max(2, math.ceil(ROTATE_BYTES / (frows * fcols * 4)))
    fx = [torch.randn(frows, fcols, device=dev, generator=gen) for _ in range(fcopies)]
    outl = torch.randperm(fcols, device=dev, generator=gen)[:fcols // 100]
    for t in fx:
        t[:, outl] *= 50.0                      # 1 % outlier channels x50
    fq = torch.empty(frows, fcols, dtype=torch.int8, device=dev)
    fs = torch.empty(frows, dtype=torch.float32, device=dev)
    qfn = lib.kc_quantize_fp8_per_token_f32

    def launch_fp8(j: int, src=fx) -> None:
        ck(qfn(src[j % len(src)].data_ptr(), fq.data_ptr(), fs.data_ptr(), frows, fcols,
               stream_ptr()), "kc_quantize_fp8_per_token_f32")
    fp8_x = hbm(fp8_bytes(frows, fcols), time_launches(torch, launch_fp8, reps))
    del fx
    fw = [torch.randn(frows, fcols, device=dev, generator=gen) * 0.02 for _ in range(fcopies)]
    fp8_w = hbm(fp8_bytes(frows, fcols),
                time_launches(torch, lambda j: launch_fp8(j, fw), reps))
    del fw
    fp8_us, fp8_gbs = fp8_x["avg_us"], fp8_x["GBps"]
    log(f"# cfg1 fp8 per-token X [{frows}x{fcols}] fp32: {fp8_us} us, {fp8_gbs} GB/s; "
        f"per-channel W: {fp8_w['avg_us']} us, {fp8_w['GBps']} GB/s")

    # ---- BASELINE cfg4: SmoothQuant + FP8, X bf16 [16384, 8192], W bf16 [28672, 8192]
    T4, D4, N4 = 16384, 8192, 28672
    outl4 = torch.randperm(D4, device=dev, generator=gen)[:D4 // 200]

    def new_x4():
        x = torch.randn(T4, D4, device=dev, generator=gen)
        x[:, outl4] *= 100.0                  # 0.5 % outlier channels x100
        return x.to(torch.bfloat16)
    # X (268 MB) and W (470 MB) each rotate over at least ROTATE_BYTES of copies
    X4s = [new_x4() for _ in range(max(2, math.ceil(ROTATE_BYTES / (T4 * D4 * 2))))]
    W4s = [(torch.randn(N4, D4, device=dev, generator=gen) * 0.02).to(torch.bfloat16)
           for _ in range(max(2, math.ceil(ROTATE_BYTES / (N4 * D4 * 2))))]

    def x4(j: int):
        return X4s[j % len(X4s)]

    def w4(j: int):
        return W4s[j % len(W4s)]
    ax, aw, sm = (torch.empty(D4, device=dev) for _ in range(3))
    qx = torch.empty(T4, D4, dtype=torch.int8, device=dev)
    qw = torch.empty(N4, D4, dtype=torch.int8, device=dev)
    sx = torch.empty(T4, device=dev)
    sw = torch.empty(N4, device=dev)

    def cfg4_stats(j: int) -> None:  # one library call: both column maxima and the factors
        ck(lib.kc_smoothquant_stats_bf16(x4(j).data_ptr(), T4, w4(j).data_ptr(), N4, D4, ax.data_ptr(),
                                         aw.data_ptr(), sm.data_ptr(), stream_ptr()),
           "smoothquant stats")

    def cfg4_stats_calls(j: int) -> None:  # the same as three calls (five launches)
        ck(lib.kc_col_absmax_bf16(x4(j).data_ptr(), ax.data_ptr(), T4, D4, stream_ptr()), "absmax X")
        ck(lib.kc_col_absmax_bf16(w4(j).data_ptr(), aw.data_ptr(), N4, D4, stream_ptr()), "absmax W")
        ck(lib.kc_smooth_factors(ax.data_ptr(), aw.data_ptr(), sm.data_ptr(), D4, stream_ptr()),
           "smooth factors")

    def cfg4_qx(j: int) -> None:
        ck(lib.kc_quantize_fp8_smooth_div_bf16(x4(j).data_ptr(), sm.data_ptr(), qx.data_ptr(),
                                               sx.data_ptr(), T4, D4, stream_ptr()), "quantize X")

    def cfg4_qw(j: int) -> None:
        ck(lib.kc_quantize_fp8_smooth_mul_bf16(w4(j).data_ptr(), sm.data_ptr(), qw.data_ptr(),
                                               sw.data_ptr(), N4, D4, stream_ptr()), "quantize W")
    stats_b = T4 * D4 * 2 + N4 * D4 * 2 + 2 * D4 * 4
    qx_b = T4 * D4 * 2 + T4 * D4 + T4 * 4 + D4 * 4
    qw_b = N4 * D4 * 2 + N4 * D4 + N4 * 4 + D4 * 4
    t_stats = time_launches(torch, cfg4_stats, 10)
    t_stats_calls = time_launches(torch, cfg4_stats_calls, 10)
    t_qx = time_launches(torch, cfg4_qx, 10)
    t_qw = time_launches(torch, cfg4_qw, 10)
    fp8_cfg4 = {"stats": dict(hbm(stats_b, t_stats), three_calls_us=round(t_stats_calls, 3)),
                "quantize_x": hbm(qx_b, t_qx),
                "quantize_w": hbm(qw_b, t_qw),
                "total": hbm(stats_b + qx_b + qw_b, t_stats + t_qx + t_qw),
                "config": "cfg4 (X and W rotating over 4 and 3 copies): col absmax X and W + "
                          "smooth factors (alpha 0.5) in one call "
                          "(kc_smoothquant_stats_bf16; three_calls_us: col absmax X, col absmax W, "
                          "factors); X/s per-token and W*s per-channel to E4M3, bf16 in"}
    log(f"# cfg4 smoothquant+fp8: stats {t_stats:.1f} us, X {t_qx:.1f} us "
        f"({fp8_cfg4['quantize_x']['GBps']} GB/s), W {t_qw:.1f} us "
        f"({fp8_cfg4['quantize_w']['GBps']} GB/s), total {fp8_cfg4['total']['GBps']} GB/s")

    # ---- the W8A8 FP8 GEMM consuming cfg4's codes: Y [16384, 28672] bf16 --
    Y4 = torch.empty(T4, N4, dtype=torch.bfloat16, device=dev)

    def gemm_fp8(j: int) -> None:
        ck(lib.kc_gemm_fp8_w8a8_bf16(qx.data_ptr(), sx.data_ptr(), qw.data_ptr(), sw.data_ptr(),
                                     Y4.data_ptr(), T4, N4, D4, stream_ptr()),
           "kc_gemm_fp8_w8a8_bf16")
    gemm_flop = 2.0 * T4 * N4 * D4
    t_gemm = time_launches(torch, gemm_fp8, 10)
    gemm_tf = gemm_flop / (t_gemm * 1e-6) / 1e12
    fp8_gemm = {"value": round(gemm_tf, 1), "unit": "TFLOP/s", "avg_us": round(t_gemm, 2),
                "roofline": {"bound": "mfma", "achieved": round(gemm_tf, 1),
                             "peak": PEAK_FP8_TFLOPS, "unit": "TFLOP/s",
                             "frac": round(gemm_tf / PEAK_FP8_TFLOPS, 4)},
                "config": "cfg4 consumer: Y = sx sw (qx . qw^T), qx [16384, 8192], qw [28672, "
                          "8192] E4M3 from the cfg4 quantizers, bf16 out"}
    # the vendor library on the same codes and scales, for reference
    try:
        a8 = qx.view(torch.float8_e4m3fn)
        b8 = qw.view(torch.float8_e4m3fn)
        sa, sb = sx.view(-1, 1), sw.view(1, -1)

        def lib_gemm(j: int) -> None:
            torch._scaled_mm(a8, b8.t(), scale_a=sa, scale_b=sb, out_dtype=torch.bfloat16)
        t_lib = time_launches(torch, lib_gemm, 10)
        fp8_gemm["torch_scaled_mm_TFLOPs"] = round(gemm_flop / (t_lib * 1e-6) / 1e12, 1)
    except Exception as e:  # noqa: BLE001 - a reference point only
        fp8_gemm["torch_scaled_mm_TFLOPs"] = f"unavailable: {type(e).__name__}"
    log(f"# fp8 gemm cfg4 consumer: {t_gemm:.1f} us, {fp8_gemm['value']} TFLOP/s "
        f"(torch._scaled_mm: {fp8_gemm['torch_scaled_mm_TFLOPs']})")
    # ---- the FP8 linear's prologue: RMSNorm -> per-token FP8 of X [16384, 8192]
    gam4 = torch.empty(D4, device=dev).uniform_(0.5, 1.5, generator=gen).to(torch.bfloat16)
    xn4 = torch.empty(T4, D4, dtype=torch.bfloat16, device=dev)

    def prologue_fused(j: int) -> None:
        ck(lib.kc_rmsnorm_quantize_fp8_bf16(x4(j).data_ptr(), gam4.data_ptr(), 1e-6, qx.data_ptr(),
                                            sx.data_ptr(), T4, D4, stream_ptr()),
           "kc_rmsnorm_quantize_fp8_bf16")

    def prologue_two(j: int) -> None:
        ck(lib.kc_rmsnorm_bf16(x4(j).data_ptr(), gam4.data_ptr(), xn4.data_ptr(), T4, D4, 1e-6,
                               stream_ptr()), "kc_rmsnorm_bf16")
        ck(lib.kc_quantize_fp8_per_token_bf16(xn4.data_ptr(), qx.data_ptr(), sx.data_ptr(), T4,
                                              D4, stream_ptr()), "kc_quantize_fp8_per_token_bf16")
    pro_b = T4 * D4 * 2 + T4 * D4 + T4 * 4 + D4 * 2
    prologue = hbm(pro_b, time_launches(torch, prologue_fused, 10))
    prologue["two_launches_us"] = round(time_launches(torch, prologue_two, 10), 3)
    prologue["config"] = ("RMSNorm (bf16 h [16384, 8192], gamma, eps 1e-6) -> per-token E4M3 "
                          "codes + fp32 scales in one pass (kc_rmsnorm_quantize_fp8_bf16), "
                          "against kc_rmsnorm_bf16 + kc_quantize_fp8_per_token_bf16")
    log(f"# fp8 prologue (rmsnorm -> fp8) cfg4 X: fused {prologue['avg_us']} us "
        f"({prologue['GBps']} GB/s), two launches {prologue['two_launches_us']} us")
    del X4s, W4s, qx, qw, Y4, xn4

    # ---- decode fusion: the RMSNorm in front of the QKV and gate/up GEMVs ----
    # (kc_rmsnorm_bf16 then kc_gemv_int4_bf16, against the fused launch)
    fusion = {"config": "RMSNorm (bf16 h, gamma [4096], eps 1e-5) + INT4 GEMV, two launches "
                        "vs kc_rmsnorm_gemv_int4_bf16; GB/s of the GEMV's algorithmic bytes "
                        "plus gamma"}
    h_ = torch.randn(4096, device=dev, generator=gen).to(torch.bfloat16)
    gam = torch.empty(4096, device=dev).uniform_(0.5, 1.5, generator=gen).to(torch.bfloat16)
    xn = torch.empty(4096, dtype=torch.bfloat16, device=dev)
    for i in (0, 2):
        name, n, k = LLAMA[i]
        yf = torch.empty(n, dtype=torch.bfloat16, device=dev)

        def two(j: int, i=i, n=n, k=k, yf=yf) -> None:
            p, sc, z = pools[i][j % len(pools[i])]
            ck(lib.kc_rmsnorm_bf16(h_.data_ptr(), gam.data_ptr(), xn.data_ptr(), 1, k, 1e-5,
                                   stream_ptr()), "kc_rmsnorm_bf16")
            ck(lib.kc_gemv_int4_bf16(p.data_ptr(), sc.data_ptr(), z.data_ptr(), xn.data_ptr(),
                                     yf.data_ptr(), n, k, GS, stream_ptr()), "kc_gemv_int4_bf16")

        def fused(j: int, i=i, n=n, k=k, yf=yf) -> None:
            p, sc, z = pools[i][j % len(pools[i])]
            ck(lib.kc_rmsnorm_gemv_int4_bf16(h_.data_ptr(), gam.data_ptr(), 1e-5, p.data_ptr(),
                                             sc.data_ptr(), z.data_ptr(), yf.data_ptr(), n, k, GS,
                                             stream_ptr()), "kc_rmsnorm_gemv_int4_bf16")
        nb = gemv_bytes(n, k) + 2 * k
        r = hbm(nb, time_launches(torch, fused, reps))
        r["two_launches_us"] = round(time_launches(torch, two, reps), 3)
        fusion[name] = r
        log(f"# fusion {name}: fused {r['avg_us']} us ({r['GBps']} GB/s), two launches "
            f"{r['two_launches_us']} us")

    # ---- checkpoint conversion: GPTQ and AWQ gate/up layer to the layout ----
    kc_, nc_, gc_ = 4096, 28672, 4096 // GS
    conv_b = (kc_ * nc_ // 2 + gc_ * nc_ // 2 + gc_ * nc_ * 2      # qweight, qzeros, fp16 scales
              + nc_ * kc_ // 2 + nc_ * gc_ * 4 + nc_ * gc_ // 2)   # packed, fp32 scales, zeros
    cv_copies = max(2, math.ceil(ROTATE_BYTES / conv_b))   # sources and outputs, >= 1 GiB
    srcs = [(torch.randint(-2**31, 2**31 - 1, (kc_ // 8, nc_), dtype=torch.int32, device=dev,
                           generator=gen),
             torch.randint(-2**31, 2**31 - 1, (gc_, nc_ // 8), dtype=torch.int32, device=dev,
                           generator=gen),
             torch.empty(gc_, nc_, device=dev).uniform_(0.001, 0.05, generator=gen).half())
            for _ in range(cv_copies)]
    dsts = [(torch.empty(nc_, kc_ // 2, dtype=torch.uint8, device=dev),
             torch.empty(nc_, gc_, device=dev),
             torch.empty(nc_, gc_ // 2, dtype=torch.uint8, device=dev)) for _ in range(cv_copies)]

    def conv_gptq(j: int) -> None:
        (qw_, qz_, s_), (p_, so_, z_) = srcs[j % cv_copies], dsts[j % cv_copies]
        ck(lib.kc_convert_gptq_int4(qw_.data_ptr(), qz_.data_ptr(), s_.data_ptr(), None, kc_, nc_,
                                    GS, 1, p_.data_ptr(), so_.data_ptr(), z_.data_ptr(),
                                    stream_ptr()), "kc_convert_gptq_int4")

    def conv_awq(j: int) -> None:
        (qw_, qz_, s_), (p_, so_, z_) = srcs[j % cv_copies], dsts[j % cv_copies]
        # the same buffers read as AWQ [K, N/8] words (equal byte counts)
        ck(lib.kc_convert_awq_int4(qw_.data_ptr(), qz_.data_ptr(), s_.data_ptr(), kc_, nc_, GS,
                                   p_.data_ptr(), so_.data_ptr(), z_.data_ptr(), stream_ptr()),
           "kc_convert_awq_int4")
    convert = {"gptq": hbm(conv_b, time_launches(torch, conv_gptq, 20)),
               "awq": hbm(conv_b, time_launches(torch, conv_awq, 20)),
               "config": "GPTQ (original format) and AWQ checkpoints of the gate/up layer "
                         "(K 4096, N 28672, group 128) to the reference layout; bytes read + "
                         "written"}
    log(f"# convert gate/up: GPTQ {convert['gptq']['avg_us']} us ({convert['gptq']['GBps']} GB/s), "
        f"AWQ {convert['awq']['avg_us']} us ({convert['awq']['GBps']} GB/s)")
    del srcs, dsts

    # ---- stream floors on this GPU (see measure_floors) ------------------------
    floors = measure_floors(torch, dev, quick=True)
    of_floor = {nm: round(floors["read"][nm]["avg_us"] / kernel_us[nm], 4) for nm, _, _ in LLAMA}
    of_floor["cfg0"] = round(floors["read"]["cfg0_weights"]["avg_us"] / cfg0["avg_us"], 4)
    of_floor["fp8_cfg1_x"] = round(floors["copy"]["cfg1_fp32_to_e4m3"]["avg_us"] / fp8_us, 4)
    of_floor["fp8_cfg4_x"] = round(floors["copy"]["cfg4_x_bf16_to_e4m3"]["avg_us"] / t_qx, 4)
    of_floor["fp8_cfg4_w"] = round(floors["copy"]["cfg4_w_bf16_to_e4m3"]["avg_us"] / t_qw, 4)
    of_floor["fp8_prologue"] = round(floors["copy"]["cfg4_x_bf16_to_e4m3"]["avg_us"]
                                     / prologue["avg_us"], 4)
    floors["kernel_fraction_of_floor"] = of_floor
    log(f"# floors: gate/up read {floors['read']['gate_up']['avg_us']} us, cfg1 copy "
        f"{floors['copy']['cfg1_fp32_to_e4m3']['avg_us']} us; kernel/floor {of_floor}")

    # ---- CPU baseline: the oracle's scalar loops on the host cores ----------
    cpu = None
    if args.cpu_seconds > 0:
        cpu = cpu_baseline(torch, np, layers[0], xs, layer_bytes, args.cpu_seconds)

    out = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(elapsed * 1e3 / args.steps, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int4w-bf16a-f32acc",
        "data": "synthetic",
        "config": {"workload": "int4_gemv_llama3_8b_decode_layer",
                   "shapes_NK": [[n, k] for _, n, k in LLAMA], "group_size": GS, "M": 1,
                   "bytes_per_step": layer_bytes, "rotation_copies": copies,
                   "per_kernel_rotation_copies": {nm: len(pools[i])
                                                  for i, (nm, _, _) in enumerate(LLAMA)},
                   "launch": launch_mode, "launch_modes_GBps": modes_gbs},
        "dependent_chain": dependent,
        "pct_of_peak": round(100.0 * value / PEAK_HBM_GBS, 2),
        "roofline": roofline,
        "kernel_us": {k: round(v, 3) for k, v in kernel_us.items()},
        "kernel_GBps": {nm: round(gemv_bytes(n, k) / (kernel_us[nm] * 1e-6) / 1e9, 1)
                        for nm, n, k in LLAMA},
        "fp8_quant": {"value": round(fp8_gbs, 1), "unit": "GB/s",
                      "config": "cfg1 per-token X fp32 [4096,4096], 1% outlier channels x50",
                      "bytes_per_launch": fp8_bytes(frows, fcols), "avg_us": round(fp8_us, 3),
                      "frac": round(fp8_gbs / PEAK_HBM_GBS, 4),
                      "per_channel_w": fp8_w},
        "fp8_cfg4": fp8_cfg4,
        "fp8_gemm_cfg4": fp8_gemm,
        "gemv_cfg0": cfg0,
        "gemm_cfg3": cfg3,
        "gemm_cfg3_shuffled": cfg3_shuf,
        "gemv_shuffled_layout": shuffled,
        "convert_int4": convert,
        "decode_fusion": fusion,
        "fp8_prologue_cfg4": prologue,
        "floors": floors,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
