"""Benchmark of the attention hot path on one MI355X.

Headline workload (one "step"): the Qwen3-0.6B decode step of configuration 2 —
28 layers, batch 32, GQA 16/8, head_dim 128, block 16, contexts U[60, 600],
each layer with its own 4096-block KV pool (7 GiB in total, so every layer's
43.5 MB of K/V is read cold from HBM rather than from the 256 MB MALL) and the
store of the 32 new K/V rows fused into the same launch.  The 28 launches are
captured once in a HIP graph and replayed, as the engine's decode graph does.

Prints ONE JSON line: value = algorithmic HBM GB/s of the decode step (bytes
defined in voiceagent_amd.workloads.decode_bytes plus the stored rows) over
the timed region; also µs per layer, the roofline object of the decode
kernel, the prefill (config 3) TFLOP/s, the encoder (config 4) time, and the
CPU baseline (the per-sequence fp32 fallback on the host's cores).
"""

from __future__ import annotations

import argparse
import json
import math
import os
import platform
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from voiceagent_amd import ops, workloads  # noqa: E402

METRIC = "decode-attn µs/layer & HBM GB/s at B=32; prefill TFLOP/s; vs CPU ref"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def profiled_traffic(summary: str = "paged_decode_cfg2.md") -> int | None:
    """HBM bytes per decode launch measured by the FETCH_SIZE / WRITE_SIZE
    counter runs recorded in profiles/ (None when no summary is present)."""
    path = os.path.join(ROOT, "profiles", summary)
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1])
    except (OSError, ValueError):
        return None
    return None


def decode_kernel_name() -> str:
    """The decode kernel config 2 runs: the matrix-core kernel unless
    VA_DECODE_KERNEL=general selects the general one."""
    if os.environ.get("VA_DECODE_KERNEL") == "general":
        return "paged_decode_kernel<BF16,128,2,true,false>"
    return "paged_decode_mfma_kernel<BF16,128,2,false,false,false,0>"


TIMINGS: dict[str, dict] = {}  # per timed graph: median / mean / min ms per replay


def timed_graph(fn, steps: int, warmup: int, stream: torch.cuda.Stream, name: str = ""):
    """Capture fn() in a graph, replay warmup + steps times; return the median
    ms per replay.

    Every timed replay is bracketed by its own pair of events on the replay
    stream (so the events bracket exactly the replayed kernels); the median,
    mean and minimum are kept in TIMINGS[name].
    """
    with torch.cuda.stream(stream):
        fn()  # eager warm-up
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        fn()
    torch.cuda.synchronize()
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(steps)]
    with torch.cuda.stream(stream):
        for _ in range(warmup):
            graph.replay()
        torch.cuda.synchronize()
        for start, end in events:
            start.record(stream)
            graph.replay()
            end.record(stream)
    torch.cuda.synchronize()
    times = sorted(start.elapsed_time(end) for start, end in events)
    median = times[len(times) // 2] if len(times) % 2 else 0.5 * (
        times[len(times) // 2 - 1] + times[len(times) // 2])
    if name:
        TIMINGS[name] = {"median_ms": round(median, 5), "mean_ms": round(sum(times) / len(times), 5),
                         "min_ms": round(times[0], 5), "replays": len(times)}
    return median, graph


def gpu_state() -> dict:
    """Clock, performance-level, power and temperature readings of the GPU
    from rocm-smi (best effort: empty when the tool is missing or fails)."""
    import subprocess

    try:
        r = subprocess.run(["rocm-smi", "--showclocks", "--showperflevel", "--showpower",
                            "--showtemp", "--json"], capture_output=True, text=True, timeout=20)
        data = json.loads(r.stdout)
    except Exception as exc:  # noqa: BLE001 - a diagnostic, never fatal
        return {"error": str(exc)[:200]}
    card = next(iter(data.values())) if isinstance(data, dict) and data else {}
    keep = {}
    for key, val in card.items():
        low = key.lower()
        if any(w in low for w in ("clk", "perf", "power", "temp", "throttl")):
            keep[key] = val
    return keep


def copy_calibration(dev, nbytes: int = 256 << 20, reps: int = 3) -> None:
    """A plain device copy of known size (read nbytes, write nbytes), run so a
    counter profile of this command also holds the scale factor between the
    FETCH_SIZE / WRITE_SIZE counters and real bytes."""
    src = torch.empty(nbytes // 2, dtype=torch.bfloat16, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"[calibration] {reps} copies of {nbytes} bytes")


def bench_decode(args, dev, stream):
    lens = workloads.cfg2_lens(0)
    layers = workloads.LAYERS
    log(f"[decode] building 28 layer pools (B=32, ctx {min(lens)}..{max(lens)}, "
        f"sum {sum(lens)})")
    batch = workloads.make_decode_batch(lens, num_blocks=4096, num_layers=layers,
                                        dtype=torch.bfloat16, kv_std=0.5, device=dev, seed=0,
                                        device_rng=True)
    g = torch.Generator(device=dev).manual_seed(7)
    B = batch.num_seqs
    qs = torch.randn(layers, B, workloads.HQ, workloads.HEAD_DIM, generator=g, device=dev
                     ).to(torch.bfloat16)
    nks = (torch.randn(layers, B, workloads.HKV, workloads.HEAD_DIM, generator=g, device=dev)
           * 0.5).to(torch.bfloat16)
    nvs = (torch.randn(layers, B, workloads.HKV, workloads.HEAD_DIM, generator=g, device=dev)
           * 0.5).to(torch.bfloat16)
    outs = torch.empty_like(qs)

    def step():
        for i in range(layers):
            ops.paged_decode(qs[i], batch.k_pools[i], batch.v_pools[i], batch.block_tables,
                             batch.cu_seqlens_k, lens_cumulative=True,
                             max_seq_len=batch.max_seq_len, scale=batch.scale, new_k=nks[i],
                             new_v=nvs[i], new_slots=batch.slot_mapping, out=outs[i],
                             split_tokens=args.split)

    ms, _ = timed_graph(step, args.steps, args.warmup, stream, name="decode_cfg2")
    per_layer_bytes = decode_launch_bytes(lens)
    us_layer = ms * 1000.0 / layers
    gbs = per_layer_bytes / (us_layer * 1e-6) / 1e9
    log(f"[decode] {ms:.3f} ms/step, {us_layer:.2f} us/layer, {gbs:.0f} GB/s "
        f"({per_layer_bytes / 1e6:.2f} MB/layer)")
    return dict(ms=ms, us_layer=us_layer, gbs=gbs, bytes_layer=per_layer_bytes, lens=lens,
                batch=batch, qs=qs, nks=nks, nvs=nvs)


def bench_decode_warm(args, dev, stream, dec):
    """Config 2's step with every one of the 28 launches on layer 0's pool
    (46 MB, resident in the 256 MB MALL after the first): the kernel's own
    start-up, rounds and tail without the cold HBM reads.  Not a headline
    figure; it tells how much of the cold time the HBM reads themselves take."""
    batch, layers = dec["batch"], workloads.LAYERS
    outs = torch.empty_like(dec["qs"])

    def step():
        for i in range(layers):
            ops.paged_decode(dec["qs"][i], batch.k_pools[0], batch.v_pools[0],
                             batch.block_tables, batch.cu_seqlens_k, lens_cumulative=True,
                             max_seq_len=batch.max_seq_len, scale=batch.scale,
                             new_k=dec["nks"][i], new_v=dec["nvs"][i],
                             new_slots=batch.slot_mapping, out=outs[i], split_tokens=args.split)

    ms, _ = timed_graph(step, args.steps, args.warmup, stream, name="decode_cfg2_warm")
    us = ms * 1000.0 / layers
    gbs = dec["bytes_layer"] / (us * 1e-6) / 1e9
    log(f"[decode warm] {us:.2f} us/layer with layer 0's pool in every launch ({gbs:.0f} GB/s; "
        f"cold {dec['us_layer']:.2f})")
    return {"us_per_layer": round(us, 2), "gbs": round(gbs, 1),
            "note": "all 28 launches on layer 0's pool (MALL-resident); not the headline"}


def bench_decode_batches(args, dev, stream):
    """Config 2's decode at larger batches (contexts U[60, 600], 28 cold layers),
    over the bf16 pools and over FP8 copies of them: with several rounds of
    workgroups the dispatcher hands each CU a new pair as it frees, so the
    longest contexts no longer set the end alone.  Reported beside the
    headline, not instead of it."""
    res = {}
    for B in (64, 128, 256):
        lens = workloads.cfg2_lens(0, batch=B)
        blocks = sum(math.ceil(n / workloads.BLOCK) for n in lens) + 64
        batch = workloads.make_decode_batch(lens, num_blocks=blocks, num_layers=workloads.LAYERS,
                                            dtype=torch.bfloat16, kv_std=0.5, device=dev, seed=0,
                                            device_rng=True)
        g = torch.Generator(device=dev).manual_seed(7)
        layers = workloads.LAYERS
        qs = torch.randn(layers, B, workloads.HQ, workloads.HEAD_DIM, generator=g, device=dev
                         ).to(torch.bfloat16)
        nks = (torch.randn(layers, B, workloads.HKV, workloads.HEAD_DIM, generator=g, device=dev)
               * 0.5).to(torch.bfloat16)
        nvs = torch.randn_like(nks) * 0.5
        outs = torch.empty_like(qs)

        def step():
            for i in range(layers):
                ops.paged_decode(qs[i], batch.k_pools[i], batch.v_pools[i], batch.block_tables,
                                 batch.cu_seqlens_k, lens_cumulative=True,
                                 max_seq_len=batch.max_seq_len, scale=batch.scale, new_k=nks[i],
                                 new_v=nvs[i], new_slots=batch.slot_mapping, out=outs[i])

        ms, _ = timed_graph(step, args.steps, args.warmup, stream, name=f"decode_b{B}")
        us = ms * 1000.0 / layers
        nbytes = decode_launch_bytes(lens)
        gbs = nbytes / (us * 1e-6) / 1e9
        log(f"[decode batch] B={B}: {us:.2f} us/layer, {gbs:.0f} GB/s of {nbytes / 1e6:.1f} MB "
            f"({gbs / HBM_PEAK_GBS:.3f} of HBM peak)")
        res[f"b{B}"] = {"us_per_layer": round(us, 2), "gbs": round(gbs, 1),
                        "frac": round(gbs / HBM_PEAK_GBS, 4), "bytes_per_layer": nbytes}
        # The same step over FP8 copies of the pools (half the K/V bytes).
        kf, vf = fp8_pools(batch.k_pools, batch.v_pools)

        def step_fp8():
            for i in range(layers):
                ops.paged_decode(qs[i], kf[i], vf[i], batch.block_tables, batch.cu_seqlens_k,
                                 lens_cumulative=True, max_seq_len=batch.max_seq_len,
                                 scale=batch.scale, new_k=nks[i], new_v=nvs[i],
                                 new_slots=batch.slot_mapping, out=outs[i], k_scale=FP8_SCALE,
                                 v_scale=FP8_SCALE)

        ms8, _ = timed_graph(step_fp8, args.steps, args.warmup, stream, name=f"decode_b{B}_fp8")
        us8 = ms8 * 1000.0 / layers
        nbytes8 = decode_launch_bytes(lens, kv_elem=1)
        gbs8 = nbytes8 / (us8 * 1e-6) / 1e9
        log(f"[decode batch fp8] B={B}: {us8:.2f} us/layer, {gbs8:.0f} GB/s of "
            f"{nbytes8 / 1e6:.1f} MB ({gbs8 / HBM_PEAK_GBS:.3f} of HBM peak)")
        res[f"b{B}"]["fp8"] = {"us_per_layer": round(us8, 2), "gbs": round(gbs8, 1),
                               "frac": round(gbs8 / HBM_PEAK_GBS, 4), "bytes_per_layer": nbytes8}
        del batch, qs, nks, nvs, outs, kf, vf
        torch.cuda.empty_cache()
    return res


def decode_launch_bytes(lens, kv_elem: int = 2) -> int:
    """Algorithmic bytes of one config-2 decode launch (attention + fused
    store): K/V rows of every context token (kv_elem bytes per element: 2 for
    bf16, 1 for FP8 codes), q in and out (bf16), the used block-table entries,
    the lengths, the stored rows and their slots."""
    B = len(lens)
    h, d = workloads.HKV, workloads.HEAD_DIM
    kv = sum(lens) * h * d * kv_elem * 2
    qo = 2 * B * workloads.HQ * d * 2
    tables = sum(math.ceil(n / workloads.BLOCK) for n in lens) * 4
    return kv + qo + tables + 4 * B + 2 * B * h * d * kv_elem + 4 * B


FP8_SCALE = 2.0 ** -4  # k_scale = v_scale of the FP8 rows (a power of two)


def fp8_pools(k_pools, v_pools, scale: float = FP8_SCALE):
    """FP8 (e4m3) copies of 16-bit NHD pools, every slot written by the
    library's own quantising store."""
    ks, vs = [], []
    for kp, vp in zip(k_pools, v_pools):
        nb, bs, hkv, d = kp.shape
        kf = torch.empty(kp.shape, dtype=ops.FP8_KV_DTYPE, device=kp.device)
        vf = torch.empty_like(kf)
        slots = torch.arange(nb * bs, dtype=torch.int32, device=kp.device)
        ops.store_kvcache(kp.view(nb * bs, hkv, d), vp.view(nb * bs, hkv, d), kf, vf, slots,
                          k_scale=scale, v_scale=scale)
        ks.append(kf)
        vs.append(vf)
    torch.cuda.synchronize()
    return ks, vs


def bench_decode_fp8(args, dev, stream, dec):
    """Config 2's decode step over FP8 copies of the 28 layer pools (half the
    K/V bytes); the current rows are stored quantised."""
    batch, layers = dec["batch"], workloads.LAYERS
    kf, vf = fp8_pools(batch.k_pools, batch.v_pools)
    outs = torch.empty_like(dec["qs"])

    def step():
        for i in range(layers):
            ops.paged_decode(dec["qs"][i], kf[i], vf[i], batch.block_tables, batch.cu_seqlens_k,
                             lens_cumulative=True, max_seq_len=batch.max_seq_len,
                             scale=batch.scale, new_k=dec["nks"][i], new_v=dec["nvs"][i],
                             new_slots=batch.slot_mapping, out=outs[i], k_scale=FP8_SCALE,
                             v_scale=FP8_SCALE)

    ms, _ = timed_graph(step, args.steps, args.warmup, stream, name="decode_cfg2_fp8")
    del kf, vf
    us = ms * 1000.0 / layers
    nbytes = decode_launch_bytes(dec["lens"], kv_elem=1)
    gbs = nbytes / (us * 1e-6) / 1e9
    log(f"[fp8] config 2 over FP8 pools: {us:.2f} us/layer, {gbs:.0f} GB/s of {nbytes / 1e6:.2f} "
        f"MB (bf16 pools {dec['us_layer']:.2f} us/layer)")
    return {"us_per_layer": round(us, 2), "gbs": round(gbs, 1),
            "frac": round(gbs / HBM_PEAK_GBS, 4), "bytes_per_layer": nbytes,
            "kv_format": "OCP e4m3 codes, k_scale = v_scale = 2^-4",
            "speedup_vs_bf16_pool": round(dec["us_layer"] / us, 3)}


def bench_host_overhead(dev, dec, pre):
    """Host microseconds per ops.paged_decode and ops.varlen_attention call
    (argument checks, the struct, the C call and the launch), from 300 eager
    calls of config 2's layer 0 and config 3's layer 0 without waiting for the
    GPU."""
    batch = dec["batch"]
    out = torch.empty_like(dec["qs"][0])

    def decode_call():
        ops.paged_decode(dec["qs"][0], batch.k_pools[0], batch.v_pools[0], batch.block_tables,
                         batch.cu_seqlens_k, lens_cumulative=True, max_seq_len=batch.max_seq_len,
                         scale=batch.scale, new_k=dec["nks"][0], new_v=dec["nvs"][0],
                         new_slots=batch.slot_mapping, out=out)

    res = {}
    for name, call in (("paged_decode", decode_call), ("varlen_attention", pre["call0"])):
        for _ in range(20):
            call()
        torch.cuda.synchronize()
        n = 300
        t0 = time.perf_counter()
        for _ in range(n):
            call()
        t1 = time.perf_counter()
        torch.cuda.synchronize()
        res[name] = round((t1 - t0) / n * 1e6, 2)
    log(f"[host] us per call: paged_decode {res['paged_decode']}, varlen_attention "
        f"{res['varlen_attention']}")
    return res


PROBE_MODES = {"plain": 0, "nt": 1, "lds_dma": 2}  # include/voiceagent_bench.h
_BENCH_LIB = None


def bench_lib():
    """libvoiceagent_bench.so (include/voiceagent_bench.h): bench-only probes,
    apart from the drop-in library."""
    global _BENCH_LIB
    if _BENCH_LIB is None:
        import ctypes

        from voiceagent_amd.build import BENCH_LIB_PATH

        lib = ctypes.CDLL(str(BENCH_LIB_PATH))
        lib.va_bench_hbm_read.restype = ctypes.c_int
        lib.va_bench_hbm_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int,
                                          ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
        lib.va_bench_hbm_copy.restype = ctypes.c_int
        lib.va_bench_hbm_copy.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
                                          ctypes.c_size_t, ctypes.c_int, ctypes.c_void_p]
        lib.va_bench_empty.restype = ctypes.c_int
        lib.va_bench_empty.argtypes = [ctypes.c_int, ctypes.c_void_p]
        lib.va_bench_hbm_depth.restype = ctypes.c_int
        lib.va_bench_hbm_depth.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_size_t,
                                           ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                           ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
        lib.va_bench_last_error.restype = ctypes.c_char_p
        lib.va_bench_last_error.argtypes = []
        _BENCH_LIB = lib
    return _BENCH_LIB


def hbm_read(buf: torch.Tensor, workgroups: int, mode: str, sink: torch.Tensor) -> None:
    """Stream the contiguous GPU tensor `buf` once in one launch of
    `workgroups` workgroups through load path `mode` (va_bench_hbm_read); `sink`
    is an int32 tensor of at least `workgroups` elements, never written."""
    if not (buf.is_cuda and buf.is_contiguous() and sink.dtype == torch.int32 and
            sink.numel() >= workgroups):
        raise ValueError("hbm_read needs a contiguous GPU tensor and an int32 sink per workgroup")
    nbytes = buf.numel() * buf.element_size()
    rc = bench_lib().va_bench_hbm_read(buf.data_ptr(), nbytes, int(workgroups), PROBE_MODES[mode],
                                       sink.data_ptr(), torch.cuda.current_stream().cuda_stream)
    if rc != 0:
        raise ValueError(bench_lib().va_bench_last_error().decode())


def hbm_copy(src: torch.Tensor, dst: torch.Tensor, workgroups: int) -> None:
    """Read all of `src` and write all of `dst` (contiguous GPU tensors) in one
    launch of `workgroups` workgroups (va_bench_hbm_copy)."""
    if not (src.is_cuda and dst.is_cuda and src.is_contiguous() and dst.is_contiguous()):
        raise ValueError("hbm_copy needs contiguous GPU tensors")
    rc = bench_lib().va_bench_hbm_copy(src.data_ptr(), src.numel() * src.element_size(),
                                       dst.data_ptr(), dst.numel() * dst.element_size(),
                                       int(workgroups), torch.cuda.current_stream().cuda_stream)
    if rc != 0:
        raise ValueError(bench_lib().va_bench_last_error().decode())


def empty_launch(workgroups: int) -> None:
    """One launch of a kernel that does nothing over `workgroups` 512-lane
    workgroups (va_bench_empty)."""
    rc = bench_lib().va_bench_empty(int(workgroups), torch.cuda.current_stream().cuda_stream)
    if rc != 0:
        raise ValueError(bench_lib().va_bench_last_error().decode())


def launch_floor(args, stream) -> dict:
    """Fixed cost of a launch: 28 launches of an empty kernel per graph
    replay, as the attention legs replay 28 layers, at the decode's grid
    (256 workgroups) and at 2048."""
    table = {}
    for wgs in (256, 2048):
        def step(wgs=wgs):
            for _ in range(workloads.LAYERS):
                empty_launch(wgs)

        ms, _ = timed_graph(step, args.steps, args.warmup, stream)
        table[wgs] = ms * 1000.0 / workloads.LAYERS
    log("[launch floor] empty kernel, 28 launches per graph replay: "
        + ", ".join(f"{w} workgroups {t:.2f}" for w, t in table.items()) + " us/launch")
    return {str(w): round(t, 2) for w, t in table.items()}


def copy_floor(name: str, read_bytes: int, write_bytes: int, launches: int, args, dev,
               stream) -> dict:
    """Mixed read/write floor: `read_bytes` read and `write_bytes` written in
    one launch (va_bench_hbm_copy), `launches` launches per graph replay on
    distinct windows (cold), at several grid sizes; the fastest is reported."""
    rb, wb = read_bytes // 16 * 16, write_bytes // 16 * 16
    rs, ws = (rb + 65535) // 65536 * 65536, (wb + 65535) // 65536 * 65536
    src = torch.ones(rs * launches, dtype=torch.uint8, device=dev)
    dst = torch.zeros(ws * launches, dtype=torch.uint8, device=dev)
    pairs = [(src[i * rs:i * rs + rb], dst[i * ws:i * ws + wb]) for i in range(launches)]
    table = {}
    for wgs in (256, 512, 1024, 2048):
        def step(wgs=wgs):
            for a, b in pairs:
                hbm_copy(a, b, wgs)

        ms, _ = timed_graph(step, args.steps, args.warmup, stream)
        table[wgs] = ms * 1000.0 / launches
    wgs, us = min(table.items(), key=lambda kv: kv[1])
    gbs = (rb + wb) / (us * 1e-6) / 1e9
    log(f"[copy floor] {name}: read {rb / 1e6:.2f} MB + write {wb / 1e6:.2f} MB: "
        + ", ".join(f"{w}: {t:.2f}" for w, t in table.items())
        + f" us/launch; best {us:.2f} us at {wgs} workgroups, {gbs:.0f} GB/s")
    del src, dst, pairs
    return {"us_per_launch": round(us, 2), "gbs": round(gbs, 1), "workgroups": wgs,
            "read_bytes": rb, "write_bytes": wb,
            "us_by_grid": {str(w): round(t, 2) for w, t in table.items()}}


# (DMA KiB, register KiB) in flight per wave; x 8 waves per CU.
DEPTH_CONFIGS = ((4, 0), (8, 0), (16, 0), (0, 4), (0, 8), (8, 4), (8, 8), (16, 4), (16, 8))
# (workgroups, bytes per workgroup): one CU alone, 32 CUs (a decode's tail),
# every CU.
DEPTH_SHAPES = ((1, 8 << 20), (32, 4 << 20), (256, 2 << 20))


def depth_probe(dev, stream) -> list:
    """Per-CU HBM read rate against the bytes one CU keeps in flight
    (va_bench_hbm_depth): every (shape, depth) three timed launches after one
    untimed, each on a window of a 2 GiB buffer not read since it was filled
    (cold: the 256 MB MALL holds the last bytes written or read).  Rates are
    per workgroup, from its own start and end stamps."""
    buf = torch.empty(2 << 30, dtype=torch.uint8, device=dev)
    buf.fill_(1)
    times = torch.zeros(2 * 256, dtype=torch.int64, device=dev)
    sink = torch.zeros(256, dtype=torch.int32, device=dev)
    torch.cuda.synchronize()
    lib, cursor, rows = bench_lib(), 0, []
    for wgs, per_wg in DEPTH_SHAPES:
        for dma, vgpr in DEPTH_CONFIGS:
            unit = 8 * (dma + vgpr) * 1024
            read = per_wg // unit * unit  # bytes a workgroup actually reads
            rates, agg = [], []
            for rep in range(4):
                need = wgs * per_wg
                if cursor + need > buf.numel():
                    cursor = 0
                rc = lib.va_bench_hbm_depth(buf.data_ptr() + cursor, buf.numel() - cursor, per_wg,
                                            wgs, dma, vgpr, times.data_ptr(), sink.data_ptr(),
                                            stream.cuda_stream)
                if rc != 0:
                    raise ValueError(lib.va_bench_last_error().decode())
                stream.synchronize()
                cursor += need
                if rep == 0:
                    continue
                t = times[:2 * wgs].view(wgs, 2).cpu().double()
                dt = (t[:, 1] - t[:, 0]) * 10e-9  # 100 MHz ticks
                rates += (read / dt / 1e9).tolist()
                agg.append(wgs * read / ((t[:, 1].max() - t[:, 0].min()).item() * 10e-9) / 1e9)
            rates.sort()
            rows.append({"workgroups": wgs, "dma_kib_per_cu": 8 * dma, "vgpr_kib_per_cu": 8 * vgpr,
                         "gbs_per_cu_median": round(rates[len(rates) // 2], 1),
                         "gbs_per_cu_min": round(rates[0], 1), "gbs_per_cu_max": round(rates[-1], 1),
                         "gbs_all": round(sum(agg) / len(agg), 1)})
            r = rows[-1]
            log(f"[depth] {wgs:3d} CUs, {8 * dma:3d} KiB DMA + {8 * vgpr:2d} KiB registers in flight "
                f"per CU: {r['gbs_per_cu_median']:.1f} GB/s per CU (min {r['gbs_per_cu_min']:.1f}, "
                f"max {r['gbs_per_cu_max']:.1f}), {r['gbs_all']:.0f} GB/s over all")
    del buf
    return rows


def bench_floor(args, dev, stream):
    """HBM read floor for config 2's launch size: a contiguous read of the
    same number of bytes in one launch (va_bench_hbm_read), 28 launches per
    graph replay on distinct windows of a 1.3 GB buffer (cold, past the 256 MB
    MALL), through three load paths (plain loads, non-temporal loads, the
    decode's non-temporal LDS DMA) at several grid sizes; the fastest
    (path, grid) is reported.  Also the varlen launches' read + write floors
    and the fixed cost of an empty launch."""
    nbytes = decode_launch_bytes(workloads.cfg2_lens(0)) // 16 * 16
    layers = workloads.LAYERS
    stride = (nbytes + 65535) // 65536 * 65536
    buf = torch.ones(stride * layers, dtype=torch.uint8, device=dev)
    sink = torch.zeros(4096, dtype=torch.int32, device=dev)
    views = [buf[i * stride:i * stride + nbytes] for i in range(layers)]
    table = {}
    for mode in PROBE_MODES:
        for wgs in (256, 512, 1024, 2048):
            def step(wgs=wgs, mode=mode):
                for v in views:
                    hbm_read(v, wgs, mode, sink)

            ms, _ = timed_graph(step, args.steps, args.warmup, stream)
            table[(mode, wgs)] = ms * 1000.0 / layers
        log(f"[floor] {mode}: " + ", ".join(f"{w}: {table[(mode, w)]:.2f}"
                                            for w in (256, 512, 1024, 2048)) + " us/launch")
    (mode, wgs), us = min(table.items(), key=lambda kv: kv[1])
    gbs = nbytes / (us * 1e-6) / 1e9
    log(f"[floor] best: {mode} at {wgs} workgroups, {us:.2f} us/launch for "
        f"{nbytes / 1e6:.2f} MB, {gbs:.0f} GB/s ({gbs / HBM_PEAK_GBS:.3f} of peak)")
    del buf, views
    # Mixed floors of the varlen launches: their algorithmic reads (q, k, v)
    # and writes (output, and for prefill the stored K/V rows).
    pre_lens, wins = workloads.cfg3_lens(0), workloads.cfg4_windows(0)
    # varlen_bytes counts q, k, v and out; at GQA 16/8 out is a third of it and
    # the stored K/V rows are as large as k + v.
    pre_r = workloads.varlen_bytes(pre_lens, workloads.HQ, workloads.HKV,
                                   workloads.HEAD_DIM) * 2 // 3  # q + k + v
    pre_w = pre_r  # output + stored K/V rows
    enc_all = workloads.varlen_bytes(wins, 14, 14, 64)
    # store_kvcache of config 3's rows: K and V read, then written.
    st_rw = workloads.store_bytes(sum(pre_lens)) // 2
    copies = {"prefill_cfg3": copy_floor("prefill cfg3", pre_r, pre_w, layers, args, dev, stream),
              "encoder_cfg4": copy_floor("encoder cfg4", enc_all * 3 // 4, enc_all // 4, 18,
                                         args, dev, stream),
              "store_cfg3": copy_floor("store cfg3", st_rw, st_rw, layers, args, dev, stream)}
    empty = launch_floor(args, stream)
    depth = depth_probe(dev, stream)
    return {"us_per_launch": round(us, 2), "gbs": round(gbs, 1), "copy": copies,
            "empty_launch_us": empty, "per_cu_depth": depth,
            "frac": round(gbs / HBM_PEAK_GBS, 4), "bytes": nbytes, "mode": mode,
            "workgroups": wgs,
            "us_by_mode_grid": {f"{m}/{w}": round(t, 2) for (m, w), t in table.items()},
            "note": "va_bench_hbm_read: contiguous read of config 2's per-launch bytes, "
                    "28 cold launches per graph replay"}


TTS_SHAPES = ((1, 600), (4, 1500), (8, 300))


def bench_tts(args, dev, stream):
    """The TTS talker's decode through the drop-in paged_attention_decode
    (qwen_tts_paged_attention.py:383-516 signature): HND pool with 16-token
    pages, int64 page table and lengths, a key mask over kernel_seq_len tokens
    (left padding: the first 5% of each row masked, then random holes) and the
    current rows written in the same launch; 16 query / 8 kv heads, head_dim
    128, 28 layers with their own pools per graph replay.  Each shape is timed
    with the mask and without it."""
    from voiceagent_amd.agent import paged_attention_decode

    hq, hkv, d, page, layers = workloads.HQ, workloads.HKV, workloads.HEAD_DIM, 16, workloads.LAYERS
    g = torch.Generator(device=dev).manual_seed(11)
    res = {}
    for B, L in TTS_SHAPES:
        need = (L + page - 1) // page
        pages = B * need + 8
        perm = torch.randperm(pages, device=dev, generator=g)
        table = perm[:B * need].view(B, need).to(torch.long)
        lens = torch.full((B,), L, dtype=torch.long, device=dev)
        kernel_seq_len = (L + 127) // 128 * 128
        mask = torch.rand(B, kernel_seq_len, device=dev, generator=g) < 0.9
        mask[:, :L // 20] = False
        kps = [(torch.randn(pages, hkv, page, d, device=dev, generator=g) * 0.5).to(torch.bfloat16)
               for _ in range(layers)]
        vps = [(torch.randn(pages, hkv, page, d, device=dev, generator=g) * 0.5).to(torch.bfloat16)
               for _ in range(layers)]
        q = torch.randn(layers, B, hq, 1, d, device=dev, generator=g).to(torch.bfloat16)
        nk = (torch.randn(layers, B, hkv, 1, d, device=dev, generator=g) * 0.5).to(torch.bfloat16)
        nv = (torch.randn(layers, B, hkv, 1, d, device=dev, generator=g) * 0.5).to(torch.bfloat16)
        # K/V rows read, q read, out written, tables and lengths, mask bytes up to
        # each length, current rows read and written.
        nbytes = (B * L * hkv * d * 2 * 2 + 2 * B * hq * d * 2 + B * need * 8 + B * 8 +
                  B * L + 2 * 2 * B * hkv * d * 2)
        row = {}
        for use_mask in (True, False):
            def step(use_mask=use_mask):
                for i in range(layers):
                    paged_attention_decode(q[i], kps[i], vps[i], table, lens,
                                           mask if use_mask else None, new_key=nk[i],
                                           new_value=nv[i], kernel_seq_len=kernel_seq_len,
                                           kernel_page_count=need, validate=False)

            ms, _ = timed_graph(step, args.steps, args.warmup, stream)
            row["mask" if use_mask else "no_mask"] = ms * 1000.0 / layers
        us = row["mask"]
        gbs = nbytes / (us * 1e-6) / 1e9
        log(f"[tts] B={B} L={L}: {us:.2f} us/layer with the key mask ({gbs:.0f} GB/s, "
            f"{nbytes / 1e6:.2f} MB/layer), {row['no_mask']:.2f} without")
        res[f"B{B}_L{L}"] = {"us_per_layer": round(us, 2), "gbs": round(gbs, 1),
                             "frac": round(gbs / HBM_PEAK_GBS, 4), "bytes_per_layer": nbytes,
                             "us_per_layer_no_mask": round(row["no_mask"], 2)}
    return res


def bench_kv_format(args, dev, stream, dec):
    """Config 2 decode with the pools in the head-major layout [num_blocks, Hkv,
    block_size, D] (one (block, kv head) is a contiguous 4 KiB run) instead of
    the engine's [num_blocks, block_size, Hkv, D]; same values, same step."""
    batch, layers = dec["batch"], workloads.LAYERS
    kps = [k.permute(0, 2, 1, 3).contiguous() for k in batch.k_pools]
    vps = [v.permute(0, 2, 1, 3).contiguous() for v in batch.v_pools]
    outs = torch.empty_like(dec["qs"])

    def step():
        for i in range(layers):
            ops.paged_decode(dec["qs"][i], kps[i], vps[i], batch.block_tables,
                             batch.cu_seqlens_k, lens_cumulative=True,
                             max_seq_len=batch.max_seq_len, scale=batch.scale,
                             layout=ops.LAYOUT_HND, new_k=dec["nks"][i], new_v=dec["nvs"][i],
                             new_slots=batch.slot_mapping, out=outs[i], split_tokens=args.split)

    ms, _ = timed_graph(step, args.steps, args.warmup, stream)
    del kps, vps
    us = ms * 1000.0 / layers
    gbs = dec["bytes_layer"] / (us * 1e-6) / 1e9
    log(f"[kv format] head-major pool: {us:.2f} us/layer, {gbs:.0f} GB/s "
        f"(engine layout {dec['us_layer']:.2f} us/layer)")
    return {"us_per_layer": round(us, 2), "gbs": round(gbs, 1),
            "frac": round(gbs / HBM_PEAK_GBS, 4),
            "layout": "[num_blocks, Hkv, block_size, D]",
            "engine_layout_us_per_layer": round(dec["us_layer"], 2)}


def bench_prologue(args, dev, stream, dec):
    """Config 2's decode step with Qwen3's q/k RMSNorm + RoPE in front
    (models/qwen3.py:44-49): fused into the decode launch vs the standalone
    prologue kernel followed by the decode launch."""
    from voiceagent_amd.layers.qwen3 import rotary_cos_sin_cache

    batch, qs, nks, nvs = dec["batch"], dec["qs"], dec["nks"], dec["nvs"]
    layers = workloads.LAYERS
    g = torch.Generator(device=dev).manual_seed(17)
    wq = (torch.rand(layers, workloads.HEAD_DIM, generator=g, device=dev) + 0.5).to(torch.bfloat16)
    wk = (torch.rand(layers, workloads.HEAD_DIM, generator=g, device=dev) + 0.5).to(torch.bfloat16)
    cs = rotary_cos_sin_cache(workloads.HEAD_DIM, 4096, 1_000_000.0).to(dev)
    pos = (batch.context_lens.long() - 1).to(dev)
    pros = [ops.QKPrologue(wq[i], wk[i], 1e-6, cs, pos) for i in range(layers)]
    outs = torch.empty_like(qs)
    common = dict(lens_cumulative=True, max_seq_len=batch.max_seq_len, scale=batch.scale,
                  new_slots=batch.slot_mapping)

    def fused():
        for i in range(layers):
            ops.paged_decode(qs[i], batch.k_pools[i], batch.v_pools[i], batch.block_tables,
                             batch.cu_seqlens_k, new_k=nks[i], new_v=nvs[i], out=outs[i],
                             prologue=pros[i], **common)

    qn = torch.empty_like(qs[0])
    kn = torch.empty_like(nks[0])

    def two_launch():
        for i in range(layers):
            ops.qk_norm_rope(qs[i], nks[i], pros[i], q_out=qn, k_out=kn)
            ops.paged_decode(qn, batch.k_pools[i], batch.v_pools[i], batch.block_tables,
                             batch.cu_seqlens_k, new_k=kn, new_v=nvs[i], out=outs[i], **common)

    # A prefill-sized batch (config 3's prompts, one position per token): the
    # standalone kernel, which runs in front of every prefill.
    lens = workloads.cfg3_lens(0)
    total = sum(lens)
    hq, hkv, d = workloads.HQ, workloads.HKV, workloads.HEAD_DIM
    qp = torch.randn(layers, total, hq, d, generator=g, device=dev).to(torch.bfloat16)
    kp = torch.randn(layers, total, hkv, d, generator=g, device=dev).to(torch.bfloat16)
    qpo, kpo = torch.empty_like(qp), torch.empty_like(kp)
    ppos = torch.cat([torch.arange(n) for n in lens]).to(dev)
    ppros = [ops.QKPrologue(wq[i], wk[i], 1e-6, cs, ppos) for i in range(layers)]

    def prefill_prologue():
        for i in range(layers):
            ops.qk_norm_rope(qp[i], kp[i], ppros[i], q_out=qpo[i], k_out=kpo[i])

    # Config 3's prefill (fused store into a block-16 pool) with the prologue:
    # the keys through the standalone kernel and the queries normalised and
    # rotated inside the varlen launch, against the standalone kernel over q
    # and k followed by the varlen launch.
    vp_ = torch.randn(layers, total, hkv, d, generator=g, device=dev).to(torch.bfloat16)
    cu = torch.zeros(len(lens) + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(lens, dtype=torch.int32), 0)
    cu = cu.to(dev)
    bs = workloads.BLOCK
    nb = sum(math.ceil(n / bs) for n in lens) + 8
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(12)).tolist()
    rows, cur, slots = [], 0, []
    for n in lens:
        m = math.ceil(n / bs)
        rows.append(perm[cur:cur + m] + [-1] * (max(math.ceil(x / bs) for x in lens) - m))
        slots += [perm[cur + t // bs] * bs + t % bs for t in range(n)]
        cur += m
    table = torch.tensor(rows, dtype=torch.int32, device=dev)
    slots = torch.tensor(slots, dtype=torch.int32, device=dev)
    kpool = torch.zeros(layers, nb, bs, hkv, d, dtype=torch.bfloat16, device=dev)
    vpool = torch.zeros_like(kpool)
    pout = torch.empty_like(qp)

    def prefill_call(i, q, k, prologue=None):
        ops.varlen_attention(q, k, vp_[i], cu, cu, max(lens), max(lens), scale=d ** -0.5,
                             causal=True, k_cache=kpool[i], v_cache=vpool[i], block_tables=table,
                             slot_mapping=slots, out=pout[i], prologue=prologue)

    def prefill_two_launch():
        for i in range(layers):
            ops.qk_norm_rope(qp[i], kp[i], ppros[i], q_out=qpo[i], k_out=kpo[i])
            prefill_call(i, qpo[i], kpo[i])

    def prefill_fused():
        for i in range(layers):
            ops.qk_norm_rope(None, kp[i], ppros[i], k_out=kpo[i])
            prefill_call(i, qp[i], kpo[i], ppros[i])

    res = {}
    for name, fn in (("fused", fused), ("two_launch", two_launch), ("prefill", prefill_prologue),
                     ("prefill_two_launch", prefill_two_launch),
                     ("prefill_fused", prefill_fused)):
        ms, _ = timed_graph(fn, args.steps, args.warmup, stream, name=f"prologue_{name}")
        res[name] = ms * 1000.0 / layers
    # q and k rows read and written, the positions and each token's cos | sin row.
    pbytes = total * (hq + hkv) * d * 2 * 2 + total * (8 + d * 4)
    pgbs = pbytes / (res["prefill"] * 1e-6) / 1e9
    log(f"[prologue] decode + q/k norm + rope: fused {res['fused']:.2f} us/layer, "
        f"two launches {res['two_launch']:.2f} us/layer; standalone over config 3's "
        f"{total} prompt tokens {res['prefill']:.2f} us/layer ({pgbs:.0f} GB/s of "
        f"{pbytes / 1e6:.1f} MB)")
    log(f"[prologue] config 3 prefill with the prologue: fused (keys alone, queries in the "
        f"varlen launch) {res['prefill_fused']:.2f} us/layer, two launches "
        f"{res['prefill_two_launch']:.2f} us/layer")
    del qp, kp, qpo, kpo, vp_, kpool, vpool, pout
    return {"fused_us_per_layer": round(res["fused"], 2),
            "two_launch_us_per_layer": round(res["two_launch"], 2),
            "prefill_cfg3_us_per_layer": round(res["prefill"], 2),
            "prefill_cfg3_gbs": round(pgbs, 1), "prefill_cfg3_bytes": pbytes,
            "prefill_cfg3_with_prologue_fused_us_per_layer": round(res["prefill_fused"], 2),
            "prefill_cfg3_with_prologue_two_launch_us_per_layer":
                round(res["prefill_two_launch"], 2),
            "config": "cfg2 decode step (B=32, 28 layers) with Qwen3 q/k RMSNorm + RoPE "
                      "applied to the raw projections; the standalone kernel alone over "
                      "config 3's prompts; config 3's prefill (fused store) with the "
                      "prologue: keys through the standalone kernel and queries in the "
                      "varlen launch, or both through the standalone kernel first"}


MAX_MODEL_LEN = 65536  # max_position_embeddings of the decoder (qwen_asr_vllm/config.py:71)


def bench_longform(args, dev, stream):
    """Config 5: long-form decode, (i) one 16384-token context, (ii) 8 contexts
    U[4096, 16384]; 28 layers with their own pools, fused store, contexts split
    into partitions and merged.  The exact-maximum rows split as an eager
    engine step does (PagedAttention passes SPLIT_EXACT: its max_seqlen_k is
    the batch's longest context, model_runner.py:213).  Each variant also runs
    with max_seq_len = max_model_len and the automatic split, as the engine's
    decode graph passes it (qwen_asr_vllm/engine/graph_runner.py:85-93)."""
    res = {}
    layers = workloads.LAYERS
    for variant in ("single", "batch8"):
        lens = workloads.cfg5_lens(variant, 0)
        nb = sum(math.ceil(n / workloads.BLOCK) for n in lens) + 64
        batch = workloads.make_decode_batch(lens, num_blocks=nb, num_layers=layers,
                                            dtype=torch.bfloat16, kv_std=0.5, device=dev,
                                            seed=5, device_rng=True)
        g = torch.Generator(device=dev).manual_seed(9)
        B = batch.num_seqs
        qs = torch.randn(layers, B, workloads.HQ, workloads.HEAD_DIM, generator=g, device=dev
                         ).to(torch.bfloat16)
        nks = (torch.randn(layers, B, workloads.HKV, workloads.HEAD_DIM, generator=g,
                           device=dev) * 0.5).to(torch.bfloat16)
        nvs = (torch.randn(layers, B, workloads.HKV, workloads.HEAD_DIM, generator=g,
                           device=dev) * 0.5).to(torch.bfloat16)
        outs = torch.empty_like(qs)

        exact_split = args.split if args.split else ops.SPLIT_EXACT

        def make_step(max_seq_len, kps, vps, kv_scale=1.0, split=exact_split):
            def step():
                for i in range(layers):
                    ops.paged_decode(qs[i], kps[i], vps[i],
                                     batch.block_tables, batch.cu_seqlens_k,
                                     lens_cumulative=True, max_seq_len=max_seq_len,
                                     scale=batch.scale, new_k=nks[i], new_v=nvs[i],
                                     new_slots=batch.slot_mapping, out=outs[i],
                                     split_tokens=split, k_scale=kv_scale,
                                     v_scale=kv_scale)
            return step

        nbytes = decode_launch_bytes(lens)
        ms, _ = timed_graph(make_step(batch.max_seq_len, batch.k_pools, batch.v_pools),
                            args.steps, args.warmup, stream, name=f"longform_{variant}")
        us = ms * 1000.0 / layers
        gbs = nbytes / (us * 1e-6) / 1e9
        ms_g, _ = timed_graph(make_step(MAX_MODEL_LEN, batch.k_pools, batch.v_pools,
                                        split=args.split),
                              args.steps, args.warmup, stream)
        us_g = ms_g * 1000.0 / layers
        log(f"[longform {variant}] B={B} ctx sum {sum(lens)}: {us:.2f} us/layer, {gbs:.0f} GB/s "
            f"({nbytes / 1e6:.1f} MB/layer, {gbs / HBM_PEAK_GBS:.3f} of HBM peak); "
            f"max_seq_len={MAX_MODEL_LEN}: {us_g:.2f} us/layer")
        # The same step over FP8 copies of the pools.
        kf, vf = fp8_pools(batch.k_pools, batch.v_pools)
        del batch.k_pools[:], batch.v_pools[:]
        torch.cuda.empty_cache()
        ms8, _ = timed_graph(make_step(batch.max_seq_len, kf, vf, FP8_SCALE), args.steps,
                             args.warmup, stream, name=f"longform_{variant}_fp8")
        us8 = ms8 * 1000.0 / layers
        nbytes8 = decode_launch_bytes(lens, kv_elem=1)
        gbs8 = nbytes8 / (us8 * 1e-6) / 1e9
        log(f"[longform {variant} fp8] {us8:.2f} us/layer, {gbs8:.0f} GB/s of "
            f"{nbytes8 / 1e6:.1f} MB/layer ({gbs8 / HBM_PEAK_GBS:.3f} of HBM peak)")
        res[variant] = {"us_per_layer": round(us, 2), "gbs": round(gbs, 1),
                        "frac": round(gbs / HBM_PEAK_GBS, 4), "bytes_per_layer": nbytes,
                        "batch": B, "context_tokens": sum(lens),
                        "us_per_layer_max_model_len": round(us_g, 2),
                        "split": ("exact-bound (SPLIT_EXACT, as an eager step)" if not args.split
                                  else f"split_tokens {args.split}"),
                        "split_max_model_len": ("automatic (as a captured decode graph)"
                                                if not args.split
                                                else f"split_tokens {args.split}"),
                        "fp8": {"us_per_layer": round(us8, 2), "gbs": round(gbs8, 1),
                                "frac": round(gbs8 / HBM_PEAK_GBS, 4),
                                "bytes_per_layer": nbytes8}}
        del batch, qs, nks, nvs, outs, kf, vf
        torch.cuda.empty_cache()
    return res


def bench_store(args, dev, stream, dec):
    """store_kvcache alone: 32 rows per layer over the 28 pools (latency-bound)."""
    batch = dec["batch"]
    B = batch.num_seqs

    def step():
        for i in range(workloads.LAYERS):
            ops.store_kvcache(batch.new_k, batch.new_v, batch.k_pools[i], batch.v_pools[i],
                              batch.slot_mapping)

    ms, _ = timed_graph(step, args.steps, args.warmup, stream)
    us = ms * 1000.0 / workloads.LAYERS
    nbytes = workloads.store_bytes(B)
    log(f"[store] {us:.2f} us/layer ({nbytes} B, latency-bound)")
    res = dict(us_layer=us, gbs=nbytes / (us * 1e-6) / 1e9)

    # A prefill-sized store, as an unfused caller runs it: config 3's 8561 new K
    # and V rows per layer scattered into a block-16 pool, 28 layers each with
    # its own rows and pool (cold), slots in a shuffled block order.
    lens = workloads.cfg3_lens(0)
    total, layers, bs = sum(lens), workloads.LAYERS, workloads.BLOCK
    g = torch.Generator(device=dev).manual_seed(21)
    kr = torch.randn(layers, total, workloads.HKV, workloads.HEAD_DIM, generator=g,
                     device=dev).to(torch.bfloat16)
    vr = torch.randn_like(kr)
    nb = sum(math.ceil(n / bs) for n in lens) + 8
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(22)).tolist()
    slots, cur = [], 0
    for n in lens:
        slots += [perm[cur + p // bs] * bs + p % bs for p in range(n)]
        cur += math.ceil(n / bs)
    slots = torch.tensor(slots, dtype=torch.int32, device=dev)
    kp = torch.zeros(layers, nb, bs, workloads.HKV, workloads.HEAD_DIM, dtype=torch.bfloat16,
                     device=dev)
    vp = torch.zeros_like(kp)

    def step_prefill():
        for i in range(layers):
            ops.store_kvcache(kr[i], vr[i], kp[i], vp[i], slots)

    ms, _ = timed_graph(step_prefill, args.steps, args.warmup, stream, name="store_cfg3")
    us3 = ms * 1000.0 / layers
    nbytes3 = workloads.store_bytes(total)
    gbs3 = nbytes3 / (us3 * 1e-6) / 1e9
    log(f"[store cfg3] {total} rows: {us3:.2f} us/layer, {gbs3:.0f} GB/s of {nbytes3 / 1e6:.1f} MB "
        f"({gbs3 / 8000:.3f} of HBM peak)")
    res["cfg3_rows"] = dict(us_layer=round(us3, 2), gbs=round(gbs3, 1), bytes=nbytes3,
                            frac=round(gbs3 / 8000, 4))
    del kr, vr, kp, vp
    return res


def bench_prefill(args, dev, stream):
    lens = workloads.cfg3_lens(0)
    layers = 28
    total = sum(lens)
    log(f"[prefill] 32 prompts, {total} tokens, 28 rotating input sets, fused store")
    g = torch.Generator(device=dev).manual_seed(11)
    q = torch.randn(layers, total, 16, 128, generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn(layers, total, 8, 128, generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn(layers, total, 8, 128, generator=g, device=dev).to(torch.bfloat16)
    out = torch.empty_like(q)
    cu = torch.zeros(len(lens) + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(lens, dtype=torch.int32), 0)
    cu = cu.to(dev)
    bs = 16
    width = max(math.ceil(n / bs) for n in lens)
    nb = sum(math.ceil(n / bs) for n in lens) + 8
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(12)).tolist()
    rows, cur, slots = [], 0, []
    for n in lens:
        m = math.ceil(n / bs)
        rows.append(perm[cur:cur + m] + [-1] * (width - m))
        slots += [perm[cur + p // bs] * bs + p % bs for p in range(n)]
        cur += m
    table = torch.tensor(rows, dtype=torch.int32, device=dev)
    slots = torch.tensor(slots, dtype=torch.int32, device=dev)
    kp = torch.zeros(layers, nb, bs, 8, 128, dtype=torch.bfloat16, device=dev)
    vp = torch.zeros_like(kp)
    scale = 128 ** -0.5

    def step():
        for i in range(layers):
            ops.varlen_attention(q[i], k[i], v[i], cu, cu, max(lens), max(lens), scale=scale,
                                 causal=True, k_cache=kp[i], v_cache=vp[i], block_tables=table,
                                 slot_mapping=slots, out=out[i])

    ms, _ = timed_graph(step, args.steps, args.warmup, stream, name="prefill_cfg3")
    us = ms * 1000.0 / layers
    flops = workloads.causal_flops(lens)
    tflops = flops / (us * 1e-6) / 1e12
    nbytes = workloads.varlen_bytes(lens, 16, 8, 128) + total * 2 * 8 * 128 * 2
    log(f"[prefill] {us:.2f} us/layer, {tflops:.1f} TFLOP/s ({flops / 1e9:.2f} GFLOP), "
        f"{nbytes / (us * 1e-6) / 1e9:.0f} GB/s")

    # Warm: the same 28 launches, every one on input set 0 (q, k, v and the
    # pool MALL-resident, as the QKV projection leaves them in the engine).
    def step_warm():
        for _ in range(layers):
            ops.varlen_attention(q[0], k[0], v[0], cu, cu, max(lens), max(lens), scale=scale,
                                 causal=True, k_cache=kp[0], v_cache=vp[0], block_tables=table,
                                 slot_mapping=slots, out=out[0])

    ms_w, _ = timed_graph(step_warm, args.steps, args.warmup, stream, name="prefill_cfg3_warm")
    us_w = ms_w * 1000.0 / layers
    tflops_w = flops / (us_w * 1e-6) / 1e12
    log(f"[prefill warm] {us_w:.2f} us/layer, {tflops_w:.1f} TFLOP/s "
        f"({tflops_w / BF16_PEAK_TFLOPS:.3f} of the bf16 MFMA peak)")
    def call0():
        ops.varlen_attention(q[0], k[0], v[0], cu, cu, max(lens), max(lens), scale=scale,
                             causal=True, k_cache=kp[0], v_cache=vp[0], block_tables=table,
                             slot_mapping=slots, out=out[0])

    return dict(us_layer=us, tflops=tflops, flops=flops, bytes=nbytes, us_layer_warm=us_w,
                tflops_warm=tflops_w, inputs=(q[0], k[0], v[0], cu, scale, True), call0=call0)


def bench_encoder(args, dev, stream):
    wins = workloads.cfg4_windows(0)
    layers = 18
    total = sum(wins)
    g = torch.Generator(device=dev).manual_seed(13)
    q = torch.randn(layers, total, 14, 64, generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn(layers, total, 14, 64, generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn(layers, total, 14, 64, generator=g, device=dev).to(torch.bfloat16)
    out = torch.empty_like(q)
    cu = torch.zeros(len(wins) + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(wins, dtype=torch.int32), 0)
    cu = cu.to(dev)

    def step():
        for i in range(layers):
            ops.varlen_attention(q[i], k[i], v[i], cu, cu, max(wins), max(wins), scale=0.125,
                                 causal=False, out=out[i])

    ms, _ = timed_graph(step, args.steps, args.warmup, stream, name="encoder_cfg4")
    us = ms * 1000.0 / layers
    flops = workloads.bidir_flops(wins)
    nbytes = workloads.varlen_bytes(wins, 14, 14, 64)
    log(f"[encoder] {len(wins)} windows, {total} tokens: {us:.2f} us/layer, "
        f"{flops / (us * 1e-6) / 1e12:.1f} TFLOP/s, {nbytes / (us * 1e-6) / 1e9:.0f} GB/s")

    # Warm: every one of the 18 launches on layer 0's q, k, v (MALL-resident).
    def step_warm():
        for _ in range(layers):
            ops.varlen_attention(q[0], k[0], v[0], cu, cu, max(wins), max(wins), scale=0.125,
                                 causal=False, out=out[0])

    ms_w, _ = timed_graph(step_warm, args.steps, args.warmup, stream, name="encoder_cfg4_warm")
    us_w = ms_w * 1000.0 / layers
    log(f"[encoder warm] {us_w:.2f} us/layer, {flops / (us_w * 1e-6) / 1e12:.1f} TFLOP/s")
    return dict(us_layer=us, tflops=flops / (us * 1e-6) / 1e12,
                gbs=nbytes / (us * 1e-6) / 1e9, windows=len(wins), tokens=total, flops=flops,
                us_layer_warm=us_w, tflops_warm=flops / (us_w * 1e-6) / 1e12,
                inputs=(q[0], k[0], v[0], cu, 0.125, False))


def cpu_varlen_baseline(inputs, budget_s: float, label: str):
    """The oracle's per-sequence fp32 attention (bf16 inputs upcast) for one
    layer of config 3 or 4 on the host's cores; median seconds per layer."""
    from oracle import attention as oracle

    torch.set_num_threads(os.cpu_count() or 1)
    q, k, v, cu, scale, causal = inputs
    q, k, v, cu = q.cpu(), k.cpu(), v.cpu(), cu.cpu()
    oracle.varlen_attention(q, k, v, cu, cu, scale, causal)  # warm-up
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < 3 or time.perf_counter() < t_end:
        t0 = time.perf_counter()
        oracle.varlen_attention(q, k, v, cu, cu, scale, causal)
        times.append(time.perf_counter() - t0)
        if len(times) >= 500:
            break
    times.sort()
    med = times[len(times) // 2]
    log(f"[cpu {label}] {med * 1e6:.0f} us/layer median of {len(times)} reps")
    return med, len(times)


def cpu_baseline(dec, budget_s: float):
    """The oracle's per-sequence fp32 fallback on the host, one cfg-2 layer per rep."""
    from oracle import attention as oracle

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    batch = dec["batch"]
    q = dec["qs"][0].cpu()
    kp, vp = batch.k_pools[0].cpu(), batch.v_pools[0].cpu()
    table, lens = batch.block_tables.cpu(), batch.context_lens.cpu()
    oracle.paged_decode(q, kp, vp, table, lens, batch.scale)  # warm-up
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < 5 or time.perf_counter() < t_end:
        t0 = time.perf_counter()
        oracle.paged_decode(q, kp, vp, table, lens, batch.scale)
        times.append(time.perf_counter() - t0)
        if len(times) >= 2000:
            break
    times.sort()
    med = times[len(times) // 2]
    gbs = dec["bytes_layer"] / med / 1e9
    cpu_model = platform.processor() or ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu_model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    log(f"[cpu] {med * 1e6:.0f} us/layer median of {len(times)} reps on {threads} threads "
        f"({cpu_model})")
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"config 2, one layer (B=32 decode, bf16 pool upcast to fp32) through the "
                      f"per-sequence matmul/softmax fallback, {len(times)} reps, median "
                      f"{med * 1e6:.0f} us/layer; host CPU: {cpu_model}",
            "us_per_layer": round(med * 1e6, 1)}


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--split", type=int, default=0, help="decode split_tokens (0 = auto)")
    ap.add_argument("--only", choices=["decode", "batches", "prefill", "encoder", "store",
                                       "longform", "prologue", "kvformat", "floor", "tts", "fp8",
                                       "all"],
                    default="all")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="run a 256 MiB device copy first (counter scale for profiles)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only; --gpus {args.gpus} is not supported "
              "(this build has no multi-GPU path).", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.Stream(dev)
    torch.manual_seed(0)

    if args.calibrate_copy:
        copy_calibration(dev)
    result = {}
    if args.only in ("prefill",):
        result["prefill"] = bench_prefill(args, dev, stream)
        print(json.dumps({"prefill": {k: v for k, v in result["prefill"].items()
                                      if k not in ("inputs", "call0")}}))
        return
    if args.only in ("encoder",):
        enc = bench_encoder(args, dev, stream)
        print(json.dumps({"encoder": {k: v for k, v in enc.items() if k != "inputs"}}))
        return
    if args.only == "longform":
        print(json.dumps({"longform": bench_longform(args, dev, stream)}))
        return
    if args.only == "batches":
        print(json.dumps({"decode_batches": bench_decode_batches(args, dev, stream)}))
        return
    if args.only == "floor":
        print(json.dumps({"hbm_read_floor": bench_floor(args, dev, stream)}))
        return
    if args.only == "tts":
        print(json.dumps({"tts_decode": bench_tts(args, dev, stream)}))
        return
    # rocm-smi runs only in the default run: under a profiler its child
    # process would start with the profiler's library loaded.
    full = args.only == "all"
    state_before = gpu_state() if full else {}
    dec = bench_decode(args, dev, stream)
    state_after = gpu_state() if full else {}
    if args.only == "fp8":
        print(json.dumps({"fp8_decode": bench_decode_fp8(args, dev, stream, dec)}))
        return
    if args.only == "store":
        print(json.dumps({"store": bench_store(args, dev, stream, dec)}))
        return
    if args.only == "prologue":
        print(json.dumps({"qwen3_prologue": bench_prologue(args, dev, stream, dec)}))
        return
    if args.only == "kvformat":
        print(json.dumps({"kv_format_hnd": bench_kv_format(args, dev, stream, dec)}))
        return
    extra = {}
    if args.only == "all":
        extra["decode_warm"] = bench_decode_warm(args, dev, stream, dec)
        extra["decode_batches"] = bench_decode_batches(args, dev, stream)
        extra["fp8_decode"] = bench_decode_fp8(args, dev, stream, dec)
        extra["store"] = bench_store(args, dev, stream, dec)
        extra["qwen3_prologue"] = bench_prologue(args, dev, stream, dec)
        extra["kv_format_hnd"] = bench_kv_format(args, dev, stream, dec)
        extra["hbm_read_floor"] = bench_floor(args, dev, stream)
        extra["tts_decode"] = bench_tts(args, dev, stream)
        pre = bench_prefill(args, dev, stream)
        enc = bench_encoder(args, dev, stream)
        extra["prefill"] = {"us_per_layer": round(pre["us_layer"], 2),
                            "tflops": round(pre["tflops"], 2),
                            "mfma_frac": round(pre["tflops"] / BF16_PEAK_TFLOPS, 4),
                            "hbm_gbs": round(pre["bytes"] / (pre["us_layer"] * 1e-6) / 1e9, 1),
                            "config": "cfg3: 32 prompts U[50,450], GQA 16/8, D128, fused store, "
                                      "28 rotating input sets (cold)",
                            "warm": {"us_per_layer": round(pre["us_layer_warm"], 2),
                                     "tflops": round(pre["tflops_warm"], 2),
                                     "mfma_frac": round(pre["tflops_warm"] / BF16_PEAK_TFLOPS, 4),
                                     "config": "the same 28 launches on input set 0 "
                                               "(MALL-resident inputs, warm)"}}
        extra["host_us_per_call"] = bench_host_overhead(dev, dec, pre)
        extra["longform"] = bench_longform(args, dev, stream)
        extra["encoder"] = {"us_per_layer": round(enc["us_layer"], 2),
                            "tflops": round(enc["tflops"], 2),
                            "hbm_gbs": round(enc["gbs"], 1),
                            "config": f"cfg4: {enc['windows']} windows / {enc['tokens']} tokens, "
                                      "14 heads x 64, 18 rotating layers (cold)",
                            "warm": {"us_per_layer": round(enc["us_layer_warm"], 2),
                                     "tflops": round(enc["tflops_warm"], 2),
                                     "mfma_frac": round(enc["tflops_warm"] / BF16_PEAK_TFLOPS, 4),
                                     "config": "the same 18 launches on layer 0's inputs "
                                               "(MALL-resident, warm)"}}
    cpu = None
    if not args.no_cpu and args.only == "all":
        cpu = cpu_baseline(dec, args.cpu_seconds)
        threads = os.cpu_count() or 1
        for key, res, label in (("prefill", pre, "cfg3"), ("encoder", enc, "cfg4")):
            med, reps = cpu_varlen_baseline(res["inputs"], args.cpu_seconds / 2, label)
            extra[key]["cpu_baseline"] = {
                "us_per_layer": round(med * 1e6, 1), "tflops": round(res["flops"] / med / 1e12, 4),
                "cores": threads, "kind": "port",
                "sample": f"one layer of {label} through the oracle's per-sequence fp32 "
                          f"masked softmax (bf16 inputs upcast), {reps} reps, median"}
    line = {
        "metric": METRIC,
        "value": round(dec["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dec["ms"], 4),
        "timing": "median of the per-replay HIP-event times of the timed replays "
                  "(TIMINGS below holds mean and minimum too)",
        "us_per_layer": round(dec["us_layer"], 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (K/V N(0,1)*0.5 bf16, q N(0,1), seed 0)",
        "config": {"workload": "cfg2: Qwen3-0.6B paged decode step, 28 layers, B=32, "
                               "GQA 16q/8kv, head_dim 128, block 16, ctx U[60,600], "
                               "4096-block pool per layer, store of 32 rows/layer fused",
                   "batch": 32, "layers": 28, "context_tokens": sum(dec["lens"]),
                   "parallelism": "single GPU, HIP graph replay"},
        "roofline": {"bound": "hbm", "achieved": round(dec["gbs"], 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(dec["gbs"] / HBM_PEAK_GBS, 4),
                     "traffic": profiled_traffic(),
                     "kernel": decode_kernel_name(),
                     "bytes_per_launch": dec["bytes_layer"]},
        "cpu_baseline": cpu,
    }
    line.update(extra)
    line["timings"] = TIMINGS
    line["gpu_state"] = {"before": state_before, "after": state_after}
    if line["roofline"]["frac"] > 1.0:
        log("[bench] WARNING: achieved bandwidth above the HBM peak: measurement error")
    print(json.dumps(line))


if __name__ == "__main__":
    main()
