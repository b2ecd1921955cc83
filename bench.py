"""Benchmark of the packed rotated KV-cache decode hot path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--workload M] [--no-cpu-baseline]

A step is one decode of one query token per query head over the whole packed
cache: query rotation, split-K packed attention with online softmax,
cross-workgroup log-sum-exp merge and inverse rotation -- one tq_decode call
(the split kernel, then the merge kernel).  Inputs (packed K/V slabs) are resident in HBM before timing; the
timed loop cycles through enough slab replicas (> 512 MiB together) that the
256 MB Infinity Cache cannot hold the working set.

Prints one JSON line: value = packed KV GB/s over the timed loop (wall clock,
bracketed by device synchronisation); roofline = algorithmic bytes per launch
over the kernel's own duration (HIP events bound to the kernel); the
fp16-dense decode kernel of the same shape is timed the same way; the CPU
oracle is timed on a bounded sample on the host cores.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time
from math import ceil
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "torque-mlx_amd"))
sys.path.insert(0, str(REPO))

METRIC = "packed decode-attn µs/step + achieved HBM GB/s (% peak) at 4-bit, 32K ctx"
HBM_PEAK_GBPS = 8000.0
FP32_MATRIX_PEAK_TFLOPS = 157.3  # MI355X dense fp32 matrix peak

WORKLOADS = {
    # name: (layers, kv_heads, query_heads, head_dim, bits, seq_len, std, description)
    "M": (1, 8, 32, 128, 4, 32768, 1.0, "M: head_dim 128, 4-bit, seq_len 32768, 8 KV heads, 32 query heads (GQA 4)"),
    "C3": (1, 8, 32, 128, 2, 32768, 1.0, "C3: head_dim 128, 2-bit, seq_len 32768, 8 KV heads, 32 query heads"),
    "C4": (1, 2, 8, 256, 4, 131072, 0.5, "C4: head_dim 256, 4-bit, seq_len 131072, 2 KV heads, 8 query heads"),
    "C1": (1, 8, 8, 128, 4, 512, 1.0, "C1: head_dim 128, 4-bit, seq_len 512, 8 KV heads, 8 query heads"),
    "C5L": (1, 4, 16, 256, 4, 8192, 1.0, "C5 one layer: head_dim 256, 4-bit, seq_len 8192, 4 KV heads, 16 query heads"),
}

# Decode loops: prefill seq_len tokens, then `steps` steps of (append one token + decode) in every layer.
LOOP_WORKLOADS = {
    # name: (layers, kv_heads, query_heads, head_dim, bits, prefill, steps, std, description)
    "C2": (1, 4, 16, 64, 3, 4096, 64, 1.0, "C2: head_dim 64, 3-bit, 4 KV / 16 query heads, prefill 4096, 64 steps"),
    "C5": (24, 4, 16, 256, 4, 8192, 128, 1.0,
           "C5: 24 layers, head_dim 256, 4-bit, 4 KV / 16 query heads, prefill 8192, 128 steps"),
}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class Hip:
    """hipEvent helpers through the HIP runtime torch already loaded."""

    def __init__(self) -> None:
        self.lib = ctypes.CDLL("libamdhip64.so.7")
        self.lib.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.lib.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.lib.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        self.lib.hipEventDestroy.argtypes = [ctypes.c_void_p]
        self.lib.hipStreamCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.lib.hipStreamDestroy.argtypes = [ctypes.c_void_p]
        self.lib.hipStreamSynchronize.argtypes = [ctypes.c_void_p]
        self.lib.hipStreamBeginCapture.argtypes = [ctypes.c_void_p, ctypes.c_int]
        self.lib.hipStreamEndCapture.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)]
        self.lib.hipGraphInstantiate.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_void_p, ctypes.c_void_p,
                                                 ctypes.c_void_p, ctypes.c_size_t]
        self.lib.hipGraphLaunch.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self.lib.hipGraphDestroy.argtypes = [ctypes.c_void_p]
        self.lib.hipGraphExecDestroy.argtypes = [ctypes.c_void_p]

    def event(self) -> ctypes.c_void_p:
        ev = ctypes.c_void_p()
        rc = self.lib.hipEventCreate(ctypes.byref(ev))
        if rc != 0:
            raise RuntimeError(f"hipEventCreate failed: {rc}")
        return ev

    def elapsed_ms(self, a, b) -> float:
        self.lib.hipEventSynchronize(b)
        ms = ctypes.c_float()
        rc = self.lib.hipEventElapsedTime(ctypes.byref(ms), a, b)
        if rc != 0:
            raise RuntimeError(f"hipEventElapsedTime failed: {rc}")
        return float(ms.value)


def _hip_ok(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what} failed with HIP error {rc}")


def synthetic(seed, layers, kv_heads, query_heads, seq_len, head_dim, std):
    """Seeded fp16 N(0, std) Q/K/V; K scaled by one log-normal(0, 1) factor per (layer, KV head, channel)."""
    rng = np.random.default_rng(seed)
    q = rng.normal(0.0, std, size=(layers, query_heads, head_dim)).astype(np.float32)
    k = rng.normal(0.0, std, size=(layers, kv_heads, seq_len, head_dim)).astype(np.float32)
    v = rng.normal(0.0, std, size=(layers, kv_heads, seq_len, head_dim)).astype(np.float32)
    k *= rng.lognormal(0.0, 1.0, size=(layers, kv_heads, 1, head_dim)).astype(np.float32)
    return q.astype(np.float16), k.astype(np.float16), v.astype(np.float16)


_CPU_JOB: dict = {}


def _cpu_head(qh: int):
    """Worker: the oracle decode of query head qh against its KV head (cache.py:98-140 restated, which
    expands the KV rows per query head), single-threaded."""
    from threadpoolctl import threadpool_limits

    from oracle import torque_oracle as o

    j = _CPU_JOB
    h = qh // j["group"]
    with threadpool_limits(1):
        q_rot = o.rotation_apply(j["q"][:, qh : qh + 1], j["sl"], j["sr"])[0]
        idx = np.array([h])
        out_rot = o.decode_packed_reference(
            q_rot, j["kc"][0][idx], j["vc"][0][idx], j["kcent"], j["vcent"], bit_width=j["bits"],
            head_dim=j["head_dim"], key_scales=None if j["ks"] is None else j["ks"][0][idx],
            value_scales=None if j["vs"] is None else j["vs"][0][idx],
        )
        return qh, o.rotation_inverse(out_rot, j["sl"], j["sr"])[0]


def cpu_pool_size() -> int:
    """Worker processes for the CPU baseline: every core this process may run on, at most 16 (one GPU's
    share of the box's host cores)."""
    return max(1, min(16, len(os.sched_getaffinity(0))))


def cpu_baseline(q, k_codes, v_codes, cache, budget_s: float, gpu_out, k_scales=None, v_scales=None):
    """Time the CPU oracle (vectorised numpy restatement of cache.py:98-140) on all host cores.

    One step decodes every query head at the full sequence length, one query
    head per task on a pool of forked single-threaded workers; steps repeat
    until `budget_s` seconds have elapsed and the median step is reported.
    """
    import multiprocessing as mp
    from concurrent.futures import ProcessPoolExecutor

    cfg = cache.config
    _CPU_JOB.update(
        group=q.shape[1] // cfg.kv_heads, q=q.astype(np.float32), kc=k_codes, vc=v_codes, ks=k_scales, vs=v_scales,
        sl=cache.rotation.signs_left, sr=cache.rotation.signs_right, kcent=cache.key_codebook.centroids,
        vcent=cache.value_codebook.centroids, bits=cfg.bit_width, head_dim=cfg.head_dim,
    )
    workers = cpu_pool_size()
    hq = q.shape[1]
    out = np.zeros((hq, cfg.head_dim), np.float32)
    times = []
    with ProcessPoolExecutor(max_workers=workers, mp_context=mp.get_context("fork")) as pool:
        list(pool.map(_cpu_head, range(min(workers, hq))))  # fork and warm the workers
        t_start = time.perf_counter()
        while time.perf_counter() - t_start < budget_s or len(times) < 1:
            t0 = time.perf_counter()
            for qh, o_h in pool.map(_cpu_head, range(hq)):
                out[qh] = o_h
            times.append(time.perf_counter() - t0)
    _CPU_JOB.clear()
    per_step = float(np.median(times))
    ref = gpu_out[0]
    err = float(np.max(np.abs(ref - out)))
    rel = float(np.linalg.norm(ref - out) / max(np.linalg.norm(out), 1e-30))
    return per_step, len(times), workers, err, rel


def cpu_literal_baseline(q, k_codes, v_codes, cache, budget_s: float):
    """The reference's literal per-element path, timed single-threaded: the per-code unpack loop of
    quantization.py:272-290 for every row, centroid gather, then the online-softmax loop of
    reference.py:8-42 token by token for every query head (the oracle's unpack_indices and
    streaming_attention_decode), with the rotations of cache.py:98-140.  Small workloads only."""
    from oracle import torque_oracle as o

    cfg = cache.config
    g = q.shape[1] // cfg.kv_heads
    sl, sr = cache.rotation.signs_left, cache.rotation.signs_right
    kcent, vcent = cache.key_codebook.centroids, cache.value_codebook.centroids

    def one():
        q_rot = o.rotation_apply(q.astype(np.float32), sl, sr)[0]
        out = np.empty_like(q_rot)
        for h in range(cfg.kv_heads):
            keys = o.dequantize(np.stack([o.unpack_indices(w, cfg.bit_width, cfg.head_dim) for w in k_codes[0, h]]), kcent)
            values = o.dequantize(np.stack([o.unpack_indices(w, cfg.bit_width, cfg.head_dim) for w in v_codes[0, h]]), vcent)
            for j in range(g):
                out[h * g + j] = o.streaming_attention_decode(q_rot[h * g + j], keys, values)
        return o.rotation_inverse(out, sl, sr)

    times = []
    t_start = time.perf_counter()
    while time.perf_counter() - t_start < budget_s or len(times) < 1:
        t0 = time.perf_counter()
        one()
        times.append(time.perf_counter() - t0)
    return float(np.median(times)), len(times)


FP16_MATRIX_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 matrix peak


def compute_roofline(matrix_kernel: bool, L: int, hkv: int, hq: int, d: int, s: int, kern_us: float) -> dict:
    """The split kernel against its arithmetic ceiling.

    Algorithmic work: 4 L Hq S D flops per step (a multiply-add per query head
    and packed code for the score and for the value update).  The float32
    kernel runs it as 4x4x1 fp32 products (fp32 matrix peak); the matrix
    kernel as 16x16x32 f16 products of hi/lo splits (fp16 matrix peak), which
    execute 16 products of 16x16x32 per 16-token tile and group of 4 query
    heads (half of each product's rows or columns carry data).
    """
    algo = 4 * L * hq * s * d
    if matrix_kernel:
        tiles = L * hkv * (hq // hkv // 4) * ((s + 15) // 16)
        executed = tiles * (d // 16) * 2 * 2 * 16 * 16 * 32
        tflops = executed / (kern_us * 1e-6) / 1e12
        return {"bound": "mfma", "achieved": round(tflops, 2), "peak": FP16_MATRIX_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": round(tflops / FP16_MATRIX_PEAK_TFLOPS, 4), "flops_per_launch": executed,
                "algorithmic_flops_per_launch": algo}
    tflops = algo / (kern_us * 1e-6) / 1e12
    return {"bound": "mfma", "achieved": round(tflops, 2), "peak": FP32_MATRIX_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(tflops / FP32_MATRIX_PEAK_TFLOPS, 4), "flops_per_launch": algo}


def measured_traffic(kernel: str, workload: str) -> tuple[int | None, str | None]:
    """HBM bytes per launch of `kernel` on `workload`, from a committed rocprofv3 PMC summary.

    The summaries under profiles/ carry a line
    ``traffic_bytes_per_launch: <kernel> <workload> <bytes>`` (FETCH_SIZE and
    WRITE_SIZE passes, each scaled by the same counter on a copy of known size).
    """
    for path in sorted((REPO / "profiles").glob("*hbm_traffic*.md")):
        for line in path.read_text().splitlines():
            parts = line.split()
            if len(parts) == 4 and parts[0] == "traffic_bytes_per_launch:" and parts[1:3] == [kernel, workload]:
                return int(parts[3]), f"profiles/{path.name}"
    return None, None


def read_ceiling(torch, _lib, hip, dev, step_bytes: int, total_mib: int) -> dict:
    """Streaming-read ceiling of the device (tq_stream_read): one pass over `total_mib`, and reads of
    `step_bytes` (one decode step's packed K+V) cycling through the same buffer."""
    chunk = (step_bytes + 255) // 256 * 256
    n_chunks = max(3, total_mib * 2**20 // chunk)
    buf = torch.empty(n_chunks * chunk, dtype=torch.uint8, device=dev)
    buf.view(torch.int32).random_()
    sink = torch.empty(8 * 1024, dtype=torch.float32, device=dev)
    fn = _lib.load().tq_stream_read
    stream = torch.cuda.current_stream(dev).cuda_stream
    base = buf.data_ptr()
    for i in range(3):
        _lib.check(fn(base, n_chunks * chunk, sink.data_ptr(), 0, stream, None, None))
    ev = [(hip.event(), hip.event()) for _ in range(5)]
    for e0, e1 in ev:
        _lib.check(fn(base, n_chunks * chunk, sink.data_ptr(), 0, stream, e0, e1))
    torch.cuda.synchronize()
    full_us = float(np.median([hip.elapsed_ms(a, b) for a, b in ev]) * 1e3)
    ev = [(hip.event(), hip.event()) for _ in range(100)]
    for i, (e0, e1) in enumerate(ev):
        _lib.check(fn(base + (i % n_chunks) * chunk, step_bytes // 16 * 16, sink.data_ptr(), 0, stream, e0, e1))
    torch.cuda.synchronize()
    step_us = float(np.mean([hip.elapsed_ms(a, b) for a, b in ev]) * 1e3)
    del buf
    return {
        "gbps_full_pass": round(n_chunks * chunk / (full_us * 1e-6) / 1e9, 1),
        "full_pass_bytes": n_chunks * chunk,
        "gbps_step_bytes": round(step_bytes / (step_us * 1e-6) / 1e9, 1),
        "step_bytes": step_bytes,
        "kernel": "stream_read_kernel (nontemporal 16-byte loads, 4 in flight per thread, 512 threads, 1 workgroup per CU)",
    }


def run_loop(args, torch, th, _lib, ops, hip, dev) -> int:
    """Decode loop (C2, C5): one num_layers=1 cache per layer, as the reference's Qwen adapter builds them;
    each step appends one token and decodes in every layer, layer after layer."""
    L, hkv, hq, d, bits, s0, steps, std, desc = LOOP_WORKLOADS[args.workload]
    if args.steps_given:
        steps = args.steps
    log(f"workload {desc} ({steps} timed steps)")
    g = torch.Generator(device=dev).manual_seed(args.seed)
    caches = []
    for _ in range(L):
        cfg = th.TorqueConfig(bit_width=bits, head_dim=d, num_layers=1, kv_heads=hkv, rotation_seed=args.seed)
        cache = th.TorqueKVCacheHIP(config=cfg, initial_capacity=s0 + steps, decode_tail_capacity=0)
        k = torch.randn((1, hkv, s0, d), generator=g, device=dev) * std
        k *= torch.exp(torch.randn((1, hkv, 1, d), generator=g, device=dev))
        v = torch.randn((1, hkv, s0, d), generator=g, device=dev) * std
        cache.append_many(key=k.half(), value=v.half())
        caches.append(cache)
        del k, v
    new_k = (torch.randn((steps, L, hkv, d), generator=g, device=dev) * std).half()
    new_v = (torch.randn((steps, L, hkv, d), generator=g, device=dev) * std).half()
    queries = (torch.randn((steps, L, hq, d), generator=g, device=dev) * std).half()
    torch.cuda.synchronize()

    stores = [c._store for c in caches]
    w = stores[0].layout.packed_words
    loop_kernel = _lib.split_kernel(hkv, hq, d, bits, 0, _lib.TQ_F16, s0 + steps)
    matrix_kernel = loop_kernel.startswith("decode_mx_kernel")
    n_splits = [ops.plan_splits(1, hkv, hq, d, s0 + steps, dev, bit_width=bits) for _ in range(L)]
    ws = ops.workspace_for(1, hkv, hq, d, args.splits, dev)
    out = torch.empty((L, hq, d), dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    lib = _lib.load()
    rot = _lib.TQ_ROTATE_KEYS | _lib.TQ_ROTATE_VALUES
    dflags = _lib.TQ_ROTATE_QUERY | _lib.TQ_INVERSE_OUTPUT
    # Per step and layer: tq_decode_append (pack the new token and decode with it, one launch) -- the
    # default -- or the two-launch tq_append + tq_decode sequence it replaces (`unfused`).
    calls, calls_unfused = [], []
    for t in range(steps):
        seq = s0 + t
        fused_step, unfused_step = [], []
        for l, st in enumerate(stores):
            fused_step.append((lib.tq_decode_append, (
                queries[t, l].data_ptr(), _lib.TQ_F16, new_k[t, l].data_ptr(), new_v[t, l].data_ptr(), _lib.TQ_F16, 1,
                hq, hkv, d, bits, st.key_codes.data_ptr(), st.value_codes.data_ptr(), st.capacity, seq,
                st.key_centroids.data_ptr(), st.value_centroids.data_ptr(), st.key_boundaries.data_ptr(),
                st.value_boundaries.data_ptr(), st.signs_left.data_ptr(), st.signs_right.data_ptr(), rot, dflags,
                args.splits, ws.data_ptr(), ws.numel(), out[l].data_ptr(), stream)))
            unfused_step.append((lib.tq_append, (
                new_k[t, l].data_ptr(), new_v[t, l].data_ptr(), _lib.TQ_F16, 1, hkv, 1, d, bits, st.signs_left.data_ptr(),
                st.signs_right.data_ptr(), rot, st.key_boundaries.data_ptr(), st.value_boundaries.data_ptr(),
                st.key_codes.data_ptr(), st.value_codes.data_ptr(), st.capacity, seq, stream)))
            unfused_step.append((lib.tq_decode, (
                queries[t, l].data_ptr(), _lib.TQ_F16, 1, hq, hkv, d, bits, st.key_codes.data_ptr(),
                st.value_codes.data_ptr(), st.capacity, seq + 1, st.key_centroids.data_ptr(),
                st.value_centroids.data_ptr(), st.signs_left.data_ptr(), st.signs_right.data_ptr(), dflags, None, None,
                args.splits, ws.data_ptr(), ws.numel(), out[l].data_ptr(), stream)))
        calls.append(fused_step)
        calls_unfused.append(unfused_step)

    # warm-up: decode-only passes over every layer at the prefill length (the caches are not changed)
    for _ in range(args.warmup):
        for l, st in enumerate(stores):
            _lib.check(lib.tq_decode(queries[0, l].data_ptr(), _lib.TQ_F16, 1, hq, hkv, d, bits, st.key_codes.data_ptr(),
                                     st.value_codes.data_ptr(), st.capacity, s0, st.key_centroids.data_ptr(),
                                     st.value_centroids.data_ptr(), st.signs_left.data_ptr(),
                                     st.signs_right.data_ptr(), dflags, None, None, args.splits, ws.data_ptr(), ws.numel(),
                                     out[l].data_ptr(), stream))
    # a 1 GiB read between steps evicts the slabs from the 256 MB Infinity Cache; it is outside the events
    flush = torch.empty(2**30, dtype=torch.uint8, device=dev)
    sink = torch.empty(8 * 1024, dtype=torch.float32, device=dev)
    hip.lib.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]

    def timed_steps(stream_handle, launch_step):
        events = [(hip.event(), hip.event()) for _ in range(steps)]
        torch.cuda.synchronize()
        t_start = time.perf_counter()
        for t in range(steps):
            _lib.check(lib.tq_stream_read(flush.data_ptr(), 2**30, sink.data_ptr(), 0, stream_handle, None, None))
            hip.lib.hipEventRecord(events[t][0], stream_handle)
            launch_step(t)
            hip.lib.hipEventRecord(events[t][1], stream_handle)
        # Host time to enqueue the steps (the flush reads give the host room to
        # run ahead, so this is the launch cost, not a wait on the GPU).
        host = (time.perf_counter() - t_start) / steps
        hip.lib.hipStreamSynchronize(ctypes.c_void_p(stream_handle))
        torch.cuda.synchronize()
        return np.array([hip.elapsed_ms(a, b) for a, b in events]) * 1e3, host

    def eager_step(t):
        for fn, a in calls[t]:
            rc = fn(*a)
            if rc != 0:
                _lib.check(rc)

    # The unfused sequence first; every variant replays the same steps (a step rewrites the same token at
    # the same row), so each starts from the same cache contents.
    unfused_us, _ = timed_steps(stream, lambda t: [_lib.check(fn(*a)) for fn, a in calls_unfused[t]])
    unfused_out = out.clone()
    step_us, host_s = timed_steps(stream, eager_step)
    eager_out = out.clone()
    fused_dev = float(np.max(np.abs(eager_out.cpu().numpy() - unfused_out.cpu().numpy())))

    # The same steps captured as one HIP graph per step (the appended offset and the sequence length change
    # every step) and replayed once each: the device-side step latency without host launch overhead.
    # Replaying a step is idempotent (the same token is written at the same offset).
    hl = hip.lib
    gstream = ctypes.c_void_p()
    _hip_ok(hl.hipStreamCreate(ctypes.byref(gstream)), "hipStreamCreate")
    graph_calls = []
    for t in range(steps):
        step_calls = []
        for fn, a in calls[t]:
            a = list(a)
            a[-1] = gstream.value
            step_calls.append((fn, tuple(a)))
        graph_calls.append(step_calls)
    execs = []
    for t in range(steps):
        _hip_ok(hl.hipStreamBeginCapture(gstream, 2), "hipStreamBeginCapture")
        for fn, a in graph_calls[t]:
            rc = fn(*a)
            if rc != 0:
                _lib.check(rc)
        graph = ctypes.c_void_p()
        _hip_ok(hl.hipStreamEndCapture(gstream, ctypes.byref(graph)), "hipStreamEndCapture")
        exe = ctypes.c_void_p()
        _hip_ok(hl.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, ctypes.c_size_t(0)), "hipGraphInstantiate")
        _hip_ok(hl.hipGraphDestroy(graph), "hipGraphDestroy")
        execs.append(exe)
    graph_us, graph_host = timed_steps(gstream.value, lambda t: _hip_ok(hl.hipGraphLaunch(execs[t], gstream),
                                                                      "hipGraphLaunch"))
    graph_dev = float(np.max(np.abs(out.cpu().numpy() - eager_out.cpu().numpy())))
    for exe in execs:
        hl.hipGraphExecDestroy(exe)
    hl.hipStreamDestroy(gstream)
    packed = [L * hkv * (s0 + t + 1) * 2 * w * 4 for t in range(steps)]
    total_bytes = float(sum(packed))
    mean_us = float(step_us.mean())
    log(f"eager step mean {mean_us:.1f} us (median {np.median(step_us):.1f}; host enqueue {host_s * 1e6:.1f} us/step); "
        f"graph-replayed step mean {graph_us.mean():.1f} us (host enqueue {graph_host * 1e6:.1f} us/step); "
        f"graph vs eager output max diff {graph_dev:.1e}")
    log(f"unfused (tq_append + tq_decode) eager step mean {unfused_us.mean():.1f} us; fused vs unfused output max "
        f"diff {fused_dev:.1e}")

    result = {
        "metric": f"decode-loop step latency and packed KV GB/s ({args.workload})",
        "value": round(total_bytes / (step_us.sum() * 1e-6) / 1e9, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(mean_us / 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16-hilo-split/f32-acc" if loop_kernel.startswith("decode_mx_kernel") else "f32",
        "arithmetic": (
            "float32 accumulation of exact float16 hi/lo split products (16x16x32 matrix cores); "
            "softmax, merge and rotations in float32" if matrix_kernel else
            "float32 products and accumulation (4x4x1 fp32 matrix products / VALU FMAs)"
        ),
        "data": "synthetic",
        "config": {
            "workload": desc,
            "layers": L,
            "kv_heads": hkv,
            "query_heads": hq,
            "head_dim": d,
            "bits": bits,
            "prefill": s0,
            "query_dtype": "f16",
            "n_splits_at_prefill": args.splits or n_splits[0],
            "split_kernel": loop_kernel,
            "step": "per layer: tq_decode_append (pack the new token and decode with it) + merge kernel",
        },
        "step_us_mean": round(mean_us, 2),
        "step_us_median": round(float(np.median(step_us)), 2),
        "step_us_min": round(float(step_us.min()), 2),
        "timing": "per step: HIP events around the step's launches on the stream (all layers), a 1 GiB read "
        "between steps outside the events gives the host time to run ahead",
        "host_enqueue_us_per_step": round(host_s * 1e6, 1),
        "graph": {
            "step_us_mean": round(float(graph_us.mean()), 2),
            "host_enqueue_us_per_step": round(graph_host * 1e6, 1),
            "note": "the same steps captured as one HIP graph per step and replayed once each",
        },
        "graph_vs_eager_max_abs": graph_dev,
        "unfused": {
            "step_us_mean": round(float(unfused_us.mean()), 2),
            "step": "per layer: tq_append + tq_decode (two launches plus the merge)",
            "fused_vs_unfused_max_abs": fused_dev,
        },
        "packed_bytes_last_step": packed[-1],
    }
    if not args.no_cpu_baseline:
        from oracle import torque_oracle as o

        st0, c0 = stores[0], caches[0]
        kc_np = st0.key_codes[:, :, :s0].cpu().numpy().view(np.uint32)
        vc_np = st0.value_codes[:, :, :s0].cpu().numpy().view(np.uint32)
        q0 = queries[0, 0].float().cpu().numpy()
        gq = hq // hkv
        times = []
        t_begin = time.perf_counter()
        while time.perf_counter() - t_begin < args.cpu_budget or not times:
            t1 = time.perf_counter()
            q_rot = o.rotation_apply(q0, c0.rotation.signs_left, c0.rotation.signs_right)
            idx = np.arange(hq) // gq
            o.rotation_inverse(o.decode_packed_reference(q_rot, kc_np[0][idx], vc_np[0][idx],
                                                         c0.key_codebook.centroids, c0.value_codebook.centroids,
                                                         bit_width=bits, head_dim=d),
                               c0.rotation.signs_left, c0.rotation.signs_right)
            times.append(time.perf_counter() - t1)
        per_step = float(np.median(times)) * L
        result["cpu_baseline"] = {
            "value": round(packed[0] / per_step / 1e9, 4),
            "unit": "GB/s",
            "us_per_step": round(per_step * 1e6, 1),
            "cores": 1,
            "kind": "port",
            "sample": f"numpy oracle decode of layer 0 at the prefill length, {len(times)} repetitions, "
            f"median scaled by {L} layers (appends not included)",
        }
    calibration_copies(args, torch, dev, result)
    print(json.dumps(result), flush=True)
    return 0


def calibration_copies(args, torch, dev, result) -> None:
    """Five device copies of --calibration-copy-mib MiB: the known-size kernel that scales PMC byte counters."""
    if args.calibration_copy_mib <= 0:
        return
    n = args.calibration_copy_mib * 2**20 // 4
    src = torch.randn(n, device=dev)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    result["calibration_copy_bytes"] = n * 4


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="M", choices=sorted(WORKLOADS) + sorted(LOOP_WORKLOADS))
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--replica-mib", type=int, default=768, help="combined size of the slab replicas cycled through")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-dense", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=12.0)
    ap.add_argument("--splits", type=int, default=0, help="split count (0 = library default)")
    ap.add_argument("--scale-mode", default="none", choices=["none", "rms"],
                    help="per-vector scales of the cache (single-step workloads; 'none' is the reference format)")
    ap.add_argument(
        "--calibration-copy-mib",
        type=int,
        default=0,
        help="also run 5 device copies of this many MiB (the known-size kernel that scales PMC byte counters)",
    )
    args = ap.parse_args()
    args.steps_given = "--steps" in sys.argv

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(
            "bench.py measures one GPU: the decode path would shard by KV head (no exchange) or by sequence "
            "(one all-gather of per-head (max, sum, accumulator) partials, then the same log-sum-exp merge) "
            "across GPUs, but this build runs and reports a single MI355X only.",
            file=sys.stderr,
        )
        return 2

    import torch

    import torque_hip as th
    from torque_hip import _lib, ops

    assert torch.cuda.is_available(), "bench.py needs a HIP device"
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    _lib.load()
    hip = Hip()
    if args.workload in LOOP_WORKLOADS:
        return run_loop(args, torch, th, _lib, ops, hip, dev)

    L, hkv, hq, d, bits, s, std, desc = WORKLOADS[args.workload]
    log(f"workload {desc}")
    q_np, k_np, v_np = synthetic(args.seed, L, hkv, hq, s, d, std)
    scaled = args.scale_mode == "rms"
    cfg = th.TorqueConfig(bit_width=bits, head_dim=d, num_layers=L, kv_heads=hkv, rotation_seed=args.seed,
                          scale_mode=args.scale_mode)
    cache = th.TorqueKVCacheHIP(config=cfg, initial_capacity=s, decode_tail_capacity=0)
    cache.append_many(key=torch.from_numpy(k_np).to(dev), value=torch.from_numpy(v_np).to(dev))
    torch.cuda.synchronize()
    store = cache._store
    w = store.layout.packed_words
    packed_bytes = L * hkv * s * 2 * (w * 4 + (4 if scaled else 0))  # codes (+ one float32 scale per vector)
    algo_bytes = packed_bytes + L * hq * d * (2 + 4)  # + fp16 query in, fp32 output
    n_rep = max(3, ceil(args.replica_mib * 2**20 / packed_bytes))
    log(f"packed K+V {packed_bytes / 2**20:.1f} MiB per step, {n_rep} replicas")
    slabs = (store.key_codes, store.value_codes) + ((store.key_scales, store.value_scales) if scaled else ())
    reps = [slabs] + [tuple(t.clone() for t in slabs) for _ in range(n_rep - 1)]
    queries = [torch.from_numpy(q_np).to(dev)] + [
        torch.randn((L, hq, d), generator=torch.Generator(device=dev).manual_seed(i), device=dev).half()
        for i in range(1, 4)
    ]
    n_splits = args.splits or ops.plan_splits(L, hkv, hq, d, s, dev, bit_width=bits,
                                              flags=_lib.TQ_F32_PRODUCTS if scaled else 0)
    ws = ops.workspace_for(L, hkv, hq, d, n_splits, dev)
    out = torch.empty((L, hq, d), dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    fn = _lib.load().tq_decode_scaled_timed if scaled else _lib.load().tq_decode_timed
    # unscaled calls bind the caller's events to the merge launch as well (tq_decode_step_timed), so a step's
    # time is the split kernel's plus the merge kernel's
    step_fn = None if scaled else _lib.load().tq_decode_step_timed
    flags = _lib.TQ_ROTATE_QUERY | _lib.TQ_INVERSE_OUTPUT
    call_args = []
    for i in range(n_rep):
        qt = queries[i % len(queries)]
        slab_ptrs = tuple(t.data_ptr() for t in reps[i])  # key codes, value codes (, key scales, value scales)
        call_args.append(
            (qt.data_ptr(), _lib.TQ_F16, L, hq, hkv, d, bits, *slab_ptrs, store.capacity, s,
             store.key_centroids.data_ptr(), store.value_centroids.data_ptr(), store.signs_left.data_ptr(),
             store.signs_right.data_ptr(), flags, None, None, n_splits, ws.data_ptr(), ws.numel(), out.data_ptr(),
             stream)
        )

    def run(k_steps, events=None):
        for i in range(k_steps):
            a = call_args[i % n_rep]
            if events is None:
                rc = fn(*a, None, None)
            elif step_fn is not None:
                rc = step_fn(*a, *events[i])
            else:
                rc = fn(*a, events[i][0], events[i][1])
            if rc != 0:
                _lib.check(rc)

    # parity of the benchmarked call (query 0, replica 0) is checked below against the oracle
    run(1)
    torch.cuda.synchronize()
    gpu_out0 = out.cpu().numpy()

    run(args.warmup)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    run(args.steps)
    t_enq = time.perf_counter() - t0
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = wall * 1e3 / args.steps

    # kernel durations: events bound to each launch (hipExtLaunchKernel start/stop)
    n_ev = min(args.steps, 200)
    evs = [(hip.event(), hip.event(), hip.event(), hip.event()) for _ in range(n_ev)]
    torch.cuda.synchronize()
    run(n_ev, evs)
    torch.cuda.synchronize()
    kern_ms = np.array([hip.elapsed_ms(e[0], e[1]) for e in evs])
    kern_us = float(np.mean(kern_ms) * 1e3)
    kern_med_us = float(np.median(kern_ms) * 1e3)
    merge_us = None
    if step_fn is not None and n_splits > 1:
        merge_us = float(np.mean([hip.elapsed_ms(e[2], e[3]) for e in evs]) * 1e3)
    elif n_splits == 1:
        merge_us = 0.0
    achieved = algo_bytes / (kern_us * 1e-6) / 1e9
    kernel_name = _lib.split_kernel(hkv, hq, d, bits, flags | (_lib.TQ_F32_PRODUCTS if scaled else 0), _lib.TQ_F16, s,
                                    num_layers=L, n_splits=n_splits)
    matrix_kernel = kernel_name.startswith("decode_mx_kernel")
    if scaled:
        kernel_name += ",scaled"
    traffic, traffic_src = measured_traffic(kernel_name, args.workload)
    log(f"decode kernel {kernel_name}: mean {kern_us:.2f} us (median {kern_med_us:.2f}), "
        f"wall {ms_per_step * 1e3:.2f} us/step (host enqueue {t_enq * 1e6 / args.steps:.2f} us/step)")
    if merge_us is not None:
        log(f"merge kernel mean {merge_us:.2f} us; step (split + merge) {kern_us + merge_us:.2f} us")

    f32_products = None
    if matrix_kernel:
        # the float32-product split kernel on the same calls (TQ_F32_PRODUCTS), timed the same way
        # call tuple (unscaled): ..., signs_right, flags [15], cur_k, cur_v, n_splits [18], ws, ws bytes, out, stream
        n_f32 = ops.plan_splits(L, hkv, hq, d, s, dev, bit_width=bits, flags=flags | _lib.TQ_F32_PRODUCTS)
        ws32 = ops.workspace_for(L, hkv, hq, d, n_f32, dev)
        f32_args = [a[:15] + (flags | _lib.TQ_F32_PRODUCTS, None, None, n_f32, ws32.data_ptr(), ws32.numel()) + a[21:]
                    for a in call_args]
        for i in range(args.warmup):
            _lib.check(fn(*f32_args[i % n_rep], None, None))
        evs32 = [(hip.event(), hip.event()) for _ in range(n_ev)]
        torch.cuda.synchronize()
        for i in range(n_ev):
            _lib.check(fn(*f32_args[i % n_rep], evs32[i][0], evs32[i][1]))
        torch.cuda.synchronize()
        k32 = np.array([hip.elapsed_ms(a, b) for a, b in evs32]) * 1e3
        f32_products = {
            "kernel": _lib.split_kernel(hkv, hq, d, bits, flags | _lib.TQ_F32_PRODUCTS, _lib.TQ_F16, s,
                                        num_layers=L, n_splits=n_f32),
            "n_splits": n_f32,
            "kernel_us_per_step": round(float(np.mean(k32)), 3),
            "kernel_us_median": round(float(np.median(k32)), 3),
            "frac": round(algo_bytes / (float(np.mean(k32)) * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4),
        }
        log(f"float32-product kernel {f32_products['kernel']}: mean {f32_products['kernel_us_per_step']:.2f} us "
            f"(median {f32_products['kernel_us_median']:.2f})")

    result = {
        "metric": METRIC,
        "value": round(packed_bytes * args.steps / wall / 1e9, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16-hilo-split/f32-acc" if matrix_kernel else "f32",
        "arithmetic": (
            "float32 accumulation of exact float16 hi/lo split products (16x16x32 matrix cores); "
            "softmax, merge and rotations in float32" if matrix_kernel else
            "float32 products and accumulation (4x4x1 fp32 matrix products / VALU FMAs)"
        ),
        "data": "synthetic",
        "config": {
            "workload": desc,
            "layers": L,
            "kv_heads": hkv,
            "query_heads": hq,
            "head_dim": d,
            "bits": bits,
            "seq_len": s,
            "query_dtype": "f16",
            "n_splits": n_splits,
            "slab_replicas": n_rep,
            "scale_mode": args.scale_mode,
        },
        "kernel_us_per_step": round(kern_us, 3),
        "kernel_us_median": round(kern_med_us, 3),
        "host_enqueue_us_per_step": round(t_enq * 1e6 / args.steps, 2),
        "pct_peak": round(100.0 * achieved / HBM_PEAK_GBPS, 2),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": traffic,
            "traffic_source": traffic_src,
            "kernel": kernel_name,
            "algorithmic_bytes_per_launch": algo_bytes,
            # frac above: the split kernel alone (the dominant kernel); below: one whole decode step as the
            # reference's metric times it, the split kernel plus the merge kernel (event-timed means)
            "merge_us": None if merge_us is None else round(merge_us, 3),
            "step_us": None if merge_us is None else round(kern_us + merge_us, 3),
            "step_frac": None if merge_us is None else round(
                algo_bytes / ((kern_us + merge_us) * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4),
        },
        "roofline_compute": compute_roofline(matrix_kernel, L, hkv, hq, d, s, kern_us),
    }
    if f32_products is not None:
        result["f32_products"] = f32_products

    if not args.no_dense:
        # fp16-dense comparator: same shape, dense K/V fp16 slabs, same split-K kernel structure
        dense_bytes = L * hkv * s * d * 2 * 2
        n_drep = max(3, ceil(args.replica_mib * 2**20 / dense_bytes))
        kd = torch.from_numpy(k_np).to(dev)
        vd = torch.from_numpy(v_np).to(dev)
        dreps = [(kd, vd)] + [(kd.clone(), vd.clone()) for _ in range(n_drep - 1)]
        dfn = _lib.load().tq_decode_dense_timed
        dargs = [
            (queries[i % len(queries)].data_ptr(), _lib.TQ_F16, dreps[i][0].data_ptr(), dreps[i][1].data_ptr(),
             _lib.TQ_F16, L, hq, hkv, d, s, s, None, None, 0, n_splits, ws.data_ptr(), ws.numel(), out.data_ptr(),
             stream)
            for i in range(n_drep)
        ]
        for i in range(args.warmup):
            _lib.check(dfn(*dargs[i % n_drep], None, None))
        devs = [(hip.event(), hip.event()) for _ in range(n_ev)]
        torch.cuda.synchronize()
        for i in range(n_ev):
            _lib.check(dfn(*dargs[i % n_drep], devs[i][0], devs[i][1]))
        torch.cuda.synchronize()
        d_us = float(np.mean([hip.elapsed_ms(a, b) for a, b in devs]) * 1e3)
        result["fp16_dense"] = {
            "kernel_us_per_step": round(d_us, 3),
            "hbm_gbps": round((dense_bytes + L * hq * d * 6) / (d_us * 1e-6) / 1e9, 1),
            "bytes_per_step": dense_bytes,
            "packed_speedup": round(d_us / kern_us, 3),
        }
        log(f"fp16-dense kernel {d_us:.2f} us, packed speedup {d_us / kern_us:.2f}x")
        del dreps, kd, vd

    ceiling = read_ceiling(torch, _lib, hip, dev, packed_bytes, args.replica_mib)
    result["hbm_read_ceiling"] = ceiling
    result["roofline"]["frac_of_read_ceiling"] = round(achieved / ceiling["gbps_step_bytes"], 4)
    log(f"streaming-read ceiling {ceiling['gbps_full_pass']:.0f} GB/s (full pass), "
        f"{ceiling['gbps_step_bytes']:.0f} GB/s at {packed_bytes / 2**20:.0f} MiB per launch")

    if not args.no_cpu_baseline:
        kc_np = store.key_codes[:, :, :s].cpu().numpy().view(np.uint32)
        vc_np = store.value_codes[:, :, :s].cpu().numpy().view(np.uint32)
        ks_np = store.key_scales[:, :, :s].cpu().numpy() if scaled else None
        vs_np = store.value_scales[:, :, :s].cpu().numpy() if scaled else None
        per_step, n, workers, err, rel = cpu_baseline(q_np, kc_np, vc_np, cache, args.cpu_budget, gpu_out0, ks_np, vs_np)
        result["cpu_baseline"] = {
            "value": round(packed_bytes / per_step / 1e9, 4),
            "unit": "GB/s",
            "us_per_step": round(per_step * 1e6, 1),
            "cores": workers,
            "kind": "port",
            "sample": f"numpy oracle decode of all {hq} query heads at the full sequence length, one query head "
            f"per task on {workers} forked single-threaded worker processes, {n} steps, median",
            "host_cpu_count": os.cpu_count(),
            "host_affinity_cores": len(os.sched_getaffinity(0)),
            "thread_env": {k: os.environ.get(k) for k in ("OMP_NUM_THREADS", "OPENBLAS_NUM_THREADS", "MKL_NUM_THREADS")},
            "worker_threads": 1,
        }
        result["parity_vs_oracle"] = {"max_abs": err, "rel_l2": rel, "heads_checked": hq}
        log(f"cpu baseline {per_step * 1e6:.0f} us/step on {workers} processes; parity max-abs {err:.2e} rel-L2 {rel:.2e}")
        if L * hkv * s <= 8 * 1024 and not scaled:
            lit, n_lit = cpu_literal_baseline(q_np, kc_np, vc_np, cache, min(args.cpu_budget, 10.0))
            result["cpu_baseline_literal"] = {
                "value": round(packed_bytes / lit / 1e9, 6),
                "unit": "GB/s",
                "us_per_step": round(lit * 1e6, 1),
                "cores": 1,
                "kind": "port",
                "sample": "literal per-element path, single thread: per-code unpack loop (quantization.py:272-290) "
                f"of every row and the per-token online-softmax loop (reference.py:8-42), {n_lit} steps, median",
            }
            log(f"cpu literal per-element path {lit * 1e6:.0f} us/step")

    calibration_copies(args, torch, dev, result)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
