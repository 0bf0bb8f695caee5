"""KV store+retrieve throughput on one MI355X.

Workload (Llama-3-8B KV shape): 32 layers, 8 KV heads x 128, bf16, block size
128, SEPARATE_KV paged caches of 2048 blocks per layer and plane (N(0,1) from
a seed); 4 requests of 1000, 1100, 996 and 1000 tokens (each ends in a
partial block) laid out in 33 blocks drawn from a seeded permutation; the
4096 tokens are stored into / retrieved from 16 LMCache memory objects of
[2, 32, 256, 1024].

One step = store (paged -> memory objects) + retrieve (memory objects ->
paged) of the whole batch, device to device, each direction one launch of
the gather/scatter kernel.  `value` = payload bytes of both directions
(each valid (layer, token, plane) row counted once per direction, decimal
GB) / step time.  The same line reports the pinned-host (PCIe) mode, the
per-chunk drop-in call path, the kernel's HBM roofline fraction (HIP events
on the launch stream) and the CPU oracle on a bounded sample.

    python bench.py [--gpus 1] [--steps K] [--warmup W]
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "lmcache-ascend_amd"))
sys.path.insert(0, REPO)

METRIC = "KV store+retrieve GB/s, 8B-shape 32L 4096 tok bf16; % of HBM/PCIe roofline"
HBM_PEAK_GBS = 8000.0      # MI355X HBM3E, published
PCIE_PEAK_GBS = 64.0       # PCIe Gen5 x16, per direction, nominal

L, NB, BS, H, D = 32, 2048, 128, 8, 128
W = H * D
ES = 2
REQUEST_LENGTHS = [1000, 1100, 996, 1000]
CHUNK = 256


def block_slots(block_ids, block_size, lengths):
    """Slots of consecutive requests, each filling fresh blocks in order."""
    out, it = [], iter(block_ids)
    for n in lengths:
        blocks = [next(it) for _ in range((n + block_size - 1) // block_size)]
        out.extend(blocks[i // block_size] * block_size + i % block_size for i in range(n))
    return out


def build_workload(torch, ops, device):
    torch.manual_seed(0)
    flat = []
    for _ in range(L):
        flat.append(torch.randn((NB, BS, H, D), device=device, dtype=torch.bfloat16))
        flat.append(torch.randn((NB, BS, H, D), device=device, dtype=torch.bfloat16))
    ptrs = torch.tensor([t.data_ptr() for t in flat], dtype=torch.int64, device=device)
    gen = torch.Generator().manual_seed(1)
    blocks = torch.randperm(NB, generator=gen).tolist()
    slots_list = block_slots(blocks, BS, REQUEST_LENGTHS)
    slots = torch.tensor(slots_list, dtype=torch.int64, device=device)
    n_tok = len(slots_list)
    starts = list(range(0, n_tok, CHUNK))
    chunks = [torch.empty((2, L, min(CHUNK, n_tok - s), W), dtype=torch.bfloat16, device=device) for s in starts]
    return flat, ptrs, slots, starts, chunks, n_tok


def time_events(torch, stream, fn, iters):
    """Median / mean of `fn` on `stream` measured with HIP events."""
    evs = []
    for _ in range(iters):
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(stream)
        fn()
        b.record(stream)
        evs.append((a, b))
    torch.cuda.synchronize()
    ms = [a.elapsed_time(b) for a, b in evs]
    return statistics.median(ms), statistics.mean(ms), ms


def cpu_oracle_rate(budget_s=3.0):
    """The oracle's numpy gather/scatter (one thread) on the same sample as
    cpu_torch_rate: GB/s of store+retrieve payload."""
    import numpy as np

    from oracle import kv_transfer as ok

    rng = np.random.default_rng(0)
    nb_cpu = 64
    pbs = nb_cpu * BS
    table = [np.full(pbs * W * ES, i, dtype=np.uint8) for i in range(2 * L)]
    blocks = [int(b) for b in rng.permutation(nb_cpu)[:33]]
    slots = np.asarray(block_slots(blocks, BS, REQUEST_LENGTHS), dtype=np.int64)
    lmc = [np.zeros(2 * L * CHUNK * W * ES, np.uint8) for _ in range(len(slots) // CHUNK)]
    payload = 0
    t0 = time.perf_counter()
    while True:
        for i, buf in enumerate(lmc):
            s = slots[i * CHUNK:(i + 1) * CHUNK]
            ok.multi_layer_kv_transfer(buf, table, s, pbs, True, False, 2, L, W, ES)
            ok.multi_layer_kv_transfer(buf, table, s, pbs, False, False, 2, L, W, ES)
            payload += 2 * (2 * L * len(s) * W * ES)
        if time.perf_counter() - t0 >= budget_s:
            break
    return round(payload / (time.perf_counter() - t0) / 1e9, 3)


def cpu_model() -> str:
    """lscpu's model name (falls back to /proc/cpuinfo)."""
    try:
        import subprocess

        res = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20)
        for line in res.stdout.splitlines():
            if line.strip().startswith("Model name:"):
                return line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def usable_cores() -> int:
    """Cores this process may run on: os.cpu_count(), limited to the CPU
    affinity set the host gives the process."""
    n = os.cpu_count() or 1
    try:
        n = min(n, len(os.sched_getaffinity(0)))
    except (AttributeError, OSError):
        pass
    return max(1, n)


def cpu_torch_rate(torch, threads, budget_s):
    """The reference's CPU path (tools/cpu_vllm_runtime.py:352-419:
    index_select for the store, index_copy_ for the retrieve, per layer and
    plane) on the benchmark's 16 chunks x 32 layers x 2 planes x 2 KiB rows
    against a 64-block-per-layer host pool (the full 32 GiB pool does not fit
    the host; the pool size does not change the per-row work), with
    `threads` torch threads.  Returns (GB/s of payload, tokens/s, passes,
    seconds)."""
    g = torch.Generator().manual_seed(0)
    nb_cpu = 64
    pool = [[torch.randn((nb_cpu * BS, W), generator=g).to(torch.bfloat16) for _ in range(2)] for _ in range(L)]
    blocks = [int(b) for b in torch.randperm(nb_cpu, generator=g)[:33]]
    slots = torch.tensor(block_slots(blocks, BS, REQUEST_LENGTHS), dtype=torch.int64)
    n_chunks = len(slots) // CHUNK
    lmc = [torch.empty((2, L, CHUNK, W), dtype=torch.bfloat16) for _ in range(n_chunks)]

    def one_pass():
        for i in range(n_chunks):
            s = slots[i * CHUNK:(i + 1) * CHUNK]
            for l in range(L):
                for p in range(2):
                    torch.index_select(pool[l][p], 0, s, out=lmc[i][p, l])
            for l in range(L):
                for p in range(2):
                    pool[l][p].index_copy_(0, s, lmc[i][p, l])
        return 2 * 2 * L * len(slots) * W * ES

    before = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        one_pass()
        payload, passes, t0 = 0, 0, time.perf_counter()
        while True:
            payload += one_pass()
            passes += 1
            if time.perf_counter() - t0 >= budget_s:
                break
        dt = time.perf_counter() - t0
    finally:
        torch.set_num_threads(before)
    return round(payload / dt / 1e9, 3), round(payload / (2 * 2 * L * W * ES) / dt), passes, dt


def cpu_baseline(torch, budget_s=10.0):
    """The reference's CPU path (cpu_torch_rate) on every usable core, with
    the one-thread rate and the numpy oracle's one-thread rate beside it."""
    cores = usable_cores()
    value, tok_s, passes, dt = cpu_torch_rate(torch, cores, budget_s)
    one, one_tok, _, _ = cpu_torch_rate(torch, 1, min(3.0, budget_s))
    return {
        "value": value,
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": f"{passes} x (store+retrieve of 16 chunks [2,32,256,1024] bf16, SEPARATE_KV) against a "
                  f"64-block/layer host pool, torch index_select / index_copy_ (tools/cpu_vllm_runtime.py "
                  f"style), {cores} threads, {dt:.1f} s",
        "tokens_per_s": tok_s,
        "cpu_model": cpu_model(),
        "os_cpu_count": os.cpu_count(),
        "threads_1": {"value": one, "tokens_per_s": one_tok},
        "numpy_oracle_threads_1": {"value": cpu_oracle_rate(min(3.0, budget_s))},
    }


def load_traffic():
    """HBM traffic per launch from the committed rocprofv3 --pmc summary."""
    path = os.path.join(REPO, "profiles", "kv_rows_copy_llama8b_4096tok_traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get("traffic_bytes_per_launch")


CG_LAYERS, CG_TOKENS, CG_CHANNELS, CG_CHUNK = 32, 256, 1024, 256


def quantize_gpu(torch, x, bins):
    """Per-(layer, channel) symmetric quantiser of [L, T, C] data into
    [0, bins - 2] (bins per layer)."""
    half = (bins // 2 - 1).to(torch.float32).view(-1, 1, 1)
    amax = x.abs().amax(dim=1, keepdim=True).clamp_min(1e-30)
    return (torch.round(x / amax * half) + half).to(torch.uint8)


def bench_cachegen(torch, ops, dev, stream):
    """calculate_cdf / encode / decode of one K+V chunk: 32 layers x 256
    tokens x 1024 channels per K and V; K layers 0-9 quantised to 32 bins,
    later K layers and all V layers to 16."""
    g = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn((2 * CG_LAYERS, CG_TOKENS, CG_CHANNELS), generator=g, device=dev)
    bins = torch.full((2 * CG_LAYERS,), 16, device=dev)
    bins[:10] = 32
    sym = quantize_gpu(torch, x, bins)
    cdf = ops.calculate_cdf(sym, 32)
    out = torch.zeros((2 * CG_LAYERS, CG_CHANNELS, CG_CHUNK), dtype=torch.uint8, device=dev)
    lens = torch.zeros((2 * CG_LAYERS, CG_CHANNELS), dtype=torch.int32, device=dev)
    ops.encode_fast_new(cdf, sym, out, lens)
    torch.cuda.synchronize()
    rows = out.view(-1, CG_CHUNK)
    keep = torch.arange(CG_CHUNK, device=dev)[None, :] < lens.view(-1, 1)
    stream_bytes = rows[keep].contiguous()
    pref = lens.view(-1).cumsum(0).to(torch.int32).view_as(lens)
    dec = torch.empty_like(sym)
    t_cdf = time_events(torch, stream, lambda: ops.calculate_cdf(sym, 32), 20)[0]
    t_enc = time_events(torch, stream, lambda: ops.encode_fast_new(cdf, sym, out, lens), 20)[0]
    t_dec = time_events(torch, stream, lambda: ops.decode_fast_prefsum(cdf, stream_bytes, pref, dec), 20)[0]
    ok = bool(torch.equal(dec, sym))
    n_sym = sym.numel()
    enc_bytes = int(stream_bytes.numel())
    cdf_bytes = cdf.numel() * 2
    return {
        "cachegen_calculate_cdf": {"ms": round(t_cdf, 4), "Gsym_per_s": round(n_sym / t_cdf / 1e6, 2),
                                   "GBps": round((n_sym + cdf_bytes) / t_cdf / 1e6, 1)},
        "cachegen_encode": {"ms": round(t_enc, 4), "Gsym_per_s": round(n_sym / t_enc / 1e6, 2),
                            "GBps": round((n_sym + cdf_bytes + enc_bytes) / t_enc / 1e6, 1),
                            "bits_per_symbol": round(8 * enc_bytes / n_sym, 3)},
        "cachegen_decode": {"ms": round(t_dec, 4), "Gsym_per_s": round(n_sym / t_dec / 1e6, 2),
                            "GBps": round((n_sym + cdf_bytes + enc_bytes) / t_dec / 1e6, 1),
                            "round_trip_exact": ok},
    }


def bench_rope(torch, ops, dev, stream):
    """rotary_embedding_k_fused: 4096 tokens x 8 heads x 128 bf16 K,
    positions 0..4095 -> 1000..5095, theta 500000, neox."""
    T, Hh, Dh, base = 4096, 8, 128, 500000.0
    inv = 1.0 / (base ** (torch.arange(0, Dh, 2, dtype=torch.float32, device=dev) / Dh))
    ang = torch.outer(torch.arange(8192, dtype=torch.float32, device=dev), inv)
    cache = torch.cat((ang.cos(), ang.sin()), dim=-1).to(torch.bfloat16)
    k = torch.randn((T, Hh * Dh), device=dev).to(torch.bfloat16)
    old = torch.arange(T, device=dev)
    new = old + 1000
    t = time_events(torch, stream, lambda: ops.rotary_embedding_k_fused(old, new, k, Dh, cache, True), 20)[0]
    nbytes = 2 * k.numel() * 2 + 2 * T * Dh * 2 + 16 * T
    # The floor for one launch moving this much: the runtime's device copy
    # of the same 8 MiB of K (read once, written once).
    k2 = torch.empty_like(k)
    t_copy = time_events(torch, stream, lambda: k2.copy_(k), 20)[0]
    return {"rope_k_fused": {"ms": round(t, 4), "GBps": round(nbytes / t / 1e6, 1),
                             "hbm_frac": round(nbytes / t / 1e6 / HBM_PEAK_GBS, 4),
                             "tokens_per_s": round(T / t * 1e3)},
            "hipmemcpy_d2d_rope_key_8MiB": {"ms": round(t_copy, 4),
                                            "GBps": round(2 * k.numel() * 2 / t_copy / 1e6, 1)}}


def bench_blend(torch, ops, dev, stream, flat, slots):
    """The CacheBlend layerwise retrieve as the reference's connector runs it
    (lmcache_ascend/v1/npu_connector/npu_connectors.py:556-689,
    VLLMBufferLayerwiseNPUConnector.batched_to_gpu): for each of the 32
    layers, 16 pinned KV_2TD memory objects [2, 256, 1024] are copied into a
    [2, 4096, 1024] load buffer on a load stream; the buffer loaded one step
    earlier has its K re-rotated in place (rotary_embedding_k_fused, cached
    positions 0..4095 -> 1000..5095, theta 500000); the buffer of two steps
    earlier is scattered into the paged caches (single_layer_kv_transfer);
    a device-wide synchronize separates the steps and two buffers ping-pong.
    Also timed: the same work with three buffers ordered by events instead
    of device-wide synchronizes, each stage alone, and the 32 layers through
    blend_layer_to_paged (one kernel per layer, objects read in place)."""
    T = slots.numel()
    n_obj = T // CHUNK
    host = torch.randn((L, n_obj, 2, CHUNK, W), dtype=torch.float32).to(torch.bfloat16).pin_memory()
    bufs = [torch.empty((2, T, W), dtype=torch.bfloat16, device=dev) for _ in range(3)]
    inv = 1.0 / (500000.0 ** (torch.arange(0, D, 2, dtype=torch.float32, device=dev) / D))
    ang = torch.outer(torch.arange(8192, dtype=torch.float32, device=dev), inv)
    cache = torch.cat((ang.cos(), ang.sin()), dim=-1).to(torch.bfloat16)
    old = torch.arange(T, dtype=torch.int64, device=dev)
    new = old + 1000
    load_stream = torch.cuda.Stream(dev)

    def h2d(buf, layer):
        for c in range(n_obj):
            buf[0][c * CHUNK:(c + 1) * CHUNK].copy_(host[layer, c, 0], non_blocking=True)
            buf[1][c * CHUNK:(c + 1) * CHUNK].copy_(host[layer, c, 1], non_blocking=True)

    def rope(buf):
        ops.rotary_embedding_k_fused(old, new, buf[0], D, cache, True)

    def scatter(buf, layer):
        ops.single_layer_kv_transfer(buf, (flat[2 * layer], flat[2 * layer + 1]), slots, False, 2, False, False)

    def reference_pattern():
        compute, load = bufs[0], bufs[1]
        mapping = {}
        for layer_id in range(L + 2):
            if layer_id > 1:
                scatter(mapping.pop(layer_id - 2), layer_id - 2)
            if 0 < layer_id <= L:
                torch.cuda.synchronize()
                compute, load = load, compute
                rope(compute)
                mapping[layer_id - 1] = compute
            if layer_id < L:
                with torch.cuda.stream(load_stream):
                    h2d(load, layer_id)
        torch.cuda.synchronize()

    def event_pipelined():
        loaded = [torch.cuda.Event() for _ in range(L)]
        done = [torch.cuda.Event() for _ in range(L)]
        for layer in range(L):
            buf = bufs[layer % 3]
            with torch.cuda.stream(load_stream):
                if layer >= 3:
                    load_stream.wait_event(done[layer - 3])
                h2d(buf, layer)
                loaded[layer].record(load_stream)
            stream.wait_event(loaded[layer])
            rope(buf)
            scatter(buf, layer)
            done[layer].record(stream)
        torch.cuda.synchronize()

    def wall(fn, reps=5):
        fn()
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            ts.append((time.perf_counter() - t0) * 1e3)
        return statistics.median(ts)

    # The same 32 layers through blend_layer_to_paged: one kernel per layer
    # reads the layer's pinned objects in place, re-rotates K and scatters
    # (no load buffer, no copy-engine copies).
    objs = [[host[layer, c] for c in range(n_obj)] for layer in range(L)]
    obj_starts = [c * CHUNK for c in range(n_obj)]

    def fused_layers():
        for layer in range(L):
            ops.blend_layer_to_paged(objs[layer], obj_starts, (flat[2 * layer], flat[2 * layer + 1]), slots,
                                     old_positions=old, new_positions=new, cos_sin_cache=cache, head_size=D,
                                     is_neox=True, kvcache_format_raw=2)
        torch.cuda.synchronize()

    t_ref = wall(reference_pattern)
    t_evt = wall(event_pipelined)
    t_fused = wall(fused_layers)
    t_fused_one = time_events(torch, stream, lambda: ops.blend_layer_to_paged(
        objs[0], obj_starts, (flat[0], flat[1]), slots, old_positions=old, new_positions=new, cos_sin_cache=cache,
        head_size=D, is_neox=True, kvcache_format_raw=2), 20)[0]
    # The same calls with the memory objects in device memory (an HBM-bound
    # layer load: 2 x 16 MiB of traffic per layer), each layer its own objects.
    dhost = host.to(dev)
    dobjs = [[dhost[layer, c] for c in range(n_obj)] for layer in range(L)]

    def fused_layers_device():
        for layer in range(L):
            ops.blend_layer_to_paged(dobjs[layer], obj_starts, (flat[2 * layer], flat[2 * layer + 1]), slots,
                                     old_positions=old, new_positions=new, cos_sin_cache=cache, head_size=D,
                                     is_neox=True, kvcache_format_raw=2)

    fused_layers_device()
    t_fused_dev = time_events(torch, stream, fused_layers_device, 5)[0]
    del dhost, dobjs
    with torch.cuda.stream(load_stream):
        t_h2d = time_events(torch, load_stream, lambda: h2d(bufs[0], 0), 10)[0]
    t_rope = time_events(torch, stream, lambda: rope(bufs[1]), 20)[0]
    t_scatter = time_events(torch, stream, lambda: scatter(bufs[1], 0), 20)[0]
    layer_bytes = 2 * T * W * ES
    out = {}
    for name, t in (("blend_layerwise_reference_pattern_32_layers", t_ref),
                    ("blend_layerwise_event_pipelined_32_layers", t_evt),
                    ("blend_layer_to_paged_fused_32_layers", t_fused)):
        out[name] = {"ms": round(t, 4), "ms_per_layer": round(t / L, 4),
                     "payload_GBps": round(L * layer_bytes / (t * 1e-3) / 1e9, 2),
                     "pcie_frac": round(L * layer_bytes / (t * 1e-3) / 1e9 / PCIE_PEAK_GBS, 4)}
    out["blend_stage_h2d_16_objects_one_layer"] = {"ms": round(t_h2d, 4),
                                                   "payload_GBps": round(layer_bytes / (t_h2d * 1e-3) / 1e9, 2)}
    out["blend_stage_rope_one_layer"] = {"ms": round(t_rope, 4)}
    out["blend_layer_to_paged_one_layer"] = {"ms": round(t_fused_one, 4),
                                             "payload_GBps": round(layer_bytes / (t_fused_one * 1e-3) / 1e9, 2),
                                             "pcie_frac": round(layer_bytes / (t_fused_one * 1e-3) / 1e9 / PCIE_PEAK_GBS,
                                                                4)}
    out["blend_layer_to_paged_device_objects_32_layers"] = {
        "ms": round(t_fused_dev, 4), "ms_per_layer": round(t_fused_dev / L, 4),
        "hbm_GBps": round(2 * layer_bytes * L / (t_fused_dev * 1e-3) / 1e9, 1),
        "hbm_frac": round(2 * layer_bytes * L / (t_fused_dev * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    out["blend_stage_scatter_one_layer"] = {"ms": round(t_scatter, 4),
                                            "hbm_GBps": round(2 * layer_bytes / (t_scatter * 1e-3) / 1e9, 1)}
    del host, bufs
    return out


def bench_qwen32b_long_prefix(torch, ops, dev, stream):
    """Qwen3-32B shape: 64 layers x 8x128 bf16, block 128; one 32768-token
    request as 128 memory objects of 256 tokens; its 256 blocks drawn without
    replacement from a 4096-block pool; 1638 slots (5%) set to -1 and
    skipped.  Batched multi-layer store/retrieve, then
    single_layer_kv_transfer layer by layer ([2, 32768, 1024] per layer)."""
    L3, NB3, T3 = 64, 4096, 32768
    torch.manual_seed(3)
    flat = [torch.randn((NB3, BS, H, D), device=dev, dtype=torch.bfloat16) for _ in range(2 * L3)]
    ptrs = torch.tensor([t.data_ptr() for t in flat], dtype=torch.int64, device=dev)
    gen = torch.Generator().manual_seed(3)
    blocks = torch.randperm(NB3, generator=gen)[: T3 // BS].tolist()
    slots = torch.tensor(block_slots(blocks, BS, [T3]), dtype=torch.int64)
    pad = torch.randperm(T3, generator=gen)[: round(0.05 * T3)]
    slots[pad] = -1
    valid = int((slots >= 0).sum())
    slots = slots.to(dev)
    starts = list(range(0, T3, CHUNK))
    chunks = [torch.empty((2, L3, CHUNK, W), dtype=torch.bfloat16, device=dev) for _ in starts]
    pbs3 = NB3 * BS
    store = lambda: ops.multi_layer_kv_transfer_batched(chunks, ptrs, slots, starts, dev, pbs3, True, False, 2, W, W, 0)
    retr = lambda: ops.multi_layer_kv_transfer_batched(chunks, ptrs, slots, starts, dev, pbs3, False, False, 2, W, W, 0)
    store(); retr()
    t_s = time_events(torch, stream, store, 5)[0]
    t_r = time_events(torch, stream, retr, 5)[0]
    buf = torch.empty((2, T3, W), dtype=torch.bfloat16, device=dev)

    def sl(direction):
        for l in range(L3):
            ops.single_layer_kv_transfer(buf, (flat[2 * l], flat[2 * l + 1]), slots, direction, 2)

    sl(True); sl(False)
    t_ss = time_events(torch, stream, lambda: sl(True), 3)[0]
    t_sr = time_events(torch, stream, lambda: sl(False), 3)[0]
    P3 = L3 * valid * 2 * W * ES
    out = {}
    for name, t in (("qwen32b_multi_layer_store", t_s), ("qwen32b_multi_layer_retrieve", t_r),
                    ("qwen32b_single_layer_store_64_layers", t_ss), ("qwen32b_single_layer_retrieve_64_layers", t_sr)):
        out[name] = {"ms": round(t, 3), "payload_GBps": round(P3 / t / 1e6, 1),
                     "hbm_frac": round(2 * P3 / t / 1e6 / HBM_PEAK_GBS, 4)}
    out["qwen32b_valid_tokens"] = valid
    del flat, chunks, buf
    torch.cuda.empty_cache()
    return out


def bench_mla_576(torch, ops, dev, stream):
    """DeepSeek-V3-style latent cache: 61 layers, one [1024, 64, 576] bf16
    tensor per layer (use_mla=True), N(0, 0.5); 8 requests x 2048 tokens in
    a random block permutation; memory objects [1, 61, 2048, 576]."""
    L4, NB4, BS4, W4, NR, TR = 61, 1024, 64, 576, 8, 2048
    torch.manual_seed(4)
    caches = [torch.randn((NB4, BS4, W4), device=dev, dtype=torch.bfloat16) * 0.5 for _ in range(L4)]
    ptrs = torch.tensor([t.data_ptr() for t in caches], dtype=torch.int64, device=dev)
    gen = torch.Generator().manual_seed(4)
    blocks = torch.randperm(NB4, generator=gen).tolist()
    slots = torch.tensor(block_slots(blocks, BS4, [TR] * NR), dtype=torch.int64, device=dev)
    starts = [i * TR for i in range(NR)]
    objs = [torch.empty((1, L4, TR, W4), dtype=torch.bfloat16, device=dev) for _ in range(NR)]
    pbs4 = NB4 * BS4
    store = lambda: ops.multi_layer_kv_transfer_batched(objs, ptrs, slots, starts, dev, pbs4, True, True, 1, 0, 0, 0)
    retr = lambda: ops.multi_layer_kv_transfer_batched(objs, ptrs, slots, starts, dev, pbs4, False, True, 1, 0, 0, 0)
    store(); retr()
    t_s = time_events(torch, stream, store, 10)[0]
    t_r = time_events(torch, stream, retr, 10)[0]
    # Ceilings for the same bytes: identity slots (blocks 0..255 in order, so
    # every (layer, object) pair is one contiguous run on both sides) and the
    # runtime's device copy of the whole payload at once.
    ident = torch.arange(NR * TR, dtype=torch.int64, device=dev)
    store_i = lambda: ops.multi_layer_kv_transfer_batched(objs, ptrs, ident, starts, dev, pbs4, True, True, 1, 0, 0, 0)
    retr_i = lambda: ops.multi_layer_kv_transfer_batched(objs, ptrs, ident, starts, dev, pbs4, False, True, 1, 0, 0, 0)
    store_i(); retr_i()
    t_si = time_events(torch, stream, store_i, 10)[0]
    t_ri = time_events(torch, stream, retr_i, 10)[0]
    P4 = L4 * NR * TR * W4 * ES
    m_src = torch.empty(P4, dtype=torch.uint8, device=dev)
    m_dst = torch.empty_like(m_src)
    m_dst.copy_(m_src)
    t_m = time_events(torch, stream, lambda: m_dst.copy_(m_src), 10)[0]
    del m_src, m_dst
    out = {}
    for name, t in (("mla576_store", t_s), ("mla576_retrieve", t_r), ("mla576_identity_slots_store", t_si),
                    ("mla576_identity_slots_retrieve", t_ri), ("hipmemcpy_d2d_mla576_same_bytes", t_m)):
        out[name] = {"ms": round(t, 4), "payload_GBps": round(P4 / t / 1e6, 1),
                     "hbm_frac": round(2 * P4 / t / 1e6 / HBM_PEAK_GBS, 4)}
    del caches, objs
    torch.cuda.empty_cache()
    return out


def bench_direct(torch, ops, dev, stream):
    """Sparse / direct single-layer transfers on one DeepSeek-style MLA layer
    (kv_lora 512 + rope 64 bf16, 1024 blocks of 64 slots): dense direct store
    and load of 16384 tokens in 64 pinned memory objects of 256 tokens
    (PCIe); sparse direct retrieve of 2048 selected tokens from those
    objects (PCIe); sparse single-layer scatter of 65536 selected tokens from
    a device staging buffer (HBM); and the staged batched path on one
    Llama-shape SEPARATE_KV layer (8 x 128, 4096 tokens in 16 pinned objects
    of 256; PCIe)."""
    NB, BS, KH, VH = 1024, 64, 512, 64
    gen = torch.Generator().manual_seed(7)
    k = torch.randn((NB, BS, 1, KH), device=dev, dtype=torch.bfloat16)
    v = torch.randn((NB, BS, 1, VH), device=dev, dtype=torch.bfloat16)
    caches = (k, v)
    row = (KH + VH) * ES
    T, CS = 16384, 256
    slots = torch.randperm(NB * BS, generator=gen)[:T].to(dev)
    objs = [torch.zeros(CS * (KH + VH), dtype=torch.bfloat16, pin_memory=True) for _ in range(T // CS)]
    ptrs = ops._chunk_ptrs_for(objs, dev)
    offs = torch.arange(0, T, CS, dtype=torch.int32, device=dev)
    sizes = torch.full((T // CS,), CS, dtype=torch.int32, device=dev)
    st = ops.prepare_sparse_direct_destination_state(caches, slots, 3, 0, 0, 0)
    lay = ops.prepare_sparse_direct_layer_state(objs[0], caches, slots, False, False, 3, 0, 0, 0, CS)
    store = lambda: ops.dense_mla_dsa_batched_direct_kv_transfer_fast(lay, slots, ptrs, offs, sizes, T, False, True,
                                                                      False, CS)
    load = lambda: ops.dense_mla_dsa_batched_direct_kv_transfer_prepared(st, slots, ptrs, offs, sizes, T, False,
                                                                         False, CS)
    NS = 2048
    sel = torch.randperm(T, generator=gen)[:NS].to(torch.int32).to(dev)
    sslots = torch.randperm(NB * BS, generator=gen)[:NS].to(dev)
    sparse = lambda: ops.sparse_mla_dsa_batched_direct_kv_transfer_prepared(st, sslots, sel, ptrs, CS, T, False)
    store(); load(); sparse()
    t_st = time_events(torch, stream, store, 20)[0]
    t_ld = time_events(torch, stream, load, 20)[0]
    t_sp = time_events(torch, stream, sparse, 20)[0]
    TH = 65536
    staging = torch.randn(TH * (KH + VH), device=dev, dtype=torch.bfloat16)
    hsel = torch.randperm(TH, generator=gen).to(torch.int32).to(dev)
    hslots = torch.randperm(NB * BS, generator=gen)[:TH].to(dev)
    scatter = lambda: ops.sparse_single_layer_kv_transfer(staging, caches, hslots, hsel, 3)
    scatter()
    t_sc = time_events(torch, stream, scatter, 20)[0]
    # staged batched path, one Llama-shape layer
    LT, LW = 4096, 8 * 128
    lk = torch.randn((2048, 128, 8, 128), device=dev, dtype=torch.bfloat16)
    lv = torch.randn((2048, 128, 8, 128), device=dev, dtype=torch.bfloat16)
    lslots = torch.randperm(2048 * 128, generator=gen)[:LT].to(dev)
    lobjs = [torch.zeros((2, 256, LW), dtype=torch.bfloat16, pin_memory=True) for _ in range(LT // 256)]
    lstg = torch.empty((2, LT, LW), dtype=torch.bfloat16, device=dev)
    loffs, lsizes = list(range(0, LT, 256)), [256] * (LT // 256)
    bf_from = lambda: ops.batched_fused_single_layer_kv_transfer(lobjs, lstg, (lk, lv), lslots, loffs, lsizes, True, 2)
    bf_to = lambda: ops.batched_fused_single_layer_kv_transfer(lobjs, lstg, (lk, lv), lslots, loffs, lsizes, False, 2)
    bf_from(); bf_to()
    t_bf = time_events(torch, stream, bf_from, 10)[0]
    t_bt = time_events(torch, stream, bf_to, 10)[0]
    torch.cuda.synchronize()

    def pcie(nbytes, ms):
        return {"ms": round(ms, 4), "payload_GBps": round(nbytes / ms / 1e6, 2),
                "pcie_frac": round(nbytes / ms / 1e6 / PCIE_PEAK_GBS, 4)}

    out = {
        "direct_dense_store_mla_16k": pcie(T * row, t_st),
        "direct_dense_load_mla_16k": pcie(T * row, t_ld),
        "direct_sparse_load_mla_2048_of_16k": pcie(NS * row, t_sp),
        "sparse_single_layer_mla_64k": {"ms": round(t_sc, 4), "payload_GBps": round(TH * row / t_sc / 1e6, 1),
                                        "hbm_frac": round(2 * TH * row / t_sc / 1e6 / HBM_PEAK_GBS, 4)},
        "batched_fused_from_gpu_llama_layer": pcie(2 * LT * LW * ES, t_bf),
        "batched_fused_to_gpu_llama_layer": pcie(2 * LT * LW * ES, t_bt),
    }
    del k, v, objs, staging, lk, lv, lobjs, lstg
    torch.cuda.empty_cache()
    return out


def _planner_rows(pool, chunk, n_chunks, cache_addrs, plane_bytes, blocks, bs, d2h):
    """(dst, src, bytes) rows for chunks of `chunk` tokens laid out [plane,
    token, row] back to back from `pool`: one row per plane for every token
    range that stays on consecutive block ids."""
    rows = []
    for c in range(n_chunks):
        t, e = c * chunk, (c + 1) * chunk
        while t < e:
            b = t // bs
            while (b + 1) * bs < e and blocks[b + 1] == blocks[b] + 1:
                b += 1
            t1 = min(e, (b + 1) * bs)
            slot = blocks[t // bs] * bs + t % bs
            off = 0
            for addr, pbytes in zip(cache_addrs, plane_bytes):
                host = pool + c * chunk * sum(plane_bytes) + chunk * off + (t - c * chunk) * pbytes
                dev = addr + slot * pbytes
                rows.append((host, dev, (t1 - t) * pbytes) if d2h else (dev, host, (t1 - t) * pbytes))
                off += pbytes
            t = t1
    return rows


def bench_layerwise_dma(torch, ops, dev, stream):
    """Layerwise prefill copies of one Llama-shape SEPARATE_KV layer (8 x 128
    bf16 per plane, 2048 blocks of 128 tokens): 4096 tokens in 16 memory
    objects of 256 tokens carved from one pinned pool, rows bound as the
    connector's planner binds them, for scattered and for consecutive block
    ids, both directions.  The one-copy-per-row submission the reference
    uses is timed beside it."""
    torch.cuda.empty_cache()  # fresh allocations, not blocks cached by earlier modes
    T, CS, BS, NB, W = 4096, 256, 128, 2048, 1024
    pb = [W * ES, W * ES]
    pool = torch.empty(T * sum(pb), dtype=torch.uint8, pin_memory=True)
    caches = [torch.empty(NB * BS * b, dtype=torch.uint8, device=dev) for b in pb]
    nch = T // CS
    gen = torch.Generator().manual_seed(17)
    out = {}
    for layout in ("scattered", "consecutive"):
        blocks = (torch.randperm(NB, generator=gen)[:T // BS] if layout == "scattered"
                  else torch.arange(64, 64 + T // BS)).tolist()
        for d2h in (False, True):
            rows = _planner_rows(pool.data_ptr(), CS, nch, [c.data_ptr() for c in caches], pb, blocks, BS, d2h)
            nbytes = sum(r[2] for r in rows)
            ours = lambda: ops.layerwise_prefill_dma_copy(rows, d2h)
            per_row = lambda: ops.layerwise_prefill_dma_copy_diagnose(rows, d2h)
            ours(); per_row()
            t_o = statistics.median(time_events(torch, stream, ours, 20)[0] for _ in range(3))
            t_p = time_events(torch, stream, per_row, 10)[0]
            name = f"layerwise_dma_{'store' if d2h else 'load'}_{layout}_llama_layer"
            out[name] = {"ms": round(t_o, 4), "rows": len(rows), "payload_GBps": round(nbytes / t_o / 1e6, 2),
                         "pcie_frac": round(nbytes / t_o / 1e6 / PCIE_PEAK_GBS, 4),
                         "per_row_copies_GBps": round(nbytes / t_p / 1e6, 2)}
    torch.cuda.synchronize()
    del pool, caches
    return out


def bench_c8_graph(torch, ops, dev, stream):
    """DeepSeek-V3.2-shape sparse-attention side paths.  Indexer C8: 8
    layers of int8 keys [2048 blocks, 128, 1, 128] with float16 scales,
    16384 prefill tokens in 16 packets of 1024 per layer at block-scattered
    slots, packed into device packets (HBM) and into pinned packets (PCIe),
    and unpacked back.  Sparse graph copy: 64 requests x 2048 selected tokens
    of an MLA layer (512 + 64 bf16) from device chunk sources of 256
    tokens into distinct cache slots (HBM)."""
    torch.cuda.empty_cache()  # fresh allocations, not blocks cached by earlier modes
    L, NB, T, CC = 8, 2048, 16384, 1024
    gen = torch.Generator().manual_seed(23)
    keys = [torch.randint(-128, 127, (NB, 128, 1, 128), dtype=torch.int8, generator=gen).to(dev) for _ in range(L)]
    scales = [torch.randn((NB, 128, 1, 1), generator=gen).to(torch.float16).to(dev) for _ in range(L)]
    state = ops.IndexerC8GroupState([ops.IndexerC8State(k, s) for k, s in zip(keys, scales)])
    blocks = torch.randperm(NB, generator=gen)[:T // 128]
    slots = (blocks[:, None] * 128 + torch.arange(128)).reshape(-1).to(dev)
    nch = T // CC
    offs = torch.arange(0, T, CC, dtype=torch.int32, device=dev)
    cnts = torch.full((nch,), CC, dtype=torch.int32, device=dev)
    nbytes = L * T * 130
    out = {}
    for where in ("device", "pinned"):
        if where == "device":
            pk = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        else:
            pk = torch.empty(nbytes, dtype=torch.uint8, pin_memory=True)
        base = pk.data_ptr() if where == "device" else ops.get_device_ptr(pk.data_ptr(), nbytes)
        if base == 0:
            raise RuntimeError("pinned packet buffer is not device-mapped")
        ptrs = torch.tensor([[base + (l * T + c * CC) * 130 for c in range(nch)] for l in range(L)],
                            dtype=torch.int64, device=dev)
        pack = lambda: ops.indexer_c8_group_transfer_prepared(state, ptrs, offs, cnts, slots, CC, True)
        unpack = lambda: ops.indexer_c8_group_transfer_prepared(state, ptrs, offs, cnts, slots, CC, False)
        pack(); unpack()
        t_p = time_events(torch, stream, pack, 20)[0]
        t_u = time_events(torch, stream, unpack, 20)[0]
        for name, t in (("pack", t_p), ("unpack", t_u)):
            e = {"ms": round(t, 4), "payload_GBps": round(nbytes / t / 1e6, 2)}
            if where == "device":
                e["hbm_frac"] = round(2 * nbytes / t / 1e6 / HBM_PEAK_GBS, 4)
            else:
                e["pcie_frac"] = round(nbytes / t / 1e6 / PCIE_PEAK_GBS, 4)
            out[f"indexer_c8_{name}_{where}_8x16k"] = e
        del pk
    # sparse graph copy
    R, Wsel, CS, KH, PH = 64, 2048, 256, 512, 64
    MB, BSZ = 4096, 64
    k = torch.zeros((MB, BSZ, 1, KH), dtype=torch.bfloat16, device=dev)
    pe = torch.zeros((MB, BSZ, 1, PH), dtype=torch.bfloat16, device=dev)
    limit = 8192
    cpr = limit // CS
    src_k = torch.randn((R * cpr, CS, KH), generator=gen).to(torch.bfloat16).to(dev)
    src_p = torch.randn((R * cpr, CS, PH), generator=gen).to(torch.bfloat16).to(dev)
    ptrs = torch.stack([src_k.data_ptr() + torch.arange(R * cpr, dtype=torch.int64) * CS * KH * ES,
                        src_p.data_ptr() + torch.arange(R * cpr, dtype=torch.int64) * CS * PH * ES]).to(dev)
    sel = torch.stack([torch.randperm(limit, generator=gen)[:Wsel] for _ in range(R)]).to(torch.int32).to(dev)
    gslots = torch.randperm(MB * BSZ, generator=gen)[:R * Wsel].reshape(R, Wsel).to(dev)
    counts = torch.full((R,), Wsel, dtype=torch.int32, device=dev)
    limits = torch.full((R,), limit, dtype=torch.int32, device=dev)
    st = ops.prepare_sparse_direct_destination_state((k, pe), torch.zeros(1, device=dev), 5, 0, 0, 0)
    graph = lambda: ops.sparse_graph_kv_transfer(st, gslots, sel, counts, ptrs, limits, CS)
    graph()
    t_g = time_events(torch, stream, graph, 20)[0]
    gbytes = R * Wsel * (KH + PH) * ES
    out["sparse_graph_copy_mla_64x2048"] = {"ms": round(t_g, 4), "payload_GBps": round(gbytes / t_g / 1e6, 1),
                                            "hbm_frac": round(2 * gbytes / t_g / 1e6 / HBM_PEAK_GBS, 4)}
    # the same selections from chunk sources in pinned host memory (PCIe)
    hk = src_k.cpu().pin_memory()
    hp = src_p.cpu().pin_memory()
    hkd, hpd = ops.get_device_ptr(hk.data_ptr(), hk.numel() * ES), ops.get_device_ptr(hp.data_ptr(), hp.numel() * ES)
    if hkd == 0 or hpd == 0:
        raise RuntimeError("pinned chunk sources are not device-mapped")
    hptrs = torch.stack([hkd + torch.arange(R * cpr, dtype=torch.int64) * CS * KH * ES,
                         hpd + torch.arange(R * cpr, dtype=torch.int64) * CS * PH * ES]).to(dev)
    hgraph = lambda: ops.sparse_graph_kv_transfer(st, gslots, sel, counts, hptrs, limits, CS)
    hgraph()
    t_h = time_events(torch, stream, hgraph, 10)[0]
    out["sparse_graph_copy_mla_64x2048_pinned_sources"] = {
        "ms": round(t_h, 4), "payload_GBps": round(gbytes / t_h / 1e6, 2),
        "pcie_frac": round(gbytes / t_h / 1e6 / PCIE_PEAK_GBS, 4)}
    torch.cuda.synchronize()
    del keys, scales, state, k, pe, src_k, src_p, hk, hp
    torch.cuda.empty_cache()
    return out


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--modes", default="d2d,per_chunk,flash,call_overhead,contiguous,pinned,staged,memcpy,blend,cachegen,rope,qwen32b,mla576,direct,dma,c8graph",
                    help="comma list; the timed D2D step always runs")
    args = ap.parse_args(argv)
    sel = set(args.modes.split(","))
    if args.gpus != 1:
        print("bench.py measures one GPU: this library has no multi-GPU path "
              "(the KV gather/scatter shards per rank with no exchange step).", file=sys.stderr)
        return 2

    import torch

    import lmcache_amd

    ops = lmcache_amd.c_ops
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream(dev)

    flat, ptrs, slots, starts, chunks, n_tok = build_workload(torch, ops, dev)
    pbs = NB * BS
    payload = 2 * L * n_tok * W * ES           # bytes per direction

    def store():
        ops.multi_layer_kv_transfer_batched(chunks, ptrs, slots, starts, dev, pbs, True, False, 2, W, W, 0)

    def retrieve():
        ops.multi_layer_kv_transfer_batched(chunks, ptrs, slots, starts, dev, pbs, False, False, 2, W, W, 0)

    for _ in range(args.warmup):
        store()
        retrieve()
    torch.cuda.synchronize()

    # Timed region: exactly `steps` store+retrieve steps between two HIP
    # events on the launch stream; the only kernels in it are the 2 * steps
    # gather/scatter launches, so the event time over 2 * steps is the
    # kernel's average launch duration (inter-launch gaps included).
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(args.steps):
        store()
        retrieve()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = e0.elapsed_time(e1)
    step_ms = wall * 1e3 / args.steps
    value = 2 * payload * args.steps / wall / 1e9
    kern_avg_ms = gpu_ms / (2 * args.steps)
    achieved = 2 * payload / (kern_avg_ms * 1e-3) / 1e9   # HBM bytes (read + write) per launch
    roofline = {
        "bound": "hbm",
        "achieved": round(achieved, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4),
        "traffic": load_traffic(),
    }
    # Per-direction split (outside the timed region).
    store_ms = time_events(torch, stream, store, 10)[2]
    retr_ms = time_events(torch, stream, retrieve, 10)[2]

    extra = {}
    extra_cg, extra_rope, extra_calls = {}, {}, {}
    if "per_chunk" in sel:
        # Per-chunk drop-in call path (one multi_layer_kv_transfer per chunk).
        def store_per_chunk():
            for x, s in zip(chunks, starts):
                ops.multi_layer_kv_transfer(x, ptrs, slots[s: s + x.shape[2]], dev, pbs, True, False, 2, W, W, 0)

        def retrieve_per_chunk():
            for x, s in zip(chunks, starts):
                ops.multi_layer_kv_transfer(x, ptrs, slots[s: s + x.shape[2]], dev, pbs, False, False, 2, W, W, 0)

        extra["d2d_per_chunk_calls_store"] = time_events(torch, stream, store_per_chunk, 10)[0]
        extra["d2d_per_chunk_calls_retrieve"] = time_events(torch, stream, retrieve_per_chunk, 10)[0]

        # Floors for one launch per memory object: the same 16 calls with the
        # identity slots 0..4095 (each call then copies contiguous rows), and
        # the runtime's own device copy of the same 32 MiB per call.
        lin = torch.arange(n_tok, dtype=torch.int64, device=dev)

        def identity_per_chunk(direction):
            for x, s in zip(chunks, starts):
                ops.multi_layer_kv_transfer(x, ptrs, lin[s: s + x.shape[2]], dev, pbs, direction, False, 2, W, W, 0)

        identity_per_chunk(True)
        extra["d2d_per_chunk_identity_slots_store"] = time_events(
            torch, stream, lambda: identity_per_chunk(True), 10)[0]
        extra["d2d_per_chunk_identity_slots_retrieve"] = time_events(
            torch, stream, lambda: identity_per_chunk(False), 10)[0]
        flat_src = torch.empty(2 * L * CHUNK * W * ES * len(chunks), dtype=torch.uint8, device=dev)
        flat_dst = torch.empty_like(flat_src)
        cb = 2 * L * CHUNK * W * ES

        def memcpy_per_chunk():
            for i in range(len(chunks)):
                flat_dst[i * cb:(i + 1) * cb].copy_(flat_src[i * cb:(i + 1) * cb])

        memcpy_per_chunk()
        extra["hipmemcpy_d2d_per_chunk_32MiB"] = time_events(torch, stream, memcpy_per_chunk, 10)[0]
        del flat_src, flat_dst

        # The same 16 calls captured once in a HIP graph and replayed: no host
        # work per call.
        graphs = {}
        for name, fn in (("store", store_per_chunk), ("retrieve", retrieve_per_chunk)):
            side = torch.cuda.Stream(dev)
            side.wait_stream(stream)
            with torch.cuda.stream(side):
                fn()
            stream.wait_stream(side)
            torch.cuda.synchronize()
            graphs[name] = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graphs[name]):
                fn()
            torch.cuda.synchronize()
        extra["d2d_per_chunk_graph_store"] = time_events(torch, stream, graphs["store"].replay, 10)[0]
        extra["d2d_per_chunk_graph_retrieve"] = time_events(torch, stream, graphs["retrieve"].replay, 10)[0]

    if "flash" in sel:
        # load_and_reshape_flash / reshape_and_cache_back_flash: one call per
        # layer over the 4096 tokens of a [2, L, T, W] buffer, as the
        # layer-by-layer connector calls them.
        kvbuf = torch.empty((2, L, n_tok, W), dtype=torch.bfloat16, device=dev)

        def flash_store():
            for l in range(L):
                ops.load_and_reshape_flash(kvbuf, flat[2 * l], flat[2 * l + 1], slots, l)

        def flash_retrieve():
            for l in range(L):
                ops.reshape_and_cache_back_flash(kvbuf, flat[2 * l], flat[2 * l + 1], slots, l)

        flash_store()
        flash_retrieve()
        extra["d2d_flash_per_layer_calls_store"] = time_events(torch, stream, flash_store, 10)[0]
        extra["d2d_flash_per_layer_calls_retrieve"] = time_events(torch, stream, flash_retrieve, 10)[0]
        # Floors for one launch per layer: the same 32 calls with the identity
        # slots (contiguous rows), and the runtime's device copy of the same
        # 16 MiB per call.
        lin_f = torch.arange(n_tok, dtype=torch.int64, device=dev)

        def flash_identity():
            for l in range(L):
                ops.load_and_reshape_flash(kvbuf, flat[2 * l], flat[2 * l + 1], lin_f, l)

        flash_identity()
        extra["d2d_flash_per_layer_identity_slots_store"] = time_events(torch, stream, flash_identity, 10)[0]
        lb = 2 * n_tok * W * ES
        f_src = torch.empty(L * lb, dtype=torch.uint8, device=dev)
        f_dst = torch.empty_like(f_src)

        def memcpy_per_layer():
            for l in range(L):
                f_dst[l * lb:(l + 1) * lb].copy_(f_src[l * lb:(l + 1) * lb])

        memcpy_per_layer()
        extra["hipmemcpy_d2d_per_layer_16MiB"] = time_events(torch, stream, memcpy_per_layer, 10)[0]
        del kvbuf, f_src, f_dst

    if "call_overhead" in sel:
        # Host time per drop-in call on a 1-token transfer, through the C++
        # binding and through ctypes (wall clock per call, stream not drained).
        one = slots[:1]
        tiny = torch.empty((2, L, 1, W), dtype=torch.bfloat16, device=dev)
        paths = {"binding": ops.multi_layer_kv_transfer, "ctypes": ops._multi_layer_kv_transfer_ctypes}
        for name, fn in paths.items():
            if name == "binding" and getattr(ops, "_ext", None) is None:
                continue
            for _ in range(50):
                fn(tiny, ptrs, one, dev, pbs, True, False, 2, W, W, 0)
            torch.cuda.synchronize()
            n_calls = 2000
            t0 = time.perf_counter()
            for _ in range(n_calls):
                fn(tiny, ptrs, one, dev, pbs, True, False, 2, W, W, 0)
            host_us = (time.perf_counter() - t0) / n_calls * 1e6
            torch.cuda.synchronize()
            extra_calls[f"host_us_per_call_{name}"] = round(host_us, 2)

    if "pinned" in sel or "staged" in sel:
        # Memory objects in page-locked host memory.
        host_chunks = [torch.empty(x.shape, dtype=x.dtype).pin_memory() for x in chunks]

    if "pinned" in sel:
        # Zero copy: the kernel reads/writes host memory over PCIe.
        def store_host():
            ops.multi_layer_kv_transfer_batched(host_chunks, ptrs, slots, starts, dev, pbs, True, False, 2, W, W, 0)

        def retrieve_host():
            ops.multi_layer_kv_transfer_batched(host_chunks, ptrs, slots, starts, dev, pbs, False, False, 2, W, W, 0)

        store_host()
        retrieve_host()
        torch.cuda.synchronize()
        extra["pinned_zero_copy_store"] = time_events(torch, stream, store_host, 5)[0]
        extra["pinned_zero_copy_retrieve"] = time_events(torch, stream, retrieve_host, 5)[0]

    if "staged" in sel:
        # The reference's fused path: HBM staging buffer + one DMA per chunk.
        staging = torch.empty((2, L, CHUNK, W), dtype=torch.bfloat16, device=dev)

        def store_fused():
            for x, s in zip(host_chunks, starts):
                ops.fused_multi_layer_kv_transfer(x, staging[:, :, : x.shape[2]], ptrs, slots[s: s + x.shape[2]],
                                                  dev, pbs, True, False, 2, W, W, 0)

        def retrieve_fused():
            for x, s in zip(host_chunks, starts):
                ops.fused_multi_layer_kv_transfer(x, staging[:, :, : x.shape[2]], ptrs, slots[s: s + x.shape[2]],
                                                  dev, pbs, False, False, 2, W, W, 0)

        extra["pinned_staged_store"] = time_events(torch, stream, store_fused, 5)[0]
        extra["pinned_staged_retrieve"] = time_events(torch, stream, retrieve_fused, 5)[0]

    if "contiguous" in sel:
        # The same kernel and bytes with slots 0..4095 (consecutive blocks):
        # a contiguous copy, the ceiling the scattered-slot case is judged by.
        lin = torch.arange(n_tok, dtype=torch.int64, device=dev)
        c_store = lambda: ops.multi_layer_kv_transfer_batched(chunks, ptrs, lin, starts, dev, pbs, True, False, 2,
                                                               W, W, 0)
        c_retr = lambda: ops.multi_layer_kv_transfer_batched(chunks, ptrs, lin, starts, dev, pbs, False, False, 2,
                                                              W, W, 0)
        c_store(); c_retr()
        extra["d2d_contiguous_slots_store"] = time_events(torch, stream, c_store, 10)[0]
        extra["d2d_contiguous_slots_retrieve"] = time_events(torch, stream, c_retr, 10)[0]

    if "memcpy" in sel:
        # Reference copies: hipMemcpy D2D of the same byte count, pinned H2D/D2H.
        big_a = torch.empty(payload, dtype=torch.uint8, device=dev)
        big_b = torch.empty_like(big_a)
        host_big = torch.empty(payload, dtype=torch.uint8).pin_memory()
        extra["hipmemcpy_d2d_same_bytes"] = time_events(torch, stream, lambda: big_b.copy_(big_a), 10)[0]
        extra["hipmemcpy_h2d_pinned"] = time_events(
            torch, stream, lambda: big_a.copy_(host_big, non_blocking=True), 5)[0]
        extra["hipmemcpy_d2h_pinned"] = time_events(
            torch, stream, lambda: host_big.copy_(big_a, non_blocking=True), 5)[0]

    if "blend" in sel:
        extra_calls.update(bench_blend(torch, ops, dev, stream, flat, slots))
    if "cachegen" in sel:
        extra_cg = bench_cachegen(torch, ops, dev, stream)
    if "rope" in sel:
        extra_rope = bench_rope(torch, ops, dev, stream)

    extra_big = {}
    if "qwen32b" in sel or "mla576" in sel:
        # Free the Llama-shape pool before the larger configurations.
        del flat, chunks
        if "pinned" in sel or "staged" in sel:
            del host_chunks
        torch.cuda.empty_cache()
    if "qwen32b" in sel:
        extra_big.update(bench_qwen32b_long_prefix(torch, ops, dev, stream))
    if "mla576" in sel:
        extra_big.update(bench_mla_576(torch, ops, dev, stream))
    if "direct" in sel:
        extra_big.update(bench_direct(torch, ops, dev, stream))
    if "dma" in sel:
        extra_big.update(bench_layerwise_dma(torch, ops, dev, stream))
    if "c8graph" in sel:
        extra_big.update(bench_c8_graph(torch, ops, dev, stream))

    def gbs(nbytes, ms):
        return round(nbytes / (ms * 1e-3) / 1e9, 2)

    med_s, med_r = statistics.median(store_ms), statistics.median(retr_ms)
    modes = {
        "d2d_store": {"ms": round(med_s, 4), "payload_GBps": gbs(payload, med_s), "hbm_GBps": gbs(2 * payload, med_s)},
        "d2d_retrieve": {"ms": round(med_r, 4), "payload_GBps": gbs(payload, med_r),
                         "hbm_GBps": gbs(2 * payload, med_r)},
        "tokens_per_s_store_retrieve": round(2 * n_tok * args.steps / wall),
    }
    for name, ms in extra.items():
        entry = {"ms": round(ms, 4)}
        if name.startswith("hipmemcpy_d2d"):
            entry["hbm_GBps"] = gbs(2 * payload, ms)
        elif name.startswith("d2d_"):
            entry["payload_GBps"] = gbs(payload, ms)
            entry["hbm_GBps"] = gbs(2 * payload, ms)
        else:
            entry["payload_GBps"] = gbs(payload, ms)
        if name.startswith("pinned") or name in ("hipmemcpy_h2d_pinned", "hipmemcpy_d2h_pinned"):
            entry["pcie_frac"] = round(payload / (ms * 1e-3) / 1e9 / PCIE_PEAK_GBS, 4)
        modes[name] = entry
    modes.update(extra_cg)
    modes.update(extra_rope)
    modes.update(extra_big)
    modes.update(extra_calls)

    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) paged caches)",
        "config": {
            "workload": "llama3-8b-shape KV store+retrieve, device to device: 32 layers x 8 heads x 128 bf16, "
                        "block 128, 2048 blocks/layer/plane SEPARATE_KV, 4 requests [1000,1100,996,1000] = "
                        "4096 tokens in 16 memory objects [2,32,256,1024]",
            "payload_bytes_per_direction": payload,
            "kernel": "kv_rows_copy (one launch per direction)",
        },
        "roofline": roofline,
        "modes": modes,
    }
    if not args.skip_cpu:
        out["cpu_baseline"] = cpu_baseline(torch, args.cpu_seconds)
    print(json.dumps(out))
    return 0


if __name__ == "__main__":
    sys.exit(main())
