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


def cpu_baseline(budget_s=10.0):
    """The oracle's numpy gather/scatter (one thread) on a bounded sample of
    the same workload: the same 16 chunks x 32 layers x 2 planes x 2 KiB
    rows, against a 64-block-per-layer host pool (the full 32 GiB pool does
    not fit the host budget; the pool size does not change the per-row work).
    """
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
    passes = 0
    while True:
        for i, buf in enumerate(lmc):
            s = slots[i * CHUNK:(i + 1) * CHUNK]
            ok.multi_layer_kv_transfer(buf, table, s, pbs, True, False, 2, L, W, ES)
            ok.multi_layer_kv_transfer(buf, table, s, pbs, False, False, 2, L, W, ES)
            payload += 2 * (2 * L * len(s) * W * ES)
        passes += 1
        if time.perf_counter() - t0 >= budget_s:
            break
    dt = time.perf_counter() - t0
    return {
        "value": round(payload / dt / 1e9, 3),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": f"{passes} x (store+retrieve of 16 chunks [2,32,256,1024] bf16, SEPARATE_KV) "
                  f"against a {nb_cpu}-block/layer host pool; numpy oracle, 1 thread, {dt:.1f} s",
    }


def load_traffic():
    """HBM traffic per launch from the committed rocprofv3 --pmc summary."""
    path = os.path.join(REPO, "profiles", "kv_rows_copy_llama8b_4096tok_traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get("traffic_bytes_per_launch")


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--modes", default="d2d,per_chunk,pinned,staged,memcpy",
                    help="comma list; the timed D2D step always runs")
    args = ap.parse_args(argv)
    sel = set(args.modes.split(","))
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
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

    # Timed region: exactly `steps` store+retrieve steps, with HIP events
    # around every launch on the launch stream.
    ev = []
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        a, b, c = (torch.cuda.Event(enable_timing=True) for _ in range(3))
        a.record(stream)
        store()
        b.record(stream)
        retrieve()
        c.record(stream)
        ev.append((a, b, c))
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    store_ms = [a.elapsed_time(b) for a, b, _ in ev]
    retr_ms = [b.elapsed_time(c) for _, b, c in ev]
    step_ms = wall * 1e3 / args.steps
    value = 2 * payload * args.steps / wall / 1e9

    kern_avg_ms = (statistics.mean(store_ms) + statistics.mean(retr_ms)) / 2
    achieved = 2 * payload / (kern_avg_ms * 1e-3) / 1e9   # HBM bytes (read + write) per launch
    roofline = {
        "bound": "hbm",
        "achieved": round(achieved, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4),
        "traffic": load_traffic(),
    }

    extra = {}
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
        else:
            entry["payload_GBps"] = gbs(payload, ms)
        if name.startswith("pinned") or name in ("hipmemcpy_h2d_pinned", "hipmemcpy_d2h_pinned"):
            entry["pcie_frac"] = round(payload / (ms * 1e-3) / 1e9 / PCIE_PEAK_GBS, 4)
        modes[name] = entry

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
        out["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(out))
    return 0


if __name__ == "__main__":
    sys.exit(main())
