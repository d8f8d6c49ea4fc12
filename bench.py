#!/usr/bin/env python3
"""Benchmark of the QStore int8 hot path on one MI355X.

Headline: the dense decoder linear stack -- 28 layers of
Qwen2.5-1.5B-shaped int8 qrow linears (q 1536x1536, k/v 256x1536, o 1536x1536,
gate/up 8960x1536, down 1536x8960), bf16 activations N(0,1), weights U{-127..127} with
scales U(0.5,1.5)/127, fully resident in HBM.  One step = one decode pass over the 28
layers (per layer: fused q/k/v launch, o, paired gate/up + SwiGLU, down), captured in a
HIP graph; the timed region replays it K times.

``value`` = algorithmic bytes of one pass (weights + scales + per-linear activation
in/out, 1,315,084,288 B at M=1) / measured time per pass, in GB/s.  ``roofline`` is the
dominant kernel (the paired gate/up + SwiGLU launch) timed on its own stream with HIP
events; ``cpu_baseline`` is the reference CPU path (oracle/cpu_path.py) on a bounded
sample of the same stack on this host's cores.  ``secondary`` holds the same stack at
config 2's other batch sizes (M = 4, 16, 32) and configs 1, 3, 4 and 5, never ``value``.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--m 1] [--no-cpu] [--no-secondary]
       python bench.py --profile {swiglu,stack,copy}   (eager launches for counter runs)
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, 8 TB/s
HIDDEN, HEADS_KV, HEAD_DIM, INTER, LAYERS = 1536, 2, 128, 8960, 28
KV = HEADS_KV * HEAD_DIM
SHAPES = {  # name -> (out, in)
    "q": (HIDDEN, HIDDEN),
    "k": (KV, HIDDEN),
    "v": (KV, HIDDEN),
    "o": (HIDDEN, HIDDEN),
    "gate": (INTER, HIDDEN),
    "up": (INTER, HIDDEN),
    "down": (HIDDEN, INTER),
}


def algorithmic_bytes_per_pass(m: int) -> int:
    """Weights + scales + bf16 activation in/out per linear, 28 layers."""
    per_layer = 0
    for out, inn in SHAPES.values():
        per_layer += out * inn + out * 4 + 2 * m * (inn + out)
    return per_layer * LAYERS


def swiglu_launch_bytes(m: int) -> int:
    return 2 * (INTER * HIDDEN + INTER * 4) + 2 * m * HIDDEN + 2 * m * INTER


def build_stack(torch, dev, seed: int = 0):
    """All 28 layers' qrow pages in one HBM arena (256 B aligned blocks)."""
    from mrun_pub_amd.qrow import CompactQRowPage

    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    layout, off = [], 0
    for layer in range(LAYERS):
        for name, (out, inn) in SHAPES.items():
            c_off = off
            off = (off + out * inn + 255) // 256 * 256
            s_off = off
            off = (off + out * 4 + 255) // 256 * 256
            layout.append((layer, name, out, inn, c_off, s_off))
    arena = torch.empty(off, dtype=torch.uint8, device=dev)
    pages = [dict() for _ in range(LAYERS)]
    for layer, name, out, inn, c_off, s_off in layout:
        codes = arena[c_off : c_off + out * inn].view(torch.int8).view(out, inn)
        codes.copy_(torch.randint(-127, 128, (out, inn), dtype=torch.int8, device=dev, generator=gen))
        scales = arena[s_off : s_off + out * 4].view(torch.float32)
        scales.copy_((torch.rand(out, device=dev, generator=gen) + 0.5) / 127.0)
        pages[layer][name] = CompactQRowPage(f"L{layer}.{name}", 0, out, inn, codes, scales)
    return arena, pages


def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform

    return platform.processor() or "unknown"


def _timed_loop(fn, seconds: float, min_calls: int = 1) -> tuple[int, float]:
    done, t0 = 0, time.perf_counter()
    while True:
        fn()
        done += 1
        dt = time.perf_counter() - t0
        if dt >= seconds and done >= min_calls:
            return done, dt


def cpu_baseline(seconds: float = 6.0, m: int = 1, threads: int | None = None) -> dict:
    """Reference CPU path (QStore.matmul, bf16 compute) over a bounded sample of the config-2
    stack: whole decoder layers, every linear dequantised then multiplied."""
    import numpy as np
    import torch

    from oracle import cpu_path

    prev = torch.get_num_threads()
    torch.set_num_threads(threads or os.cpu_count() or prev)
    try:
        rng = np.random.default_rng(0)
        layer = [
            (rng.integers(-127, 128, size=s, dtype=np.int8), (rng.uniform(0.5, 1.5, size=s[0]) / 127).astype(np.float32))
            for s in SHAPES.values()
        ]
        xs = {inn: torch.randn(m, inn).to(torch.bfloat16) for _, inn in SHAPES.values()}
        layer_bytes = algorithmic_bytes_per_pass(m) // LAYERS

        def one_layer():
            for q, sc in layer:
                cpu_path.qstore_matmul(q, sc, xs[q.shape[1]])

        done, dt = _timed_loop(one_layer, seconds)
        return {
            "value": round(done * layer_bytes / dt / 1e9, 3),
            "unit": "GB/s",
            "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"{done} decoder layers (7 qrow linears each, M={m}, bf16 compute) of the config-2 stack "
            f"through the reference CPU path restated in oracle/cpu_path.py, {dt:.1f} s",
        }
    finally:
        torch.set_num_threads(prev)


def cpu_baselines_per_config(seconds: float = 2.0) -> dict:
    """The reference's CPU paths for configs 1, 3, 4 and 5 (oracle/cpu_path.py) on bounded
    samples, at all torch threads and at one thread, in the metric's unit."""
    import numpy as np
    import torch

    from oracle import cpu_path

    rng = np.random.default_rng(7)
    all_threads = os.cpu_count() or torch.get_num_threads()
    out: dict = {"cpu_model": _cpu_model(), "threads_all": all_threads}

    def both(name, fn, unit_per_call, unit, sample):
        res = {"unit": unit, "sample": sample}
        for tag, th in (("all_threads", all_threads), ("one_thread", 1)):
            torch.set_num_threads(th)
            try:
                done, dt = _timed_loop(fn, seconds)
            finally:
                torch.set_num_threads(all_threads)
            res[tag] = round(done * unit_per_call / dt, 3)
        out[name] = res

    # config 1: fp32 GEMV [1,1024] x [4096,1024]
    q1 = rng.integers(-127, 128, size=(4096, 1024), dtype=np.int8)
    s1 = (rng.uniform(0.5, 1.5, 4096) / 127).astype(np.float32)
    x1 = torch.randn(1, 1024)
    both("config1_fp32_gemv", lambda: cpu_path.qstore_matmul(q1, s1, x1, torch.float32), 4231168 / 1e9, "GB/s",
         "QStore.matmul fp32 (dequant + GEMV) of the config-1 block")
    # config 3: W8A8 over one GPU share of the weight rows (1792 of 14336), M = 512
    N3, K3 = 1792, 4096
    qw = torch.from_numpy(rng.integers(-127, 128, size=(N3, K3), dtype=np.int8))
    sw = torch.from_numpy((rng.uniform(0.5, 1.5, N3) / 127).astype(np.float32))
    x3 = torch.randn(512, K3)
    x3[:, :4] *= 20
    both("config3_w8a8_m512", lambda: cpu_path.w8a8_matmul(qw, sw, x3, protect_k=8), 2 * 512 * N3 * K3 / 1e12,
         "TOPS", "w8a8_matmul CPU path (fp32 side path top-8, torch._int_mm) on M=512 x 1792 of the 14336 weight "
         "rows (one eighth of config 3's N)")
    # config 4: routed MoE, H 2048, I 768, T = 64, top-8 over 128 experts; sample = 8 experts
    E, k, H, I, T = 128, 8, 2048, 768, 64
    ex = list(range(8))
    gu_q = rng.integers(-127, 128, size=(8, 2 * I, H), dtype=np.int8)
    gu_s = (rng.uniform(0.5, 1.5, size=(8, 2 * I)) / 127).astype(np.float32)
    dn_q = rng.integers(-127, 128, size=(8, H, I), dtype=np.int8)
    dn_s = (rng.uniform(0.5, 1.5, size=(8, H)) / 127).astype(np.float32)
    logits = torch.randn(T, E)
    w4, i4 = torch.softmax(logits, -1).topk(k, -1)
    i4 = i4 % 8  # routes that land in the sampled experts
    w4 = (w4 / w4.sum(-1, keepdim=True)).to(torch.bfloat16)
    src = torch.randn(T, H).to(torch.bfloat16)
    page = 2 * I * H + 2 * I * 4 + H * I + H * 4
    both("config4_moe_t64", lambda: cpu_path.moe_layer(src, i4, w4, gu_q, gu_s, dn_q, dn_s, experts=ex),
         8 * page / 1e9, "GB/s", "streamed_moe_forward expert math (bf16, int8 experts dequantised per active "
         "expert) over 8 of the 128 experts, T=64 routed onto them")
    # config 5: int3 G64 fp16 scale/zero [11008, 4096] M = 1, 2048 of the rows
    N5, K5 = 2048, 4096
    packed = rng.integers(0, 256, size=(N5, K5 * 3 // 8), dtype=np.uint8)
    sc5 = ((rng.uniform(0.5, 1.5, size=(N5, K5 // 64))) / 7).astype(np.float16)
    z5 = (rng.uniform(0, 7, size=(N5, K5 // 64))).astype(np.float16)
    x5 = torch.randn(1, K5)
    b5 = N5 * (K5 * 3 // 8) + 2 * 2 * N5 * (K5 // 64) + 2 * K5 + 4 * N5
    both("config5_int3_m1", lambda: cpu_path.lowbit_matmul(packed, sc5, z5, x5, K5, 3, 64, 0.0), b5 / 1e9, "GB/s",
         "QStoreInt3.matmul CPU path (chunked np.unpackbits dequant + sgemm) on 2048 of the 11008 rows")
    # offline codecs: the numpy writers restated in oracle/ (single-threaded numpy), bytes as
    # in the device codec lines
    from oracle import lowbit as olow
    from oracle import qrow as oq

    Wq = rng.standard_normal((1024, 4096)).astype(np.float32)
    done, dt = _timed_loop(lambda: oq.quant_row_int8(Wq), seconds)
    out["codec_int8"] = {"unit": "GB/s", "sample": "_quant_row_int8 on 1024 x 4096 fp32 rows (numpy)",
                         "one_thread": round(done * (5 * 1024 * 4096 + 4 * 1024) / dt / 1e9, 3)}
    Wl = rng.standard_normal((256, 4096)).astype(np.float32)
    done, dt = _timed_loop(lambda: olow.quant_row_int3(Wl), seconds)
    out["codec_int3"] = {"unit": "GB/s", "sample": "_quant_row_int3 + packing on 256 x 4096 fp32 rows (numpy)",
                         "one_thread": round(done * (4 * 256 * 4096 + 256 * 1536 + 4 * 256 * 32) / dt / 1e9, 3)}
    # whole-weight dequant: the reference's numpy dequant restated in oracle/, fp32 out
    qd = rng.integers(-127, 128, size=(1024, 4096), dtype=np.int8)
    sd = (rng.uniform(0.5, 1.5, 1024) / 127).astype(np.float32)
    done, dt = _timed_loop(lambda: oq.dequant_qrow(qd, sd), seconds)
    out["dequant_qrow_f32"] = {"unit": "GB/s", "sample": "_dequant_qrow of 1024 x 4096 int8 rows to fp32 (numpy)",
                               "one_thread": round(done * (5 * 1024 * 4096 + 4 * 1024) / dt / 1e9, 3)}
    pk = rng.integers(0, 256, size=(256, 1536), dtype=np.uint8)
    s3 = (rng.uniform(0.5, 1.5, size=(256, 64)) / 7).astype(np.float16)
    z3 = rng.uniform(0, 7, size=(256, 64)).astype(np.float16)
    done, dt = _timed_loop(lambda: olow.dequant(pk, s3, 4096, 3, 64, zeros=z3), seconds)
    out["dequant_int3_f32"] = {"unit": "GB/s", "sample": "int3 G64 dequant (np.unpackbits) of 256 x 4096 to fp32 (numpy)",
                               "one_thread": round(done * (256 * 1536 + 4 * 256 * 64 + 4 * 256 * 4096) / dt / 1e9, 3)}
    return out


def _graph_time(torch, stream, fn, calls: int, reps: int = 50, warmup: int = 10) -> float:
    """Median seconds per call of ``fn`` (one launch sequence), captured ``calls`` times in
    a graph; each of ``reps`` replays after untimed ones (``warmup`` at a time, until at
    least 50 ms have run: the first milliseconds of a burst run at a lower clock, e.g.
    38.6 against 35.7 us for config 3's M = 512 GEMM) is timed with its own pair of HIP
    events on ``stream``."""
    with torch.cuda.stream(stream):
        fn(0)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            for i in range(calls):
                fn(i)
        per = _replay_times(torch, stream, g, reps, warmup=warmup, min_warm_s=0.05)
    return _median(per) / calls


def _median(v: list[float]) -> float:
    v = sorted(v)
    n = len(v)
    return v[n // 2] if n % 2 else 0.5 * (v[n // 2 - 1] + v[n // 2])


def _replay_times(torch, stream, graph, reps: int, warmup: int, min_warm_s: float = 0.0) -> list[float]:
    """Seconds of each of ``reps`` replays (after ``warmup`` untimed ones, repeated until
    ``min_warm_s`` seconds have passed), HIP events on the replay stream around every
    replay."""
    t0 = time.perf_counter()
    while True:
        for _ in range(warmup):
            graph.replay()
        torch.cuda.synchronize()
        if time.perf_counter() - t0 >= min_warm_s:
            break
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
    with torch.cuda.stream(stream):
        ev[0].record(stream)
        for r in range(reps):
            graph.replay()
            ev[r + 1].record(stream)
    torch.cuda.synchronize()
    return [ev[r].elapsed_time(ev[r + 1]) * 1e-3 for r in range(reps)]


def paged_measurement(torch, dev, pages, x_h, x_i, passes: int = 6) -> dict:
    """Config 2 as BASELINE words it: the same stack streamed from pinned host memory in
    2 MiB pages through the HBM slot ring (PCIe-inclusive; never the headline value), from
    a pinned tier holding the whole stack and, in bounded mode, through three pinned
    staging buffers refilled from a store file's mapping."""
    from mrun_pub_amd.paged import PAGE_BYTES, TRANSFER_BYTES, PagedQStore, PinnedHostTier

    tier = PinnedHostTier.from_pages({p.name: p for L in pages for p in L.values()})
    torch.cuda.synchronize()
    # raw pinned -> HBM copy rate of the whole tier, for comparison
    dst = torch.empty(tier.nbytes, dtype=torch.uint8, device=dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    dst.copy_(tier.host[: tier.nbytes], non_blocking=True)
    e1.record()
    torch.cuda.synchronize()
    raw_gbs = tier.nbytes / (e0.elapsed_time(e1) * 1e-3) / 1e9
    del dst
    store = PagedQStore(tier, device=dev, compute_dtype="bf16", slots=4, depth=3)

    def timed(store, store_passes):
        def one_pass():
            for L in range(LAYERS):
                for n in ("q", "k", "v"):
                    store.matmul(f"L{L}.{n}", x_h)
                store.matmul(f"L{L}.o", x_h)
                store.fused_swiglu(f"L{L}.gate", f"L{L}.up", x_h)
                store.matmul(f"L{L}.down", x_i)

        one_pass()  # the successor oracle learns the order
        torch.cuda.synchronize()
        h0 = dict(store.ring.stats)
        t0 = time.perf_counter()
        for _ in range(store_passes):
            one_pass()
        torch.cuda.synchronize()
        dt = (time.perf_counter() - t0) / store_passes
        st = store.ring.stats
        moved = (st["h2d_bytes"] - h0["h2d_bytes"]) / store_passes
        return {
            "ms_per_pass": round(dt * 1e3, 3),
            "tokens_per_s": round(x_h.shape[0] / dt, 2),
            "h2d_GB/s": round(moved / dt / 1e9, 2),
            "pages_per_pass": (st["h2d_pages"] - h0["h2d_pages"]) // store_passes,
            "hits": st["hits"] - h0["hits"],
            "misses": st["misses"] - h0["misses"],
            "bytes_per_pass": int(moved),
        }

    res = {"raw_pinned_h2d_GB/s": round(raw_gbs, 2), "page_bytes": PAGE_BYTES, "max_transfer_bytes": TRANSFER_BYTES,
           "slots": 4, "depth": 3}
    res.update(timed(store, passes))
    res["pinned_bytes"] = tier.nbytes
    store.close()
    del store, tier
    # bounded mode: three pinned staging buffers refilled from the store file's mapping
    # (the file written here sits in the page cache, as a store read once does)
    import tempfile

    from mrun_pub_amd.store import write_qstore

    with tempfile.TemporaryDirectory(dir="/tmp") as tmp:
        write_qstore(tmp, {p.name: (p.codes.cpu().numpy(), p.scales.cpu().numpy()) for L in pages for p in L.values()},
                     legacy=True)
        staged = PagedQStore(tmp, device=dev, compute_dtype="bf16", slots=4, depth=3, staging_buffers=3)
        res["bounded_staging"] = {**timed(staged, passes), "staging_buffers": 3, "pinned_bytes": staged.tier.nbytes}
        staged.close()
    return res


def paged_moe_measurement(torch, dev, E: int, topk: int, H: int, I: int, layers: int = 2,
                          steps: int = 4) -> dict:
    """Config 4's expert layers served from the packed expert store through the HBM slot
    cache (``ExpertPageCache``), timed by wall clock around the whole sequence of layer
    calls with one device sync at its end (host bookkeeping and H2D fills are not
    capturable in a graph).  A layer whose pages are not all resident reads its routes
    on the host (one sync in that call); a fully resident layer binds its slots through
    the device slot table without one.

    * ``slots_all``: slots for every page of ``layers`` layers, all preloaded: every layer
      is fully resident, so a call costs the resident kernels plus the slot-table binding.
    * ``slots_one_layer_tier``: slots for one layer only and every page in the pinned host
      tier, so each layer change refills most slots over PCIe (``h2d_GB/s``).
    """
    import tempfile

    import numpy as np
    from mrun_pub_amd import expert_cache, moe

    rng = np.random.default_rng(11)
    gu = rng.integers(-127, 128, size=(layers, E, 2 * I, H), dtype=np.int8)
    gus = (rng.uniform(0.5, 1.5, size=(layers, E, 2 * I)) / 127).astype(np.float32)
    dn = rng.integers(-127, 128, size=(layers, E, H, I), dtype=np.int8)
    dns = (rng.uniform(0.5, 1.5, size=(layers, E, H)) / 127).astype(np.float32)
    gen = torch.Generator(device=dev)
    gen.manual_seed(5)
    res = {}
    with tempfile.TemporaryDirectory(dir="/tmp") as tmp:
        store = expert_cache.PackedInt8ExpertStore(expert_cache.write_int8_expert_store(tmp, gu, gus, dn, dns))
        del gu, gus, dn, dns
        stride = store.layout.page_stride
        total_mb = layers * E * stride / 1e6 + 1
        tier = expert_cache.HostPageTier(store, host_cache_mb=total_mb)
        tier.warm()
        cases = (("slots_all", dict(cache_mb=total_mb, host_tier=None)),
                 ("slots_one_layer_tier", dict(cache_mb=0, host_tier=tier)))
        for T in (64, 512):
            routes = []
            for _ in range(steps + 1):
                for layer in range(layers):
                    w, idx = moe.route_topk(torch.randn(T, E, device=dev, generator=gen), topk)
                    routes.append((layer, torch.randn(T, H, device=dev, generator=gen).to(torch.bfloat16), idx, w))
            for name, kw in cases:
                cache = expert_cache.ExpertPageCache(store, device=dev, max_active_pages=E, **kw)
                if name == "slots_all":
                    cache.preload()  # every page resident: the device slot-table binding
                backend = moe.Int8ExpertBackend(page_cache=cache)
                for r in routes[:layers]:
                    backend.moe(*r)
                torch.cuda.synchronize()
                s0 = cache.stats.as_dict()
                t0 = time.perf_counter()
                for r in routes[layers:]:
                    backend.moe(*r)
                torch.cuda.synchronize()
                dt = time.perf_counter() - t0
                s1 = cache.stats.as_dict()
                n = len(routes) - layers
                h2d = s1["host_to_device_bytes"] - s0["host_to_device_bytes"]
                req = s1["page_requests"] - s0["page_requests"]
                res[f"config4_moe_paged_t{T}_{name}"] = {
                    "ms_per_layer": round(dt / n * 1e3, 3), "slots": cache.capacity,
                    "hit_rate": round((s1["page_hits"] - s0["page_hits"]) / max(1, req), 4),
                    "h2d_MB_per_layer": round(h2d / n / 1e6, 1), "h2d_GB/s": round(h2d / dt / 1e9, 1),
                    "device_table_layers": cache.device_table_stats["device_table_layers"],
                }
                cache.close()
                del backend, cache
        store.release()
    return res


def profile_lowbit(torch, dev, calls: int) -> dict:
    """Eager launches of config 5 (int3 / int2 G64, fp16 scale + zero, both shapes, M = 1
    and 8), ``calls`` per case on weight copies that rotate past the Infinity Cache, for
    kernel traces and counter runs; prints each case's algorithmic bytes."""
    from mrun_pub_amd import lowbit

    gen = torch.Generator(device=dev)
    gen.manual_seed(3)
    out: dict = {"profile": "lowbit", "calls": calls}
    for bits in (3, 2):
        for (N5, K5) in ((11008, 4096), (4096, 11008)):
            rb = K5 * bits // 8
            ng = K5 // 64
            copies = max(2, (512 << 20) // (N5 * rb) + 1)
            packed = torch.randint(0, 256, (copies, N5, rb), dtype=torch.uint8, device=dev, generator=gen)
            sc = ((torch.rand(copies, N5, ng, device=dev, generator=gen) + 0.5) / 7).to(torch.float16)
            zp = (torch.rand(copies, N5, ng, device=dev, generator=gen) * 7).to(torch.float16)
            pages = [lowbit.LowbitPage("w", bits, 64, K5, packed[c], sc[c], zp[c]) for c in range(copies)]
            for M5 in (1, 8):
                x5 = torch.randn(M5, K5, device=dev, generator=gen).to(torch.bfloat16)
                for i in range(calls):
                    lowbit.lowbit_matmul(pages[i % copies], x5)
                out[f"int{bits}_{N5}x{K5}_m{M5}_bytes"] = N5 * rb + 2 * 2 * N5 * ng + 2 * M5 * K5 + 4 * M5 * N5
            del packed, sc, zp, pages
    torch.cuda.synchronize()
    return out


def profile_codecs(torch, dev, calls: int) -> dict:
    """Eager launches of the offline codecs, ``calls`` each: int8 rows of an fp32 [14336,
    4096] weight, int3 and int2 (G 128) of an fp32 [11008, 4096] one; prints each one's
    algorithmic bytes (fp32 input + codes + fp32 scales)."""
    from mrun_pub_amd import codecs

    gen = torch.Generator(device=dev)
    gen.manual_seed(3)
    out: dict = {"profile": "codec", "calls": calls}
    W = torch.randn(14336, 4096, device=dev, generator=gen)
    for _ in range(calls):
        codecs.quant_row_int8(W)
    out["int8_14336x4096_bytes"] = 5 * 14336 * 4096 + 4 * 14336
    del W
    W = torch.randn(11008, 4096, device=dev, generator=gen)
    for bits, fn in ((3, codecs.quant_row_int3), (2, codecs.quant_row_int2)):
        for _ in range(calls):
            fn(W)
        out[f"int{bits}_11008x4096_bytes"] = 4 * 11008 * 4096 + 11008 * 4096 * bits // 8 + 4 * 11008 * 32
    torch.cuda.synchronize()
    return out


def profile_dequant(torch, dev, calls: int) -> dict:
    """Eager launches of the whole-weight dequants, ``calls`` each: int8 rows [14336, 4096]
    to bf16 and fp32, int3 / int2 G64 (fp16 scale + zero) [11008, 4096] to fp32; prints
    each one's algorithmic bytes."""
    from mrun_pub_amd import lowbit, qrow

    gen = torch.Generator(device=dev)
    gen.manual_seed(3)
    out: dict = {"profile": "dequant", "calls": calls}
    cd = torch.randint(-127, 128, (14336, 4096), dtype=torch.int8, device=dev, generator=gen)
    sd = (torch.rand(14336, device=dev, generator=gen) + 0.5) / 127
    for dname, dt, es in (("bf16", torch.bfloat16, 2), ("f32", torch.float32, 4)):
        for _ in range(calls):
            qrow.qrow_dequant(cd, sd, dt)
        out[f"qrow_{dname}_bytes"] = 14336 * 4096 * (1 + es) + 4 * 14336
    del cd, sd
    for bits in (3, 2):
        rb = 4096 * bits // 8
        pk = torch.randint(0, 256, (11008, rb), dtype=torch.uint8, device=dev, generator=gen)
        sc = ((torch.rand(11008, 64, device=dev, generator=gen) + 0.5) / 7).to(torch.float16)
        zp = (torch.rand(11008, 64, device=dev, generator=gen) * 7).to(torch.float16)
        pg = lowbit.LowbitPage("w", bits, 64, 4096, pk, sc, zp)
        for _ in range(calls):
            lowbit.lowbit_dequant(pg)
        out[f"int{bits}_bytes"] = 11008 * rb + 2 * 2 * 11008 * 64 + 4 * 11008 * 4096
    torch.cuda.synchronize()
    return out


def profile_mfma_kernels(torch, dev, which: str, calls: int) -> dict:
    """Eager launches of config 3's fused W8A8 GEMM or config 4's MoE layer, for counter runs
    (MFMA utilisation, HBM bytes); prints the algorithmic figures to compare against."""
    from mrun_pub_amd import _native as nat
    from mrun_pub_amd import moe, w8a8

    gen = torch.Generator(device=dev)
    gen.manual_seed(3)
    out: dict = {"profile": which, "calls": calls}
    if which == "w8a8p":
        # the whole protect_k=8 call: column maxima, selection + quantization + side operands,
        # GEMM with the side path (0.1% outlier channels x20, as config 3)
        N, K = 14336, 4096
        qw = torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev, generator=gen)
        sw = (torch.rand(N, device=dev, generator=gen) + 0.5) / 127
        for M in (512, 2048):
            x = torch.randn(M, K, device=dev, generator=gen)
            x[:, torch.randint(0, K, (4,), device=dev, generator=gen)] *= 20.0
            xb = x.to(torch.bfloat16)
            for _ in range(calls):
                w8a8.w8a8_matmul(qw, sw, xb, protect_k=8, out_dtype=torch.bfloat16)
            out[f"m{M}_ops_per_call"] = 2 * M * N * K
    elif which == "w8a8":
        N, K = 14336, 4096
        qw = torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev, generator=gen)
        sw = (torch.rand(N, device=dev, generator=gen) + 0.5) / 127
        for M in (512, 2048):
            xb = torch.randn(M, K, device=dev, generator=gen).to(torch.bfloat16)
            qx, asc = w8a8.quantize_activation(xb)
            y = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
            for _ in range(calls):
                nat.call("qs_w8a8_gemm", nat.ptr(qx), nat.ptr(asc), nat.ptr(qw), nat.ptr(sw), None, None, 0,
                         nat.ptr(y), nat.QS_BF16, M, N, K, nat.stream_of(dev))
            out[f"m{M}_ops_per_call"] = 2 * M * N * K
    else:
        E, topk, H, I = 128, 8, 2048, 768
        layer = moe.Int8ExpertLayer.from_arrays(
            torch.randint(-127, 128, (E, 2 * I, H), dtype=torch.int8, device=dev, generator=gen),
            (torch.rand(E, 2 * I, device=dev, generator=gen) + 0.5) / 127,
            torch.randint(-127, 128, (E, H, I), dtype=torch.int8, device=dev, generator=gen),
            (torch.rand(E, H, device=dev, generator=gen) + 0.5) / 127, dev)
        backend = moe.Int8ExpertBackend([layer], w8a16=which == "moe16")
        for T in (64, 512):
            tw, ti = moe.route_topk(torch.randn(T, E, device=dev, generator=gen), topk)
            xs = torch.randn(T, H, device=dev, generator=gen).to(torch.bfloat16)
            for _ in range(calls):
                backend.moe(0, xs, ti, tw)
            out[f"t{T}_active_experts"] = int(torch.unique(ti).numel())
            out[f"t{T}_ops_per_layer"] = 2 * T * topk * (2 * I * H + H * I)
    torch.cuda.synchronize()
    return out


def secondary_measurements(torch, dev, stream) -> dict:
    """Configs 1, 3, 4, 5 of BASELINE.json, measured with HIP graphs on one stream."""
    from mrun_pub_amd import lowbit, moe, qrow, w8a8

    gen = torch.Generator(device=dev)
    gen.manual_seed(3)
    res = {}

    # config 1: fp32 decode GEMV [1,1024] x [4096,1024], 128 distinct weight copies (> MALL)
    n, k, copies = 4096, 1024, 128
    codes = torch.randint(-127, 128, (copies, n, k), dtype=torch.int8, device=dev, generator=gen)
    scales = (torch.rand(copies, n, device=dev, generator=gen) + 0.5) / 127
    x = torch.randn(1, k, device=dev, generator=gen)
    t = _graph_time(torch, stream, lambda i: qrow.qrow_matmul(codes[i % copies], scales[i % copies], x), 64)
    b = n * k + n * 4 + 4 * k + 4 * n
    res["config1_fp32_gemv"] = {"us_per_call": round(t * 1e6, 3), "GB/s": round(b / t / 1e9, 1),
                                "hbm_frac": round(b / t / 1e9 / HBM_PEAK_GBS, 4), "bytes": b}
    del codes, scales

    # config 3: W8A8 prefill, W [14336,4096], M in {512, 2048}, 0.1% outlier channels x20
    N, K = 14336, 4096
    qw = torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev, generator=gen)
    sw = (torch.rand(N, device=dev, generator=gen) + 0.5) / 127
    for M in (512, 2048):
        xb = torch.randn(M, K, device=dev, generator=gen)
        xb[:, torch.randperm(K, device=dev, generator=gen)[:4]] *= 20.0
        xb = xb.to(torch.bfloat16)
        qx, asc = w8a8.quantize_activation(xb)
        y = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
        from mrun_pub_amd import _native as nat

        def gemm(_i):
            nat.call("qs_w8a8_gemm", nat.ptr(qx), nat.ptr(asc), nat.ptr(qw), nat.ptr(sw), None, None, 0,
                     nat.ptr(y), nat.QS_BF16, M, N, K, nat.stream_of(dev))

        tg = _graph_time(torch, stream, gemm, 10)
        tf = _graph_time(torch, stream, lambda i: w8a8.w8a8_matmul(qw, sw, xb, protect_k=8, out_dtype=torch.bfloat16), 10)
        # the int32 GEMM alone, and the vendor library's int8 GEMM (torch._int_mm, hipBLASLt)
        # on the same operands: a reference point for the MFMA fraction, not part of the path
        ti = _graph_time(torch, stream, lambda i: w8a8._int8_gemm(qx, qw, True), 10)
        wt = qw.t()
        tv = _graph_time(torch, stream, lambda i: torch._int_mm(qx, wt), 10)
        ops = 2 * M * N * K
        res[f"config3_w8a8_m{M}"] = {
            "gemm_us": round(tg * 1e6, 2), "gemm_TOPS": round(ops / tg / 1e12, 1),
            "mfma_frac": round(ops / tg / 5.0e15, 4),
            "w8a8_matmul_protect8_us": round(tf * 1e6, 2), "end_to_end_TOPS": round(ops / tf / 1e12, 1),
            "int32_gemm_TOPS": round(ops / ti / 1e12, 1),
            "hipblaslt_int_mm_TOPS": round(ops / tv / 1e12, 1),
        }
    del qw, sw

    # decode-step neighbour: fused W8A16 lm_head + top-2 (no logits in memory), the
    # 151,936 x 1536 head of the config-2 model family, one bf16 decode row, 2 copies
    V, Kh, hc = 151936, 1536, 2
    hcodes = torch.randint(-127, 128, (hc, V, Kh), dtype=torch.int8, device=dev, generator=gen)
    hscales = (torch.rand(hc, V, device=dev, generator=gen) + 0.5) / 127
    hx = torch.randn(1, Kh, device=dev, generator=gen).to(torch.bfloat16)
    hpages = [qrow.CompactQRowPage("lm_head", 0, V, Kh, hcodes[i], hscales[i]) for i in range(hc)]
    th = _graph_time(torch, stream, lambda i: qrow.fused_qrow_top2(hpages[i % hc], hx), 8)
    hb = V * Kh + V * 4 + Kh * 2
    res["head_top2_m1"] = {"us": round(th * 1e6, 2), "GB/s": round(hb / th / 1e9, 1),
                           "hbm_frac": round(hb / th / 1e9 / HBM_PEAK_GBS, 4), "bytes": hb}
    del hcodes, hscales, hpages

    # config 4: routed MoE, 128 experts top-8, H 2048, I 768, T in {64, 512}
    E, topk, H, I = 128, 8, 2048, 768
    layer = moe.Int8ExpertLayer.from_arrays(
        torch.randint(-127, 128, (E, 2 * I, H), dtype=torch.int8, device=dev, generator=gen),
        (torch.rand(E, 2 * I, device=dev, generator=gen) + 0.5) / 127,
        torch.randint(-127, 128, (E, H, I), dtype=torch.int8, device=dev, generator=gen),
        (torch.rand(E, H, device=dev, generator=gen) + 0.5) / 127, dev)
    backend = moe.Int8ExpertBackend([layer])
    backend16 = moe.Int8ExpertBackend([layer], w8a16=True)
    page_bytes = layer.layout.gate_up_codes_bytes + layer.layout.gate_up_scales_bytes + \
        layer.layout.down_codes_bytes + layer.layout.down_scales_bytes
    for T in (64, 512):
        logits = torch.randn(T, E, device=dev, generator=gen)
        xs = torch.randn(T, H, device=dev, generator=gen).to(torch.bfloat16)
        tw, ti = moe.route_topk(logits, topk)
        active = int(torch.unique(ti).numel())
        byts = active * page_bytes + T * H * 2 * 2
        ops = 2 * T * topk * (2 * I * H + H * I)
        # W8A8 flow, then the weight-only (W8A16) flow over the same pages and routes
        for key, bk in ((f"config4_moe_t{T}", backend), (f"config4_moe_w8a16_t{T}", backend16)):
            tt = _graph_time(torch, stream, lambda i: bk.moe(0, xs, ti, tw), 10)
            res[key] = {"us": round(tt * 1e6, 2), "GB/s": round(byts / tt / 1e9, 1),
                        "hbm_frac": round(byts / tt / 1e9 / HBM_PEAK_GBS, 4),
                        "TOPS": round(ops / tt / 1e12, 2), "active_experts": active}
    del layer, backend, backend16
    res.update(paged_moe_measurement(torch, dev, E, topk, H, I))

    # config 5: packed int3/int2 GEMV, G=64 fp16 scale+zero, [11008,4096] and [4096,11008]
    for bits in (3, 2):
        for (N5, K5) in ((11008, 4096), (4096, 11008)):
            rb = K5 * bits // 8
            ng = K5 // 64
            copies = max(2, (512 << 20) // (N5 * rb) + 1)
            packed = torch.randint(0, 256, (copies, N5, rb), dtype=torch.uint8, device=dev, generator=gen)
            sc = ((torch.rand(copies, N5, ng, device=dev, generator=gen) + 0.5) / 7).to(torch.float16)
            zp = (torch.rand(copies, N5, ng, device=dev, generator=gen) * 7).to(torch.float16)
            pages = [lowbit.LowbitPage("w", bits, 64, K5, packed[c], sc[c], zp[c]) for c in range(copies)]
            for M5 in (1, 8):
                x5 = torch.randn(M5, K5, device=dev, generator=gen).to(torch.bfloat16)
                t5 = _graph_time(torch, stream, lambda i: lowbit.lowbit_matmul(pages[i % copies], x5), 16)
                b5 = N5 * rb + 2 * 2 * N5 * ng + 2 * M5 * K5 + 4 * M5 * N5
                res[f"config5_int{bits}_{N5}x{K5}_m{M5}"] = {
                    "us": round(t5 * 1e6, 2), "GB/s": round(b5 / t5 / 1e9, 1),
                    "hbm_frac": round(b5 / t5 / 1e9 / HBM_PEAK_GBS, 4)}
            del packed, sc, zp, pages

    # offline codecs (the store writer's row quantizers) on the device: int8 rows of config
    # 3's fp32 weight [14336, 4096], int3 / int2 (G 128, the writers' default) of config 5's
    # [11008, 4096]; bytes = fp32 input + codes + fp32 scales
    from mrun_pub_amd import codecs

    Nc, Kc = 14336, 4096
    Wc = torch.randn(Nc, Kc, device=dev, generator=gen)
    tc = _graph_time(torch, stream, lambda i: codecs.quant_row_int8(Wc), 4)
    bc = 4 * Nc * Kc + Nc * Kc + 4 * Nc
    res["codec_int8_14336x4096"] = {"us": round(tc * 1e6, 2), "GB/s": round(bc / tc / 1e9, 1),
                                    "hbm_frac": round(bc / tc / 1e9 / HBM_PEAK_GBS, 4)}
    del Wc
    Nc, Kc, Gc = 11008, 4096, codecs.GROUP
    Wc = torch.randn(Nc, Kc, device=dev, generator=gen)
    for bits, fn in ((3, codecs.quant_row_int3), (2, codecs.quant_row_int2)):
        tc = _graph_time(torch, stream, lambda i: fn(Wc), 4)
        bc = 4 * Nc * Kc + Nc * ((Kc * bits + 7) // 8) + 4 * Nc * ((Kc + Gc - 1) // Gc)
        res[f"codec_int{bits}_{Nc}x{Kc}"] = {"us": round(tc * 1e6, 2), "GB/s": round(bc / tc / 1e9, 1),
                                             "hbm_frac": round(bc / tc / 1e9 / HBM_PEAK_GBS, 4)}
    del Wc

    # whole-weight dequant (QStore.weight / fp32 of the qrow and low-bit stores): int8 rows
    # of config 3's [14336, 4096] to bf16 and fp32; int3 / int2 G64 (fp16 scale + zero) of
    # config 5's [11008, 4096] to fp32; bytes = codes + scales (+ zeros) + output
    for dname, dt, es in (("bf16", torch.bfloat16, 2), ("f32", torch.float32, 4)):
        Nd, Kd = 14336, 4096
        cd = torch.randint(-127, 128, (Nd, Kd), dtype=torch.int8, device=dev, generator=gen)
        sd = (torch.rand(Nd, device=dev, generator=gen) + 0.5) / 127
        td = _graph_time(torch, stream, lambda i: qrow.qrow_dequant(cd, sd, dt), 4)
        bd = Nd * Kd + 4 * Nd + es * Nd * Kd
        res[f"dequant_qrow_{dname}_{Nd}x{Kd}"] = {"us": round(td * 1e6, 2), "GB/s": round(bd / td / 1e9, 1),
                                                 "hbm_frac": round(bd / td / 1e9 / HBM_PEAK_GBS, 4)}
        del cd, sd
    for bits in (3, 2):
        Nd, Kd = 11008, 4096
        rb = Kd * bits // 8
        pk = torch.randint(0, 256, (Nd, rb), dtype=torch.uint8, device=dev, generator=gen)
        sc = ((torch.rand(Nd, Kd // 64, device=dev, generator=gen) + 0.5) / 7).to(torch.float16)
        zp = (torch.rand(Nd, Kd // 64, device=dev, generator=gen) * 7).to(torch.float16)
        pg = lowbit.LowbitPage("w", bits, 64, Kd, pk, sc, zp)
        td = _graph_time(torch, stream, lambda i: lowbit.lowbit_dequant(pg), 4)
        bd = Nd * rb + 2 * 2 * Nd * (Kd // 64) + 4 * Nd * Kd
        res[f"dequant_int{bits}_{Nd}x{Kd}"] = {"us": round(td * 1e6, 2), "GB/s": round(bd / td / 1e9, 1),
                                               "hbm_frac": round(bd / td / 1e9 / HBM_PEAK_GBS, 4)}
        del pk, sc, zp, pg
    return res


class DecodeChain:
    """One decoder pass as a decoder orders its linears: the layer input feeds the fused
    q/k/v launch, q's output feeds o, o's output feeds the paired gate/up + SwiGLU, whose
    output feeds down, and down's output is the next layer's input.  (Attention, norms and
    residuals sit between these in a real decoder; they are not on this path.)  Every
    launch therefore depends on the one before it, as in a real decode step."""

    def __init__(self, torch, dev, pages, m: int, gen):
        self.pages = pages
        self.m = m
        bf = dict(dtype=torch.bfloat16, device=dev)
        self.x0 = torch.randn(m, HIDDEN, device=dev, generator=gen).to(torch.bfloat16)
        self.q = torch.empty(m, HIDDEN, **bf)
        self.k = torch.empty(m, KV, **bf)
        self.v = torch.empty(m, KV, **bf)
        self.o = torch.empty(m, HIDDEN, **bf)
        self.h = torch.empty(m, INTER, **bf)
        self.d = [torch.empty(m, HIDDEN, **bf) for _ in range(2)]

    def per_linear(self, _i=0):
        from mrun_pub_amd import qrow

        x = self.x0
        for li, L in enumerate(self.pages):
            qrow.qrow_matmul_multi([(L[n].codes, L[n].scales) for n in ("q", "k", "v")], x,
                                   out=[self.q, self.k, self.v])
            qrow.qrow_matmul(L["o"].codes, L["o"].scales, self.q, out=self.o)
            qrow.qrow_swiglu_into(L["gate"], L["up"], self.o, self.h)
            nxt = self.d[li % 2]
            qrow.qrow_matmul(L["down"].codes, L["down"].scales, self.h, out=nxt)
            x = nxt
        return x


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--m", type=int, default=1, help="decode tokens per pass (1, 4, 16, 32)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=6.0)
    ap.add_argument("--no-secondary", action="store_true", help="skip configs 1/3/4/5")
    ap.add_argument("--profile", choices=("swiglu", "stack", "copy", "w8a8", "w8a8p", "moe", "moe16", "lowbit", "codec",
                                          "dequant"),
                    help="for rocprofv3 runs: replay exactly the timed graph of the roofline kernel (28 "
                    "paired gate/up+SwiGLU launches) or of the headline pass, --steps times after "
                    "--warmup replays; a plain 256 MiB device copy x5 (counter calibration); or config 3's "
                    "fused W8A8 GEMM (M=512 and 2048), config 3's whole w8a8_matmul with protect_k=8 (w8a8p) / "
                    "config 4's MoE layer (T=64 and 512; moe16: the weight-only flow), or config 5's low-bit "
                    "GEMV/GEMM (both shapes, int3/int2, M=1 and 8), the offline codecs (int8, int3, "
                    "int2), or the whole-weight dequants (qrow bf16/fp32, int3/int2 fp32), --steps calls each")
    ap.add_argument("--eager", action="store_true",
                    help="with --profile swiglu/stack: launch the same sequence eagerly instead of replaying "
                    "the graph (counter collection needs eager dispatches)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(
            f"bench.py: this build measures one MI355X only (--gpus {args.gpus} requested); "
            "the QStore path is single-GPU here (sharding by output rows / experts is design only)",
            file=sys.stderr,
        )
        return 2

    import torch

    import __graft_entry__

    __graft_entry__.load_package()
    from mrun_pub_amd import qrow

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    m = args.m
    if args.profile == "copy":
        n = 256 << 20
        src = torch.randint(0, 255, (n,), dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"profile": "copy", "launches": 5, "read_bytes": n, "write_bytes": n}), flush=True)
        return 0
    if args.profile in ("w8a8", "w8a8p", "moe", "moe16"):
        print(json.dumps(profile_mfma_kernels(torch, dev, args.profile, args.steps)), flush=True)
        return 0
    if args.profile == "lowbit":
        print(json.dumps(profile_lowbit(torch, dev, args.steps)), flush=True)
        return 0
    if args.profile == "codec":
        print(json.dumps(profile_codecs(torch, dev, args.steps)), flush=True)
        return 0
    if args.profile == "dequant":
        print(json.dumps(profile_dequant(torch, dev, args.steps)), flush=True)
        return 0
    arena, pages = build_stack(torch, dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(1)
    chain = DecodeChain(torch, dev, pages, m, gen)
    stream = torch.cuda.Stream(device=dev)

    def capture(fn):
        with torch.cuda.stream(stream):
            fn()  # eager warm-up (also loads the library)
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                fn()
        return g

    graph = capture(chain.per_linear)

    # the dominant kernel: the paired gate/up + SwiGLU launch, 28 distinct layers per replay
    # (input: the chain's own o-projection output buffer)
    def swiglu_28():
        for L in pages:
            qrow.qrow_swiglu_into(L["gate"], L["up"], chain.o, chain.h)

    sw_graph = capture(swiglu_28)
    if args.profile and args.eager:
        with torch.cuda.stream(stream):
            for _ in range(args.warmup + args.steps):
                swiglu_28() if args.profile == "swiglu" else chain.per_linear()
        torch.cuda.synchronize()
        print(json.dumps({"profile": args.profile, "m": m, "eager_passes": args.warmup + args.steps,
                          "swiglu_launch_bytes": swiglu_launch_bytes(m), "pass_bytes": algorithmic_bytes_per_pass(m)}),
              flush=True)
        return 0
    if args.profile:
        g = sw_graph if args.profile == "swiglu" else graph
        times = _replay_times(torch, stream, g, args.steps, args.warmup)
        per_launch = _median(times) / (LAYERS if args.profile == "swiglu" else 1)
        print(json.dumps({"profile": args.profile, "m": m, "replays": args.steps, "median_us": round(per_launch * 1e6, 3),
                          "swiglu_launch_bytes": swiglu_launch_bytes(m)}), flush=True)
        return 0

    # timed region: exactly --steps replays of the pass, synchronised on both sides; each
    # replay is also bracketed by its own events on the replay stream (median reported)
    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
    t0 = time.perf_counter()
    with torch.cuda.stream(stream):
        ev[0].record(stream)
        for r in range(args.steps):
            graph.replay()
            ev[r + 1].record(stream)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    per_replay = [ev[r].elapsed_time(ev[r + 1]) * 1e-3 for r in range(args.steps)]
    per_pass = _median(per_replay)
    sw_times = _replay_times(torch, stream, sw_graph, max(50, args.steps), 5)
    sw_s = _median(sw_times) / LAYERS

    value = algorithmic_bytes_per_pass(m) / per_pass / 1e9
    sw_gbs = swiglu_launch_bytes(m) / sw_s / 1e9
    traffic = trace = None
    traffic_file = ROOT / "profiles" / "traffic.json"
    if traffic_file.exists():
        committed = json.loads(traffic_file.read_text())
        traffic = committed.get(f"qrow_swiglu_m{m}")
        tr = committed.get(f"qrow_swiglu_m{m}_trace")
        if tr:
            # the committed kernel trace of this same graph: its per-launch median and what
            # HIP events read inside the traced process, beside this run's event figure
            t_gbs = swiglu_launch_bytes(m) / (tr["median_us"] * 1e-6) / 1e9
            trace = {
                "median_us": tr["median_us"],
                "achieved": round(t_gbs, 1),
                "frac": round(t_gbs / HBM_PEAK_GBS, 4),
                "rel_diff_vs_event_frac": round(abs(t_gbs - sw_gbs) / sw_gbs, 4),
                "event_us_under_tracer": tr["event_us_under_tracer"],
                "tracer_share_us": round(tr["event_us_under_tracer"] - tr["event_us_plain"], 3),
                "source": "profiles/decode_gemv_m1.md (rocprofv3 --kernel-trace of bench.py --profile swiglu)",
            }
    out = {
        "metric": "HBM GB/s (% peak) int8 QStore decode GEMV; TOPS (% MFMA peak) W8A8/MoE",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(per_pass * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "dense decoder int8 qrow linear stack (BASELINE configs[1]), one decode pass with "
            "each linear's input the previous linear's output",
            "layers": LAYERS,
            "hidden": HIDDEN,
            "intermediate": INTER,
            "tokens_m": m,
            "weights": "int8 U{-127..127}, fp32 row scales U(0.5,1.5)/127, HBM resident",
            "pass_bytes": algorithmic_bytes_per_pass(m),
            "launches_per_pass": 4 * LAYERS,
            "hbm_frac_of_peak": round(value / HBM_PEAK_GBS, 4),
            "timing": f"median of {args.steps} graph replays (HIP events per replay) after {args.warmup} "
            f"warm-up replays; mean {sum(per_replay) / len(per_replay) * 1e3:.4f} ms, wall "
            f"{elapsed / args.steps * 1e3:.4f} ms per replay",
        },
        "roofline": {
            "kernel": "paired gate/up W8A16 + SwiGLU (qs_qrow_swiglu, k_gemv_xg_swi)",
            "bound": "hbm",
            "achieved": round(sw_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(sw_gbs / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "traffic_source": "committed figure: profiles/traffic.json (rocprofv3 --pmc FETCH_SIZE and "
            "WRITE_SIZE runs of bench.py --profile stack --eager, scaled by a 256 MiB copy; "
            "profiles/decode_gemv_m1.md)",
            "launch_us": round(sw_s * 1e6, 3),
            "bytes_per_launch": swiglu_launch_bytes(m),
            "timing": f"median of {len(sw_times)} replays of a graph of the 28 launches, / 28",
            "trace": trace,
        },
    }
    if not args.no_secondary:
        # config 2's other batch sizes (M = 4, 16, 32): the same chained pass and protocol
        batches = {}
        for mm in (4, 16, 32):
            if mm == m:
                continue
            cm = DecodeChain(torch, dev, pages, mm, gen)
            tp = _graph_time(torch, stream, lambda _i, c=cm: c.per_linear(), 1)
            batches[f"config2_stack_m{mm}"] = {
                "ms_per_pass": round(tp * 1e3, 4),
                "GB/s": round(algorithmic_bytes_per_pass(mm) / tp / 1e9, 1),
                "hbm_frac": round(algorithmic_bytes_per_pass(mm) / tp / 1e9 / HBM_PEAK_GBS, 4),
            }
        x_h = chain.x0
        x_i = torch.randn(m, INTER, device=dev, generator=gen).to(torch.bfloat16)
        paged = paged_measurement(torch, dev, pages, x_h, x_i)
        del arena, pages, graph, sw_graph, chain
        out["secondary"] = {**batches, "config2_paged_pinned_host": paged,
                            **secondary_measurements(torch, dev, stream)}
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(args.cpu_seconds, m)
        out["cpu_baseline"]["one_thread"] = cpu_baseline(args.cpu_seconds / 2, m, threads=1)["value"]
        out["cpu_baseline"]["cpu_model"] = _cpu_model()
        if not args.no_secondary:
            out["cpu_baselines_per_config"] = cpu_baselines_per_config()
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
