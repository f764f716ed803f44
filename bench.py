#!/usr/bin/env python3
"""Benchmark of the paged-KV hot path on one MI355X.

Headline (``value``): paged GQA decode-attention HBM throughput at the
Llama-3-8B shape (config 2): batch 16, 32 q / 8 kv heads, head_dim
128, contexts U[1024, 32768], 64-token pages at random pool slots, one query
token per sequence.  A step is one decode-attention call over the whole batch
with every input already resident in HBM; value = algorithmic bytes per step
/ step time.  The dominant kernel's average duration is measured with HIP
events on the stream the kernels are launched on.

The CPU baseline times the oracle's restatement of the reference algorithm
(concatenate pages, then fp32 SDPA; oracle/paged_attention.py) on the host
cores for one step of the same workload.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


GRAPH_MIN_CALLS = 16


def graph_seconds(calls, reps: int, rounds: int = 3) -> float:
    """Seconds per call of the launches in `calls` (a list of no-argument
    functions), captured once into a HIP graph and replayed `reps` times
    between two events, in `rounds` separate rounds; the median round is
    returned (short, MFMA-heavy calls vary by a few percent with the clock the
    GPU runs at in a given moment).  Replaying keeps the GPU busy back to
    back, so the events measure the device, not the rate at which Python
    issues launches (which, for calls of a few tens of microseconds, is the
    slower of the two).  The list is repeated in the graph up to at least
    GRAPH_MIN_CALLS calls (and `reps` divided accordingly): the gap between
    one replay and the next, about 17 us, would otherwise land on a few short
    calls, while a decode loop's graph holds every layer's launches.  Every
    call must already have run eagerly once, so its workspaces exist."""
    import torch

    copies = -(-GRAPH_MIN_CALLS // len(calls))
    calls = list(calls) * copies
    reps = max(1, reps // copies)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            for fn in calls:
                fn()
    torch.cuda.current_stream().wait_stream(side)
    graph.replay()
    torch.cuda.synchronize()
    times = []
    for _ in range(rounds):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            graph.replay()
        e1.record()
        torch.cuda.synchronize()
        times.append(e0.elapsed_time(e1) / 1e3 / (reps * len(calls)))
    return sorted(times)[len(times) // 2]


def profiled_traffic(name: str) -> int | None:
    """HBM bytes per launch recorded by rocprofv3 PMC runs in profiles/<name>.md.

    The figure is FETCH_SIZE + WRITE_SIZE scaled by the counters' reading for
    a kernel of known size (the summary states the scale and the commands).
    """
    path = ROOT / "profiles" / f"{name}.md"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return int(line.split(":", 1)[1].strip())
    return None


def cpu_threads() -> int:
    try:
        from threadpoolctl import threadpool_info

        n = [d.get("num_threads", 1) for d in threadpool_info() if d.get("user_api") == "blas"]
        return int(max(n)) if n else 1
    except Exception:  # pragma: no cover
        return 1


def host_cpus() -> dict:
    """The host's CPU model (as lscpu reports it), the logical CPU count and
    the CPUs this process may run on.  CPU legs use one thread per allowed
    CPU: os.cpu_count() counts the whole host, which a container or a
    scheduler's affinity mask may not grant."""
    model = None
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:  # pragma: no cover
        pass
    try:
        allowed = sorted(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        allowed = list(range(os.cpu_count() or 1))
    spans, start = [], None
    for i, c in enumerate(allowed):
        if start is None:
            start = c
        if i + 1 == len(allowed) or allowed[i + 1] != c + 1:
            spans.append(f"{start}-{c}" if c != start else f"{c}")
            start = None
    return {"cpu_model": model, "host_cpu_count": os.cpu_count(),
            "affinity": ",".join(spans), "threads": len(allowed)}


def set_cpu_threads() -> dict:
    import torch

    info = host_cpus()
    torch.set_num_threads(info["threads"])
    return info


def gqa_gather_floor(inp, reps: int = 20) -> dict:
    """Floor of config 2's page pattern: the calibration gather
    (voom_gather_read, ordinary 16-byte loads) over exactly the partials
    kernel's K and V bytes -- each 32-token block of each (sequence, kv head)
    as two 4 KiB rows of each pool, in the kernel's (sequence, kv head, block)
    order -- graph-replayed over 1024-8192 workgroups; then a linear read of
    the same byte count.  Returns GB/s per grid."""
    import numpy as np
    import torch

    from voom_amd import calibrate

    slots, NKV, PT, D = inp.k_pool.shape
    row = 2048  # bf16 elements per 4 KiB row
    kr = inp.k_pool.view(-1, row)
    vr = inp.v_pool.view(-1, row)
    rows_per_page = PT * D // row
    rows = []
    for b, ctx in enumerate(inp.ctx_host):
        j = np.arange((int(ctx) + 31) // 32)                     # 32-token blocks
        slot = inp.table_host[b][j * 32 // PT].astype(np.int64)
        first = (j * 32 % PT) * D // row                          # the block's first row
        for kvh in range(NKV):
            base = (slot * NKV + kvh) * rows_per_page + first
            rows.append(np.stack([base, base + 1], 1).reshape(-1))
    idx = torch.from_numpy(np.concatenate(rows).astype(np.int32)).cuda()
    nbytes = idx.numel() * row * 2 * 2
    sink = torch.zeros(8192, dtype=torch.int32, device="cuda")
    res = {"bytes": nbytes}
    for wg in (1024, 2048, 4096, 8192):
        f = lambda wg=wg: calibrate.gather_read(kr, idx, sink, base2=vr, workgroups=wg)
        f()
        res[f"gather_gbs_wg{wg}"] = nbytes / graph_seconds([f] * 4, reps) / 1e9
    lin = torch.empty(nbytes // 2, dtype=torch.int16, device="cuda")
    for wg in (2048, 8192):
        g = lambda wg=wg: calibrate.stream_read(lin, sink, workgroups=wg)
        g()
        res[f"linear_gbs_wg{wg}"] = nbytes / graph_seconds([g] * 4, reps) / 1e9
    del lin
    torch.cuda.empty_cache()
    return res


def bench_gqa(steps: int, warmup: int, cpu_sample: bool, gather_floor: bool = False) -> dict:
    import numpy as np
    import torch

    from voom_amd import ops, synthetic

    log("building config-2 inputs (B=16, 32q/8kv, D=128, ctx U[1024,32768], 64-token pages)")
    inp = synthetic.gqa_decode_inputs(device="cuda")
    torch.cuda.synchronize()
    nbytes = inp.algorithmic_bytes()
    out = torch.empty_like(inp.q)
    splits = ops.default_splits()
    ws = ops.workspace(inp.q.device, ops.gqa_workspace_bytes(16, 32, 8, 128, splits), tag=7)
    stream = torch.cuda.current_stream()

    max_pages = inp.block_table.shape[1]

    def step(ev=None):
        # The decode op is its two halves, launched back to back on one stream.
        # One event before each half: the first pair brackets the page-streaming
        # kernel, the second half runs until the next step's first event.
        if ev is not None:
            ev[0].record(stream)
        ops.paged_gqa_partials(inp.q, inp.k_pool, inp.v_pool, inp.block_table, inp.ctx_lens,
                               scale=inp.scale, num_splits=splits, ws=ws, stream=stream)
        if ev is not None:
            ev[1].record(stream)
        ops.paged_gqa_combine(inp.ctx_lens, out, ws, num_kv_heads=8, page_tokens=64,
                              max_pages=max_pages, num_splits=splits, stream=stream)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    log(f"warmup done ({warmup} steps); timing {steps} steps")
    # the timed region: exactly `steps` decode ops back to back, nothing else
    # on the stream between the two bracketing events
    t_all0 = torch.cuda.Event(enable_timing=True)
    t_all1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_all0.record(stream)
    for _ in range(steps):
        step()
    t_all1.record(stream)
    torch.cuda.synchronize()
    total_ms = t_all0.elapsed_time(t_all1)
    # a second, instrumented pass for the per-kernel figures: an event before
    # each half of every op (the events themselves add a few microseconds per
    # step, which is why the timed region above has none)
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(steps)]
    t_end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    for i in range(steps):
        step(evs[i])
    t_end.record(stream)
    torch.cuda.synchronize()
    nxt = [evs[i + 1][0] for i in range(steps - 1)] + [t_end]
    main_ms = sorted(e[0].elapsed_time(e[1]) for e in evs)
    comb_ms = sorted(e[1].elapsed_time(n) for e, n in zip(evs, nxt))
    op_ms = sorted(e[0].elapsed_time(n) for e, n in zip(evs, nxt))
    avg = lambda xs: sum(xs) / len(xs)
    ms_per_step = total_ms / steps
    gbs = nbytes / (ms_per_step * 1e-3) / 1e9
    # the page-streaming kernel moves everything but the output rows
    main_bytes = nbytes - 16 * 32 * 128 * 2
    achieved = main_bytes / (avg(main_ms) * 1e-3) / 1e9
    log(f"step {ms_per_step * 1e3:.1f} us, op avg {avg(op_ms) * 1e3:.1f} us, partials kernel "
        f"{avg(main_ms) * 1e3:.1f} us (min {main_ms[0] * 1e3:.1f}, max {main_ms[-1] * 1e3:.1f}), "
        f"combine + step gap {avg(comb_ms) * 1e3:.1f} us; {gbs:.0f} GB/s per step, "
        f"{achieved:.0f} GB/s partials kernel")

    res = {
        "value": gbs,
        "ms_per_step": ms_per_step,
        "bytes_per_step": nbytes,
        "op_avg_us": avg(op_ms) * 1e3,
        "op_gbs": nbytes / (avg(op_ms) * 1e-3) / 1e9,
        "combine_avg_us": avg(comb_ms) * 1e3,
        "roofline": {
            "bound": "hbm",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": profiled_traffic("gqa_decode_config2"),
            "traffic_source": "rocprofv3 --pmc FETCH_SIZE/WRITE_SIZE, calibrated; "
                              "profiles/gqa_decode_config2.md",
            "kernel": "gqa_decode_kernel<128,3,1> (voom_paged_gqa_partials), timed with HIP "
                      "events on its launch stream; algorithmic bytes = K+V of every live "
                      "token + q + table + lengths",
            "kernel_avg_us": avg(main_ms) * 1e3,
            "algorithmic_bytes": main_bytes,
        },
        "context_tokens": int(inp.ctx_host.sum()),
        "num_splits": splits,
    }
    if gather_floor:
        fl = gqa_gather_floor(inp)
        res["page_gather_floor"] = fl
        log("gather floor of these blocks (ordinary loads): " +
            ", ".join(f"{k} {v:.0f}" for k, v in fl.items() if k != "bytes"))

    if cpu_sample:
        from oracle import paged_attention as opa
        from voom_amd.page_pool import v_pages_to_tokens

        info = set_cpu_threads()
        log(f"cpu baseline: torch-CPU fp32 SDPA over the concatenated pages, "
            f"{info['threads']} threads ({info['cpu_model']}), repeated for >= 10 s")
        q_c = inp.q.cpu()
        k_c = inp.k_pool.cpu()
        v_c = v_pages_to_tokens(inp.v_pool).contiguous().cpu()
        n_cpu = 0
        t0 = time.perf_counter()
        while True:
            ref = opa.paged_decode_torch(q_c, k_c, v_c, inp.table_host, inp.ctx_host, inp.scale)
            n_cpu += 1
            dt = time.perf_counter() - t0
            if dt >= 10.0 or n_cpu >= 200:
                break
        got = out.float().cpu()
        err = float((got - ref).abs().max())
        res["cpu_baseline"] = {
            "value": n_cpu * nbytes / dt / 1e9,
            "unit": "GB/s",
            "cores": info["threads"],
            "kind": "port",
            "sample": f"{n_cpu} full config-2 decode steps (16 sequences, all pages, "
                      f"{dt:.1f} s): per sequence, pages concatenated in logical order, then "
                      "torch-CPU fp32 scaled_dot_product_attention with the GQA broadcast "
                      "(oracle/paged_attention.py paged_decode_torch; reference-algorithm "
                      "CPU restatement)",
            "seconds": dt,
            "steps": n_cpu,
            **info,
        }
        res["parity_max_abs_err_vs_oracle"] = err
        log(f"cpu baseline {n_cpu * nbytes / dt / 1e9:.2f} GB/s ({n_cpu} steps in {dt:.2f}s); "
            f"max |gpu-oracle| {err:.4f}")
        del k_c, v_c
    return res


def copy_calibration(nbytes: int = 1 << 30, reps: int = 5) -> None:
    """A plain streaming kernel of known size, the scale for PMC byte counters.

    voom's contiguous byte-plane split (kernel ``split_kernel``) over ``nbytes``
    of 16-bit data reads exactly ``nbytes`` and writes exactly ``nbytes``.
    """
    import torch

    from voom_amd import ops

    src = torch.ones(nbytes // 2, dtype=torch.int16, device="cuda")
    lo = torch.empty(nbytes // 2, dtype=torch.uint8, device="cuda")
    hi = torch.empty_like(lo)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        ops.byteplane_split(src, lo, hi)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    log(f"copy calibration (split_kernel): {nbytes} B read + {nbytes} B written per launch, "
        f"{ms * 1e3:.1f} us, {2 * nbytes / ms / 1e6:.0f} GB/s (read+write)")
    del src, lo, hi


def link_ceiling(nbytes: int = 256 << 20, reps: int = 5) -> dict:
    """Pinned host <-> device copy bandwidth (hipMemcpyAsync through torch)."""
    import torch

    host = torch.empty(nbytes, dtype=torch.uint8, pin_memory=True)
    dev = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    res = {}
    for name, dst, src in (("h2d", dev, host), ("d2h", host, dev)):
        dst.copy_(src, non_blocking=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            dst.copy_(src, non_blocking=True)
        torch.cuda.synchronize()
        res[name + "_gbs"] = nbytes * reps / (time.perf_counter() - t0) / 1e9
    return res


def bench_spill_reload(cpu_sample: bool) -> dict:
    """Config 3: 32 layers x 32768 tokens x 8 kv heads x 128, evict the oldest
    50 % of pages (2 GiB) through the byte-plane split into pinned host memory,
    reload into free pool slots, compare all 4 GiB bitwise."""
    import numpy as np
    import torch

    # first, before the 4 GiB of config 3 exist in this process
    fragmented = bench_fragmented_spills()

    from voom_amd import ops
    from voom_amd.kv_paged import PagedKVCache

    L, S, NKV, D, PT = 32, 32768, 8, 128, 64
    log("config 3: building 32 x 32768-token layers (4 GiB of bf16 K/V)")
    gen = torch.Generator(device="cuda").manual_seed(6)
    chans = np.random.default_rng(6).choice(D, size=(NKV, 4), replace=True)
    for h in range(NKV):
        chans[h] = np.random.default_rng(6 + h).choice(D, size=4, replace=False)
    outlier = torch.ones((1, NKV, 1, D), device="cuda")
    for h in range(NKV):
        outlier[0, h, 0, torch.from_numpy(chans[h]).cuda()] = 20.0
    kv = PagedKVCache(num_layers=L, max_bytes=1 << 62, page_positions=PT, resident_pages=1,
                      initial_slots=S // PT)
    orig = []
    for layer in range(L):
        k = (torch.randn((1, NKV, S, D), generator=gen, device="cuda") * outlier).to(torch.bfloat16)
        v = (torch.randn((1, NKV, S, D), generator=gen, device="cuda") * 0.5).to(torch.bfloat16)
        kv.append(layer, k, v)
        orig.append((k, v))
    spill_bytes = L * (S // PT // 2) * kv.page_nbytes
    kv.arena.reserve(spill_bytes + (64 << 20))
    torch.cuda.synchronize()
    link = link_ceiling()
    # One untimed cycle first: the first transfers into freshly pinned host
    # pages pay a one-time mapping cost (reported as the cold figures).
    kv.max_bytes = kv.nbytes() - spill_bytes
    t0 = time.perf_counter()
    kv.spill()
    torch.cuda.synchronize()
    t_spill_cold = time.perf_counter() - t0
    t0 = time.perf_counter()
    kv.reload()
    torch.cuda.synchronize()
    t_reload_cold = time.perf_counter() - t0
    # Warm cycles: the host link's rate into the same pinned pages varies from
    # cycle to cycle on these boxes (other work shares the host), so several
    # cycles are timed and the median is reported (the best alongside).
    cycles = []
    for _ in range(5):
        kv.max_bytes = kv.nbytes() - spill_bytes
        t0 = time.perf_counter()
        n_spilled = kv.spill()
        t_spill_host = time.perf_counter() - t0
        torch.cuda.synchronize()
        t_spill = time.perf_counter() - t0
        assert n_spilled == L * (S // PT // 2), n_spilled
        assert all(not kv._pages[l][i].resident for l in range(L) for i in range(S // PT // 2))
        t0 = time.perf_counter()
        n_reloaded = kv.reload()
        t_reload_host = time.perf_counter() - t0
        torch.cuda.synchronize()
        t_reload = time.perf_counter() - t0
        cycles.append((t_spill, t_reload, t_spill_host, t_reload_host))
    t_spill = sorted(c[0] for c in cycles)[len(cycles) // 2]
    t_reload = sorted(c[1] for c in cycles)[len(cycles) // 2]
    t_spill_host = sorted(c[2] for c in cycles)[len(cycles) // 2]
    t_reload_host = sorted(c[3] for c in cycles)[len(cycles) // 2]
    best_spill = min(c[0] for c in cycles)
    best_reload = min(c[1] for c in cycles)
    # The host link measured on the arena's own pages: plain copies of the
    # same 32 record-sized blocks the spill wrote (first fit puts them where
    # the spill's records were), in both directions: the ceiling the spill
    # and reload can reach with this memory.  (The copy engine's first read
    # of freshly pinned pages is slow; reserve() pays that before any spill.)
    rec_bytes = (S // PT // 2) * kv.page_nbytes + 4096
    blocks = [kv.arena.alloc(rec_bytes) for _ in range(L)]
    dev_rec = torch.empty(rec_bytes, dtype=torch.uint8, device="cuda")
    side = torch.cuda.Stream()
    arena_link = {}
    for name in ("d2h", "h2d"):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        with torch.cuda.stream(side):
            for blk in blocks:
                if name == "d2h":
                    blk.view.copy_(dev_rec, non_blocking=True)
                else:
                    dev_rec.copy_(blk.view, non_blocking=True)
        side.synchronize()
        arena_link[name + "_gbs"] = L * rec_bytes / (time.perf_counter() - t0) / 1e9
    for blk in blocks:
        kv.arena.free(blk)
    del dev_rec
    exact = True
    for layer in range(L):
        k2, v2 = ops.gather_kv(kv._pools[layer].k, kv._pools[layer].v, kv._tables[layer], S)
        exact &= torch.equal(k2.view(torch.int16), orig[layer][0].view(torch.int16))
        exact &= torch.equal(v2.view(torch.int16), orig[layer][1].view(torch.int16))
    torch.cuda.synchronize()
    res = {
        "workload": "config 3: 32 layers x 32768 tokens x 8 kv x 128 bf16, evict oldest 50% "
                    "(8192 pages of 256 KiB) via byte-plane split to pinned host, reload",
        "spill_bytes": spill_bytes,
        "spill_gbs": spill_bytes / t_spill / 1e9,
        "reload_gbs": spill_bytes / t_reload / 1e9,
        "spill_s": t_spill,
        "reload_s": t_reload,
        "warm_cycles": len(cycles),
        "spill_gbs_per_cycle": [round(spill_bytes / c[0] / 1e9, 2) for c in cycles],
        "reload_gbs_per_cycle": [round(spill_bytes / c[1] / 1e9, 2) for c in cycles],
        "spill_best_gbs": spill_bytes / best_spill / 1e9,
        "reload_best_gbs": spill_bytes / best_reload / 1e9,
        "spill_cold_gbs": spill_bytes / t_spill_cold / 1e9,
        "reload_cold_gbs": spill_bytes / t_reload_cold / 1e9,
        "spill_host_return_s": t_spill_host,
        "reload_host_return_s": t_reload_host,
        "pages": n_spilled,
        "reloaded": n_reloaded,
        "bit_exact": bool(exact),
        "link_ceiling": link,
        "spill_frac_of_link": spill_bytes / t_spill / 1e9 / link["d2h_gbs"],
        "reload_frac_of_link": spill_bytes / t_reload / 1e9 / link["h2d_gbs"],
        "arena_link": arena_link,
        "spill_frac_of_arena_link": spill_bytes / t_spill / 1e9 / arena_link["d2h_gbs"],
        "reload_frac_of_arena_link": spill_bytes / t_reload / 1e9 / arena_link["h2d_gbs"],
    }
    # the same spill with compress_spill: zstd level 1 of the high planes runs
    # on worker threads after each record's copy lands (the raw planes stay in
    # the arena); timed to the copies landing and to the last zstd frame
    kv.compress_spill = True
    kv.max_bytes = kv.nbytes() - spill_bytes
    t0 = time.perf_counter()
    n_c = kv.spill()
    t_c_host = time.perf_counter() - t0
    torch.cuda.synchronize()
    t_c_copy = time.perf_counter() - t0
    kv._wait_host_work()
    t_c_all = time.perf_counter() - t0
    st = kv.stats
    assert n_c == n_spilled
    kv.compress_spill = False
    kv.reload()
    torch.cuda.synchronize()
    exact_c = True
    for layer in range(L):
        k2, v2 = ops.gather_kv(kv._pools[layer].k, kv._pools[layer].v, kv._tables[layer], S)
        exact_c &= torch.equal(k2.view(torch.int16), orig[layer][0].view(torch.int16))
        exact_c &= torch.equal(v2.view(torch.int16), orig[layer][1].view(torch.int16))
    res_c = {
        "spill_gbs": spill_bytes / t_c_copy / 1e9,
        "spill_host_return_s": t_c_host,
        "zstd_done_s": t_c_all,
        "zstd_gbs_hi_planes": spill_bytes / 2 / t_c_all / 1e9,
        "zstd_ratio_hi_plane": (st.spill_bytes_raw / 2) / (st.spill_bytes_compressed
                                                            - st.spill_bytes_raw / 2),
        "ratio_page": st.spill_bytes_raw / st.spill_bytes_compressed,
        "workers": kv._workers._max_workers if kv._workers is not None else 0,
        "bit_exact_after_reload": bool(exact_c),
    }
    res["compress_spill"] = res_c
    log(f"config 3 compressed: spill {res_c['spill_gbs']:.1f} GB/s to the arena, zstd of the "
        f"high planes done after {t_c_all * 1e3:.1f} ms ({res_c['zstd_gbs_hi_planes']:.2f} GB/s, "
        f"{res_c['workers']} threads), page ratio {res_c['ratio_page']:.3f}")
    log(f"config 3: spill() returned after {t_spill_host * 1e3:.1f} ms of {t_spill * 1e3:.1f} ms, "
        f"reload() after {t_reload_host * 1e3:.1f} ms of {t_reload * 1e3:.1f} ms")
    log(f"config 3: spill {res['spill_gbs']:.1f} GB/s, reload {res['reload_gbs']:.1f} GB/s, "
        f"link d2h {link['d2h_gbs']:.1f} / h2d {link['h2d_gbs']:.1f} GB/s (on the arena's pages "
        f"{arena_link['d2h_gbs']:.1f} / {arena_link['h2d_gbs']:.1f}), exact={exact}")
    if cpu_sample:
        from concurrent.futures import ThreadPoolExecutor

        from oracle import byteplane as ob

        lib = ob.load_c()
        info = host_cpus()
        nthreads = info["threads"] if lib is not None else 1
        # layer 0's K and V (128 MiB of bf16), split into one piece per thread;
        # the C restatement runs without the GIL, so the pieces run in parallel
        sample = torch.cat([orig[0][0].reshape(-1), orig[0][1].reshape(-1)])
        sample = sample.view(torch.int16).cpu().numpy().view(np.uint16)
        pieces = np.array_split(sample, nthreads)

        def roundtrip(piece):
            lo, hi = ob.split_c(lib, piece) if lib is not None else ob.split(piece)
            back = ob.merge_c(lib, lo, hi) if lib is not None else ob.merge(lo, hi)
            return bool(np.array_equal(back, piece))

        n_cpu = 0
        ok = True
        t0 = time.perf_counter()
        with ThreadPoolExecutor(nthreads) as pool:
            while True:
                results = list(pool.map(roundtrip, pieces))
                ok &= all(results)
                n_cpu += 1
                dt = time.perf_counter() - t0
                if dt >= 10.0 or n_cpu >= 5000:
                    break
        assert ok
        res["cpu_baseline"] = {
            "value": n_cpu * 2 * sample.nbytes / dt / 1e9, "unit": "GB/s (split+merge bytes)",
            "cores": nthreads, "kind": "port",
            "sample": f"{n_cpu} byte-plane split + merge round trips of layer 0's K and V "
                      f"(128 MiB) in {nthreads} pieces on {nthreads} threads, "
                      "oracle/byteplane.c (reference-algorithm CPU restatement)",
            "seconds": dt, **info,
        }
        from voom_amd import zstd as vz

        if vz.available():
            hi_np = ob.split(sample[: 16 << 20])[1]
            t0 = time.perf_counter()
            z = vz.compress(hi_np, 1)
            dtz = time.perf_counter() - t0
            res["zstd_hi_plane"] = {"ratio": hi_np.nbytes / z.nbytes,
                                   "compress_gbs_1core": hi_np.nbytes / dtz / 1e9,
                                   "sample": "16 MiB of layer-0 K hi plane, level 1"}
    del orig
    kv.release()
    torch.cuda.empty_cache()
    res["fragmented_spills"] = fragmented
    return res


def bench_fragmented_spills() -> dict:
    """Pages spilled one at a time, as the budget leaves them in a growing
    decode: 100 pages of 256 KiB (one sequence, 8 kv heads, D = 128, 64-token
    pages) spilled by one call (one host record) or by 100 calls (100 one-page
    records), then attend() over the layer (the spilled pages reloaded for the
    call) and reload() of them, on one cache; host-timed with a wait per call."""
    import torch

    from voom_amd.kv_paged import PagedKVCache

    NQ, NKV, D, PT, n = 64, 8, 128, 64, 100
    gen = torch.Generator(device="cuda").manual_seed(3)
    k = torch.randn((1, NKV, 200 * PT, D), generator=gen, device="cuda").to(torch.bfloat16)
    v = torch.randn((1, NKV, 200 * PT, D), generator=gen, device="cuda").to(torch.bfloat16)
    q = torch.randn((1, NQ, 1, D), generator=gen, device="cuda").to(torch.bfloat16)
    kv = PagedKVCache(num_layers=1, max_bytes=1 << 40, page_positions=PT, resident_pages=1)
    kv.append(0, k, v)
    kv.arena.reserve(2 * n * kv.page_nbytes)
    main = torch.cuda.current_stream()
    res = {"pages": n, "page_bytes": kv.page_nbytes}
    for mode in ("one_record", "one_page_records"):
        att, rel = [], []
        for cycle in range(4):
            if mode == "one_record":
                kv.spill([(0, i) for i in range(n)])
            else:
                for i in range(n):
                    kv.spill([(0, i)])
            torch.cuda.synchronize()
            for rep in range(4):
                t0 = time.perf_counter()
                kv.attend(0, q)
                main.synchronize()
                if cycle and rep:
                    att.append(time.perf_counter() - t0)
            t0 = time.perf_counter()
            kv.reload()
            torch.cuda.synchronize()
            if cycle:
                rel.append(time.perf_counter() - t0)
        res[mode] = {"attend_ms": sorted(att)[len(att) // 2] * 1e3,
                     "reload_ms": sorted(rel)[len(rel) // 2] * 1e3}
    K, V = kv.gather(0)
    torch.cuda.synchronize()
    res["exact"] = bool(torch.equal(K.view(torch.int16), k.view(torch.int16))
                        and torch.equal(V.view(torch.int16), v.view(torch.int16)))
    kv.release()
    log(f"spills of one page at a time ({n} x {res['page_bytes'] >> 10} KiB): attend "
        f"{res['one_page_records']['attend_ms']:.2f} ms, reload "
        f"{res['one_page_records']['reload_ms']:.2f} ms (one record: "
        f"{res['one_record']['attend_ms']:.2f} / {res['one_record']['reload_ms']:.2f} ms), "
        f"exact={res['exact']}")
    return res


def bench_long_context(steps: int, cpu_sample: bool) -> dict:
    """Config 4: one sequence, 64 q / 8 kv heads, 131072 tokens in 64-token
    pages, oldest 40 % spilled; each decode step appends a token and attends,
    reloading the spilled pages on the side stream while the resident pages
    are attended (reference semantics: reload every call)."""
    import numpy as np
    import torch

    from voom_amd import ops, synthetic
    from voom_amd.kv_paged import PagedKVCache

    NQ, NKV, D, PT, S = 64, 8, 128, 64, 131072
    log("config 4: building a 131072-token sequence (1 GiB of bf16 K/V)")
    gen = torch.Generator(device="cuda").manual_seed(9)
    kv = PagedKVCache(num_layers=1, max_bytes=1 << 62, page_positions=PT, resident_pages=1,
                      initial_slots=S // PT + 8)
    pos = torch.arange(S, device="cuda")
    chunk = 16384
    for c0 in range(0, S, chunk):
        kr = torch.randn((1, NKV, chunk, D), generator=gen, device="cuda")
        cos, sin = synthetic.rope_tables(pos[c0:c0 + chunk], D, 5e5)
        k = synthetic.apply_rope_neox(kr, cos, sin).to(torch.bfloat16)
        v = torch.randn((1, NKV, chunk, D), generator=gen, device="cuda").to(torch.bfloat16)
        kv.append(0, k, v)
    n_spill = int(0.4 * (S // PT))
    qs = torch.randn((steps, 1, NQ, 1, D), generator=gen, device="cuda").to(torch.bfloat16)
    new_k = torch.randn((steps, 1, NKV, 1, D), generator=gen, device="cuda").to(torch.bfloat16)
    new_v = torch.randn((steps, 1, NKV, 1, D), generator=gen, device="cuda").to(torch.bfloat16)
    # attention alone over the fully resident sequence
    ctx = torch.full((1,), S, dtype=torch.int32, device="cuda")
    pool = kv._pools[0]
    for _ in range(3):
        ops.paged_gqa_decode(qs[0], pool.k, pool.v, kv._tables[0], ctx)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(10):
        ops.paged_gqa_decode(qs[i % steps], pool.k, pool.v, kv._tables[0], ctx)
    e1.record()
    torch.cuda.synchronize()
    t_attn = e0.elapsed_time(e1) / 10 / 1e3
    spill_pages = [(0, i) for i in range(n_spill)]
    kv.arena.reserve(n_spill * kv.page_nbytes + (16 << 20))
    kv.spill(spill_pages)
    torch.cuda.synchronize()
    reload_bytes = n_spill * kv.page_nbytes
    link_h2d_gbs = link_ceiling()["h2d_gbs"]
    # reload alone (transient, as inside attend)
    spilled = [p for p in kv._pages[0] if not p.resident]
    stage = kv._stage_pool(0)
    kv._stream_in(0, spilled, stage, lambda chunk, slots: None, transient=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(3):
        kv._stream_in(0, spilled, stage, lambda chunk, slots: None, transient=True)
    torch.cuda.synchronize()
    t_reload = (time.perf_counter() - t0) / 3
    # decode steps
    for i in range(2):
        kv.append(0, new_k[i], new_v[i])
        kv.attend(0, qs[i])
    torch.cuda.synchronize()
    # A decode loop waits for each step's output on the main stream (the next
    # query depends on it); the side-stream upload started at the end of the
    # step keeps the host link busy across that wait.
    main = torch.cuda.current_stream()
    t0 = time.perf_counter()
    for i in range(steps):
        kv.append(0, new_k[i], new_v[i])
        out = kv.attend(0, qs[i])
        main.synchronize()
    torch.cuda.synchronize()
    t_step = (time.perf_counter() - t0) / steps
    t0 = time.perf_counter()
    for i in range(steps):
        kv.append(0, new_k[i], new_v[i])
        out = kv.attend(0, qs[i])
    torch.cuda.synchronize()
    t_free = (time.perf_counter() - t0) / steps
    # The same bytes as one plain pinned-host -> device copy (events on the
    # copy's stream): the time the step's reload needs on the link by itself.
    host_buf = torch.empty(reload_bytes, dtype=torch.uint8, pin_memory=True)
    dev_buf = torch.empty(reload_bytes, dtype=torch.uint8, device="cuda")
    dev_buf.copy_(host_buf, non_blocking=True)
    torch.cuda.synchronize()
    c0, c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    c0.record()
    for _ in range(3):
        dev_buf.copy_(host_buf, non_blocking=True)
    c1.record()
    torch.cuda.synchronize()
    copy_ms = c0.elapsed_time(c1) / 3
    del host_buf, dev_buf
    # The same upload from where the spilled records actually sit, the
    # arena's pages (each step's upload follows the last one on the copy
    # stream, so this is the step's floor).
    held = {id(p.host): p.host for p in kv._pages[0] if not p.resident and p.host is not None}
    records = [sb.record(r) for sb in held.values()
               for r in range(-(-sb.n_pages // sb.chunk))]
    dev_rec = torch.empty(max(r.numel() for r in records), dtype=torch.uint8, device="cuda")
    side = torch.cuda.Stream()
    a0, a1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(side):
        for rec in records:
            dev_rec[:rec.numel()].copy_(rec, non_blocking=True)
        a0.record(side)
        for _ in range(3):
            for rec in records:
                dev_rec[:rec.numel()].copy_(rec, non_blocking=True)
        a1.record(side)
    side.synchronize()
    arena_copy_ms = a0.elapsed_time(a1) / 3
    del dev_rec
    # What the overlap hides: the part of a step beyond the time its reload
    # bytes need as one plain copy is exposed work; the attention it would
    # otherwise add is attention_only_ms (all pages resident).
    link_ms = reload_bytes / (link_h2d_gbs * 1e9) * 1e3 if link_h2d_gbs else None
    exposed_vs_copy_ms = max(0.0, t_step * 1e3 - copy_ms)
    hidden_vs_copy = min(1.0, max(0.0, 1.0 - exposed_vs_copy_ms / (t_attn * 1e3)))
    exposed_ms = max(0.0, t_step * 1e3 - link_ms) if link_ms is not None else None
    hidden = (min(1.0, max(0.0, 1.0 - exposed_ms / (t_attn * 1e3)))
              if exposed_ms is not None else None)
    exposed_vs_arena_ms = max(0.0, t_step * 1e3 - arena_copy_ms)
    hidden_vs_arena = min(1.0, max(0.0, 1.0 - exposed_vs_arena_ms / (t_attn * 1e3)))
    res = {
        "workload": "config 4: 1 x 131072 tokens, 64q/8kv, D=128, 40% (819 pages) spilled, "
                    f"{steps} decode steps with per-step reload overlapped with attention",
        "step_ms": t_step * 1e3,
        "step_ms_free_running": t_free * 1e3,
        "link_bound_ms": link_ms,
        "exposed_ms": exposed_ms,
        "hidden_attention_frac": hidden,
        "copy_only_ms": copy_ms,
        "exposed_vs_copy_ms": exposed_vs_copy_ms,
        "hidden_attention_frac_vs_copy": hidden_vs_copy,
        "arena_copy_ms": arena_copy_ms,
        "exposed_vs_arena_copy_ms": exposed_vs_arena_ms,
        "hidden_attention_frac_vs_arena_copy": hidden_vs_arena,
        "overlap_note": "exposed_ms = step_ms - link_bound_ms (the link probe's peak rate); "
                        "exposed_vs_copy_ms = step_ms - copy_only_ms (one plain H2D copy of "
                        "the step's reload bytes from a fresh pinned buffer); "
                        "exposed_vs_arena_copy_ms = step_ms - arena_copy_ms (the same upload "
                        "from the arena pages the spilled records sit in, the step's floor); "
                        "hidden fractions = 1 - exposed / attention_only_ms, clamped to [0, 1]",
        "link_utilisation": (link_ms / (t_step * 1e3)) if link_ms is not None else None,
        "reload_bytes_per_step": reload_bytes,
        "reload_gbs": reload_bytes / t_step / 1e9,
        "reload_only_ms_no_prefetch": t_reload * 1e3,
        "attention_only_ms": t_attn * 1e3,
        "attention_gbs": S * NKV * D * 4 / t_attn / 1e9,
        "steps": steps,
    }
    log(f"config 4: step {t_step * 1e3:.2f} ms (free-running {t_free * 1e3:.2f} ms), "
        f"link bound {link_ms if link_ms is None else round(link_ms, 3)} ms, exposed "
        f"{exposed_ms if exposed_ms is None else round(exposed_ms, 3)} ms of "
        f"{t_attn * 1e3:.3f} ms attention (hidden {hidden}); one plain copy of the reload "
        f"bytes {copy_ms:.3f} ms, exposed beyond it {exposed_vs_copy_ms:.3f} ms; the same "
        f"upload from the arena's pages {arena_copy_ms:.3f} ms, exposed beyond it "
        f"{exposed_vs_arena_ms:.3f} ms (hidden {hidden_vs_arena:.2f})")
    if cpu_sample:
        from oracle import paged_attention as opa

        info = set_cpu_threads()
        K, V = kv.gather(0)
        Sn = K.shape[2]
        k_c = K[0].cpu()
        v_c = V[0].cpu()
        q_c = qs[steps - 1][0, :, 0].cpu()
        n_cpu = 0
        t0 = time.perf_counter()
        while True:
            ref = opa.sdpa_decode_torch(q_c, k_c, v_c, D ** -0.5)
            n_cpu += 1
            dt = time.perf_counter() - t0
            if dt >= 10.0 or n_cpu >= 500:
                break
        err = float((out[0, :, 0].float().cpu() - ref).abs().max())
        res["cpu_baseline"] = {"value": n_cpu * Sn * NKV * D * 4 / dt / 1e9, "unit": "GB/s",
                               "cores": info["threads"], "kind": "port",
                               "sample": f"{n_cpu} decode steps over the {Sn} concatenated "
                                         "tokens, all resident (torch-CPU fp32 SDPA with the "
                                         "GQA broadcast, oracle/paged_attention.py; "
                                         "reference-algorithm CPU restatement)",
                               "seconds": dt, **info}
        res["parity_max_abs_err_vs_oracle"] = err
    kv.release()
    torch.cuda.empty_cache()
    return res


def bench_mla(steps: int, warmup: int, cpu_sample: bool) -> dict:
    """Config 5: absorbed-MLA paged decode, B=8, H=128, ctx 16384, latent 512+64.

    Four input sets (4 x 151 MB > 512 MB) rotate so the 256 MB Infinity Cache
    cannot hold the working set; the latent kernel (+ its reduce) is timed
    with HIP events around replays of a captured graph of the four steps,
    the absorption GEMMs separately.
    """
    import numpy as np
    import torch

    from voom_amd import calibrate, ops, synthetic

    log("config 5: building 4 rotating input sets (B=8, H=128, ctx 16384, latent 576)")
    sets = [synthetic.mla_decode_inputs(seed=8 + 100 * i) for i in range(4)]
    inp = sets[0]
    w_uk, w_uv_t = ops.split_kv_b(inp.kv_b, 128, inp.dn, inp.dv)
    q_lats = []
    for s_ in sets:
        q_abs = torch.bmm(s_.q_nope.transpose(0, 1).contiguous(), w_uk).transpose(0, 1)
        q_lats.append(torch.cat([q_abs, s_.q_rope], -1).contiguous())
    out = torch.empty((8, 128, 512), dtype=torch.bfloat16, device="cuda")
    ws = ops.workspace(inp.q_nope.device, ops.mla_workspace_bytes(8, 128, 0), tag=8)

    def step(i):
        s_ = sets[i % 4]
        ops.mla_latent_decode(q_lats[i % 4], s_.lat_pool, s_.block_table, s_.ctx_lens,
                              scale=s_.scale, out=out, ws=ws)

    for i in range(max(warmup, 4)):
        step(i)
    torch.cuda.synchronize()
    # one graph of the four rotating steps, replayed
    t = graph_seconds([lambda i=i: step(i) for i in range(4)], max(1, steps // 4))
    nbytes = inp.latent_bytes() + 8 * 128 * 576 * 2 + 8 * 128 * 512 * 2
    flops = inp.latent_flops()
    # absorption GEMMs (q_nope . W_UK, weighted_c . W_UV) on their own, replayed
    # from a graph like the contraction (eager launches from Python would
    # time the host).  Eight weight sets (8 x 33.6 MB) rotate so that the
    # 256 MB Infinity Cache cannot serve them.
    # The weights are packed once, as a deployment would at load time.
    gw = torch.Generator(device="cuda").manual_seed(77)
    w_sets = [(w_uk, w_uv_t)] + [
        ((torch.randn(w_uk.shape, generator=gw, device="cuda") * 0.02).to(torch.bfloat16),
         (torch.randn(w_uv_t.shape, generator=gw, device="cuda") * 0.02).to(torch.bfloat16))
        for _ in range(7)]
    w_sets = [(ops.pack_head_weights(a), ops.pack_head_weights(b)) for a, b in w_sets]

    def absorb(i):
        wk, wv = w_sets[i % 8]
        ops.mla_absorb_query(inp.q_nope, inp.q_rope, wk)
        ops.mla_project_out(out, wv)

    for i in range(8):
        absorb(i)
    torch.cuda.synchronize()
    t_gemm = graph_seconds([lambda i=i: absorb(i) for i in range(8)], max(1, steps // 8))

    # the whole decode step of config 5: q absorption (with q_rope, one
    # launch), latent kernel, merge of its partials fused with weighted_c .
    # W_UV; rotating latent and weight sets
    def full(i):
        s_ = sets[i % 4]
        wk, wv = w_sets[i % 8]
        return ops.mla_absorbed_decode(s_.q_nope, s_.q_rope, s_.lat_pool, s_.block_table,
                                       s_.ctx_lens, wk, wv, scale=s_.scale)

    for i in range(8):
        full(i)
    torch.cuda.synchronize()
    t_full = graph_seconds([lambda i=i: full(i) for i in range(8)], max(1, steps // 8))

    # the floor of one launch that streams one weight set's 16.8 MB: a plain
    # read kernel over 8 rotating buffers of that size
    w_bytes = 128 * 128 * 512 * 2  # H x dn x c of W_UK (= H x c x dv of W_UV)
    floor_bufs = [torch.empty(w_bytes, dtype=torch.uint8, device="cuda") for _ in range(8)]
    sink = torch.zeros(512, dtype=torch.int32, device="cuda")
    for i in range(8):
        calibrate.stream_read(floor_bufs[i], sink)
    torch.cuda.synchronize()
    t_floor = graph_seconds([lambda i=i: calibrate.stream_read(floor_bufs[i], sink) for i in range(8)],
                            max(1, steps // 8))
    del floor_bufs
    # floors of the latent kernel's loads: the same decomposition (16 ranges per
    # sequence, the two 64-head groups of a range each filling its tiles into
    # LDS) with no arithmetic, and one workgroup per range with twice the ranges
    # (each tile filled into one CU only)
    # ranges the latent kernel picks by default: enough (sequence, range, head
    # group) workgroups for one per CU
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    nr = max(1, -(-cus // (8 * 2)))
    rows_buf = torch.empty(8 * 2 * nr * 64 * 512, dtype=torch.float16, device="cuda")
    tsink = torch.zeros(8 * 2 * nr, dtype=torch.int32, device="cuda")

    def tile_pass(i, ranges, groups):
        s_ = sets[i % 4]
        calibrate.tile_read(s_.lat_pool, s_.block_table, 16384, ranges, groups, rows_buf, tsink,
                      q=q_lats[i % 4])

    load_floor = {}
    for ranges, groups in ((nr, 2), (2 * nr, 1)):
        for i in range(4):
            tile_pass(i, ranges, groups)
        torch.cuda.synchronize()
        load_floor[groups] = graph_seconds(
            [lambda i=i: tile_pass(i, ranges, groups) for i in range(8)], max(1, steps // 8))
    del rows_buf
    res = {
        "workload": "config 5: absorbed MLA decode, B=8, H=128, ctx 16384, latent 512+64 bf16 "
                    "in 64-token pages, 4 rotating input sets",
        "latent_and_merge_us": t * 1e6,
        "latent_and_merge_note": "the latent kernel and the merge of its range partials (two "
                                 "launches per step, graph replay); the latent kernel alone "
                                 "is in profiles/mla_config5.md's kernel trace",
        "hbm_gbs": nbytes / t / 1e9,
        "hbm_frac": nbytes / t / 1e9 / HBM_PEAK_GBS,
        "mfma_tflops": flops / t / 1e12,
        "mfma_frac_bf16_dense": flops / t / 1e12 / 2500.0,
        "bytes_per_call": nbytes,
        "flops_per_call": flops,
        "absorption_gemms_us": t_gemm * 1e6,
        "absorption_gemms_note": "q_nope . W_UK with q_rope (one launch) + weighted_c . W_UV "
                                 "(head_gemv), packed weights, 8 rotating weight sets",
        "stream_floor_us": t_floor * 1e6,
        "stream_floor_note": "one launch of a plain read kernel over one weight set's bytes "
                             "(16.8 MB), 8 rotating buffers: the floor of each absorption "
                             "product, so two dependent products cost at least twice this",
        "latent_load_floor_us": load_floor[2] * 1e6,
        "latent_load_floor_one_fill_us": load_floor[1] * 1e6,
        "latent_load_floor_note": "voom_tile_read: the latent kernel's loads alone (q rows, "
                                  "64-token tiles through two LDS buffers, fp16 partial-row "
                                  "stores), at its decomposition (16 ranges x 2 head groups "
                                  "filling each range's tiles) and with 32 ranges x 1 group "
                                  "(each tile filled once; twice the partials)",
        "decode_step_us": t_full * 1e6,
        "decode_step_note": "absorb_query + latent kernel + merge fused with the W_UV "
                            "projection (3 launches), rotating inputs and weights",
        "traffic": profiled_traffic("mla_config5"),
        "traffic_source": "rocprofv3 --pmc FETCH_SIZE/WRITE_SIZE, calibrated; "
                          "profiles/mla_config5.md (latent kernel + reduce)",
    }
    log(f"config 5: latent kernel + merge {t * 1e6:.1f} us, {res['hbm_gbs']:.0f} GB/s "
        f"({100 * res['hbm_frac']:.1f}% HBM), {res['mfma_tflops']:.0f} TFLOP/s; "
        f"absorption GEMMs {t_gemm * 1e6:.1f} us (one 16.8 MB streaming launch: "
        f"{t_floor * 1e6:.2f} us); whole decode step {t_full * 1e6:.1f} us; loads alone "
        f"{load_floor[2] * 1e6:.1f} us (one fill per tile: {load_floor[1] * 1e6:.1f} us)")
    if cpu_sample:
        from oracle import mla as omla

        info = set_cpu_threads()
        lat = torch.from_numpy(synthetic.mla_logical_latent(inp, 0)).to(torch.bfloat16)[None]
        ql = q_lats[0][0:1].cpu()
        n_cpu = 0
        t0 = time.perf_counter()
        while True:
            ref = omla.absorbed_weighted_c_torch(ql, lat, 64, inp.scale)
            n_cpu += 1
            dt = time.perf_counter() - t0
            if dt >= 10.0 or n_cpu >= 2000:
                break
        step(0)
        torch.cuda.synchronize()
        err = float((out[0].float().cpu() - ref[0]).abs().max())
        res["cpu_baseline"] = {"value": n_cpu * lat.numel() * 2 / dt / 1e9,
                               "unit": "GB/s (bf16 latent)",
                               "cores": info["threads"], "kind": "port",
                               "sample": f"{n_cpu} latent contractions of sequence 0 (16384 "
                                         "tokens, 128 heads): torch-CPU fp32 scores, bf16 "
                                         "softmax, P.c (oracle/mla.py; reference-algorithm "
                                         "CPU restatement)",
                               "seconds": dt, **info}
        res["parity_max_abs_err_vs_oracle"] = err
    del sets
    torch.cuda.empty_cache()
    return res


def bench_position_free(steps: int, warmup: int, cpu_sample: bool) -> dict:
    """Position-free decode: Llama-3-8B shape, one request,
    32768 keys in one-token pages drawn at random from a 40000-page pool,
    keys stored before RoPE and rotated in the kernel at positions 0..32767,
    one query at position 32767.  Four rotating page pools (4 x 164 MB) keep the
    working set out of the Infinity Cache.

    Algorithmic bytes per key: K + V rows of all 8 KV heads (4096 B), its table
    entry and position (8 B) and its cos/sin rows (2 x 64 fp32 = 512 B)."""
    import numpy as np
    import torch

    from voom_amd import calibrate, ops

    NQ, NKV, D, TK, P = 32, 8, 128, 32768, 40000
    log("position-free: 4 rotating pools of 40000 one-token pages, 32768 keys, 32q/8kv, D=128")
    sets = []
    for i in range(4):
        g = torch.Generator().manual_seed(30 + i)
        kp = torch.randn((P, NKV, 1, D), generator=g).to(torch.bfloat16).cuda()
        vp = torch.randn((P, NKV, 1, D), generator=g).to(torch.bfloat16).cuda()
        table = torch.randperm(P, generator=g)[:TK].to(torch.int32).cuda()
        q = torch.randn((1, NQ, 1, D), generator=g).to(torch.bfloat16).cuda()
        sets.append((q, kp, vp, table))
    kpos = torch.arange(TK, dtype=torch.int32, device="cuda")
    qpos = torch.tensor([TK - 1], dtype=torch.int32, device="cuda")
    cos, sin = ops.rope_cache(TK, D, 500000.0, device="cuda")
    scale = D ** -0.5

    def step(i):
        q, kp, vp, table = sets[i % 4]
        return ops.position_free_paged_attention(q, kp, vp, table, kpos, qpos, cos, sin,
                                                 scale=scale)

    for i in range(max(warmup, 4)):
        step(i)
    torch.cuda.synchronize()
    t = graph_seconds([lambda i=i: step(i) for i in range(4)], max(1, steps // 4))
    nbytes = TK * (2 * NKV * D * 2 + 8 + D * 4) + 2 * NQ * D * 2
    res = {
        "workload": "position-free decode: B=1, 32q/8kv, D=128, 32768 keys in one-token pages "
                    "(random ids from 40000), in-kernel RoPE theta 5e5, 4 rotating pools",
        "op_us": t * 1e6,
        "hbm_gbs": nbytes / t / 1e9,
        "hbm_frac": nbytes / t / 1e9 / HBM_PEAK_GBS,
        "bytes_per_call": nbytes,
        "traffic": profiled_traffic("position_free_decode"),
        "traffic_source": "rocprofv3 --pmc FETCH_SIZE/WRITE_SIZE, calibrated; "
                          "profiles/position_free_decode.md (attention kernel)",
    }
    # the floor of this page pattern: a plain gather kernel reading the same
    # K and V page rows (2 KiB each, the call's table), nothing else
    sink = torch.zeros(2048, dtype=torch.int32, device="cuda")

    def gather(i):
        q, kp, vp, table = sets[i % 4]
        calibrate.gather_read(kp, table, sink, base2=vp, workgroups=2048)

    for i in range(4):
        gather(i)
    torch.cuda.synchronize()
    t_g = graph_seconds([lambda i=i: gather(i) for i in range(4)], max(1, steps // 4))
    g_bytes = TK * 2 * NKV * D * 2
    res["page_gather_floor_us"] = t_g * 1e6
    res["page_gather_floor_gbs"] = g_bytes / t_g / 1e9
    res["page_gather_floor_note"] = ("plain gather kernel over the same K and V page rows "
                                     "(one launch, 4 KiB per key): the rate this page "
                                     "pattern delivers without any compute")
    res["frac_of_page_gather_floor"] = res["hbm_gbs"] / res["page_gather_floor_gbs"]
    log(f"position-free: {t * 1e6:.1f} us per call, {res['hbm_gbs']:.0f} GB/s "
        f"({100 * res['hbm_frac']:.1f}% HBM); a plain gather of the same K/V pages runs at "
        f"{res['page_gather_floor_gbs']:.0f} GB/s")
    if cpu_sample:
        from oracle import position_free as opf

        info = set_cpu_threads()
        q, kp, vp, table = sets[0]
        args_t = tuple(x.cpu() for x in (q, kp, vp, table, kpos, qpos, cos, sin))
        n_cpu = 0
        t0 = time.perf_counter()
        while True:
            ref_t = opf.attention_torch(*args_t, scale)
            n_cpu += 1
            dt = time.perf_counter() - t0
            if dt >= 10.0 or n_cpu >= 2000:
                break
        out = step(0)
        torch.cuda.synchronize()
        res["cpu_baseline"] = {"value": n_cpu * TK / dt, "unit": "keys/s (all 8 KV heads)",
                               "cores": info["threads"], "kind": "port",
                               "sample": f"{n_cpu} full calls (32768 keys each) in torch on the "
                                         "CPU: table gather, fp32 rotation rounded to bf16, "
                                         "masked fp32 SDPA (oracle/position_free.py "
                                         "attention_torch; reference-algorithm CPU "
                                         "restatement)",
                               "seconds": dt, **info}
        res["gpu_keys_per_s"] = TK / t
        args_np = (q.float().cpu().numpy(), kp.float().cpu().numpy(), vp.float().cpu().numpy(),
                   table.cpu().numpy().astype(np.int64), kpos.cpu().numpy().astype(np.int64),
                   qpos.cpu().numpy().astype(np.int64), cos.cpu().numpy(), sin.cpu().numpy())
        ref = opf.attention(*args_np, scale)
        res["parity_max_abs_err_vs_oracle"] = float(
            np.abs(out.float().cpu().numpy() - ref).max())
        res["cpu_torch_max_abs_err_vs_oracle"] = float(np.abs(ref_t.numpy() - ref).max())
    del sets
    torch.cuda.empty_cache()
    return res


def bench_dsa(steps: int, warmup: int, cpu_sample: bool) -> dict:
    """DSA decode step: B=1, 131,072 cached tokens, index
    keys [131072, 128] bf16, 32 index heads, top-2048, then the absorbed-MLA
    contraction (128 heads, latent 576 in 64-token pages) over the selected
    rows only.  Eight rotating index-key sets (8 x 33.5 MB) keep the scoring
    kernel's reads out of the Infinity Cache.  Each stage is timed with HIP
    events around replays of its own captured graph; the scoring kernel's
    algorithmic bytes are the index keys (256 B per token) plus q, w and the
    scores it writes (4 B per token)."""
    import numpy as np
    import torch

    from voom_amd import ops, synthetic

    S, NH, K, H = 131072, 32, 2048, 128
    log("dsa: 8 rotating index-key sets of 131072 x 128 bf16, top-2048, 128 MLA heads")
    g = torch.Generator(device="cuda").manual_seed(40)
    keys = [torch.randn((1, S, 128), generator=g, device="cuda").to(torch.bfloat16)
            for _ in range(8)]
    q_idx = torch.randn((1, NH, 128), generator=g, device="cuda").to(torch.bfloat16)
    w_head = (torch.randn((1, NH), generator=g, device="cuda") * NH ** -0.5).float()
    lens = torch.tensor([S], dtype=torch.int32, device="cuda")
    # one score row and one selection per key set, so that the selections and
    # the sparse contractions of a graph differ from call to call
    scores_all = [torch.empty((1, S), dtype=torch.float32, device="cuda") for _ in range(8)]
    scores = scores_all[0]
    inp = synthetic.mla_decode_inputs(batch=1, heads=H, ctx=S, seed=41)
    w_uk, _ = ops.split_kv_b(inp.kv_b, H, inp.dn, inp.dv)
    q_abs = torch.bmm(inp.q_nope.transpose(0, 1).contiguous(), w_uk).transpose(0, 1)
    q_lat = torch.cat([q_abs, inp.q_rope], -1).contiguous()
    out_c = torch.empty((1, H, 512), dtype=torch.bfloat16, device="cuda")

    sel_all = [torch.empty((1, K), dtype=torch.int32, device="cuda") for _ in range(8)]
    lens_all = [torch.empty((1,), dtype=torch.int32, device="cuda") for _ in range(8)]
    sel, sel_lens = sel_all[0], lens_all[0]

    def scores_of(i):
        ops.dsa_index_scores(q_idx, w_head, keys[i % 8], lens, scale=128 ** -0.5,
                             out=scores_all[i % 8])

    def select(i=0):
        ops.dsa_topk(scores_all[i % 8], lens, K, sel=sel_all[i % 8], sel_lens=lens_all[i % 8])

    def contract(i=0):
        ops.mla_sparse_decode(q_lat, inp.lat_pool, inp.block_table, sel_all[i % 8],
                              lens_all[i % 8], scale=inp.scale, out=out_c)

    for i in range(max(warmup, 8)):
        scores_of(i)
        select(i)
        contract(i)
    torch.cuda.synchronize()
    # each stage from its own graph of eight calls over the eight key sets (a
    # graph replay costs more than one of these short calls: one call per
    # graph would time the replay, not the call)
    reps = max(1, steps // 8)
    t_sc = graph_seconds([lambda i=i: scores_of(i) for i in range(8)], reps)
    t_tk = graph_seconds([lambda i=i: select(i) for i in range(8)], reps)
    t_mla = graph_seconds([lambda i=i: contract(i) for i in range(8)], reps)
    sc_bytes = S * 128 * 2 + NH * 128 * 2 + NH * 4 + S * 4
    sel_bytes = K * 576 * 2 + H * 576 * 2 + H * 512 * 2 + K * 4
    # the dense contraction the selection replaces, same cache
    def dense():
        ops.mla_latent_decode(q_lat, inp.lat_pool, inp.block_table, inp.ctx_lens,
                              scale=inp.scale, out=out_c)

    dense()
    t_dense = graph_seconds([dense] * 4, max(1, steps // 4))
    res = {
        "workload": "DSA decode: B=1, 131072 cached tokens, index 32 heads x 128 bf16, top-2048, "
                    "absorbed MLA 128 heads over the selected latent rows (64-token pages)",
        "index_scores_us": t_sc * 1e6,
        "index_scores_gbs": sc_bytes / t_sc / 1e9,
        "index_scores_hbm_frac": sc_bytes / t_sc / 1e9 / HBM_PEAK_GBS,
        "topk_us": t_tk * 1e6,
        "sparse_mla_us": t_mla * 1e6,
        "step_us": (t_sc + t_tk + t_mla) * 1e6,
        "dense_mla_same_cache_us": t_dense * 1e6,
        "index_scores_bytes": sc_bytes,
        "sparse_mla_bytes": sel_bytes,
    }
    log(f"dsa: scores {t_sc * 1e6:.1f} us ({res['index_scores_gbs']:.0f} GB/s), top-k "
        f"{t_tk * 1e6:.1f} us, sparse MLA {t_mla * 1e6:.1f} us; dense MLA over all "
        f"{S} tokens {t_dense * 1e6:.1f} us")
    if cpu_sample:
        from oracle import dsa as odsa

        # the selection checked is the one made from the key set it is
        # compared against: score and select key set 0 once more first
        scores_of(0)
        select(0)
        torch.cuda.synchronize()
        kk = keys[0][0].float().cpu().numpy()
        qq = q_idx[0].float().cpu().numpy()
        ww = w_head[0].cpu().numpy()
        ref = odsa.select(qq, ww, kk, S, K, 128 ** -0.5)
        ref_sc = odsa.index_scores(qq, ww, kk, 128 ** -0.5)
        kth = np.sort(ref_sc)[::-1][K - 1]
        got = set(sel[0].cpu().numpy().tolist())
        off = [i for i in got ^ set(ref.tolist())
               if abs(ref_sc[i] - kth) > 1e-5 * abs(kth) + 1e-5]
        info = set_cpu_threads()
        k_t, q_t, w_t = keys[0][0].cpu(), q_idx[0].cpu(), w_head[0].cpu()
        n_cpu = 0
        t0 = time.perf_counter()
        while True:
            odsa.select_torch(q_t, w_t, k_t, K, 128 ** -0.5)
            n_cpu += 1
            dt = time.perf_counter() - t0
            if dt >= 10.0 or n_cpu >= 5000:
                break
        res["cpu_baseline"] = {"value": n_cpu * S / dt, "unit": "keys/s (scores + top-k)",
                               "cores": info["threads"], "kind": "port",
                               "sample": f"{n_cpu} selections over 131072 keys in torch on the "
                                         "CPU (relu-weighted index scores, top-2048; "
                                         "oracle/dsa.py select_torch; reference-algorithm CPU "
                                         "restatement)",
                               "seconds": dt, **info}
        res["selection_matches_oracle"] = not off
    del keys
    torch.cuda.empty_cache()
    return res


def bench_e2e(cpu_sample: bool) -> dict:
    """Config 1: SmolLM2-135M-shaped decoder, random N(0, 0.02) bf16 weights
    (seed 0), a 512-token prompt of uniform ids (seed 1), greedy decode of 128
    tokens through PagedKVCache with 64-token pages and no spill.  Decode is
    launch- and weight-bandwidth-bound: the roofline figure is the weight bytes
    read per token over the per-token time."""
    import torch

    from voom_amd.decoder import DecoderConfig, PagedDecoder, random_weights

    cfg = DecoderConfig()
    log("config 1: SmolLM2-135M-shaped decoder, 512-token prompt, 128 greedy tokens")
    weights = random_weights(cfg, seed=0)
    dec = PagedDecoder(cfg, weights)
    prompt = torch.randint(0, cfg.vocab_size, (1, 512), generator=torch.Generator().manual_seed(1))
    dec.generate(prompt[:, :64], 4, dec.new_cache())  # warm the GEMM heuristics
    dec.generate_graph(prompt[:, :64], 4, dec.new_cache())
    torch.cuda.synchronize()
    # eager loop (one host-driven forward per token)
    kv_e = dec.new_cache(page_positions=64)
    toks_e, _, times_e = dec.generate(prompt, 128, kv_e)
    # the same loop with every decode step replayed from one captured HIP graph
    kv = dec.new_cache(page_positions=64)
    toks, prefill_s, times = dec.generate_graph(prompt, 128, kv)
    decode_s = sum(times)
    tok_s = len(times) / decode_s
    weight_bytes = cfg.param_count * 2
    res = {
        "workload": "config 1: SmolLM2-135M-shaped decoder (30 layers, 9q/3kv, D=64), random "
                    "N(0,0.02) bf16 weights seed 0, 512-token prompt seed 1, greedy 128 tokens, "
                    "PagedKVCache 64-token pages, no spill; decode steps replayed from a "
                    "captured HIP graph",
        "decode_tokens_per_s": tok_s,
        "ms_per_token": 1e3 * decode_s / len(times),
        "eager_decode_tokens_per_s": len(times_e) / sum(times_e),
        "eager_ms_per_token": 1e3 * sum(times_e) / len(times_e),
        "graph_tokens_equal_eager": toks == toks_e,
        "prefill_ms": prefill_s * 1e3,
        "prefill_tokens_per_s": 512 / prefill_s,
        "weight_gbs_per_token": weight_bytes * tok_s / 1e9,
        "weight_hbm_frac": weight_bytes * tok_s / 1e9 / HBM_PEAK_GBS,
        "kv_pages": sum(len(p) for p in kv._pages),
        "first_tokens": toks[:8],
    }
    log(f"config 1: prefill {prefill_s * 1e3:.1f} ms, decode {res['ms_per_token']:.3f} ms/token "
        f"({tok_s:.1f} tok/s) with the graph, eager {res['eager_ms_per_token']:.2f} ms/token; "
        f"tokens equal: {toks == toks_e}")
    if cpu_sample:
        from transformers import LlamaConfig, LlamaForCausalLM

        hcfg = LlamaConfig(vocab_size=cfg.vocab_size, hidden_size=cfg.hidden_size,
                           intermediate_size=cfg.intermediate_size,
                           num_hidden_layers=cfg.num_hidden_layers,
                           num_attention_heads=cfg.num_attention_heads,
                           num_key_value_heads=cfg.num_key_value_heads, head_dim=cfg.head_dim,
                           rms_norm_eps=cfg.rms_norm_eps, rope_theta=cfg.rope_theta,
                           tie_word_embeddings=True, max_position_embeddings=4096)
        m = LlamaForCausalLM(hcfg).eval()
        m.load_state_dict({k: v.float() for k, v in weights.items()}, strict=False)
        n_cpu = 16
        with torch.no_grad():
            out = m(prompt, use_cache=True)
            past = out.past_key_values
            nxt = int(out.logits[0, -1].argmax())
            ref_toks = [nxt]
            t0 = time.perf_counter()
            for _ in range(n_cpu):
                out = m(torch.tensor([[nxt]]), past_key_values=past, use_cache=True)
                past = out.past_key_values
                nxt = int(out.logits[0, -1].argmax())
                ref_toks.append(nxt)
            dt = time.perf_counter() - t0
        agree = 0
        for a, b in zip(toks, ref_toks):
            if a != b:
                break
            agree += 1
        # The random-init model's greedy stream is nearly constant, so the
        # greedy agreement pins little: teacher-force 16 random tokens after
        # the prompt through both models and compare every logit row (the
        # prompt's 512 rows from the paged prefill, the 16 decode rows from
        # the captured graph the timing replays).
        forced = torch.randint(0, cfg.vocab_size, (16,), generator=torch.Generator().manual_seed(7))
        with torch.no_grad():
            out = m(prompt, use_cache=True)
            ref_rows = [out.logits[0]]
            past = out.past_key_values
            for t in forced.tolist():
                out = m(torch.tensor([[t]]), past_key_values=past, use_cache=True)
                past = out.past_key_values
                ref_rows.append(out.logits[0])
        ref_l = torch.cat(ref_rows).numpy()                 # 512 + 16 rows
        kv_t = dec.new_cache(page_positions=64)
        got_rows = [dec.forward(prompt.cuda(), kv_t)[0].cpu()]
        logits = torch.empty((1, cfg.vocab_size), dtype=torch.float32, device="cuda")
        graph, tok, _ = dec.capture_decode(kv_t, 512 + 16, logits=logits)
        # row 512 + i is the logits after forced token i; the decode input
        # of step i is forced[i]
        for t in forced.tolist():
            tok.fill_(t)
            graph.replay()
            kv_t.advance(1)
            got_rows.append(logits.cpu().clone())
        got_l = torch.cat(got_rows).numpy()
        import numpy as np

        rel = np.linalg.norm(got_l - ref_l, axis=-1) / np.linalg.norm(ref_l, axis=-1)
        res["teacher_forced_vs_cpu_fp32"] = {
            "rows": int(ref_l.shape[0]),
            "rel_l2_max": float(rel.max()),
            "abs_max": float(np.abs(got_l - ref_l).max()),
            "argmax_agreement": float((got_l.argmax(-1) == ref_l.argmax(-1)).mean()),
            "distinct_reference_argmax": int(len(set(ref_l.argmax(-1).tolist()))),
        }
        del graph, kv_t
        res["cpu_baseline"] = {"value": n_cpu / dt, "unit": "tokens/s (decode)",
                               "cores": torch.get_num_threads(), "kind": "port",
                               "sample": f"{n_cpu} greedy decode steps after the same 512-token "
                                         "prompt, Hugging Face LlamaForCausalLM fp32 on the "
                                         "host CPU with its KV cache"}
        res["greedy_prefix_agreement_vs_cpu_fp32"] = agree
        res["greedy_distinct_tokens"] = len(set(toks))
        tf = res["teacher_forced_vs_cpu_fp32"]
        log(f"config 1: cpu baseline {n_cpu / dt:.1f} tok/s; greedy tokens agree for the first "
            f"{agree} of {len(ref_toks)} ({len(set(toks))} distinct tokens in the GPU stream); "
            f"teacher-forced over {tf['rows']} rows: rel L2 max {tf['rel_l2_max']:.4f}, "
            f"argmax agreement {tf['argmax_agreement']:.3f} "
            f"({tf['distinct_reference_argmax']} distinct reference argmax)")
    del dec, weights, kv, kv_e
    torch.cuda.empty_cache()
    return res


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--only", default="gqa,spill,long,mla,pf,dsa,e2e",
                    help="comma list of legs: gqa (config 2, headline), spill (config 3), "
                         "long (config 4), mla (config 5), pf (position-free), dsa (DSA decode), "
                         "e2e (config 1)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run a known-size 1 GiB streaming kernel (PMC byte-counter calibration)")
    ap.add_argument("--gather-floor", action="store_true",
                    help="also time the calibration gather over config 2's own K/V blocks")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this build measures one GPU only; sharding the paged-KV path over "
              "several GPUs is designed but not built.", file=sys.stderr)
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py: no ROCm GPU visible", file=sys.stderr)
        return 1
    if args.copy_calibration:
        copy_calibration()
    gqa = bench_gqa(args.steps, args.warmup, cpu_sample=not args.no_cpu,
                    gather_floor=args.gather_floor)
    line = {
        "metric": "paged decode-attn HBM GB/s (% peak) + spill/reload GB/s, Llama-3-8B shape",
        "value": round(gqa["value"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(gqa["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "paged GQA decode attention, Llama-3-8B shape (config 2)",
            "batch": 16, "num_q_heads": 32, "num_kv_heads": 8, "head_dim": 128,
            "page_tokens": 64, "ctx": "U[1024,32768] seed 2",
            "context_tokens": gqa["context_tokens"],
            "bytes_per_step": gqa["bytes_per_step"],
            "seeds": {"ctx": 2, "kv": 3, "rope_pos": 4, "slots": 5},
        },
        "roofline": gqa["roofline"],
        "cpu_baseline": gqa.get("cpu_baseline"),
        "pct_hbm_peak": round(100 * gqa["value"] / HBM_PEAK_GBS, 2),
        "op_avg_us": round(gqa["op_avg_us"], 2),
        "op_gbs": round(gqa["op_gbs"], 2),
        "combine_avg_us": round(gqa["combine_avg_us"], 2),
    }
    if "parity_max_abs_err_vs_oracle" in gqa:
        line["parity_max_abs_err_vs_oracle"] = gqa["parity_max_abs_err_vs_oracle"]
    if "page_gather_floor" in gqa:
        line["page_gather_floor"] = {k: round(v, 2) for k, v in gqa["page_gather_floor"].items()}
    legs = set(args.only.split(","))
    extra = {}
    if "spill" in legs:
        extra["spill_reload"] = bench_spill_reload(cpu_sample=not args.no_cpu)
        line["spill_gbs"] = round(extra["spill_reload"]["spill_gbs"], 2)
        line["reload_gbs"] = round(extra["spill_reload"]["reload_gbs"], 2)
    if "long" in legs:
        extra["long_context"] = bench_long_context(64, cpu_sample=not args.no_cpu)
    if "mla" in legs:
        extra["mla"] = bench_mla(args.steps, args.warmup, cpu_sample=not args.no_cpu)
    if "pf" in legs:
        extra["position_free"] = bench_position_free(args.steps, args.warmup,
                                                     cpu_sample=not args.no_cpu)
    if "dsa" in legs:
        extra["dsa"] = bench_dsa(args.steps, args.warmup, cpu_sample=not args.no_cpu)
    if "e2e" in legs:
        extra["e2e"] = bench_e2e(cpu_sample=not args.no_cpu)
    if extra:
        line["other_configs"] = extra
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
