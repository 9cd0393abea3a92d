#!/usr/bin/env python3
"""Benchmark of the MI355X quantized-matrix path (one JSON line on stdout).

A step is one pass of the hot path over one batch of synthetic input.  The
headline workload is BASELINE configs[1] (C2): the Q6_K output head,
151936 x 4096, batch 1, GEMV plus the greedy argmax, with weights and
activation resident in HBM before the timed region.  ``value`` is the
algorithmic bytes of a step divided by the wall time per step on the
compute stream (HIP events, all launches of the step included).

``roofline`` describes the dominant kernel, the one the timed step runs
(the int8 Q6_K GEMV with the argmax folded into its epilogue, one launch per
step): its average launch duration is the region time per step of the
back-to-back timed loop; ``traffic`` is the HBM bytes per launch from
rocprofv3 FETCH_SIZE/WRITE_SIZE runs (profiles/), when present.

``cpu_baseline`` times the CPU port of src/cpu.rs (oracle/dm_oracle.c) on
the same C2 workload, on this machine's host cores, with the thread count
rayon's default pool would take (std::thread::available_parallelism).

``details`` holds the other BASELINE configurations (C1, C3, C4, C5), each
measured the same way, a Q8_0 GEMV entry (the third k-quant of the north
star, which no configuration uses) and F16 / F32 / Q5_0 GEMV entries (the
other row types of a Gemma-class GGUF).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--only c1|c2|c3|c4|c5|q8|dense|st|attn|attn_host|host|copy]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "Q4_K/Q6_K GEMV achieved HBM GB/s (% peak); prefill GEMM TFLOP/s; decode tok/s"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
Q4_K, Q6_K, Q8_0 = 12, 14, 8


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class Timed:
    """Wall time of the enclosed work on the compute stream: an event before
    and after it, nothing else recorded.  Kernel durations come from the
    rocprofv3 kernel traces in profiles/, not from this program."""

    def __init__(self, ctx):
        self.ctx = ctx

    def __enter__(self):
        self.ctx.synchronize()
        self.start = self.ctx.event_record()
        return self

    def __exit__(self, *exc):
        stop = self.ctx.event_record()
        self.ctx.synchronize()
        self.wall_ms = self.ctx.event_elapsed_ms(self.start, stop)
        self.ctx.event_free(self.start)
        self.ctx.event_free(stop)


def timed_loop(ctx, body, steps):
    """Wall ms on the compute stream of `steps` calls of body(i)."""
    with Timed(ctx) as wall:
        for i in range(steps):
            body(i)
    return wall.wall_ms


def upload(ctx, arr):
    return ctx.device_array(np.ascontiguousarray(arr))


# ---------------------------------------------------------------------------
def bench_c2(ctx, synth, steps, warmup):
    rows, cols = 151936, 4096
    log("C2: generating weights")
    w = synth.quantized_matrix(Q6_K, rows, cols, synth.weight_seed(2))
    x = synth.normal(synth.activation_seed(2), cols)
    wb, xb = upload(ctx, w), upload(ctx, x)
    yb, ib = ctx.new_owned_buffer(rows * 4), ctx.new_owned_buffer(4)
    step_bytes = w.size + cols * 4 + rows * 4  # 511,129,088 B
    for _ in range(warmup):
        ctx.matvec_argmax_device(Q6_K, rows, cols, wb.device_ptr, xb.device_ptr, yb.device_ptr, ib.device_ptr)
    idx = ctx.argmax_result()
    # The box slows by several percent within milliseconds of sustained load:
    # each timed pass starts after the same short idle period.
    time.sleep(0.2)
    with Timed(ctx) as t:
        for _ in range(steps):
            ctx.matvec_argmax_device(Q6_K, rows, cols, wb.device_ptr, xb.device_ptr, yb.device_ptr, ib.device_ptr)
    ms = t.wall_ms / steps
    # A step is one launch (the int8 GEMV with the argmax folded into its
    # epilogue), back to back: the region time per step is that kernel's
    # average launch duration plus the dispatch gap, so the roofline figure
    # is the timed step's kernel.  The kernel without the argmax epilogue
    # (matvec_device) is timed the same way for comparison.
    ctx.matvec_device(Q6_K, rows, cols, wb.device_ptr, 1, xb.device_ptr, yb.device_ptr)
    ctx.synchronize()
    time.sleep(0.2)
    with Timed(ctx) as k:
        for _ in range(steps):
            ctx.matvec_device(Q6_K, rows, cols, wb.device_ptr, 1, xb.device_ptr, yb.device_ptr)
    kms = k.wall_ms / steps
    log(f"C2: {ms * 1e3:.1f} us/step, GEMV kernel {kms * 1e3:.1f} us per launch, argmax={idx}")
    return {
        "rows": rows, "columns": cols, "weight_bytes": int(w.size), "step_bytes": int(step_bytes),
        "ms_per_step": ms, "gbps": step_bytes / (ms * 1e-3) / 1e9,
        "gemv_no_argmax_ms": kms, "gemv_no_argmax_gbps": step_bytes / (kms * 1e-3) / 1e9, "argmax": int(idx),
    }, (w, x)


def bench_c1(ctx, synth, steps, warmup):
    rows = cols = 4096
    w = synth.quantized_matrix(Q4_K, rows, cols, synth.weight_seed(1))
    x = synth.normal(synth.activation_seed(1), cols)
    copies = 40  # 40 x 9.4 MB = 377 MB > 256 MB MALL: each launch reads from HBM
    wbs = [upload(ctx, w)]
    for _ in range(copies - 1):
        b = ctx.new_owned_buffer(w.size)
        ctx.copy_device(b.device_ptr, wbs[0].device_ptr, w.size)
        wbs.append(b)
    xb, yb = upload(ctx, x), ctx.new_owned_buffer(rows * 4)
    step_bytes = w.size + cols * 4 + rows * 4  # 9,469,952 B
    out = {"rows": rows, "columns": cols, "step_bytes": step_bytes}
    for mode, bufs in (("cold", wbs), ("warm", wbs[:1])):
        n = max(steps, 2 * copies)
        for i in range(warmup + 1):
            ctx.matvec_device(Q4_K, rows, cols, bufs[i % len(bufs)].device_ptr, 1, xb.device_ptr, yb.device_ptr)
        # one GEMV launch per step, back to back: the region time per launch
        # is the kernel's average launch duration
        with Timed(ctx) as t:
            for i in range(n):
                ctx.matvec_device(Q4_K, rows, cols, bufs[i % len(bufs)].device_ptr, 1, xb.device_ptr, yb.device_ptr)
        ms = t.wall_ms / n
        out[mode] = {"ms_per_step": ms, "gbps": step_bytes / (ms * 1e-3) / 1e9,
                     "frac_of_peak": step_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS}
    # Sustained: 8 distinct cold matrices sharing x in one grouped launch
    # (matvec_batch_device), so the ~2.4 us launch floor is paid once per 8
    # matvecs; and 16, a layer's same-input matvecs.  Time and bytes are
    # reported per matrix.
    for group, key in ((8, "sustained"), (16, "sustained_16")):
        yg = ctx.new_owned_buffer(group * rows * 4)
        sets = [[b.device_ptr for b in wbs[j * group:(j + 1) * group]] for j in range(copies // group)]
        for i in range(warmup + 1):
            ctx.matvec_batch_device(Q4_K, rows, cols, sets[i % len(sets)], xb.device_ptr, 0, yg.device_ptr, rows)
        n = max(steps, 2 * len(sets))
        with Timed(ctx) as t:
            for i in range(n):
                ctx.matvec_batch_device(Q4_K, rows, cols, sets[i % len(sets)], xb.device_ptr, 0, yg.device_ptr,
                                        rows)
        ms = t.wall_ms / (n * group)
        per = w.size + rows * 4 + cols * 4 / group
        out[key] = {"matrices_per_launch": group, "ms_per_matrix": ms, "bytes_per_matrix": per,
                    "gbps": per / (ms * 1e-3) / 1e9, "frac_of_peak": per / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS}
        yg.free()
    log(f"C1: cold {out['cold']['ms_per_step'] * 1e3:.2f} us per launch ({out['cold']['gbps']:.0f} GB/s); "
        f"sustained {out['sustained']['ms_per_matrix'] * 1e3:.2f} us per matrix ({out['sustained']['gbps']:.0f} GB/s), "
        f"{out['sustained_16']['ms_per_matrix'] * 1e3:.2f} us with 16 per launch "
        f"({out['sustained_16']['gbps']:.0f} GB/s)")
    out["floor"] = c1_floor(ctx, wbs, w.size, step_bytes, steps)
    return out


def c1_floor(ctx, wbs, wbytes, step_bytes, steps):
    """What bounds a single C1 launch: back-to-back durations of an empty
    kernel (256 x 256, the GEMV's grid) and of a kernel that only reads the
    same 9.4 MB (cold: rotating copies; warm: one copy), from the launch-floor
    probes of libdmhip_diag.so (include/dmhip_diag.h).  None when that
    library is not built."""
    import ctypes
    path = os.path.join(ROOT, "diskmule_amd", "libdmhip_diag.so")
    if not os.path.exists(path):
        return None
    lib = ctypes.CDLL(path)
    lib.dmhip_diag_time_empty.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_size_t,
                                          ctypes.POINTER(ctypes.c_double)]
    lib.dmhip_diag_time_read.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t, ctypes.c_size_t,
                                         ctypes.c_size_t, ctypes.POINTER(ctypes.c_double)]
    n = max(steps, 2 * len(wbs))
    ctx.synchronize()

    def read(bufs):
        us = ctypes.c_double()
        srcs = (ctypes.c_void_p * len(bufs))(*[b.device_ptr for b in bufs])
        assert lib.dmhip_diag_time_read(srcs, len(bufs), wbytes - wbytes % 16, n, ctypes.byref(us)) == 0
        return us.value

    empty = ctypes.c_double()
    assert lib.dmhip_diag_time_empty(256, 256, n, ctypes.byref(empty)) == 0
    res = {"empty_kernel_us": empty.value, "read_only_cold_us": read(wbs), "read_only_warm_us": read(wbs[:1])}
    res["read_only_cold_gbps"] = step_bytes / (res["read_only_cold_us"] * 1e-6) / 1e9
    log(f"C1 floor: empty {res['empty_kernel_us']:.2f} us, read-only cold {res['read_only_cold_us']:.2f} / warm "
        f"{res['read_only_warm_us']:.2f} us")
    return res


def bench_q8(ctx, synth, steps, warmup):
    """Q8_0 (named in the north star; no BASELINE config): batch-1 GEMV at the
    C2 and C1 shapes, weights resident, back-to-back launches."""
    Q8_0 = 8
    out = {}
    for rows, cols in ((151936, 4096), (4096, 4096)):
        w = synth.quantized_matrix(Q8_0, rows, cols, synth.weight_seed(8, rows))
        x = synth.normal(synth.activation_seed(8), cols)
        wb, xb, yb = upload(ctx, w), upload(ctx, x), ctx.new_owned_buffer(rows * 4)
        for _ in range(warmup):
            ctx.matvec_device(Q8_0, rows, cols, wb.device_ptr, 1, xb.device_ptr, yb.device_ptr)
        ctx.synchronize()
        time.sleep(0.2)
        with Timed(ctx) as t:
            for _ in range(steps):
                ctx.matvec_device(Q8_0, rows, cols, wb.device_ptr, 1, xb.device_ptr, yb.device_ptr)
        ms = t.wall_ms / steps
        step_bytes = w.size + 4 * cols + 4 * rows
        out[f"{rows}x{cols}"] = {"ms": ms, "gbps": step_bytes / (ms * 1e-3) / 1e9,
                                 "frac_of_peak": step_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS}
        log(f"Q8_0 {rows}x{cols}: {ms * 1e3:.1f} us per launch ({out[f'{rows}x{cols}']['gbps']:.0f} GB/s)")
    return out


def bench_dense(ctx, synth, steps, warmup):
    """The other GGUF row types a Gemma-class model holds (F16, F32, Q5_0;
    no BASELINE config): batch-1 GEMV at 12288 x 4096 and 4096 x 4096 (F32
    only the latter) over rotating copies (more than the 256 MB MALL),
    back-to-back launches."""
    out = {}
    for kind, tag, shapes in ((1, "F16", ((12288, 4096), (4096, 4096))), (0, "F32", ((4096, 4096),)),
                              (6, "Q5_0", ((12288, 4096), (4096, 4096)))):
        for rows, cols in shapes:
            w = synth.quantized_matrix(kind, rows, cols, synth.weight_seed(9, kind))
            x = synth.normal(synth.activation_seed(9), cols)
            copies = max(2, -(-300_000_000 // w.size))
            wbs = [upload(ctx, w)]
            for _ in range(copies - 1):
                b = ctx.new_owned_buffer(w.size)
                ctx.copy_device(b.device_ptr, wbs[0].device_ptr, w.size)
                wbs.append(b)
            xb, yb = upload(ctx, x), ctx.new_owned_buffer(rows * 4)
            n = max(steps, 2 * copies)
            for i in range(warmup):
                ctx.matvec_device(kind, rows, cols, wbs[i % copies].device_ptr, 1, xb.device_ptr, yb.device_ptr)
            ctx.synchronize()
            time.sleep(0.2)
            with Timed(ctx) as t:
                for i in range(n):
                    ctx.matvec_device(kind, rows, cols, wbs[i % copies].device_ptr, 1, xb.device_ptr, yb.device_ptr)
            ms = t.wall_ms / n
            step_bytes = w.size + 4 * cols + 4 * rows
            key = f"{tag}_{rows}x{cols}"
            out[key] = {"ms": ms, "gbps": step_bytes / (ms * 1e-3) / 1e9,
                        "frac_of_peak": step_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS}
            log(f"{key}: {ms * 1e3:.1f} us per launch ({out[key]['gbps']:.0f} GB/s)")
            for b in wbs:
                b.free()
    return out


def bench_c3(ctx, synth, steps, warmup):
    hidden, ffn = 4096, 12288
    g = synth.quantized_matrix(Q4_K, ffn, hidden, synth.weight_seed(3, 0))
    u = synth.quantized_matrix(Q4_K, ffn, hidden, synth.weight_seed(3, 1))
    d = synth.quantized_matrix(Q6_K, hidden, ffn, synth.weight_seed(3, 2))
    weight_bytes = g.size + u.size + d.size  # 97,910,784 B
    # 3 copies of the layer (294 MB > the 256 MB MALL): "cold" rotates them so
    # every call streams its weights from HBM; "warm" repeats copy 0.
    layers = [(upload(ctx, g), upload(ctx, u), upload(ctx, d))]
    for _ in range(2):
        copy = []
        for src, arr in zip(layers[0], (g, u, d)):
            b = ctx.new_owned_buffer(arr.size)
            ctx.copy_device(b.device_ptr, src.device_ptr, arr.size)
            copy.append(b)
        layers.append(tuple(copy))
    out = {}
    for batch in (1, 4, 8):
        h = synth.normal(synth.activation_seed(3, batch), batch * hidden)
        hb, yb = upload(ctx, h), ctx.new_owned_buffer(batch * hidden * 4)
        ws = ctx.new_owned_buffer(ctx.ffn_workspace_bytes(batch, hidden, ffn))

        def call(i, sets):
            gb, ub, db = sets[i % len(sets)]
            ctx.ffn_device(batch, hidden, ffn, Q4_K, gb.device_ptr, Q4_K, ub.device_ptr, Q6_K, db.device_ptr,
                           1e-6, hb.device_ptr, yb.device_ptr, ws.device_ptr, len(ws))

        step_bytes = weight_bytes + 2 * batch * hidden * 4
        res = {}
        for mode, sets in (("cold", layers), ("warm", layers[:1])):
            for i in range(warmup):
                call(i, sets)
            n = max(steps, 2 * len(sets))
            ms = timed_loop(ctx, lambda i: call(i, sets), n) / n
            res[mode] = {"layer_ms": ms, "gbps": step_bytes / (ms * 1e-3) / 1e9,
                         "frac_of_peak": step_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                         "tok_per_s": batch / (ms * 1e-3)}
        out[f"B{batch}"] = res
        log(f"C3 B={batch}: {res['cold']['layer_ms'] * 1e3:.1f} us/layer cold, "
            f"{res['warm']['layer_ms'] * 1e3:.1f} us warm")
    return out


def bench_c4(ctx, synth, steps, warmup):
    from diskmule_amd import ExpertCache, ExpertLayerLayout
    from diskmule_amd.hip import PinnedHostBuffer
    hidden, width, experts, k, slots = 2048, 768, 128, 8, 8
    router = synth.to_bf16_bits(synth.normal(synth.weight_seed(4, 9), experts * hidden) * np.float32(0.02))
    gu_bytes = 2 * width * synth.row_bytes(Q4_K, hidden)
    dn_bytes = hidden * synth.row_bytes(Q6_K, width)
    src = PinnedHostBuffer(experts * (gu_bytes + dn_bytes))
    src.array[:experts * gu_bytes] = synth.quantized_matrix(Q4_K, experts * 2 * width, hidden, synth.weight_seed(4, 0))
    src.array[experts * gu_bytes:] = synth.quantized_matrix(Q6_K, experts * hidden, width, synth.weight_seed(4, 1))
    layout = ExpertLayerLayout(experts, 0, gu_bytes, experts * gu_bytes, dn_bytes)
    rb = upload(ctx, router)
    out = {"expert_bytes": gu_bytes + dn_bytes, "slots_per_layer": slots}
    for batch in (1, 4, 16):
        cache = ExpertCache(ctx, src, [layout], slots)
        xs = [upload(ctx, synth.normal(synth.activation_seed(4, 100 * batch + i), batch * hidden))
              for i in range(steps + warmup)]
        yb = ctx.new_owned_buffer(batch * hidden * 4)
        for i in range(warmup):
            ctx.moe_layer(cache, 0, batch, hidden, width, experts, k, rb.device_ptr, Q4_K, Q6_K,
                          xs[i].device_ptr, yb.device_ptr)
        # Wall time of the layer calls (host clock: each call ends with the
        # host reading the router's selection).
        s0 = cache.stats()
        t0 = time.perf_counter()
        for i in range(warmup, warmup + steps):
            ctx.moe_layer(cache, 0, batch, hidden, width, experts, k, rb.device_ptr, Q4_K, Q6_K,
                          xs[i].device_ptr, yb.device_ptr)
        wall = time.perf_counter() - t0
        s1 = cache.stats()
        misses = s1["misses"] - s0["misses"]
        hits = s1["hits"] - s0["hits"]
        up_bytes = s1["bytes_read"] - s0["bytes_read"]
        layer = {
            "layer_ms": wall / steps * 1e3, "hits": hits, "misses": misses,
            "evictions": s1["evictions"] - s0["evictions"],
            "upload_bytes": up_bytes, "upload_gbps_wall": up_bytes / wall / 1e9,
        }
        cache.free()
        # All-resident layer: a cache with a slot for every expert, warmed
        # with the token's experts, then the same call repeated (no upload;
        # the eight-slot cache above cannot hold the 30+ distinct experts of
        # B = 4 or 16).  One token takes the device-side slot lookup here.
        cache = ExpertCache(ctx, src, [layout], experts)
        for _ in range(3):
            ctx.moe_layer(cache, 0, batch, hidden, width, experts, k, rb.device_ptr, Q4_K, Q6_K,
                          xs[0].device_ptr, yb.device_ptr)
        r0 = cache.stats()["misses"]
        # host clock around back-to-back synchronous calls (each returns after
        # its work is done)
        hot_calls = 20
        t0 = time.perf_counter()
        for _ in range(hot_calls):
            ids, _ = ctx.moe_layer(cache, 0, batch, hidden, width, experts, k, rb.device_ptr, Q4_K, Q6_K,
                                   xs[0].device_ptr, yb.device_ptr)
        hot_ms = (time.perf_counter() - t0) / hot_calls * 1e3
        assert cache.stats()["misses"] == r0, "the all-resident pass loaded an expert"
        # The same, over the distinct token batches of the timed pass in turn
        # (a decode step never repeats its input): the router's exact fold of
        # the rows its bounds cannot order runs for the tokens that need it
        # (about 2% of tokens on this data) instead of on every call or none.
        for x in xs:
            ctx.moe_layer(cache, 0, batch, hidden, width, experts, k, rb.device_ptr, Q4_K, Q6_K, x.device_ptr,
                          yb.device_ptr)
        r1 = cache.stats()["misses"]
        t0 = time.perf_counter()
        for i in range(hot_calls):
            ctx.moe_layer(cache, 0, batch, hidden, width, experts, k, rb.device_ptr, Q4_K, Q6_K,
                          xs[i % len(xs)].device_ptr, yb.device_ptr)
        rot_ms = (time.perf_counter() - t0) / hot_calls * 1e3
        assert cache.stats()["misses"] == r1, "the all-resident pass loaded an expert"
        layer.update({
            "all_resident_layer_ms": hot_ms,
            "all_resident_calls": hot_calls,
            "all_resident_experts": len(set(ids.ravel().tolist())),
            "all_resident_distinct_inputs_layer_ms": rot_ms,
            "all_resident_distinct_inputs": min(hot_calls, len(xs)),
        })
        out[f"B{batch}"] = layer
        log(f"C4 B={batch}: {wall / steps * 1e3:.2f} ms/layer, misses {misses}, hits {hits}; all-resident "
            f"{hot_ms:.3f} ms (one input), {rot_ms:.3f} ms (distinct inputs)")
        cache.free()
    # Upload link rate on its own: one expert from pinned memory per copy.
    dst = ctx.new_owned_buffer(gu_bytes + dn_bytes)
    n = 32
    t0 = time.perf_counter()
    for i in range(n):
        ctx.copy_to_device(dst.device_ptr, src.array[i * gu_bytes:(i + 1) * gu_bytes])
    out["pinned_h2d_gbps"] = n * gu_bytes / (time.perf_counter() - t0) / 1e9
    src.free()
    return out


def bench_host(ctx, synth, steps, warmup):
    """The drop-in host-slice path an unchanged graph takes (src/metal.rs:
    1562-1604, :1801-1882: host x in, host y out, synchronous per call):
    matvec_mapped at the C1 and C2 shapes over a mapped GGUF-like buffer, and
    at the C4 shape one routed expert as the Gemma 4 graph runs it
    (src/gemma4/metal.rs:1003-1031): acquire -> matvec_owned gate_up ->
    silu_mul -> matvec_owned down -> release, all slots resident.  Host clock
    per call, next to the device-resident kernel time of the same shape
    (matvec_device, events, back to back)."""
    from diskmule_amd import ExpertCache, ExpertLayerLayout
    out = {}
    for tag, kind, rows, cols in (("C1", Q4_K, 4096, 4096), ("C2", Q6_K, 151936, 4096)):
        w = synth.quantized_matrix(kind, rows, cols, synth.weight_seed(1 if tag == "C1" else 2))
        x = synth.normal(synth.activation_seed(1 if tag == "C1" else 2), cols)
        mb = ctx.map_read_only(w)
        y = np.zeros(rows, np.float32)
        for _ in range(warmup + 2):
            ctx.matvec_mapped(kind, rows, cols, mb, 0, w.size, x, y)
        n = max(steps, 50 if tag == "C1" else 20)
        t0 = time.perf_counter()
        for _ in range(n):
            ctx.matvec_mapped(kind, rows, cols, mb, 0, w.size, x, y)
        call_us = (time.perf_counter() - t0) / n * 1e6
        xb, yb = upload(ctx, x), ctx.new_owned_buffer(rows * 4)
        dev_us = timed_loop(ctx, lambda i: ctx.matvec_device(kind, rows, cols, mb.device_ptr, 1, xb.device_ptr,
                                                              yb.device_ptr), n) / n * 1e3
        out[tag] = {"rows": rows, "columns": cols, "call_us": call_us, "device_kernel_us": dev_us,
                    "host_overhead_us": call_us - dev_us}
        log(f"host-slice {tag}: matvec_mapped {call_us:.1f} us per call, device-resident {dev_us:.1f} us")
        for b in (mb, xb, yb):
            b.free()
    hidden, width, experts, slots = 2048, 768, 16, 8
    gu_bytes = 2 * width * synth.row_bytes(Q4_K, hidden)
    dn_bytes = hidden * synth.row_bytes(Q6_K, width)
    gu = synth.quantized_matrix(Q4_K, experts * 2 * width, hidden, synth.weight_seed(4, 0))
    dn = synth.quantized_matrix(Q6_K, experts * hidden, width, synth.weight_seed(4, 1))
    src = np.concatenate([gu, dn])
    cache = ExpertCache(ctx, src, [ExpertLayerLayout(experts, 0, gu_bytes, gu.size, dn_bytes)], slots)
    x = synth.normal(synth.activation_seed(4, 7), hidden)
    g_u = np.zeros(2 * width, np.float32)
    act = np.zeros(width, np.float32)
    y = np.zeros(hidden, np.float32)

    def expert(e):
        slot, gub, dnb = cache.acquire(0, e)
        ctx.matvec_owned(Q4_K, 2 * width, hidden, gub, 0, gu_bytes, x, g_u)
        ctx.silu_mul(g_u[:width], g_u[width:], act)
        ctx.matvec_owned(Q6_K, hidden, width, dnb, 0, dn_bytes, act, y)
        cache.release(0, slot)

    for e in range(slots):
        expert(e)
    n = max(steps, 40)
    t0 = time.perf_counter()
    for i in range(n):
        expert(i % slots)
    out["C4_expert"] = {"per_expert_us": (time.perf_counter() - t0) / n * 1e6, "calls_per_expert": 3,
                        "note": "acquire (hit), matvec_owned gate_up 1536x2048 Q4_K, silu_mul, matvec_owned "
                                "down 2048x768 Q6_K, release"}
    log(f"host-slice C4 expert: {out['C4_expert']['per_expert_us']:.1f} us per expert (3 synchronous calls)")
    cache.free()
    return out


def bench_c5(ctx, synth, steps, warmup):
    """C5: 512-token prefill GEMM at K = 4096, N = 4096 and 12288, for Q4_K
    (the headline) and the other two quantized types of the path.  `ms` is
    the whole call (A preparation + GEMM); the GEMM kernel alone is in the
    kernel trace of profiles/c5_gemm_kernel_stats.md."""
    m, k = 512, 4096
    a = synth.to_bf16_bits(synth.normal(synth.activation_seed(5), m * k))
    ab = upload(ctx, a)
    ws = ctx.new_owned_buffer(ctx.gemm_workspace_bytes(m, k))
    out = {}
    for kind, tag in ((Q4_K, ""), (Q6_K, "_q6_k"), (Q8_0, "_q8_0")):
        for n in (4096, 12288):
            w = synth.quantized_matrix(kind, n, k, synth.weight_seed(5, n))
            wb, cb = upload(ctx, w), ctx.new_owned_buffer(m * n * 4)
            call = lambda: ctx.gemm_device(kind, m, n, k, ab.device_ptr, wb.device_ptr, cb.device_ptr, ws.device_ptr,
                                           len(ws))
            for _ in range(warmup):
                call()
            ms = timed_loop(ctx, lambda i: call(), steps) / steps
            flops = 2.0 * m * n * k
            out[f"N{n}{tag}"] = {"ms": ms, "tflops": flops / (ms * 1e-3) / 1e12,
                                 "frac_of_bf16_peak": flops / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS}
            log(f"C5{tag} N={n}: {ms * 1e3:.1f} us, {out[f'N{n}{tag}']['tflops']:.1f} TFLOP/s")
            wb.free()
            cb.free()
    out["mfma_util_counters"] = load_mfma_util()
    return out


def bench_st(ctx, synth, steps, warmup):
    """GLM safetensors GEMV (src/metal.rs:738-1146; no BASELINE config):
    12288 x 6144 in BF16, F8_E4M3FN (128 x 128 block scales), row INT8 and
    grouped INT4 (group 32), and an INT4 expert-sized 2048 x 6144, batch 1,
    over rotating copies (more than the 256 MB MALL), back-to-back launches.
    Algorithmic bytes: weights + scales + 4 columns + 4 rows."""
    out = {}
    rng = np.random.default_rng(61)
    configs = (("BF16", 12288, 6144, 0), ("F8_E4M3", 12288, 6144, 0), ("I8", 12288, 6144, 0),
               ("I4_g32", 12288, 6144, 32), ("I4_g32", 2048, 6144, 32))
    for tag, rows, cols, group in configs:
        if tag == "BF16":
            w = (synth.normal(synth.activation_seed(50), rows * cols) * 0.05).view(np.uint32) >> 16
            w = w.astype("<u2").view(np.uint8)
            scales, dtype = None, "BF16"
        elif tag == "F8_E4M3":
            w = rng.integers(0, 0x7F, rows * cols, dtype=np.uint8) | (rng.integers(0, 2, rows * cols, dtype=np.uint8) << 7)
            scales, dtype = rng.uniform(1e-3, 4e-3, (rows // 128) * (cols // 128)).astype(np.float32), "F8_E4M3"
        elif tag == "I8":
            w = rng.integers(0, 256, rows * cols, dtype=np.uint8)
            scales, dtype = rng.uniform(1e-3, 1e-2, rows).astype(np.float32), "U8"
        else:
            w = rng.integers(0, 256, rows * cols // 2, dtype=np.uint8)
            scales, dtype = rng.uniform(1e-3, 1e-2, rows * (cols // group)).astype(np.float32), "U8"
        x = synth.normal(synth.activation_seed(51), cols)
        step_bytes = w.size + (0 if scales is None else scales.nbytes) + 4 * cols + 4 * rows
        copies = max(2, -(-300_000_000 // step_bytes))
        wbs = [upload(ctx, w)]
        for _ in range(copies - 1):
            b = ctx.new_owned_buffer(w.size)
            ctx.copy_device(b.device_ptr, wbs[0].device_ptr, w.size)
            wbs.append(b)
        sbs = [None] * copies if scales is None else [upload(ctx, scales) for _ in range(copies)]
        xb, yb = upload(ctx, x), ctx.new_owned_buffer(rows * 4)

        def call(i):
            sb = sbs[i % copies]
            ctx.matvec_safetensor_device(dtype, rows, cols, wbs[i % copies].device_ptr, w.size,
                                         None if sb is None else sb.device_ptr, 0 if scales is None else scales.size,
                                         xb.device_ptr, yb.device_ptr)

        for i in range(warmup):
            call(i)
        n = max(steps, 2 * copies)
        ms = timed_loop(ctx, call, n) / n
        key = f"{tag}_{rows}x{cols}"
        out[key] = {"ms": ms, "bytes": step_bytes, "gbps": step_bytes / (ms * 1e-3) / 1e9,
                    "frac_of_peak": step_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS}
        log(f"safetensors {key}: {ms * 1e3:.1f} us per launch ({out[key]['gbps']:.0f} GB/s)")
        for b in wbs + [xb, yb] + [b for b in sbs if b is not None]:
            b.free()
    return out


def bench_attn(ctx, synth, steps, warmup):
    """Decode attention over a KV ring (src/metal.rs:1270-1323) at the Gemma 4
    26B shapes (src/gemma4.rs:150-230): full layers (16 query heads over 2 KV
    heads of 512 dims) at 32768 and 131072 positions, and sliding layers (16
    query heads over 8 KV heads of 256 dims, 1024-position window, ring
    wrapped) rotating over 24 layers (403 MB, more than the MALL) as a decode
    step does.  Algorithmic bytes per call: the visible keys and values
    (2 x visible x width x 4) plus query and output.  cpu_port_ms: one call
    of the oracle's restatement of src/gemma4/cpu.rs:900-946 on one thread."""
    from oracle import capi
    out = {}
    configs = (("full_32k", 16, 2, 512, 32768, None, 32768, 1),
               ("full_128k", 16, 2, 512, 131072, None, 131072, 1),
               ("sliding_1k", 16, 8, 256, 8192, 1024, 4096, 24))
    for key, qh, kvh, hd, max_ctx, window, positions, nlayers in configs:
        width, pool = kvh * hd, 1024
        kpool = synth.normal(synth.activation_seed(40, hd), pool * width)
        vpool = synth.normal(synth.activation_seed(41, hd), pool * width)
        kb, vb = upload(ctx, kpool), upload(ctx, vpool)
        layers = [ctx.new_kv_layer(width, max_ctx, window) for _ in range(nlayers)]
        for layer in layers:
            for p in range(positions):
                j = (p % pool) * width * 4
                ctx.append_kv_device(layer, p, kb.device_ptr + j, width, vb.device_ptr + j, width)
        ctx.synchronize()
        q = (synth.normal(synth.activation_seed(42, hd), qh * hd) / np.sqrt(hd)).astype(np.float32)
        qb, ob = upload(ctx, q), ctx.new_owned_buffer(qh * hd * 4)
        cap = layers[0].capacity()
        visible = min(positions, cap)
        step_bytes = 2 * visible * width * 4 + 2 * qh * hd * 4

        def call(i):
            ctx.attention_cached_device(qb.device_ptr, qh * hd, layers[i % nlayers], qh, kvh, hd, ob.device_ptr,
                                        qh * hd)

        for i in range(warmup):
            call(i)
        n = max(steps, 2 * nlayers)
        ms = timed_loop(ctx, call, n) / n
        ctx.attention_result()
        res = {"qh": qh, "kvh": kvh, "head_dim": hd, "visible": visible, "bytes_per_call": step_bytes,
               "call_ms": ms, "gbps_call": step_bytes / (ms * 1e-3) / 1e9,
               "frac_of_peak": step_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS}
        if positions <= 32768:
            ring_k = np.zeros((cap, width), dtype=np.float32)
            ring_v = np.zeros((cap, width), dtype=np.float32)
            kp2, vp2 = kpool.reshape(pool, width), vpool.reshape(pool, width)
            for p in range(positions - visible, positions):
                ring_k[p % cap], ring_v[p % cap] = kp2[p % pool], vp2[p % pool]
            t0 = time.perf_counter()
            want = capi.attention(q, ring_k, ring_v, cap, width, qh, kvh, hd, positions - visible, visible)
            res["cpu_port_ms"] = (time.perf_counter() - t0) * 1e3
            got = ob.read(0, qh * hd * 4, np.float32)
            res["max_abs_diff_vs_port"] = float(np.abs(got - want).max())
        out[key] = res
        log(f"attention {key}: {ms * 1e3:.1f} us per call ({res['gbps_call']:.0f} GB/s)")
        for b in layers + [kb, vb, qb, ob]:
            b.free()
    return out


def bench_attn_host(ctx, synth, steps, warmup):
    """Three calls of host-cache attention (`dmhip_attention`) at the Gemma 4
    full-layer shape, 32768 positions: a short program for the HBM counter
    passes (no per-position append copies in the dispatch list)."""
    qh, kvh, hd, seq = 16, 2, 512, 32768
    keys = synth.normal(synth.activation_seed(43), seq * kvh * hd)
    values = synth.normal(synth.activation_seed(44), seq * kvh * hd)
    q = (synth.normal(synth.activation_seed(45), qh * hd) / np.sqrt(hd)).astype(np.float32)
    out = np.zeros(qh * hd, dtype=np.float32)
    for _ in range(3):
        ctx.attention(q, keys, values, qh, kvh, hd, None, out)
    return {"calls": 3, "bytes_per_call": 2 * seq * kvh * hd * 4 + 2 * qh * hd * 4}


def bench_copy(ctx, synth, steps, warmup):
    """A plain device copy of known size (512 MiB read + 512 MiB written):
    the calibration kernel for the FETCH_SIZE/WRITE_SIZE counter runs."""
    n = 512 << 20
    src, dst = ctx.new_owned_buffer(n), ctx.new_owned_buffer(n)
    for _ in range(warmup):
        ctx.copy_device(dst.device_ptr, src.device_ptr, n)
    with Timed(ctx) as t:
        for _ in range(steps):
            ctx.copy_device(dst.device_ptr, src.device_ptr, n)
    ms = t.wall_ms / steps
    return {"bytes_read": n, "bytes_written": n, "ms": ms, "gbps": 2 * n / (ms * 1e-3) / 1e9}


def host_parallelism():
    """The thread count Rust's std::thread::available_parallelism() reports
    (rayon's default pool size): the CPUs in this process's affinity mask,
    capped by a cgroup v2 CPU quota when one is set."""
    try:
        n = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        n = os.cpu_count() or 1
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            quota, period = f.read().split()[:2]
        if quota != "max":
            n = max(1, min(n, int(int(quota) // int(period))))
    except (OSError, ValueError):
        pass
    return n


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def cpu_baseline(w, x, seconds):
    """The CPU port of src/cpu.rs:345-399 + :275-293 on the C2 workload, on
    the thread count the reference's rayon pool would use."""
    from oracle import capi
    threads = host_parallelism()
    rows, cols = 151936, 4096
    step_bytes = w.size + cols * 4 + rows * 4
    reps, t0 = 0, time.perf_counter()
    while True:
        y = capi.matvec(Q6_K, rows, cols, w, x, threads=threads)
        idx = capi.argmax(y)
        reps += 1
        if time.perf_counter() - t0 >= seconds:
            break
    dt = time.perf_counter() - t0
    # one more step on a single thread (the scalar rate per core)
    t1 = time.perf_counter()
    capi.argmax(capi.matvec(Q6_K, rows, cols, w, x, threads=1))
    dt1 = time.perf_counter() - t1
    return {"value": step_bytes * reps / dt / 1e9, "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"full C2 step (Q6_K 151936x4096 matvec + argmax) repeated {reps}x in {dt:.1f}s "
                      f"on {threads} host threads; oracle/dm_oracle.c (gcc -O3 -ffp-contract=off) restating "
                      f"src/cpu.rs (the Rust reference cannot be built here)",
            "nproc": os.cpu_count(), "cpu_model": cpu_model(),
            "value_1_thread": step_bytes / dt1 / 1e9,
            "argmax": int(idx)}


def load_mfma_util():
    """MFMA utilisation of the C5 GEMM per N from the counter pass committed
    under profiles/ (SQ_VALU_MFMA_BUSY_CYCLES / GRBM_GUI_ACTIVE), or None."""
    path = os.path.join(ROOT, "profiles", "c5_prefill_gemm_mfma_util.json")
    try:
        with open(path) as f:
            return json.load(f)
    except (OSError, ValueError):
        return None


def load_traffic():
    path = os.path.join(ROOT, "profiles", "c2_q6k_gemv_traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get("hbm_bytes_per_launch")


def main() -> int:
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--only", default=None,
                   help="c1..c5: run one GPU configuration, print its record; copy: the counter "
                        "calibration copy")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    args = p.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported (this build has no "
              "multi-GPU path; the kernels work on one GPU's share of the rows)", file=sys.stderr)
        return 2

    from diskmule_amd import HipContext, synth
    ctx = HipContext(0)
    log("device:", ctx.device_name())
    if args.only:
        fn = {"c1": bench_c1, "c2": bench_c2, "c3": bench_c3, "c4": bench_c4, "c5": bench_c5,
              "q8": bench_q8, "dense": bench_dense, "st": bench_st, "attn": bench_attn, "attn_host": bench_attn_host,
              "host": bench_host, "copy": bench_copy}[args.only]
        res = fn(ctx, synth, args.steps, args.warmup)
        print(json.dumps(res[0] if isinstance(res, tuple) else res))
        return 0

    c2, (w2, x2) = bench_c2(ctx, synth, args.steps, args.warmup)
    details = {"C2": c2}
    for name, fn in (("C1", bench_c1), ("C3", bench_c3), ("C4", bench_c4), ("C5", bench_c5), ("Q8_0", bench_q8),
                     ("dense", bench_dense), ("safetensors", bench_st), ("attention", bench_attn),
                     ("host_slice", bench_host)):
        details[name] = fn(ctx, synth, max(3, args.steps // 2), args.warmup)
    log("CPU baseline")
    cpu = cpu_baseline(w2, x2, args.cpu_seconds)
    details["argmax_equal_cpu"] = cpu.pop("argmax") == c2["argmax"]

    record = {
        "metric": METRIC,
        "value": round(c2["gbps"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": c2["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "C2: Q6_K output head 151936x4096 GEMV + greedy argmax, batch 1 "
                               "(BASELINE configs[1]); weights resident in HBM",
                   "weight_type": "Q6_K", "rows": 151936, "columns": 4096, "batch": 1,
                   "arithmetic": "int8 MFMA on the raw 6-bit codes and 3-term int8 activations (22 bits "
                                 "per 256-value block): exact int32 group dots, fp32 block accumulation"},
        "roofline": {"bound": "hbm", "achieved": round(c2["gbps"], 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(c2["gbps"] / HBM_PEAK_GBS, 4),
                     "traffic": load_traffic()},
        "cpu_baseline": cpu,
        "details": details,
    }
    print(json.dumps(record))
    return 0


if __name__ == "__main__":
    sys.exit(main())
