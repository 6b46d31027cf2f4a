#!/usr/bin/env python3
"""Benchmark of the MI355X paged-KV hot path (one GPU).

Headline workload ("c5"): Qwen2-7B-shaped serving
stress — 64 sessions with seeded log-uniform contexts in [1k, 32k], int8 KV
with f16 scales in 16-token pages, each step appends 4 draft tokens per
session and runs 4-query causal (speculative-verify) decode attention in all
28 layers; every 16 steps 8 sessions release their pages and 8 new
2k-context sessions reuse them. It is the configuration the >= 70 %-of-HBM
target is stated for. A "step" is one pass of the hot path over the batch:
plan + 28 x (decode attention whose launch also quantizes and stores the new
rows, split reduction), through the product's Qwen2 KV driver.

value = algorithmic bytes (append + attention, per the formulas in
synth.algorithmic_bytes_*) of the timed steps / their wall time, GB/s.
roofline = the paged decode kernel alone (the dominant kernel; the split
merge kernel is timed beside it): the last step's layer calls replayed over
all layers, each kernel bracketed by HIP events that the library records on
the launch stream (tge_batch_set_profiling); its algorithmic bytes are the
attention's plus the append's it performs. traffic = HBM bytes per
dispatch: the committed rocprofv3 counter summary for this workload gives
traffic per algorithmic byte, scaled to this run's spans (the source is
stated in the line). measured_copy_peak = device-to-device copy GB/s on this
GPU, beside the 8 TB/s spec peak. cpu_baseline = the reference's own AVX2 attention kernel
(oracle/_ref, built from the reference sources) under the reference's
forward_batch schedule, on a bounded sample of the same workload.
The other four configurations are measured briefly and reported under
"configs" (they are parity cases, not the headline), each with its own
"cpu_baseline": the reference's AVX2 kernels under the schedule the
reference runs for that configuration (decode of one sequence, a batched
step, block prefill per chunk), timed for a few seconds at most. Beside
them: shared-prefix decode ("prefix"), a mixed verify + prefill step
("mixed"), and 256-dim heads (synth.wide_head_configs: a verify decode
"d256" and a chunked prompt "p256").

Usage: python bench.py [--gpus 1] [--steps 32] [--warmup 4] [--no-others]
       [--no-cpu] [--cpu-seconds 10]
"""
import argparse
import ctypes as C
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
for sub in ("aegean-tge_amd", "oracle"):
    sys.path.insert(0, os.path.join(ROOT, sub))

HBM_PEAK_GBS = 8000.0       # MI355X HBM3E
MFMA_F16_PEAK_TFLOPS = 2500.0  # dense f16/bf16
WORKLOAD_C5 = ("c5: Qwen2-7B-shaped serving stress, 64 sessions, log-uniform 1k-32k "
               "contexts, int8 KV + f16 scales, 16-token pages, 4-query verify "
               "decode, churn 8 sessions / 16 steps")
METRIC = ("paged-KV decode attention: achieved HBM GB/s (% of peak), "
          "µs per layer-step")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# CPU threads one GPU's job may use on the GPU box (its CPU share), whatever
# the host reports.
CPU_SHARE = 16


def host_cores():
    """(logical, physical) cores this process may run on: the affinity set,
    and the distinct (package, core) pairs among it."""
    cpus = sorted(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else \
        list(range(os.cpu_count() or 1))
    phys = set()
    for c in cpus:
        base = f"/sys/devices/system/cpu/cpu{c}/topology"
        try:
            with open(f"{base}/physical_package_id") as f:
                pkg = f.read().strip()
            with open(f"{base}/core_id") as f:
                core = f.read().strip()
            phys.add((pkg, core))
        except OSError:
            phys.add(("?", str(c)))
    return len(cpus), max(1, len(phys))


def decode_threads():
    """The reference's decode rule: one worker per physical core
    (resolve_decode_threads, dispatch.cpp:77-94), within the CPU share."""
    return min(CPU_SHARE, host_cores()[1])


def prefill_threads():
    """The reference's default pool: every logical core
    (default_thread_count, thread_pool.cpp:337-340), within the CPU share."""
    return min(CPU_SHARE, host_cores()[0])


def cores_fields(threads, rule):
    logical, physical = host_cores()
    return {"cores": threads, "host_logical_cores": logical, "host_physical_cores": physical,
            "thread_rule": rule}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=32)
    ap.add_argument("--warmup", type=int, default=4)
    ap.add_argument("--replay", type=int, default=3, help="replays of the last step's attention")
    ap.add_argument("--others", dest="others", action="store_true", default=True)
    ap.add_argument("--no-others", dest="others", action="store_false")
    ap.add_argument("--cpu", dest="cpu", action="store_true", default=True)
    ap.add_argument("--no-cpu", dest="cpu", action="store_false")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--only", default="",
                    help="run one config key (c1..c5, prefix, mixed, d256, p256) and print it")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only time 1 GiB device-to-device copies (counter calibration)")
    ap.add_argument("--read-ceiling", action="store_true",
                    help="only run the HBM read-ceiling sweep (tge_read_ceiling) and print it")
    ap.add_argument("--fragment-c5", action="store_true",
                    help="shuffle the c5 pool's free list before the sessions fill it")
    return ap.parse_args()


class DecodeBench:
    """Runs a decode configuration through the Qwen2 KV driver."""

    def __init__(self, tk, synth, cfg, total_steps):
        self.tk, self.synth, self.cfg = tk, synth, cfg
        sh = cfg.shape
        self.sh = sh
        self.n_seq = len(cfg.contexts)
        grow = total_steps * cfg.n_new
        fill_max = max(cfg.contexts + [cfg.churn_context])
        self.fill_max = fill_max
        context = min(32768, max(c + grow for c in cfg.contexts + [cfg.churn_context]) + 16)
        if cfg.pool_pages:
            pages = cfg.pool_pages
        else:
            need = sum(math.ceil((c + grow) / 16) for c in cfg.contexts)
            churn = cfg.churn_sessions * math.ceil((cfg.churn_context + grow) / 16)
            pages = int(need * 1.1) + churn + 64
        self.pages = pages
        self.model = tk.Qwen2KvPath(sh.layers, sh.q_heads, sh.kv_heads, sh.head_dim,
                                    context=context, sequences=self.n_seq, pages=pages,
                                    fmt=cfg.fmt, scale_format=tk.SCALE_F16)
        if cfg.fragmented:
            self.model.table().fragment(cfg.seed + 1000)
        rng = np.random.default_rng(cfg.seed)
        self.rng = rng
        rows = self.n_seq * cfg.n_new
        self.rows = rows
        k, v = synth.make_kv(rng, rows, sh.kv_dim, cfg)
        self.q = tk.DeviceArray.from_numpy(synth.make_q(rng, rows, sh.q_dim, cfg))
        self.k = tk.DeviceArray.from_numpy(k)
        self.v = tk.DeviceArray.from_numpy(v)
        self.out = tk.DeviceArray((rows, sh.q_dim), np.float32)
        # K/V source rows for context fills: 2 x fill_max rows, read from a
        # seeded offset per (session, layer) so sessions differ.
        kf, vf = synth.make_kv(rng, 2 * fill_max, sh.kv_dim, cfg)
        self.kfill = tk.DeviceArray.from_numpy(kf)
        self.vfill = tk.DeviceArray.from_numpy(vf)
        self.lengths = [0] * self.n_seq
        self.churn_rng = np.random.default_rng(cfg.seed + 99)
        t0 = time.perf_counter()
        for s, c in enumerate(cfg.contexts):
            self.fill(s, c)
        tk.hip().sync()
        self.fill_s = time.perf_counter() - t0

    def fill(self, s, ctx):
        self.model.begin_prefill(s, 0, ctx)
        row_bytes = self.sh.kv_dim * 4
        for layer in range(self.sh.layers):
            off = int(self.rng.integers(0, self.fill_max)) * row_bytes
            self.model.store(layer, self.kfill.ptr + off, self.vfill.ptr + off)
        self.lengths[s] = ctx

    def churn(self):
        for s in self.churn_rng.choice(self.n_seq, self.cfg.churn_sessions, replace=False):
            self.model.reset(int(s))
            self.fill(int(s), self.cfg.churn_context)

    def step(self):
        n = self.cfg.n_new
        positions = [self.lengths[s] + i for s in range(self.n_seq) for i in range(n)]
        sequences = [s for s in range(self.n_seq) for _ in range(n)]
        self.model.begin_forward_batch(positions, sequences)
        for layer in range(self.sh.layers):
            self.model.layer_ptrs(layer, self.q.ptr, self.k.ptr, self.v.ptr, self.out.ptr)
        for s in range(self.n_seq):
            self.lengths[s] += n
        return [self.lengths[s] for s in range(self.n_seq)]

    def bytes_per_layer(self, spans):
        sy = self.synth
        att = sy.algorithmic_bytes_decode(self.sh, self.cfg.fmt, spans, self.cfg.n_new)
        app = sy.algorithmic_bytes_append(self.sh, self.cfg.fmt, self.rows)
        return att, app

    def run(self, steps, warmup, replay):
        tk = self.tk
        hip = tk.hip()
        # Timed steps run back to back (the host plans step i+1 while the GPU
        # still works on step i); the clock stops only around the churn
        # (session release and 2k-token refills between steps), which is not
        # part of a decode step.
        times, total_bytes, att_bytes_sum = [], 0, 0
        spans = None
        t0 = None
        for i in range(warmup + steps):
            timed = i >= warmup
            if timed and t0 is None:
                hip.sync()
                t0 = time.perf_counter()
            spans = self.step()
            if timed:
                att, app = self.bytes_per_layer(spans)
                total_bytes += (att + app) * self.sh.layers
                att_bytes_sum += att * self.sh.layers
            last = i == warmup + steps - 1
            churn = bool(self.cfg.churn_every) and (i + 1) % self.cfg.churn_every == 0 and not last
            if t0 is not None and (churn or last):
                hip.sync()
                times.append(time.perf_counter() - t0)
                t0 = None
            if churn:
                self.churn()
        hip.sync()
        step_s = sum(times)
        # Roofline leg: replay the last step's decode attention over every
        # layer (idempotent: same cache, same q) and its append; HIP events
        # on the launch stream bracket each block of launches.
        lib = tk.lib()
        pool, batch = self.model.pool_handle(), self.model.batch_handle()
        L = self.sh.layers
        # Per-kernel durations (paged attention kernel alone, split merge
        # alone) from the library's timing events, calls issued back to back:
        # the decode kernel of the layer step itself (tge_decode_step) where
        # that launch also stores the new rows, else the persistent decode
        # kernel of tge_decode_attention.
        step_wg, step_pieces, stores = C.c_int(), C.c_int(), C.c_int()
        tk.check(lib.tge_batch_step_info(batch, C.byref(step_wg), C.byref(step_pieces)))
        tk.check(lib.tge_batch_decode_stores_rows(batch, C.byref(stores)))
        fold = bool(stores.value)
        tk.check(lib.tge_batch_set_profiling(batch, 1))
        for _ in range(replay):
            for layer in range(L):
                if fold:
                    tk.check(lib.tge_decode_step(batch, pool, layer, self.q.ptr, self.k.ptr, self.v.ptr,
                                                 self.out.ptr, None))
                else:
                    tk.check(lib.tge_decode_attention(batch, pool, layer, self.q.ptr, self.out.ptr, None))
        n_calls, a_us, mg_us = C.c_int(), C.c_float(), C.c_float()
        tk.check(lib.tge_batch_kernel_times(batch, C.byref(n_calls), C.byref(a_us), C.byref(mg_us)))
        tk.check(lib.tge_batch_set_profiling(batch, 0))
        k_us = [a_us.value / n_calls.value]
        m_us = [mg_us.value / n_calls.value]
        e0, e1, e2 = hip.event(), hip.event(), hip.event()
        hip.record(e0)
        for _ in range(replay):
            for layer in range(L):
                tk.check(lib.tge_decode_attention(batch, pool, layer, self.q.ptr, self.out.ptr, None))
        hip.record(e1)
        for _ in range(replay):
            for layer in range(L):
                tk.check(lib.tge_kv_append(batch, pool, layer, self.k.ptr, self.v.ptr, None))
        hip.record(e2)
        # The fused variant of the same append: bias + NeoX RoPE of q and k
        # before the store (tge_kv_append_rope), rotated q to its own buffer.
        sh = self.sh
        rng = np.random.default_rng(self.cfg.seed + 5)
        max_pos = max(spans) + 1
        cos_t, sin_t = tk.rope_tables(sh.head_dim, max_pos)
        dcos, dsin = tk.DeviceArray.from_numpy(cos_t), tk.DeviceArray.from_numpy(sin_t)
        biases = [tk.DeviceArray.from_numpy(rng.standard_normal(n).astype(np.float32))
                  for n in (sh.q_dim, sh.kv_dim, sh.kv_dim)]
        q_rot = tk.DeviceArray((self.rows, sh.q_dim), np.float32)
        args = tk.rope_args(self.k, self.v, dcos, dsin, max_pos, q=self.q, q_out=q_rot,
                            q_bias=biases[0], k_bias=biases[1], v_bias=biases[2])
        e2r, e3 = hip.event(), hip.event()
        hip.record(e2r)
        for _ in range(replay):
            for layer in range(L):
                tk.check(lib.tge_kv_append_rope(batch, pool, layer, C.byref(args), None))
        hip.record(e3)
        # The whole layer step as the driver issues it (tge_decode_step: one
        # kernel for a small step, else append + decode + merge), replayed
        # (idempotent: the same rows stored at the same positions again).
        e4, e5 = hip.event(), hip.event()
        hip.record(e4)
        for _ in range(replay):
            for layer in range(L):
                tk.check(lib.tge_decode_step(batch, pool, layer, self.q.ptr, self.k.ptr, self.v.ptr,
                                             self.out.ptr, None))
        hip.record(e5)
        att_ms = hip.elapsed_ms(e0, e1) / (replay * L)
        step_launch_ms = hip.elapsed_ms(e4, e5) / (replay * L)
        app_ms = hip.elapsed_ms(e1, e2) / (replay * L)
        rope_ms = hip.elapsed_ms(e2r, e3) / (replay * L)
        # Static sparse attention (sink 4, window 512) at stride 4 (every
        # page still read) and 32 (middle pages with nothing kept skipped).
        sparse_us = {}
        for stride in (4, 32):
            tk.check(lib.tge_batch_set_sparse(batch, 1, 4, 512, stride))
            tk.check(lib.tge_batch_set_profiling(batch, 1))
            for layer in range(L):
                tk.check(lib.tge_decode_attention(batch, pool, layer, self.q.ptr, self.out.ptr, None))
            tk.check(lib.tge_batch_kernel_times(batch, C.byref(n_calls), C.byref(a_us), C.byref(mg_us)))
            tk.check(lib.tge_batch_set_profiling(batch, 0))
            sparse_us[f"sink4_window512_stride{stride}"] = a_us.value / n_calls.value
        tk.check(lib.tge_batch_set_sparse(batch, 0, 0, 0, 0))
        att_b, app_b = self.bytes_per_layer(spans)
        kernel_b = att_b + (app_b if fold else 0)  # the timed kernel's algorithmic bytes
        # + q read and written, the two table rows of each token, the biases
        rope_b = (app_b + self.rows * sh.q_dim * 8 + self.rows * sh.head_dim * 4
                  + (sh.q_dim + 2 * sh.kv_dim) * 4)
        for a in [dcos, dsin, q_rot] + biases:
            a.close()
        rows, work_items, splits = tk.batch_info(batch)
        return {
            "steps": steps,
            "step_ms": 1e3 * step_s / steps,
            "us_per_layer_step": 1e6 * step_s / (steps * L),
            "gbs": total_bytes / step_s / 1e9,
            "tokens_per_s": self.rows * steps / step_s,
            "attn_launch_us": att_ms * 1e3,
            "attn_kernel_us": float(np.mean(k_us)),
            "merge_kernel_us": float(np.mean(m_us)),
            "attn_bytes_per_launch": att_b,
            "attn_gbs": att_b / (att_ms * 1e-3) / 1e9,
            "attn_kernel_gbs": kernel_b / (float(np.mean(k_us)) * 1e-6) / 1e9,
            "kernel_bytes_per_launch": kernel_b,
            "kernel_stores_rows": fold,
            "append_launch_us": app_ms * 1e3,
            "step_launch_us": step_launch_ms * 1e3,
            "step_path": (f"one kernel, {step_wg.value} workgroups, up to {step_pieces.value} "
                          f"pieces per context" if step_wg.value
                          else "decode (storing the new rows) + merge" if fold
                          else "append + decode + merge"),
            "step_gbs": (att_b + app_b) / (step_launch_ms * 1e-3) / 1e9,
            "append_bytes_per_launch": app_b,
            "append_gbs": app_b / (app_ms * 1e-3) / 1e9,
            "append_rope_launch_us": rope_ms * 1e3,
            "sparse_attn_kernel_us": sparse_us,
            "append_rope_bytes_per_launch": rope_b,
            "append_rope_gbs": rope_b / (rope_ms * 1e-3) / 1e9,
            "work_items": work_items,
            "max_splits": splits,
            "pool_pages": self.pages,
            "mean_context": float(np.mean(spans)),
            "fill_s": self.fill_s,
        }


def run_prefill(tk, synth, cfg, reps=3):
    sh = cfg.shape
    L = sh.layers
    model = tk.Qwen2KvPath(L, sh.q_heads, sh.kv_heads, sh.head_dim, context=cfg.prompt,
                           sequences=1, pages=cfg.pool_pages, fmt=tk.KV_F16)
    model.table().fragment(cfg.seed + 1000)
    rng = np.random.default_rng(cfg.seed)
    n = cfg.prompt
    k, v = synth.make_kv(rng, n, sh.kv_dim, cfg)
    q = tk.DeviceArray.from_numpy(synth.make_q(rng, n, sh.q_dim, cfg))
    dk, dv = tk.DeviceArray.from_numpy(k), tk.DeviceArray.from_numpy(v)
    out = tk.DeviceArray((n, sh.q_dim), np.float32)
    hip = tk.hip()
    ch = cfg.prefill_chunk
    per_chunk = np.zeros(n // ch)
    kern_us = np.zeros(n // ch)   # block-prefill kernel alone, per layer
    merge_us = np.zeros(n // ch)
    lib = tk.lib()
    for r in range(reps + 1):
        model.reset(0)
        for c in range(n // ch):
            hip.sync()
            t0 = time.perf_counter()
            model.begin_prefill(0, c * ch, ch)
            for layer in range(L):
                model.layer_ptrs(layer, q.ptr + c * ch * sh.q_dim * 4, dk.ptr + c * ch * sh.kv_dim * 4,
                                 dv.ptr + c * ch * sh.kv_dim * 4, out.ptr + c * ch * sh.q_dim * 4)
            hip.sync()
            if r:
                per_chunk[c] += time.perf_counter() - t0
                # the kernels of one layer-chunk, timed on their own (back to back)
                batch, pool = model.batch_handle(), model.pool_handle()
                tk.check(lib.tge_batch_set_profiling(batch, 1))
                for layer in range(L):
                    tk.check(lib.tge_prefill_attention(batch, pool, layer,
                                                       q.ptr + c * ch * sh.q_dim * 4,
                                                       out.ptr + c * ch * sh.q_dim * 4, None))
                n_calls, a_us, m_us = C.c_int(), C.c_float(), C.c_float()
                tk.check(lib.tge_batch_kernel_times(batch, C.byref(n_calls), C.byref(a_us),
                                                    C.byref(m_us)))
                tk.check(lib.tge_batch_set_profiling(batch, 0))
                kern_us[c] += a_us.value / n_calls.value
                merge_us[c] += m_us.value / n_calls.value
    per_chunk /= reps
    kern_us /= reps
    merge_us /= reps
    flops = [synth.prefill_flops(sh, c * ch, ch) * L for c in range(n // ch)]
    total_s = float(per_chunk.sum())
    tflops = sum(flops) / total_s / 1e12
    kern_tflops = sum(flops) / (float(kern_us.sum()) * L * 1e-6) / 1e12
    res = {
        "us_per_layer_chunk": [1e6 * t / L for t in per_chunk],
        "tflops": tflops,
        "mfma_util": tflops / MFMA_F16_PEAK_TFLOPS,
        "attn_kernel_us_per_chunk": [float(x) for x in kern_us],
        "merge_kernel_us_per_chunk": [float(x) for x in merge_us],
        "attn_kernel_tflops": kern_tflops,
        "attn_kernel_mfma_util": kern_tflops / MFMA_F16_PEAK_TFLOPS,
        "prompt_ms": 1e3 * total_s,
        "tokens_per_s": n / total_s,
    }
    model.close()
    return res


def run_prefix(tk, synth, cfg, sessions=8, prefix=2048, private=256, reps=3):
    """Shared-prefix serving on the c5 shape: `sessions` sessions whose first
    `prefix` tokens are one remembered page chain (attached by reference
    count), each followed by `private` tokens of its own, against the same
    sessions holding every page privately. Reports the attach cost (host),
    the prefix's store cost it replaces, pages saved, the copy-on-write cost
    of one page, and the decode attention kernel (4-query verify) on both."""
    sh = cfg.shape
    L = sh.layers
    rng = np.random.default_rng(cfg.seed + 7)
    toks = [int(x) for x in rng.integers(0, 150000, prefix)]
    span = prefix + private
    pages_each = -(-(span + cfg.n_new) // 16)
    kf, vf = synth.make_kv(rng, span, sh.kv_dim, cfg)
    dk, dv = tk.DeviceArray.from_numpy(kf), tk.DeviceArray.from_numpy(vf)
    rows = sessions * cfg.n_new
    q = tk.DeviceArray.from_numpy(synth.make_q(rng, rows, sh.q_dim, cfg))
    kn, vn = synth.make_kv(rng, rows, sh.kv_dim, cfg)
    dkn, dvn = tk.DeviceArray.from_numpy(kn), tk.DeviceArray.from_numpy(vn)
    out = tk.DeviceArray((rows, sh.q_dim), np.float32)
    hip = tk.hip()
    lib = tk.lib()
    row_bytes = sh.kv_dim * 4

    def store(model, s, start, count):
        model.begin_prefill(s, start, count)
        for layer in range(L):
            model.store(layer, dk.ptr + start * row_bytes, dv.ptr + start * row_bytes)

    def decode_kernel_us(model):
        positions = [span + i for s in range(sessions) for i in range(cfg.n_new)]
        seqs = [s for s in range(sessions) for _ in range(cfg.n_new)]
        model.begin_forward_batch(positions, seqs)
        for layer in range(L):
            model.store(layer, dkn.ptr, dvn.ptr)
        batch, pool = model.batch_handle(), model.pool_handle()
        tk.check(lib.tge_batch_set_profiling(batch, 1))
        for _ in range(reps):
            for layer in range(L):
                tk.check(lib.tge_decode_attention(batch, pool, layer, q.ptr, out.ptr, None))
        n, a, m = C.c_int(), C.c_float(), C.c_float()
        tk.check(lib.tge_batch_kernel_times(batch, C.byref(n), C.byref(a), C.byref(m)))
        tk.check(lib.tge_batch_set_profiling(batch, 0))
        return a.value / n.value, m.value / n.value

    res = {"sessions": sessions, "prefix_tokens": prefix, "private_tokens": private,
           "queries_per_session": cfg.n_new}
    # shared: session 0 stores the prefix and keys it; the others attach it
    shared = tk.Qwen2KvPath(L, sh.q_heads, sh.kv_heads, sh.head_dim, context=span + 64,
                            sequences=sessions, pages=sessions * pages_each, fmt=cfg.fmt,
                            scale_format=tk.SCALE_F16)
    hip.sync()
    t0 = time.perf_counter()
    store(shared, 0, 0, prefix)
    hip.sync()
    res["prefix_store_ms"] = 1e3 * (time.perf_counter() - t0)
    shared.remember_prefix(0, toks)
    t0 = time.perf_counter()
    for s in range(1, sessions):
        assert shared.attach_prefix(s, toks) == prefix
    res["attach_us_per_session"] = 1e6 * (time.perf_counter() - t0) / (sessions - 1)
    for s in range(sessions):
        store(shared, s, prefix, private)
    hip.sync()
    a_sh, m_sh = decode_kernel_us(shared)
    # copy-on-write of one page (every layer) into a spare page, timed with events
    pool = shared.pool_handle()
    used = shared.pages(0)[0]
    tab = shared.table()
    fresh = tab.allocate()
    e0, e1 = hip.event(), hip.event()
    hip.record(e0)
    for _ in range(10):
        tk.check(lib.tge_kv_copy_page(pool, used, fresh, None))
    hip.record(e1)
    res["copy_page_us"] = hip.elapsed_ms(e0, e1) * 1e3 / 10
    tab.release(fresh)
    free_shared = shared.free_pages()
    shared.close()
    # private: every session stores the prefix itself
    priv = tk.Qwen2KvPath(L, sh.q_heads, sh.kv_heads, sh.head_dim, context=span + 64,
                          sequences=sessions, pages=sessions * pages_each, fmt=cfg.fmt,
                          scale_format=tk.SCALE_F16)
    for s in range(sessions):
        store(priv, s, 0, span)
    hip.sync()
    a_pr, m_pr = decode_kernel_us(priv)
    res["pages_saved"] = free_shared - priv.free_pages()
    priv.close()
    att_b = synth.algorithmic_bytes_decode(sh, cfg.fmt, [span + cfg.n_new] * sessions, cfg.n_new)
    res.update({
        "attn_bytes_per_launch": att_b,
        "attn_kernel_us_shared": a_sh, "merge_kernel_us_shared": m_sh,
        "attn_kernel_us_private": a_pr, "merge_kernel_us_private": m_pr,
        "attn_gbs_shared": att_b / (a_sh * 1e-6) / 1e9,
        "attn_gbs_private": att_b / (a_pr * 1e-6) / 1e9,
    })
    for a in (dk, dv, q, dkn, dvn, out):
        a.close()
    return res


def run_mixed(tk, synth, cfg, decode_sessions=32, chunk=512, prompt_done=1536, reps=5):
    """A continuous-batching step on the c5 shape (one layer's attention):
    `decode_sessions` sessions verifying 4 draft tokens next to one session
    prefilling a `chunk`-token chunk after `prompt_done` prompt tokens.
    Times the mixed call (tge_batch_attention: one paged_mixed_kernel
    launch whose workgroups take the decode shares of the short sessions
    and the block-prefill tiles of the chunk), the same step forced through
    the block-prefill kernel alone, and the two kinds as separate steps."""
    from types import SimpleNamespace
    sh = cfg.shape
    ctxs = list(cfg.contexts[:decode_sessions]) + [prompt_done]
    n_new = [cfg.n_new] * decode_sessions + [chunk]
    totals = [c + n for c, n in zip(ctxs, n_new)]
    pages = sum(-(-t // 16) for t in totals) + 8
    table = synth.fragmented_table(pages, cfg.seed + 3)
    pool = tk.KvPool(1, pages, sh.kv_heads, sh.head_dim, cfg.fmt, tk.SCALE_F16)
    ids = [[table.allocate() for _ in range(-(-t // 16))] for t in totals]
    rng = np.random.default_rng(cfg.seed + 11)
    src_rows = max(totals)
    kf, vf = synth.make_kv(rng, src_rows, sh.kv_dim, cfg)
    dk, dv = tk.DeviceArray.from_numpy(kf), tk.DeviceArray.from_numpy(vf)
    for c, p in zip(ctxs, ids):  # context rows, one plan per session
        b = tk.Batch().plan(pool, [tk.Session(0, c, p)], sh.q_heads)
        b.append(pool, 0, dk, dv)
        b.close()
    rows = sum(n_new)
    q = tk.DeviceArray.from_numpy(synth.make_q(rng, rows, sh.q_dim, cfg))
    out = tk.DeviceArray((rows, sh.q_dim), np.float32)
    hip = tk.hip()
    sess = [tk.Session(c, n, p) for c, n, p in zip(ctxs, n_new, ids)]

    def timed(calls):
        for f in calls:  # warm: builds the lazily planned lists
            f()
        hip.sync()
        e0, e1 = hip.event(), hip.event()
        hip.record(e0)
        for _ in range(reps):
            for f in calls:
                f()
        hip.record(e1)
        return hip.elapsed_ms(e0, e1) * 1e3 / reps

    mixed = tk.Batch().plan(pool, sess, sh.q_heads)
    mixed.append(pool, 0, SimpleNamespace(ptr=dk.ptr), SimpleNamespace(ptr=dv.ptr))
    t_mixed = timed([lambda: mixed.attention(pool, 0, q, out)])
    t_prefill_only = timed([lambda: mixed.prefill(pool, 0, q, out)])
    dec = tk.Batch().plan(pool, sess[:-1], sh.q_heads)
    pf = tk.Batch().plan(pool, sess[-1:], sh.q_heads)
    q_pf = SimpleNamespace(ptr=q.ptr + decode_sessions * cfg.n_new * sh.q_dim * 4)
    out_pf = SimpleNamespace(ptr=out.ptr + decode_sessions * cfg.n_new * sh.q_dim * 4)
    t_split = timed([lambda: dec.decode(pool, 0, q, out), lambda: pf.prefill(pool, 0, q_pf, out_pf)])
    for b in (mixed, dec, pf):
        b.close()
    att_b = synth.algorithmic_bytes_decode(sh, cfg.fmt, [c + n for c, n in zip(ctxs[:-1], n_new[:-1])],
                                           cfg.n_new)
    flops = synth.prefill_flops(sh, prompt_done, chunk)
    res = {
        "decode_sessions": decode_sessions, "queries_per_session": cfg.n_new,
        "prefill_chunk": chunk, "prefill_after": prompt_done,
        "decode_attn_bytes": att_b, "prefill_flops": flops,
        "us_mixed_call": t_mixed, "us_prefill_kernel_only": t_prefill_only,
        "us_separate_steps": t_split,
        "tokens_per_s_mixed": rows / (t_mixed * 1e-6),
    }
    for a in (dk, dv, q, out):
        a.close()
    pool.close()
    return res


def cpu_baseline_c5(synth, cfg, seconds):
    """The reference's forward_batch attention schedule (per (row, head)
    attention_head_avx2, parallel over rows) with its own AVX2 kernels from
    oracle/_ref, on a seeded sample of 16 of the 64 sessions, i8 KV with the
    reference's fp32 scales."""
    import oracle as O
    ref = O.ref()
    if ref is None:
        return None
    sh = cfg.shape
    threads = decode_threads()
    rng = np.random.default_rng(cfg.seed + 5)
    sample = sorted(rng.choice(len(cfg.contexts), 16, replace=False))
    n_q = cfg.n_new
    spans, bases, kv_rows = [], [], 0
    for s in sample:
        ctx = cfg.contexts[s]
        for i in range(n_q):
            spans.append(ctx + i + 1)
            bases.append(kv_rows * sh.kv_dim)
        kv_rows += ctx + n_q
    kc = rng.integers(-127, 128, size=(kv_rows, sh.kv_dim), dtype=np.int8)
    vc = rng.integers(-127, 128, size=(kv_rows, sh.kv_dim), dtype=np.int8)
    ks = rng.uniform(0.005, 0.05, size=(kv_rows, sh.kv_dim // 32)).astype(np.float32)
    vs = rng.uniform(0.005, 0.05, size=(kv_rows, sh.kv_dim // 32)).astype(np.float32)
    rows = len(spans)
    q = rng.standard_normal((rows, sh.q_dim)).astype(np.float32)
    out = np.empty((rows, sh.q_dim), np.float32)
    max_span = max(spans)
    scores = np.empty(rows * sh.q_heads * max_span, np.float32)
    b_arr = np.array(bases, np.int64)
    s_arr = np.array(spans, np.int32)
    fp = lambda a: a.ctypes.data_as(C.c_void_p)
    team = ref.ref_team_create(threads)
    reps, t_total = 0, 0.0
    try:
        while t_total < seconds and reps < 1000:
            t0 = time.perf_counter()
            ref.ref_baseline_batch_heads(team, O.I8, fp(q), fp(kc), fp(vc), fp(ks), fp(vs),
                                         fp(b_arr), fp(s_arr), rows, sh.q_heads, sh.kv_heads,
                                         sh.head_dim, max_span, fp(scores), fp(out))
            t_total += time.perf_counter() - t0
            reps += 1
    finally:
        ref.ref_team_destroy(team)
    sess_spans = [cfg.contexts[s] + n_q for s in sample]
    kv = sh.kv_dim
    alg = sum(2 * S * kv + 2 * S * (kv // 32) * 4 + 2 * n_q * sh.q_dim * 4 + math.ceil(S / 16) * 4
              for S in sess_spans)
    per = t_total / reps
    all_spans = [c + n_q for c in cfg.contexts]
    scale = sum(all_spans) / sum(sess_spans)
    return {
        "value": alg / per / 1e9,
        "unit": "GB/s",
        **cores_fields(threads, "decode: one thread per physical core (dispatch.cpp:77-94), "
                                f"at most the GPU's CPU share of {CPU_SHARE}"),
        "kind": "reference",
        "sample": (f"reference attention_head_avx2 (oracle/_ref, built from the reference "
                   f"sources) under the forward_batch schedule (qwen2.cpp:1705-1747), "
                   f"{threads} threads, 16 of 64 sessions (sum of spans {sum(sess_spans)}), "
                   f"4 queries x 28 heads, one layer-step repeated {reps}x in {t_total:.1f} s; "
                   f"{1e6 * per:.0f} us per sampled layer-step, ~{1e6 * per * scale:.0f} us "
                   f"per full 64-session layer-step by span scaling"),
        "us_per_layer_step_est": 1e6 * per * scale,
    }


def _ref_team(seconds, threads):
    import oracle as O
    ref = O.ref()
    if ref is None or seconds <= 0:
        return None, None, 0
    return O, ref, threads


def _timed(fn, seconds, min_reps=3, max_reps=1000):
    reps, total = 0, 0.0
    while reps < min_reps or (total < seconds and reps < max_reps):
        t0 = time.perf_counter()
        fn()
        total += time.perf_counter() - t0
        reps += 1
    return total / reps, reps, total


def cpu_baseline_decode(synth, cfg, seconds):
    """The reference's decode attention for one layer-step of c1-c3 on its
    own AVX2 kernels (oracle/_ref): one sequence goes through
    Qwen2::attention (qwen2.cpp:1319-1380: attention_group_avx2 over span
    chunks + merge_gqa_chunks from 256 positions on), several sessions
    through forward_batch (qwen2.cpp:1705-1747: attention_head_avx2 per row
    and head). Every session sits at its context + half the decode steps
    (the run's mean span); the reference's flat cache, its own f32 int8
    scales. Attention only (the one-row store per session is a copy)."""
    O, ref, threads = _ref_team(seconds, decode_threads())
    if ref is None:
        return None
    sh = cfg.shape
    rng = np.random.default_rng(cfg.seed + 9)
    spans = [c + cfg.steps // 2 + 1 for c in cfg.contexts]
    rows_kv = sum(spans)
    i8 = cfg.fmt == synth.tge_kv.KV_I8
    if i8:
        kc = rng.integers(-127, 128, size=(rows_kv, sh.kv_dim), dtype=np.int8)
        vc = rng.integers(-127, 128, size=(rows_kv, sh.kv_dim), dtype=np.int8)
        ks = rng.uniform(0.005, 0.05, size=(rows_kv, sh.kv_dim // 32)).astype(np.float32)
        vs = rng.uniform(0.005, 0.05, size=(rows_kv, sh.kv_dim // 32)).astype(np.float32)
    else:
        kc = rng.standard_normal((rows_kv, sh.kv_dim)).astype(np.float16).view(np.uint16)
        vc = rng.standard_normal((rows_kv, sh.kv_dim)).astype(np.float16).view(np.uint16)
        ks = vs = np.zeros(1, np.float32)
    n = len(spans)
    q = rng.standard_normal((n, sh.q_dim)).astype(np.float32)
    out = np.empty((n, sh.q_dim), np.float32)
    fp = lambda a: a.ctypes.data_as(C.c_void_p)
    fmt = O.I8 if i8 else O.F16
    team = ref.ref_team_create(threads)
    try:
        if n == 1:
            group = sh.q_heads // sh.kv_heads
            scratch = np.empty(sh.kv_heads * 16 * group * (sh.head_dim + 2)
                               + sh.q_heads * spans[0] + sh.head_dim, np.float32)
            fn = lambda: ref.ref_baseline_decode(team, fmt, fp(q), fp(kc), fp(vc), fp(ks), fp(vs),
                                                 sh.q_heads, sh.kv_heads, sh.head_dim, spans[0],
                                                 fp(scratch), fp(out))
            schedule = "Qwen2::attention (qwen2.cpp:1319-1380)"
        else:
            bases = np.cumsum([0] + spans[:-1]).astype(np.int64) * sh.kv_dim
            s_arr = np.array(spans, np.int32)
            scores = np.empty(n * sh.q_heads * max(spans), np.float32)
            fn = lambda: ref.ref_baseline_batch_heads(team, fmt, fp(q), fp(kc), fp(vc), fp(ks),
                                                      fp(vs), fp(bases), fp(s_arr), n, sh.q_heads,
                                                      sh.kv_heads, sh.head_dim, max(spans),
                                                      fp(scores), fp(out))
            schedule = "forward_batch (qwen2.cpp:1705-1747)"
        per, reps, total = _timed(fn, seconds)
    finally:
        ref.ref_team_destroy(team)
    elem = 1 if i8 else 2
    alg = sum(2 * S * sh.kv_dim * elem + (2 * S * (sh.kv_dim // 32) * 4 if i8 else 0)
              + 2 * sh.q_dim * 4 for S in spans)
    return {
        "value": alg / per / 1e9,
        "unit": "GB/s",
        **cores_fields(threads, "decode: one thread per physical core (dispatch.cpp:77-94), "
                                f"at most the GPU's CPU share of {CPU_SHARE}"),
        "kind": "reference",
        "us_per_layer_step": 1e6 * per,
        "sample": (f"reference {'attention_group_avx2 + attention_head_avx2' if n == 1 else 'attention_head_avx2'} "
                   f"(oracle/_ref) under {schedule}, {threads} threads, spans {spans}, "
                   f"one layer-step's attention repeated {reps}x in {total:.1f} s"),
    }


def cpu_baseline_prefill(synth, cfg, seconds):
    """The reference's block prefill (attention_batch's query-block path,
    qwen2.cpp:1524-1571: attention_block_head_avx2, one task per query head)
    for each causal chunk of the c4 prompt over a flat f16 cache, on its own
    AVX2 kernel (oracle/_ref)."""
    O, ref, threads = _ref_team(seconds, prefill_threads())
    if ref is None:
        return None
    sh = cfg.shape
    rng = np.random.default_rng(cfg.seed + 9)
    n, ch = cfg.prompt, cfg.prefill_chunk
    kc = rng.standard_normal((n, sh.kv_dim)).astype(np.float16).view(np.uint16)
    vc = rng.standard_normal((n, sh.kv_dim)).astype(np.float16).view(np.uint16)
    q = rng.standard_normal((ch, sh.q_dim)).astype(np.float32)
    out = np.empty((ch, sh.q_dim), np.float32)
    scores = np.empty(sh.q_heads * ch * n, np.float32)
    fp = lambda a: a.ctypes.data_as(C.c_void_p)
    team = ref.ref_team_create(threads)
    per_chunk, reps_used = [], []
    try:
        for c in range(n // ch):
            ctx = (c + 1) * ch
            fn = lambda: ref.ref_baseline_block_prefill(team, O.F16, fp(q), fp(kc), fp(vc), ch,
                                                        c * ch, sh.q_heads, sh.kv_heads,
                                                        sh.head_dim, ctx, fp(scores), fp(out))
            per, reps, _ = _timed(fn, seconds / (n // ch), min_reps=1)
            per_chunk.append(per)
            reps_used.append(reps)
    finally:
        ref.ref_team_destroy(team)
    flops = sum(synth.prefill_flops(sh, c * ch, ch) for c in range(n // ch))
    return {
        "value": flops / sum(per_chunk) / 1e12,
        "unit": "TFLOP/s",
        **cores_fields(threads, "prefill: every logical core (thread_pool.cpp:337-340), "
                                f"at most the GPU's CPU share of {CPU_SHARE}"),
        "kind": "reference",
        "us_per_layer_chunk": [1e6 * t for t in per_chunk],
        "prompt_ms_est": 1e3 * sum(per_chunk) * sh.layers,
        "sample": (f"reference attention_block_head_avx2 (oracle/_ref) under attention_batch's "
                   f"query-block schedule (qwen2.cpp:1540-1571), {threads} threads, each of the "
                   f"{n // ch} chunks of one layer timed {reps_used}x; prompt time scaled to "
                   f"{sh.layers} layers"),
    }


def measured_traffic(workload, algorithmic_bytes):
    """HBM bytes per dispatch of the paged attention kernel at this run's
    algorithmic bytes, and where the figure comes from: the committed
    rocprofv3 counter summary of this workload (FETCH_SIZE and WRITE_SIZE per
    dispatch, each scaled by what the counter reads for a copy of known
    size) gives traffic per algorithmic byte, which scales to this run's
    spans. (None, None) when no summary covers the workload."""
    path = os.path.join(ROOT, "profiles", "paged_decode_kernel_c5_traffic.json")
    if not os.path.exists(path):
        return None, None
    with open(path) as f:
        t = json.load(f)
    if t.get("workload") != workload or not t.get("traffic_over_algorithmic"):
        return None, None
    ratio = float(t["traffic_over_algorithmic"])
    source = (f"rocprofv3 FETCH_SIZE + WRITE_SIZE per dispatch of this workload "
              f"(profiles/paged_decode_kernel_c5_traffic.json: {t['traffic_bytes_per_dispatch']} B "
              f"at {t['algorithmic_bytes_per_dispatch']} algorithmic B, ratio {ratio:.4f}) "
              f"times this run's algorithmic bytes")
    return int(round(ratio * algorithmic_bytes)), source


def copy_peak(nbytes=1 << 30, reps=5):
    """Read + write GB/s of device-to-device copies of 1 GiB on this GPU
    (the runtime's copy kernel; best of `reps`): the measured peak the
    roofline fraction is also quoted against."""
    import tge_kv as tk
    hip = tk.hip()
    src, dst = hip.malloc(nbytes), hip.malloc(nbytes)
    hip.memset(src, 1, nbytes)
    hip.sync()
    e0, e1 = hip.event(), hip.event()
    best = None
    for _ in range(reps + 1):
        hip.record(e0)
        hip.ok(hip.h.hipMemcpyAsync(C.c_void_p(dst), C.c_void_p(src), nbytes, hip.D2D, None),
               "hipMemcpyAsync D2D")
        hip.record(e1)
        ms = hip.elapsed_ms(e0, e1)
        best = ms if best is None else min(best, ms)
    hip.free(src)
    hip.free(dst)
    return 2 * nbytes / (best * 1e-3) / 1e9


def read_peak(nbytes=4 << 30, block_bytes=4352, reps=3):
    """HBM read ceiling of this GPU by hand-written read-only kernels
    (tge_read_ceiling): every byte of a 4 GiB buffer read once per launch
    (16x the 256 MB last-level cache), swept over workgroups per CU, best of
    `reps` launches per shape, timed with HIP events on the launch stream.
    "stream": 4 KiB chunks over the grid, 16 B per lane; "blocks": scattered
    page blocks of `block_bytes` (the c5 pool's 4352 B), one wave per block,
    the decode kernel's access shape."""
    import tge_kv as tk
    hip = tk.hip()
    lib = tk.lib()
    buf = hip.malloc(nbytes)
    hip.memset(buf, 1, nbytes)
    hip.sync()
    e0, e1 = hip.event(), hip.event()
    out = {"bytes": nbytes, "reps": reps, "kernel": "tge_read_ceiling (read_ceiling.hip)"}
    for name, pattern, sweep in (("stream", 0, (1, 2, 3, 4, 6, 8)), ("blocks", 1, (1, 2, 3, 4, 6, 8))):
        size = nbytes if pattern == 0 else (nbytes // block_bytes) * block_bytes
        best = {}
        for wpc in sweep:
            ms_best = None
            for _ in range(reps + 1):  # (the first launch warms up)
                hip.record(e0)
                tk.check(lib.tge_read_ceiling(buf, size, pattern, wpc, block_bytes, None), "read_ceiling")
                hip.record(e1)
                ms = hip.elapsed_ms(e0, e1)
                ms_best = ms if ms_best is None else min(ms_best, ms)
            best[wpc] = size / (ms_best * 1e-3) / 1e9
        top = max(best, key=best.get)
        out[name] = {"gbs": round(best[top], 1), "workgroups_per_cu": top,
                     "waves_per_cu": 4 * top,
                     "sweep_gbs": {str(k): round(v, 1) for k, v in best.items()}}
        if pattern == 1:
            out[name]["block_bytes"] = block_bytes
    hip.free(buf)
    return out


def calibrate_copy(nbytes=1 << 30, reps=3):
    """Device-to-device copies of a known size: the reference point that
    scales FETCH_SIZE / WRITE_SIZE readings to bytes (run under rocprofv3)."""
    import tge_kv as tk
    tk.require_gpu()
    hip = tk.hip()
    src, dst = hip.malloc(nbytes), hip.malloc(nbytes)
    hip.memset(src, 1, nbytes)
    hip.sync()
    e0, e1 = hip.event(), hip.event()
    hip.record(e0)
    for _ in range(reps):
        hip.ok(hip.h.hipMemcpyAsync(C.c_void_p(dst), C.c_void_p(src), nbytes, hip.D2D, None),
               "hipMemcpyAsync D2D")
    hip.record(e1)
    ms = hip.elapsed_ms(e0, e1) / reps
    hip.free(src)
    hip.free(dst)
    print(json.dumps({"copy_bytes": nbytes, "reps": reps, "ms_per_copy": round(ms, 4),
                      "read_plus_write_gbs": round(2 * nbytes / (ms * 1e-3) / 1e9, 1)}))


def main():
    args = parse()
    if args.calibrate_copy:
        calibrate_copy()
        return
    if args.read_ceiling:
        import tge_kv as tk
        tk.require_gpu()
        print(json.dumps(read_peak()), flush=True)
        return
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only: this build measures the single-GPU hot path "
              f"(asked for --gpus {args.gpus}); multi-GPU runs are not part of it.",
              file=sys.stderr)
        sys.exit(2)
    import synth
    import tge_kv as tk
    tk.require_gpu()
    cfgs = synth.configs()
    cfgs.update(synth.wide_head_configs())
    others = {}
    keys = [args.only] if args.only else (["c1", "c2", "c3", "c4", "prefix", "mixed", "d256",
                                           "p256"] if args.others else [])
    for key in keys:
        if key == "c5":
            continue
        if key == "prefix":
            log("[bench] prefix: 8 sessions sharing a 2048-token prefix (c5 shape)")
            others[key] = run_prefix(tk, synth, cfgs["c5"])
            log(f"[bench] prefix: {json.dumps(others[key])}")
            continue
        if key == "mixed":
            log("[bench] mixed: 32 verify sessions + one 512-token prefill chunk (c5 shape)")
            others[key] = run_mixed(tk, synth, cfgs["c5"])
            log(f"[bench] mixed: {json.dumps(others[key])}")
            continue
        cfg = cfgs[key]
        log(f"[bench] {key}: {cfg.note}")
        cpu_s = min(2.0, args.cpu_seconds / 5) if args.cpu else 0.0
        if key in ("c4", "p256"):
            others[key] = run_prefill(tk, synth, cfg)
            others[key]["cpu_baseline"] = cpu_baseline_prefill(synth, cfg, cpu_s)
        else:
            b = DecodeBench(tk, synth, cfg, cfg.steps + 4)
            r = b.run(cfg.steps, 4, 3)
            r["frac_attn"] = r["attn_gbs"] / HBM_PEAK_GBS
            r["frac_attn_kernel"] = r["attn_kernel_gbs"] / HBM_PEAK_GBS
            b.model.close()
            r["cpu_baseline"] = cpu_baseline_decode(synth, cfg, cpu_s)
            others[key] = r
        log(f"[bench] {key}: {json.dumps(others[key])}")
    if args.only and args.only != "c5":
        print(json.dumps({args.only: others[args.only]}))
        return
    copy_gbs = copy_peak()
    log(f"[bench] device-to-device copy: {copy_gbs:.0f} GB/s read + write")
    ceiling = read_peak()
    log(f"[bench] read ceiling: {json.dumps(ceiling)}")
    if args.others and not args.only and not args.fragment_c5:
        # c5 on a fragmented pool (free list shuffled before the sessions
        # allocate, so no session's pages are adjacent), a shorter run
        fcfg = synth.configs()["c5"]
        fcfg.fragmented = True
        log(f"[bench] c5 fragmented: {fcfg.note} (fragmented pool)")
        fb = DecodeBench(tk, synth, fcfg, 2 + 12)
        fr = fb.run(12, 2, 2)
        fb.model.close()
        fr["pool"] = "fragmented (free list shuffled before the sessions allocate)"
        fr["frac_attn_kernel"] = fr["attn_kernel_gbs"] / HBM_PEAK_GBS
        others["c5_fragmented"] = fr
        log(f"[bench] c5 fragmented: {json.dumps(fr)}")
    cfg = cfgs["c5"]
    if args.fragment_c5:
        cfg.fragmented = True
    log(f"[bench] c5: {cfg.note}{' (fragmented pool)' if cfg.fragmented else ''}")
    bench = DecodeBench(tk, synth, cfg, args.warmup + args.steps)
    log(f"[bench] c5 filled {sum(cfg.contexts)} positions x {cfg.shape.layers} layers in "
        f"{bench.fill_s:.1f} s; pool {bench.pages} pages")
    r = bench.run(args.steps, args.warmup, args.replay)
    log(f"[bench] c5: {json.dumps(r)}")
    cpu = None
    if args.cpu:
        cpu = cpu_baseline_c5(synth, cfg, args.cpu_seconds)
        log(f"[bench] cpu baseline: {json.dumps(cpu)}")
    traffic, traffic_source = measured_traffic(WORKLOAD_C5, r["kernel_bytes_per_launch"])
    line = {
        "metric": METRIC,
        "value": round(r["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["step_ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 KV (f16 scales) -> f16 MFMA, fp32 accumulate",
        "data": "synthetic (seeded N(0,1) q/k/v, 1% k outlier channels x8)",
        "config": {
            "workload": WORKLOAD_C5,
            "layers": cfg.shape.layers, "q_heads": cfg.shape.q_heads,
            "kv_heads": cfg.shape.kv_heads, "head_dim": cfg.shape.head_dim,
            "sessions": len(cfg.contexts), "queries_per_session": cfg.n_new,
            "mean_span": round(r["mean_context"], 1),
            "us_per_layer_step": round(r["us_per_layer_step"], 3),
            "tokens_per_s": round(r["tokens_per_s"], 1),
            "frac_of_hbm_peak": round(r["gbs"] / HBM_PEAK_GBS, 4),
            "attn_launch_us": round(r["attn_launch_us"], 3),
            "attn_kernel_us": round(r["attn_kernel_us"], 3),
            "merge_kernel_us": round(r["merge_kernel_us"], 3),
            "append_launch_us": round(r["append_launch_us"], 3),
            "append_rope_launch_us": round(r["append_rope_launch_us"], 3),
            "step_launch_us": round(r["step_launch_us"], 3),
            "step_path": r["step_path"],
            "sparse_attn_kernel_us": {k: round(v, 3) for k, v in r["sparse_attn_kernel_us"].items()},
            "decode_work_items": r["work_items"], "max_splits": r["max_splits"],
            "pool": "fragmented" if cfg.fragmented else "fresh (LIFO reuse after churn)",
        },
        "roofline": {
            "bound": "hbm",
            "kernel": ("paged_decode_kernel (int8 KV + f16 scales, head_dim 128, 2 row groups, 4 waves x 2 "
                       "workgroups per CU" + (", storing the step's new rows)" if r["kernel_stores_rows"] else ")")),
            "achieved": round(r["attn_kernel_gbs"], 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(r["attn_kernel_gbs"] / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "traffic_source": traffic_source,
            "kernel_us": round(r["attn_kernel_us"], 3),
            "algorithmic_bytes": r["kernel_bytes_per_launch"],
            "measured_copy_peak": round(copy_gbs, 1),
            "frac_of_measured_copy_peak": round(r["attn_kernel_gbs"] / copy_gbs, 4),
            "measured_read_peak": ceiling["stream"]["gbs"],
            "frac_of_measured_read_peak": round(r["attn_kernel_gbs"] / ceiling["stream"]["gbs"], 4),
            "measured_block_read_peak": ceiling["blocks"]["gbs"],
            "frac_of_measured_block_read_peak": round(r["attn_kernel_gbs"] / ceiling["blocks"]["gbs"], 4),
            "read_ceiling": ceiling,
        },
        "cpu_baseline": cpu,
        "configs": others,
    }
    print(json.dumps(line), flush=True)
    log(summary_line(line))


def summary_line(line):
    """One compact line with every configuration's headline figures (the
    tail of the run's stderr): us per layer-step (decode) or per layer-chunk
    (prefill), tokens/s, fraction of the HBM (decode) or f16 MFMA (prefill)
    peak, and the CPU baseline beside it."""
    parts = []
    cfgs = line.get("configs") or {}
    for key in ("c1", "c2", "c3"):
        r = cfgs.get(key)
        if not r:
            continue
        cpu = r.get("cpu_baseline") or {}
        parts.append(f"{key} {r['us_per_layer_step']:.2f}us/layer-step {r['tokens_per_s']:.0f}tok/s "
                     f"step-kernel {r['step_launch_us']:.2f}us {r['step_gbs']:.0f}GB/s "
                     f"frac {r['step_gbs'] / HBM_PEAK_GBS:.3f} "
                     f"cpu {cpu.get('us_per_layer_step', float('nan')):.0f}us")
    r = cfgs.get("c4")
    if r:
        cpu = r.get("cpu_baseline") or {}
        parts.append(f"c4 {'/'.join(f'{x:.1f}' for x in r['us_per_layer_chunk'])}us/layer-chunk "
                     f"{r['tokens_per_s']:.0f}tok/s {r['tflops']:.0f}TF/s mfma {r['mfma_util']:.3f} "
                     f"(kernel {r['attn_kernel_mfma_util']:.3f}) cpu {cpu.get('value', float('nan')):.2f}TF/s")
    c = line["config"]
    cpu = line.get("cpu_baseline") or {}
    parts.append(f"c5 {c['us_per_layer_step']:.1f}us/layer-step {c['tokens_per_s']:.0f}tok/s "
                 f"{line['value']:.0f}GB/s step {c['frac_of_hbm_peak']:.3f} kernel "
                 f"{line['roofline']['frac']:.3f} of 8TB/s, "
                 f"{line['roofline'].get('frac_of_measured_block_read_peak', float('nan')):.3f} of the "
                 f"measured block-read ceiling; cpu {cpu.get('value', float('nan')):.2f}GB/s")
    return "[bench] summary: " + " | ".join(parts)


if __name__ == "__main__":
    main()
