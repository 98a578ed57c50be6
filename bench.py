"""Benchmark of the paged-attention hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--configs 1,2,3,4,5,6,7,8,9] [--no-cpu]

One "step" is one pass of the hot path over one batch of synthetic input already resident in
HBM. The headline (the JSON `value`) is BASELINE.json's decode metric on configs[1]: batched
paged decode, batch 64, Qwen3-0.6B heads (16 q / 8 kv, d=128), contexts U[128, 4096], one
step = KV-cache write of the 64 new tokens + decode attention; value = algorithmic KV bytes
read per step (K+V of every context position, once per (sequence, kv_head)) / step time.
The step runs as one launch pair (ccinfer_decode_attention_write_kv: the KV write inside the
decode kernel, then the merge); the reference's two launcher calls (write_kv_cache, then
decode_attention) are timed beside it (configs."2...".unfused_*).
The other configurations are reported under "configs"; "6" is the fused decode prologue
(split QKV + q/k RMSNorm + RoPE + KV write in one launch), in algorithmic bytes per second;
"7" is the per-step batch metadata built on the device, beside the reference's host path;
"8" is decode over an fp8 (E4M3, per-row scale) cache, in bytes actually read and in the
bf16 bytes the same attention covers, and the configs[2] prefill over an fp8 cache. rank 0 prints ONE JSON line.

Timing: about 0.2 s of untimed repetitions (clock settle) and W untimed warm-up steps, then
exactly K steps bracketed by device synchronisation; CPU baselines run after all GPU timings;
per-op kernel time is measured with HIP events recorded on the stream the kernels run on.
cpu_baseline: the CPU oracle (a C restatement of the reference's CPU attention path) on the
box's host cores, on the same workload. `--profile-op NAME` runs only that op in a loop (for
rocprofv3 counter runs) and prints nothing else.
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

from ccinfer_amd import SideStream, _lib  # noqa: E402
from ccinfer_amd import workloads as W  # noqa: E402

HBM_PEAK = 8.0e12          # B/s, MI355X HBM3E
BF16_PEAK = 2.5e15         # FLOP/s, MI355X dense bf16 MFMA
PROFILES = ROOT / "profiles"


class Ops:
    """Preallocated C-ABI calls on one stream (no allocation inside the timed loop)."""

    def __init__(self, w: W.PagedWorkload, dev, stream: torch.cuda.Stream):
        self.w, self.dev, self.stream = w, dev, stream
        self.lib = _lib.load()
        self.meta = w.device_meta(dev)
        self.s = stream.cuda_stream
        self.out = torch.empty_like(w.q)
        if w.query_start_loc is None:
            n = self.lib.ccinfer_decode_workspace_size(w.batch, w.mbpr, w.hq, w.hkv, w.d, 16)
        else:
            n = self.lib.ccinfer_prefill_workspace_size(w.batch, w.q.shape[0], w.mbpr, w.hq,
                                                        w.hkv, w.d, 16)
        self.ws_bytes = int(n)
        self.ws = torch.zeros(max(1, self.ws_bytes), dtype=torch.uint8, device=dev)
        # a mixed batch's decode items run on this side stream beside the prompt tiles
        self.side = SideStream(dev)

    def write(self):
        w = self.w
        rc = self.lib.ccinfer_write_kv_cache(
            w.k_new.data_ptr(), w.v_new.data_ptr(), w.k_cache.data_ptr(), w.v_cache.data_ptr(),
            self.meta["slot_mapping"].data_ptr(), w.k_new.shape[0], w.hkv, w.d,
            w.k_cache.shape[0], self.s)
        assert rc == 0, rc

    def decode(self):
        w = self.w
        rc = self.lib.ccinfer_decode_attention(
            w.q.data_ptr(), w.k_cache.data_ptr(), w.v_cache.data_ptr(),
            self.meta["block_table"].data_ptr(), self.meta["context_lens"].data_ptr(),
            self.out.data_ptr(), w.batch, w.mbpr, w.hq, w.hkv, w.d, 16, self.ws.data_ptr(),
            self.ws_bytes, self.s)
        assert rc == 0, rc

    def decode_write(self):
        """The decode step with the new tokens' KV write in the decode launch."""
        w = self.w
        rc = self.lib.ccinfer_decode_attention_write_kv(
            w.q.data_ptr(), w.k_new.data_ptr(), w.v_new.data_ptr(), w.k_cache.data_ptr(),
            w.v_cache.data_ptr(), self.meta["block_table"].data_ptr(),
            self.meta["context_lens"].data_ptr(), self.out.data_ptr(), w.batch, w.mbpr, w.hq,
            w.hkv, w.d, 16, w.k_cache.shape[0], self.ws.data_ptr(), self.ws_bytes, self.s)
        assert rc == 0, rc

    def prefill(self):
        w = self.w
        rc = self.lib.ccinfer_prefill_attention_overlap(
            w.q.data_ptr(), w.k_cache.data_ptr(), w.v_cache.data_ptr(),
            self.meta["block_table"].data_ptr(), self.meta["query_start_loc"].data_ptr(),
            self.meta["context_lens"].data_ptr(), self.out.data_ptr(), w.batch, w.q.shape[0],
            w.mbpr, w.hq, w.hkv, w.d, 16, self.ws.data_ptr(), self.ws_bytes, self.s,
            *self.side.handles())
        assert rc == 0, rc


SETTLE_S = 0.2  # untimed repetitions of the step before its warm-up, so clocks are ramped


def time_loop(fn, steps: int, warmup: int, stream: torch.cuda.Stream):
    """Returns (event ms per step, host-clock ms per step): SETTLE_S seconds of untimed
    repetitions, `warmup` untimed steps, then exactly `steps` timed steps."""
    with torch.cuda.stream(stream):
        t_settle = time.perf_counter()
        while time.perf_counter() - t_settle < SETTLE_S:
            for _ in range(4):
                fn()
            torch.cuda.synchronize()
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        start.record(stream)
        for _ in range(steps):
            fn()
        end.record(stream)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
    return start.elapsed_time(end) / steps, (t1 - t0) * 1e3 / steps


def side_span_ms(ops: "Ops", stream: torch.cuda.Stream, n: int) -> float:
    """Median time from the start of a mixed prefill step (on `stream`) to the end of its
    side-stream work (the decode items), over n steps."""
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(n)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(n)]
    with torch.cuda.stream(stream):
        for a, b in zip(starts, ends):
            a.record(stream)
            ops.prefill()
            b.record(ops.side.stream)
            torch.cuda.synchronize()
    return float(np.median([a.elapsed_time(b) for a, b in zip(starts, ends)]))


def traffic_from_profiles(kernel_tag: str):
    """HBM bytes per dispatch recorded by the rocprofv3 --pmc runs (profiles/*.md)."""
    f = PROFILES / f"{kernel_tag}.pmc.md"
    if not f.exists():
        return None
    m = re.search(r"hbm_bytes_per_dispatch:\s*([0-9.eE+]+)", f.read_text())
    return float(m.group(1)) if m else None


def cpu_threads() -> int:
    return max(1, min(16, os.cpu_count() or 1))


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def u16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def cpu_decode_baseline(w: W.PagedWorkload, budget_s: float, pairs=None, nthreads=None):
    """Times the oracle decode on the host (all rows, or `pairs`); returns (s/step, reps)."""
    import oracle  # test infrastructure: the baseline being reported, never the product
    q, k, v = u16(w.q), u16(w.k_cache), u16(w.v_cache)
    nt = nthreads or cpu_threads()
    reps, t0 = 0, time.perf_counter()
    while True:
        oracle.decode(q, k, v, w.block_table, w.context_lens, nthreads=nt, pairs=pairs)
        reps += 1
        if time.perf_counter() - t0 >= budget_s:
            break
    return (time.perf_counter() - t0) / reps, reps


def cpu_prefill_baseline(w: W.PagedWorkload, pairs, budget_s: float):
    import oracle
    q, k, v = u16(w.q), u16(w.k_cache), u16(w.v_cache)
    nt = cpu_threads()
    reps, t0 = 0, time.perf_counter()
    while True:
        oracle.prefill(q, k, v, w.block_table, w.query_start_loc, w.context_lens, nthreads=nt,
                       pairs=pairs)
        reps += 1
        if time.perf_counter() - t0 >= budget_s:
            break
    return (time.perf_counter() - t0) / reps, reps


def prologue_call(w: W.PrologueWorkload, stream: torch.cuda.Stream):
    lib = _lib.load()
    args = (w.qkv.data_ptr(), w.q_norm_w.data_ptr(), w.k_norm_w.data_ptr(),
            w.positions.data_ptr(), w.rope_cache.data_ptr(), w.slot_mapping.data_ptr(),
            w.q_out.data_ptr(), w.k_cache.data_ptr(), w.v_cache.data_ptr(), w.tokens, w.hq,
            w.hkv, w.d, w.rope_cache.shape[0], w.k_cache.shape[0], 1e-6, stream.cuda_stream)

    def fn():
        rc = lib.ccinfer_qkv_prologue(*args)
        assert rc == 0, rc
    return fn


def cpu_prologue_baseline(w: W.PrologueWorkload, budget_s: float):
    """Times the oracle prologue (the reference's five steps in sequence) on one host core."""
    import oracle
    qkv, qn, kn = u16(w.qkv), u16(w.q_norm_w), u16(w.k_norm_w)
    pos, sm = w.positions.cpu().numpy(), w.slot_mapping.cpu().numpy()
    rc = w.rope_cache.cpu().numpy()
    kc, vc = u16(w.k_cache), u16(w.v_cache)
    reps, t0 = 0, time.perf_counter()
    while True:
        oracle.qkv_prologue(qkv, qn, kn, pos, rc, sm, kc, vc, w.hq, w.hkv, w.d, 1e-6)
        reps += 1
        if time.perf_counter() - t0 >= budget_s:
            break
    return (time.perf_counter() - t0) / reps, reps


def batch_items(rng, batch: int, ctx_lo: int, ctx_hi: int, new_tokens: int, decode: bool):
    """Compact per-item records of one step (tokens in the cache, new tokens, flags, block
    lists as CSR) with distinct random blocks."""
    ctx = rng.integers(ctx_lo, ctx_hi + 1, batch).astype(np.int64) + new_tokens
    kvw = (ctx - new_tokens).astype(np.int32)
    new = np.full(batch, new_tokens, np.int32)
    flags = np.full(batch, 1 if decode else 2, np.int32)
    counts = -(-ctx // 16)
    start = np.zeros(batch + 1, np.int32)
    start[1:] = np.cumsum(counts)
    blocks = rng.permutation(int(start[-1]) * 2)[:start[-1]].astype(np.int32)
    return kvw, new, flags, start, blocks, int(counts.max()), int(start[-1]) * 2


def host_metadata_path(items, T, mbpr, ncb, dev, reps: int):
    """The reference's host path for one step, timed: build the arrays on the host (the
    oracle restates BatchTranslator's loops), upload them with seven synchronous copies
    (batch_translator.cpp:387-420), copy four back and check them (model_runner.h:102-171).
    Returns ms per step."""
    import oracle
    kvw, new, flags, start, blocks = items
    b = len(kvw)
    bufs = {k: torch.empty(n, dtype=torch.int32, device=dev)
            for k, n in (("tok", T), ("pos", T), ("sm", T), ("bt", b * mbpr), ("qsl", b + 1),
                         ("ctx", b), ("li", b))}
    t0 = time.perf_counter()
    for _ in range(reps):
        st, o = oracle.build_batch_metadata(kvw, new, flags, start, blocks, T, mbpr, 16, ncb)
        host = {"tok": o["positions"], "pos": o["positions"], "sm": o["slot_mapping"],
                "bt": o["block_table"].ravel(), "qsl": o["query_start_loc"],
                "ctx": o["context_lens"], "li": o["logits_indices"]}
        for k, v in host.items():
            bufs[k].copy_(torch.from_numpy(v))
        torch.cuda.synchronize()
        for k in ("qsl", "pos", "ctx", "li"):
            v = bufs[k].cpu().numpy()
            assert v.size > 0
    return (time.perf_counter() - t0) * 1e3 / reps


def prefill_pair_flops(w: W.PagedWorkload, pairs) -> int:
    """FLOPs of the (query row, head) pairs: 4*D per visible key."""
    qsl = w.query_start_loc
    tot = 0
    for r, _h in pairs:
        b = int(np.searchsorted(qsl, r, side="right") - 1)
        ql = int(qsl[b + 1] - qsl[b])
        pre = int(w.context_lens[b]) - ql
        tot += pre + (r - int(qsl[b])) + 1
    return 4 * w.d * tot


def bench_decode(w, dev, steps, warmup, with_write, stream):
    """with_write: the step is the KV write of the new tokens + decode, timed both as one
    launch (ccinfer_decode_attention_write_kv: the step) and as the reference's two launcher
    calls (write_kv_cache, then decode_attention: "unfused_*")."""
    ops = Ops(w, dev, stream)
    step = ops.decode_write if with_write else ops.decode
    ms, host_ms = time_loop(step, steps, warmup, stream)
    dec_ms, _ = time_loop(ops.decode, steps, warmup, stream)
    res = {"ms_per_step": ms, "host_ms_per_step": host_ms, "decode_ms": dec_ms,
           "kv_bytes": w.kv_bytes()}
    if with_write:
        wr_ms, _ = time_loop(ops.write, steps, warmup, stream)
        un_ms, _ = time_loop(lambda: (ops.write(), ops.decode()), steps, warmup, stream)
        res["write_ms"] = wr_ms
        res["unfused_ms_per_step"] = un_ms
        res["unfused_kv_GBps"] = w.kv_bytes() / (un_ms * 1e-3) / 1e9
    res["kv_GBps"] = w.kv_bytes() / (ms * 1e-3) / 1e9
    res["decode_kernel_GBps"] = w.kv_bytes() / (dec_ms * 1e-3) / 1e9
    res["hbm_frac"] = res["decode_kernel_GBps"] * 1e9 / HBM_PEAK
    return res


def run(args):
    dev = torch.device("cuda:0")
    stream = torch.cuda.Stream(device=dev)  # default priority
    configs = [int(c) for c in args.configs.split(",") if c]
    out = {}
    head = None
    nt = cpu_threads()
    # CPU baselines run after every GPU measurement, so no GPU timing follows an idle GPU
    deferred = []

    if 1 in configs:
        w = W.decode_single(device=dev)
        r = bench_decode(w, dev, max(args.steps, 50), args.warmup, False, stream)

        def cpu1(w=w, r=r):
            s, reps = cpu_decode_baseline(w, 1.0)
            r["cpu_GBps"] = w.kv_bytes() / s / 1e9
        deferred.append(cpu1)
        out["1_decode_b1_ctx512"] = r
        del w

    if 2 in configs:
        w = W.decode_batched(device=dev)
        r = bench_decode(w, dev, args.steps, args.warmup, True, stream)

        def cpu2(w=w, r=r):
            s, reps = cpu_decode_baseline(w, args.cpu_budget)
            r["cpu_GBps"] = w.kv_bytes() / s / 1e9
            r["cpu_reps"] = reps
            # the faithful single-thread loop, on sequences 0-7 (all q-heads)
            pairs = np.array([[b, h] for b in range(8) for h in range(w.hq)], np.int32)
            s1, _ = cpu_decode_baseline(w, 2.0, pairs=pairs, nthreads=1)
            r["cpu_1thread_GBps"] = (int(w.context_lens[:8].astype(np.int64).sum()) * w.hkv *
                                     w.d * 4 / s1 / 1e9)
        deferred.append(cpu2)
        head = (w, r)
        out["2_decode_b64_ctx128-4096"] = r

    if 3 in configs:
        w = W.prefill_prefix(device=dev)
        ops = Ops(w, dev, stream)
        ms, host_ms = time_loop(ops.prefill, args.steps, args.warmup, stream)
        wr_ms, _ = time_loop(ops.write, args.steps, args.warmup, stream)
        flops = W.prefill_flops(w)
        r = {"ms_per_step": ms, "host_ms_per_step": host_ms, "write_ms": wr_ms, "flops": flops,
             "TFLOPs": flops / (ms * 1e-3) / 1e12}
        r["mfma_frac"] = r["TFLOPs"] * 1e12 / BF16_PEAK

        def cpu3(w=w, r=r):
            rng = np.random.default_rng(0)
            pairs = np.stack([rng.integers(0, w.q.shape[0], 256), rng.integers(0, w.hq, 256)],
                             1).astype(np.int32)
            s, reps = cpu_prefill_baseline(w, pairs, 1.0)
            r["cpu_TFLOPs"] = prefill_pair_flops(w, pairs) / s / 1e12
            r["cpu_sample"] = "256 random (query row, q_head) pairs"
        deferred.append(cpu3)
        out["3_prefill_8x(512+1536)"] = r
        del w, ops

    if 4 in configs:
        w = W.mixed_step(device=dev)
        ops = Ops(w, dev, stream)
        ms, host_ms = time_loop(ops.prefill, args.steps, args.warmup, stream)
        flops = W.prefill_flops(w)
        dbytes = W.decode_items_kv_bytes(w)
        roof_s = dbytes / HBM_PEAK + flops / BF16_PEAK
        r = {"ms_per_step": ms, "host_ms_per_step": host_ms, "decode_kv_bytes": dbytes,
             "prefill_flops": flops, "roofline_ms": roof_s * 1e3,
             "roofline_frac": roof_s / (ms * 1e-3)}
        # The decode items run on the side stream beside the prompt tiles: their span is
        # from the step's start (planner included) to the side stream's last kernel.
        span = side_span_ms(ops, stream, max(5, args.steps // 4))
        r["decode_span_ms"] = span
        r["decode_GBps"] = dbytes / (span * 1e-3) / 1e9
        r["decode_hbm_frac"] = dbytes / (span * 1e-3) / HBM_PEAK
        out["4_mixed_4x512+128dec"] = r
        del w, ops

    if 5 in configs:
        w = W.decode_long(device=dev)
        r = bench_decode(w, dev, max(5, args.steps // 2), args.warmup, False, stream)

        def cpu5(w=w, r=r):
            pairs = np.array([[0, h] for h in range(w.hq)], np.int32)
            s, reps = cpu_decode_baseline(w, 1.0, pairs=pairs)
            r["cpu_GBps"] = int(w.context_lens[0]) * w.hkv * w.d * 4 / s / 1e9
            r["cpu_sample"] = "sequence 0, all 32 q-heads"
        deferred.append(cpu5)
        out["5_decode_b32_ctx32768_gqa4"] = r
        del w

    if 6 in configs:
        # fused decode prologue: a decode batch of 64 tokens (configs[1]'s batch) and the
        # 12288 query tokens of configs[2] (the HBM-bound size)
        for tokens, key in ((64, "6_prologue_t64"), (12288, "6_prologue_t12288")):
            w = W.prologue(device=dev, tokens=tokens)
            ms, host_ms = time_loop(prologue_call(w, stream), max(args.steps, 50),
                                    args.warmup, stream)
            r = {"ms_per_step": ms, "host_ms_per_step": host_ms, "bytes": w.bytes(),
                 "GBps": w.bytes() / (ms * 1e-3) / 1e9}
            r["hbm_frac"] = r["GBps"] * 1e9 / HBM_PEAK
            if tokens == 64:
                def cpu6(w=w, r=r):
                    s, reps = cpu_prologue_baseline(w, 1.0)
                    r["cpu_GBps"] = w.bytes() / s / 1e9
                    r["cpu_sample"] = "the same 64 tokens, 1 thread"
                deferred.append(cpu6)
            out[key] = r
            del w

    if 7 in configs:
        # per-step metadata built on the device (BatchTranslator's arrays + checks) for the
        # configs[1] decode batch and the configs[2] prefill batch
        lib = _lib.load()
        rng = np.random.default_rng(7)
        for key, shape in (("7_batch_meta_decode_b64", (64, 128, 4096, 1, True)),
                           ("7_batch_meta_prefill_8x1536", (8, 512, 512, 1536, False))):
            kvw, new, flags, start, blocks, mbpr, ncb = batch_items(rng, *shape)
            T = int(new.sum())
            d = [torch.from_numpy(a).to(dev) for a in (kvw, new, flags, start, blocks)]
            outs = [torch.empty(n, dtype=torch.int32, device=dev)
                    for n in (T, T, len(kvw) * mbpr, len(kvw) + 1, len(kvw), len(kvw), 1)]

            def build():
                rc = lib.ccinfer_build_batch_metadata(
                    *[t.data_ptr() for t in d], len(kvw), T, len(blocks), mbpr, 16, ncb,
                    *[t.data_ptr() for t in outs], stream.cuda_stream)
                assert rc == 0, rc
            ms, host_ms = time_loop(build, max(args.steps, 50), args.warmup, stream)
            assert int(outs[-1].item()) == 0
            r = {"ms_per_step": ms, "host_ms_per_step": host_ms, "batch": len(kvw),
                 "tokens": T, "max_blocks_per_req": mbpr}
            if not args.no_cpu:
                r["reference_host_path_ms"] = host_metadata_path(
                    (kvw, new, flags, start, blocks), T, mbpr, ncb, dev, 20)
                r["reference_host_path_note"] = ("host build (oracle restatement of the "
                                                 "translator loops) + 7 uploads + sync + "
                                                 "4 validation copy-backs")
            out[key] = r

    if 8 in configs:
        # fp8 KV cache: the configs[1] and configs[4] batches with their caches quantised by
        # the fp8 write kernel; bytes = K+V bytes plus the row scales actually read
        lib = _lib.load()
        def quantise(w):
            slots = w.k_cache.shape[0]
            kc = torch.empty((slots, w.hkv, w.d), dtype=torch.uint8, device=dev)
            vc = torch.empty_like(kc)
            nsc = -(-slots // 16) * 16 * w.hkv
            ks = torch.empty(nsc, dtype=torch.float32, device=dev)
            vs = torch.empty_like(ks)
            ident = torch.arange(slots, dtype=torch.int32, device=dev)
            rc = lib.ccinfer_write_kv_cache_fp8(
                w.k_cache.data_ptr(), w.v_cache.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                ks.data_ptr(), vs.data_ptr(), ident.data_ptr(), slots, w.hkv, w.d, slots,
                stream.cuda_stream)
            assert rc == 0, rc
            return kc, vc, ks, vs

        for key, make in (("8_fp8_decode_b64_ctx128-4096", W.decode_batched),
                          ("8_fp8_decode_b32_ctx32768_gqa4", W.decode_long)):
            w = make(device=dev)
            kc, vc, ks, vs = quantise(w)
            meta = w.device_meta(dev)
            outp = torch.empty_like(w.q)
            n = lib.ccinfer_decode_workspace_size(w.batch, w.mbpr, w.hq, w.hkv, w.d, 16)
            ws = torch.zeros(max(1, n), dtype=torch.uint8, device=dev)

            def dec():
                rc = lib.ccinfer_decode_attention_fp8(
                    w.q.data_ptr(), kc.data_ptr(), vc.data_ptr(), ks.data_ptr(), vs.data_ptr(),
                    meta["block_table"].data_ptr(), meta["context_lens"].data_ptr(),
                    outp.data_ptr(), w.batch, w.mbpr, w.hq, w.hkv, w.d, 16, ws.data_ptr(), n,
                    stream.cuda_stream)
                assert rc == 0, rc
            ms, host_ms = time_loop(dec, args.steps, args.warmup, stream)
            sum_ctx = int(w.context_lens.astype(np.int64).sum())
            nbytes = sum_ctx * w.hkv * (w.d + 4) * 2
            r = {"ms_per_step": ms, "host_ms_per_step": host_ms, "bytes": nbytes,
                 "GBps": nbytes / (ms * 1e-3) / 1e9,
                 "bf16_equivalent_GBps": w.kv_bytes() / (ms * 1e-3) / 1e9}
            r["hbm_frac"] = r["GBps"] * 1e9 / HBM_PEAK
            out[key] = r
            del w, kc, vc, ks, vs

        # prefill over the fp8 cache: the configs[2] batch (same FLOPs as "3")
        w = W.prefill_prefix(device=dev)
        kc, vc, ks, vs = quantise(w)
        meta = w.device_meta(dev)
        outp = torch.empty_like(w.q)
        T = w.q.shape[0]
        n = lib.ccinfer_prefill_workspace_size(w.batch, T, w.mbpr, w.hq, w.hkv, w.d, 16)
        ws = torch.zeros(max(1, n), dtype=torch.uint8, device=dev)

        def pre8():
            rc = lib.ccinfer_prefill_attention_fp8(
                w.q.data_ptr(), kc.data_ptr(), vc.data_ptr(), ks.data_ptr(), vs.data_ptr(),
                meta["block_table"].data_ptr(), meta["query_start_loc"].data_ptr(),
                meta["context_lens"].data_ptr(), outp.data_ptr(), w.batch, T, w.mbpr, w.hq,
                w.hkv, w.d, 16, ws.data_ptr(), n, stream.cuda_stream)
            assert rc == 0, rc
        ms, host_ms = time_loop(pre8, args.steps, args.warmup, stream)
        flops = W.prefill_flops(w)
        r = {"ms_per_step": ms, "host_ms_per_step": host_ms, "flops": flops,
             "TFLOPs": flops / (ms * 1e-3) / 1e12}
        r["mfma_frac"] = r["TFLOPs"] * 1e12 / BF16_PEAK
        out["8_fp8_prefill_8x(512+1536)"] = r
        del w, kc, vc, ks, vs

    if 9 in configs:
        # shared cached prompts: 64 requests on one 2048-token prefix + U[128, 1024] private
        # tokens (prefix-cache hits), through the shared-prefix entry and through plain
        # decode; bytes = every request's positions (the plain decode's algorithmic bytes)
        # and the distinct positions (each prefix once)
        lib = _lib.load()
        for key, groups in (("9_decode_shared_b64_1x2048+128-1024", 1),
                            ("9_decode_shared_b64_4x2048+128-1024", 4)):
            w = W.decode_shared_prefix(device=dev, groups=groups)
            meta = w.device_meta(dev)
            outp = torch.empty_like(w.q)
            n = lib.ccinfer_decode_shared_workspace_size(w.batch, w.mbpr, w.hq, w.hkv, w.d, 16)
            ws = torch.zeros(max(1, n), dtype=torch.uint8, device=dev)

            def shared_call(w=w, meta=meta, outp=outp, n=n, ws=ws):
                rc = lib.ccinfer_decode_attention_shared_prefix(
                    w.q.data_ptr(), w.k_cache.data_ptr(), w.v_cache.data_ptr(),
                    meta["block_table"].data_ptr(), meta["context_lens"].data_ptr(),
                    outp.data_ptr(), w.batch, w.mbpr, w.hq, w.hkv, w.d, 16, ws.data_ptr(), n,
                    stream.cuda_stream)
                assert rc == 0, rc
            ms, host_ms = time_loop(shared_call, args.steps, args.warmup, stream)
            plain_ms, _ = time_loop(Ops(w, dev, stream).decode, args.steps, args.warmup, stream)
            uniq = w.info["unique_kv_bytes"]
            r = {"ms_per_step": ms, "host_ms_per_step": host_ms, "plain_decode_ms": plain_ms,
                 "kv_bytes": w.kv_bytes(), "unique_kv_bytes": uniq,
                 "kv_GBps": w.kv_bytes() / (ms * 1e-3) / 1e9,
                 "unique_GBps": uniq / (ms * 1e-3) / 1e9,
                 "plain_kv_GBps": w.kv_bytes() / (plain_ms * 1e-3) / 1e9}
            r["unique_hbm_frac"] = r["unique_GBps"] * 1e9 / HBM_PEAK
            out[key] = r
            del w, ws

    torch.cuda.synchronize()
    if not args.no_cpu:
        for f in deferred:
            f()
    return head, out, nt


COPY_BYTES = 1 << 30


def profile(op: str, iters: int) -> None:
    """Runs one op `iters` times on its benchmark workload (for rocprofv3 runs)."""
    dev = torch.device("cuda:0")
    stream = torch.cuda.Stream(device=dev)
    if op == "copy":  # calibration: a plain copy of known size (1 GiB read + 1 GiB written)
        src = torch.ones(COPY_BYTES // 2, dtype=torch.bfloat16, device=dev)
        dst = torch.empty_like(src)
        fn = lambda: dst.copy_(src)  # noqa: E731
    elif op == "prologue":
        fn = prologue_call(W.prologue(device=dev, tokens=12288), stream)
    elif op in ("decode_b600", "decode_b2048"):
        # batches past 256 requests (the flat plan's index kernel): 600 x U[100, 3000]
        # positions (snapped ranges), 2048 x U[100, 1000] (one range per request)
        batch, lo, hi = (600, 100, 3000) if op == "decode_b600" else (2048, 100, 1000)
        w = W.decode_batched(device=dev, seed=5, batch=batch, ctx_lo=lo, ctx_hi=hi, hq=32,
                             hkv=8, with_write=False)
        fn = Ops(w, dev, stream).decode
    elif op in ("decode_d64", "decode_d80", "decode_d96", "decode_d128", "decode_d192",
                "decode_g32", "decode_g32_hkv1"):
        # the sweep's 64 x 4096 decode at other head dims and query-group sizes
        hq, hkv, d = {"decode_d64": (16, 8, 64), "decode_d80": (16, 8, 80),
                      "decode_d96": (16, 8, 96), "decode_d128": (16, 8, 128),
                      "decode_d192": (8, 4, 192), "decode_g32": (64, 2, 128),
                      "decode_g32_hkv1": (32, 1, 128)}[op]
        w = W.decode_batched(device=dev, batch=64, ctx_lo=4096, ctx_hi=4096, hq=hq, hkv=hkv,
                             d=d, with_write=False)
        fn = Ops(w, dev, stream).decode
    elif op in ("decode_shared", "decode_unshared"):
        # 64 requests on one 2048-token cached prompt + U[128, 1024] private tokens, through
        # the shared-prefix entry or plain decode
        w = W.decode_shared_prefix(device=dev)
        ops = Ops(w, dev, stream)
        if op == "decode_shared":
            lib = _lib.load()
            meta = w.device_meta(dev)
            n = lib.ccinfer_decode_shared_workspace_size(w.batch, w.mbpr, w.hq, w.hkv, w.d, 16)
            ws = torch.zeros(max(1, n), dtype=torch.uint8, device=dev)

            def fn():
                rc = lib.ccinfer_decode_attention_shared_prefix(
                    w.q.data_ptr(), w.k_cache.data_ptr(), w.v_cache.data_ptr(),
                    meta["block_table"].data_ptr(), meta["context_lens"].data_ptr(),
                    ops.out.data_ptr(), w.batch, w.mbpr, w.hq, w.hkv, w.d, 16, ws.data_ptr(),
                    n, stream.cuda_stream)
                assert rc == 0, rc
        else:
            fn = ops.decode
    elif op in ("shared_prefix", "private_prefix"):
        # 16 sequences x (4096 cached + 256 new): one prefix shared by all, or 16 copies
        share = tuple((i, 0) for i in range(1, 16)) if op == "shared_prefix" else ()
        w = W.prefill_prefix(device=dev, seed=11, n_seqs=16, prefix=4096, new=256,
                             share_pairs=share)
        fn = Ops(w, dev, stream).prefill
    elif op in ("shared_prefix_ragged", "private_prefix_ragged"):
        # 16 sequences x (4096 cached + 64..1024 new): unequal new lengths, one shared prefix
        # (or 16 private copies) -- the sharers' tiles differ in length
        share = tuple((i, 0) for i in range(1, 16)) if op == "shared_prefix_ragged" else ()
        w = W.prefill_prefix(device=dev, seed=12, n_seqs=16, prefix=4096,
                             new=[64 + 64 * i for i in range(16)], share_pairs=share)
        fn = Ops(w, dev, stream).prefill
    else:
        w = {"decode": W.decode_batched, "write": W.decode_batched, "prefill": W.prefill_prefix,
             "mixed": W.mixed_step, "long": W.decode_long}[op](device=dev)
        ops = Ops(w, dev, stream)
        fn = {"decode": ops.decode, "write": ops.write, "prefill": ops.prefill,
              "mixed": ops.prefill, "long": ops.decode}[op]
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        for _ in range(iters):
            fn()
    torch.cuda.synchronize()


def sweep(kind: str) -> None:
    """Prints a markdown table of the decode or prefill op across shapes beyond the fixed
    configs (synthetic data, event timing as in the configs)."""
    dev = torch.device("cuda:0")
    stream = torch.cuda.Stream()
    print(f"| {kind} shape | time (us) | achieved | fraction of peak |")
    print("|---|---|---|---|")
    if kind == "decode":
        for hq, hkv in ((16, 8), (32, 8)):
            for batch, ctx in ((1, 4096), (8, 4096), (32, 4096), (64, 1024), (64, 4096),
                               (128, 2048), (256, 1024), (16, 32768), (64, 16384)):
                w = W.decode_batched(device=dev, batch=batch, ctx_lo=ctx, ctx_hi=ctx, hq=hq,
                                     hkv=hkv, with_write=False)
                ops = Ops(w, dev, stream)
                ms, _ = time_loop(ops.decode, 20, 3, stream)
                gbs = w.kv_bytes() / (ms * 1e-3) / 1e9
                print(f"| B={batch} ctx={ctx} Hq/Hkv={hq}/{hkv} | {ms * 1e3:.1f} | "
                      f"{gbs:.0f} GB/s | {gbs * 1e9 / HBM_PEAK:.0%} HBM |", flush=True)
                del w, ops
                torch.cuda.empty_cache()
        # other head dims (below 64 / 128 / 256: padded MFMA tiles) and query-group sizes
        for hq, hkv, d in ((16, 8, 64), (16, 8, 96), (16, 8, 80), (8, 4, 192), (16, 8, 256),
                           (64, 2, 128), (32, 1, 128)):
            w = W.decode_batched(device=dev, batch=64, ctx_lo=4096, ctx_hi=4096, hq=hq,
                                 hkv=hkv, d=d, with_write=False)
            ops = Ops(w, dev, stream)
            ms, _ = time_loop(ops.decode, 20, 3, stream)
            gbs = w.kv_bytes() / (ms * 1e-3) / 1e9
            print(f"| B=64 ctx=4096 Hq/Hkv={hq}/{hkv} d={d} | {ms * 1e3:.1f} | "
                  f"{gbs:.0f} GB/s | {gbs * 1e9 / HBM_PEAK:.0%} HBM |", flush=True)
            del w, ops
            torch.cuda.empty_cache()
        # spread context lengths and batches past 256 requests (the flat plan's index kernel:
        # equal, snapped or whole-request ranges)
        for batch, lo, hi, hq, hkv in ((64, 100, 3000, 32, 8), (256, 100, 3000, 32, 8),
                                       (600, 100, 3000, 32, 8), (1024, 100, 3000, 32, 4),
                                       (1000, 500, 1500, 32, 8), (2048, 100, 1000, 32, 8)):
            w = W.decode_batched(device=dev, seed=5, batch=batch, ctx_lo=lo, ctx_hi=hi, hq=hq,
                                 hkv=hkv, with_write=False)
            ops = Ops(w, dev, stream)
            ms, _ = time_loop(ops.decode, 20, 3, stream)
            gbs = w.kv_bytes() / (ms * 1e-3) / 1e9
            print(f"| B={batch} ctx=U[{lo},{hi}] Hq/Hkv={hq}/{hkv} | {ms * 1e3:.1f} | "
                  f"{gbs:.0f} GB/s | {gbs * 1e9 / HBM_PEAK:.0%} HBM |", flush=True)
            del w, ops
            torch.cuda.empty_cache()
    else:
        for n_seqs, prefix, new, hq, hkv in ((8, 512, 1536, 16, 8), (8, 0, 2048, 16, 8),
                                             (4, 4096, 2048, 16, 8), (2, 16384, 2048, 16, 8),
                                             (8, 512, 1536, 32, 8), (8, 512, 1536, 32, 4),
                                             (16, 0, 512, 16, 8), (1, 0, 8192, 32, 8)):
            w = W.prefill_prefix(device=dev, n_seqs=n_seqs, prefix=prefix, new=new, hq=hq,
                                 hkv=hkv, share_pairs=())
            ops = Ops(w, dev, stream)
            ms, _ = time_loop(ops.prefill, 20, 3, stream)
            tf = W.prefill_flops(w) / (ms * 1e-3) / 1e12
            print(f"| {n_seqs} x ({prefix} cached + {new} new) Hq/Hkv={hq}/{hkv} | "
                  f"{ms * 1e3:.1f} | {tf:.0f} TFLOP/s | {tf * 1e12 / BF16_PEAK:.0%} bf16 MFMA |",
                  flush=True)
            del w, ops
            torch.cuda.empty_cache()
        # other head dims (padded MFMA tiles below 64 / 128 / 256) and query-group sizes;
        # the FLOPs count the real head dim
        for hq, hkv, d in ((16, 8, 64), (16, 8, 96), (16, 8, 80), (8, 4, 192), (16, 8, 256),
                           (64, 2, 128)):
            w = W.prefill_prefix(device=dev, n_seqs=8, prefix=512, new=1536, hq=hq, hkv=hkv,
                                 d=d, share_pairs=())
            ops = Ops(w, dev, stream)
            ms, _ = time_loop(ops.prefill, 20, 3, stream)
            tf = W.prefill_flops(w) / (ms * 1e-3) / 1e12
            print(f"| 8 x (512 cached + 1536 new) Hq/Hkv={hq}/{hkv} d={d} | "
                  f"{ms * 1e3:.1f} | {tf:.0f} TFLOP/s | {tf * 1e12 / BF16_PEAK:.0%} bf16 MFMA |",
                  flush=True)
            del w, ops
            torch.cuda.empty_cache()


def sweep_generic() -> None:
    """The cost of layouts beyond the native kernels at the configs' shapes: views that are
    only 2-byte aligned (q / output offset by one element) and cache blocks other than 16."""
    dev = torch.device("cuda:0")
    stream = torch.cuda.Stream()
    lib = _lib.load()
    print("| case | aligned call (us) | this call (us) | ratio |")
    print("|---|---|---|---|")

    def misaligned(t, elems=1):
        buf = torch.empty(t.numel() + 8, dtype=t.dtype, device=t.device)
        v = buf[elems:elems + t.numel()].view(t.shape)
        v.copy_(t)
        return v

    def rebin(w, bs):
        """The workload's context lengths over a table of bs-token blocks of the same cache."""
        rng = np.random.default_rng(bs)
        nslots = w.k_cache.shape[0]
        nb = (w.context_lens + bs - 1) // bs
        perm = rng.permutation(nslots // bs).astype(np.int32)
        bt = np.full((w.batch, int(nb.max())), -1, np.int32)
        cur = 0
        for b in range(w.batch):
            # blocks are reused once the cache runs out (reads only, the timing is the same)
            bt[b, :nb[b]] = perm[(cur + np.arange(nb[b])) % perm.size]
            cur += nb[b]
        return torch.from_numpy(bt).to(dev)

    # decode, configs[1]
    w = W.decode_batched(device=dev, with_write=False)
    meta = w.device_meta(dev)
    out = torch.empty_like(w.q)
    n = lib.ccinfer_decode_workspace_size(w.batch, w.mbpr, w.hq, w.hkv, w.d, 16)
    ws = torch.zeros(max(1, n), dtype=torch.uint8, device=dev)

    def dec(q, o, bt, mbpr, bs):  # decode takes 16-token blocks only
        def f():
            rc = lib.ccinfer_decode_attention(q.data_ptr(), w.k_cache.data_ptr(),
                                              w.v_cache.data_ptr(), bt.data_ptr(),
                                              meta["context_lens"].data_ptr(), o.data_ptr(),
                                              w.batch, mbpr, w.hq, w.hkv, w.d, bs,
                                              ws.data_ptr(), n, stream.cuda_stream)
            assert rc == 0, rc
        return time_loop(f, 20, 3, stream)[0] * 1e3
    base = dec(w.q, out, meta["block_table"], w.mbpr, 16)
    qm, om = misaligned(w.q), misaligned(out)
    t = dec(qm, om, meta["block_table"], w.mbpr, 16)
    print(f"| decode configs[1], q and output 2-byte aligned (MFMA on row copies) | {base:.1f} "
          f"| {t:.1f} | {t / base:.2f}x |", flush=True)
    kshift = misaligned(w.k_cache)
    def dec_k():
        rc = lib.ccinfer_decode_attention(w.q.data_ptr(), kshift.data_ptr(),
                                          w.v_cache.data_ptr(), meta["block_table"].data_ptr(),
                                          meta["context_lens"].data_ptr(), out.data_ptr(),
                                          w.batch, w.mbpr, w.hq, w.hkv, w.d, 16,
                                          ws.data_ptr(), n, stream.cuda_stream)
        assert rc == 0, rc
    t = time_loop(dec_k, 20, 3, stream)[0] * 1e3
    print(f"| decode configs[1], k_cache 2-byte aligned (MFMA, 2-byte pieces) | {base:.1f} | "
          f"{t:.1f} | {t / base:.2f}x |", flush=True)
    kshift = misaligned(w.k_cache, 2)
    t = time_loop(dec_k, 20, 3, stream)[0] * 1e3
    print(f"| decode configs[1], k_cache 4-byte aligned (MFMA, 4-byte pieces) | {base:.1f} | "
          f"{t:.1f} | {t / base:.2f}x |", flush=True)
    del kshift
    del w, ws
    torch.cuda.empty_cache()

    # prefill, configs[2]
    w = W.prefill_prefix(device=dev)
    meta = w.device_meta(dev)
    out = torch.empty_like(w.q)
    T = w.q.shape[0]
    n = max(lib.ccinfer_prefill_workspace_size(w.batch, T, w.mbpr, w.hq, w.hkv, w.d, bs)
            for bs in (16, 32, 64))
    ws = torch.zeros(max(1, n), dtype=torch.uint8, device=dev)

    def pre(q, o, bt, mbpr, bs, steps=10):
        def f():
            rc = lib.ccinfer_prefill_attention(q.data_ptr(), w.k_cache.data_ptr(),
                                               w.v_cache.data_ptr(), bt.data_ptr(),
                                               meta["query_start_loc"].data_ptr(),
                                               meta["context_lens"].data_ptr(), o.data_ptr(),
                                               w.batch, T, mbpr, w.hq, w.hkv, w.d, bs,
                                               ws.data_ptr(), n, stream.cuda_stream)
            assert rc == 0, rc
        return time_loop(f, steps, 2, stream)[0] * 1e3
    base = pre(w.q, out, meta["block_table"], w.mbpr, 16)
    qm, om = misaligned(w.q), misaligned(out)
    t = pre(qm, om, meta["block_table"], w.mbpr, 16, 3)
    print(f"| prefill configs[2], q and output 2-byte aligned (MFMA on row copies) | "
          f"{base:.1f} | {t:.1f} | {t / base:.2f}x |", flush=True)
    for bs in (32, 64):
        btb = rebin(w, bs)
        t = pre(w.q, out, btb, btb.shape[1], bs, 5)
        print(f"| prefill configs[2], {bs}-token blocks (MFMA, 16-token table) | {base:.1f} | "
              f"{t:.1f} | {t / base:.2f}x |", flush=True)
    bt8 = rebin(w, 8)
    t = pre(w.q, out, bt8, bt8.shape[1], 8, 5)
    print(f"| prefill configs[2], 8-token blocks (MFMA tile kernel, register staging) | "
          f"{base:.1f} | {t:.1f} | {t / base:.2f}x |", flush=True)
    kshift, vshift = misaligned(w.k_cache), misaligned(w.v_cache)

    def pre_k():
        rc = lib.ccinfer_prefill_attention(w.q.data_ptr(), kshift.data_ptr(), vshift.data_ptr(),
                                           meta["block_table"].data_ptr(),
                                           meta["query_start_loc"].data_ptr(),
                                           meta["context_lens"].data_ptr(), out.data_ptr(),
                                           w.batch, T, w.mbpr, w.hq, w.hkv, w.d, 16,
                                           ws.data_ptr(), n, stream.cuda_stream)
        assert rc == 0, rc
    t = time_loop(pre_k, 5, 2, stream)[0] * 1e3
    print(f"| prefill configs[2], k / v caches 2-byte aligned (MFMA tile kernel, shifted "
          f"16-byte loads) | {base:.1f} | {t:.1f} | {t / base:.2f}x |", flush=True)
    del kshift, vshift, w, ws
    torch.cuda.empty_cache()

    def pre_shape(d, prefix, new, n_seqs, hq=16, hkv=8, steps=5):
        w2 = W.prefill_prefix(device=dev, n_seqs=n_seqs, prefix=prefix, new=new, hq=hq,
                              hkv=hkv, d=d, share_pairs=())
        ops = Ops(w2, dev, stream)
        ms = time_loop(ops.prefill, steps, 2, stream)[0] * 1e3
        del w2, ops
        torch.cuda.empty_cache()
        return ms
    # a head dim that is not a multiple of 8 (element-wise staging) against the next one
    # that is (padded native kernel)
    a, b = pre_shape(96, 512, 1536, 8), pre_shape(100, 512, 1536, 8)
    print(f"| prefill configs[2] shape, d=100 (MFMA tile kernel, shifted loads) vs "
          f"d=96 | {a:.1f} | {b:.1f} | {b / a:.2f}x |", flush=True)
    # head dim 256 past 4096 table blocks (ids read from global memory) against 4096 blocks
    a = pre_shape(256, 65536 - 2048, 2048, 1, hq=8, hkv=4, steps=3)
    b = pre_shape(256, 65536 + 2048, 2048, 1, hq=8, hkv=4, steps=3)
    print(f"| prefill d=256, 1 x (63488 / 67584 cached + 2048 new): 4,096 blocks (native "
          f"tile kernel) vs 4,352 (any-layout, table in global memory) | {a:.1f} | {b:.1f} | "
          f"{b / a:.2f}x |", flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--configs", default="1,2,3,4,5,6,7,8,9")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=5.0)
    ap.add_argument("--sweep", choices=("decode", "prefill", "generic"),
                    help="print a table of the op across shapes and exit")
    ap.add_argument("--profile-op", choices=["decode", "write", "prefill", "mixed", "long",
                                             "decode_b600", "decode_b2048",
                                             "decode_shared", "decode_unshared",
                                             "prologue", "shared_prefix", "private_prefix",
                                             "shared_prefix_ragged", "private_prefix_ragged",
                                             "copy", "decode_d64", "decode_d80",
                                             "decode_d96", "decode_d128", "decode_d192",
                                             "decode_g32", "decode_g32_hkv1"], default=None)
    ap.add_argument("--profile-iters", type=int, default=5)
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build targets one GPU; --gpus {args.gpus} is not supported "
              "(each GPU would own whole sequences or whole kv_heads, with no exchange "
              "inside attention; only the one-GPU share is built).", file=sys.stderr)
        sys.exit(2)
    if args.sweep == "generic":
        sweep_generic()
        return
    if args.sweep:
        sweep(args.sweep)
        return
    if args.profile_op:
        profile(args.profile_op, args.profile_iters)
        return
    if 2 not in [int(c) for c in args.configs.split(",") if c]:
        args.configs = "2," + args.configs
    head, out, nt = run(args)
    w, r = head
    ms = r["ms_per_step"]
    value = r["kv_GBps"]
    dec_ms = r["decode_ms"]
    traffic = traffic_from_profiles("decode_split_b64")
    line = {
        "metric": "paged-decode KV GB/s (% HBM peak) + paged-prefill TFLOPS (% bf16 MFMA peak)",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) bf16 Q/K/V, random block tables)",
        "config": {"workload": "configs[1]: batched paged decode, batch 64, 16q/8kv heads, "
                               "d=128, ctx U[128,4096], block 16, + KV write of 64 new tokens "
                               "(in the decode launch: ccinfer_decode_attention_write_kv)",
                   "batch": w.batch, "num_q_heads": w.hq, "num_kv_heads": w.hkv,
                   "head_dim": w.d, "block_size": 16, "sum_ctx": int(w.context_lens.sum()),
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "kernel": "decode (split-KV kernel + LSE merge)",
                     "achieved": round(w.kv_bytes() / (dec_ms * 1e-3) / 1e9, 2),
                     "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                     "frac": round(w.kv_bytes() / (dec_ms * 1e-3) / HBM_PEAK, 4),
                     "traffic": traffic},
        "cpu_baseline": None if "cpu_GBps" not in r else {
            "value": round(r["cpu_GBps"], 3), "unit": "GB/s", "cores": nt, "kind": "port",
            "sample": f"full configs[1] batch (all 1024 (seq, q_head) rows), {r['cpu_reps']} "
                      f"repetition(s), oracle/attn_oracle.c over {nt} threads, {cpu_model()}",
            "single_thread_value": round(r.get("cpu_1thread_GBps", 0.0), 3),
            "single_thread_sample": "sequences 0-7, all 16 q-heads, 1 thread"},
        "configs": {k: {kk: (round(vv, 5) if isinstance(vv, float) else vv)
                        for kk, vv in v.items()} for k, v in out.items()},
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
