"""Benchmark of the kvskip_amd decode-attention hot path on one MI355X.

A "step" is one decode-attention layer-step of BASELINE config 2 (Llama-3.1-8B attention layer:
B 1, 32 query / 8 KV heads, D 128, T 32768, bf16): dense split-K decode over the whole KV cache.
`value` is its achieved HBM bandwidth (algorithmic bytes: K + V + q + out + lse) over the K timed
steps, launched from a HIP graph that cycles through 8 distinct KV copies (1.07 GB, far more than
L2 + the 256 MB Infinity Cache, so every step streams from HBM). The same line carries the masked
block-list + block-statistics path (config 2's 35% list), the two-pass V-skip (config 2's layer
and a layer with peaked attention), the single-pass V-skip (config 3, T 65536), config 1, the
measured read ceiling, the device planner loops (configs 4 and 5), per-kernel HIP-event durations
(roofline) and the reference-semantics PyTorch CPU path timed on this host (cpu_baseline).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--splits S]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_GBS = 8000.0
METRIC = "decode-attn HBM GB/s (% of MI355X peak) + us/layer-step at 32k, dense vs masked"
NCOPY = 8


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def attn_bytes(B, Hq, Hkv, D, rows_kv, stats_nb=0, list_entries=0):
    """Algorithmic bytes of one attention op: K+V rows read (bf16), q, bf16 out, fp32 lse,
    block-list entries read, stats written (2 fp32 per query head per block)."""
    return (2 * rows_kv * D * 2 + B * Hq * D * 2 + B * Hq * D * 2 + B * Hq * 4 + list_entries * 4
            + 2 * B * Hq * stats_nb * 4)


class Flush:
    """Reads a 512 MiB buffer (more than L2 + the 256 MB Infinity Cache) with the read-ceiling
    kernel before each timed call: evicts the previous call's data and keeps the stream busy while
    the host enqueues the timed call, so the events bracket device time only."""

    def __init__(self, dev):
        import torch

        from kvskip_amd import ext as E
        self.E = E
        self.x = torch.ones(256 << 20, dtype=torch.bfloat16, device=dev)
        self.o = torch.zeros(1, dtype=torch.int32, device=dev)

    def __call__(self):
        self.E.read_bw(self.x, self.o, 1024)


def time_events(fn, n, rotate, flush=None):
    """Per-call HIP-event durations (us) on the current stream, cycling `rotate` inputs."""
    import torch

    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
    for i in range(n):
        if flush is not None:
            flush()
        evs[i][0].record()
        fn(i % rotate)
        evs[i][1].record()
    torch.cuda.synchronize()
    return [a.elapsed_time(b) * 1e3 for a, b in evs]


def graph_of(fn, count):
    """HIP graph of fn(0), ..., fn(count - 1) captured on a side stream."""
    import torch

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(count):      # warm the allocator outside the capture
            fn(i)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(count):
            fn(i)
    torch.cuda.synchronize()
    return g


def timed_steps(fn, steps, warmup):
    """Run `warmup` then exactly `steps` steps from graphs of NCOPY steps (+ one of the remainder);
    returns elapsed seconds of the timed steps (synchronised on both sides)."""
    import torch

    full = graph_of(fn, NCOPY)
    rem = steps % NCOPY
    tail = graph_of(fn, rem) if rem else None
    for _ in range(max(1, warmup // NCOPY)):
        full.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps // NCOPY):
        full.replay()
    if tail is not None:
        tail.replay()
    torch.cuda.synchronize()
    return time.perf_counter() - t0


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--splits", type=int, default=None, help="override the split count of the dense op")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--events", type=int, default=64, help="event-timed calls per path")
    ap.add_argument("--no-planner", action="store_true", help="skip the config-4 planner loop")
    ap.add_argument("--planner-layers", type=int, default=32)
    ap.add_argument("--planner-steps", type=int, default=128)
    ap.add_argument("--cfg5-steps", type=int, default=64, help="decode steps of the config-5 ragged loop (its 64)")
    ap.add_argument("--roofline-only", action="store_true",
                    help="only the dominant kernel's timed region (the rocprofv3 --stats target), then exit")
    ap.add_argument("--pmc-target", action="store_true",
                    help="profiling target only: 20 dense config-2 decodes + copy kernels of known size, then exit")
    ap.add_argument("--pmc-paths", action="store_true",
                    help="profiling target only: config 2 masked + stats, the peaked two-pass V-skip op, short "
                         "config-4 and B 32 / 64k planner loops, + copy kernels of known size, then exit")
    ap.add_argument("--planner-only", action="store_true",
                    help="profiling target only: the config-4 planner loop (--planner-layers x --planner-steps), "
                         "its result as one JSON line, then exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1 "
                                   "(multi-GPU sharding is a design note, not implemented)"}))
        sys.exit(2)

    import torch

    from kvskip_amd import ext as E
    from kvskip_amd import kvskip as K
    from kvskip_amd import workloads as W

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    props = torch.cuda.get_device_properties(dev)
    log(f"device {props.name}, {props.multi_processor_count} CUs")
    if args.planner_only:
        res = bench_planner(dev, layers=args.planner_layers, steps=args.planner_steps)
        print(json.dumps({"planner_cfg4": res}, default=float))
        return

    # ---- config 2 inputs: one structured layer, NCOPY distinct copies of K/V in HBM
    L, keep = W.cfg2(device=dev)
    B, Hq, D = L.q.shape
    Hkv, T = L.k.shape[1], L.k.shape[2]
    nb = math.ceil(T / 64)
    ks = [L.k.clone() for _ in range(NCOPY)]
    vs = [L.v.clone() for _ in range(NCOPY)]
    q = L.q.contiguous()
    S_dense = args.splits or K.num_splits_for(B * Hkv, nb)
    bi, bc = W.block_list(keep)
    bi, bc = bi.to(dev), bc.to(dev)
    kept_rows = int(sum(min(T, (blk + 1) * 64) - blk * 64 for blk in torch.nonzero(keep.cpu())[:, 2].tolist()))
    S_mask = K.num_splits_for(B * Hkv, int(bc.max()))
    log(f"cfg2: T {T}, splits dense {S_dense} masked {S_mask}, kept blocks {keep.float().mean():.3f}")

    def dense(i):
        return E.decode(q, ks[i], vs[i], L.scale, None, None, False, True, S_dense, 2, False, False)

    if args.pmc_target:
        pmc_target(dense, dev)
        return
    if args.pmc_paths:
        pmc_paths(q, ks, vs, L.scale, bi, bc, dev)
        return

    def masked(i):
        return E.decode(q, ks[i], vs[i], L.scale, bi, bc, True, True, S_mask, 2, False, False)

    bytes_dense = attn_bytes(B, Hq, Hkv, D, B * Hkv * T)
    bytes_mask = attn_bytes(B, Hq, Hkv, D, kept_rows, stats_nb=nb, list_entries=int(bc.sum()))

    res = {"dense": {}}
    flush = Flush(dev)
    for name, fn, nbytes in () if args.roofline_only else (("dense", dense, bytes_dense),
                                                            ("masked_stats", masked, bytes_mask)):
        for i in range(NCOPY):
            fn(i)
        torch.cuda.synchronize()
        us = time_events(fn, args.events, NCOPY, flush)
        med = statistics.median(us)
        res[name] = {"us_per_op_median": med, "us_per_op_mean": statistics.mean(us), "bytes": nbytes,
                     "GBs_event_median": nbytes / med / 1e3}
        log(f"{name}: event median {med:.1f} us -> {nbytes / med / 1e3:.0f} GB/s")

    # ---- the dominant kernel on its own: the split pass of the dense op, `steps` launches back to
    # back from a HIP graph cycling the 8 KV copies, HIP events around the timed replays (average
    # per launch); per-launch event medians after a flush as well (they carry ~5 us of event and
    # dispatch overhead per call)
    ops = [E.DecodeOp(q, ks[i], vs[i], L.scale, S_dense) for i in range(NCOPY)]
    t_split = events_region(lambda i: ops[i].splits(), args.steps, args.warmup)
    t_merge = events_region(lambda i: ops[i].merge(), args.steps, args.warmup)
    ev_split, ev_merge = (math.nan, math.nan) if args.roofline_only else split_merge_events(ops, args.events, flush)
    bytes_split = 2 * B * Hkv * T * D * 2 + B * Hq * D * 2          # K + V + q, the split pass's reads
    res["dense"].update(split_pass_us=t_split, merge_us=t_merge, split_pass_us_event_median=ev_split,
                        merge_us_event_median=ev_merge, split_pass_bytes=bytes_split)
    log(f"dense split pass: {t_split:.2f} us per launch ({bytes_split / t_split / 1e3:.0f} GB/s), merge "
        f"{t_merge:.2f} us; per-call event medians {ev_split:.2f} / {ev_merge:.2f} us")
    del ops

    def read_same_bytes():
        # the read-ceiling kernel over the same bytes, timed the same way (8 buffers of the split
        # pass's read size, launches back to back): a pure stream of these bytes at this size,
        # launch ramp and tail included (best of 512 and 768 workgroups). Run after the headline
        # steps: a burst of full-bandwidth reads right before them slows the next ones.
        o_r = torch.zeros(1, dtype=torch.int32, device=dev)
        xr = [torch.ones(bytes_split // 2, dtype=torch.bfloat16, device=dev) for _ in range(NCOPY)]
        t = min(events_region(lambda i: E.read_bw(xr[i], o_r, nblk), args.steps, args.warmup) for nblk in (512, 768))
        del xr
        res["dense"].update(read_same_bytes_us=t, split_pass_vs_read=t / t_split)
        log(f"read kernel over the same {bytes_split / 1e6:.1f} MB: {t:.2f} us per launch "
            f"({bytes_split / t / 1e3:.0f} GB/s); split pass at {100 * t / t_split:.1f}% of it")
        return t

    if args.roofline_only:
        t_read = read_same_bytes()
        print(json.dumps({"roofline_only": True, "split_pass_us": t_split, "merge_us": t_merge,
                          "GBs": bytes_split / t_split / 1e3, "read_same_bytes_us": t_read}), flush=True)
        return

    # ---- timed steps (dense, the headline) and the masked path, from graphs
    el = timed_steps(dense, args.steps, args.warmup)
    us_step = el / args.steps * 1e6
    gbs = bytes_dense * args.steps / el / 1e9
    res["dense"].update(us_per_step=us_step, GBs=gbs, pct_peak=100 * gbs / PEAK_GBS, num_splits=S_dense)
    elm = timed_steps(masked, args.steps, args.warmup)
    us_m = elm / args.steps * 1e6
    res["masked_stats"].update(us_per_step=us_m, GBs=bytes_mask * args.steps / elm / 1e9,
                               pct_peak=100 * bytes_mask * args.steps / elm / 1e9 / PEAK_GBS,
                               kept_block_frac=float(keep.float().mean()), time_vs_dense=us_m / us_step,
                               num_splits=S_mask)
    log(f"dense: {us_step:.2f} us/step, {gbs:.0f} GB/s ({100 * gbs / PEAK_GBS:.1f}% of peak); "
        f"masked: {us_m:.2f} us/step (x{us_m / us_step:.3f} of dense)")
    # the dense op over a paged cache: each copy's K / V as 64-token pages of a pool in a random
    # order, with a block table; the same bytes as the dense op, timed the same way
    table, kps, vps = W.paged_pools(ks, vs, seed=21)

    def dense_paged(i):
        return E.decode(q, kps[i], vps[i], L.scale, None, None, False, True, S_dense, 2, False, False,
                        block_table=table, T=T)

    elp = timed_steps(dense_paged, args.steps, args.warmup)
    us_p = elp / args.steps * 1e6
    res["dense_paged"] = {"us_per_step": us_p, "GBs": bytes_dense * args.steps / elp / 1e9,
                          "time_vs_dense": us_p / us_step, "pages": int(kps[0].shape[0]), "num_splits": S_dense}
    log(f"dense over pages: {us_p:.2f} us/step (x{us_p / us_step:.3f} of contiguous)")
    del kps, vps, table
    t_read = read_same_bytes()

    # ---- two-pass V-skip (kernels/kvskip.py:157-179) on config 2's layer (flat N(0, 1) keys: top-p
    # 0.99 keeps every block, so the path can only show its cost) and on a layer of the config-4
    # generator with an aimed query (attention on a few planted blocks + the sink)
    res["vskip2_cfg2"] = bench_two_pass(E, K, q, ks, vs, L.scale, S_dense, us_step, args, flush, "vskip2 cfg2")
    run_p = W.planner_run(layers=1, T0=T, steps=1, seed=44, device=dev)
    q_p = run_p.q0[0].to(torch.bfloat16).contiguous()
    ks_p = [run_p.k[0][:, :, :T].clone() for _ in range(NCOPY)]
    vs_p = [run_p.v[0][:, :, :T].clone() for _ in range(NCOPY)]
    del run_p
    res["vskip2_peaked"] = bench_two_pass(E, K, q_p, ks_p, vs_p, L.scale, S_dense, us_step, args, flush,
                                          "vskip2 peaked")
    # single-pass V-skip on the same peaked layer (config 3's rule: tau 1e-4, local 2, the exact lse
    # perturbed +-5% as lse_prev): the V blocks it skips, and its time against the dense pass
    lp_p = W.perturbed_lse(K.decode(q_p, ks_p[0], vs_p[0], L.scale)["lse"], seed=45).contiguous()
    cnt_p = E.vskip1(q_p, ks_p[0], vs_p[0], L.scale, 1e-4, 2, S_dense, False, True, lp_p)[3]
    vfrac = float(cnt_p.sum()) / (Hkv * (T // 64))
    t_v1 = events_region(lambda i: E.vskip1(q_p, ks_p[i], vs_p[i], L.scale, 1e-4, 2, S_dense, False, False, lp_p),
                         args.steps // 2, args.warmup)
    t_d1 = events_region(lambda i: E.decode(q_p, ks_p[i], vs_p[i], L.scale, None, None, False, True, S_dense, 2, False,
                                            False), args.steps // 2, args.warmup)
    res["vskip1_peaked"] = {"v_block_frac": vfrac, "us_per_op": t_v1, "dense_us_per_op": t_d1,
                            "time_vs_dense": t_v1 / t_d1, "bytes_vs_dense": 0.5 + 0.5 * vfrac, "num_splits": S_dense}
    log(f"vskip1 peaked: V read {vfrac:.3f}; {t_v1:.2f} us vs dense {t_d1:.2f} us (x{t_v1 / t_d1:.3f}; bytes "
        f"x{0.5 + 0.5 * vfrac:.3f})")
    del ks_p, vs_p

    # ---- config 3: single-pass V-skip at T 65536 with a +-5% lse_prev
    del ks, vs
    torch.cuda.empty_cache()
    L3 = W.cfg3(device=dev)
    r = K.decode(L3.q, L3.k, L3.v, L3.scale)
    lp = W.perturbed_lse(r["lse"], seed=33).contiguous()
    n3 = 4
    k3 = [L3.k.clone() for _ in range(n3)]
    v3 = [L3.v.clone() for _ in range(n3)]
    T3 = L3.k.shape[2]
    nb3 = math.ceil(T3 / 64)
    S3 = K.num_splits_for(Hkv, nb3)
    cnt = E.vskip1(L3.q, k3[0], v3[0], L3.scale, 1e-4, 2, S3, False, True, lp)[3]
    v_blocks = int(cnt.sum())
    bytes_v1 = 2 * (Hkv * T3 * D) + 2 * v_blocks * 64 * D + 2 * (2 * Hq * D) + Hq * 4

    def vsk(i):
        return E.vskip1(L3.q, k3[i % n3], v3[i % n3], L3.scale, 1e-4, 2, S3, False, False, lp)

    def dense3(i):
        return E.decode(L3.q, k3[i % n3], v3[i % n3], L3.scale, None, None, False, True, S3, 2, False, False)

    for fn in (vsk, dense3):
        for i in range(n3):
            fn(i)
    torch.cuda.synchronize()
    us_v = statistics.median(time_events(vsk, args.events, n3, flush))
    us_d3 = statistics.median(time_events(dense3, args.events, n3, flush))
    # config 2's shape at T 65536 (config 3's K / V, cycled over its copies): the whole dense op
    # graph-timed as the headline is
    us_d3g = timed_steps(dense3, args.steps // 2, args.warmup) / (args.steps // 2) * 1e6
    bytes_d3 = attn_bytes(1, Hq, Hkv, D, Hkv * T3)
    res["dense_64k"] = {"us_per_step": us_d3g, "GBs": bytes_d3 / us_d3g / 1e3,
                        "pct_peak": 100 * bytes_d3 / us_d3g / 1e3 / PEAK_GBS, "T": T3, "num_splits": S3,
                        "kv_copies": n3}
    log(f"dense 64k: {us_d3g:.2f} us/step, {bytes_d3 / us_d3g / 1e3:.0f} GB/s "
        f"({100 * bytes_d3 / us_d3g / 1e3 / PEAK_GBS:.1f}% of peak)")
    res["vskip1_cfg3"] = {"us_per_op_median": us_v, "bytes": bytes_v1, "GBs_event_median": bytes_v1 / us_v / 1e3,
                          "v_block_frac": v_blocks / (Hkv * nb3), "dense_us_per_op_median": us_d3,
                          "time_vs_dense": us_v / us_d3, "num_splits": S3}
    log(f"vskip1 cfg3: {us_v:.1f} us (dense {us_d3:.1f} us), V read {v_blocks / (Hkv * nb3):.3f}")
    cfg3_cpu = None if args.no_cpu else (L3.q.cpu(), L3.k.cpu(), L3.v.cpu(), L3.scale, lp.cpu())
    del k3, v3, L3
    torch.cuda.empty_cache()

    # ---- config 1 (latency-bound) and the read ceiling
    L1 = W.cfg1(device=dev)
    S1 = K.num_splits_for(8, 64)
    us1 = statistics.median(time_events(lambda i: E.decode(L1.q, L1.k, L1.v, L1.scale, None, None, False, True, S1,
                                                           2, False, False), args.events, 1, flush))
    b1 = attn_bytes(1, 32, 8, 64, 8 * 4096)
    # graph-replayed back to back as the headline op, over 64 copies of the K / V (537 MB, more than
    # L2 + the Infinity Cache): the op's device time without a per-call event and dispatch gap
    n1 = 64
    ops1 = [E.DecodeOp(L1.q, L1.k.clone(), L1.v.clone(), L1.scale, S1) for _ in range(n1)]
    g1 = graph_of(lambda i: ops1[i].run(), n1)
    for _ in range(4):
        g1.replay()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(16):
        g1.replay()
    e1.record()
    torch.cuda.synchronize()
    us1g = e0.elapsed_time(e1) * 1e3 / (16 * n1)
    del g1, ops1
    res["cfg1_dense"] = {"us_per_op_graph": us1g, "GBs_graph": b1 / us1g / 1e3, "splits": S1,
                         "us_per_op_median": us1, "bytes": b1, "GBs_event_median": b1 / us1 / 1e3}
    # the read ceiling: 2 GiB, best over workgroup counts (per-call event medians)
    x = torch.ones(1 << 30, dtype=torch.bfloat16, device=dev)
    o = torch.zeros(1, dtype=torch.int32, device=dev)
    best = 0.0
    for blocks in (256, 512, 768, 1024, 2048):
        E.read_bw(x, o, blocks)
        us = statistics.median(time_events(lambda i: E.read_bw(x, o, blocks), 10, 1))
        best = max(best, x.numel() * 2 / us / 1e3)
    res["read_ceiling_GBs"] = best
    del x
    log(f"cfg1: {us1g:.2f} us per op graph-replayed ({us1:.1f} per call, event median); read ceiling {best:.0f} GB/s")

    # ---- config 4: 32-layer decode loop with the device-side planner (stage-4 policy, layer 0 dense)
    if not args.no_planner:
        res["planner_cfg4"] = bench_planner(dev, layers=args.planner_layers, T0=32768, steps=args.planner_steps)
        res["planner_cfg4"]["oracle_agreement"] = planner_agreement(dev)
        torch.cuda.empty_cache()
        # the same loop with queries that revert to their planted direction between jumps:
        # attention stays on the planted blocks, so the policy skips most of the cache
        res["planner_cfg4_focused"] = bench_planner(dev, layers=args.planner_layers, T0=32768,
                                                    steps=min(args.planner_steps, 64), revert=True,
                                                    tag="cfg4-focused")
        # the reference's "refresh" mode (trigger after the masked pass, then a dense + statistics
        # pass for the refreshing heads) on config 4's loop
        res["planner_cfg4_refresh_mode"] = bench_planner(dev, layers=args.planner_layers, T0=32768,
                                                         steps=min(args.planner_steps, 64), post=True,
                                                         tag="cfg4-refresh-mode")
        torch.cuda.empty_cache()
        # the reference's operating point for the planner (README.md:100-105: batch 8 at 32k): config 4's
        # loop with 8 sequences of T 32768
        res["planner_b8"] = bench_planner(dev, layers=args.planner_layers, T0=32768, B=8,
                                          steps=min(args.planner_steps, 64), tag="b8")
        torch.cuda.empty_cache()
        # the same batch with queries that stay on their planted blocks and re-aim rarely (0.3% per
        # query head and step): the regime where the reference reports its planner's gain
        # (README.md:100-105, attention time -33% at batch 8 / 32k)
        res["planner_b8_stable"] = bench_planner(dev, layers=args.planner_layers, T0=32768, B=8,
                                                 steps=min(args.planner_steps, 64), revert=True, p_jump=0.003,
                                                 tag="b8-stable")
        torch.cuda.empty_cache()
        # the reference's largest point (batch 32 at 64k, README.md:100-105), 4 layers (8.6 GB of K / V
        # each) x 32 steps, stable queries
        res["planner_b32_64k_stable"] = bench_planner(dev, layers=4, T0=65536, B=32, steps=min(args.planner_steps, 32),
                                                      revert=True, p_jump=0.003, chunk=8, tag="b32-64k-stable")
        torch.cuda.empty_cache()
        # config 5: batch 16 of Qwen2.5-7B layers (28 / 4 heads, G 7), contexts log-uniform in
        # [4096, 65536], 28 layers, ragged split-K over the batch
        g5 = torch.Generator().manual_seed(5)
        lens5 = [int(round(math.exp(x))) for x in
                 (torch.rand(16, generator=g5, dtype=torch.float64) * math.log(16) + math.log(4096)).tolist()]
        res["planner_cfg5"] = bench_planner(dev, layers=28, steps=min(args.planner_steps, args.cfg5_steps), B=16,
                                            Hq=28, Hkv=4, ragged=lens5, dense_layer0=False, seed=5, chunk=8,
                                            tag="cfg5", one_launch_plan=True)
        torch.cuda.empty_cache()
        res["planner_cfg5"]["oracle_agreement"] = planner_agreement(dev, cfg=5)
        torch.cuda.empty_cache()

    achieved = bytes_split / t_split / 1e3
    roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / PEAK_GBS, 4), "traffic": read_traffic(),
            "kernel": f"decode_kernel<128,4,dense,mfma> (split pass, {S_dense} splits) at config 2: K+V+q bytes / "
                      f"average launch duration, {args.steps} launches back to back from HIP graphs over 8 KV "
                      "copies (1.07 GB), HIP events around the timed region",
            "algorithmic_bytes": bytes_split, "us_per_launch": round(t_split, 3),
            "read_ceiling_GBs": round(res["read_ceiling_GBs"], 1),
            "read_same_bytes_GBs": round(bytes_split / t_read / 1e3, 1),
            "frac_of_read_same_bytes": round(t_read / t_split, 4)}

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline((L.q.cpu(), L.k.cpu(), L.v.cpu(), L.scale, keep.cpu()), cfg3_cpu, bytes_dense, bytes_mask,
                           res["vskip1_cfg3"]["bytes"])

    line = {
        "metric": METRIC, "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": us_step / 1e3, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: seeded structured q/K/V (config 2 generator), 8 HBM copies cycled",
        "config": {"workload": "config 2: Llama-3.1-8B attention layer, dense split-K decode, B 1, 32 Q / 8 KV heads, "
                               "D 128, T 32768, bf16 in, fp32 accumulate", "B": 1, "Hq": 32, "Hkv": 8, "D": 128,
                   "T": 32768, "num_splits": S_dense},
        "pct_of_peak": round(100 * gbs / PEAK_GBS, 2), "us_per_layer_step": round(us_step, 2),
        "qk_engine": os.environ.get("KVSKIP_AMD_QK", "mfma"),
        "paths": res, "roofline": roof, "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def bench_two_pass(E, K, q, ks, vs, scale, S1, us_dense, args, flush, tag):
    """Two-pass V-skip on one layer (NCOPY KV copies), top-p 0.99 GQA union: pass 1 (stats-only + fp16
    P; its split pass alone, as the op runs it), the device selection (kvskip_select: kept set, lists,
    per-block scales), pass 2 (pv over the kept blocks, sized by the longest list) and pass 2 with the
    selection in it (kvskip_pv_select, sized by nb) each timed as a graph-replayed region, and the
    whole op as the front-end runs it without a host read-back (kvskip.vskip_two_pass(sync=False):
    pass 1, then pass 2 with the selection), also replayed."""
    import torch

    B, Hq, D = q.shape
    Hkv, T = ks[0].shape[1], ks[0].shape[2]
    G, nb = Hq // Hkv, math.ceil(T / 64)
    dev = q.device
    r1 = E.decode(q, ks[0], vs[0], scale, None, None, True, False, S1, 2, False, True, merge=False)
    keep = torch.empty(B, Hkv, nb, dtype=torch.uint8, device=dev)
    idx = torch.empty(B, Hkv, nb, dtype=torch.int32, device=dev)
    cnt = torch.empty(B, Hkv, dtype=torch.int32, device=dev)
    scales = torch.empty(B, Hkv, nb, G, dtype=torch.float32, device=dev)

    def select(i):
        E.select(r1[2], r1[3], Hkv, "topp", 0.99, 2, keep=keep, block_idx=idx, block_cnt=cnt, blk_scale=scales)

    select(0)
    kept = int(cnt.sum())
    S2 = K.num_splits_for(B * Hkv, int(cnt.max()))
    P1 = r1[5]
    t_p1 = events_region(lambda i: E.decode(q, ks[i], vs[i], scale, None, None, True, False, S1, 2, False, True,
                                            merge=False), args.steps // 2, args.warmup)
    t_sel = events_region(select, args.steps // 2, args.warmup)
    t_p2 = events_region(lambda i: E.pv(P1, vs[i], scales, idx, cnt, S2, False), args.steps // 2, args.warmup)
    S2n = K.num_splits_for(B * Hkv, nb)             # the op's pass 2 split count (sized by nb)
    t_p2s = events_region(lambda i: E.pv_select(P1, vs[i], r1[2], r1[3], "topp", 0.99, 2, S2n, False),
                          args.steps // 2, args.warmup)
    t_op = events_region(lambda i: K.vskip_two_pass(q, ks[i], vs[i], scale, sync=False), args.steps // 2,
                         args.warmup)
    bytes_p1 = B * Hkv * T * D * 2 + B * Hq * D * 2 + B * Hq * nb * 64 * 2 + 2 * B * Hq * nb * 4
    bytes_p2 = kept * 64 * D * 2 + kept * G * 64 * 2 + kept * G * 4 + kept * 4
    out = {"kept_block_frac": kept / (B * Hkv * nb), "pass1_us": t_p1, "select_us": t_sel, "pass2_us": t_p2,
           "pass1_bytes": bytes_p1, "pass2_bytes": bytes_p2, "pass1_GBs": bytes_p1 / t_p1 / 1e3,
           "pass2_GBs": bytes_p2 / t_p2 / 1e3, "kernels_vs_dense": (t_p1 + t_sel + t_p2) / us_dense,
           "num_splits_pass2": S2, "pass2_with_select_us": t_p2s, "num_splits_pass2_with_select": S2n,
           "op_us": t_op, "op_vs_dense": t_op / us_dense, "op_vs_passes": t_op / (t_p1 + t_p2),
           "op_vs_pass1_and_pass2_with_select": t_op / (t_p1 + t_p2s)}
    log(f"{tag}: kept {kept / (B * Hkv * nb):.3f}; pass 1 {t_p1:.2f} us ({bytes_p1 / t_p1 / 1e3:.0f} GB/s), select "
        f"{t_sel:.2f} us, pass 2 {t_p2:.2f} us ({bytes_p2 / t_p2 / 1e3:.0f} GB/s); pass 2 with the selection in it "
        f"{t_p2s:.2f} us; whole op {t_op:.2f} us (x{t_op / us_dense:.3f} of dense, x{t_op / (t_p1 + t_p2):.3f} of "
        f"pass 1 + pass 2, x{t_op / (t_p1 + t_p2s):.3f} of pass 1 + pass 2 with the selection)")
    return out


def events_region(fn, steps, warmup):
    """Average us per launch of fn(i) (i cycling NCOPY inputs): `steps` launches replayed from HIP
    graphs of NCOPY launches each, HIP events on the current stream around the timed replays."""
    import torch

    g = graph_of(fn, NCOPY)
    for _ in range(max(1, warmup // NCOPY)):
        g.replay()
    reps = max(1, steps // NCOPY)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (reps * NCOPY)


def split_merge_events(ops, n, flush):
    """Median HIP-event durations (us) of the split pass and of the split merge of DecodeOps,
    cycling the ops; a flush precedes every pair."""
    import torch

    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(n)]
    for op in ops:
        op.run()
    torch.cuda.synchronize()
    for i in range(n):
        flush()
        ev[i][0].record()
        ops[i % len(ops)].splits()
        ev[i][1].record()
        ops[i % len(ops)].merge()
        ev[i][2].record()
    torch.cuda.synchronize()
    split = statistics.median(a.elapsed_time(b) * 1e3 for a, b, _ in ev)
    merge = statistics.median(b.elapsed_time(c) * 1e3 for _, b, c in ev)
    return split, merge


PMC_FILE = ROOT / "profiles" / "decode_dense_cfg2_pmc.txt"


def read_traffic():
    """HBM bytes per launch of the dense split pass from the committed rocprofv3 --pmc summary
    (FETCH_SIZE + WRITE_SIZE per dispatch, scaled by the copy-kernel factors), or None."""
    try:
        for line in PMC_FILE.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch:"):
                return int(float(line.split(":", 1)[1]))
    except OSError:
        pass
    return None


def pmc_target(dense, dev):
    """Profiling target for rocprofv3 --pmc: 20 dense config-2 decodes, then a 256 MiB torch copy
    (reads and writes 256 MiB) and a 256 MiB read_bw (reads 256 MiB) 5 times each, as the known
    sizes that scale FETCH_SIZE / WRITE_SIZE to bytes."""
    import torch

    from kvskip_amd import ext as E
    for i in range(20):
        dense(i % NCOPY)
    a = torch.ones(128 << 20, dtype=torch.bfloat16, device=dev)
    b = torch.empty_like(a)
    o = torch.zeros(1, dtype=torch.int32, device=dev)
    for _ in range(5):
        b.copy_(a)
    for _ in range(5):
        E.read_bw(a, o, 1024)
    torch.cuda.synchronize()
    print(json.dumps({"pmc_target": "done", "copy_bytes": a.numel() * 2, "read_bytes": a.numel() * 2}), flush=True)


def pmc_paths(q, ks, vs, scale, bi, bc, dev):
    """Profiling target for rocprofv3 --pmc beyond the dense pass: 20 config-2 masked + statistics
    ops (the bench's list), 20 two-pass V-skip ops on the peaked layer (pass 1, select, pass 2),
    a config-4 planner loop of 4 layers x 12 steps (updates carried), a B 32 / 64k stable-query loop
    of 2 layers x 6 steps (each planned pass's listed blocks printed, to price it), then the
    known-size copy and read of pmc_target."""
    import torch

    from kvskip_amd import ext as E
    from kvskip_amd import kvskip as K
    from kvskip_amd import workloads as W
    from kvskip_amd.planner import FusedPlanner, Policy, UpdateCarrier

    Hkv, T = ks[0].shape[1], ks[0].shape[2]
    S_mask = K.num_splits_for(Hkv, int(bc.max()))
    for i in range(20):
        E.decode(q, ks[i % NCOPY], vs[i % NCOPY], scale, bi, bc, True, True, S_mask, 2, False, False)
    run = W.planner_run(layers=1, T0=T, steps=1, seed=44, device=dev)
    q_p = run.q0[0].to(torch.bfloat16).contiguous()
    for i in range(20):
        K.vskip_two_pass(q_p, run.k[0][:, :, :T], run.v[0][:, :, :T], run.scale, sync=False)
    del run
    layers, steps = 4, 12
    run = W.planner_run(layers=layers, T0=T, steps=steps, seed=4, device=dev)
    qps = [W.QueryProcess(run, l, noise=0.25) for l in range(layers)]
    ids = run.ids.to(dev)
    pol = Policy(calib=0.05, calib_kind="peak", calib_warm=(32, 8), calib_auto_ix=0.1)
    carrier = UpdateCarrier()
    pls = [FusedPlanner(pol, count=False, carrier=carrier) for _ in range(layers)]
    for t in range(steps):
        for l in range(layers):
            k, v = run.k[l][:, :, :T + t + 1], run.v[l][:, :, :T + t + 1]
            ql = qps[l].next().to(dev)
            if t == 0:
                pls[l].first(ql, k, v, run.scale)
            else:
                pls[l].step(ql, k, v, run.scale, ids=ids)
    carrier.flush()
    torch.cuda.synchronize()
    del run, pls
    # B 32 at 64k with stable queries (the planner_b32_64k_stable leg's shape), 2 planned layers x 6
    # steps, updates carried: plan (scores, decision), the masked pass over all KV heads' lists cut
    # together with the previous layer's update in it (1025 blocks: 24 slots per lane), the merge
    layers, steps, B32, T32 = 2, 6, 32, 65536
    run = W.planner_run(layers=layers, B=B32, T0=T32, steps=steps, seed=4, device=dev)
    qps = [W.QueryProcess(run, l, noise=0.25, revert=True, p_jump=0.003) for l in range(layers)]
    ids = run.ids.to(dev)
    NBC = math.ceil((T32 + 1) / 64) + 64
    idx = torch.zeros(B32, NBC, dtype=torch.uint8, device=dev)
    carrier = UpdateCarrier()
    pls = [FusedPlanner(pol, count=False, carrier=carrier) for _ in range(layers)]
    b32_lists = []  # (step, layer, blocks listed by its planned pass), in launch order
    for t in range(steps):
        E.token_index(ids, T32 + t + 1, NBC, out=idx)   # as the bench's loop: the index found beforehand
        for l in range(layers):
            k, v = run.k[l][:, :, :T32 + t + 1], run.v[l][:, :, :T32 + t + 1]
            ql = qps[l].next().to(dev)
            if t == 0:
                pls[l].first(ql, k, v, run.scale)
            else:
                pls[l].step(ql, k, v, run.scale, idx=idx)
                b32_lists.append((t, l, int(pls[l].state["block_cnt"].sum())))
    carrier.flush()
    torch.cuda.synchronize()
    del run, pls
    a = torch.ones(128 << 20, dtype=torch.bfloat16, device=dev)
    b = torch.empty_like(a)
    o = torch.zeros(1, dtype=torch.int32, device=dev)
    for _ in range(5):
        b.copy_(a)
    for _ in range(5):
        E.read_bw(a, o, 1024)
    torch.cuda.synchronize()
    print(json.dumps({"pmc_paths": "done", "copy_bytes": a.numel() * 2, "read_bytes": a.numel() * 2,
                      "b32_pass_blocks": b32_lists, "b32_block_bytes": 2 * 64 * 128 * 2}), flush=True)


def bench_planner(dev, layers=32, T0=32768, steps=128, chunk=16, noise=0.25, revert=False, tag="cfg4", B=1, Hq=32,
                  Hkv=8, ragged=None, dense_layer0=True, seed=4, p_jump=0.03, post=False, one_launch_plan=False):
    """The device-side planner loop over `layers` attention layers for `steps` decode steps (one
    token appended per step and sequence), query drift + jumps, stage-4 policy (delta 0.05, max
    age 32, calibration 0.05 peak, warm-up (32, 8), token-index latch at 0.1;
    reproduce/04-tails.sh:16,63-69). Config 4: B 1, 32 / 8 heads, T0 32768, layer 0 dense.
    Config 5: `ragged` per-sequence prefix lengths (views of a common capacity, seq_lens). One
    eager pass with counters gives the read fraction and refresh rate; the timed passes replay HIP
    graphs of `chunk` steps x all layers (decisions still made on the device) for the planner loop
    and for dense decode of every layer. post: the reference's "refresh" mode instead (PostPlanner,
    the trigger after the masked pass; its default policy: delta 0.05, max age 32, no calibration).
    one_launch_plan: also time the loop with plan as one launch (FusedPlanner.plan_one_launch), where
    plan decides in its own launch(es): three launches per layer-step."""
    import torch

    from kvskip_amd import ext as E
    from kvskip_amd import kvskip as K
    from kvskip_amd import workloads as W
    from kvskip_amd.planner import FusedPlanner, Policy, PostPlanner, UpdateCarrier

    t_gen = time.perf_counter()
    run = W.planner_run(layers=layers, B=B, Hq=Hq, Hkv=Hkv, T0=T0, steps=steps, seed=seed, ragged=ragged, device=dev)
    _, _, Tcap, D = run.k[0].shape
    qps = [W.QueryProcess(run, l, p_jump=p_jump, noise=noise, revert=revert) for l in range(layers)]
    qs = torch.stack([torch.stack([qps[l].next() for l in range(layers)]) for _ in range(steps)]).to(dev)
    ids = run.ids.to(dev)
    if ragged is None:
        NBC = math.ceil((T0 + 1) / 64) + 64
        sl_all = [None] * steps
    else:
        NBC = math.ceil(Tcap / 64) + 64
        base = torch.tensor(ragged, dtype=torch.int32, device=dev)
        sl_all = [(base + t + 1).contiguous() for t in range(steps)]
    idx_all = torch.zeros(steps, B, NBC, dtype=torch.uint8, device=dev)
    for t in range(steps):
        E.token_index(ids, T0 + t + 1 if ragged is None else Tcap, NBC, out=idx_all[t], seq_lens=sl_all[t])
    pol = Policy() if post else Policy(calib=0.05, calib_kind="peak", calib_warm=(32, 8), calib_auto_ix=0.1)
    first_planned = 1 if dense_layer0 else 0
    ctx = f"T {T0}" if ragged is None else f"ragged T in [{min(ragged)}, {max(ragged)}], sum {sum(ragged)}"
    log(f"{tag}: {layers} layers x {steps} steps, B {B}, {Hq} / {Hkv} heads, {ctx}, generated in "
        f"{time.perf_counter() - t_gen:.1f} s")

    def kv(l, t):
        if ragged is not None:
            return run.k[l], run.v[l]
        T = T0 + t + 1
        return run.k[l][:, :, :T], run.v[l][:, :, :T]

    def dense_layer(l, t):
        k, v = kv(l, t)
        return K.decode(qs[t, l], k, v, run.scale, seq_lens=sl_all[t])["out"]

    def planner_pass(planners, t):
        for l in range(layers):
            if l < first_planned:
                dense_layer(l, t)
                continue
            k, v = kv(l, t)
            if t == 0:
                planners[l].first(qs[t, l], k, v, run.scale, seq_lens=sl_all[t])
            elif post:
                planners[l].step(qs[t, l], k, v, run.scale)
            else:
                planners[l].step(qs[t, l], k, v, run.scale, idx=idx_all[t], seq_lens=sl_all[t])

    def make(count, carrier, **kw):
        return [None] * first_planned + [PostPlanner(pol, count=count, carrier=carrier) if post else
                                         FusedPlanner(pol, count=count, carrier=carrier, **kw)
                                         for _ in range(first_planned, layers)]

    # eager pass with counters
    carrier = UpdateCarrier()
    planners = make(True, carrier)
    for t in range(steps):
        planner_pass(planners, t)
    carrier.flush()
    torch.cuda.synchronize()
    pl = planners[first_planned:]
    read = sum(float(p.counters["blocks_read"]) for p in pl)
    total = sum(float(p.counters["blocks_total"]) for p in pl)
    refresh = sum(float(p.counters.get("dense_heads", 0)) for p in pl) - len(pl) * B * Hkv
    head_steps = len(pl) * (steps - 1) * B * Hkv
    log(f"{tag} eager: blocks read {read / total:.3f}, refresh rate {refresh / head_steps:.3f}")

    def capture(fn_step, t0, t1, tail=None):
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            for t in range(t0, t1):
                fn_step(t)
            if tail is not None:
                tail()
        return g

    def timed(fn_step, init=None, tail=None):
        """tail: launches that close the last step (a carried update still pending), in the last graph."""
        if init is not None:
            init()
        torch.cuda.synchronize()
        graphs = [capture(fn_step, t0, min(steps, t0 + chunk), tail if t0 + chunk >= steps else None)
                  for t0 in range(1, steps, chunk)]
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for g in graphs:
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3          # us for steps 1 .. steps-1, all layers

    # timed: updates carried by the next layer's pass (the loop's default form here), then beside
    # the merge of their own layer
    carrier = UpdateCarrier()
    planners = make(False, carrier)
    us_plan = timed(lambda t: planner_pass(planners, t), init=lambda: planner_pass(planners, 0), tail=carrier.flush)
    del planners
    planners = make(False, None)
    us_plan_own = timed(lambda t: planner_pass(planners, t), init=lambda: planner_pass(planners, 0))
    del planners
    us_plan_one = math.nan
    if one_launch_plan:
        carrier = UpdateCarrier()
        planners = make(False, carrier, plan_one_launch=True)
        us_plan_one = timed(lambda t: planner_pass(planners, t), init=lambda: planner_pass(planners, 0),
                            tail=carrier.flush)
        del planners
    us_dense = timed(lambda t: [dense_layer(l, t) for l in range(layers)])
    n = (steps - 1) * layers
    us_replay, n_replay = replay_one_graph(run, qs, ids, pol, layers, first_planned, steps, T0) \
        if ragged is None and B == 1 and not post else (math.nan, 0)
    out = {"layers": layers, "steps": steps, "B": B, "Hq": Hq, "Hkv": Hkv,
           "T0": T0 if ragged is None else list(ragged), "query_noise": noise, "query_revert": revert,
           "query_jump_prob": p_jump,
           "mode": "refresh (trigger after the masked pass)" if post else "refresh_pre (trigger before the pass)",
           "policy": ("delta 0.05, max age 32" if post else
                      "stage 4 (delta 0.05, max age 32, calib 0.05 peak, warm (32, 8), auto index 0.1)")
                     + (", layer 0 dense" if dense_layer0 else ""),
           "blocks_read_frac": read / total,
           "refresh_rate": refresh / head_steps, "us_per_layer_step_policy": us_plan / n,
           "us_per_layer_step_policy_update_own_launch": us_plan_own / n,
           "us_per_layer_step_policy_one_launch_plan": us_plan_one / n if one_launch_plan else None,
           "us_per_layer_step_policy_one_graph_replayed": us_replay / n_replay if n_replay else None,
           "us_per_layer_step_dense": us_dense / n, "time_vs_dense": us_plan / us_dense,
           "dense_GBs": (B * Hkv * (T0 + steps // 2) * D * 4 / (us_dense / n) / 1e3) if ragged is None else None,
           "ms_per_decode_step_policy": us_plan / (steps - 1) / 1e3,
           "ms_per_decode_step_dense": us_dense / (steps - 1) / 1e3}
    log(f"{tag}: policy {us_plan / n:.2f} us/layer-step ({'refresh mode, ' if post else ''}updates carried; "
        f"{us_plan_own / n:.2f} with their own launch) vs dense {us_dense / n:.2f} (x{us_plan / us_dense:.3f}), {us_plan / (steps - 1) / 1e3:.3f} ms per "
        f"{layers}-layer step" + (f"; one graph replayed per step: {us_replay / n_replay:.2f}" if n_replay else "")
        + (f"; plan as one launch: {us_plan_one / n:.2f}" if one_launch_plan else ""))
    del run, qs
    return out


def planner_agreement(dev, cfg=4):
    """Decision agreement of the device planner loop with the oracle's refresh_pre loop as frozen in
    tests/golden/planner_cfg{4,5}.npz (untimed). Config 4: its two planned layers, 128 steps, updates
    carried, the decision in the pass, the token index found from the ids. Config 5: B 16 ragged
    contexts, 28 / 4 heads, 64 steps, one layer (plan's decision launch). Inputs regenerated on the
    CPU and checked against the fixture's digest. Per (layer or sequence, step, KV head): identical
    read sets (the reference's criterion, bench/test_planner.py:100-133) and identical refresh
    decisions; the oracle's smallest decision margin |estimate - delta| over the run (a refresh by
    age or a forced head has none), and the margins of the head-steps whose decision differs (a
    free-running loop that leaves the oracle at a float32 near tie stays apart until a common
    refresh: tests/test_gpu_loop_full.py tracks that)."""
    import numpy as np
    import torch

    from kvskip_amd import workloads as W
    from kvskip_amd.planner import FusedPlanner, Policy, UpdateCarrier

    d = np.load(Path(__file__).resolve().parent / "tests" / "golden" / f"planner_cfg{cfg}.npz", allow_pickle=False)
    run, layers, qs = W.loop_inputs(cfg)
    if W.input_digest(run, layers, qs) != str(d["digest"]):
        return {"error": f"the regenerated config-{cfg} inputs differ from the fixture's"}
    pol = Policy(calib=0.05, calib_kind="peak", calib_warm=(32, 8), calib_auto_ix=0.1)
    n = same_read = same_trig = 0
    min_margin, differ = math.inf, []

    def compare(rec, t, read, trig):
        nonlocal n, same_read, same_trig, min_margin, differ
        rr = d["read"][rec, t]
        ref_read = np.unpackbits(rr, axis=-1, count=rr.shape[-1] * 8)[..., :read.shape[-1]].astype(bool)
        ref_trig, m = d["trig"][rec, t], d["margin"][rec, t]
        n += trig.size
        same_read += int((~(read != ref_read).any(-1)).sum())
        same_trig += int((trig == ref_trig).sum())
        fin = m[np.isfinite(m)]
        if fin.size:
            min_margin = min(min_margin, float(fin.min()))
        differ += [float(m[h]) for h in np.nonzero(trig != ref_trig)[0]]

    ids = run.ids.to(dev)
    if cfg == 4:
        carrier = UpdateCarrier()
        fps = {l: FusedPlanner(pol, count=False, carrier=carrier) for l in layers}
        kv = {l: (run.k[l].to(dev), run.v[l].to(dev)) for l in layers}
        for t in range(run.steps):
            T = run.T0[0] + t + 1
            for i, l in enumerate(layers):
                k, v = kv[l][0][:, :, :T], kv[l][1][:, :, :T]
                q = qs[l][t].to(dev)
                if t == 0:
                    fps[l].first(q, k, v, run.scale)
                    continue
                fps[l].step(q, k, v, run.scale, ids=ids)
                compare(i, t, fps[l].read_mask(math.ceil(T / 64)).cpu().numpy()[0],
                        fps[l].state["trig"].bool().cpu().numpy()[0])
        what = f"{len(layers)} layers"
    else:
        fp = FusedPlanner(pol, count=False)
        k, v = run.k[0].to(dev), run.v[0].to(dev)
        base = torch.tensor(run.T0, dtype=torch.int32)
        for t in range(run.steps):
            sl = (base + t + 1).to(dev)
            q = qs[0][t].to(dev)
            if t == 0:
                fp.first(q, k, v, run.scale, seq_lens=sl)
                continue
            fp.step(q, k, v, run.scale, ids=ids, seq_lens=sl)
            bi, bc = fp.state["block_idx"].cpu().numpy(), fp.state["block_cnt"].cpu().numpy()
            trig = fp.state["trig"].bool().cpu().numpy()
            for b, T0 in enumerate(run.T0):
                nb = math.ceil((T0 + t + 1) / 64)
                read = np.zeros((bi.shape[1], nb), dtype=bool)
                for h in range(bi.shape[1]):
                    read[h, bi[b, h, :bc[b, h]]] = True
                compare(b, t, read, trig[b])
        what = f"{len(run.T0)} ragged sequences"
    out = {"fixture": f"tests/golden/planner_cfg{cfg}.npz", "records": what, "steps": run.steps - 1,
           "head_steps": n, "read_sets_identical": same_read / n, "decisions_identical": same_trig / n,
           "min_oracle_decision_margin": min_margin, "differing_decision_margins": differ}
    log(f"cfg{cfg} vs oracle: read sets identical on {same_read}/{n} head-steps, decisions on {same_trig}/{n}; "
        f"smallest oracle decision margin {min_margin:.2e}; differing decisions' margins {differ}")
    return out


def replay_one_graph(run, qs, ids, pol, layers, first_planned, steps, T0):
    """The config-4 loop as a server would run it: the step's length in device memory (seq_lens,
    B 1), one HIP graph of a whole step (length advance, every layer's plan / pass / merge with the
    updates carried) captured after the policy's warm-up and replayed for each later step; the
    query of each step is copied into the graph's input buffer between replays. Returns (us of the
    replayed steps, their layer-steps)."""
    import torch

    from kvskip_amd import kvskip as K
    from kvskip_amd.planner import FusedPlanner, UpdateCarrier

    dev = qs.device
    carrier = UpdateCarrier()
    planners = [None] * first_planned + [FusedPlanner(pol, count=False, carrier=carrier)
                                         for _ in range(first_planned, layers)]
    sl = torch.tensor([T0], dtype=torch.int32, device=dev)
    qbuf = torch.empty_like(qs[0])

    def step(t):
        sl.add_(1)
        for l in range(layers):
            if l < first_planned:
                K.decode(qbuf[l], run.k[l], run.v[l], run.scale, seq_lens=sl)
            elif t == 0:
                planners[l].first(qbuf[l], run.k[l], run.v[l], run.scale, seq_lens=sl)
            else:
                planners[l].step(qbuf[l], run.k[l], run.v[l], run.scale, ids=ids, seq_lens=sl)

    w = (pol.calib_warm[0] if pol.calib_warm else 0) + 1
    if steps <= w + 1:
        return math.nan, 0
    for t in range(w):
        qbuf.copy_(qs[t])
        step(t)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        step(w)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for t in range(w, steps):
        qbuf.copy_(qs[t])
        g.replay()
    e1.record()
    carrier.flush()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3, (steps - w) * layers


def _median_time(fn, reps, budget_s):
    """Median seconds of fn() over up to `reps` calls after one warm-up call, within budget_s."""
    fn()
    ts = []
    t_end = time.perf_counter() + budget_s
    while len(ts) < reps and (len(ts) < 5 or time.perf_counter() < t_end):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts), len(ts)


def cpu_baseline(cfg2, cfg3, bytes_dense, bytes_mask, bytes_v1, budget_s=6.0):
    """The reference-semantics PyTorch CPU path (the oracle's restatement in float32, all host
    threads) on a bounded sample of each path, median of >= 5 calls after one warm-up: config 2's
    dense layer-step, its masked + block-statistics step over the 35% list, config 3's single-pass
    V-skip (the keep rule, then attention over the kept V), and one refresh_pre layer-step of the
    planner (config 4's shape: plan, masked + statistics attention, update)."""
    import torch

    from kvskip_amd import workloads as W
    from oracle import attention as O
    from oracle import planner as OP

    n_threads = os.cpu_count() or 1
    torch.set_num_threads(n_threads)
    f32 = torch.float32
    q, k, v, scale, keep = cfg2
    paths = {}

    def record(name, fn, nbytes, what):
        med, n = _median_time(fn, 9, budget_s)
        paths[name] = {"us_per_layer_step": round(med * 1e6, 1), "samples": n, "what": what}
        if nbytes:
            paths[name]["GBs"] = round(nbytes / med / 1e9, 2)
        log(f"cpu {name}: {med * 1e3:.1f} ms per layer-step")

    record("dense_cfg2", lambda: O.decode(q, k, v, scale, dtype=f32), bytes_dense,
           "config 2 dense decode, fp32 einsum -> softmax -> einsum")
    record("masked_stats_cfg2", lambda: (O.decode(q, k, v, scale, keep=keep, dtype=f32),
                                         O.block_stats(q, k, scale, keep=keep, dtype=f32)), bytes_mask,
           "config 2 masked decode over the 35% list + per-block statistics, fp32")
    q3, k3, v3, scale3, lp3 = cfg3
    record("vskip1_cfg3", lambda: O.vskip1(q3, k3, v3, scale3, 1e-4, 2, lse_prev=lp3.double(), dtype=f32), bytes_v1,
           "config 3 single-pass V-skip (T 65536): block statistics, the keep rule, attention over the kept V, fp32")
    del q3, k3, v3
    run = W.planner_run(layers=1, T0=32768, steps=16, seed=4)
    qp = W.QueryProcess(run, 0)
    pol = OP.Policy(calib=0.05, calib_kind="peak", calib_warm=(32, 8), calib_auto_ix=0.1)
    box = {"T": 32769}
    st, _ = OP.init(qp.next(), run.k[0][:, :, :32769], run.v[0][:, :, :32769], run.scale, pol)
    ids = run.ids.numpy()

    def planner_step():
        box["T"] += 1
        T = box["T"]
        OP.step(st, qp.next(), run.k[0][:, :, :T], run.v[0][:, :, :T], pol,
                idx=torch.from_numpy(OP.index_blocks(ids, T)), dtype=f32)

    record("refresh_pre_step_cfg4", planner_step, None,
           "one refresh_pre layer-step of config 4's shape after a dense first step: plan (centroid drift "
           "estimate, decision, list; float64), masked + statistics attention (float32), update (top-p, references, "
           "calibration; float64)")
    d = paths["dense_cfg2"]
    return {"value": d["GBs"], "unit": "GB/s", "cores": n_threads, "kind": "port",
            "us_per_layer_step": d["us_per_layer_step"],
            "sample": "config 2 dense decode steps (one layer, T 32768), median of >= 5 after one warm-up; "
                      "the other paths in `paths`",
            "cpu": _cpu_model(), "paths": paths}


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


if __name__ == "__main__":
    main()
