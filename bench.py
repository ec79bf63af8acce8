#!/usr/bin/env python3
"""Fused tiered decode attention on one MI355X: us/step, achieved HBM GB/s, fraction of peak.

Workload (default): the Llama-3-8B-shaped decode step across all 32 layers --
32 query heads / 8 KV heads (GQA 4:1), head_dim 128, FP32 Q, batch 1, context
32768 with 4 sinks + 256 recent + 1639 heavy hitters (5%) in FP32 and the other
30869 tokens 2-bit packed in 1930 16-token blocks (last block 5 valid + 11
masked). K ~ N(0,1) with 4 outlier channels per KV head scaled x8, V ~ N(0,1);
synthetic, generated on the GPU from a seed, packed by the library's own
quantisers. Each layer has its own tier tables (1.57 GB in HBM in total), so
every step streams from HBM, not from the 256 MB Infinity Cache.

One step = the 32 layers one after another, each with its attention output and
its mean attention weights, replayed as one HIP graph: per layer the split-K
partials (tt_attention_partials) and one finalize launch that merges this
layer's partials and computes the previous layer's mean weights
(tt_attention_finalize_deferred, two workspaces taking turns); the last
layer's mean weights get a launch of their own. The same step as one
tt_fused_attention_decode_ws call per layer (merge and mean weights of a layer
in one launch) is timed beside it (`us_per_step_per_layer_calls`), and both
are checked to give the same outputs (bit for bit) and mean weights (1e-6).
Steps of fewer than 16 layers (the 8-layer MHA case) report the per-layer
calls as `value`: there the extra launch outweighs what deferring saves.
The dominant kernel (attn_packed_kernel: split-K partials, the packed blocks on
the matrix cores and the FP32 tiers on the VALU) is also timed on its own: a
HIP graph of the 32 layers' partials launches, HIP events on the launch
stream, time / 32 per launch (the figure rocprofv3 reports as the kernel's
average duration). `traffic` is the kernel's HBM bytes per launch from
rocprofv3 counters, read from the committed counter summary under profiles/
(made with --pmc-driver and --pmc-summary, see there).

The CPU baseline is the reference's own AVX2+OpenMP kernel
(oracle/_ref/libttref.so, compiled from the reference sources) on the host
cores, on a bounded sample of the same workload (whole layers, scaled to a
32-layer step); the GPU output of that layer is checked against it.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0
METRIC = "decode-attn µs/step + achieved HBM GB/s (% of peak), 32k ctx Llama-3-8B shape"

CONFIGS = {
    # name: (Hq, Hkv, D, ctx, layers, k_outliers)
    "llama3-8b-32k": (32, 8, 128, 32768, 32, "x8"),
    # the single-layer 8k MHA case, as 8 independent layers (438 MB) so that no step is served from the
    # 256 MB Infinity Cache
    "mha-8k-8layers": (32, 32, 128, 8192, 8, None),
    "qwen2-7b-128k": (28, 4, 128, 131072, 28, "t3"),
    # head_dim 64 (the SmolLM / TinyLlama / Qwen2-0.5B head size), GQA 4:1: KV heads taken in pairs as heads of
    # 128 channels on the matrix-core kernel
    "llama-hd64-32k": (32, 8, 64, 32768, 32, "x8"),
    # head sizes on the VALU split kernel: head_dim 256 with GQA 2:1 (the Gemma-2-9B shape, 42 layers) and
    # head_dim 80 with 32/32 heads (the Phi-2 shape, 32 layers)
    "gemma2-9b-hd256-8k": (16, 8, 256, 8192, 42, "x8"),
    "phi2-hd80-2k": (32, 32, 80, 2048, 32, None),
}


def dominant_kernel(D: int, Hkv: int) -> str:
    """The partials kernel a layer of this shape runs: the matrix-core one for head_dim 128 and for head_dim 64 with
    an even KV-head count (heads taken in pairs), the VALU split kernel for every other head_dim."""
    return "attn_packed_kernel" if D == 128 or (D == 64 and Hkv % 2 == 0) else "attn_split_kernel"


def tier_sizes(ctx: int):
    S, R = 4, 256
    hh = int(math.ceil(float(ctx) * 0.05))
    nd = S + hh + R
    npk = ctx - nd
    nb = (npk + 15) // 16
    return nd, npk, nb


def bytes_read_per_layer(Hq, Hkv, D, ctx, meta_bytes, with_ids=True):
    """Bytes the split kernel reads per (sequence, layer): Q, FP32 tiers, packed
    words, scale/zero metadata, and the int64 token ids it checks for masking."""
    nd, _, nb = tier_sizes(ctx)
    b = Hq * D * 4
    b += 2 * nd * Hkv * D * 4
    b += nb * Hkv * D * 4                      # K words (16 tokens per int32)
    b += nb * Hkv * D * 2 * meta_bytes         # K scale + zero per (block, head, channel)
    b += nb * 16 * Hkv * (D // 16) * 4         # V words (16 channels per int32)
    b += nb * 16 * Hkv * 2 * meta_bytes        # V scale + zero per (token, head)
    if with_ids:
        b += nb * 16 * 8
    return b


def build_layers(torch, L, Hq, Hkv, D, ctx, layers, outliers, seed, metas=("32", "16")):
    nd, npk, nb = tier_sizes(ctx)
    g = torch.Generator(device="cuda").manual_seed(seed)
    dev = "cuda"
    out = []
    for layer in range(layers):
        K = torch.randn((nb * 16 + nd, Hkv, D), generator=g, device=dev)
        V = torch.randn((nb * 16 + nd, Hkv, D), generator=g, device=dev)
        if outliers == "x8":
            for h in range(Hkv):
                ch = torch.randperm(D, generator=g, device=dev)[:4]
                K[:, h, ch] *= 8.0
        elif outliers == "t3":
            for h in range(Hkv):
                ch = torch.randperm(D, generator=g, device=dev)[:4]
                z = torch.randn((K.shape[0], 4), generator=g, device=dev)
                chi = (torch.randn((K.shape[0], 4, 3), generator=g, device=dev) ** 2).sum(-1)
                K[:, h, ch] = z / torch.sqrt(chi / 3.0)
        pad = nb * 16 - npk
        if pad:  # pad the last block with copies of its last valid token
            K[nd + npk:] = K[nd + npk - 1]
            V[nd + npk:] = V[nd + npk - 1]
        Q = torch.randn((Hq, D), generator=g, device=dev)
        d = {"Q": Q, "dK": K[:nd].contiguous(), "dV": V[:nd].contiguous()}
        pk, pv = K[nd:].contiguous(), V[nd:].contiguous()
        d["KP"] = torch.empty((nb, Hkv, D), dtype=torch.int32, device=dev)
        d["VP"] = torch.empty((nb * 16, Hkv, D // 16), dtype=torch.int32, device=dev)
        for tag, fp16, mdt in (("32", 0, torch.float32), ("16", 1, torch.uint16)):
            if tag not in metas:
                continue
            ks = torch.empty((nb, Hkv, D), dtype=mdt, device=dev)
            kz = torch.empty_like(ks)
            vs = torch.empty((nb * 16, Hkv), dtype=mdt, device=dev)
            vz = torch.empty_like(vs)
            L.check(L.load().tt_quantize_k_block(pk.data_ptr(), d["KP"].data_ptr(), ks.data_ptr(), kz.data_ptr(), nb,
                                                 Hkv, D, 16, fp16, C.c_void_p(torch.cuda.current_stream().cuda_stream)))
            L.check(L.load().tt_quantize_v_block(pv.data_ptr(), d["VP"].data_ptr(), vs.data_ptr(), vz.data_ptr(),
                                                 nb * 16, Hkv, D, fp16,
                                                 C.c_void_p(torch.cuda.current_stream().cuda_stream)))
            d["KS" + tag], d["KZ" + tag], d["VS" + tag], d["VZ" + tag] = ks, kz, vs, vz
        ids = torch.arange(nb * 16, dtype=torch.int64, device=dev) + nd
        if pad:
            ids[-pad:] = -1
        d["ids"] = ids
        d["out"] = torch.empty((Hq, D), dtype=torch.float32, device=dev)
        d["mw"] = torch.empty((nd + nb * 16,), dtype=torch.float32, device=dev)
        del K, V, pk, pv
        out.append(d)
    torch.cuda.synchronize()
    return out, (nd, npk, nb)


PMC_TRAFFIC_MD = os.path.join(ROOT, "profiles", "attn_packed_kernel_llama3-8b-32k_hbm_traffic.md")
DEFER_MIN_LAYERS = 16  # steps of at least this many layers time the deferred-mean-weights layout


KERNEL_SOURCES = ("tt_attn.hip", "tt_attn_mfma.h", "tt_attn.h", "tt_common.h")


def kernel_source_digest():
    """SHA-256 (first 16 hex digits) of the attention kernels' sources: stamps a counter summary with the code it
    measured."""
    import hashlib

    h = hashlib.sha256()
    for f in KERNEL_SOURCES:
        h.update(open(os.path.join(ROOT, "tritiercache_amd", "csrc", f), "rb").read())
    return h.hexdigest()[:16]


def traffic_from_profile(config, meta):
    """(HBM bytes per partials launch, reads + writes, from the committed counter summary; whether that summary
    is stale). The figure is None when the summary does not cover this workload and metadata type, or when it
    was measured on other kernel sources than the ones built here (then stale is True)."""
    if config != "llama3-8b-32k" or not os.path.exists(PMC_TRAFFIC_MD):
        return None, False
    stamp, val = None, None
    for line in open(PMC_TRAFFIC_MD):
        if line.startswith("kernel_sources_sha256:"):
            stamp = line.split(":")[1].strip()
        if line.startswith(f"traffic_bytes_per_launch[{meta}]:"):
            val = int(line.split(":")[1])
    if stamp != kernel_source_digest():
        return None, True
    return val, False


def pmc_driver(torch, lib, L, data, layer_args, tag, fp16, ws, ws_bytes, sp):
    """Workload for rocprofv3 --pmc: the calibration copy, then 5 partials launches of layer 0 with cache
    eviction in between (so every launch reads its layer from HBM)."""
    src = torch.empty(64 << 20, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    d = data[0]
    for _ in range(5):
        L.check(lib.tt_attention_partials(*layer_args(d, tag), 16, fp16, 1, ws.data_ptr(), ws_bytes, sp()),
                "partials")
        dst.copy_(src)
    torch.cuda.synchronize()
    print("[bench] pmc driver done", file=sys.stderr)


def pmc_summary(dirs):
    """Markdown summary of rocprofv3 --pmc runs of --pmc-driver: per-dispatch counter values of the partials
    kernel and of the 256 MiB copy (calibration), and the HBM bytes per launch they give."""
    import collections
    import csv
    import glob
    import re

    vals = collections.defaultdict(list)  # (kernel, counter) -> per-dispatch totals
    for d in dirs:
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            per = collections.defaultdict(float)
            names = {}
            for r in csv.DictReader(open(f)):
                k = r["Kernel_Name"]
                # attn_packed_kernel<4, float> or <4, float, false> (the unpaired instantiation)
                kind = ("attn_packed_kernel<4, float>" if re.search(r"attn_packed_kernel<4, float(, false)?>", k) else
                        "attn_packed_kernel<4, unsigned short>"
                        if re.search(r"attn_packed_kernel<4, unsigned short(, false)?>", k) else
                        "copy 256 MiB (calibration)" if "copyBuffer" in k else None)
                if kind is None:
                    continue
                per[(r["Dispatch_Id"], r["Counter_Name"])] += float(r["Counter_Value"])
                names[r["Dispatch_Id"]] = kind
            for (did, c), v in per.items():
                vals[(names[did], c)].append(v)
    med = {k: sorted(v)[len(v) // 2] for k, v in vals.items()}
    print("| dispatch | counter | per dispatch (median) | dispatches |")
    print("|:--|:--|--:|--:|")
    for (k, c), v in sorted(vals.items()):
        print(f"| {k} | {c} | {med[(k, c)]:.0f} | {len(v)} |")
    copy = "copy 256 MiB (calibration)"
    fs, ws_ = med.get((copy, "FETCH_SIZE")), med.get((copy, "WRITE_SIZE"))
    if not fs or not ws_:
        return
    ff, wf = 262144.0 / fs, 262144.0 / ws_
    print(f"\ncalibration: the copy reads and writes 262144 KiB; FETCH_SIZE reads {fs:.0f} KiB (factor {ff:.3f}), "
          f"WRITE_SIZE {ws_:.0f} KiB (factor {wf:.3f})\n")
    for k, meta in (("attn_packed_kernel<4, float>", "fp32"), ("attn_packed_kernel<4, unsigned short>", "fp16")):
        if (k, "FETCH_SIZE") in med and (k, "WRITE_SIZE") in med:
            rd = med[(k, "FETCH_SIZE")] * ff * 1024
            wr = med[(k, "WRITE_SIZE")] * wf * 1024
            print(f"{k}: reads {rd / 1e6:.2f} MB, writes {wr / 1e6:.2f} MB per launch\n")
            print(f"traffic_bytes_per_launch[{meta}]: {int(rd + wr)}\n")
    print(f"kernel_sources_sha256: {kernel_source_digest()}\n")


def trace_summary(db_path):
    """Markdown table of kernel durations (calls, average, median, min, max, share of GPU time) from a
    rocprofv3 --kernel-trace results database."""
    import collections
    import sqlite3

    rows = sqlite3.connect(db_path).execute("select name, start, end from kernels").fetchall()
    dur = collections.defaultdict(list)
    for name, s, e in rows:
        n = name.replace("(anonymous namespace)::", "").replace("void ", "")
        dur[n.split("(")[0]].append((e - s) / 1e3)
    total = sum(sum(v) for v in dur.values())
    print("| kernel | calls | avg (us) | median (us) | min (us) | max (us) | % of GPU time |")
    print("|:--|--:|--:|--:|--:|--:|--:|")
    for k, v in sorted(dur.items(), key=lambda kv: -sum(kv[1]))[:8]:
        v.sort()
        print(f"| `{k[:70]}` | {len(v)} | {sum(v) / len(v):.2f} | {v[len(v) // 2]:.2f} | {v[0]:.2f} | {v[-1]:.2f} | "
              f"{100.0 * sum(v) / total:.1f} |")


ENGINE_CONFIGS = {
    # Long-context decode through the engine: per layer one TriTierCacheEngine prefilled with `ctx` tokens,
    # then `steps` decode steps of (ring ingest -> eviction routing -> waiting-room pack -> fused attention ->
    # score feedback) over all layers. K outlier channels Student-t (nu = 3).
    "qwen2-7b-128k-engine": dict(mode="step", Hq=28, Hkv=4, D=128, ctx=131072, layers=28, steps=256, S=4, R=256,
                                 hr=0.05, decay=0.999, iv=32, kgs=16, meta="fp32", outliers="t3"),
    # Tier maintenance alone: 2048 appends at 32 KV heads x 128 (ingest, routing, flush), each followed by the
    # decayed score update with injected per-token weights, softmax of N(0, 2^2) logits over the visible set.
    "maint-2048-32kv": dict(mode="inject", Hq=32, Hkv=32, D=128, ctx=0, layers=1, steps=2048, S=4, R=256, hr=0.05,
                            decay=0.999, iv=32, kgs=16, meta="fp32", outliers=None, msl=2048),
}


def engine_bench(args, torch, L, lib):
    """Engine configurations: µs per decode step over all layers (eager calls, one stream). Steps of 16 layers or
    more also run with each layer's mean weights and score feedback in the next layer's finalize launch
    (tt_engine_step_deferred, the last layer's flushed), on a fresh set of engines with the same data; `value` is
    that layout's, `us_per_step_per_layer_calls` the per-layer tt_engine_step figure."""
    import numpy as np

    cfg = ENGINE_CONFIGS[args.config]
    Hq, Hkv, D, layers, steps = cfg["Hq"], cfg["Hkv"], cfg["D"], cfg["layers"], cfg["steps"]
    msl = cfg.get("msl", cfg["ctx"] + steps + 64)
    sp = lambda: C.c_void_p(torch.cuda.current_stream().cuda_stream)  # noqa: E731
    names = lib.tt_engine_counter_names().decode().split()

    def run_mode(deferred):
        g = torch.Generator(device="cuda").manual_seed(args.seed)
        engines = []
        t0 = time.time()
        for layer in range(layers):
            h = C.c_void_p()
            L.check(lib.tt_engine_create(C.byref(h), Hq, Hkv, D, msl, cfg["S"], cfg["R"], cfg["hr"], cfg["decay"],
                                         cfg["iv"], cfg["kgs"], cfg["meta"].encode(), sp()), "engine_create")
            engines.append(h)
            if cfg["ctx"]:
                K = torch.randn((cfg["ctx"], Hkv, D), generator=g, device="cuda")
                V = torch.randn((cfg["ctx"], Hkv, D), generator=g, device="cuda")
                if cfg["outliers"] == "t3":
                    for hh in range(Hkv):
                        ch = torch.randperm(D, generator=g, device="cuda")[:4]
                        z = torch.randn((cfg["ctx"], 4), generator=g, device="cuda")
                        chi = (torch.randn((cfg["ctx"], 4, 3), generator=g, device="cuda") ** 2).sum(-1)
                        K[:, hh, ch] = z / torch.sqrt(chi / 3.0)
                L.check(lib.tt_engine_prefill(h, K.data_ptr(), V.data_ptr(), cfg["ctx"], sp()), "prefill")
                del K, V
        torch.cuda.synchronize()
        print(f"[bench] {layers} engines ready in {time.time() - t0:.1f}s", file=sys.stderr, flush=True)
        n_in = 8  # distinct input sets, cycled
        Q = torch.randn((n_in, layers, Hq * D), generator=g, device="cuda")
        Kn = torch.randn((n_in, layers, Hkv * D), generator=g, device="cuda")
        Vn = torch.randn((n_in, layers, Hkv * D), generator=g, device="cuda")
        out = torch.empty((layers, Hq * D), device="cuda")
        if cfg["mode"] == "inject":
            w = torch.softmax(2.0 * torch.randn((n_in, msl + 1024), generator=g, device="cuda"), dim=-1)

        def run(s):
            i = s % n_in
            for layer, h in enumerate(engines):
                if cfg["mode"] == "step" and deferred:
                    prev = engines[layer - 1] if layer > 0 else None
                    L.check(lib.tt_engine_step_deferred(h, Q[i, layer].data_ptr(), Kn[i, layer].data_ptr(),
                                                        Vn[i, layer].data_ptr(), out[layer].data_ptr(), prev, sp()),
                            "step_deferred")
                elif cfg["mode"] == "step":
                    L.check(lib.tt_engine_step(h, Q[i, layer].data_ptr(), Kn[i, layer].data_ptr(),
                                               Vn[i, layer].data_ptr(), out[layer].data_ptr(), sp()), "step")
                else:
                    L.check(lib.tt_engine_ingest(h, Kn[i, layer].data_ptr(), Vn[i, layer].data_ptr(), sp()), "ingest")
                    L.check(lib.tt_engine_feedback(h, w[i].data_ptr(), sp()), "feedback")
            if cfg["mode"] == "step" and deferred:
                L.check(lib.tt_engine_flush_feedback(engines[-1], sp()), "flush")

        warm = min(args.warmup, 8)
        for s in range(warm):
            run(s)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for s in range(warm, steps):
            run(s)
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1000.0 / (steps - warm)
        cnt = np.zeros(23, np.int64)
        L.check(lib.tt_engine_counters(engines[0], cnt.ctypes.data, sp()), "counters")
        c = dict(zip(names, (int(x) for x in cnt)))
        roof = engine_kernel_roofline(engines) if deferred and cfg["mode"] == "step" else None
        for h in engines:
            lib.tt_engine_destroy(h)
        torch.cuda.synchronize()
        return us, warm, c, roof

    def engine_kernel_roofline(engines, reps=20):
        """The attention partials kernel over the engines' own tiers as they stand after the timed steps, with
        the counts from each engine's counters: per layer the FP32 tiers (sinks, heavy hitters, recent window)
        gathered into one dense array -- the rows and bytes the engine's launch reads from its three buffers --
        and the packed store used in place. A HIP graph of the layers' partials launches, HIP events on the
        launch stream around `reps` replays after 10 untimed ones: µs per launch, and the algorithmic bytes
        per launch from the actual tier counts (averaged over the layers)."""
        from tritiercache_amd._C import _DeviceView

        def view(h, which, shape, typestr):
            p, n, es = C.c_void_p(), C.c_int64(), C.c_int()
            L.check(lib.tt_engine_buffer(h, which, C.byref(p), C.byref(n), C.byref(es), sp()), "buffer")
            want = int(np.prod(shape))
            assert want <= n.value, (which, shape, n.value)
            if want == 0:
                return None
            return torch.as_tensor(_DeviceView(p.value, shape, typestr, None), device="cuda")

        mt = "<u2" if cfg["meta"] == "fp16" else "<f4"
        kgs, W = cfg["kgs"], cfg["kgs"] // 16
        fp16 = 1 if cfg["meta"] == "fp16" else 0
        layer_in, total_bytes, max_ws = [], 0, 0
        for h in engines:
            cnt = np.zeros(23, np.int64)
            L.check(lib.tt_engine_counters(h, cnt.ctypes.data, sp()), "counters")
            cc = dict(zip(names, (int(x) for x in cnt)))
            s_, hh, rw, nb = cc["s_count"], cc["hh_count"], cc["rw_count"], cc["pbs_blocks_used"]
            ks, vs = [], []
            for wk, wv, n_rows in ((0, 1, s_), (4, 5, hh), (2, 3, rw)):
                if n_rows:
                    ks.append(view(h, wk, (n_rows, Hkv, D), "<f4"))
                    vs.append(view(h, wv, (n_rows, Hkv, D), "<f4"))
            nd = s_ + hh + rw
            dK, dV = torch.cat(ks).contiguous(), torch.cat(vs).contiguous()
            pk = (view(h, 11, (nb * W, Hkv, D), "<i4"), view(h, 12, (nb, Hkv, D), mt), view(h, 13, (nb, Hkv, D), mt),
                  view(h, 14, (nb * kgs, Hkv, D // 16), "<i4"), view(h, 15, (nb * kgs, Hkv), mt),
                  view(h, 16, (nb * kgs, Hkv), mt), view(h, 17, (nb * kgs,), "<i8"))
            q = torch.randn((Hq, D), device="cuda")
            layer_in.append((q, dK, dV, nd, pk, nb))
            b = Hq * D * 4 + 2 * nd * Hkv * D * 4 + nb * W * Hkv * D * 4 + nb * Hkv * D * 2 * (2 if fp16 else 4) \
                + nb * kgs * Hkv * (D // 16) * 4 + nb * kgs * Hkv * 2 * (2 if fp16 else 4) + nb * kgs * 8
            total_bytes += b
            max_ws = max(max_ws, int(lib.tt_fused_attention_workspace_bytes(nd, nb, Hq, Hkv, D, kgs, 1)))
        ws = torch.empty(max_ws, dtype=torch.uint8, device="cuda")

        def partials():
            for q, dK, dV, nd, pk, nb in layer_in:
                L.check(lib.tt_attention_partials(q.data_ptr(), dK.data_ptr(), dV.data_ptr(), nd,
                                                  *[t.data_ptr() for t in pk], nb, Hq, Hkv, D, kgs, fp16, 1,
                                                  ws.data_ptr(), max_ws, sp()), "partials")

        partials()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            partials()
        for _ in range(10):
            g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        us_launch = e0.elapsed_time(e1) * 1000.0 / (reps * len(layer_in))
        bpl = total_bytes / len(layer_in)
        del g
        return {"bound": "hbm", "kernel": dominant_kernel(D, Hkv),
                "achieved": round(bpl / (us_launch * 1e-6) / 1e9, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                "frac": round(bpl / (us_launch * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4), "traffic": None,
                "bytes_per_launch": int(bpl), "avg_launch_us": round(us_launch, 3),
                "tiers_layer0": {"dense": layer_in[0][3], "blocks": layer_in[0][5]},
                "how": "partials launches over the engines' own tiers after the timed steps (FP32 tiers gathered "
                       "into one array), graph of all layers, HIP events"}

    deferred = cfg["mode"] == "step" and layers >= DEFER_MIN_LAYERS
    us_per_layer_calls = None
    roof = None
    if deferred:
        us, warm, c, roof = run_mode(True)
        us_per_layer_calls, _, c_ref, _ = run_mode(False)
        same_state = c == c_ref
    else:
        us, warm, c, _ = run_mode(False)
    result = {
        "metric": f"engine decode step µs/step ({args.config})",
        "value": round(us, 2), "unit": "us/step", "n_gpus": 1, "steps": steps - warm, "warmup": warm,
        "ms_per_step": round(us / 1000.0, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic (seeded on the GPU)",
        "config": {"workload": args.config, **{k: v for k, v in cfg.items()}, "max_seq_len": msl, "seed": args.seed,
                   "finalize": "mean weights and score feedback of each layer in the next layer's finalize launch"
                   if deferred else ("per layer: tt_engine_step" if cfg["mode"] == "step" else
                                     "per layer: tt_engine_ingest, then tt_engine_feedback with injected weights")},
        "final_state_layer0": {k: c[k] for k in ("total_processed_tokens", "s_count", "hh_count", "rw_count",
                                                 "wr_count", "pbs_count", "pbs_blocks_used", "total_evictions")},
    }
    if deferred:
        result["us_per_step_per_layer_calls"] = round(us_per_layer_calls, 2)
        result["per_layer_calls_same_counters"] = bool(same_state)
    if cfg["mode"] == "step":
        nd = c["s_count"] + c["hh_count"] + c["rw_count"]
        nb = c["pbs_blocks_used"]
        mb = 2 if cfg["meta"] == "fp16" else 4
        b = Hq * D * 4 + 2 * nd * Hkv * D * 4 + nb * Hkv * D * 4 * (cfg["kgs"] // 16) + nb * Hkv * D * 2 * mb \
            + nb * cfg["kgs"] * Hkv * (D // 16) * 4 + nb * cfg["kgs"] * Hkv * 2 * mb + nb * cfg["kgs"] * 8
        result["attention_bytes_per_step"] = b * layers
        result["attention_GBps"] = round(b * layers / (us * 1e-6) / 1e9, 1)
    if roof is not None:
        result["roofline"] = roof
    print(json.dumps(result), flush=True)


BATCH_CONFIGS = {
    # Batched ragged decode: `batch` sequences with contexts ~ U[lo, hi] drawn from the seed, each with its own tier
    # tables (4 sinks, 256 recent, 5% heavy hitters FP32, the rest 2-bit) in every layer; one
    # tt_fused_attention_decode_batched call per layer, the 32 layers replayed as one HIP graph.
    "mistral-7b-batch16": dict(Hq=32, Hkv=8, D=128, batch=16, lo=2048, hi=32768, layers=32),
}


def batch_bench(args, torch, L, lib):
    """Batched ragged decode: µs per step (all sequences, all layers), HBM GB/s on the bytes the step reads."""
    import numpy as np

    cfg = BATCH_CONFIGS[args.config]
    Hq, Hkv, D, B, layers = cfg["Hq"], cfg["Hkv"], cfg["D"], cfg["batch"], cfg["layers"]
    fp16 = 1 if args.meta == "fp16" else 0
    tag = "16" if fp16 else "32"
    mb = 2 if fp16 else 4
    ctxs = [int(c) for c in np.random.default_rng(args.seed).integers(cfg["lo"], cfg["hi"] + 1, size=B)]
    sp = lambda: C.c_void_p(torch.cuda.current_stream().cuda_stream)  # noqa: E731
    t0 = time.time()
    data = []  # [layer][seq] -> tier tables
    for layer in range(layers):
        row = []
        for i, ctx in enumerate(ctxs):
            d, sizes = build_layers(torch, L, Hq, Hkv, D, ctx, 1, None, args.seed + 7919 * layer + i, metas=(tag,))
            d[0]["sizes"] = sizes
            row.append(d[0])
        data.append(row)
    print(f"[bench] built {layers} layers x {B} sequences (ctx {min(ctxs)}..{max(ctxs)}) in {time.time() - t0:.1f}s",
          file=sys.stderr, flush=True)
    descs, ws_bytes = [], 0
    for row in data:
        arr = (L.DecodeSeq * B)()
        for i, d in enumerate(row):
            nd, _, nb = d["sizes"]
            s = arr[i]
            s.Q, s.dense_K, s.dense_V = d["Q"].data_ptr(), d["dK"].data_ptr(), d["dV"].data_ptr()
            s.PBS_K_Packed, s.PBS_K_Scales, s.PBS_K_Zeroes = (d["KP"].data_ptr(), d["KS" + tag].data_ptr(),
                                                              d["KZ" + tag].data_ptr())
            s.PBS_V_Packed, s.PBS_V_Scales, s.PBS_V_Zeroes = (d["VP"].data_ptr(), d["VS" + tag].data_ptr(),
                                                              d["VZ" + tag].data_ptr())
            s.PBS_token_ids, s.attn_output, s.mean_attn_weights = (d["ids"].data_ptr(), d["out"].data_ptr(),
                                                                   d["mw"].data_ptr())
            s.dense_count, s.num_blocks = nd, nb
        dev = torch.from_numpy(np.frombuffer(bytes(arr), dtype=np.uint8).copy()).cuda()
        descs.append((arr, dev))
        ws_bytes = max(ws_bytes, int(lib.tt_batched_decode_workspace_bytes(arr, B, Hq, Hkv, D, 16)))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")

    def step():
        for arr, dev in descs:
            L.check(lib.tt_fused_attention_decode_batched(arr, dev.data_ptr(), B, Hq, Hkv, D, 16, fp16, ws.data_ptr(),
                                                          ws_bytes, sp()), "batched")

    step()
    torch.cuda.synchronize()
    run, graphed = step, False
    if not args.no_graph:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            step()
        run, graphed = g.replay, True
    for _ in range(args.warmup):
        run()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        run()
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1000.0 / args.steps
    per_seq = [bytes_read_per_layer(Hq, Hkv, D, c, mb) for c in ctxs]
    bstep = sum(per_seq) * layers
    gbps = bstep / (us * 1e-6) / 1e9

    cpu = parity = None
    if not args.no_cpu:
        from oracle.binding import load_oracle, load_reference

        impl = load_reference() or load_oracle()
        tot = 0.0
        toks = 0
        n = 0
        for i in range(B):  # layer 0, sequences in order, within the time bound
            d = data[0][i]
            nd, _, nb = d["sizes"]
            h = {k: (v.cpu().numpy() if v.dtype != torch.uint16 else v.cpu().view(torch.int16).numpy().view(np.uint16))
                 for k, v in d.items() if k != "sizes"}
            cargs = (h["Q"], h["dK"], h["dV"], nd, h["KP"].reshape(nb, 1, Hkv, D), h["KS" + tag], h["KZ" + tag],
                     h["VP"], h["VS" + tag], h["VZ" + tag], h["ids"], nb, Hq, Hkv, D, 16, bool(fp16))
            t1 = time.perf_counter()
            ro, rmw = impl.fused_attention_decode(*cargs)
            tot += time.perf_counter() - t1
            toks += nd + nb * 16
            n += 1
            if i == 0:
                parity = {
                    "seq0_layer0_out_max_rel_err": float(np.abs(h["out"] - ro).max() / np.abs(ro).max()),
                    "seq0_layer0_mean_weights_max_rel_err": float(np.abs(h["mw"] - rmw).max() / np.abs(rmw).max()),
                    "checked_against": impl.kind,
                }
            if tot >= args.cpu_seconds:
                break
        all_toks = sum(tier_sizes(c)[0] + tier_sizes(c)[2] * 16 for c in ctxs) * layers
        threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1)) if impl.kind == "reference" else 1
        cpu = {"value": tot / toks * all_toks * 1e6, "unit": "us/step", "cores": threads, "kind": impl.kind,
               "sample": f"layer 0 of the first {n} sequences ({toks} tokens), {tot:.1f}s, scaled by tokens to "
                         f"{B} sequences x {layers} layers"}
    result = {
        "metric": f"batched ragged decode-attn µs/step ({args.config})",
        "value": round(us, 2), "unit": "us/step", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(us / 1000.0, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic (seeded N(0,1) on the GPU; packed by the library quantisers)",
        "config": {"workload": f"{args.config}: {B} sequences, ctx {ctxs}, {Hq} q heads / {Hkv} KV heads, head_dim "
                               f"{D}, {layers} layers, {args.meta} metadata, mean attention weights computed",
                   "ctxs": ctxs, "layers": layers, "hip_graph": graphed, "seed": args.seed},
        "achieved_GBps": round(gbps, 1),
        "pct_of_hbm_peak": round(100.0 * gbps / HBM_PEAK_GBPS, 2),
        "bytes_read_per_step": bstep,
        "roofline": {"bound": "hbm", "kernel": "step (attn_batched_kernel + attn_finalize_batched_kernel)",
                     "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": None},
        "cpu_baseline": cpu,
        "parity": parity,
    }
    print(json.dumps(result), flush=True)


def host_cores():
    """(physical cores, logical CPUs) this process may run on: the affinity mask, cores counted as distinct
    (socket, core) pairs from lscpu."""
    import subprocess

    cpus = sorted(os.sched_getaffinity(0))
    phys = None
    try:
        out = subprocess.run(["lscpu", "-p=CPU,CORE,SOCKET"], capture_output=True, text=True, check=True).stdout
        pairs = {}
        for line in out.splitlines():
            if line and not line.startswith("#"):
                c, core, sock = line.split(",")[:3]
                pairs[int(c)] = (sock, core)
        phys = len({pairs[c] for c in cpus if c in pairs}) or None
    except Exception:
        pass
    return phys, len(cpus)


def set_omp_threads(n):
    """Threads of the OpenMP runtime the compiled reference kernel uses (libgomp), for this process."""
    import ctypes

    try:
        ctypes.CDLL("libgomp.so.1").omp_set_num_threads(int(n))
        return True
    except OSError:
        return False


ARITHMETIC = ("f32 inputs and outputs; FP32 tiers in f32 (on the matrix cores, v_mfma_f32_16x16x4_f32, for query "
              "groups of four or more heads; on the VALU for one or two); packed tiles on the matrix cores "
              "(v_mfma_f32_16x16x32_f16, f32 accumulation) with exact f16 2-bit codes (V codes centred, 2q-3) and "
              "the f32 coefficients Q*k_scale and p*v_scale each split into an f16 high and low part (~22 "
              "significant bits); softmax in f32 with v_exp_f32")


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="llama3-8b-32k",
                    choices=sorted(CONFIGS) + sorted(ENGINE_CONFIGS) + sorted(BATCH_CONFIGS))
    ap.add_argument("--meta", default="fp32", choices=["fp32", "fp16"], help="metadata dtype of the headline number")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="bound on the CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-graph", action="store_true", help="launch layers directly instead of a HIP graph")
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--pmc-driver", action="store_true",
                    help="counter-run workload: a 256 MiB device copy (calibration), then the partials kernel of one "
                         "layer 5 times, each after a 256 MiB copy that evicts the caches; run under rocprofv3 --pmc")
    ap.add_argument("--pmc-summary", nargs="+", metavar="DIR",
                    help="print the markdown counter summary of rocprofv3 --pmc output directories")
    ap.add_argument("--trace-summary", metavar="DB",
                    help="print the markdown kernel table of a rocprofv3 --kernel-trace results database")
    args = ap.parse_args()
    if args.pmc_summary:
        pmc_summary(args.pmc_summary)
        return
    if args.trace_summary:
        trace_summary(args.trace_summary)
        return

    if args.gpus != 1:
        print(f"bench.py: the benchmark runs on one GPU; --gpus {args.gpus} is not supported "
              "(the path would shard by KV head or by sequence; no multi-GPU run is measured).", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    from tritiercache_amd import _lib as L

    lib = L.load()
    assert torch.cuda.is_available(), "bench.py needs the GPU"
    torch.cuda.set_device(0)
    if args.config in ENGINE_CONFIGS:
        engine_bench(args, torch, L, lib)
        return
    if args.config in BATCH_CONFIGS:
        batch_bench(args, torch, L, lib)
        return
    Hq, Hkv, D, ctx, layers, outl = CONFIGS[args.config]
    t0 = time.time()
    data, (nd, npk, nb) = build_layers(torch, L, Hq, Hkv, D, ctx, 1 if args.pmc_driver else layers, outl, args.seed)
    print(f"[bench] built {layers} layers ({nd} dense + {nb} blocks each) in {time.time() - t0:.1f}s", file=sys.stderr,
          flush=True)

    stream = torch.cuda.current_stream()
    sp = lambda: C.c_void_p(torch.cuda.current_stream().cuda_stream)  # noqa: E731
    fp16 = 1 if args.meta == "fp16" else 0
    tag = "16" if fp16 else "32"
    ws_bytes = int(lib.tt_fused_attention_workspace_bytes(nd, nb, Hq, Hkv, D, 16, 1))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
    ws2 = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")  # the deferred step's other workspace

    def layer_args(d, t):
        return (d["Q"].data_ptr(), d["dK"].data_ptr(), d["dV"].data_ptr(), nd, d["KP"].data_ptr(),
                d["KS" + t].data_ptr(), d["KZ" + t].data_ptr(), d["VP"].data_ptr(), d["VS" + t].data_ptr(),
                d["VZ" + t].data_ptr(), d["ids"].data_ptr(), nb, Hq, Hkv, D)

    def step_per_layer(t, f16):
        for d in data:
            L.check(lib.tt_fused_attention_decode_ws(*layer_args(d, t), d["out"].data_ptr(), d["mw"].data_ptr(), 16,
                                                     f16, ws.data_ptr(), ws_bytes, sp()), "fused")

    def step(t, f16):
        # layer i's mean weights in layer i + 1's finalize launch, the last layer's on their own
        wss = (ws, ws2)
        for i, d in enumerate(data):
            w = wss[i % 2]
            L.check(lib.tt_attention_partials(*layer_args(d, t), 16, f16, 1, w.data_ptr(), ws_bytes, sp()),
                    "partials")
            if i == 0:
                L.check(lib.tt_attention_finalize(d["Q"].data_ptr(), nd, nb, Hq, Hkv, D, d["out"].data_ptr(), None,
                                                  16, f16, 1, w.data_ptr(), ws_bytes, sp()), "merge")
            else:
                L.check(lib.tt_attention_finalize_deferred(
                    d["Q"].data_ptr(), nd, nb, Hq, Hkv, D, d["out"].data_ptr(), 16, f16, w.data_ptr(), ws_bytes,
                    nd, nb, data[i - 1]["mw"].data_ptr(), wss[(i - 1) % 2].data_ptr(), ws_bytes, sp()), "deferred")
        last = len(data) - 1
        L.check(lib.tt_attention_finalize(data[last]["Q"].data_ptr(), nd, nb, Hq, Hkv, D, None,
                                          data[last]["mw"].data_ptr(), 16, f16, 1, wss[last % 2].data_ptr(), ws_bytes,
                                          sp()), "mean")

    def time_steps(t, f16, fn=None):
        fn = fn or step
        use_graph = not args.no_graph
        g = None
        if use_graph:
            try:
                fn(t, f16)
                torch.cuda.synchronize()
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g):
                    fn(t, f16)
            except Exception as e:  # pragma: no cover
                print(f"[bench] graph capture failed ({e}); timing direct launches", file=sys.stderr)
                g = None
        run = g.replay if g is not None else (lambda: fn(t, f16))
        for _ in range(args.warmup):
            run()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(args.steps):
            run()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1000.0 / args.steps, g is not None

    def time_split_kernel(t, f16, reps):
        """Average duration of one attn_packed_kernel launch: the 32 layers' partials launches back to back
        (one HIP graph), HIP events on the launch stream around `reps` replays, after 20 untimed ones (~11 ms
        of work: replays right after the host-side checks before it ran up to 10% slower)."""
        def partials():
            for d in data:
                L.check(lib.tt_attention_partials(*layer_args(d, t), 16, f16, 1, ws.data_ptr(), ws_bytes, sp()),
                        "partials")
        run = partials
        if not args.no_graph:
            try:
                partials()
                torch.cuda.synchronize()
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g):
                    partials()
                run = g.replay
            except Exception as e:  # pragma: no cover
                print(f"[bench] graph capture of the partials failed ({e}); timing direct launches", file=sys.stderr)
        for _ in range(20):
            run()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            run()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1000.0 / (reps * len(data))

    if args.pmc_driver:
        pmc_driver(torch, lib, L, data, layer_args, tag, fp16, ws, ws_bytes, sp)
        return

    # Deferring each layer's mean weights to the next layer's finalize launch costs one extra launch per
    # step: it pays with many layers (32: ~4%), not with few (8: ~4% slower).
    deferred = layers >= DEFER_MIN_LAYERS
    main_step = step if deferred else step_per_layer
    us_step_deferred, graphed = time_steps(tag, fp16, step)
    us_step_per_layer, _ = time_steps(tag, fp16, step_per_layer)
    us_step = us_step_deferred if deferred else us_step_per_layer
    other_tag, other_fp16 = ("16", 1) if not fp16 else ("32", 0)
    us_step_other, _ = time_steps(other_tag, other_fp16, main_step)

    # The timed step against one fused call per layer: same outputs, same mean weights.
    step(tag, fp16)
    torch.cuda.synchronize()
    got = [(d["out"].clone(), d["mw"].clone()) for d in data]
    step_per_layer(tag, fp16)
    torch.cuda.synchronize()
    same_out = all(torch.equal(o, d["out"]) for (o, _), d in zip(got, data))
    mw_diff = max(float((m - d["mw"]).abs().max() / d["mw"].abs().max()) for (_, m), d in zip(got, data))
    split_us = time_split_kernel(tag, fp16, reps=max(5, min(args.steps, 20)))
    split_us_other = time_split_kernel(other_tag, other_fp16, reps=3)

    mb = 2 if fp16 else 4
    bpl = bytes_read_per_layer(Hq, Hkv, D, ctx, mb)
    bpl_other = bytes_read_per_layer(Hq, Hkv, D, ctx, 4 if fp16 else 2)
    step_gbps = bpl * layers / (us_step * 1e-6) / 1e9
    kern_gbps = bpl / (split_us * 1e-6) / 1e9

    # Parity of layer 0 and the CPU baseline: the reference's AVX2+OpenMP kernel on the host cores.
    cpu = None
    parity = None
    if not args.no_cpu:
        from oracle.binding import load_oracle, load_reference
        from oracle.exact import elementwise_ratio, exact_attention, weights_rel_err

        impl = load_reference() or load_oracle()
        d = data[0]
        h = {k: (v.cpu().numpy() if v.dtype != torch.uint16 else v.cpu().view(torch.int16).numpy().view(np.uint16))
             for k, v in d.items()}
        cargs = (h["Q"], h["dK"], h["dV"], nd, h["KP"].reshape(nb, 1, Hkv, D), h["KS" + tag], h["KZ" + tag], h["VP"],
                 h["VS" + tag], h["VZ" + tag], h["ids"], nb, Hq, Hkv, D, 16, bool(fp16))
        main_step(tag, fp16)
        torch.cuda.synchronize()
        gpu_out = data[0]["out"].cpu().numpy()  # layer 0 of the timed step
        gpu_mw = data[0]["mw"].cpu().numpy()
        phys, logical = host_cores()
        threads = int(os.environ.get("OMP_NUM_THREADS", 0) or logical) if impl.kind == "reference" else 1
        t1 = time.perf_counter()
        ro, rmw = impl.fused_attention_decode(*cargs)
        first = time.perf_counter() - t1
        n, tot = 1, first
        while tot < args.cpu_seconds and n < 200:
            t1 = time.perf_counter()
            impl.fused_attention_decode(*cargs)
            tot += time.perf_counter() - t1
            n += 1
        per_layer = tot / n
        one_thread = None
        if impl.kind == "reference" and threads > 1 and set_omp_threads(1):
            t1 = time.perf_counter()
            impl.fused_attention_decode(*cargs)
            one_thread = time.perf_counter() - t1
            set_omp_threads(threads)
        xo, xmw = exact_attention(impl, *cargs)
        parity = {
            "checked_against": impl.kind,
            "layer0_out_max_rel_err": float(np.abs(gpu_out - ro).max() / np.abs(ro).max()),
            "layer0_mean_weights_max_rel_err": float(np.abs(gpu_mw - rmw).max() / np.abs(rmw).max()),
            # elementwise: max_i |gpu_i - ref_i| / (1e-4 |ref_i| + a max|ref|), <= 1 passes
            "layer0_out_elementwise_vs_ref_a1e-5": elementwise_ratio(gpu_out, ro, atol_frac=1e-5),
            "layer0_out_elementwise_vs_exact_a1e-6": elementwise_ratio(gpu_out, xo),
            "ref_out_elementwise_vs_exact_a1e-6": elementwise_ratio(ro, xo),
            "layer0_mean_weights_max_elem_rel_err_vs_ref": weights_rel_err(gpu_mw, rmw),
            "layer0_mean_weights_max_elem_rel_err_vs_exact": weights_rel_err(gpu_mw, xmw),
            "exact": "float64 attention over the same dequantised tier values (oracle/exact.py)",
        }
        cpu = {
            "value": per_layer * layers * 1e6,
            "unit": "us/step",
            "cores": threads,
            "physical_cores_available": phys,
            "logical_cpus_available": logical,
            "one_thread_us_per_step": None if one_thread is None else one_thread * layers * 1e6,
            "kind": impl.kind,
            "sample": f"{n} calls of one layer ({nd} dense + {nb} blocks, Hq={Hq}, Hkv={Hkv}, D={D}, "
                      f"{args.meta} metadata, mean weights on) on {threads} OpenMP threads, {tot:.1f}s, scaled "
                      f"x{layers} layers; one call on 1 thread, scaled likewise",
        }

    traffic, traffic_stale = traffic_from_profile(args.config, args.meta)
    result = {
        "metric": METRIC if args.config == "llama3-8b-32k" else f"decode-attn µs/step + achieved HBM GB/s ({args.config})",
        "value": round(us_step, 2),
        "unit": "us/step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(us_step / 1000.0, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "arithmetic": ARITHMETIC,
        "data": "synthetic (seeded N(0,1) on the GPU" + {"x8": ", 4 K outlier channels per KV head x8",
                                                          "t3": ", 4 Student-t (nu=3) K outlier channels per KV head"}
        .get(outl, "") + "; packed by the library quantisers)",
        "config": {
            "workload": f"{args.config}: decode attention over {layers} layers, batch 1, ctx {ctx}, "
                        f"{Hq} q heads / {Hkv} KV heads, head_dim {D}, 4 sinks + 256 recent + "
                        f"{nd - 260} heavy hitters FP32, {npk} tokens 2-bit packed in {nb} blocks, "
                        f"{args.meta} metadata, mean attention weights computed",
            "layers": layers, "ctx": ctx, "num_q_heads": Hq, "num_kv_heads": Hkv, "head_dim": D,
            "dense_tokens": nd, "packed_tokens": npk, "blocks": nb, "meta": args.meta, "hip_graph": graphed,
            "seed": args.seed,
            "finalize": ("per layer: partials, then one launch merging this layer and computing the previous "
                         "layer's mean weights; the last layer's mean weights in a launch of their own")
            if deferred else "per layer: one fused call (partials, then merge and mean weights in one launch)",
        },
        "us_per_step_per_layer_calls": round(us_step_per_layer, 2),
        "us_per_step_deferred_mean_weights": round(us_step_deferred, 2),
        "per_layer_calls_match": {"outputs_bit_identical": bool(same_out),
                                  "mean_weights_max_rel_diff": mw_diff},
        "achieved_GBps": round(step_gbps, 1),
        "pct_of_hbm_peak": round(100.0 * step_gbps / HBM_PEAK_GBPS, 2),
        "bytes_read_per_step": bpl * layers,
        "roofline": {
            "bound": "hbm",
            "kernel": dominant_kernel(D, Hkv),
            "achieved": round(kern_gbps, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(kern_gbps / HBM_PEAK_GBPS, 4),
            "traffic": traffic,
            "traffic_stale": traffic_stale,
            "bytes_per_launch": bpl,
            "avg_launch_us": round(split_us, 3),
        },
        "other_meta": {
            "meta": "fp16" if not fp16 else "fp32",
            "us_per_step": round(us_step_other, 2),
            "achieved_GBps": round(bpl_other * layers / (us_step_other * 1e-6) / 1e9, 1),
            "split_kernel_GBps": round(bpl_other / (split_us_other * 1e-6) / 1e9, 1),
        },
        "cpu_baseline": cpu,
        "parity": parity,
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
