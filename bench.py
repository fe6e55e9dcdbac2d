#!/usr/bin/env python3
"""Packed decode-attention benchmark on one MI355X (BASELINE.json metric).

Default workload: the headline 7B GQA shape -- 28 layers,
batch 16, 28 q / 4 kv heads, head_dim 128, 256 packed pages (32768 tokens) +
100 residual tokens + the new token per sequence, target_bit 2.5 (Key 3.0
bits).  One *step* is one decode step of the attention path over all 28
layers (distinct per-layer buffers, far larger than the 256 MB Infinity
Cache); ``value`` is microseconds per layer-step.  Synthetic seeded data
(logitfill_amd.synth), resident in HBM before timing starts.

Prints one JSON line (the driver's contract) with ``roofline`` (dominant
kernel: the fused decode kernel) and ``cpu_baseline`` (the CPU oracle's dense
dequantise-then-attend path on a bounded sample, rank 0 only).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0


def parse_args():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--config", default="c2", choices=["c1", "c2", "c2_k4", "c4"])
    p.add_argument("--layers", type=int, default=None)
    p.add_argument("--kernel", default="auto", choices=["auto", "valu", "mfma"])
    p.add_argument("--pages-per-split", type=int, default=None)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-dense", action="store_true", help="skip the BF16 dense comparator")
    p.add_argument("--no-compress", action="store_true", help="skip the page-compress (config 3) timing")
    p.add_argument("--cpu-seqs", type=int, default=16,
                   help="sequences timed by the CPU baseline (default: the whole c2 batch, about 20 s of CPU work)")
    p.add_argument("--no-extra", action="store_true",
                   help="skip the other decode configs (c2 at target 3.0, c1, c4) reported beside the headline")
    p.add_argument("--no-step", action="store_true", help="skip the full decode-step timing (attention + commit)")
    p.add_argument("--compress-only", action="store_true",
                   help="only time the config-3 page compress (one JSON line; for profiling runs)")
    p.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES",
                   help="only run a plain device-to-device copy of BYTES (3 times) and exit: the reference "
                        "kernel that scales the PMC byte counters (FETCH_SIZE / WRITE_SIZE)")
    return p.parse_args()


PMC_SUMMARY = ROOT / "profiles" / "decode_mfma_c2_pmc.txt"


def measured_traffic(config: str):
    """HBM bytes per decode-kernel dispatch from the committed PMC summary (FETCH_SIZE and
    WRITE_SIZE per dispatch, each scaled by the same counter's reading for a copy of known
    size), or None when there is no summary for this workload."""
    if config != "c2" or not PMC_SUMMARY.exists():
        return None
    vals = {}
    for line in PMC_SUMMARY.read_text().splitlines():
        if ":" in line and not line.lstrip().startswith("#"):
            k, v = line.split(":", 1)
            vals[k.strip()] = v.strip()
    try:
        return int(float(vals["traffic_bytes_per_dispatch"]))
    except (KeyError, ValueError):
        return None


def copy_calibration(nbytes: int) -> None:
    import torch

    n = nbytes // 4
    src = torch.randn(n, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": n * 4, "launches": 3}), flush=True)


def algorithmic_bytes(widths, words, n_kv, n_q, D, H, R1, k_group=128, v_group=128):
    """Bytes one decode step of one sequence and layer must read/write (packed path).

    K codes 4*(w2+w4+w8) + fp16 tier 2*width16 + V codes 4*D/16 + V scale/min
    4*D/v_group per token and kv head; K scale/min 4 per (int-tier slot, Key
    group); bf16 residual K+V 4*D per token (R1 = residual + new token); bf16 q
    and output 4*D per q head.  Returns (total, payload) where payload counts
    the K codes, the fp16 tier and the V codes only.
    """
    per_tok = 4 * sum(words) + 2 * widths[3] + 4 * D // 16 + 4 * (D // v_group)
    payload_tok = 4 * sum(words) + 2 * widths[3] + 4 * D // 16
    kscale = 4 * sum(widths[:3]) * (H // k_group)
    total = n_kv * H * per_tok + n_kv * kscale + 4 * n_kv * R1 * D + 4 * n_q * D
    return total, n_kv * H * payload_tok


def build_state(cfg, layers, dev, capacity_pages=None, q_len=1):
    """Manager with ``layers`` seeded layers of config ``cfg`` and each layer's decode inputs:
    (query, key_new, value_new) of one new token ``[B, n_q, D]`` / ``[B, n_kv, D]``, or with
    ``q_len`` > 1 new tokens ``[B, n_q, q_len, D]`` / ``[B, n_kv, q_len, D]``."""
    import torch

    from logitfill_amd import synth
    from logitfill_amd.packed import PackedKVManager

    B, n_q, n_kv, D = cfg["batch"], cfg["n_q"], cfg["n_kv"], cfg["head_dim"]
    pages, resid, tb = seq_lengths(cfg)
    levels = [synth.sample_tier_levels(n_kv, D, tb, seed=layer) for layer in range(layers)]
    mgr = PackedKVManager(levels, n_q, n_kv, D, 128, 128, 128, 2, dev, batch_size=B,
                          capacity_tokens=(capacity_pages or max(pages)) * 128)
    inputs = []
    T = max(pages) * 128 + 128  # every sequence's residual slice below is 127 tokens long
    for layer in range(layers):
        d = synth.make_layer(B, n_q, n_kv, D, T, tb, seed=layer, device=dev)
        st = mgr.layers[layer]
        st.fill_pages(d.key, d.value, pages)
        if max(resid):
            # sequence b's residual: its tokens right after its pages
            rk = torch.stack([d.key[b, :, pages[b] * 128:pages[b] * 128 + 127] for b in range(B)])
            rv = torch.stack([d.value[b, :, pages[b] * 128:pages[b] * 128 + 127] for b in range(B)])
            st.set_tail(rk, rv, resid)
            del rk, rv
        if q_len == 1:
            inputs.append((d.query.contiguous(), d.key_new.contiguous(), d.value_new.contiguous()))
        else:
            g = torch.Generator(device=dev).manual_seed(9000 + layer)
            q = (torch.randn(B, n_q, q_len, D, generator=g, device=dev) * D ** -0.5).to(torch.bfloat16)
            kn = torch.randn(B, n_kv, q_len, D, generator=g, device=dev).to(torch.bfloat16)
            vn = torch.randn(B, n_kv, q_len, D, generator=g, device=dev).to(torch.bfloat16)
            inputs.append((q, kn, vn))
        del d
        torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return mgr, inputs


def context_text(cfg) -> str:
    if cfg["pages"] is None:
        return "ragged contexts U[4K, 64K] (full pages + residual 1-127, seeded)"
    return f"{cfg['pages']} pages + {cfg['residual']} residual"


def seq_lengths(cfg):
    """Per-sequence (full pages, residual tokens) and the target bit of a config; c4's contexts
    are ragged (uniform in [4K, 64K], seeded)."""
    from logitfill_amd import synth

    B = cfg["batch"]
    if cfg["pages"] is None:
        pages, resid = synth.ragged_lengths(B, seed=4)
    else:
        pages, resid = [cfg["pages"]] * B, [cfg["residual"]] * B
    return pages, resid, cfg["target_bit"]


def time_decode(mgr, inputs, steps, warmup, kernel, pages_per_split):
    import torch

    from logitfill_amd.packed.reference import decode_into

    dev = mgr.device
    outs = [torch.empty_like(q) for q, _, _ in inputs]
    scaling = mgr.head_dim ** -0.5

    def one_step():
        for layer, (q, kn, vn) in enumerate(inputs):
            decode_into(mgr, layer, q, kn, vn, scaling, outs[layer], kernel=kernel, pages_per_split=pages_per_split)

    for _ in range(warmup):
        one_step()
    torch.cuda.synchronize(dev)
    stream = torch.cuda.current_stream(dev)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(steps):
        one_step()
    end.record(stream)
    torch.cuda.synchronize(dev)
    wall = time.perf_counter() - t0
    ms = start.elapsed_time(end)
    return ms / steps, wall / steps * 1e3


def decode_point(cfg, layers, steps, warmup, kernel, pages_per_split, dev, q_len=1):
    """Build ``layers`` layers of a config, time the decode (``q_len`` new tokens per sequence);
    returns (us per layer-step, bytes per layer-step, payload bytes per layer-step, wall ms per
    step) and frees the state."""
    import torch

    mgr, inputs = build_state(cfg, layers, dev, q_len=q_len)
    ms_step, wall_ms = time_decode(mgr, inputs, steps, warmup, kernel, pages_per_split)
    split = plan_text(mgr.layers[0].decode_plan)
    n_q, n_kv, D = cfg["n_q"], cfg["n_kv"], cfg["head_dim"]
    pages, resid, _ = seq_lengths(cfg)
    tot, pay = 0, 0
    for st in mgr.layers:
        for p, r in zip(pages, resid):
            t, pl = algorithmic_bytes(st.widths, st.words, n_kv, n_q * q_len, D, p * 128, r + q_len)
            tot += t
            pay += pl
    del mgr, inputs
    torch.cuda.empty_cache()
    return ms_step * 1e3 / layers, tot / layers, pay / layers, wall_ms, split


def plan_text(plan) -> str:
    """The decode plan the planner chose, in words (reported beside the timing)."""
    pps = plan.pages_per_split
    if isinstance(pps, tuple) and pps and pps[0] == "paired":
        how = (f"paired: the first-dispatched workgroups take {pps[1]}-page items, the rest shares the CUs"
               if pps[2] == 0 else
               f"paired small batch: {pps[1]}-page first items, then {pps[2]}-page items and residual-only items")
    elif isinstance(pps, tuple):
        how = f"two-size dispatch-order split: {max(pps)} and {min(pps)} pages per item"
    else:
        how = f"{pps} pages per item"
    return f"{how}; {plan.n_work} items"


def time_real_step(cfg, layers, steps, dev, fused=False):
    """A full decode step through the drop-in API, as a model's attention layers drive it
    (reference qwen2_attention.py:234-255): for every layer ``packed_attention`` over the packed
    history, the residual page and the new token, then ``commit`` of the new token; after the
    last layer ``flush_pending`` packs every layer's completed page in one launch (the manager
    defers flushes).  The residual starts ``steps // 2`` tokens short of a full page, so the
    timed steps cross one page boundary (a flush and a new decode plan).  Returns (GPU us per
    step from HIP events on the stream, host wall us per step, enqueue-only host us per step,
    steps, pages flushed per layer).  ``fused``: ``packed_attention(..., commit=True)``, the
    commit folded into the decode launch while no page fills (as ``logitfill_amd.qwen2`` runs
    the model's layers)."""
    import torch

    from logitfill_amd.packed.reference import packed_attention

    B = cfg["batch"]
    pages, _, _ = seq_lengths(cfg)
    resid = [128 - steps // 2] * B
    c = dict(cfg, residual=resid[0])
    mgr, inputs = build_state(c, layers, dev, capacity_pages=max(pages) + 2)
    mgr.defer_flush = True
    scaling = mgr.head_dim ** -0.5
    ins = [(q[:, :, None], kn[:, :, None], vn[:, :, None]) for q, kn, vn in inputs]

    def one_step():
        for layer, (q, kn, vn) in enumerate(ins):
            if fused:
                packed_attention(mgr, layer, q, kn, vn, scaling, commit=True)
            else:
                packed_attention(mgr, layer, q, kn, vn, scaling)
                mgr.commit(layer, kn, vn)
        mgr.flush_pending()

    one_step()  # warm-up: plans, workspace, pinned staging buffers
    torch.cuda.synchronize(dev)
    hist0 = mgr.layers[0].hist_len
    stream = torch.cuda.current_stream(dev)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(steps - 1):
        one_step()
    end.record(stream)
    t_enq = time.perf_counter() - t0
    torch.cuda.synchronize(dev)
    wall = time.perf_counter() - t0
    flushed = (mgr.layers[0].hist_len - hist0) // 128
    n = steps - 1
    del mgr, inputs, ins
    torch.cuda.empty_cache()
    return start.elapsed_time(end) * 1e3 / n, wall * 1e6 / n, t_enq * 1e6 / n, n, flushed


def time_graph_step(cfg, layers, replays, dev, fused=False):
    """The same decode step (every layer's packed_attention, then the one-token commit, which
    appends on the device) captured once in a HIP graph and replayed ``replays`` times, as a
    serving loop launches it; the residual starts at 20 tokens so no replay fills a page.
    Returns GPU us per step (HIP events around the replays)."""
    import torch

    from logitfill_amd.packed.reference import packed_attention

    c = dict(cfg, residual=20)
    mgr, inputs = build_state(c, layers, dev)
    scaling = mgr.head_dim ** -0.5
    ins = [(q[:, :, None], kn[:, :, None], vn[:, :, None]) for q, kn, vn in inputs]

    def one_step():
        for layer, (q, kn, vn) in enumerate(ins):
            if fused:
                packed_attention(mgr, layer, q, kn, vn, scaling, commit=True)
            else:
                packed_attention(mgr, layer, q, kn, vn, scaling)
                mgr.commit(layer, kn, vn)

    one_step()
    torch.cuda.synchronize(dev)
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            one_step()
    torch.cuda.current_stream(dev).wait_stream(side)
    graph.replay()
    torch.cuda.synchronize(dev)
    stream = torch.cuda.current_stream(dev)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(replays):
        graph.replay()
    end.record(stream)
    torch.cuda.synchronize(dev)
    del graph, mgr, inputs, ins
    torch.cuda.empty_cache()
    return start.elapsed_time(end) * 1e3 / replays


def time_dense(cfg, steps, warmup):
    """The BF16 dense comparator (lf_dense_decode) at the same shape: one layer's K/V cache of
    all history + residual + new tokens, two layers alternated so no call reads a cache the
    previous call left in the L2/MALL.  Returns (us per layer-step, bytes per layer-step)."""
    import torch

    from logitfill_amd.packed.dense import dense_decode

    B, n_q, n_kv, D = cfg["batch"], cfg["n_q"], cfg["n_kv"], cfg["head_dim"]
    T = cfg["pages"] * 128 + cfg["residual"] + 1
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev).manual_seed(5)
    caches = []
    for _ in range(2):
        k = torch.randn(B, n_kv, T, D, device=dev, dtype=torch.bfloat16, generator=gen)
        v = torch.randn(B, n_kv, T, D, device=dev, dtype=torch.bfloat16, generator=gen)
        q = (torch.randn(B, n_q, D, device=dev, generator=gen) * D ** -0.5).to(torch.bfloat16)
        caches.append((q, k, v))
    out = torch.empty(B, n_q, D, device=dev, dtype=torch.bfloat16)
    ws = torch.empty(64 << 20, dtype=torch.uint8, device=dev)
    for i in range(warmup):
        q, k, v = caches[i & 1]
        dense_decode(q, k, v, D ** -0.5, out=out, workspace=ws)
    torch.cuda.synchronize(dev)
    stream = torch.cuda.current_stream(dev)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for i in range(steps):
        q, k, v = caches[i & 1]
        dense_decode(q, k, v, D ** -0.5, out=out, workspace=ws)
    end.record(stream)
    torch.cuda.synchronize(dev)
    us = start.elapsed_time(end) * 1e3 / steps
    nbytes = B * n_kv * T * D * 2 * 2 + 2 * B * n_q * D * 2
    del caches, ws
    torch.cuda.empty_cache()
    return us, nbytes


def time_compress(target_bit, steps, warmup):
    """page compress of 64 sequences x 1 page x 4 kv heads x 28 layers at the
    7B shape (one lf_pack_pages launch per layer, all 64 pages of the layer).  Returns
    (us per pass over the 28 layers, page-heads per pass, bytes read, bytes written)."""
    import torch

    from logitfill_amd import _native, synth
    from logitfill_amd.packed import PackedKVManager

    B, n_q, n_kv, D, L = 64, 28, 4, 128, 28
    dev = torch.device("cuda", 0)
    levels = [synth.sample_tier_levels(n_kv, D, target_bit, seed=layer) for layer in range(L)]
    mgr = PackedKVManager(levels, n_q, n_kv, D, 128, 128, 128, 2, dev, batch_size=B, capacity_tokens=128)
    srcs = []
    for layer in range(L):
        d = synth.make_layer(B, n_q, n_kv, D, 128, target_bit, seed=layer, device=dev)
        srcs.append((d.key.contiguous(), d.value.contiguous()))
        mgr.layers[layer].reserve(128)
    jobs = torch.tensor([(b, 0, 0) for b in range(B)], dtype=torch.int32, device=dev)
    structs = [mgr.layers[layer].layer_struct() for layer in range(L)]
    lib = _native.load()
    stream = torch.cuda.current_stream(dev)

    def per_layer_pass():
        for layer in range(L):
            k, v = srcs[layer]
            st = lib.lf_pack_pages(structs[layer], k.data_ptr(), v.data_ptr(), _native.LF_BF16, k.stride(0),
                                   k.stride(1), k.stride(2), jobs.data_ptr(), B, stream.cuda_stream)
            _native.check(st, "lf_pack_pages")

    # one launch for the step: every layer's pages (what a deferring manager's flush_pending does)
    host_structs = (_native.PackedLayer * L)(*structs)
    host_srcs = (_native.PackSource * L)(*[_native.PackSource(k.data_ptr(), v.data_ptr(), k.stride(0), k.stride(1),
                                                              k.stride(2)) for k, v in srcs])
    dev_structs = torch.frombuffer(bytearray(host_structs), dtype=torch.uint8).to(dev)
    dev_srcs = torch.frombuffer(bytearray(host_srcs), dtype=torch.uint8).to(dev)
    mjobs = torch.tensor([(layer, b, 0, 0) for layer in range(L) for b in range(B)], dtype=torch.int32, device=dev)

    def multi_pass():
        st = lib.lf_pack_pages_multi(dev_structs.data_ptr(), host_structs, dev_srcs.data_ptr(), host_srcs, L,
                                     _native.LF_BF16, mjobs.data_ptr(), L * B, stream.cuda_stream)
        _native.check(st, "lf_pack_pages_multi")

    def timed(fn):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize(dev)
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(steps):
            fn()
        end.record(stream)
        torch.cuda.synchronize(dev)
        return start.elapsed_time(end) * 1e3 / steps

    us_layer = timed(per_layer_pass)
    us = timed(multi_pass)
    page_heads = B * n_kv * L
    read = page_heads * 128 * D * 2 * 2
    written = 0
    for st in mgr.layers:
        w, words = st.widths, st.words
        per_head = (128 * 4 * sum(words) + 128 * 2 * w[3] + 4 * (w[0] + w[1] + w[2])   # K codes, fp16, scale+min
                    + 128 * 4 * (D // 16) + 128 * 4 * (D // 128))                      # V codes, scale+min
        written += B * n_kv * per_head
    del srcs, mgr, dev_structs, dev_srcs, mjobs
    torch.cuda.empty_cache()
    return us, us_layer, page_heads, read, written


def host_cpu():
    """(threads for the CPU baseline, logical CPUs of the host, CPU model).  The threads are
    the CPUs this process may run on, capped by OMP_NUM_THREADS when the environment sets it
    (the GPU box gives each job a share of its cores that way)."""
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count() or 1
    cap = os.environ.get("OMP_NUM_THREADS")
    threads = max(1, min(avail, int(cap))) if cap and cap.isdigit() else max(1, avail)
    model = "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return threads, os.cpu_count() or 1, model


def cpu_baseline(cfg, n_seqs):
    """The oracle's dense path (dequantise whole history, concatenate, repeat_kv, fp32
    softmax attention) on one layer for ``n_seqs`` sequences, scaled to the batch."""
    import numpy as np
    from threadpoolctl import threadpool_limits

    from logitfill_amd import synth
    from oracle import attention as oatt
    from oracle import history as ohist

    B, n_q, n_kv, D = cfg["batch"], cfg["n_q"], cfg["n_kv"], cfg["head_dim"]
    pages_b, resid_b, tb = seq_lengths(cfg)
    pages, resid = pages_b[0], resid_b[0]
    threads, host_cpus, model = host_cpu()
    times = []
    t_leg = time.perf_counter()
    with threadpool_limits(limits=threads):
        for s in range(n_seqs):
            d = synth.make_layer(1, n_q, n_kv, D, pages * 128 + resid, tb, seed=1000 + s)
            key = d.key[0].float().numpy()
            value = d.value[0].float().numpy()
            store = ohist.pack_history(d.levels, key, value)
            q = d.query[0].float().numpy()[:, None]
            kn = d.key_new[0].float().numpy()[:, None]
            vn = d.value_new[0].float().numpy()[:, None]
            oatt.reference_attention(store, q, kn, vn, D ** -0.5, n_q, n_kv)      # warm-up
            runs = []
            for _ in range(3):
                t0 = time.perf_counter()
                oatt.reference_attention(store, q, kn, vn, D ** -0.5, n_q, n_kv, out_dtype="bf16")
                runs.append(time.perf_counter() - t0)
            times.append(float(np.median(runs)))
    per_seq = float(np.mean(times))
    return {"value": round(per_seq * B * 1e6, 1), "unit": "us/step/layer", "cores": threads, "kind": "port",
            "host_cpus": host_cpus, "cpu_model": model, "wall_s": round(time.perf_counter() - t_leg, 1),
            "per_run_s": round(per_seq, 4),
            "sample": f"1 layer x {n_seqs} of {B} sequences at the full shape ({pages} pages + {resid} "
                      f"residual + 1), median of 3 after 1 warm-up, scaled x{B // n_seqs if n_seqs else 0} "
                      f"to the batch; numpy float32 with {threads} BLAS threads"}


def cpu_baseline_compress(target_bit, n_pages=16):
    """The oracle's page packer (quantize_key_page + quantize_value_page, reference
    layout.py:71-129) on ``n_pages`` config-3 page-heads of 4 kv heads (one layer's page for
    n_pages / 4 sequences), median of 3 after 1 warm-up.  Returns page-heads per second."""
    import numpy as np
    from threadpoolctl import threadpool_limits

    from logitfill_amd import synth
    from oracle import layout as ol

    threads, host_cpus, model = host_cpu()
    t_leg = time.perf_counter()
    seqs = max(1, n_pages // 4)
    d = synth.make_layer(seqs, 28, 4, 128, 128, target_bit, seed=0)
    table = ol.layer_table(d.levels)
    pages_k = [d.key[b].float().numpy() for b in range(seqs)]
    pages_v = [d.value[b].float().numpy() for b in range(seqs)]

    def run():
        for k, v in zip(pages_k, pages_v):
            ol.quantize_key_page(k, table, 128)
            ol.quantize_value_page(v, 2, 128)

    with threadpool_limits(limits=threads):
        run()
        runs = []
        for _ in range(3):
            t0 = time.perf_counter()
            run()
            runs.append(time.perf_counter() - t0)
    per_pass = float(np.median(runs))
    page_heads = 4 * seqs
    return {"value": round(page_heads / per_pass, 1), "unit": "page-heads/s", "cores": threads, "kind": "port",
            "host_cpus": host_cpus, "cpu_model": model, "wall_s": round(time.perf_counter() - t_leg, 1),
            "sample": f"{page_heads} page-heads (4 kv heads x {seqs} sequences, one 128-token page each, "
                      f"target_bit {target_bit}), median of 3 after 1 warm-up; numpy float32"}


def compress_record(steps=10, warmup=2):
    comp = {}
    for tb in (2.5, 3.0, 4.0):
        us_c, us_c_layer, ph, rd, wr = time_compress(tb, steps, warmup)
        comp[f"target_{tb}"] = {"us_per_pass": round(us_c, 1), "page_heads": ph,
                                "pages_per_s": round(ph / us_c * 1e6), "gbs": round((rd + wr) / us_c / 1e3, 1),
                                "hbm_frac": round((rd + wr) / us_c / 1e3 / HBM_PEAK_GBS, 4),
                                "bytes_read": rd, "bytes_written": wr,
                                "us_per_pass_one_launch_per_layer": round(us_c_layer, 1)}
    return {"what": "BASELINE config 3: 64 sequences x 1 page x 4 kv heads x 28 layers, bf16 K/V from the "
                    "config-0 distributions; us_per_pass = one lf_pack_pages_multi launch for the 28 layers (a "
                    "deferring manager's end-of-step flush), us_per_pass_one_launch_per_layer = 28 lf_pack_pages "
                    "launches; pages_per_s counts page-heads; GB/s = bf16 pages read + packed bytes written",
            **comp}


ARITHMETIC = ("bf16 query/residual/output; packed int2/int4/int8 codes and fp16 tier values from HBM; "
              "scores and probability x Value products on the matrix cores with fp16 hi+lo operands; "
              "fp32 accumulation and softmax")


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); this build runs the path on one GPU "
              "(its multi-GPU sharding is a design note)", file=sys.stderr)
        sys.exit(2)
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return
    import torch

    from logitfill_amd import _native, synth

    legs = {}
    if args.compress_only:
        t0 = time.perf_counter()
        rec = compress_record(args.steps, args.warmup)
        legs["compress"] = round(time.perf_counter() - t0, 2)
        print(json.dumps({"compress_c3": rec, "leg_wall_s": legs}), flush=True)
        return
    cfg = dict(synth.CONFIGS[args.config])
    layers = args.layers or cfg["layers"]
    dev = torch.device("cuda", 0)
    kernel = {"auto": _native.KERNEL_AUTO, "valu": _native.KERNEL_VALU, "mfma": _native.KERNEL_MFMA}[args.kernel]
    print(f"[bench] building {layers} layers of {args.config} and timing ...", file=sys.stderr, flush=True)
    t0 = time.perf_counter()
    us_layer, bytes_launch, pay_launch, wall_ms, split = decode_point(cfg, layers, args.steps, args.warmup, kernel,
                                                               args.pages_per_split, dev)
    legs["decode"] = round(time.perf_counter() - t0, 2)
    ms_step = us_layer * layers / 1e3
    B, n_q, n_kv, D = cfg["batch"], cfg["n_q"], cfg["n_kv"], cfg["head_dim"]
    pay_bytes = pay_launch * layers
    launch_s = us_layer / 1e6
    achieved = bytes_launch / launch_s / 1e9
    result = {
        "metric": "packed decode-attn us/step + achieved HBM GB/s (% of peak), 7B GQA shape @32K ctx",
        "value": round(us_layer, 2),
        "unit": "us/step/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "arithmetic": ARITHMETIC,
        "data": "synthetic (seeded logitfill_amd.synth: K~N(0,1)*LogNormal channel scale + outliers, V,Q~N)",
        "config": {"workload": f"{args.config}: packed decode attention, {layers} layers x batch {B}, "
                               f"{n_q}q/{n_kv}kv heads, D {D}, {context_text(cfg)}, target_bit {cfg['target_bit']}",
                   "kernel": args.kernel, "layers": layers, "batch": B, "split": split},
        "hbm_gbs": round(achieved, 1),
        "hbm_frac": round(achieved / HBM_PEAK_GBS, 4),
        "payload_gbs": round(pay_bytes / layers / launch_s / 1e9, 1),
        "bytes_per_layer_step": int(bytes_launch),
        "wall_ms_per_step": round(wall_ms, 4),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(args.config) if args.layers in (None, cfg["layers"]) else None,
                     "timed": "HIP events on the launch stream around every layer's decode kernel + split "
                              "merge; achieved = algorithmic bytes per layer-step / that time"},
    }
    if not args.no_dense and cfg["pages"] is not None:
        print("[bench] bf16 dense comparator ...", file=sys.stderr, flush=True)
        t0 = time.perf_counter()
        dense_us, dense_bytes = time_dense(cfg, max(args.steps, 10), args.warmup)
        legs["dense"] = round(time.perf_counter() - t0, 2)
        result["dense_bf16"] = {
            "what": "lf_dense_decode: BF16 dense split-K MFMA decode over the uncompressed K/V cache of the "
                    "same shape (history + residual + new token), synthetic bf16 data",
            "us_per_layer": round(dense_us, 2),
            "hbm_gbs": round(dense_bytes / dense_us / 1e3, 1),
            "bytes_per_layer_step": int(dense_bytes),
            "floor_us_at_peak": round(dense_bytes / HBM_PEAK_GBS / 1e3, 2),
            "speedup_packed_vs_dense": round(dense_us / us_layer, 3),
            "speedup_packed_vs_dense_floor": round(dense_bytes / HBM_PEAK_GBS / 1e3 / us_layer, 3),
        }
    if not args.no_compress:
        print("[bench] page compress (config 3) ...", file=sys.stderr, flush=True)
        t0 = time.perf_counter()
        result["compress_c3"] = compress_record()
        legs["compress"] = round(time.perf_counter() - t0, 2)
    if not args.no_extra and args.config == "c2" and args.layers is None:
        extra = {}
        for name, n_layers, q_len in (("c2_k4", None, 1), ("c1", None, 1), ("c4", 8, 1), ("c2_q4", None, 4)):
            c = dict(synth.CONFIGS[name.replace("_q4", "")])
            nl = n_layers or c["layers"]
            print(f"[bench] {name} ({nl} layers) ...", file=sys.stderr, flush=True)
            t0 = time.perf_counter()
            us_x, bytes_x, pay_x, _, split_x = decode_point(c, nl, 10, 2, kernel, None, dev, q_len=q_len)
            legs[name] = round(time.perf_counter() - t0, 2)
            tokens = (f", {q_len} new query tokens per sequence (speculative decoding: the right-aligned causal "
                      f"mask on the new tokens, {c['n_q'] // c['n_kv'] * q_len} query rows per kv head)"
                      if q_len > 1 else "")
            extra[name] = {"workload": f"{c['layers']}-layer model shape timed on {nl} distinct layers, batch "
                                       f"{c['batch']}, {c['n_q']}q/{c['n_kv']}kv heads, {context_text(c)}, "
                                       f"target_bit {c['target_bit']}{tokens}",
                           "us_per_layer_step": round(us_x, 2), "bytes_per_layer_step": int(bytes_x),
                           "hbm_gbs": round(bytes_x / us_x / 1e3, 1),
                           "hbm_frac": round(bytes_x / us_x / 1e3 / HBM_PEAK_GBS, 4),
                           "payload_gbs": round(pay_x / us_x / 1e3, 1), "split": split_x}
        result["other_configs"] = extra
    if not args.no_step and args.layers is None:
        for name in (args.config, "c1") if args.config != "c1" else (args.config,):
            c = dict(synth.CONFIGS[name])
            print(f"[bench] real decode step ({name}) ...", file=sys.stderr, flush=True)
            t0 = time.perf_counter()
            gpu_us, wall_us, enq_us, n, flushed = time_real_step(c, c["layers"], 40, dev)
            legs[f"step_{name}"] = round(time.perf_counter() - t0, 2)
            result.setdefault("decode_step", {})[name] = {
                "what": f"{c['layers']} layers x (packed_attention + commit) + flush_pending per step, batch "
                        f"{c['batch']}, {c['n_q']}q/{c['n_kv']}kv, {c['pages']} pages + a residual that fills a page "
                        "mid-run (deferred flush: one lf_pack_pages_multi launch for all layers), drop-in API",
                "us_per_step": round(gpu_us, 1), "us_per_layer": round(gpu_us / c["layers"], 2),
                "host_wall_us_per_step": round(wall_us, 1), "host_enqueue_us_per_step": round(enq_us, 1),
                "steps": n, "pages_flushed_per_layer": flushed}
            t0 = time.perf_counter()
            g_us = time_graph_step(c, c["layers"], 60, dev)
            legs[f"graph_step_{name}"] = round(time.perf_counter() - t0, 2)
            result["decode_step"][name]["graph_us_per_step"] = round(g_us, 1)
            result["decode_step"][name]["graph_us_per_layer"] = round(g_us / c["layers"], 2)
            # the same step with the commit folded into the decode launch (logitfill_amd.qwen2)
            t0 = time.perf_counter()
            f_us, f_wall, f_enq, _, f_flushed = time_real_step(c, c["layers"], 40, dev, fused=True)
            fg_us = time_graph_step(c, c["layers"], 60, dev, fused=True)
            legs[f"fused_step_{name}"] = round(time.perf_counter() - t0, 2)
            result["decode_step"][name]["fused_commit"] = {
                "what": "packed_attention(..., commit=True): the one-token commit appended inside the decode "
                        "launch while no residual page fills (the page-filling step commits as before)",
                "us_per_layer": round(f_us / c["layers"], 2), "host_enqueue_us_per_step": round(f_enq, 1),
                "graph_us_per_layer": round(fg_us / c["layers"], 2), "pages_flushed_per_layer": f_flushed}
    if not args.no_cpu_baseline:
        print("[bench] cpu baseline ...", file=sys.stderr, flush=True)
        t0 = time.perf_counter()
        result["cpu_baseline"] = cpu_baseline(cfg, max(1, min(args.cpu_seqs, cfg["batch"])))
        legs["cpu_baseline"] = round(time.perf_counter() - t0, 2)
        if not args.no_compress:
            t0 = time.perf_counter()
            result["cpu_baseline_compress"] = cpu_baseline_compress(2.5)
            legs["cpu_baseline_compress"] = round(time.perf_counter() - t0, 2)
    result["leg_wall_s"] = legs
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
