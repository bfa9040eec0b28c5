"""Benchmark of the MI355X-native quantized linear-layer hot path (one JSON line on stdout).

Workload: the Q4_K decode GEMV at the Llama-3-8B layer shapes, batch 1 — one step is one
decoder layer's linear products: QKV 4096->6144, O 4096->4096, gate and up 4096->14336 each, down 14336->4096. Gate
and up share their input, so their weights are stored as one [2 * 14336][row] tensor and run as one launch (the same
bytes and outputs as two launches; the layout a loader chooses when it reads the two GGUF tensors).
Weights are N(0, 0.02) from SplitMix64/Box-Muller (seed 0) quantized to Q4_K super-blocks; x is N(0, 1) (seed 1).
Inputs are resident in HBM; the activations are quantized once before the timed region (the quant_act launch is timed
separately and reported beside). Weight copies rotate over more than 2x the 256 MB Infinity Cache so every call
streams its weights from HBM.

value = algorithmic bytes (weights + 4*K fp32 x + 4*N fp32 y per GEMV) per step / seconds per step, in GB/s.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
MALL_BYTES = 256 << 20
LAYER = [("qkv", 4096, 6144), ("o", 4096, 4096), ("gate_up", 4096, 2 * 14336), ("down", 14336, 4096)]
METRIC = "Q4_K GEMV GB/s (% of HBM peak) + int8 GEMM TOPS, 1×MI355X"


def gemv_bytes(ty, n, n_out, rows=1):
    import kungfu_amd as kf

    return kf.row_bytes(ty, n) * n_out + 4 * n * rows + 4 * n_out * rows


def make_weights(ty, n, n_out, seed=0):
    import kungfu_amd as kf

    return kf.quantize(ty, kf.synth_normal(seed, 0.02, n * n_out).reshape(n_out, n))


class Shape:
    """One GEMV shape with its rotating device weight copies and resident quantized activations."""

    def __init__(self, name, ty, n, n_out, copies, dev):
        import torch

        import kungfu_amd as kf

        self.name, self.ty, self.n, self.n_out = name, ty, n, n_out
        self.host_w = make_weights(ty, n, n_out, seed=0)
        self.host_x = kf.synth_normal(1, 1.0, n).reshape(1, n)
        w = torch.from_numpy(self.host_w).to(dev)
        self.w = [w] + [w.clone() for _ in range(copies - 1)]
        self.x = torch.from_numpy(self.host_x).to(dev)
        self.act = kf.alloc_act(1, n, dev)
        self.y = torch.empty((1, n_out), device=dev)
        kf.quant_act(self.x, self.act, kf.act_kind(ty))
        self.bytes = gemv_bytes(ty, n, n_out)

    def gemv(self, i):
        import kungfu_amd as kf

        kf.gemv(self.ty, self.w[i % len(self.w)], self.act, self.y, 1, self.n, self.n_out)

    def matmul(self, i):
        import kungfu_amd as kf

        kf.matmul(self.ty, self.w[i % len(self.w)], self.x, self.act, self.y, self.n_out)


def capture(fn, count):
    """A HIP graph of count back-to-back calls fn(0..count-1): replays launch the kernels without host overhead."""
    import torch

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn(0)
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(count):
            fn(i)
    torch.cuda.synchronize()
    return g


def time_graph(g, replays):
    """Mean ms per replay of graph g, bracketed by HIP events on the stream the replays run on."""
    import torch

    g.replay()
    torch.cuda.synchronize()
    s = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(s)
    for _ in range(replays):
        g.replay()
    e1.record(s)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / replays


def time_launches(fn, iters):
    """Mean µs per call of fn(i) over iters back-to-back calls captured in one HIP graph."""
    return time_graph(capture(fn, iters), 3) * 1e3 / iters


PREFILL = [("gate_up", 4096, 14336), ("down", 14336, 4096)]
SMALL_BATCH = [8, 16, 32, 64]
# the q4_K rows also cover the range where kf_hip_matmul's cost model moves from the few-row product to the tile GEMM
SMALL_BATCH_Q4_K = SMALL_BATCH + [96, 128, 192, 256]


def gemm_section(dev, m=2048, ty=None):
    """int8 MFMA GEMM of configs[3]: M=2048 Q8_0-kind activation rows against Q8_0 weights, both prefill shapes
    (with ty = q4_K: the same shapes with Q4_K weights and Q8K-kind activations, the tile GEMM kf_hip_matmul takes for
    Q4_K prefill). TOPS = 2*M*N*K / kernel time (the quant_act launch is timed beside it); two weight copies alternate."""
    import torch

    import kungfu_amd as kf

    ty = kf.TYPE_Q8_0 if ty is None else ty
    kind = kf.act_kind(ty)
    out = {}
    for name, n, n_out in PREFILL:
        w = torch.from_numpy(make_weights(ty, n, n_out)).to(dev)
        ws = [w, w.clone()]
        x = torch.from_numpy(kf.synth_normal(1, 1.0, m * n).reshape(m, n)).to(dev)
        act = kf.alloc_act(m, n, dev)
        y = torch.empty((m, n_out), device=dev)
        kf.quant_act(x, act, kind)
        us = time_launches(lambda i: kf.gemm_i8(ty, ws[i % 2], act, y, m, n, n_out), 20)
        us_q = time_launches(lambda i: kf.quant_act(x, act, kind), 20)
        tops = 2.0 * m * n * n_out / us / 1e6
        out[name] = {"M": m, "K": n, "N": n_out, "us": round(us, 2), "TOPS": round(tops, 1),
                     "frac": round(tops / INT8_PEAK_TOPS, 4), "quant_act_us": round(us_q, 2)}
        del ws, w, x, act, y
    return out


def gemm_q4_k_section(dev):
    import kungfu_amd as kf

    return gemm_section(dev, ty=kf.TYPE_Q4_K)


def gemm_k_quants_section(dev):
    """The q5_K and q6_K prefill GEMM (SURVEY's second "next" row) at the configs[3] shapes, M = 2048."""
    import kungfu_amd as kf

    return {"q5_K": gemm_section(dev, ty=kf.TYPE_Q5_K), "q6_K": gemm_section(dev, ty=kf.TYPE_Q6_K)}


def small_batch_section(dev):
    """batch 8..64 of the Llama-3-8B shapes with Q8_0 weights: the product kernel alone on resident
    quantized activations (µs per call, weight-streaming GB/s, TOPS) and the whole kf_hip_matmul (quant_act + product)."""
    import torch

    import kungfu_amd as kf

    out = {}
    for name, n, n_out in [("qkv", 4096, 6144), ("o", 4096, 4096), ("gate", 4096, 14336), ("down", 14336, 4096)]:
        w = torch.from_numpy(make_weights(kf.TYPE_Q8_0, n, n_out)).to(dev)
        ws = [w] + [w.clone() for _ in range(max(1, -(-2 * MALL_BYTES // w.numel())))]
        res = {}
        for m in SMALL_BATCH:
            x = torch.from_numpy(kf.synth_normal(1, 1.0, m * n).reshape(m, n)).to(dev)
            act = kf.alloc_act(m, n, dev)
            y = torch.empty((m, n_out), device=dev)
            kf.quant_act(x, act, kf.ACT_Q8_0)
            us = time_launches(lambda i: kf.gemm_i8(kf.TYPE_Q8_0, ws[i % len(ws)], act, y, m, n, n_out), 50)
            us_mm = time_launches(lambda i: kf.matmul(kf.TYPE_Q8_0, ws[i % len(ws)], x, act, y, n_out), 50)
            res[str(m)] = {"us": round(us, 2), "GBs": round(gemv_bytes(kf.TYPE_Q8_0, n, n_out, m) / us / 1e3, 1),
                           "TOPS": round(2.0 * m * n * n_out / us / 1e6, 2), "us_with_quant": round(us_mm, 2)}
        out[name] = res
        del ws, w
    return out


def small_batch_q4_k_section(dev):
    """Batch 8..64 of the Llama-3-8B shapes with Q4_K weights (the reference's mm_frag range): the multi-row product
    (kf_hip_gemv: 16 activation rows a weight pass on the matrix cores) and the tile GEMM (kf_hip_gemm_i8) alone on
    resident quantized activations, and the whole kf_hip_matmul (quant_act + the product it selects); weight copies
    rotated past the MALL."""
    import torch

    import kungfu_amd as kf

    ty = kf.TYPE_Q4_K
    out = {}
    for name, n, n_out in [("qkv", 4096, 6144), ("o", 4096, 4096), ("gate", 4096, 14336), ("down", 14336, 4096)]:
        w = torch.from_numpy(make_weights(ty, n, n_out)).to(dev)
        ws = [w] + [w.clone() for _ in range(max(1, -(-2 * MALL_BYTES // w.numel())))]
        res = {}
        for m in SMALL_BATCH_Q4_K:
            x = torch.from_numpy(kf.synth_normal(1, 1.0, m * n).reshape(m, n)).to(dev)
            act = kf.alloc_act(m, n, dev)
            y = torch.empty((m, n_out), device=dev)
            kf.quant_act(x, act, kf.ACT_Q8K)
            us_r = time_launches(lambda i: kf.gemv(ty, ws[i % len(ws)], act, y, m, n, n_out), 50)
            us_g = time_launches(lambda i: kf.gemm_i8(ty, ws[i % len(ws)], act, y, m, n, n_out), 50)
            us_mm = time_launches(lambda i: kf.matmul(ty, ws[i % len(ws)], x, act, y, n_out), 50)
            b = gemv_bytes(ty, n, n_out, m)
            res[str(m)] = {"rows_us": round(us_r, 2), "rows_GBs": round(b / us_r / 1e3, 1), "gemm_us": round(us_g, 2),
                           "gemm_GBs": round(b / us_g / 1e3, 1), "matmul_us": round(us_mm, 2)}
        out[name] = res
        del ws, w
    return out


def moe_section(dev, seed=0, rows=16):
    """the routed expert layer (kf_hip_moe_ffn) for 8 Q4_K experts of gate/up 4096->14336 and down
    14336->4096, 16 tokens, top-2 uniform without replacement. GB/s over the weight bytes of the touched experts (each
    read once per call) plus the fp32 activations in and out; two copies of the expert set alternate (1.6 GB).
    With rows = 512 (1024 routed pairs, the grouped tile GEMM): also TOPS = 2 * pairs * 3 * n_ff * n_embd / time, the
    whole layer (quantize, group, gather, both products, gated activation, combine) against the int8 peak."""
    import numpy as np
    import torch

    import kungfu_amd as kf

    ty, n_exp, n_embd, n_ff, n_used = kf.TYPE_Q4_K, 8, 4096, 14336, 2
    mats = []
    for i, (n_out, n_in) in enumerate([(n_ff, n_embd), (n_ff, n_embd), (n_embd, n_ff)]):
        w = torch.from_numpy(make_weights(ty, n_in, n_exp * n_out, seed=10 + i)).to(dev)
        mats.append([w, w.clone()])
    rng = np.random.default_rng(seed)
    sel = np.stack([rng.choice(n_exp, n_used, replace=False) for _ in range(rows)]).astype(np.int32)
    wts = rng.uniform(0.1, 1.0, sel.shape).astype(np.float32)
    x = torch.from_numpy(kf.synth_normal(1, 1.0, rows * n_embd).reshape(rows, n_embd)).to(dev)
    s_, w_ = torch.from_numpy(sel).to(dev), torch.from_numpy(wts).to(dev)
    scratch = torch.empty(kf.moe_scratch_bytes(rows, n_used, n_embd, n_ff, n_exp), dtype=torch.uint8, device=dev)
    out = torch.empty((rows, n_embd), device=dev)

    def call(i):
        kf.moe_ffn(ty, mats[0][i % 2], mats[1][i % 2], mats[2][i % 2], n_exp, n_embd, n_ff, x, s_, w_, out, scratch)

    us = time_launches(call, 20 if rows <= 64 else 5)
    touched = len(np.unique(sel))
    wbytes = touched * (2 * n_ff * kf.row_bytes(ty, n_embd) + n_embd * kf.row_bytes(ty, n_ff))
    nbytes = wbytes + 4 * rows * n_embd * 2
    del mats
    rec = {"us": round(us, 2), "GBs": round(nbytes / us / 1e3, 1), "frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4),
           "touched_experts": touched, "weight_bytes": wbytes, "tokens": rows, "top_k": n_used}
    if rows * n_used > 64:
        tops = 2.0 * rows * n_used * 3 * n_ff * n_embd / us / 1e6
        rec.update(TOPS=round(tops, 1), tops_frac=round(tops / INT8_PEAK_TOPS, 4), path="grouped tile GEMM")
    return rec


def moe_prefill_section(dev):
    return moe_section(dev, rows=512)


def layer_with_producers_section(shapes, dev):
    """The decode layer step with its activation producers, batch 1, Q4_K (every product's activations made inside the
    step, the cost Op::MatMul pays at M=1), GB/s over the same algorithmic bytes as the headline step: the library's
    path (kf_hip_rms_norm_matmul for QKV and gate+up, kf_hip_matmul for O, each one launch; gated_act_q8 -> down: five
    launches), and beside it the producers as launches of their own (rms_norm_q8 -> QKV, quant_act -> O, rms_norm_q8 ->
    gate+up, gated_act_q8 -> down: eight launches)."""
    import torch

    import kungfu_amd as kf

    by = {s.name: s for s in shapes}
    x = torch.from_numpy(kf.synth_normal(6, 1.0, 4096).reshape(1, 4096)).to(dev)
    wn = torch.from_numpy(kf.synth_normal(7, 1.0, 4096)).to(dev)
    attn = torch.from_numpy(kf.synth_normal(8, 1.0, 4096).reshape(1, 4096)).to(dev)
    n_ff = 14336

    def step(i):
        kf.rms_norm_q8(x, by["qkv"].act, kf.ACT_Q8K, wn, None, 1e-5)
        by["qkv"].gemv(i)
        kf.quant_act(attn, by["o"].act, kf.ACT_Q8K)
        by["o"].gemv(i)
        kf.rms_norm_q8(x, by["gate_up"].act, kf.ACT_Q8K, wn, None, 1e-5)
        by["gate_up"].gemv(i)
        gu = by["gate_up"].y
        kf.gated_act_q8(gu[:, :n_ff], gu[:, n_ff:], by["down"].act, kf.ACT_Q8K, 1, n_ff, 2 * n_ff)
        by["down"].gemv(i)

    def step_fused(i):
        # the library's own decode path: the norm (QKV, gate+up) or the quantization (O) inside the GEMV launch
        for nm, inp in (("qkv", x), ("o", attn), ("gate_up", x)):
            sh = by[nm]
            wi = sh.w[i % len(sh.w)]
            if nm == "o":
                kf.matmul(sh.ty, wi, inp, sh.act, sh.y, sh.n_out)
            else:
                kf.rms_norm_matmul(sh.ty, wi, inp, sh.act, sh.y, sh.n_out, wn, None, 1e-5)
        gu = by["gate_up"].y
        kf.gated_act_q8(gu[:, :n_ff], gu[:, n_ff:], by["down"].act, kf.ACT_Q8K, 1, n_ff, 2 * n_ff)
        by["down"].gemv(i)

    us_sep = time_launches(step, 50)
    us = time_launches(step_fused, 50)
    nb = sum(s.bytes for s in shapes)
    return {"us": round(us, 2), "GBs": round(nb / us / 1e3, 1), "frac": round(nb / us / 1e3 / HBM_PEAK_GBS, 4), "launches": 5,
            "separate_producers": {"us": round(us_sep, 2), "GBs": round(nb / us_sep / 1e3, 1), "launches": 8}}


def fused_section(dev):
    """The fused activation producers (SURVEY's first "next" row): rms_norm_q8 over the hidden width and gated_act_q8
    over the FFN width (silu, gate and up as the halves of one fused gate+up output row), at decode (1 row) and
    prefill (2048 rows), Q8K kind (the q4_K weights' kind). GB/s over the f32 read and the scratch written; quant_act
    of the same f32 input beside it, for the cost the fusion removes (the f32 write and re-read of the normed values)."""
    import torch

    import kungfu_amd as kf

    out = {}
    for rows in (1, 2048):
        n = 4096
        x = torch.from_numpy(kf.synth_normal(2, 1.0, rows * n).reshape(rows, n)).to(dev)
        w = torch.from_numpy(kf.synth_normal(3, 1.0, n)).to(dev)
        act = kf.alloc_act(rows, n, dev)
        us = time_launches(lambda i: kf.rms_norm_q8(x, act, kf.ACT_Q8K, w, None, 1e-5), 200)
        us_q = time_launches(lambda i: kf.quant_act(x, act, kf.ACT_Q8K), 200)
        nb = 4 * rows * n + 4 * n + kf.act_bytes(rows, n)
        out[f"rms_norm_q8_{rows}x{n}"] = {"us": round(us, 3), "GBs": round(nb / us / 1e3, 1), "quant_act_us": round(us_q, 3)}
        n = 14336
        gu = torch.from_numpy(kf.synth_normal(4, 1.0, rows * 2 * n).reshape(rows, 2 * n)).to(dev)
        act = kf.alloc_act(rows, n, dev)
        us = time_launches(lambda i: kf.gated_act_q8(gu[:, :n], gu[:, n:], act, kf.ACT_Q8K, rows, n, 2 * n), 200)
        nb = 8 * rows * n + kf.act_bytes(rows, n)
        out[f"gated_act_q8_{rows}x{n}"] = {"us": round(us, 3), "GBs": round(nb / us / 1e3, 1)}
    return out


def kquant_section(dev):
    """q6_K and q5_K weights (SURVEY's second "next" row) at the Llama-3-8B shapes, batch 1 (the GEMV) and batch 8 (eight
    activation rows against one weight pass): us per call and GB/s over weight bytes + f32 activations in and out,
    weight copies rotated past the MALL."""
    import kungfu_amd as kf

    out = {}
    for ty, tname in ((kf.TYPE_Q6_K, "q6_K"), (kf.TYPE_Q5_K, "q5_K")):
        for name, n, n_out in (("o", 4096, 4096), ("gate", 4096, 14336), ("down", 14336, 4096)):
            wb = kf.row_bytes(ty, n) * n_out
            sh = Shape(name, ty, n, n_out, max(2, -(-2 * MALL_BYTES // wb) + 1), dev)
            us = time_launches(sh.gemv, 100)
            rec = {"us": round(us, 3), "GBs": round(sh.bytes / us / 1e3, 1)}
            import torch

            x8 = torch.from_numpy(kf.synth_normal(5, 1.0, 8 * n).reshape(8, n)).to(dev)
            act8 = kf.alloc_act(8, n, dev)
            y8 = torch.empty((8, n_out), device=dev)
            kf.quant_act(x8, act8, kf.ACT_Q8K)
            us8 = time_launches(lambda i: kf.gemv(ty, sh.w[i % len(sh.w)], act8, y8, 8, n, n_out), 50)
            rec["us_8_rows"] = round(us8, 3)
            rec["GBs_8_rows"] = round(gemv_bytes(ty, n, n_out, 8) / us8 / 1e3, 1)
            out[f"{tname}_{name}"] = rec
            del sh
    return out


def group_section(dev):
    """Grouped products at the Llama-3-8B shapes, batch 1, Q4_K: Q/K/V (4096, 1024, 1024 rows) and gate/up (14336
    each) as separate tensors sharing one quantized input. us per layer part for separate launches, one grouped
    launch (the segment table) and one launch over a pre-stacked copy of the same rows; weight copies rotated past
    the MALL; GB/s over weight bytes + f32 activations in and out."""
    import numpy as np
    import torch

    import kungfu_amd as kf

    ty, n = kf.TYPE_Q4_K, 4096
    x = torch.from_numpy(kf.synth_normal(1, 1.0, n).reshape(1, n)).to(dev)
    act = kf.alloc_act(1, n, dev)
    kf.quant_act(x, act, kf.ACT_Q8K)
    out = {}
    for part, sizes in (("qkv", (4096, 1024, 1024)), ("gate_up", (14336, 14336))):
        total = sum(sizes)
        wb = kf.row_bytes(ty, n) * total
        copies = max(2, -(-2 * MALL_BYTES // wb) + 1)
        stacked = [torch.from_numpy(make_weights(ty, n, total)).to(dev)]
        stacked += [stacked[0].clone() for _ in range(copies - 1)]
        rb = kf.row_bytes(ty, n)
        bounds = np.cumsum((0,) + sizes)
        # members are views into each stacked copy: the same bytes, addressed as separate tensors
        members = [[stacked[c][bounds[k] : bounds[k + 1]] for k in range(len(sizes))] for c in range(copies)]
        ys = [torch.empty((1, m), device=dev) for m in sizes]
        y_all = torch.empty((1, total), device=dev)
        nbytes = gemv_bytes(ty, n, total)

        def separate(i):
            for k, m in enumerate(sizes):
                kf.gemv(ty, members[i % copies][k], act, ys[k], 1, n, m)

        def grouped(i):
            kf.gemv_group(ty, [(members[i % copies][k], ys[k], None, None) for k in range(len(sizes))], act, 1, n)

        def one(i):
            kf.gemv(ty, stacked[i % copies], act, y_all, 1, n, total)

        rec = {}
        for name, fn in (("separate", separate), ("grouped", grouped), ("stacked", one)):
            us = time_launches(fn, 100)
            rec[name] = {"us": round(us, 3), "GBs": round(nbytes / us / 1e3, 1)}
        rec["launches_separate"] = len(sizes)
        rec["weight_bytes"] = rb * total
        out[part] = rec
        del stacked, members
    return out


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "gemv_q4k_gate_up_traffic.md")


def traffic_section(dev):
    """The dispatches the traffic counters are read on: a device copy of exactly 256 MiB (the calibration: it must
    fetch and write 256 MiB) and three gate+up GEMV launches (Q4_K 4096 -> 28672, distinct weight copies), no graph."""
    import torch

    import kungfu_amd as kf

    src = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
    src.fill_(1)
    dst = torch.empty_like(src)
    sh = Shape("gate_up", kf.TYPE_Q4_K, 4096, 2 * 14336, 4, dev)
    torch.cuda.synchronize()
    for _ in range(3):
        dst.copy_(src)
    for i in range(3):
        sh.gemv(i + 1)
    torch.cuda.synchronize()
    return {"copy_bytes": src.numel(), "gemv_algorithmic_bytes": sh.bytes}


def read_probe(gate_up, dev):
    """HBM read rate of the streaming-read probe (kf_hip_stream_read: plain 16-byte loads, the whole buffer requested at
    launch), best of 4, 8 and 16 pieces a thread: over 4 GiB (the box's steady-state peak) and over the gate+up launch's
    own weight copies in the same rotation as the GEMV (that launch size's ceiling: launch, ramp and tail included)."""
    import torch

    import kungfu_amd as kf

    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    big = torch.empty(4 << 30, dtype=torch.uint8, device=dev)
    best_big = best_same = 0.0
    for p in (4, 8, 16):
        us = time_launches(lambda i: kf.stream_read(big, sink, p), 4)
        best_big = max(best_big, big.numel() / us / 1e3)
        ws = gate_up.w
        us = time_launches(lambda i: kf.stream_read(ws[i % len(ws)], sink, p), 200)
        best_same = max(best_same, ws[0].numel() / us / 1e3)
    del big
    return {"peak_measured": round(best_big, 1), "ceiling_same_bytes": round(best_same, 1)}


def same_bytes_ceiling(ws, dev):
    """Per-launch ceiling of a GEMV shape: the streaming-read probe over the shape's own weight copies, in the GEMV's
    rotation, best of 4, 8 and 16 pieces a thread (us a launch: launch, ramp and tail included)."""
    import torch

    import kungfu_amd as kf

    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    return min(time_launches(lambda i: kf.stream_read(ws[i % len(ws)], sink, p), 200) for p in (4, 8, 16))


def read_traffic():
    """HBM bytes per gate+up GEMV launch from the committed counter summary (null when it is absent)."""
    try:
        for line in open(TRAFFIC_PROFILE):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":")[1])
    except OSError:
        pass
    return None


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(shapes, budget_s):
    """The CPU backend's product (oracle restatement of ops::matmul_slice, OpenMP over output rows, as rayon's par_iter
    over rows) on the same weights and input: whole layer passes until budget_s of wall time is spent; then the same
    for its integer path (ops::matmul_i8: the activations quantized once per call, dot_i8 per row). Threads: every
    logical core the process may run on, capped by OMP_NUM_THREADS where the host sets it (a GPU box's CPU share)."""
    import oracle

    avail = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    env = int(os.environ.get("OMP_NUM_THREADS", "0"))
    threads = min(avail, env) if env > 0 else avail
    oracle.lib()

    def run(fn):
        total_bytes, passes, t0 = 0, 0, time.perf_counter()
        while True:
            for sh in shapes:
                fn(sh.ty, sh.host_w, sh.n, sh.n_out, sh.host_x, threads=threads)
                total_bytes += sh.bytes
            passes += 1
            el = time.perf_counter() - t0
            if el >= budget_s:
                return total_bytes / el / 1e9, passes, el

    v, passes, el = run(oracle.matmul_slice)
    vi, passes_i, el_i = run(oracle.matmul_i8)
    return {"value": round(v, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{passes} full layer passes (5 Q4_K GEMVs at M=1) of oracle matmul_slice in {el:.1f} s",
            "dot_i8_value": round(vi, 3), "dot_i8_sample": f"{passes_i} layer passes of oracle matmul_i8 in {el_i:.1f} s",
            "nproc": os.cpu_count(), "affinity_cores": avail, "cpu_model": cpu_model()}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--cpu-seconds", type=float, default=5.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--decode-only", action="store_true", help="the decode layer and per-shape GEMV figures alone (no side sections, no CPU leg)")
    ap.add_argument("--only", choices=["gemm", "gemm_q4_k", "gemm_kq", "small", "small_q4_k", "moe", "moe_prefill", "fused", "kquant", "group", "traffic"], help="run one side section alone (no JSON contract line)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the path shards along n_out across GPUs, "
              "which this build does not run", file=sys.stderr)
        sys.exit(2)

    import torch

    import kungfu_amd as kf

    dev = torch.device("cuda:0")
    kf.lib()
    if args.only:
        sec = {"gemm": gemm_section, "gemm_q4_k": gemm_q4_k_section, "gemm_kq": gemm_k_quants_section, "small": small_batch_section, "small_q4_k": small_batch_q4_k_section, "moe": moe_section, "moe_prefill": moe_prefill_section, "fused": fused_section, "kquant": kquant_section, "group": group_section, "traffic": traffic_section}[args.only]
        print(json.dumps(sec(dev)), flush=True)
        return
    layer_w_bytes = sum(kf.row_bytes(kf.TYPE_Q4_K, n) * no for _, n, no in LAYER)
    copies = max(2, -(-2 * MALL_BYTES // layer_w_bytes) + 1)
    shapes = [Shape(nm, kf.TYPE_Q4_K, n, no, copies, dev) for nm, n, no in LAYER]
    step_bytes = sum(s.bytes for s in shapes)

    def step(i):
        for s in shapes:
            s.gemv(i)

    # one graph holds GSTEP steps; the timed region replays it steps/GSTEP times after warmup replays
    gstep = 10
    steps = max(gstep, args.steps // gstep * gstep)
    g = capture(step, gstep)
    for _ in range(max(1, args.warmup // gstep)):
        g.replay()
    torch.cuda.synchronize()
    s = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(s)
    for _ in range(steps // gstep):
        g.replay()
    e1.record(s)
    torch.cuda.synchronize()
    ms_step = e0.elapsed_time(e1) / steps
    args.steps = steps
    value = step_bytes / (ms_step * 1e-3) / 1e9

    # per-shape µs/call of the GEMV kernel alone and of the whole matmul (quant_act + GEMV)
    per = {}
    k1_bytes = k1_us = 0.0
    for sh in shapes:
        us = time_launches(sh.gemv, 200)
        us_mm = time_launches(sh.matmul, 200)
        ceil_us = same_bytes_ceiling(sh.w, dev)
        per[sh.name] = {"n_in": sh.n, "n_out": sh.n_out, "us": round(us, 3), "GBs": round(sh.bytes / us / 1e3, 1),
                        "frac": round(sh.bytes / us / 1e3 / HBM_PEAK_GBS, 4), "us_with_quant": round(us_mm, 3),
                        "ceiling_us": round(ceil_us, 3), "frac_of_ceiling": round(ceil_us / us, 4)}
        if sh.name == "gate_up":  # gemv_pipe_kernel<q4_K, one wave a row>, the largest share of the step
            k1_bytes += sh.bytes
            k1_us += us
    achieved = k1_bytes / k1_us / 1e3
    probe = read_probe(shapes[2], dev)

    # Q8_0 GEMV of configs[0] (4096x4096) on the GPU, rotating copies
    q8 = Shape("q8_0", kf.TYPE_Q8_0, 4096, 4096, max(2, -(-2 * MALL_BYTES // (kf.row_bytes(8, 4096) * 4096)) + 1), dev)
    us_q8 = time_launches(q8.gemv, 200)
    ceil_q8 = same_bytes_ceiling(q8.w, dev)
    del q8

    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 x q4_K (int32 dot, f32 scale)",
        "data": "synthetic: SplitMix64/Box-Muller N(0,0.02) weights quantized to Q4_K, N(0,1) activations",
        "config": {"workload": "Q4_K decode GEMV, Llama-3-8B layer shapes, batch 1 (QKV, O, gate+up as one [28672] tensor, down)",
                   "bytes_per_step": step_bytes, "weight_copies": copies,
                   "hbm_frac": round(value / HBM_PEAK_GBS, 4)},
        "roofline": {"bound": "hbm", "kernel": "gemv_pipe_kernel<q4_K, one wave a row> (the gate+up launch)",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": read_traffic(),
                     "algorithmic_bytes": gemv_bytes(kf.TYPE_Q4_K, 4096, 2 * 14336),
                     # the streaming-read probe on this box: over 4 GiB, and over the same weight bytes per launch
                     "peak_measured": probe["peak_measured"], "frac_of_measured": round(achieved / probe["peak_measured"], 4),
                     "ceiling_same_bytes": probe["ceiling_same_bytes"],
                     "frac_of_ceiling": round(achieved / probe["ceiling_same_bytes"], 4)},
        "shapes": per,
        "q8_0_gemv_4096": {"us": round(us_q8, 3), "GBs": round(gemv_bytes(8, 4096, 4096) / us_q8 / 1e3, 1),
                           "frac": round(gemv_bytes(8, 4096, 4096) / us_q8 / 1e3 / HBM_PEAK_GBS, 4),
                           "ceiling_us": round(ceil_q8, 3), "frac_of_ceiling": round(ceil_q8 / us_q8, 4)},
    }
    if args.decode_only:
        print(json.dumps(out), flush=True)
        return
    out["int8_gemm"] = gemm_section(dev)
    out["int8_gemm_tops"] = min(v["TOPS"] for v in out["int8_gemm"].values())
    out["int8_gemm_q4_k"] = gemm_q4_k_section(dev)
    out["int8_gemm_k_quants"] = gemm_k_quants_section(dev)
    out["small_batch_q8_0"] = small_batch_section(dev)
    out["small_batch_q4_k"] = small_batch_q4_k_section(dev)
    out["moe_q4_k"] = moe_section(dev)
    out["moe_q4_k_prefill"] = moe_prefill_section(dev)
    out["layer_with_producers"] = layer_with_producers_section(shapes, dev)
    out["fused_producers"] = fused_section(dev)
    out["k_quants"] = kquant_section(dev)
    out["grouped"] = group_section(dev)
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(shapes, args.cpu_seconds)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
